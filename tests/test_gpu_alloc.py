"""Heap allocations of the backend's own code on its warm paths (backend.h:42-45: after reserve(), ops within the
reserved sizes must not allocate; the reference counts every operator new in tests/alloc_tests.cpp:278-380).

tests/alloc_check.cpp replaces the global operator new and charges each allocation to the shared object of its
first caller frame outside the C/C++ runtime libraries. The backend's own code (libnibble_hip.so: HipBackend and the
C ABI) must allocate nothing in warm decode steps, prefill chunks, quantized matmuls and ragged batch decodes, nor in
the first prefill and decode calls after reserve() and reserve_rope(). The HIP runtime and rocBLAS allocate inside
the calls the backend makes to them (kernel launches, sgemm); those counts are reported, not gated: they are outside
the backend's control. The driver is a separate program, run as a child process."""
import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_bin", "alloc_check")
WARM = ["decode_steps", "prefill_chunks", "matmul_quantized", "batch_decode"]


@pytest.fixture(scope="module")
def tally():
    if not os.path.exists(BIN):
        pytest.fail("tests/_bin/alloc_check is not built (make -C nibble_amd/csrc)")
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-2000:]
    t = json.loads(r.stdout.strip().splitlines()[-1])
    for name, p in t.items():
        print(f"{name}: {p['calls']} calls, own {p['own']}, unattributed {p['unattributed']}, "
              f"libraries {p['libraries']}", flush=True)
    return t


@pytest.mark.parametrize("phase", WARM)
def test_warm_paths_allocate_nothing_in_the_backend(tally, phase):
    p = tally[phase]
    assert p["own"] == 0, p
    assert p["unattributed"] == 0, p


def test_first_calls_after_reserve_allocate_nothing_in_the_backend(tally):
    """The first prefill and decode calls after reserve() (and reserve_rope(), which builds the RoPE table that
    the first rope call would otherwise build on the host): every device buffer and the work list were sized by
    reserve(), so the backend's own code allocates nothing. The HIP runtime loads each kernel's code on its first
    launch and allocates for that."""
    p = tally["first_calls_after_reserve"]
    assert p["own"] == 0, p


def test_runtime_launch_allocations_are_reported(tally):
    """The runtime's own allocations per kernel launch, measured on a call that is one launch and nothing else: a
    number the backend cannot change, reported beside the backend's zero (and charged to the runtime's library, not
    to the backend)."""
    p = tally["runtime_fill_normal_launches"]
    assert p["own"] == 0, p
    per_launch = sum(p["libraries"].values()) / p["calls"]
    print(f"HIP runtime allocations per kernel launch: {per_launch:.2f}", flush=True)
