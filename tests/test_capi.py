"""The C ABI library loads and exports every function include/*.h declares; the product path never touches the
oracle; without the library the Python binding refuses to run. CPU only (no compute calls)."""
import ctypes
import glob
import os
import re

import pytest

import nibble_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*(nbhs?_[A-Za-z0-9_]+)\s*\(", re.M)


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        with open(h) as f:
            names |= set(DECL.findall(f.read()))
    return sorted(names)


def test_headers_declare_the_boundary():
    names = declared_functions()
    for required in ["nbh_backend_create", "nbh_backend_rope", "nbh_backend_attention", "nbh_backend_reserve",
                     "nbh_backend_alloc", "nbh_backend_free", "nbh_backend_read", "nbh_backend_copy",
                     "nbhs_attn_decode_f32", "nbhs_attn_prefill_mfma", "nbhs_rope_f32", "nbhs_append_rope_f32"]:
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(nibble_amd.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_binding_covers_the_c_abi():
    public = {n for n in declared_functions() if n.startswith("nbh_")}
    assert public == set(nibble_amd._SIGNATURES), public ^ set(nibble_amd._SIGNATURES)
    nibble_amd.lib()  # binds every signature


def test_library_is_gfx950_only():
    # The kernels are built for gfx950 alone (no dual paths): the code object names that target.
    with open(nibble_amd.LIB_PATH, "rb") as f:
        blob = f.read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    for other in (b"amdgcn-amd-amdhsa--gfx942", b"amdgcn-amd-amdhsa--gfx90a", b"nvptx"):
        assert other not in blob


def test_product_path_does_not_use_the_oracle():
    pattern = re.compile(r"\boracle\b|liboracle|libnibble_ref|_ref/")
    offenders = []
    for path in glob.glob(os.path.join(ROOT, "nibble_amd", "**", "*"), recursive=True):
        if os.path.isdir(path) or not path.endswith((".py", ".cpp", ".h", ".hip", "Makefile")):
            continue
        with open(path, errors="replace") as f:
            for i, line in enumerate(f, 1):
                if pattern.search(line):
                    offenders.append(f"{os.path.relpath(path, ROOT)}:{i}: {line.strip()}")
    assert not offenders, "\n".join(offenders)


def test_binding_fails_loudly_without_the_library(monkeypatch):
    monkeypatch.setattr(nibble_amd, "_lib", None)
    monkeypatch.setattr(nibble_amd, "LIB_PATH", os.path.join(ROOT, "does-not-exist.so"))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        nibble_amd.lib()


def test_backend_creation_without_gpu_raises():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU driver is present")
    with pytest.raises(nibble_amd.BackendError):
        nibble_amd.HipBackend(0)


def test_weight_views_keep_their_host_arrays_alive():
    """A weight made from a temporary host array (float or raw quantized blocks) still points at intact data after
    the caller's reference is gone: the backend uploads a weight at its first use, possibly much later."""
    import ctypes
    import gc

    import numpy as np

    import nibble_amd

    wf = nibble_amd.weight(np.arange(16, dtype=np.float32).reshape(4, 4))
    wq = nibble_amd.weight(np.arange(144 * 2, dtype=np.uint8) % 251, shape=(2, 256), dtype=12)
    gc.collect()
    _ = [np.ones(1 << 20, dtype=np.uint8) for _ in range(4)]  # allocations that would reuse freed memory
    got_f = np.ctypeslib.as_array((ctypes.c_float * 16).from_address(wf.data))
    got_q = np.ctypeslib.as_array((ctypes.c_uint8 * (144 * 2)).from_address(wq.data))
    assert np.array_equal(got_f, np.arange(16, dtype=np.float32))
    assert np.array_equal(got_q, np.arange(144 * 2, dtype=np.uint8) % 251)
