"""Host-side argument checks of the MFMA prefill entry point of libnibble_hip.so, on the CPU: each case is rejected
with NBHS_EINVAL before anything is launched (no GPU call is made here; the pointers are never dereferenced). Also the
host-side sizing helpers (work list bound, whole-row decode route)."""
import ctypes

import pytest

import nibble_amd

EINVAL = 1
FAKE = 256  # a non-null address the checks never follow


@pytest.fixture(scope="module")
def prefill():
    L = ctypes.CDLL(nibble_amd.LIB_PATH)
    i64, vp, cint = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
    f = L.nbhs_attn_prefill_mfma
    f.restype = cint
    f.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, i64, i64, vp, i64, cint, vp, vp, i64, vp, i64, vp, i64, cint, vp]

    def call(n=64, pos0=0, n_heads=32, n_kv=8, hd=64, rows_pad=None, fp32_rows=0, aux_words=1 << 20):
        rows_pad = ((pos0 + n + 63) // 64) * 64 if rows_pad is None else rows_pad
        return f(FAKE, FAKE, FAKE, FAKE, n, pos0, n_heads, n_kv, hd, rows_pad, None, 0, 0, FAKE, FAKE, fp32_rows,
                 FAKE, 1 << 40, FAKE, aux_words, 256, None)
    return call


def test_staged_buffers_beyond_32bit_buffer_size(prefill):
    """The kernel reads one KV head's staged K and V^T through buffer resources whose size field is 32 bits: a
    staging of rows_pad * head_dim fp16 values over 2 GiB per head is refused."""
    assert prefill(n=64, pos0=(1 << 24) - 64, hd=64, rows_pad=1 << 24) == EINVAL
    assert prefill(n=64, pos0=(1 << 23) - 64, hd=128, rows_pad=1 << 23) == EINVAL


@pytest.mark.parametrize("kw", [
    dict(hd=96),                          # head_dim other than 64 / 128
    dict(n_heads=30, n_kv=8),             # query heads not a multiple of the KV heads
    dict(n=0),                            # no rows
    dict(pos0=-1),
    dict(rows_pad=100),                   # staged rows not a multiple of the 64-row tile
    dict(n=200, pos0=0, rows_pad=128),    # staged rows short of pos0 + n
    dict(fp32_rows=64),                   # every row on the fp32 path
    dict(aux_words=8),                    # work list too small for the row tiles
])
def test_bad_shapes_are_rejected(prefill, kw):
    assert prefill(**kw) == EINVAL


def test_mfma_loop_arguments_are_checked():
    """The MFMA calibration launch rejects its bad arguments before launching anything."""
    L = ctypes.CDLL(nibble_amd.LIB_PATH)
    f = L.nbhs_mfma_loop_f16
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    assert f(None, 16, 3, 256, None) == EINVAL          # no output
    assert f(FAKE, 0, 3, 256, None) == EINVAL           # no iterations
    assert f(FAKE, (1 << 24) + 1, 3, 256, None) == EINVAL
    assert f(FAKE, 16, 0, 256, None) == EINVAL          # waves per SIMD out of 1..8
    assert f(FAKE, 16, 9, 256, None) == EINVAL
    assert f(FAKE, 16, 3, 0, None) == EINVAL            # no CUs


def test_decode_rows_route_shapes():
    """The whole-row decode route's shapes: one row, whole-wave KV-head chunks (8 heads at head_dim 64, 4 at 128),
    at most 8 chunks per row, GQA group 1, 2 or 4 (host-side predicate, no GPU call)."""
    L = ctypes.CDLL(nibble_amd.LIB_PATH)
    f = L.nbhs_attn_decode_rows_route
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int64] * 4
    yes = [(1, 32, 8, 64), (1, 8, 8, 64), (1, 16, 8, 64), (1, 32, 16, 64), (1, 32, 8, 128), (1, 16, 4, 128),
           (1, 128, 32, 128), (1, 256, 64, 64)]
    no = [(2, 32, 8, 64), (16, 32, 8, 64), (1, 14, 2, 64), (1, 32, 4, 64), (1, 64, 8, 64), (1, 48, 16, 64),
          (1, 24, 8, 96), (1, 256, 64, 128), (1, 8, 2, 128), (0, 32, 8, 64), (1, 30, 8, 64)]
    assert all(f(*a) == 1 for a in yes), [a for a in yes if f(*a) != 1]
    assert all(f(*a) == 0 for a in no), [a for a in no if f(*a) != 0]


def test_work_list_bound_covers_every_kv_head_count():
    """reserve() sizes the prefill work list with nbhs_prefill_aux_words_bound(max_rows, n_heads): it must cover
    every call of up to max_rows rows for every KV head count dividing n_heads. One KV head is not the worst case
    when max_rows * group is not a multiple of the 128-row tile (max_rows 100 with 32 / 32 heads needs 112 words,
    one KV head gives 91)."""
    L = ctypes.CDLL(nibble_amd.LIB_PATH)
    words, bound = L.nbhs_prefill_aux_words, L.nbhs_prefill_aux_words_bound
    words.restype = bound.restype = ctypes.c_int64
    words.argtypes = [ctypes.c_int64] * 3
    bound.argtypes = [ctypes.c_int64] * 2
    assert words(100, 32, 1) == 91 and words(100, 32, 32) == 112  # the under-reservation a one-head bound made
    for max_rows in (1, 17, 100, 127, 128, 129, 200, 300, 512, 1000):
        for H in (1, 2, 7, 14, 24, 32, 40, 64):
            b = bound(max_rows, H)
            need = max(words(m, H, kv) for m in {1, max_rows // 2 + 1, max_rows} for kv in range(1, H + 1)
                       if H % kv == 0)
            assert b == need, (max_rows, H, b, need)
    assert bound(0, 32) == -1 and bound(16, 0) == -1
