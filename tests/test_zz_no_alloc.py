"""The allocation-free decode entry point, nbh_attention_decode_noalloc, against the entry point it is a variant
of, nbh_backend_attention on its decode route, through the C ABI. Both run the same kernels with the same plan
(the split partials go to the library's static device array instead of the backend's workspace), so outputs must
be bit-identical; they are also held to the parity tolerance of the oracle. Calls in a row, each with a smaller
input than the one before, so each runs over the array the previous one left behind."""
import ctypes

import numpy as np
import pytest

import nibble_amd
from tests.gpu_util import Buffers, assert_parity, bits
from tests.test_gpu_parity import cpu_attention

pytestmark = pytest.mark.gpu

# (n, pos0, n_heads, n_kv_heads, head_dim): a 16-row append-sized call deep in a cache, a single decode row on the
# whole-row route, then a single row of a shape the per-head kernel serves, each smaller than the one before
CALLS = [(16, 5000, 32, 8, 64), (1, 3000, 32, 8, 64), (1, 700, 14, 2, 64)]


def test_noalloc_decode_matches_backend_attention():
    be = nibble_amd.HipBackend(0)
    try:
        stream = be.stream_handle()
        for i, (n, pos0, H, KV, D) in enumerate(CALLS):
            rng = np.random.default_rng(17 + i)
            q = rng.standard_normal((n, H, D)).astype(np.float32)
            k = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
            v = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
            with Buffers(be) as B:
                dq, dk, dv = B.upload(q), B.upload(k), B.upload(v)
                o_ref, o_new = B.alloc(q.size), B.alloc(q.size)
                be.write(o_new, np.full(q.size, np.nan, np.float32))  # every output element must be written
                be.attention(dq, dk, dv, o_ref, n, pos0, H, KV, D)
                before = be.internal_bytes()
                nibble_amd.attention_decode_noalloc(dq, dk, dv, o_new, n, pos0, H, KV, D, stream)
                got_ref, got_new = be.download(o_ref, q.shape), be.download(o_new, q.shape)
                assert be.internal_bytes() == before
            print(f"call {i}: n={n} pos0={pos0} H={H} KV={KV}", flush=True)
            assert np.array_equal(bits(got_new), bits(got_ref)), f"call {i}: differs from nbh_backend_attention"
            assert_parity(got_new, cpu_attention(q, k, v, pos0, KV), f"noalloc decode call {i}")
    finally:
        be.close()


def test_noalloc_decode_rejects_shapes_off_the_decode_route():
    be = nibble_amd.HipBackend(0)
    try:
        with Buffers(be) as B:
            d = B.alloc(64 * 64 * 8)
            with pytest.raises(nibble_amd.BackendError, match="invalid shape n=17"):
                nibble_amd.attention_decode_noalloc(d, d, d, d, 17, 0, 8, 8, 64, be.stream_handle())
            with pytest.raises(nibble_amd.BackendError, match="invalid shape"):
                nibble_amd.attention_decode_noalloc(d, d, d, d, 1, 0, 6, 4, 64, be.stream_handle())
    finally:
        be.close()


def test_noalloc_decode_whole_row_shape_beyond_the_array():
    """Llama-3-8B's decode shape (32 / 8 heads, head_dim 128) at 40000 positions qualifies for the whole-row kernel,
    but its partials (32 heads x 256 workgroups x 130 floats) exceed the 4 MiB array: the entry point takes the
    per-head split kernel instead, which nbh_backend_attention does not, so the outputs are held to the oracle's
    tolerance rather than to bit-identity; nothing is allocated."""
    n, pos0, H, KV, D = 1, 40000, 32, 8, 128
    capacity = nibble_amd.lib().nbhs_attn_decode_noalloc_capacity
    capacity.restype = ctypes.c_int64
    assert capacity() < H * 256 * (D + 2)
    be = nibble_amd.HipBackend(0)
    try:
        rng = np.random.default_rng(41)
        q = rng.standard_normal((n, H, D)).astype(np.float32)
        k = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
        v = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
        with Buffers(be) as B:
            dq, dk, dv, do = B.upload(q), B.upload(k), B.upload(v), B.alloc(q.size)
            be.write(do, np.full(q.size, np.nan, np.float32))
            be.sync()
            before = be.internal_bytes()
            nibble_amd.attention_decode_noalloc(dq, dk, dv, do, n, pos0, H, KV, D, be.stream_handle())
            got = be.download(do, q.shape)
            assert be.internal_bytes() == before
        assert_parity(got, cpu_attention(q, k, v, pos0, KV), "noalloc decode beyond the array")
    finally:
        be.close()
