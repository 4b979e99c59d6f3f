"""fp16 KV caches (an extension: the reference's cache is fp32 and its design defers an F16 KV cache,
docs/superpowers/specs/2026-10-17-nibble-design.md:181). The appended rows are bit-exact: fp16 (round to nearest
even, numpy's cast) of the reference's fp32 RoPE of the new K row, and of the new V row. The attention is pinned
to the oracle's attention over the cached fp16 values widened to fp32, with the tolerance of tests/gpu_util.py."""
import numpy as np
import pytest

import oracle
from nibble_amd import synth
from tests.gpu_util import Buffers, assert_parity, bits
from tests.test_gpu_parity import cpu_attention

pytestmark = pytest.mark.gpu


def upload_f16(B, a16):
    """An fp16 array into a backend buffer (floats: two halves each; odd sizes padded)."""
    flat = np.ascontiguousarray(a16, dtype=np.float16).reshape(-1)
    if flat.size % 2:
        flat = np.concatenate([flat, np.zeros(1, np.float16)])
    return B.upload(flat.view(np.float32))


def download_f16(be, ptr, shape):
    count = int(np.prod(shape))
    return be.download(ptr, ((count + 1) // 2,)).view(np.float16)[:count].reshape(shape)


@pytest.mark.parametrize("H,KV,D,neox,llama3", [(32, 8, 64, False, True), (14, 2, 64, True, False),
                                                 (16, 4, 128, False, True)])
@pytest.mark.parametrize("pos0", [0, 1, 33, 1023, 4113])
def test_f16kv_decode_step(backend, H, KV, D, neox, llama3, pos0):
    """One decode step over fp16 caches: the new row in the attention launch, q read unrotated."""
    base = 5e5 if llama3 else 1e4
    ff = synth.llama3_freq_factors(D, base) if llama3 else None
    rng = np.random.default_rng(pos0 * 3 + D + H)
    q = rng.standard_normal((1, H, D)).astype(np.float32)
    kn = rng.standard_normal((1, KV, D)).astype(np.float32)
    vn = rng.standard_normal((1, KV, D)).astype(np.float32)
    k0 = rng.standard_normal((pos0 + 3, KV, D)).astype(np.float16)
    v0 = rng.standard_normal((pos0 + 3, KV, D)).astype(np.float16)
    with Buffers(backend) as B:
        dq, dkn, dvn = B.upload(q), B.upload(kn), B.upload(vn)
        ck, cv = upload_f16(B, k0), upload_f16(B, v0)
        out = B.alloc(q.size)
        backend.append_rope_attention_f16kv(dq, ck, cv, dkn, dvn, out, 1, pos0, H, KV, D, base, neox, ff)
        got = backend.download(out, q.shape)
        gk, gv = download_f16(backend, ck, k0.shape), download_f16(backend, cv, v0.shape)
        gq = backend.download(dq, q.shape)
    kr = oracle.rope(kn.copy(), pos0, base, neox, ff)
    assert np.array_equal(gk[pos0].view(np.uint16), kr[0].astype(np.float16).view(np.uint16)), "appended K row"
    assert np.array_equal(gv[pos0].view(np.uint16), vn[0].astype(np.float16).view(np.uint16)), "appended V row"
    assert np.array_equal(gk[:pos0].view(np.uint16), k0[:pos0].view(np.uint16)), "rows before pos0 changed"
    assert np.array_equal(gk[pos0 + 1:].view(np.uint16), k0[pos0 + 1:].view(np.uint16)), "rows after pos0 changed"
    assert np.array_equal(bits(gq), bits(q)), "q modified"
    qr = oracle.rope(q.copy(), pos0, base, neox, ff)
    ref = cpu_attention(qr, gk[:pos0 + 1].astype(np.float32), gv[:pos0 + 1].astype(np.float32), pos0, KV)
    assert_parity(got, ref, f"f16 KV decode pos0={pos0}")


@pytest.mark.parametrize("n,pos0", [(5, 100), (16, 0), (40, 300)])
def test_f16kv_rows_and_append(backend, n, pos0):
    """Several rows: attention_f16kv over given caches (q rotated), and the append of n rows followed by the
    attention (q unrotated) in one call."""
    H, KV, D, base = 32, 8, 64, 1e4
    rng = np.random.default_rng(n + pos0)
    q = rng.standard_normal((n, H, D)).astype(np.float32)
    kn = rng.standard_normal((n, KV, D)).astype(np.float32)
    vn = rng.standard_normal((n, KV, D)).astype(np.float32)
    k0 = rng.standard_normal((pos0 + n, KV, D)).astype(np.float16)
    v0 = rng.standard_normal((pos0 + n, KV, D)).astype(np.float16)
    with Buffers(backend) as B:
        dq, dkn, dvn = B.upload(q), B.upload(kn), B.upload(vn)
        ck, cv = upload_f16(B, k0), upload_f16(B, v0)
        o1, o2 = B.alloc(q.size), B.alloc(q.size)
        backend.attention_f16kv(dq, ck, cv, o1, n, pos0, H, KV, D)
        r1 = backend.download(o1, q.shape)
        backend.append_rope_attention_f16kv(dq, ck, cv, dkn, dvn, o2, n, pos0, H, KV, D, base, False, None)
        r2 = backend.download(o2, q.shape)
        gk, gv = download_f16(backend, ck, k0.shape), download_f16(backend, cv, v0.shape)
    assert_parity(r1, cpu_attention(q, k0.astype(np.float32), v0.astype(np.float32), pos0, KV), "f16 KV rows")
    kr = oracle.rope(kn.copy(), pos0, base, False, None)
    assert np.array_equal(gk[pos0:].view(np.uint16), kr.astype(np.float16).view(np.uint16)), "appended K rows"
    assert np.array_equal(gv[pos0:].view(np.uint16), vn.astype(np.float16).view(np.uint16)), "appended V rows"
    qr = oracle.rope(q.copy(), pos0, base, False, None)
    assert_parity(r2, cpu_attention(qr, gk.astype(np.float32), gv.astype(np.float32), pos0, KV), "f16 KV append")


@pytest.mark.parametrize("n,pos0,qscale", [(300, 0, 1.0), (512, 4096, 1.0), (1024, 0, 5.0), (700, 77, 1.0)],
                         ids=["n300-pos0-0", "chunk512-pos0-4096", "n1024-qscale5", "n700-pos0-77"])
def test_f16kv_prefill_mfma_route(backend, n, pos0, qscale):
    """Prefill over fp16 caches: calls of more than 16 rows take the MFMA route - fp16 cache rows staged unchanged,
    rows below position 128 in fp32 from the fp16 cache, the error estimate and the split-operand recomputation (q
    scaled by 5 makes the scores large enough to list row tiles). First attention_f16kv over given caches (q
    rotated) against the oracle over the fp16 values; then the same rows through append_rope_attention_f16kv (the
    append fused with the staging, q unrotated): appended rows bit-exact (fp16 of the reference's fp32 RoPE), rows
    before pos0 untouched, output within tolerance."""
    H, KV, D, base = 32, 8, 64, 5e5
    ff = synth.llama3_freq_factors(D, base)
    rng = np.random.default_rng(n + pos0 + int(qscale))
    q = (rng.standard_normal((n, H, D)) * qscale).astype(np.float32)
    kn = rng.standard_normal((n, KV, D)).astype(np.float32)
    vn = rng.standard_normal((n, KV, D)).astype(np.float32)
    k0 = rng.standard_normal((pos0 + n, KV, D)).astype(np.float16)
    v0 = rng.standard_normal((pos0 + n, KV, D)).astype(np.float16)
    with Buffers(backend) as B:
        dq, dkn, dvn = B.upload(q), B.upload(kn), B.upload(vn)
        ck, cv = upload_f16(B, k0), upload_f16(B, v0)
        o1, o2 = B.alloc(q.size), B.alloc(q.size)
        backend.attention_f16kv(dq, ck, cv, o1, n, pos0, H, KV, D)
        r1 = backend.download(o1, q.shape)
        rec1 = backend.prefill_recomputed()
        backend.append_rope_attention_f16kv(dq, ck, cv, dkn, dvn, o2, n, pos0, H, KV, D, base, False, ff)
        r2 = backend.download(o2, q.shape)
        gk, gv = download_f16(backend, ck, k0.shape), download_f16(backend, cv, v0.shape)
    assert_parity(r1, cpu_attention(q, k0.astype(np.float32), v0.astype(np.float32), pos0, KV),
                  f"f16 KV prefill n={n} pos0={pos0} qscale={qscale}")
    kr = oracle.rope(kn.copy(), pos0, base, False, ff)
    assert np.array_equal(gk[pos0:].view(np.uint16), kr.astype(np.float16).view(np.uint16)), "appended K rows"
    assert np.array_equal(gv[pos0:].view(np.uint16), vn.astype(np.float16).view(np.uint16)), "appended V rows"
    assert np.array_equal(gk[:pos0].view(np.uint16), k0[:pos0].view(np.uint16)), "K rows before pos0 changed"
    assert np.array_equal(gv[:pos0].view(np.uint16), v0[:pos0].view(np.uint16)), "V rows before pos0 changed"
    qr = oracle.rope(q.copy(), pos0, base, False, ff)
    assert_parity(r2, cpu_attention(qr, gk.astype(np.float32), gv.astype(np.float32), pos0, KV),
                  f"f16 KV append + prefill n={n} pos0={pos0} qscale={qscale}")
    if qscale >= 5:
        assert rec1 > 0 and backend.prefill_recomputed() > 0


def test_f16kv_rejects_untiled_head_dim(backend):
    with Buffers(backend) as B:
        d = B.alloc(4096)
        with pytest.raises(Exception, match="head_dim must be 64 or 128"):
            backend.attention_f16kv(d, d, d, d, 1, 0, 4, 4, 32)


def test_f16kv_out_of_range_rows_store_inf(backend):
    """fp16 holds |x| <= 65504. An appended element beyond it is stored as +-inf - the IEEE conversion, bitwise
    what numpy's float16 cast gives - not saturated; the documented range limit of the fp16 cache."""
    H, KV, D, base, pos0 = 8, 2, 64, 1e4, 5
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, H, D)).astype(np.float32)
    kn = rng.standard_normal((1, KV, D)).astype(np.float32)
    vn = rng.standard_normal((1, KV, D)).astype(np.float32)
    kn[0, 0, :4] = [7e4, -7e4, 65504.0, 65520.0]  # 65520 is the first value that rounds up to inf
    vn[0, 1, 10:12] = [1e5, -1e6]
    k0 = np.zeros((pos0 + 1, KV, D), np.float16)
    with Buffers(backend) as B:
        dq, dkn, dvn = B.upload(q), B.upload(kn), B.upload(vn)
        ck, cv = upload_f16(B, k0), upload_f16(B, k0)
        out = B.alloc(q.size)
        backend.append_rope_attention_f16kv(dq, ck, cv, dkn, dvn, out, 1, pos0, H, KV, D, base, False, None)
        gk, gv = download_f16(backend, ck, k0.shape), download_f16(backend, cv, k0.shape)
    kr = oracle.rope(kn.copy(), pos0, base, False, None)
    with np.errstate(over="ignore"):
        want_k, want_v = kr[0].astype(np.float16), vn[0].astype(np.float16)
    assert np.isinf(want_k).any() and np.isinf(want_v).any()
    assert np.array_equal(gk[pos0].view(np.uint16), want_k.view(np.uint16)), "out-of-range K row"
    assert np.array_equal(gv[pos0].view(np.uint16), want_v.view(np.uint16)), "out-of-range V row"


def test_f16kv_shape_error_names_callers_head_dim(backend):
    # a cache range too short for the call: the message carries the head_dim the caller passed
    with Buffers(backend) as B:
        d = B.alloc(64)
        with pytest.raises(Exception, match="not inside one buffer"):
            backend.attention_f16kv(d, d, d, d, 1, 100, 1, 1, 64)
        with pytest.raises(Exception, match="head_dim=64"):
            backend.attention_f16kv(d, d, d, d, 1, 0, 3, 2, 64)
