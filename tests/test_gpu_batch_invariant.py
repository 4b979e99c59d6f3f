"""Batch invariance (HipBackend.set_batch_invariant): the reference's kernels compute every row with a fixed
accumulation order, and its model tests demand that batch, one-token-at-a-time and 2-token-chunk evaluation give
identical bits (tests/test_model.cpp:141-151, 253-263). The backend's default routes split work by the call's shape
(fp16-operand MFMA prefill, keys split over workgroups, rocBLAS for long float matmuls) and agree within rounding
only. With batch invariance on, every attention row takes the ordered fp32 route (one workgroup per row over its
whole window, keys in position order) and every float matmul the gemv kernel, so the bits of a row cannot depend on
how rows are grouped into calls. Checked here bit for bit at the attention level (fp32 and fp16 caches, every way of
cutting 300 rows into calls, the ragged-batch API) and at the model level (the reference's two tests, and the
head_dim-64 model whose default prefill runs on the MFMA kernel), each also against the oracle within tolerance.
"""
import numpy as np
import pytest

import oracle
from oracle import naive_model
from tests import model_util
from tests.gpu_util import Buffers, assert_parity, bits

pytestmark = pytest.mark.gpu

# (n_heads, n_kv_heads, head_dim): Llama-3-8B's 4:1 groups, Qwen2's 7:1, head_dim 128, and a head size without a
# tiled kernel (the generic kernel)
SHAPES = [(32, 8, 64), (14, 2, 64), (8, 2, 128), (4, 2, 8)]
T = 300


def _cuts(kind):
    """Calls as (first row, rows): the whole prompt, one row at a time, fixed chunks, and a ragged mix with calls
    above the decode kernel's 16 rows and across position 128 (where the default route's MFMA prefill starts)."""
    if kind == "batch":
        return [(0, T)]
    if kind == "incremental":
        return [(t, 1) for t in range(T)]
    if kind.startswith("chunks of "):
        c = int(kind.split()[-1])
        return [(t, min(c, T - t)) for t in range(0, T, c)]
    sizes, out, t = [37, 1, 100, 3, 17, 64, 16], [], 0
    for s in sizes * 3:
        if t >= T:
            break
        out.append((t, min(s, T - t)))
        t += s
    return out


CUTS = ["batch", "incremental", "chunks of 2", "chunks of 5", "ragged"]


def _inputs(H, KV, D, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    kn = rng.standard_normal((T, KV, D)).astype(np.float32)
    vn = rng.standard_normal((T, KV, D)).astype(np.float32)
    return q, kn, vn


def _append_attend(backend, f16, q, kn, vn, cuts, neox, base=10000.0):
    """append_rope_attention (fp32 caches) or append_rope_attention_f16kv over the given calls; returns the
    outputs and the caches' raw words."""
    _, H, D = q.shape
    KV = kn.shape[1]
    cache_floats = T * KV * D // (2 if f16 else 1)
    call = backend.append_rope_attention_f16kv if f16 else backend.append_rope_attention
    with Buffers(backend) as B:
        dq, dkn, dvn = B.upload(q), B.upload(kn), B.upload(vn)
        ck, cv, do = B.alloc(cache_floats), B.alloc(cache_floats), B.alloc(T * H * D)
        for t0, n in cuts:
            call(dq.at(t0 * H * D), ck, cv, dkn.at(t0 * KV * D), dvn.at(t0 * KV * D), do.at(t0 * H * D), n, t0, H, KV,
                 D, base, neox)
        out = backend.download(do, (T, H, D))
        kc = bits(backend.download(ck, (cache_floats,)))
        vc = bits(backend.download(cv, (cache_floats,)))
    return out, kc, vc


def _oracle(q, kn, vn, neox, f16, base=10000.0):
    KV = kn.shape[1]
    qr = oracle.rope(q, 0, base, neox)
    kr = oracle.rope(kn, 0, base, neox)
    v = vn
    if f16:  # the caches hold fp16(rope(k)) and fp16(v)
        kr = kr.astype(np.float16).astype(np.float32)
        v = vn.astype(np.float16).astype(np.float32)
    return oracle.attention_scalar(qr, kr, v, 0, KV)


@pytest.fixture
def invariant(backend):
    backend.set_batch_invariant(True)
    yield backend
    backend.set_batch_invariant(False)


@pytest.mark.parametrize("f16", [False, True], ids=["f32-cache", "f16-cache"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{h}x{kv}x{d}" for h, kv, d in SHAPES])
def test_append_rope_attention_bitwise_over_every_cut(invariant, shape, f16):
    H, KV, D = shape
    if f16 and D not in (64, 128):
        pytest.skip("fp16 caches: head_dim 64 and 128 only")
    neox = H % 7 == 0  # Qwen's NeoX pairing for the 14-head shape, interleaved pairs otherwise
    q, kn, vn = _inputs(H, KV, D, seed=H * 1000 + D)
    res = {c: _append_attend(invariant, f16, q, kn, vn, _cuts(c), neox) for c in CUTS}
    base_out, base_k, base_v = res["batch"]
    for c in CUTS[1:]:
        out, kc, vc = res[c]
        diff = int(np.sum(bits(out) != bits(base_out)))
        print(f"{shape} {'f16' if f16 else 'f32'} {c}: {diff} of {out.size} outputs differ from the batch call",
              flush=True)
        assert diff == 0, c
        assert np.array_equal(kc, base_k) and np.array_equal(vc, base_v), c
    assert_parity(base_out, _oracle(q, kn, vn, neox, f16), f"{shape} {'f16' if f16 else 'f32'} vs oracle")


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{h}x{kv}x{d}" for h, kv, d in SHAPES])
def test_attention_over_filled_caches_bitwise(invariant, shape):
    """attention() on rotated rows over caches already filled (no append, no rotation in the call)."""
    H, KV, D = shape
    q, kn, vn = _inputs(H, KV, D, seed=7 + D)
    qr, kr = oracle.rope(q, 0, 10000.0, False), oracle.rope(kn, 0, 10000.0, False)
    outs = {}
    with Buffers(invariant) as B:
        dq, dk, dv, do = B.upload(qr), B.upload(kr), B.upload(vn), B.alloc(T * H * D)
        for c in CUTS:
            for t0, n in _cuts(c):
                invariant.attention(dq.at(t0 * H * D), dk, dv, do.at(t0 * H * D), n, t0, H, KV, D)
            outs[c] = invariant.download(do, (T, H, D))
    for c in CUTS[1:]:
        assert np.array_equal(bits(outs[c]), bits(outs["batch"])), c
    assert_parity(outs["batch"], oracle.attention_scalar(qr, kr, vn, 0, KV), f"{shape} attention vs oracle")


def test_ragged_batch_api_matches_single_calls(invariant):
    """append_rope_attention_batch (one decode row per sequence) against one append_rope_attention call per
    sequence: the same bits, caches included."""
    H, KV, D = 32, 8, 64
    pos = [0, 5, 130, 299]
    rng = np.random.default_rng(3)
    rows = max(pos) + 1
    caches = [(rng.standard_normal((rows, KV, D)).astype(np.float32),
               rng.standard_normal((rows, KV, D)).astype(np.float32)) for _ in pos]
    q = [rng.standard_normal((H, D)).astype(np.float32) for _ in pos]
    kn = [rng.standard_normal((KV, D)).astype(np.float32) for _ in pos]
    vn = [rng.standard_normal((KV, D)).astype(np.float32) for _ in pos]
    got = []
    for batched in (True, False):
        with Buffers(invariant) as B:
            dq = [B.upload(x) for x in q]
            dkn, dvn = [B.upload(x) for x in kn], [B.upload(x) for x in vn]
            dk, dv = [B.upload(k) for k, _ in caches], [B.upload(v) for _, v in caches]
            do = [B.alloc(H * D) for _ in pos]
            if batched:
                invariant.append_rope_attention_batch(dq, dk, dv, dkn, dvn, do, pos, H, KV, D, 10000.0, False)
            else:
                for i, p in enumerate(pos):
                    invariant.append_rope_attention(dq[i], dk[i], dv[i], dkn[i], dvn[i], do[i], 1, p, H, KV, D,
                                                    10000.0, False)
            got.append(([bits(invariant.download(o, (H, D))) for o in do],
                        [bits(invariant.download(k, (rows, KV, D))) for k in dk]))
    for a, b in zip(got[0][0], got[1][0]):
        assert np.array_equal(a, b)
    for a, b in zip(got[0][1], got[1][1]):
        assert np.array_equal(a, b)


def _model_runs(backend, m, toks, n_ctx):
    """Logits of the last token: one call of every token, one token at a time, 2-token chunks and 17-token chunks
    (17 = one gemv slice of 16 rows and one of 1)."""
    out = {}
    for name, mb in (("batch", 512), ("chunks of 2", 2), ("chunks of 17", 17)):
        g = model_util.GpuModel(backend, m, n_ctx=n_ctx, max_batch=mb)
        try:
            out[name] = g.forward(toks)
        finally:
            g.close()
    g = model_util.GpuModel(backend, m, n_ctx=n_ctx)
    try:
        for t in range(len(toks)):
            inc = g.forward(toks[t:t + 1], pos0=t)
    finally:
        g.close()
    out["incremental"] = inc
    return out


@pytest.mark.parametrize("arch,rf", [("qwen2", False), ("llama", True)], ids=["qwen2", "llama-freqs"])
def test_model_incremental_and_chunked_equal_batch(invariant, arch, rf):
    """The reference's tests (test_model.cpp:141-151 for llama with rope freqs, 253-263 for qwen2): tiny model of
    seed 3, tokens {1, 50, 257, 3, 99}; batch, one-by-one and 2-token chunks give identical bits."""
    m = model_util.tiny_model(3, np.float32, arch, rf)
    toks = [1, 50, 257, 3, 99]
    out = _model_runs(invariant, m, toks, 64)
    for name, o in out.items():
        assert np.array_equal(bits(o), bits(out["batch"])), name
    d = float(np.max(np.abs(out["batch"] - naive_model.naive_logits(m, toks))))
    print(f"{arch}: |batch - naive| {d:.2e}", flush=True)
    assert d <= 1e-4


@pytest.mark.parametrize("wtype", [np.float32, np.float16], ids=["f32", "f16"])
def test_model_head_dim_64_bitwise(invariant, wtype):
    """n_embd 256, 4 heads of 64, llama with rope freqs, 150 tokens: by default the batch call runs rows 128.. on the
    MFMA prefill and its matmuls on rocBLAS; with batch invariance every cut of the prompt gives the same bits, and
    the reference's float bar against the fp64 naive model holds."""
    m = model_util.tiny_model(11, wtype, "llama", True, E=256, FF=512, scale=0.25)
    toks = np.random.default_rng(5).integers(0, 261, 150).tolist()
    out = _model_runs(invariant, m, toks, 160)
    for name, o in out.items():
        diff = int(np.sum(bits(o) != bits(out["batch"])))
        print(f"hd64 {np.dtype(wtype).name} {name}: {diff} logits differ from batch", flush=True)
        assert diff == 0, name
    naive = naive_model.naive_logits(m, toks)
    d = float(np.max(np.abs(out["batch"] - naive)))
    print(f"hd64 {np.dtype(wtype).name}: |batch - naive| {d:.2e} (max |logit| {np.max(np.abs(naive)):.2f})",
          flush=True)
    assert d <= 1e-4 * max(1.0, float(np.max(np.abs(naive))))


def test_default_route_differences_are_reported(backend):
    """Without batch invariance the same model's batch and incremental runs agree within rounding only; the number
    of differing logits is printed beside the invariant mode's zero (not gated: it is the reason for the switch)."""
    m = model_util.tiny_model(11, np.float16, "llama", True, E=256, FF=512, scale=0.25)
    toks = np.random.default_rng(5).integers(0, 261, 150).tolist()
    backend.set_batch_invariant(False)
    out = _model_runs(backend, m, toks, 160)
    for name, o in out.items():
        diff = int(np.sum(bits(o) != bits(out["batch"])))
        print(f"default route, {name}: {diff} of {o.size} logits differ from batch, "
              f"max |x - batch| {np.max(np.abs(o - out['batch'])):.2e}", flush=True)
        assert np.all(np.isfinite(o))
        assert float(np.max(np.abs(o - out["batch"]))) <= 1e-2
