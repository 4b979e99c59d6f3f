"""A whole forward on the GPU: the reference Transformer's op sequence (src/model/transformer.cpp:128-220) driven
through HipBackend, against the fp64 naive model (oracle/naive_model.py, restating tests/naive_llama.h) and the
reference's forward restated from the oracle's float ops.

Bars: the reference's own, max |logit difference| <= 1e-4 (tests/test_model.cpp:110-131), for the tiny models
(head_dim 4: every attention call takes the fp32 kernels). The head_dim-64 model runs its rows at positions >= 128
on the fp16-operand MFMA prefill kernel, whose fp16 rounding of K, V and the scaled Q is ~5e-4 relative per term:
there the bar is 1e-3 relative to the logits' largest magnitude, the attention tolerance carried to the logits
(measured values are printed). With unscaled weights (large attention scores) the kernel's error estimate sends
the affected row tiles to the split-operand recomputation, and the forward meets the reference's own float bar.

Chunking: the reference demands bitwise equality of batch, incremental and 2-token-chunk runs
(test_model.cpp:141-151); this backend's default kernels split work by shape, so chunked runs agree within tolerance
here. Its batch-invariant mode restores the reference's bitwise guarantee (tests/test_gpu_batch_invariant.py).
"""
import numpy as np
import pytest

from oracle import naive_model
from tests import model_util

pytestmark = pytest.mark.gpu
TOKS = [1, 50, 257, 3, 99]


@pytest.mark.parametrize("arch,wtype,rf", [("qwen2", np.float32, False), ("qwen2", np.float16, False),
                                           ("llama", np.float32, False), ("llama", np.float32, True),
                                           ("llama", np.float16, True)],
                         ids=["qwen2-f32", "qwen2-f16", "llama-f32", "llama-f32-freqs", "llama-f16-freqs"])
def test_forward_matches_naive_model(backend, arch, wtype, rf):
    m = model_util.tiny_model(7, wtype, arch, rf)
    g = model_util.GpuModel(backend, m, n_ctx=64)
    try:
        got = g.forward(TOKS)
    finally:
        g.close()
    naive = naive_model.naive_logits(m, TOKS)
    ref = model_util.cpu_forward(m, TOKS)
    print(f"{arch} {np.dtype(wtype).name} freqs={rf}: |gpu-naive| {np.max(np.abs(got - naive)):.2e}, "
          f"|gpu-restated ref| {np.max(np.abs(got - ref)):.2e}", flush=True)
    assert np.all(np.isfinite(got))
    assert float(np.max(np.abs(got - naive))) <= 1e-4
    assert float(np.max(np.abs(got - ref))) <= 1e-4


def test_forward_chunked_and_incremental_agree(backend):
    m = model_util.tiny_model(3, np.float32, "llama", True)
    toks = [1, 50, 257, 3, 99, 7, 8, 200, 13]
    outs = {}
    for name, mb in (("batch", 512), ("chunks of 2", 2)):
        g = model_util.GpuModel(backend, m, n_ctx=64, max_batch=mb)
        try:
            outs[name] = g.forward(toks)
        finally:
            g.close()
    g = model_util.GpuModel(backend, m, n_ctx=64)
    try:
        for t in range(len(toks)):  # one token at a time, as a decode loop calls forward
            inc = g.forward(toks[t:t + 1], pos0=t)
    finally:
        g.close()
    outs["incremental"] = inc
    naive = naive_model.naive_logits(m, toks)
    for name, o in outs.items():
        d = float(np.max(np.abs(o - outs["batch"])))
        print(f"{name}: |x - batch| {d:.2e}, |x - naive| {np.max(np.abs(o - naive)):.2e}", flush=True)
        assert d <= 1e-5
        assert float(np.max(np.abs(o - naive))) <= 1e-4


def _hd64_run(backend, m, toks, fp32=False):
    backend.set_attention_fp32(fp32)
    g = model_util.GpuModel(backend, m, n_ctx=320)
    try:
        out = [(300, g.forward(toks[:300]))]
        out += [(301 + s, g.forward(toks[300 + s:301 + s], pos0=300 + s)) for s in range(3)]
    finally:
        g.close()
        backend.set_attention_fp32(False)
    return out


def test_forward_head_dim_64_through_the_mfma_prefill(backend):
    """n_embd 256, 4 heads of 64 (the reference's kquant_dims shape), llama with rope freqs, F16 weights, 300 tokens
    in one chunk: rows 128..299 of every layer run on the MFMA prefill kernel; then 3 decode steps. The weights are
    scaled by sqrt(16 / 256) so that activations have the statistics of the n_embd-16 models (attention scores of
    order 1, as trained models have)."""
    m = model_util.tiny_model(11, np.float16, "llama", True, E=256, FF=512, scale=0.25)
    toks = np.random.default_rng(5).integers(0, 261, 303).tolist()
    for n, o in _hd64_run(backend, m, toks):
        naive = naive_model.naive_logits(m, toks[:n])
        d = float(np.max(np.abs(o - naive)))
        print(f"hd64 {n} tokens: |gpu-naive| {d:.2e} (max |logit| {np.max(np.abs(naive)):.2f})", flush=True)
        assert np.all(np.isfinite(o))
        assert d <= 1e-3 * max(1.0, float(np.max(np.abs(naive))))  # 1e-3 relative to the logits' scale


@pytest.mark.parametrize("fp32", [False, True], ids=["default-route", "fp32-attention"])
def test_forward_large_scores(backend, fp32):
    """Unscaled uniform(-0.5, 0.5) weights at n_embd 256 give attention scores of ~30 (log2 units): the softmax is
    nearly an argmax, and fp16 rounding of Q and K alone would decide near-ties (it moved the logits by ~1e-1). On
    the default route the MFMA kernel's error estimate sends those row tiles to the split-operand recomputation; with
    set_attention_fp32 every row takes the fp32 kernels. Either way the forward must stay as close to the fp64 model
    as the reference's own float forward (restated from the pinned oracle ops) is: ~1.5e-4 on logits of ~15, so the
    bar is max(1e-4, 1.5 x the reference's deviation)."""
    m = model_util.tiny_model(11, np.float16, "llama", True, E=256, FF=512)
    toks = np.random.default_rng(5).integers(0, 261, 303).tolist()
    for n, o in _hd64_run(backend, m, toks, fp32=fp32):
        naive = naive_model.naive_logits(m, toks[:n])
        d = float(np.max(np.abs(o - naive)))
        d_ref = float(np.max(np.abs(model_util.cpu_forward(m, toks[:n]) - naive)))
        print(f"hd64 large scores, {'fp32 attention' if fp32 else 'default route'}, {n} tokens: |gpu-naive| {d:.2e}, "
              f"reference float forward |ref-naive| {d_ref:.2e} (max |logit| {np.max(np.abs(naive)):.2f})", flush=True)
        assert d <= max(1e-4, 1.5 * d_ref)
        if not fp32 and n == 300:
            assert backend.prefill_recomputed() > 0


@pytest.mark.parametrize("wkind", ["f16", "q8_0+q4_0"])
def test_first_forward_after_reserve_allocates_nothing(wkind):
    """alloc_tests.cpp:338-380 on the GPU: a fresh backend and model (whose constructor calls reserve(), as
    Transformer's does), then the very first forward - a full max_batch prefill whose rows >= 128 run on the MFMA
    route, then decode steps - grows no internal buffer. Device copies of host weights are model state, counted
    apart (weight_bytes), as nibble's weights are loaded before generation."""
    import nibble_amd
    import oracle
    from tests import quant_util as U

    m = model_util.tiny_model(11, np.float16 if wkind == "f16" else np.float32, "llama", True, E=256, FF=512)
    if wkind != "f16":
        for L in m["layers"]:
            for k in ("wq", "wk", "wv", "w_gate", "w_up"):
                L[k] = U.quantize_matrix(L[k], oracle.Q8_0)
            for k in ("wo", "w_down"):
                L[k] = U.quantize_matrix(L[k], oracle.Q4_0)
    be = nibble_amd.HipBackend(0)
    try:
        g = model_util.GpuModel(be, m, n_ctx=1024, max_batch=512)
        cap = be.internal_bytes()
        toks = [int(t) for t in np.random.default_rng(4).integers(0, 261, 512)]
        logits = g.forward(toks)
        for i in range(4):
            logits = g.forward([7 + i], pos0=512 + i)
        assert np.all(np.isfinite(logits))
        assert be.internal_bytes() == cap
        g.close()
    finally:
        be.close()

