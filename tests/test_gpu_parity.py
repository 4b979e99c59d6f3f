"""GPU parity of the HIP attention path against the CPU oracle, through the C ABI (libnibble_hip.so).

RoPE and the KV append are bit-exact; attention meets the tolerance in gpu_util (1e-3 max-abs, 1e-3 relative,
elementwise allclose) against the restated reference (scalar cpu::attention_heads, and the AVX2 tier where the
host has it); the causal mask is checked bitwise with NaN poison beyond each row's window.
"""
import os

import numpy as np
import pytest

import nibble_amd
import oracle
from nibble_amd import configs, synth
from tests.gpu_util import Buffers, assert_parity, bits

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "reference_vectors.npz"))

import importlib.util as _ilu  # noqa: E402

_spec = _ilu.spec_from_file_location("make_golden", os.path.join(HERE, "golden", "make_golden.py"))
make_golden = _ilu.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)


def cpu_attention(q, k, v, pos0, kv):
    """The reference's production CPU path (AVX2 tier, head-parallel) where available, else its scalar path."""
    if oracle.have_avx2():
        return oracle.attention_parallel(q, k, v, pos0, kv, threads=min(16, os.cpu_count() or 1))
    return oracle.attention_scalar(q, k, v, pos0, kv)


def gpu_attention(be, q, k, v, pos0, kv):
    """Uploads q and the caches k, v and runs Backend::attention."""
    n, H, D = q.shape
    with Buffers(be) as B:
        dq, dk, dv, do = B.upload(q), B.upload(k), B.upload(v), B.alloc(q.size)
        be.attention(dq, dk, dv, do, n, pos0, H, kv, D)
        return be.download(do, q.shape)


# ------------------------------------------------------------------------------------------------ RoPE

@pytest.mark.parametrize("case", make_golden.ROPE_CASES, ids=[c[0] for c in make_golden.ROPE_CASES])
def test_rope_bit_exact_vs_reference_vectors(backend, case):
    name, n, heads, hd, pos0, base, neox, l3 = case
    i = int(GOLD[f"rope/{name}/params"][0])
    x = make_golden.rope_input(i, n, heads, hd)
    ff = synth.llama3_freq_factors(hd, base) if l3 else None
    with Buffers(backend) as B:
        dx = B.upload(x)
        backend.rope(dx, n, heads, hd, pos0, base, neox, ff)
        y = backend.download(dx, x.shape)
    ref = oracle.rope(x.copy(), pos0, base, neox, ff)
    assert np.array_equal(bits(y), bits(ref)), f"{name}: {np.sum(bits(y) != bits(ref))} elements differ"


@pytest.mark.parametrize("shape", [configs.QWEN25_05B, configs.TINYLLAMA_11B, configs.LLAMA32_1B],
                         ids=lambda s: s.name)
def test_append_rope_bit_exact_and_rows_outside_untouched(backend, shape):
    H, KV, D = shape.n_heads, shape.n_kv_heads, shape.head_dim
    ff = shape.freq_factors()
    n_ctx, pos0, n = 600, 517, 20
    q = synth.normal_array((n, H, D), 3, 1)
    kn = synth.normal_array((n, KV, D), 3, 2)
    vn = synth.normal_array((n, KV, D), 3, 3)
    with Buffers(backend) as B:
        dq, dkn, dvn = B.upload(q), B.upload(kn), B.upload(vn)
        ck, cv = B.alloc(n_ctx * KV * D), B.alloc(n_ctx * KV * D)
        backend.append_rope(dq, ck, cv, dkn, dvn, n, pos0, H, KV, D, shape.rope_base, shape.neox, ff)
        gq = backend.download(dq, q.shape)
        gk = backend.download(ck, (n_ctx, KV, D))
        gv = backend.download(cv, (n_ctx, KV, D))
        # the same through the drop-in ops: write rows, then rope in place on the cache rows (transformer.cpp:198)
        ck2 = B.alloc(n_ctx * KV * D)
        backend.write(ck2.at(pos0 * KV * D), kn)
        backend.rope(ck2.at(pos0 * KV * D), n, KV, D, pos0, shape.rope_base, shape.neox, ff)
        gk2 = backend.download(ck2, (n_ctx, KV, D))
    assert np.array_equal(bits(gq), bits(oracle.rope(q.copy(), pos0, shape.rope_base, shape.neox, ff)))
    rk = oracle.rope(kn.copy(), pos0, shape.rope_base, shape.neox, ff)
    assert np.array_equal(bits(gk[pos0:pos0 + n]), bits(rk))
    assert np.array_equal(bits(gv[pos0:pos0 + n]), bits(vn))
    assert not np.any(bits(gk[:pos0])) and not np.any(bits(gk[pos0 + n:]))
    assert not np.any(bits(gv[:pos0])) and not np.any(bits(gv[pos0 + n:]))
    assert np.array_equal(bits(gk2), bits(gk))


# ------------------------------------------------------------------------------------------------ attention

@pytest.mark.parametrize("case", make_golden.ATTN_CASES, ids=[c[0] for c in make_golden.ATTN_CASES])
def test_attention_golden_cases(backend, case):
    name, n, pos0, H, KV, D, qs = case
    i = int(GOLD[f"attn/{name}/shape"][0])
    q, k, v = make_golden.attn_inputs(i, n, pos0, H, KV, D, qs)
    ref = oracle.attention_scalar(q, k, v, pos0, KV)
    key = f"attn/{name}/scalar"
    # the oracle reproduces the reference's vector (whole, or its SHA-256 for large outputs)
    if key in GOLD.files:
        assert np.array_equal(bits(ref), bits(GOLD[key]))
    else:
        assert np.array_equal(make_golden.sha(ref), GOLD[key + "_sha256"])
    got = gpu_attention(backend, q, k, v, pos0, KV)
    assert_parity(got, ref, name)
    if qs >= 5 and n > 16:  # scores this large leave the fp16 operand error unaveraged: tiles are recomputed
        assert backend.prefill_recomputed() > 0


LARGE_SCORE_CASES = [c for c in make_golden.ATTN_CASES if c[0].startswith(("prefill_", "chunk_"))]


@pytest.mark.parametrize("case", LARGE_SCORE_CASES, ids=[c[0] for c in LARGE_SCORE_CASES])
def test_large_scores_through_fused_append(backend, case):
    """The large-score golden shapes through append_rope_attention on the default route: q unrotated, the call's
    rows arriving as k_new / v_new (Llama-3 RoPE), cache rows [0, pos0) given. Appended rows bit-exact, outputs
    within the parity tolerance of the reference's attention over the rotated rows."""
    name, n, pos0, H, KV, D, qs = case
    i = int(GOLD[f"attn/{name}/shape"][0])
    q, k, v = make_golden.attn_inputs(i, n, pos0, H, KV, D, qs)
    base, ff = 5e5, synth.llama3_freq_factors(D, 5e5)
    kn, vn = np.ascontiguousarray(k[pos0:]), np.ascontiguousarray(v[pos0:])
    ck0, cv0 = k.copy(), v.copy()
    ck0[pos0:] = 0
    cv0[pos0:] = 0
    with Buffers(backend) as B:
        dq, dkn, dvn = B.upload(q), B.upload(kn), B.upload(vn)
        dk, dv, do = B.upload(ck0), B.upload(cv0), B.alloc(q.size)
        backend.append_rope_attention(dq, dk, dv, dkn, dvn, do, n, pos0, H, KV, D, base, False, ff)
        got = backend.download(do, q.shape)
        gk, gv = backend.download(dk, k.shape), backend.download(dv, v.shape)
        recomputed = backend.prefill_recomputed()
    kr = oracle.rope(kn.copy(), pos0, base, False, ff)
    assert np.array_equal(bits(gk[pos0:]), bits(kr)), "appended K rows"
    assert np.array_equal(bits(gv[pos0:]), bits(vn)), "appended V rows"
    assert np.array_equal(bits(gk[:pos0]), bits(k[:pos0])), "cache rows before pos0 changed"
    qr = oracle.rope(q.copy(), pos0, base, False, ff)
    ref = cpu_attention(qr, gk, gv, pos0, KV)
    assert_parity(got, ref, f"{name} fused")
    if qs >= 5:
        assert recomputed > 0


def corr_golden(case):
    """Inputs of a correlated golden case, with the oracle's output checked against the reference's vector."""
    name, n, pos0, H, KV, D, qs, rank, vmix = case
    i = int(GOLD[f"attn/{name}/shape"][0])
    q, k, v = make_golden.corr_inputs(i, n, pos0, H, KV, D, qs, rank, vmix)
    assert np.array_equal(make_golden.sha(q, k, v), GOLD[f"attn/{name}/input_sha256"]), "inputs regenerated differ"
    ref = oracle.attention_scalar(q, k, v, pos0, KV)
    key = f"attn/{name}/scalar"
    if key in GOLD.files:
        assert np.array_equal(bits(ref), bits(GOLD[key]))
    else:
        assert np.array_equal(make_golden.sha(ref), GOLD[key + "_sha256"])
    return q, k, v, ref


# On prefill_corr_r2_q05 every row tile stays on the MFMA route. An exact CPU emulation of the kernel's rounding puts
# its largest error at 8.6e-5 with the query split into fp16 high and low parts, and at 5.3e-4 with the query rounded
# to fp16 once (K and V correlate, so that rounding, shared by the row's 4096 keys, adds up): the bound below tells
# the two apart.
CORR_MAX_ABS = {"prefill_corr_r2_q05": 2.5e-4}


@pytest.mark.parametrize("case", make_golden.CORR_CASES, ids=[c[0] for c in make_golden.CORR_CASES])
def test_attention_golden_correlated(backend, case):
    """K and V projected from shared low-rank hidden states (reference vectors from the compiled reference), through
    Backend::attention on the default route: within the parity tolerance, and on the all-MFMA case within the split
    query's error level."""
    name = case[0]
    q, k, v, ref = corr_golden(case)
    got = gpu_attention(backend, q, k, v, case[2], case[4])
    p = assert_parity(got, ref, name)
    if name in CORR_MAX_ABS:
        assert p["max_abs"] <= CORR_MAX_ABS[name], p
    if name.startswith("prefill_corr_r1"):
        assert backend.prefill_recomputed() > 0


@pytest.mark.parametrize("case", make_golden.CORR_CASES, ids=[c[0] for c in make_golden.CORR_CASES])
def test_attention_golden_correlated_through_fused_append(backend, case):
    """The correlated cases through append_rope_attention: the call's rows arrive as k_new / v_new and are rotated
    (Llama-3 RoPE) into the cache, q is rotated on load; appended rows bit-exact, outputs within the parity tolerance
    of the reference's attention over the rotated rows."""
    name, n, pos0, H, KV, D = case[:6]
    q, k, v, _ = corr_golden(case)
    base, ff = 5e5, synth.llama3_freq_factors(D, 5e5)
    kn, vn = np.ascontiguousarray(k[pos0:]), np.ascontiguousarray(v[pos0:])
    ck0, cv0 = k.copy(), v.copy()
    ck0[pos0:] = 0
    cv0[pos0:] = 0
    with Buffers(backend) as B:
        dq, dkn, dvn = B.upload(q), B.upload(kn), B.upload(vn)
        dk, dv, do = B.upload(ck0), B.upload(cv0), B.alloc(q.size)
        backend.append_rope_attention(dq, dk, dv, dkn, dvn, do, n, pos0, H, KV, D, base, False, ff)
        got = backend.download(do, q.shape)
        gk, gv = backend.download(dk, k.shape), backend.download(dv, v.shape)
    assert np.array_equal(bits(gk[pos0:]), bits(oracle.rope(kn.copy(), pos0, base, False, ff))), "appended K rows"
    assert np.array_equal(bits(gv[pos0:]), bits(vn)), "appended V rows"
    qr = oracle.rope(q.copy(), pos0, base, False, ff)
    assert_parity(got, cpu_attention(qr, gk, gv, pos0, KV), f"{name} fused")


def repeat_golden(case):
    """Inputs of a repeated-value golden case, with the oracle's output checked against the reference's vector."""
    name, n, pos0, H, KV, D = case[:6]
    i = int(GOLD[f"attn/{name}/shape"][0])
    q, k, v = make_golden.repeat_inputs(i, *case[1:])
    assert np.array_equal(make_golden.sha(q, k, v), GOLD[f"attn/{name}/input_sha256"]), "inputs regenerated differ"
    ref = oracle.attention_scalar(q, k, v, pos0, KV)
    assert np.array_equal(make_golden.sha(ref), GOLD[f"attn/{name}/scalar_sha256"])
    return q, k, v, ref


@pytest.mark.parametrize("case", make_golden.REPEAT_CASES, ids=[c[0] for c in make_golden.REPEAT_CASES])
def test_attention_golden_repeated_values(backend, case):
    """Equal value rows whose large elements sit 0.1-0.49 fp16 ulp off the grid (reference vectors from the compiled
    reference): rounded to nearest, the rows' shared rounding error (1.9e-3) would reach every output; the staging's
    stochastic rounding makes the rows' errors independent, so they average out. Within the parity tolerance; on
    `repeat_const_chunk` (every V row equal, 64 rows on the key-split route, every row kept by the estimate in the
    CPU emulation) nothing is recomputed and the MFMA route's own output is within 5e-4."""
    name, n, pos0, H, KV, D = case[:6]
    q, k, v, ref = repeat_golden(case)
    got = gpu_attention(backend, q, k, v, pos0, KV)
    recomputed = backend.prefill_recomputed()
    p = assert_parity(got, ref, name)
    if name == "repeat_const_chunk":
        assert recomputed == 0, recomputed
        assert p["max_abs"] <= 5e-4, p


def test_stochastic_staging_matches_its_restatement(backend):
    """The staging's stochastic rounding as the CPU restates it (tests/test_error_estimate.py: the kernel's hash and
    bit manipulation, then the MFMA route's arithmetic in float64) predicts the GPU's output on `repeat_const_chunk`
    (every V row equal, so each output is the weighted mean of that row's stochastic roundings): the GPU stays within
    3e-5 of the emulated rows while both are ~2.5e-4 from the reference, and rounding V to nearest instead would put
    every large element 0.1-0.49 ulp (up to 1.9e-3) off. A different hash, bit field or position key would leave
    differences the size of the error itself."""
    from tests import test_error_estimate as est
    case = next(c for c in make_golden.REPEAT_CASES if c[0] == "repeat_const_chunk")
    name, n, pos0, H, KV, D = case[:6]
    q, k, v, ref = repeat_golden(case)
    got = gpu_attention(backend, q, k, v, pos0, KV)
    assert backend.prefill_recomputed() == 0
    g = H // KV
    emu = np.empty(ref.shape, np.float64)
    for r in range(n):
        for h in range(H):
            ctx = pos0 + r + 1
            emu[r, h] = est.emulate(q[r, h].astype(np.float64), k[:ctx, h // g].astype(np.float64),
                                    v[:ctx, h // g].astype(np.float64), g=h // g)[4]
    d_emu = float(np.max(np.abs(got - emu)))
    d_ref = float(np.max(np.abs(got - ref)))
    print(f"{name}: |gpu - emulation| {d_emu:.2e}, |gpu - reference| {d_ref:.2e}", flush=True)
    assert d_emu <= 3e-5 and d_ref > 4 * d_emu, (d_emu, d_ref)


def layer0_prompt(seed, n_tok, vocab, KV, D, vmax):
    """A first layer's K and V for a prompt over a small vocabulary (Zipf-distributed token ids): each token's
    hidden state is its embedding, so K rows (before RoPE) and V rows repeat exactly wherever the token recurs. V is
    scaled so that its largest element is vmax."""
    rng = np.random.default_rng(seed)
    dm = 4 * D
    emb = rng.standard_normal((vocab, dm))
    toks = np.minimum(rng.zipf(1.3, n_tok) - 1, vocab - 1)
    wk = rng.standard_normal((dm, KV * D)) / np.sqrt(dm)
    wv = 0.5 * wk + 0.5 * rng.standard_normal((dm, KV * D)) / np.sqrt(dm)
    k = (emb[toks] @ wk).reshape(n_tok, KV, D)
    v = (emb[toks] @ wv).reshape(n_tok, KV, D)
    v *= vmax / np.abs(v).max()
    return toks, k.astype(np.float32), v.astype(np.float32)


@pytest.mark.parametrize("vmax", [2.0, 6.0])
def test_repeated_tokens_of_a_first_layer(backend, vmax):
    """A 2048-token prompt over a 40-token vocabulary through append_rope_attention in four 512-row chunks (Llama-3
    RoPE on q and the new keys): every V row of a token is the same wherever it recurs, the keys differ only by
    their rotation, and the query of a row is its own token's projection. Rounded to nearest, such values would
    carry one error per token into the weighted mean; the stochastic staging keeps each chunk within the parity
    tolerance of the reference over the rotated rows."""
    H, KV, D, n, c = 32, 8, 64, 2048, 512
    base, ff = 5e5, synth.llama3_freq_factors(D, 5e5)
    toks, kn, vn = layer0_prompt(int(vmax * 10), n, 40, KV, D, vmax)
    rng = np.random.default_rng(5)
    dm = 4 * D
    emb = np.random.default_rng(int(vmax * 10)).standard_normal((40, dm))
    wq = rng.standard_normal((dm, H * D)) / np.sqrt(dm)
    q = (emb[toks] @ wq).reshape(n, H, D).astype(np.float32)
    with Buffers(backend) as B:
        dq, dkn, dvn = B.upload(q), B.upload(kn), B.upload(vn)
        dk, dv, do = B.alloc(n * KV * D), B.alloc(n * KV * D), B.alloc(q.size)
        for p0 in range(0, n, c):
            print(f"chunk pos0={p0}", flush=True)
            backend.append_rope_attention(dq.at(p0 * H * D), dk, dv, dkn.at(p0 * KV * D), dvn.at(p0 * KV * D),
                                          do.at(p0 * H * D), c, p0, H, KV, D, base, False, ff)
        got = backend.download(do, q.shape)
        gk, gv = backend.download(dk, kn.shape), backend.download(dv, vn.shape)
    assert np.array_equal(bits(gk), bits(oracle.rope(kn.copy(), 0, base, False, ff))), "appended K rows"
    assert np.array_equal(bits(gv), bits(vn)), "appended V rows"
    qr = oracle.rope(q.copy(), 0, base, False, ff)
    for p0 in range(0, n, c):
        ref = cpu_attention(qr[p0:p0 + c], gk[:p0 + c], gv[:p0 + c], p0, KV)
        assert_parity(got[p0:p0 + c], ref, f"vmax={vmax} chunk {p0}")


@pytest.mark.parametrize("mag", [10.0, 20.0, 40.0])
def test_keys_with_outlier_channels(backend, mag):
    """Keys sharing two channels of magnitude `mag` (+-20 %) that the query also weights (channels LLM keys carry),
    512 rows deep in a 2048-row cache: within the parity tolerance of the reference."""
    H, KV, D, n, pos0 = 32, 8, 64, 512, 1536
    rng = np.random.default_rng(int(mag))
    q = rng.standard_normal((n, H, D)).astype(np.float32)
    k = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
    v = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
    dims = [5, 37]
    k[:, :, dims] = (mag * (1 + 0.2 * rng.standard_normal((pos0 + n, KV, 2)))).astype(np.float32)
    q[:, :, dims] = (mag / 8 * rng.choice([-1, 1], (n, H, 2))).astype(np.float32)
    got = gpu_attention(backend, q, k, v, pos0, KV)
    assert_parity(got, cpu_attention(q, k, v, pos0, KV), f"outlier channels x{mag}")


@pytest.mark.parametrize("qscale", [1e-4, 1e-2])
def test_flat_scores_with_correlated_values(backend, qscale):
    """A near-zero query (nearly uniform attention, scores spanning less than one fp16 step of the weights) over K
    and V projected from shared rank-1 hidden states with values up to 10: the weights' rounding correlates with V;
    within the parity tolerance of the reference."""
    H, KV, D, n, pos0 = 32, 8, 64, 512, 1536
    rng = np.random.default_rng(int(1 / qscale))
    ctx, dm = pos0 + n, 4 * D
    h = np.outer(rng.standard_normal(ctx), rng.standard_normal(dm)) + 0.01 * rng.standard_normal((ctx, dm))
    wk = rng.standard_normal((dm, KV * D)) / np.sqrt(dm)
    k = (h @ wk).reshape(ctx, KV, D)
    v = (h @ wk).reshape(ctx, KV, D)
    v = (v * (10.0 / np.abs(v).max())).astype(np.float32)
    k = k.astype(np.float32)
    q = (rng.standard_normal((n, H, D)) * qscale).astype(np.float32)
    got = gpu_attention(backend, q, k, v, pos0, KV)
    assert_parity(got, cpu_attention(q, k, v, pos0, KV), f"flat scores q x {qscale}")


def structured_case(seed):
    """One seeded mix of the structures the prefill route's error estimate must cover: query scale 1e-3 .. 10, keys
    N(0,1) / from shared low-rank hidden states / with two outlier channels, values N(0,1) / correlated with the keys
    / repeated in runs / offset by 3 / scaled by 8, at several depths, head groupings and head sizes."""
    rng = np.random.default_rng(1000 + seed)
    H, KV = [(32, 8), (14, 2), (8, 2)][seed % 3]
    D = (64, 128)[(seed // 3) % 2]
    n = int(rng.choice([160, 256, 512]))
    pos0 = int(rng.choice([0, 384, 1536]))
    ctx, dm = pos0 + n, 4 * D
    qs = float(rng.choice([1e-3, 0.3, 1.0, 3.0, 10.0]))
    kkind = rng.choice(["n01", "lowrank", "outlier"])
    vkind = rng.choice(["n01", "corr", "runs", "offset", "big"])
    h = rng.standard_normal((ctx, 2)) @ rng.standard_normal((2, dm)) + 0.1 * rng.standard_normal((ctx, dm))
    wk = rng.standard_normal((dm, KV * D)) / np.sqrt(dm)
    k = (h @ wk if kkind == "lowrank" else rng.standard_normal((ctx, KV * D))).reshape(ctx, KV, D)
    if kkind == "outlier":
        k[:, :, [3, 17]] += 12.0
    if vkind == "corr":
        v = (h @ (0.8 * wk + 0.2 * rng.standard_normal((dm, KV * D)) / np.sqrt(dm))).reshape(ctx, KV, D)
    else:
        v = rng.standard_normal((ctx, KV, D))
    if vkind == "runs":
        for s0 in rng.integers(0, ctx - 32, 8):
            v[s0:s0 + 32] = v[s0]
    elif vkind == "offset":
        v = v + 3.0
    elif vkind == "big":
        v = v * 8.0
    q = rng.standard_normal((n, H, D)) * qs
    if kkind == "outlier":
        q[:, :, [3, 17]] += 1.5 * np.sign(rng.standard_normal((n, H, 2)))
    name = f"seed{seed}: H{H}/KV{KV} D{D} n{n} pos0 {pos0} q x {qs} K {kkind} V {vkind}"
    return name, q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), pos0, KV


@pytest.mark.parametrize("seed", range(24))
def test_structured_inputs_sweep(backend, seed):
    """Seeded mixes of query scale, key and value structure, depth and head shape (structured_case) through
    Backend::attention on the default route: within the parity tolerance of the reference."""
    name, q, k, v, pos0, KV = structured_case(seed)
    print(name, flush=True)
    got = gpu_attention(backend, q, k, v, pos0, KV)
    assert_parity(got, cpu_attention(q, k, v, pos0, KV), name)


@pytest.mark.parametrize("case", make_golden.REPEAT_CASES, ids=[c[0] for c in make_golden.REPEAT_CASES])
def test_attention_golden_repeated_values_through_fused_append(backend, case):
    """The repeated-value cases through append_rope_attention (Llama-3 RoPE on q and the new keys; V rows are
    appended unrotated, so they stay equal): appended rows bit-exact, outputs within the parity tolerance."""
    name, n, pos0, H, KV, D = case[:6]
    q, k, v, _ = repeat_golden(case)
    base, ff = 5e5, synth.llama3_freq_factors(D, 5e5)
    kn, vn = np.ascontiguousarray(k[pos0:]), np.ascontiguousarray(v[pos0:])
    ck0, cv0 = k.copy(), v.copy()
    ck0[pos0:] = 0
    cv0[pos0:] = 0
    with Buffers(backend) as B:
        dq, dkn, dvn = B.upload(q), B.upload(kn), B.upload(vn)
        dk, dv, do = B.upload(ck0), B.upload(cv0), B.alloc(q.size)
        backend.append_rope_attention(dq, dk, dv, dkn, dvn, do, n, pos0, H, KV, D, base, False, ff)
        got = backend.download(do, q.shape)
        gk, gv = backend.download(dk, k.shape), backend.download(dv, v.shape)
    assert np.array_equal(bits(gk[pos0:]), bits(oracle.rope(kn.copy(), pos0, base, False, ff))), "appended K rows"
    assert np.array_equal(bits(gv[pos0:]), bits(vn)), "appended V rows"
    qr = oracle.rope(q.copy(), pos0, base, False, ff)
    assert_parity(got, cpu_attention(qr, gk, gv, pos0, KV), f"{name} fused")


@pytest.mark.parametrize("D", [2, 8, 13, 16, 24, 64, 128])
@pytest.mark.parametrize("H,KV", [(4, 4), (6, 3), (8, 2), (14, 2), (32, 4), (16, 1)])
def test_attention_head_shapes(backend, D, H, KV):
    rng = np.random.default_rng(D * 131 + H * 7 + KV)
    for n, pos0 in [(1, 0), (1, 77), (3, 50), (40, 0), (37, 300)]:
        q = rng.standard_normal((n, H, D)).astype(np.float32)
        k = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
        v = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
        assert_parity(gpu_attention(backend, q, k, v, pos0, KV), oracle.attention_scalar(q, k, v, pos0, KV),
                      f"D={D} H={H} KV={KV} n={n} pos0={pos0}")


def test_config1_qwen_decode(backend):
    """Qwen shape, one layer, one token at position 512 over 512 cached rows."""
    s = configs.QWEN25_05B
    H, KV, D, pos0 = s.n_heads, s.n_kv_heads, s.head_dim, 512
    cache_k = synth.normal_array((pos0, KV, D), 1, 0, configs.T_KCACHE)
    cache_v = synth.normal_array((pos0, KV, D), 1, 0, configs.T_VCACHE)
    q = synth.normal_array((1, H, D), 1, 0, configs.T_Q)
    kn = synth.normal_array((1, KV, D), 1, 0, configs.T_K)
    vn = synth.normal_array((1, KV, D), 1, 0, configs.T_V)
    with Buffers(backend) as B:
        ck, cv = B.alloc((pos0 + 1) * KV * D), B.alloc((pos0 + 1) * KV * D)
        backend.write(ck, cache_k)
        backend.write(cv, cache_v)
        dq, dkn, dvn, do = B.upload(q), B.upload(kn), B.upload(vn), B.alloc(H * D)
        backend.append_rope(dq, ck, cv, dkn, dvn, 1, pos0, H, KV, D, s.rope_base, s.neox, None)
        backend.attention(dq, ck, cv, do, 1, pos0, H, KV, D)
        got = backend.download(do, (1, H, D))
        gk = backend.download(ck, (pos0 + 1, KV, D))
    qr = oracle.rope(q.copy(), pos0, s.rope_base, s.neox)
    kr = oracle.rope(kn.copy(), pos0, s.rope_base, s.neox)
    assert np.array_equal(bits(gk[pos0]), bits(kr[0]))
    k_all = np.concatenate([cache_k, kr])
    v_all = np.concatenate([cache_v, vn])
    ref = oracle.attention_scalar(qr, k_all, v_all, pos0, KV)
    assert_parity(got, ref, "config1 vs scalar")
    if oracle.have_avx2():
        assert_parity(got, oracle.attention_avx2(qr, k_all, v_all, pos0, KV), "config1 vs avx2")
    assert_parity(got, oracle.attention_f64(qr, k_all, v_all, pos0, KV), "config1 vs fp64")


@pytest.mark.parametrize("n,pos0", [(1, 0), (1, 63), (1, 4095), (2, 1000), (7, 333), (16, 2500), (17, 10),
                                    (300, 0), (600, 100), (1024, 0)])
def test_causal_mask_poison(backend, n, pos0):
    """Rows past the causal window (and past the context) are NaN: the result must be finite and bitwise equal
    to the run without poison (decode, fp32-prefix and MFMA paths)."""
    H, KV, D = 32, 8, 64
    q = synth.normal_array((n, H, D), 7, n, pos0, 1)
    k = synth.normal_array((pos0 + n, KV, D), 7, n, pos0, 2)
    v = synth.normal_array((pos0 + n, KV, D), 7, n, pos0, 3)
    clean = gpu_attention(backend, q, k, v, pos0, KV)
    # Poison inside the window of later rows cannot be used (they legitimately see it); poison only rows > ctx.
    with Buffers(backend) as B:
        pad = 200
        kp = np.concatenate([k, np.full((pad, KV, D), np.nan, np.float32)])
        vp = np.concatenate([v, np.full((pad, KV, D), np.nan, np.float32)])
        dq, dk, dv, do = B.upload(q), B.upload(kp), B.upload(vp), B.alloc(q.size)
        backend.attention(dq, dk, dv, do, n, pos0, H, KV, D)
        poisoned = backend.download(do, q.shape)
    assert np.all(np.isfinite(poisoned))
    assert np.array_equal(bits(clean), bits(poisoned))
    # Per-row poison: row t of a separate single-row call at position pos0+t sees NaN right after its window.
    rng = np.random.default_rng(n + pos0)
    for t in sorted(set(rng.integers(0, n, 3).tolist())):
        with Buffers(backend) as B:
            L = pos0 + t + 1
            kp = np.concatenate([k[:L], np.full((5, KV, D), np.nan, np.float32)])
            vp = np.concatenate([v[:L], np.full((5, KV, D), np.nan, np.float32)])
            dq, dk, dv, do = B.upload(q[t:t + 1]), B.upload(kp), B.upload(vp), B.alloc(H * D)
            backend.attention(dq, dk, dv, do, 1, pos0 + t, H, KV, D)
            row = backend.download(do, (1, H, D))
        assert np.all(np.isfinite(row))
    assert_parity(clean, cpu_attention(q, k, v, pos0, KV), f"poison case n={n} pos0={pos0}")


def test_long_recomputation_list(backend):
    """A 4352-row prefill at q x 30 (scores ~30 log2) lists nearly every MFMA row tile (at most 1056 of the call's
    1088: rows 0..127 run in fp32) - more than the precise kernel keeps in registers while it schedules (1024), and
    more units than workgroups, so its schedule scans the list in several chunks and each workgroup takes several
    units. Sampled row blocks across the call (the oracle over those rows alone: same keys, pos0 moved to the block)
    are within the parity tolerance."""
    H, KV, D, n = 32, 8, 64, 4352
    rng = np.random.default_rng(4352)
    q = (rng.standard_normal((n, H, D)) * 30).astype(np.float32)
    k = rng.standard_normal((n, KV, D)).astype(np.float32)
    v = rng.standard_normal((n, KV, D)).astype(np.float32)
    got = gpu_attention(backend, q, k, v, 0, KV)
    recomputed = backend.prefill_recomputed()
    assert 1024 < recomputed <= (n - 128) * (H // KV) // 128 * KV, recomputed
    for r0, r1 in ((128, 160), (1500, 1532), (3000, 3016), (4320, 4352)):
        ref = cpu_attention(q[r0:r1], k[:r1], v[:r1], r0, KV)
        assert_parity(got[r0:r1], ref, f"rows {r0}..{r1}")


def test_prefill_chunks_match_one_call_and_repeat_bitwise(backend):
    """A prefill split into max_batch chunks (transformer.cpp:135-136) matches one call within tolerance: short
    chunks split each row's keys over several workgroups to fill the chip, and the merged rows differ from the
    unsplit ones in rounding only. Every call is deterministic: repeating the chunked pass reproduces its bits."""
    H, KV, D, n = 32, 8, 64, 1536
    q = synth.normal_array((n, H, D), 8, 1)
    k = synth.normal_array((n, KV, D), 8, 2)
    v = synth.normal_array((n, KV, D), 8, 3)
    with Buffers(backend) as B:
        dq, dk, dv = B.upload(q), B.upload(k), B.upload(v)
        whole, parts, again = B.alloc(q.size), B.alloc(q.size), B.alloc(q.size)
        backend.attention(dq, dk, dv, whole, n, 0, H, KV, D)
        for dst in (parts, again):
            for off in range(0, n, 512):
                backend.attention(dq.at(off * H * D), dk, dv, dst.at(off * H * D), 512, off, H, KV, D)
        a = backend.download(whole, q.shape)
        b = backend.download(parts, q.shape)
        c = backend.download(again, q.shape)
    assert np.array_equal(bits(b), bits(c))
    ref = cpu_attention(q, k, v, 0, KV)
    assert_parity(a, ref, "prefill 1536 in one call")
    assert_parity(b, ref, "prefill 1536 in 512-row chunks")
    assert_parity(b, a, "chunks vs one call")


def test_small_chunks_match_batch_within_tolerance(backend):
    """Incremental (n=1), 2-token chunks and one batch agree within tolerance (the reference requires bitwise
    equality of its CPU paths, test_model.cpp:141-151; here n <= 16 calls take the fp32 kernel and larger batches
    the fp16-operand MFMA kernel)."""
    H, KV, D, n = 14, 2, 64, 300
    q = synth.normal_array((n, H, D), 9, 1)
    k = synth.normal_array((n, KV, D), 9, 2)
    v = synth.normal_array((n, KV, D), 9, 3)
    with Buffers(backend) as B:
        dq, dk, dv = B.upload(q), B.upload(k), B.upload(v)
        whole, ones, twos = B.alloc(q.size), B.alloc(q.size), B.alloc(q.size)
        backend.attention(dq, dk, dv, whole, n, 0, H, KV, D)
        for t in range(n):
            backend.attention(dq.at(t * H * D), dk, dv, ones.at(t * H * D), 1, t, H, KV, D)
        for t in range(0, n, 2):
            backend.attention(dq.at(t * H * D), dk, dv, twos.at(t * H * D), 2, t, H, KV, D)
        a, b, c = (backend.download(x, q.shape) for x in (whole, ones, twos))
    ref = oracle.attention_scalar(q, k, v, 0, KV)
    for got, what in ((a, "batch"), (b, "one-by-one"), (c, "2-token chunks")):
        assert_parity(got, ref, what)


@pytest.mark.parametrize("n,pos0", [(512, 4096), (1024, 7168)])
def test_long_context_chunk_every_row_diffuse(backend, n, pos0):
    """A prefill chunk whose every row sees thousands of keys, as nibble's Transformer runs a long prompt
    (max_batch rows per call, transformer.cpp:135-136): N(0,1) data at Llama-3.2 shape, the whole [n, 32, 64] output
    against the oracle. Each output is a long average, so the fp16 operand rounding (rms relative ~4.3e-4) is the
    whole error and no row tile goes to the recomputation; the infinity-norm ratio is printed, not gated (it reaches
    ~1e-3 on outputs this many and this small). A structural error (a wrong key, shift or normaliser) would be
    orders of magnitude above the rel_l2 ceiling asserted here."""
    H, KV, D = 32, 8, 64
    q, k, v = make_golden.attn_inputs(40 + n // 512, n, pos0, H, KV, D, 1.0)
    ref = cpu_attention(q, k, v, pos0, KV)
    got = gpu_attention(backend, q, k, v, pos0, KV)
    p = assert_parity(got, ref, f"chunk n={n} pos0={pos0}")
    assert p["rel_l2"] <= 6e-4


# ------------------------------------------------------------------------------------------------ full-size configs

def test_config4_prefill_8k_one_layer_sampled_rows(backend):
    """Config 4 prefill at its full size (8192 tokens, Llama-3.2 shape) for layer 0: RoPE'd K rows land in the cache
    bit-exactly; attention output checked against the oracle on a sample of rows spread over the sequence."""
    s = configs.LLAMA32_1B
    H, KV, D, n = s.n_heads, s.n_kv_heads, s.head_dim, 8192
    ff = s.freq_factors()
    q = synth.normal_array((n, H, D), 4, 0, configs.T_Q)
    kn = synth.normal_array((n, KV, D), 4, 0, configs.T_K)
    vn = synth.normal_array((n, KV, D), 4, 0, configs.T_V)
    with Buffers(backend) as B:
        dq, dkn, dvn = B.upload(q), B.upload(kn), B.upload(vn)
        ck, cv, do = B.alloc(n * KV * D), B.alloc(n * KV * D), B.alloc(q.size)
        backend.append_rope(dq, ck, cv, dkn, dvn, n, 0, H, KV, D, s.rope_base, s.neox, ff)
        backend.attention(dq, ck, cv, do, n, 0, H, KV, D)
        got = backend.download(do, q.shape)
        gk = backend.download(ck, kn.shape)
        gq = backend.download(dq, q.shape)
    kr = oracle.rope(kn.copy(), 0, s.rope_base, s.neox, ff)
    qr = oracle.rope(q.copy(), 0, s.rope_base, s.neox, ff)
    assert np.array_equal(bits(gk), bits(kr)) and np.array_equal(bits(gq), bits(qr))
    rows = sorted(set([0, 1, 2, 63, 64, 127, 255, 256, 257, 511, 4095, 4096, 8190, 8191] +
                      np.random.default_rng(4).integers(0, n, 40).tolist()))
    for t in rows:
        ref = cpu_attention(qr[t:t + 1], kr[:t + 1], vn[:t + 1], t, KV)
        assert_parity(got[t:t + 1], ref, f"prefill row {t}")


def test_config4_decode_32k(backend):
    """Config 4 decode: one layer, 32768-row cache (rows 0..8191 from the prefill stream, rest seeded), one new token
    appended at 32768 and attended; two more steps."""
    s = configs.LLAMA32_1B
    H, KV, D, ctx = s.n_heads, s.n_kv_heads, s.head_dim, 32768
    ff = s.freq_factors()
    cache_k = synth.normal_array((ctx, KV, D), 4, 0, configs.T_KCACHE)
    cache_v = synth.normal_array((ctx, KV, D), 4, 0, configs.T_VCACHE)
    with Buffers(backend) as B:
        cap = ctx + 64
        ck, cv = B.alloc(cap * KV * D), B.alloc(cap * KV * D)
        backend.write(ck, cache_k)
        backend.write(cv, cache_v)
        k_all, v_all = cache_k, cache_v
        for step in range(3):
            pos0 = ctx + step
            q = synth.normal_array((1, H, D), 4, 0, 100 + step, configs.T_Q)
            kn = synth.normal_array((1, KV, D), 4, 0, 100 + step, configs.T_K)
            vn = synth.normal_array((1, KV, D), 4, 0, 100 + step, configs.T_V)
            dq, dkn, dvn, do = B.upload(q), B.upload(kn), B.upload(vn), B.alloc(H * D)
            backend.append_rope(dq, ck, cv, dkn, dvn, 1, pos0, H, KV, D, s.rope_base, s.neox, ff)
            backend.attention(dq, ck, cv, do, 1, pos0, H, KV, D)
            got = backend.download(do, (1, H, D))
            kr = oracle.rope(kn.copy(), pos0, s.rope_base, s.neox, ff)
            qr = oracle.rope(q.copy(), pos0, s.rope_base, s.neox, ff)
            row = backend.download(ck.at(pos0 * KV * D), (1, KV, D))
            assert np.array_equal(bits(row), bits(kr))
            k_all = np.concatenate([k_all, kr])
            v_all = np.concatenate([v_all, vn])
            assert_parity(got, cpu_attention(qr, k_all, v_all, pos0, KV), f"decode step {step} @ {pos0}")


# ------------------------------------------------------------------------------------------------ boundary behaviour

def test_out_of_range_arguments_raise_before_launch(backend):
    import nibble_amd

    H, KV, D = 8, 2, 64
    with Buffers(backend) as B:
        q, out = B.alloc(H * D), B.alloc(H * D)
        k, v = B.alloc(100 * KV * D), B.alloc(100 * KV * D)
        backend.attention(q, k, v, out, 1, 99, H, KV, D)  # exactly fits
        with pytest.raises(nibble_amd.BackendError, match="not inside"):
            backend.attention(q, k, v, out, 1, 100, H, KV, D)  # needs 101 rows
        with pytest.raises(nibble_amd.BackendError, match="not inside"):
            backend.attention(q, k, v, out, 2, 0, H, KV, D)  # q too short for 2 rows
        with pytest.raises(nibble_amd.BackendError, match="multiple"):
            backend.attention(q, k, v, out, 1, 0, 6, 4, D)
        with pytest.raises(nibble_amd.BackendError, match="even"):
            backend.rope(q, 1, H, 63, 0, 1e4, False)
        with pytest.raises(nibble_amd.BackendError, match="not inside"):
            backend.rope(q.at(1), 1, H, D, 0, 1e4, False)
        host = np.zeros(10, np.float32)
        with pytest.raises(nibble_amd.BackendError):
            backend.read(0x1000, 10, host)
        backend.sync()


def test_alloc_free_bookkeeping(backend):
    base = backend.live_allocations()
    a = backend.alloc(100)
    assert backend.live_allocations() == base + 1
    assert not np.any(backend.read(a, 100))  # zeroed
    backend.free(a)
    backend.free(None)
    backend.free(a)  # unknown now: ignored
    assert backend.live_allocations() == base


def test_reserve_prevents_workspace_growth(backend):
    """After reserve() and reserve_attention(), decode at every position up to n_ctx and prefill chunks allocate
    nothing (the HIP counterpart of test_cpu_backend.cpp:89-103)."""
    import nibble_amd

    be = nibble_amd.HipBackend(0)
    try:
        H, KV, D, n_ctx = 32, 8, 64, 4096
        be.reserve(n_ctx, H, 512, 2048)
        be.reserve_attention(KV, D)
        be.reserve_rope(D, 5e5, False, synth.llama3_freq_factors(D, 5e5))
        cap = be.internal_bytes()
        q, out = be.alloc(512 * H * D), be.alloc(512 * H * D)
        k, v = be.alloc(n_ctx * KV * D), be.alloc(n_ctx * KV * D)
        for pos in list(range(0, 64)) + list(range(64, n_ctx, 97)) + [n_ctx - 1]:
            be.attention(q, k, v, out, 1, pos, H, KV, D)
            be.rope(q, 1, H, D, pos, 5e5, False, synth.llama3_freq_factors(D, 5e5))
        for off in range(0, n_ctx, 512):
            be.attention(q, k, v, out, 512, off, H, KV, D)
        be.sync()
        assert be.internal_bytes() == cap
    finally:
        be.close()


def test_reserve_covers_every_op_at_its_limits():
    """backend.h:42-45 (and alloc_tests.cpp:278-337): after reserve() alone - no HIP-only pre-sizing call - ops at
    the reserved limits allocate nothing: quantized matmul_multi of every type at n = max_rows and width max_width
    (row-chunked and tiled routes, every activation format), embed of max_rows ids from a quantized table, an F16
    weight inside an allocated buffer at n = max_rows, overlapping copies larger than the bounce buffer, RoPE and the
    MFMA prefill route. internal_bytes() stays what reserve() left."""
    import nibble_amd
    from tests import quant_util as U

    be = nibble_amd.HipBackend(0)
    try:
        max_rows, width, n_ctx, H, KV, D = 512, 512, 2048, 8, 2, 64
        be.reserve(n_ctx, H, max_rows, width)
        cap = be.internal_bytes()
        x, y = be.alloc(max_rows * width), be.alloc(max_rows * 3 * 256)
        be.fill_normal(x, max_rows * width, 5, 0.5)
        for t in [oracle.Q4_0, oracle.Q5_0, oracle.Q5_1, oracle.Q8_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K]:
            ws = [U.random_qmat(t, 256, width, 10 * t + i).nbh_tensor() for i in range(3)]
            for n in (1, 5, 16, 100, max_rows):
                be.matmul_multi(ws, x, [y, y.at(n * 256), y.at(2 * n * 256)], n)
            be.sync()
            assert be.internal_bytes() == cap, U.NAMES[t]
        emb = U.random_qmat(oracle.Q8_0, 300, width, 3).nbh_tensor()
        be.embed(emb, np.arange(max_rows, dtype=np.int32) % 300, x)
        w16 = be.alloc(256 * width // 2)  # a 256 x width F16 weight in an allocated buffer
        be.matmul(w16, x, y, max_rows, shape=(256, width), dtype=nibble_amd.F16)
        big = be.alloc(3 * (1 << 20))
        be.copy(big.at(5), big, 2 * (1 << 20) + 7)  # moving up, 2M floats through the 1M-float bounce buffer
        be.copy(big, big.at(3), 2 * (1 << 20))      # moving down
        q, out = be.alloc(max_rows * H * D), be.alloc(max_rows * H * D)
        k, v = be.alloc(n_ctx * KV * D), be.alloc(n_ctx * KV * D)
        for pos0 in range(0, n_ctx, max_rows):  # chunked prefill, rows >= 128 on the MFMA route
            be.rope(q, max_rows, H, D, pos0, 5e5, False, synth.llama3_freq_factors(D, 5e5))
            be.attention(q, k, v, out, max_rows, pos0, H, KV, D)
        be.attention(q, k, v, out, 1, n_ctx - 1, H, KV, D)
        be.sync()
        assert be.internal_bytes() == cap
        for p in (x, y, w16, big, q, out, k, v):
            be.free(p)
    finally:
        be.close()


@pytest.mark.parametrize("max_rows,H,KV", [(200, 32, 32), (200, 32, 8), (100, 32, 32), (300, 14, 2), (129, 8, 1)])
def test_reserve_covers_the_prefill_work_list_for_any_kv_heads(max_rows, H, KV):
    """The prefill work list reserve() allocates serves calls of up to max_rows rows whatever the KV head count (one
    word per row tile and KV head: n_kv ceil(n G / 128)); the shapes where one KV head is not the worst case (max_rows
    * G not a multiple of 128) allocate nothing after reserve()."""
    import nibble_amd

    be = nibble_amd.HipBackend(0)
    try:
        D, n_ctx = 64, 1024
        be.reserve(n_ctx, H, max_rows, H * D)
        cap = be.internal_bytes()
        q, out = be.alloc(max_rows * H * D), be.alloc(max_rows * H * D)
        k, v = be.alloc(n_ctx * KV * D), be.alloc(n_ctx * KV * D)
        be.fill_normal(q, max_rows * H * D, 3, 1.0)
        be.fill_normal(k, n_ctx * KV * D, 4, 1.0)
        be.fill_normal(v, n_ctx * KV * D, 5, 1.0)
        for n, pos0 in [(max_rows, 128), (max_rows, n_ctx - max_rows), (max_rows // 2 + 17, 300)]:
            be.attention(q, k, v, out, n, pos0, H, KV, D)
        be.sync()
        assert be.internal_bytes() == cap
        for p_ in (q, out, k, v):
            be.free(p_)
    finally:
        be.close()


def test_rope_table_growing_within_the_slab_keeps_it():
    """A RoPE table living in the slab reserve() sized (n_ctx x max_width / n_heads floats) that grows past n_ctx
    but still fits the slab stays in it: no allocation, and the rotation at the new positions is bit-exact."""
    import nibble_amd

    be = nibble_amd.HipBackend(0)
    try:
        H, D, n_ctx = 8, 64, 1024
        be.reserve(n_ctx, H, 64, 4 * H * D)  # the slab holds 4 n_ctx rows of a head_dim-64 table
        cap = be.internal_bytes()
        x = synth.normal_array((2, H, D), 7, 1)
        with Buffers(be) as B:
            for pos0 in (100, 1500, 3000):  # 1500 and 3000 grow the table, to 2048 and then 4096 rows
                dx = B.upload(x)
                be.rope(dx, 2, H, D, pos0, 1e4, False, None)
                y = be.download(dx, x.shape)
                assert np.array_equal(bits(y), bits(oracle.rope(x.copy(), pos0, 1e4, False, None))), pos0
                be.sync()
                assert be.internal_bytes() == cap, pos0
    finally:
        be.close()


@pytest.mark.parametrize("count,src_off,dst_off", [(1, 0, 0), (5, 1, 3), (1000, 0, 0), (1003, 2, 1), (4097, 4, 8),
                                                   (262147, 0, 4), (262147, 3, 0)])
def test_copy_exact_and_neighbours_untouched(backend, count, src_off, dst_off):
    """Backend::copy (backend.h:32) on the copy kernel: every alignment class (16-byte vectors, words), ragged
    tails, and no write outside [dst, dst + count)."""
    rng = np.random.default_rng(count + 7 * src_off + 13 * dst_off)
    src = rng.standard_normal(count + 16).astype(np.float32)
    dst0 = rng.standard_normal(count + 16).astype(np.float32)
    with Buffers(backend) as B:
        ds, dd = B.upload(src), B.upload(dst0)
        backend.copy(dd.at(dst_off), ds.at(src_off), count)
        got = backend.download(dd, dst0.shape)
    want = dst0.copy()
    want[dst_off:dst_off + count] = src[src_off:src_off + count]
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("shift", [-5, -1, 1, 4, 1000])
def test_copy_overlapping_is_memmove(backend, shift):
    """Overlapping ranges copy as if through a temporary: the reference's Backend::copy is std::memmove
    (cpu_backend.cpp:260-263)."""
    n, count = 6000, 4000
    x = np.random.default_rng(abs(shift)).standard_normal(n).astype(np.float32)
    s0 = 1000
    with Buffers(backend) as B:
        dx = B.upload(x)
        backend.copy(dx.at(s0 + shift), dx.at(s0), count)
        got = backend.download(dx, x.shape)
    want = x.copy()
    want[s0 + shift:s0 + shift + count] = x[s0:s0 + count]
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("H,KV,D,neox,llama3", [(32, 8, 64, False, True), (14, 2, 64, True, False),
                                                 (32, 4, 64, False, False), (16, 8, 128, True, False),
                                                 (16, 4, 128, False, True), (8, 2, 24, True, False)])
@pytest.mark.parametrize("n,pos0", [(1, 1000), (7, 333), (600, 0), (300, 100), (512, 4096)])
def test_append_rope_attention_equals_unfused(backend, H, KV, D, neox, llama3, n, pos0):
    """The fused op (K/V append with RoPE, q rotated on load, append fused with the fp16 staging on the MFMA route)
    gives bit-identical outputs and caches to append_rope followed by attention, and leaves q unrotated."""
    base = 5e5 if llama3 else 1e4
    ff = synth.llama3_freq_factors(D, base) if llama3 else None
    rng = np.random.default_rng(n * 31 + pos0 + D)
    q = rng.standard_normal((n, H, D)).astype(np.float32)
    kn = rng.standard_normal((n, KV, D)).astype(np.float32)
    vn = rng.standard_normal((n, KV, D)).astype(np.float32)
    k0 = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
    v0 = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
    with Buffers(backend) as B:
        dq1, dq2, dkn, dvn = B.upload(q), B.upload(q), B.upload(kn), B.upload(vn)
        ck1, cv1, ck2, cv2 = B.upload(k0), B.upload(v0), B.upload(k0), B.upload(v0)
        o1, o2 = B.alloc(q.size), B.alloc(q.size)
        backend.append_rope(dq1, ck1, cv1, dkn, dvn, n, pos0, H, KV, D, base, neox, ff)
        backend.attention(dq1, ck1, cv1, o1, n, pos0, H, KV, D)
        backend.append_rope_attention(dq2, ck2, cv2, dkn, dvn, o2, n, pos0, H, KV, D, base, neox, ff)
        r1, r2 = backend.download(o1, q.shape), backend.download(o2, q.shape)
        gk1, gk2 = backend.download(ck1, k0.shape), backend.download(ck2, k0.shape)
        gv1, gv2 = backend.download(cv1, v0.shape), backend.download(cv2, v0.shape)
        gq2 = backend.download(dq2, q.shape)
    assert np.array_equal(bits(r1), bits(r2)), "outputs differ"
    assert np.array_equal(bits(gk1), bits(gk2)) and np.array_equal(bits(gv1), bits(gv2)), "caches differ"
    assert np.array_equal(bits(gq2), bits(q)), "fused op modified q"


@pytest.mark.parametrize("H,KV,D,neox,llama3", [(32, 8, 64, False, True), (14, 2, 64, True, False),
                                                 (16, 8, 128, True, False), (16, 4, 128, False, True)])
@pytest.mark.parametrize("pos0", [0, 1, 31, 32, 33, 255, 1023, 4113, 32768])
def test_append_rope_attention_decode_single_row(backend, H, KV, D, neox, llama3, pos0):
    """Decode step of the fused op: the new row rides in the attention launch (the workgroup owning row pos0 takes it
    from k_new / v_new). Output and caches are bit-identical to append_rope + attention at positions on both sides
    of the 32-row group and chunk boundaries, and q is left unrotated."""
    base = 5e5 if llama3 else 1e4
    ff = synth.llama3_freq_factors(D, base) if llama3 else None
    rng = np.random.default_rng(pos0 * 7 + D + H)
    q = rng.standard_normal((1, H, D)).astype(np.float32)
    kn = rng.standard_normal((1, KV, D)).astype(np.float32)
    vn = rng.standard_normal((1, KV, D)).astype(np.float32)
    k0 = rng.standard_normal((pos0 + 3, KV, D)).astype(np.float32)
    v0 = rng.standard_normal((pos0 + 3, KV, D)).astype(np.float32)
    with Buffers(backend) as B:
        dq1, dq2, dkn, dvn = B.upload(q), B.upload(q), B.upload(kn), B.upload(vn)
        ck1, cv1, ck2, cv2 = B.upload(k0), B.upload(v0), B.upload(k0), B.upload(v0)
        o1, o2 = B.alloc(q.size), B.alloc(q.size)
        backend.append_rope(dq1, ck1, cv1, dkn, dvn, 1, pos0, H, KV, D, base, neox, ff)
        backend.attention(dq1, ck1, cv1, o1, 1, pos0, H, KV, D)
        backend.append_rope_attention(dq2, ck2, cv2, dkn, dvn, o2, 1, pos0, H, KV, D, base, neox, ff)
        r1, r2 = backend.download(o1, q.shape), backend.download(o2, q.shape)
        gk1, gk2 = backend.download(ck1, k0.shape), backend.download(ck2, k0.shape)
        gv1, gv2 = backend.download(cv1, v0.shape), backend.download(cv2, v0.shape)
        gq2 = backend.download(dq2, q.shape)
    assert np.array_equal(bits(r1), bits(r2)), "outputs differ"
    assert np.array_equal(bits(gk1), bits(gk2)), "K caches differ"
    assert np.array_equal(bits(gv1), bits(gv2)), "V caches differ"
    assert np.array_equal(bits(gq2), bits(q)), "fused op modified q"
    assert np.array_equal(bits(gk2[pos0 + 1:]), bits(k0[pos0 + 1:])), "rows after pos0 changed"
    if pos0 <= 1023:
        kr = oracle.rope(kn.copy(), pos0, base, neox, ff)
        qr = oracle.rope(q.copy(), pos0, base, neox, ff)
        assert np.array_equal(bits(gk2[pos0]), bits(kr[0])), "appended K row"
        assert_parity(r2, cpu_attention(qr, np.concatenate([k0[:pos0], kr]), np.concatenate([v0[:pos0], vn]), pos0,
                                        KV), f"fused decode pos0={pos0}")


@pytest.mark.parametrize("pos0", [0, 5, 40, 20000])
def test_append_rope_attention_decode_never_reads_the_unwritten_row(backend, pos0):
    """The fused decode step must take row pos0 from k_new / v_new, not from the cache it is about to write: with
    cache rows pos0.. poisoned with NaN the output is finite and bitwise equal to the unpoisoned run, row pos0 holds
    the new row afterwards and the rows after it keep their NaN."""
    H, KV, D = 32, 8, 64
    rng = np.random.default_rng(pos0 + 99)
    q = rng.standard_normal((1, H, D)).astype(np.float32)
    kn = rng.standard_normal((1, KV, D)).astype(np.float32)
    vn = rng.standard_normal((1, KV, D)).astype(np.float32)
    k0 = rng.standard_normal((pos0 + 40, KV, D)).astype(np.float32)
    v0 = rng.standard_normal((pos0 + 40, KV, D)).astype(np.float32)
    kp, vp = k0.copy(), v0.copy()
    kp[pos0:] = np.nan
    vp[pos0:] = np.nan
    with Buffers(backend) as B:
        dq, dkn, dvn = B.upload(q), B.upload(kn), B.upload(vn)
        ck1, cv1, ck2, cv2 = B.upload(k0), B.upload(v0), B.upload(kp), B.upload(vp)
        o1, o2 = B.alloc(q.size), B.alloc(q.size)
        backend.append_rope_attention(dq, ck1, cv1, dkn, dvn, o1, 1, pos0, H, KV, D, 1e4, False, None)
        backend.append_rope_attention(dq, ck2, cv2, dkn, dvn, o2, 1, pos0, H, KV, D, 1e4, False, None)
        r1, r2 = backend.download(o1, q.shape), backend.download(o2, q.shape)
        gk1, gk2 = backend.download(ck1, k0.shape), backend.download(ck2, k0.shape)
        gv2 = backend.download(cv2, v0.shape)
    assert np.all(np.isfinite(r2))
    assert np.array_equal(bits(r1), bits(r2))
    assert np.array_equal(bits(gk1[pos0]), bits(gk2[pos0]))
    assert np.array_equal(bits(gv2[pos0]), bits(vn[0]))
    assert np.all(np.isnan(gk2[pos0 + 1:])) and np.all(np.isnan(gv2[pos0 + 1:]))


BATCH_POS = [0, 5, 31, 32, 100, 1000, 4096, 20000]


@pytest.mark.parametrize("H,KV,D,neox", [(32, 8, 64, False), (14, 2, 64, True), (32, 4, 64, False),
                                         (16, 8, 128, True), (8, 2, 24, False)])
def test_attention_batch_matches_oracle_and_single_calls(backend, H, KV, D, neox):
    """Ragged batch: each sequence's output is its own single-row attention (oracle and the single-sequence call,
    within tolerance: the context split differs), for positions on both sides of row-group and chunk boundaries;
    head_dim 24 takes the per-sequence fallback."""
    rng = np.random.default_rng(H * 7 + D)
    pos = BATCH_POS
    qs = [rng.standard_normal((1, H, D)).astype(np.float32) for _ in pos]
    ks = [rng.standard_normal((p + 1, KV, D)).astype(np.float32) for p in pos]
    vs = [rng.standard_normal((p + 1, KV, D)).astype(np.float32) for p in pos]
    with Buffers(backend) as B:
        dq = [B.upload(x) for x in qs]
        dk = [B.upload(x) for x in ks]
        dv = [B.upload(x) for x in vs]
        ob = [B.alloc(H * D) for _ in pos]
        o1 = [B.alloc(H * D) for _ in pos]
        backend.attention_batch(dq, dk, dv, ob, pos, H, KV, D)
        for i, p in enumerate(pos):
            backend.attention(dq[i], dk[i], dv[i], o1[i], 1, p, H, KV, D)
        gb = [backend.download(x, (1, H, D)) for x in ob]
        g1 = [backend.download(x, (1, H, D)) for x in o1]
    for i, p in enumerate(pos):
        ref = cpu_attention(qs[i], ks[i], vs[i], p, KV)
        assert_parity(gb[i], ref, f"batch seq {i} pos0={p}")
        assert_parity(gb[i], g1[i], f"batch vs single seq {i} pos0={p}")


def test_attention_batch_over_several_launches(backend):
    """More sequences than one launch takes (32): 40 sequences of mixed lengths, each checked against the oracle."""
    H, KV, D = 32, 8, 64
    rng = np.random.default_rng(40)
    pos = [int(x) for x in rng.integers(0, 3000, 40)]
    qs = [rng.standard_normal((1, H, D)).astype(np.float32) for _ in pos]
    ks = [rng.standard_normal((p + 1, KV, D)).astype(np.float32) for p in pos]
    vs = [rng.standard_normal((p + 1, KV, D)).astype(np.float32) for p in pos]
    with Buffers(backend) as B:
        dq, dk, dv = [B.upload(x) for x in qs], [B.upload(x) for x in ks], [B.upload(x) for x in vs]
        ob = [B.alloc(H * D) for _ in pos]
        backend.attention_batch(dq, dk, dv, ob, pos, H, KV, D)
        gb = [backend.download(x, (1, H, D)) for x in ob]
    for i, p in enumerate(pos):
        assert_parity(gb[i], cpu_attention(qs[i], ks[i], vs[i], p, KV), f"seq {i} pos0={p}")


@pytest.mark.parametrize("H,KV,D,neox,llama3", [(32, 8, 64, False, True), (14, 2, 64, True, False),
                                                 (16, 4, 128, False, False)])
def test_append_rope_attention_batch(backend, H, KV, D, neox, llama3):
    """Fused batch: every cache gets rope(k_new[i]) and v_new[i] at row pos0[i] bit-exactly (as the per-sequence
    fused call writes them), q is left unrotated, and each output is within tolerance of the oracle on the
    sequence alone."""
    base = 5e5 if llama3 else 1e4
    ff = synth.llama3_freq_factors(D, base) if llama3 else None
    rng = np.random.default_rng(D + H)
    pos = BATCH_POS
    qs = [rng.standard_normal((1, H, D)).astype(np.float32) for _ in pos]
    kn = [rng.standard_normal((1, KV, D)).astype(np.float32) for _ in pos]
    vn = [rng.standard_normal((1, KV, D)).astype(np.float32) for _ in pos]
    ks = [rng.standard_normal((p + 2, KV, D)).astype(np.float32) for p in pos]
    vs = [rng.standard_normal((p + 2, KV, D)).astype(np.float32) for p in pos]
    with Buffers(backend) as B:
        dq = [B.upload(x) for x in qs]
        dkn, dvn = [B.upload(x) for x in kn], [B.upload(x) for x in vn]
        dk, dv = [B.upload(x) for x in ks], [B.upload(x) for x in vs]
        dk1, dv1 = [B.upload(x) for x in ks], [B.upload(x) for x in vs]
        ob, o1 = [B.alloc(H * D) for _ in pos], [B.alloc(H * D) for _ in pos]
        backend.append_rope_attention_batch(dq, dk, dv, dkn, dvn, ob, pos, H, KV, D, base, neox, ff)
        for i, p in enumerate(pos):
            backend.append_rope_attention(dq[i], dk1[i], dv1[i], dkn[i], dvn[i], o1[i], 1, p, H, KV, D, base, neox,
                                          ff)
        gb = [backend.download(x, (1, H, D)) for x in ob]
        gk = [backend.download(x, ks[i].shape) for i, x in enumerate(dk)]
        gv = [backend.download(x, vs[i].shape) for i, x in enumerate(dv)]
        gk1 = [backend.download(x, ks[i].shape) for i, x in enumerate(dk1)]
        gq = [backend.download(x, (1, H, D)) for x in dq]
    for i, p in enumerate(pos):
        assert np.array_equal(bits(gk[i]), bits(gk1[i])), f"seq {i}: K cache differs from the per-sequence call"
        assert np.array_equal(bits(gv[i][p]), bits(vn[i][0])), f"seq {i}: appended V row"
        assert np.array_equal(bits(gv[i][p + 1:]), bits(vs[i][p + 1:])), f"seq {i}: rows after pos0 changed"
        assert np.array_equal(bits(gq[i]), bits(qs[i])), f"seq {i}: q modified"
        qr = oracle.rope(qs[i].copy(), p, base, neox, ff)
        kr = oracle.rope(kn[i].copy(), p, base, neox, ff)
        assert np.array_equal(bits(gk[i][p]), bits(kr[0])), f"seq {i}: appended K row"
        ref = cpu_attention(qr, np.concatenate([ks[i][:p], kr]), np.concatenate([vs[i][:p], vn[i]]), p, KV)
        assert_parity(gb[i], ref, f"fused batch seq {i} pos0={p}")


def test_attention_batch_causal_mask_poison(backend):
    """Rows past each sequence's window hold NaN (and, for the fused batch, row pos0 itself before the append):
    outputs stay finite and bitwise equal to the unpoisoned run."""
    H, KV, D = 32, 8, 64
    rng = np.random.default_rng(77)
    pos = [3, 64, 777, 9000]
    qs = [rng.standard_normal((1, H, D)).astype(np.float32) for _ in pos]
    kn = [rng.standard_normal((1, KV, D)).astype(np.float32) for _ in pos]
    vn = [rng.standard_normal((1, KV, D)).astype(np.float32) for _ in pos]
    ks = [rng.standard_normal((p + 9, KV, D)).astype(np.float32) for p in pos]
    vs = [rng.standard_normal((p + 9, KV, D)).astype(np.float32) for p in pos]

    def poisoned(x, p, first):
        y = x.copy()
        y[first:] = np.nan
        return y

    with Buffers(backend) as B:
        dq, dkn, dvn = [B.upload(x) for x in qs], [B.upload(x) for x in kn], [B.upload(x) for x in vn]
        outs = {}
        for tag, first in (("clean", None), ("plain", 1), ("fused", 0)):
            dk = [B.upload(ks[i] if first is None else poisoned(ks[i], p, p + first)) for i, p in enumerate(pos)]
            dv = [B.upload(vs[i] if first is None else poisoned(vs[i], p, p + first)) for i, p in enumerate(pos)]
            ob = [B.alloc(H * D) for _ in pos]
            if tag == "fused":
                dk0 = [B.upload(ks[i]) for i in range(len(pos))]
                dv0 = [B.upload(vs[i]) for i in range(len(pos))]
                oc = [B.alloc(H * D) for _ in pos]
                backend.append_rope_attention_batch(dq, dk0, dv0, dkn, dvn, oc, pos, H, KV, D, 1e4, False, None)
                outs["fused_clean"] = [backend.download(x, (1, H, D)) for x in oc]
                backend.append_rope_attention_batch(dq, dk, dv, dkn, dvn, ob, pos, H, KV, D, 1e4, False, None)
            else:
                backend.attention_batch(dq, dk, dv, ob, pos, H, KV, D)
            outs[tag] = [backend.download(x, (1, H, D)) for x in ob]
    for i in range(len(pos)):
        for tag, ref in (("plain", "clean"), ("fused", "fused_clean")):
            assert np.all(np.isfinite(outs[tag][i])), f"{tag} seq {i}"
            assert np.array_equal(bits(outs[tag][i]), bits(outs[ref][i])), f"{tag} seq {i}"


def test_attention_batch_rejects_bad_arguments(backend):
    H, KV, D = 32, 8, 64
    with Buffers(backend) as B:
        q, k, v, o = B.alloc(H * D), B.alloc(10 * KV * D), B.alloc(10 * KV * D), B.alloc(H * D)
        with pytest.raises(nibble_amd.BackendError):
            backend.attention_batch([q, q], [k], [v], [o], [3], H, KV, D)  # list lengths differ
        with pytest.raises(nibble_amd.BackendError):
            backend.attention_batch([q], [k], [v], [o], [10], H, KV, D)  # cache holds rows 0..9 only
        with pytest.raises(nibble_amd.BackendError):
            backend.attention_batch([q], [k], [v], [o], [-1], H, KV, D)
        backend.attention_batch([], [], [], [], [], H, KV, D)  # nothing to do


def test_rope_table_grows_geometrically_past_the_reservation():
    """Decoding one position at a time past the reserved n_ctx rebuilds the RoPE table only when it doubles (in whole
    1024-row blocks), not at every step; the appended rows stay bit-exact across a rebuild."""
    H, KV, D = 32, 8, 64
    be = nibble_amd.HipBackend(0)
    try:
        be.reserve(64, H, 1, 8192)
        rng = np.random.default_rng(5)
        cap = 2100
        with Buffers(be) as B:
            ck, cv = B.alloc(cap * KV * D), B.alloc(cap * KV * D)
            q = B.upload(rng.standard_normal((1, H, D)).astype(np.float32))
            kn_h = rng.standard_normal((1, KV, D)).astype(np.float32)
            kn, vn, out = B.upload(kn_h), B.alloc(KV * D), B.alloc(H * D)
            sizes = {}
            for pos in (1000, 1001, 1023, 1024, 1025, 2047):
                be.append_rope_attention(q, ck, cv, kn, vn, out, 1, pos, H, KV, D, 1e4, False, None)
                be.sync()
                sizes[pos] = be.internal_bytes()
            gk = be.download(ck, (cap, KV, D))
        assert sizes[1000] == sizes[1001] == sizes[1023], sizes  # one table of 1024 rows
        assert sizes[1024] > sizes[1023], sizes                   # grown once, to 2048 rows
        assert sizes[1024] == sizes[1025] == sizes[2047], sizes
        for pos in (1000, 1023, 1024, 2047):
            assert np.array_equal(bits(gk[pos]), bits(oracle.rope(kn_h.copy(), pos, 1e4, False)[0])), pos
    finally:
        be.close()
