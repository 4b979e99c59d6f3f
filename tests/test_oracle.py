"""Pins the CPU oracle (oracle/) before anything is checked against it. CPU only.

Sources of truth, in order:
  * tests/golden/reference_vectors.npz, written by the reference's own compiled kernels (make_golden.py):
    the restatement must reproduce them bit for bit;
  * oracle/_ref (the reference compiled from its sources) on fresh random shapes, when present;
  * the reference's known-answer tests (tests/test_ref_ops.cpp:41-135) and tolerance contracts
    (tests/test_ops.cpp:196-216, simd_helpers_test.cpp:92-137);
  * mathematics: an fp64 brute force, closed-form rotations, Llama-3 factor properties.
The last tests plant plausible mistakes in copies of the oracle's math and check that the pins reject them.
"""
import hashlib
import math
import os

import numpy as np
import pytest

import oracle
from nibble_amd import synth

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "reference_vectors.npz"))  # allow_pickle defaults to False

import importlib.util as _ilu  # noqa: E402

_spec = _ilu.spec_from_file_location("make_golden", os.path.join(HERE, "golden", "make_golden.py"))
make_golden = _ilu.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return np.frombuffer(h.digest(), dtype=np.uint8)


def matches_gold(key, y):
    """y equals the stored output bit for bit (whole array, or its SHA-256 for large outputs)."""
    if key in GOLD.files:
        return np.array_equal(GOLD[key].view(np.uint32), np.ascontiguousarray(y).view(np.uint32))
    return np.array_equal(GOLD[key + "_sha256"], sha(y))


def bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint32), np.ascontiguousarray(b).view(np.uint32))


# ---------------------------------------------------------------- golden vectors (written by the reference)

@pytest.mark.parametrize("case", make_golden.ATTN_CASES, ids=[c[0] for c in make_golden.ATTN_CASES])
def test_attention_restatement_reproduces_reference_vectors(case):
    name, n, pos0, H, KV, D, qs = case
    i = int(GOLD[f"attn/{name}/shape"][0])
    q, k, v = make_golden.attn_inputs(i, n, pos0, H, KV, D, qs)
    assert np.array_equal(GOLD[f"attn/{name}/input_sha256"], sha(q, k, v)), "input generator drifted"
    assert matches_gold(f"attn/{name}/scalar", oracle.attention_scalar(q, k, v, pos0, KV))
    if oracle.have_avx2():
        assert matches_gold(f"attn/{name}/simd", oracle.attention_avx2(q, k, v, pos0, KV))
        assert matches_gold(f"attn/{name}/simd", oracle.attention_parallel(q, k, v, pos0, KV, threads=3))


@pytest.mark.parametrize("case", make_golden.CORR_CASES, ids=[c[0] for c in make_golden.CORR_CASES])
def test_attention_restatement_reproduces_reference_vectors_correlated(case):
    """The correlated-K/V cases (K and V projected from shared low-rank hidden states)."""
    name, n, pos0, H, KV, D, qs, rank, vmix = case
    i = int(GOLD[f"attn/{name}/shape"][0])
    q, k, v = make_golden.corr_inputs(i, n, pos0, H, KV, D, qs, rank, vmix)
    assert np.array_equal(GOLD[f"attn/{name}/input_sha256"], sha(q, k, v)), "input generator drifted"
    assert matches_gold(f"attn/{name}/scalar", oracle.attention_scalar(q, k, v, pos0, KV))
    if oracle.have_avx2():
        assert matches_gold(f"attn/{name}/simd", oracle.attention_parallel(q, k, v, pos0, KV, threads=8))


@pytest.mark.parametrize("case", make_golden.REPEAT_CASES, ids=[c[0] for c in make_golden.REPEAT_CASES])
def test_attention_restatement_reproduces_reference_vectors_repeated_values(case):
    """The repeated-value-row cases (runs of equal value rows with elements near an fp16 rounding midpoint)."""
    name, n, pos0, H, KV, D = case[:6]
    i = int(GOLD[f"attn/{name}/shape"][0])
    q, k, v = make_golden.repeat_inputs(i, *case[1:])
    assert np.array_equal(GOLD[f"attn/{name}/input_sha256"], sha(q, k, v)), "input generator drifted"
    assert matches_gold(f"attn/{name}/scalar", oracle.attention_scalar(q, k, v, pos0, KV))
    if oracle.have_avx2():
        assert matches_gold(f"attn/{name}/simd", oracle.attention_parallel(q, k, v, pos0, KV, threads=8))


def test_repeated_value_cases_defeat_an_fp16_value_cache():
    """What the repeated-value cases are for: V rounded to fp16 once per row moves the reference's output by more
    than the 1e-3 bar (the equal rows' equal rounding errors survive the weighted mean). Checked on the const case
    with the scalar restatement over fp16-rounded V."""
    case = make_golden.REPEAT_CASES[0]
    assert case[6] == "const"
    name, n, pos0, H, KV, D = case[:6]
    q, k, v = make_golden.repeat_inputs(0, *case[1:])
    q, k, v = q[:4], k[:pos0 + 4], v[:pos0 + 4]
    ref = oracle.attention_scalar(q, k, v, pos0, KV)
    rounded = oracle.attention_scalar(q, k, v.astype(np.float16).astype(np.float32), pos0, KV)
    assert float(np.max(np.abs(rounded - ref))) > 1.8e-3


@pytest.mark.parametrize("case", make_golden.ROPE_CASES, ids=[c[0] for c in make_golden.ROPE_CASES])
def test_rope_restatement_reproduces_reference_vectors(case):
    name, n, heads, hd, pos0, base, neox, l3 = case
    i = int(GOLD[f"rope/{name}/params"][0])
    x = make_golden.rope_input(i, n, heads, hd)
    assert np.array_equal(GOLD[f"rope/{name}/input_sha256"], sha(x)), "input generator drifted"
    ff = synth.llama3_freq_factors(hd, base) if l3 else None
    if ff is not None:
        # The factor vector is an input of this case, stored beside the output it produced: equality only detects
        # input drift. The factors themselves are pinned by the known answers of test_llama3_factor_band_*.
        assert bits_equal(ff, GOLD[f"rope/{name}/freq_factors"]), "input drift"
    assert matches_gold(f"rope/{name}/out", oracle.rope(x.copy(), pos0, base, neox, ff))


def test_reference_known_answer_in_vectors():
    # test_ref_ops.cpp:73-81, as evaluated by the reference: out row 1 = softmax([0, 1/sqrt 2]) . v
    y = GOLD["kat/attention_2tok/out"].reshape(2, 2)
    e = math.exp(1 / math.sqrt(2))
    np.testing.assert_allclose(y, [[1, 0], [1 / (1 + e), e / (1 + e)]], rtol=1e-6, atol=1e-7)


# ---------------------------------------------------------------- the compiled reference on fresh shapes

@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built (needs the reference tree at build time)")
@pytest.mark.parametrize("seed", range(6))
def test_restatement_bit_exact_vs_compiled_reference(seed):
    rng = np.random.default_rng(seed)
    for _ in range(4):
        KV = int(rng.integers(1, 5))
        H = KV * int(rng.integers(1, 8))
        D = int(rng.choice([2, 8, 13, 16, 24, 64, 128]))
        n = int(rng.integers(1, 9))
        pos0 = int(rng.integers(0, 200))
        q = rng.standard_normal((n, H, D)).astype(np.float32) * np.float32(rng.choice([1, 5, 30]))
        k = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
        v = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
        assert bits_equal(oracle.attention_scalar(q, k, v, pos0, KV), oracle.ref_attention_scalar(q, k, v, pos0, KV))
        if oracle.have_avx2():
            assert bits_equal(oracle.attention_avx2(q, k, v, pos0, KV), oracle.ref_attention_simd(q, k, v, pos0, KV))
        base = float(rng.choice([1e4, 5e5, 1e6]))
        neox = bool(rng.integers(0, 2))
        ff = (rng.uniform(1, 8, D // 2).astype(np.float32) if D % 2 == 0 and rng.integers(0, 2) else None)
        if D % 2 == 0:
            p0 = int(rng.integers(0, 140000))
            x = rng.standard_normal((n, H, D)).astype(np.float32)
            assert bits_equal(oracle.rope(x.copy(), p0, base, neox, ff), oracle.ref_rope(x.copy(), p0, base, neox, ff))


# ---------------------------------------------------------------- the reference's known-answer tests

def rel(a, b):
    return abs(a - b) <= 1e-6 * abs(b) + 1e-7


def test_kat_rope():  # test_ref_ops.cpp:41-70
    c1, s1, c2, s2 = math.cos(1.0), math.sin(1.0), math.cos(0.01), math.sin(0.01)
    x = np.array([[[1, 0, 1, 0]]], np.float32)
    y = oracle.rope(x.copy(), 1, 10000.0, False)[0, 0]
    assert rel(y[0], c1) and rel(y[1], s1) and rel(y[2], c2) and rel(y[3], s2)
    y = oracle.rope(x.copy(), 1, 10000.0, True)[0, 0]
    assert rel(y[0], c1 - s1) and rel(y[1], 0) and rel(y[2], s1 + c1) and rel(y[3], 0)
    y = oracle.rope(x.copy(), 0, 10000.0, False)[0, 0]
    assert list(y) == [1, 0, 1, 0]
    y = oracle.rope(x.copy(), 1, 10000.0, False, np.array([1, 2], np.float32))[0, 0]
    assert rel(y[2], math.cos(0.005)) and rel(y[3], math.sin(0.005))


def test_kat_attention_two_tokens():  # test_ref_ops.cpp:73-81
    qkv = np.array([[[1, 0]], [[0, 1]]], np.float32)
    out = oracle.attention_scalar(qkv, qkv, qkv, 0, 1).reshape(2, 2)
    e = math.exp(1 / math.sqrt(2))
    assert rel(out[0, 0], 1) and rel(out[0, 1], 0)
    assert rel(out[1, 0], 1 / (1 + e)) and rel(out[1, 1], e / (1 + e))


def test_kat_attention_gqa():  # test_ref_ops.cpp:84-95
    H, KV, D, N = 4, 2, 2, 3
    q = np.ones((1, H, D), np.float32)
    k = np.zeros((N, KV, D), np.float32)
    v = np.zeros((N, KV, D), np.float32)
    for j in range(N):
        for g in range(KV):
            for d in range(D):
                v[j, g, d] = 10 * g + j + d
    for fn in (oracle.attention_scalar, oracle.attention_avx2, oracle.attention_f64):
        out = fn(q, k, v, N - 1, KV)
        if out is None:
            continue
        for h in range(H):
            for d in range(D):
                assert rel(float(out[0, h, d]), 10 * (h // 2) + 1 + d)


def test_kat_softmax_overflow_safe():  # test_ref_ops.cpp:130-135
    x = np.array([1000, 1000], np.float32)
    oracle.softmax_inplace(x)
    assert rel(x[0], 0.5) and rel(x[1], 0.5)


@pytest.mark.skipif(not oracle.have_avx2(), reason="no AVX2 on this host")
def test_exp_ps_error_bound():  # simd_helpers_test.cpp:92-137: <= 2e-7 relative over [-88, 88]
    x = np.linspace(-88, 88, 1 << 20, dtype=np.float32)
    y = oracle.exp_ps(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    assert np.max(np.abs(y - ref) / ref) <= 2e-7
    edge = oracle.exp_ps(np.array([0, -np.inf, np.inf, 89.0, -104.5, np.nan, -90, 1e-30], np.float32))
    assert edge[0] == 1 and edge[1] == 0 and np.isinf(edge[2]) and np.isinf(edge[3]) and edge[4] == 0
    assert np.isnan(edge[5]) and 0 < edge[6] < 1e-38 and edge[7] == 1


@pytest.mark.skipif(not oracle.have_avx2(), reason="no AVX2 on this host")
def test_simd_matches_scalar_within_contract():  # test_ops.cpp:196-216
    rng = np.random.default_rng(5)
    for n, pos0, H, KV, D, qs in [(1, 0, 2, 1, 8, 1), (7, 3, 6, 2, 16, 1), (4, 300, 4, 2, 64, 1),
                                  (3, 40, 2, 2, 13, 1), (2, 20, 4, 1, 128, 1), (5, 60, 4, 2, 64, 30)]:
        q = (rng.uniform(-1, 1, (n, H, D)) * qs).astype(np.float32)
        k = rng.uniform(-1, 1, (pos0 + n, KV, D)).astype(np.float32)
        v = rng.uniform(-1, 1, (pos0 + n, KV, D)).astype(np.float32)
        ref = oracle.attention_scalar(q, k, v, pos0, KV)
        got = oracle.attention_avx2(q, k, v, pos0, KV)
        assert np.max(np.abs(ref - got)) <= 2e-6 * qs


# ---------------------------------------------------------------- mathematics

def test_attention_matches_fp64_brute_force():
    rng = np.random.default_rng(11)
    for n, pos0, H, KV, D in [(1, 512, 14, 2, 64), (33, 0, 8, 2, 64), (5, 100, 4, 4, 128), (3, 7, 6, 3, 13)]:
        q = rng.standard_normal((n, H, D)).astype(np.float32)
        k = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
        v = rng.standard_normal((pos0 + n, KV, D)).astype(np.float32)
        f = oracle.attention_f64(q, k, v, pos0, KV)
        assert np.max(np.abs(oracle.attention_scalar(q, k, v, pos0, KV) - f)) < 2e-6
        if oracle.have_avx2():
            assert np.max(np.abs(oracle.attention_avx2(q, k, v, pos0, KV) - f)) < 2e-6


def test_fp64_brute_force_known_answers():
    # One key: output equals that key's value row. Identical keys: output is the mean of the value rows.
    q = np.ones((1, 2, 4), np.float32)
    v = np.arange(8, dtype=np.float32).reshape(1, 2, 4)
    assert np.array_equal(oracle.attention_f64(q, v, v, 0, 2), v.astype(np.float64))
    k = np.ones((5, 1, 4), np.float32)
    v = np.arange(20, dtype=np.float32).reshape(5, 1, 4)
    out = oracle.attention_f64(np.ones((1, 3, 4), np.float32), k, v, 4, 1)
    np.testing.assert_allclose(out[0], np.tile(v[:, 0].mean(0), (3, 1)), rtol=1e-15)


def test_rope_matches_closed_form_rotation():
    rng = np.random.default_rng(3)
    for neox in (False, True):
        for pos0 in (0, 5, 8191, 40000):
            x = rng.standard_normal((2, 3, 16)).astype(np.float32)
            y = oracle.rope(x.copy(), pos0, 5e5, neox)
            i = np.arange(8)
            for t in range(2):
                th = (pos0 + t) * 5e5 ** (-2.0 * i / 16)
                a_idx, b_idx = (i, i + 8) if neox else (2 * i, 2 * i + 1)
                a, b = x[t][:, a_idx].astype(np.float64), x[t][:, b_idx].astype(np.float64)
                np.testing.assert_allclose(y[t][:, a_idx], a * np.cos(th) - b * np.sin(th), atol=2e-6)
                np.testing.assert_allclose(y[t][:, b_idx], a * np.sin(th) + b * np.cos(th), atol=2e-6)


def test_llama3_factor_properties():
    for base, hd in [(5e5, 64), (5e5, 128), (1e4, 64)]:
        f = oracle.llama3_freq_factors(hd, base)
        assert bits_equal(f, synth.llama3_freq_factors(hd, base))
        i = np.arange(hd // 2)
        wl = 2 * np.pi / base ** (-2.0 * i / hd)
        assert np.all(f[wl < 8192 / 4] == 1) and np.all(f[wl > 8192] == 32)
        assert np.all(np.diff(f) >= 0) and f.min() >= 1 and f.max() <= 32
    # continuity at both band edges: s = 1 gives 1, s = 0 gives `factor`
    s1 = 1.0 / ((1 - 1.0) / 32 + 1.0)
    s0 = 1.0 / ((1 - 0.0) / 32 + 0.0)
    assert s1 == 1 and s0 == 32


# Known answers inside the blend band. With head_dim 2 the only frequency is base^0 = 1, so the wavelength is 2*pi
# and orig_ctx = 2*pi*c puts orig_ctx / wavelength at c. For factor 32, low 1, high 4 the blend weight is
# s = (c - 1) / 3, and the factor f = 1 / ((1 - s) / 32 + s) is a ratio of small integers:
#   c = 2: s = 1/3, f = 96/34 = 48/17;   c = 2.5: s = 1/2, f = 64/33;   c = 3: s = 2/3, f = 96/65.
LLAMA3_BAND_KATS = [(2.0, 48 / 17), (2.5, 64 / 33), (3.0, 96 / 65)]


def _llama3_f(fn, c):
    return float(fn(2, 1.0, 32.0, 1.0, 4.0, 2 * np.pi * c)[0])


@pytest.mark.parametrize("impl", ["oracle", "synth"])
def test_llama3_factor_band_known_answers(impl):
    fn = oracle.llama3_freq_factors if impl == "oracle" else synth.llama3_freq_factors
    for c, want in LLAMA3_BAND_KATS:
        # the closed form is evaluated in double and rounded once to float32; the double result can sit an ulp or
        # two from the exact rational (2*pi*c / 2*pi is c only up to rounding), far below a float32 ulp
        assert abs(_llama3_f(fn, c) - np.float32(want)) <= np.spacing(np.float32(want)), (impl, c)
    # the band edges: c = 1 (s = 0) is `factor`, c = 4 (s = 1) is 1
    assert _llama3_f(fn, 4.0 + 1e-9) == 1.0 and _llama3_f(fn, 1.0 - 1e-9) == 32.0


def test_llama3_factor_reciprocal_is_affine_in_inverse_wavelength():
    # Across the band 1/f = (1 - s)/F + s with s = (C/lambda - low)/(high - low): an affine function of 1/lambda,
    # 1/f = a + b/lambda with b = C (1 - 1/F) / (high - low) and a = 1/F - low (1 - 1/F) / (high - low). Checked on
    # every in-band entry of the BASELINE shapes (hd 64 and 128 at base 5e5: 3 and 6 entries) to float32 rounding.
    F, low, high, C = 32.0, 1.0, 4.0, 8192.0
    b = C * (1 - 1 / F) / (high - low)
    a = 1 / F - low * (1 - 1 / F) / (high - low)
    for hd in (64, 128):
        f = oracle.llama3_freq_factors(hd, 5e5).astype(np.float64)
        i = np.arange(hd // 2)
        wl = 2 * np.pi / 5e5 ** (-2.0 * i / hd)
        band = (wl >= C / high) & (wl <= C / low)
        assert band.sum() == (3 if hd == 64 else 6)
        np.testing.assert_allclose(1 / f[band], a + b / wl[band], rtol=2 ** -23)


def test_llama3_factor_planted_mistakes_fail():
    # Plausible slips in the blend must fail the known answers above: s inverted (1 - s), the blend taken linearly
    # in f instead of in 1/f, and the factor applied as its reciprocal.
    def blend(c, mistake):
        s = (c - 1.0) / 3.0
        if mistake == "inverted_s":
            s = 1 - s
        if mistake == "linear_in_f":
            return (1 - s) * 32 + s
        f = 1 / ((1 - s) / 32 + s)
        return 1 / f if mistake == "reciprocal" else f
    for mistake in ["inverted_s", "linear_in_f", "reciprocal"]:
        assert any(abs(np.float32(blend(c, mistake)) - np.float32(w)) > 1e-3 for c, w in LLAMA3_BAND_KATS), mistake
    assert all(np.float32(blend(c, None)) == np.float32(w) for c, w in LLAMA3_BAND_KATS)


# ---------------------------------------------------------------- planted mistakes must be caught

def _np_rope(x, pos0, base, neox, sign=1.0, swap=False):
    """numpy copy of the oracle's rope with optional planted mistakes (sign of sin, pairing)."""
    y = x.copy()
    n, h, hd = x.shape
    half = hd // 2
    i = np.arange(half)
    for t in range(n):
        th = (pos0 + t) * np.power(float(base), -2.0 * i / hd)
        c, s = np.cos(th).astype(np.float32), (sign * np.sin(th)).astype(np.float32)
        use_neox = (not neox) if swap else neox
        a_idx, b_idx = (i, i + half) if use_neox else (2 * i, 2 * i + 1)
        a, b = x[t][:, a_idx], x[t][:, b_idx]
        y[t][:, a_idx] = a * c - b * s
        y[t][:, b_idx] = a * s + b * c
    return y


def test_pins_reject_planted_rope_mistakes():
    name, n, heads, hd, pos0, base, neox, l3 = make_golden.ROPE_CASES[0]
    x = make_golden.rope_input(0, n, heads, hd)
    good = _np_rope(x, pos0, base, neox)
    assert bits_equal(good, oracle.rope(x.copy(), pos0, base, neox))  # the numpy copy is faithful
    assert matches_gold(f"rope/{name}/out", good)
    assert not matches_gold(f"rope/{name}/out", _np_rope(x, pos0, base, neox, sign=-1.0))
    assert not matches_gold(f"rope/{name}/out", _np_rope(x, pos0, base, neox, swap=True))
    assert not matches_gold(f"rope/{name}/out", _np_rope(x, pos0 + 1, base, neox))


def test_pins_reject_planted_attention_mistakes():
    name, n, pos0, H, KV, D, qs = make_golden.ATTN_CASES[7]  # config 1 shape
    q, k, v = make_golden.attn_inputs(7, n, pos0, H, KV, D, qs)
    key = f"attn/{name}/scalar"
    assert matches_gold(key, oracle.attention_scalar(q, k, v, pos0, KV))
    # wrong GQA mapping (h % KV instead of h // group)
    q_wrong = q.reshape(n, KV, H // KV, D).transpose(0, 2, 1, 3).reshape(n, H, D).copy()
    assert not matches_gold(key, oracle.attention_scalar(q_wrong, k, v, pos0, KV))
    # off-by-one causal window (attends one row short)
    assert not matches_gold(key, oracle.attention_scalar(q, k[:-1], v[:-1], pos0 - 1, KV))
    # missing 1/sqrt(d) scale
    assert not matches_gold(key, oracle.attention_scalar(q * np.float32(8.0), k, v, pos0, KV))
    # K and V swapped
    assert not matches_gold(key, oracle.attention_scalar(q, v, k, pos0, KV))
    # and the tolerance checks would catch them too (differences far above 1e-3)
    assert np.max(np.abs(oracle.attention_scalar(q, v, k, pos0, KV) - oracle.attention_scalar(q, k, v, pos0, KV))) > 1e-2


# ---- float matmul and bias (the QKV projection into the cache, transformer.cpp:171-194) ----

MATMUL_SHAPES = [(1, 1, 1), (1, 64, 96), (3, 129, 17), (5, 2048, 64), (16, 896, 128), (40, 256, 300)]


@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built")
@pytest.mark.parametrize("dt", [np.float32, np.float16])
@pytest.mark.parametrize("n,k,m", MATMUL_SHAPES)
def test_matmul_restatement_bit_exact_vs_reference(dt, n, k, m):
    """orc_matmul reproduces the reference's scalar float matmul (ref_ops.cpp:109-135) bit for bit."""
    rng = np.random.default_rng(n * 1000 + k + m)
    w = (rng.standard_normal((m, k)) * 0.05).astype(dt)
    x = rng.standard_normal((n, k)).astype(np.float32)
    assert bits_equal(oracle.matmul(w, x), oracle.ref_matmul_scalar(w, x))


@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built")
@pytest.mark.parametrize("dt", [np.float32, np.float16])
def test_matmul_against_fp64_and_the_reference_tier(dt):
    """The float dot's only error is float rounding: within 1e-5 of an fp64 product of the same inputs (relative to
    the row's sum of |terms|), and the reference's production tier (AVX2 gemm / matmul_rows_f, another order)
    agrees to the same bound."""
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((200, 2048)) * 0.03).astype(dt)
    x = rng.standard_normal((9, 2048)).astype(np.float32)
    y = oracle.matmul(w, x)
    scale = np.abs(x).astype(np.float64) @ np.abs(np.asarray(w, np.float64)).T
    assert np.all(np.abs(y - oracle.matmul_f64(w, x)) <= 1e-5 * scale)
    cb = oracle.RefCpuBackend(4)
    try:
        assert np.all(np.abs(cb.matmul(w, x) - y) <= 1e-5 * scale)
    finally:
        cb.close()


def test_matmul_planted_mistakes_fail():
    """A transposed weight or a reversed accumulation order does not reproduce the restatement."""
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((64, 64)) * 0.1).astype(np.float32)
    x = rng.standard_normal((4, 64)).astype(np.float32)
    y = oracle.matmul(w, x)
    assert not np.allclose(oracle.matmul(np.ascontiguousarray(w.T), x), y, atol=1e-3)
    rev = np.zeros_like(y)
    for t in range(4):
        for r in range(64):
            acc = np.float32(0)
            for kk in range(63, -1, -1):
                acc = np.float32(acc + np.float32(x[t, kk] * w[r, kk]))
            rev[t, r] = acc
    assert not bits_equal(rev, y)
    fwd = np.zeros_like(y)
    for t in range(4):
        for r in range(64):
            acc = np.float32(0)
            for kk in range(64):
                acc = np.float32(acc + np.float32(x[t, kk] * w[r, kk]))
            fwd[t, r] = acc
    assert bits_equal(fwd, y)  # the same loop in the forward order is the restatement


def test_fp16_conversion_every_half():
    """orc_fp16_to_fp32 (fp16.h:18-41 restated) on all 65536 halves, NaN payloads included, against numpy's exact
    float16 -> float32 conversion."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    assert bits_equal(oracle.fp16_to_fp32(h), want)


@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built")
def test_add_bias_bit_exact_vs_reference():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((7, 96)).astype(np.float32)
    b = rng.standard_normal(96).astype(np.float32)
    y = oracle.add_bias(x, b)
    assert bits_equal(y, oracle.ref_add_bias(x, b))
    assert bits_equal(y, x + b[None, :])


# ---------------------------------------------------------------------------- embed, rmsnorm, add, silu_mul

def ulp_diff(a, b):
    """Distance in float32 ulps (ordered integer encoding), elementwise."""
    def key(x):
        i = np.ascontiguousarray(x, np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    return np.abs(key(a) - key(b))


@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built")
@pytest.mark.parametrize("dt", [np.float32, np.float16])
def test_embed_bit_exact_vs_reference(dt):
    rng = np.random.default_rng(21)
    table = rng.standard_normal((50, 40)).astype(dt)
    ids = np.array([0, 49, 7, 7, 23], np.int32)
    got = oracle.embed(table, ids)
    assert bits_equal(got, oracle.ref_embed(table, ids))
    assert bits_equal(got, table[ids].astype(np.float32))  # numpy's widening of halves is exact
    for bad in ([50], [-1], [3, 50]):
        with pytest.raises(ValueError):
            oracle.embed(table, np.array(bad, np.int32))
        with pytest.raises(ValueError):
            oracle.ref_embed(table, np.array(bad, np.int32))


@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built")
@pytest.mark.parametrize("d", [1, 7, 64, 896, 2048])
def test_rmsnorm_bit_exact_vs_reference(d):
    rng = np.random.default_rng(d)
    x = (rng.standard_normal((5, d)) * rng.uniform(0.01, 30, (5, 1))).astype(np.float32)
    w = rng.standard_normal(d).astype(np.float32)
    got = oracle.rmsnorm(x, w, 1e-5)
    assert bits_equal(got, oracle.ref_rmsnorm(x, w, 1e-5))
    if oracle.have_avx2():  # the reference's own tier sums in another order: equal within 1 ulp
        assert int(ulp_diff(got, oracle.ref_rmsnorm(x, w, 1e-5, simd=True)).max()) <= 1


def test_rmsnorm_closed_form_and_fp64():
    """A constant row c normalises to sign(c) * w / sqrt(1 + eps / c^2); fp64 brute force on random rows. A float
    sum, a missing eps or a product in the wrong order fails one of these."""
    d = 256
    w = np.linspace(-2, 2, d).astype(np.float32)
    for c in (3.0, -0.5, 1e-3):
        x = np.full((1, d), c, np.float32)
        exact = np.float64(c) / np.sqrt(np.float64(c) ** 2 + 1e-5) * w.astype(np.float64)
        assert np.all(ulp_diff(oracle.rmsnorm(x, w, 1e-5)[0], exact.astype(np.float32)) <= 1)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, d)).astype(np.float32) * 5
    xd = x.astype(np.float64)
    exact = xd / np.sqrt((xd * xd).mean(axis=1, keepdims=True) + 1e-6) * w.astype(np.float64)
    assert np.all(ulp_diff(oracle.rmsnorm(x, w, 1e-6), exact.astype(np.float32)) <= 1)
    # eps matters at small scale: with rows of 1e-3 the eps term dominates and must not be dropped
    xs = np.full((1, d), 1e-3, np.float32)
    assert not np.allclose(oracle.rmsnorm(xs, w, 1e-5), oracle.rmsnorm(xs, w, 0.0), rtol=1e-3)


@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built")
def test_add_and_silu_mul_vs_reference():
    rng = np.random.default_rng(8)
    g = (rng.standard_normal(4099) * 6).astype(np.float32)
    g[:6] = [0.0, -0.0, 88.0, -88.0, 20.0, -100.0]
    u = rng.standard_normal(4099).astype(np.float32)
    assert bits_equal(oracle.add(g, u), oracle.ref_add(g, u))
    assert bits_equal(oracle.add(g, u), g + u)
    s = oracle.silu_mul(g, u)
    assert bits_equal(s, oracle.ref_silu_mul(g, u))  # same libm expf
    gd = g.astype(np.float64)
    exact = (gd / (1.0 + np.exp(-gd)) * u.astype(np.float64)).astype(np.float32)
    # within 2 ulp, except where expf(-g) overflows to inf for g < -88.7 (the reference's float formula then gives
    # -0 where the exact value is a denormal)
    assert np.all((ulp_diff(s, exact) <= 2) | (np.abs(exact) < 1e-37))
    assert s[5] == 0.0 and np.signbit(s[5]) == np.signbit(u[5] * -1.0)
    assert s[0] == 0.0 and s[1] == 0.0  # silu(0) = 0
    assert s[2] == np.float32(88.0) * u[2]  # silu(g) -> g for large g
    if oracle.have_avx2():  # the reference's AVX2 tier uses its own exp polynomial
        simd = oracle.ref_silu_mul(g, u, simd=True)
        assert np.all(np.abs(simd - s) <= 1e-6 * np.abs(s) + 1e-30)


# ---------------------------------------------------------------------------- the naive fp64 model (forward oracle)

from oracle import naive_model  # noqa: E402
from tests import model_util  # noqa: E402


@pytest.mark.parametrize("arch,wtype,rf", [("qwen2", np.float32, False), ("qwen2", np.float16, False),
                                           ("llama", np.float32, False), ("llama", np.float16, True)])
def test_naive_model_matches_the_restated_reference_forward(arch, wtype, rf):
    """The reference holds its production forward to naive_llama.h within 1e-4 on logits (test_model.cpp:110-131);
    the same holds between naive_logits and the reference's forward restated from the oracle's pinned float ops."""
    m = model_util.tiny_model(7, wtype, arch, rf)
    toks = [1, 50, 257, 3, 99]
    ref = model_util.cpu_forward(m, toks)
    got = naive_model.naive_logits(m, toks)
    assert got.shape == (261,)
    assert float(np.max(np.abs(got - ref))) <= 1e-4


def test_naive_model_planted_mistakes_fail():
    """Each plausible slip in the fp64 model (rope pairing, a dropped bias, a skipped layer) moves the logits far
    beyond the 1e-4 bar, so the agreement above is not vacuous; an explicit output matrix is honoured."""
    toks = [1, 50, 257, 3, 99]
    m = model_util.tiny_model(7, np.float32, "qwen2", False)
    ref = model_util.cpu_forward(m, toks)
    wrong_pairing = dict(m, arch="llama")  # llama pairing on a qwen2 model (keeps the biases)
    assert float(np.max(np.abs(naive_model.naive_logits(wrong_pairing, toks) - ref))) > 1e-2
    no_bias = dict(m, layers=[{k: v for k, v in L.items() if k not in ("bq", "bk", "bv")} for L in m["layers"]])
    assert float(np.max(np.abs(naive_model.naive_logits(no_bias, toks) - ref))) > 1e-2
    earlier = dict(m, layers=m["layers"][:1])  # one layer fewer
    assert float(np.max(np.abs(naive_model.naive_logits(earlier, toks) - ref))) > 1e-2
    m2 = model_util.tiny_model(7, np.float32, "qwen2", False, explicit_output=True)
    assert float(np.max(np.abs(naive_model.naive_logits(m2, toks) - model_util.cpu_forward(m2, toks)))) <= 1e-4
