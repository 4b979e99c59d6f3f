"""Pins the quantized-format oracle (oracle/quant.c, restating src/quant.cpp) against the reference's golden vectors
(tests/data/quant_golden.inc: llama.cpp's own outputs, extracted to tests/golden/quant_golden.json) and bit for bit
against the compiled reference (oracle/_ref) on random blocks of every type, including CpuBackend::matmul's
production tier."""
import json
import os
import struct

import numpy as np
import pytest

import oracle
from tests.golden import quant_gen as G

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "quant_golden.json")))["tables"]
Q = oracle


def f32_bits(v):
    return struct.unpack("<I", struct.pack("<f", float(v)))[0]


def test_q8_0_and_q8_1_quantizer_golden():
    for case, c1 in zip(GOLD["kQuantCases"], GOLD["kQ8_1Cases"]):
        name, x, q8_d, q8_qs = case[0], np.array(case[1], np.float32), case[2], case[3]
        b = Q.quantize(0, x)
        assert int.from_bytes(b[:2].tobytes(), "little") == q8_d, name
        assert list(b[2:].view(np.int8)) == q8_qs, name
        b1 = Q.quantize(1, x)
        assert c1[0] == name
        assert int.from_bytes(b1[:2].tobytes(), "little") == c1[1], name
        assert int.from_bytes(b1[2:4].tobytes(), "little") == c1[2], name
        assert list(b1[4:].view(np.int8)) == q8_qs, name


def test_q8_k_quantizer_golden():
    for crafted, seed, n, d_hash, out_hash in GOLD["kQ8KCases"]:
        x = G.crafted_q8k_row(crafted) if crafted >= 0 else G.q8k_rows(G.Rng(seed), n)
        b = Q.quantize(2, x).reshape(-1, 292)
        assert G.fnv1a(b[:, :4].tobytes()) == d_hash, (crafted, seed, n)
        assert G.fnv1a(b[:, 4:].tobytes()) == out_hash, (crafted, seed, n)


def test_legacy_dots_golden():
    for seed, n, h, q8q8, q4q8 in GOLD["kDotCases"]:
        r, nb = G.Rng(seed), n // 32
        w8, a8, w4 = G.fill_q8_0(r, nb), G.fill_q8_0(r, nb), G.fill_q4_0(r, nb)
        assert G.fnv1a(w8 + a8 + w4) == h
        assert f32_bits(Q.dot(Q.Q8_0, np.frombuffer(w8, np.uint8), np.frombuffer(a8, np.uint8), nb)) == q8q8
        assert f32_bits(Q.dot(Q.Q4_0, np.frombuffer(w4, np.uint8), np.frombuffer(a8, np.uint8), nb)) == q4q8
    for seed, n, h, q50, q51 in GOLD["kDot5Cases"]:
        r, nb = G.Rng(seed), n // 32
        w50, a80, w51, a81 = G.fill_q5_0(r, nb), G.fill_q8_0(r, nb), G.fill_q5_1(r, nb), G.fill_q8_1(r, nb)
        assert G.fnv1a(w50 + a80 + w51 + a81) == h
        assert f32_bits(Q.dot(Q.Q5_0, np.frombuffer(w50, np.uint8), np.frombuffer(a80, np.uint8), nb)) == q50
        assert f32_bits(Q.dot(Q.Q5_1, np.frombuffer(w51, np.uint8), np.frombuffer(a81, np.uint8), nb)) == q51


def test_k_dots_golden():
    for seed, n, h, q4k, q5k, q6k in GOLD["kKDotCases"]:
        r, nb = G.Rng(seed), n // 256
        w4, w5, w6, a8 = G.fill_q4_k(r, nb), G.fill_q5_k(r, nb), G.fill_q6_k(r, nb), G.fill_q8_k(r, nb)
        assert G.fnv1a(w4 + w5 + w6 + a8) == h
        a = np.frombuffer(a8, np.uint8)
        assert f32_bits(Q.dot(Q.Q4_K, np.frombuffer(w4, np.uint8), a, nb)) == q4k
        assert f32_bits(Q.dot(Q.Q5_K, np.frombuffer(w5, np.uint8), a, nb)) == q5k
        assert f32_bits(Q.dot(Q.Q6_K, np.frombuffer(w6, np.uint8), a, nb)) == q6k


def test_dequantize_golden():
    nb, seed = GOLD["kDequantBlocks"], GOLD["kDequantSeed"]
    r = G.Rng(seed)
    q8, q4 = G.fill_q8_0(r, nb), G.fill_q4_0(r, nb)
    assert list(Q.dequantize(Q.Q8_0, q8, nb * 32).view(np.uint32)) == GOLD["kDequantQ8_0"]
    assert list(Q.dequantize(Q.Q4_0, q4, nb * 32).view(np.uint32)) == GOLD["kDequantQ4_0"]
    r = G.Rng(seed)
    q50, q51 = G.fill_q5_0(r, nb), G.fill_q5_1(r, nb)
    assert list(Q.dequantize(Q.Q5_0, q50, nb * 32).view(np.uint32)) == GOLD["kDequantQ5_0"]
    assert list(Q.dequantize(Q.Q5_1, q51, nb * 32).view(np.uint32)) == GOLD["kDequantQ5_1"]
    kb = GOLD["kDequantKBlocks"]
    fills = {"Q4_K": (Q.Q4_K, G.fill_q4_k), "Q5_K": (Q.Q5_K, G.fill_q5_k), "Q6_K": (Q.Q6_K, G.fill_q6_k)}
    for name, h in GOLD["kDequantK"]:
        t, fill = fills[name]
        out = Q.dequantize(t, fill(G.Rng(seed), kb), kb * 256)
        assert G.fnv1a(out.tobytes()) == h, name


def test_fp32_to_fp16_against_numpy():
    """Round to nearest even with overflow to inf and gradual underflow: numpy's float16 cast is IEEE."""
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
                        np.array([65504, 65520, 65519.996, 1e-8, 2.98e-8, 5.96e-8, -0.0, np.inf, -np.inf], np.float32)])
    x = x.astype(np.float32)
    got = np.array([Q.fp32_to_fp16(v) for v in x], np.uint16)
    with np.errstate(over="ignore"):
        assert np.array_equal(got, x.astype(np.float16).view(np.uint16))


def tie_block():
    """A 32-float block whose Q8_1 sum term float(sum) * d is, as a float, exactly 1358.5 * 2^-7 (an fp16 tie: the
    reference rounds it to the even 1358 * 2^-7), while the exact product of sum and d lies just above the tie
    (rounded once, straight to fp16, it would give 1359 * 2^-7)."""
    return np.random.default_rng(9).standard_normal((80, 256)).astype(np.float32)[32, 96:128]


def test_q8_1_sum_term_rounds_twice():
    """quant.cpp:268: blk.s = fp32_to_fp16(float(sum) * d) - the product rounded to float, then to fp16."""
    from fractions import Fraction
    x = tie_block()
    blk = oracle.quantize(1, x)
    d = np.float32(np.max(np.abs(x))) / np.float32(127)
    total = int(blk[4:].view(np.int8).astype(np.int64).sum())
    prod = np.float32(total) * d
    assert Fraction(float(prod)) * 128 == Fraction(2717, 2)  # the float product is the tie
    assert Fraction(total) * Fraction(float(d)) * 128 > Fraction(2717, 2)  # the exact one lies above it
    assert blk[2:4].view(np.float16)[0] == np.float16(1358 / 128)


RAND_FILLS = {Q.Q4_0: G.fill_q4_0, Q.Q5_0: G.fill_q5_0, Q.Q5_1: G.fill_q5_1, Q.Q8_0: G.fill_q8_0, Q.Q4_K: G.fill_q4_k,
              Q.Q5_K: G.fill_q5_k, Q.Q6_K: G.fill_q6_k}
ACT_FILLS = {0: G.fill_q8_0, 1: G.fill_q8_1, 2: G.fill_q8_k}


@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built")
@pytest.mark.parametrize("t", Q.QUANT_TYPES)
def test_random_blocks_bit_exact_vs_reference(t):
    nb = 24 if Q.block_elems(t) == 32 else 6
    n = nb * Q.block_elems(t)
    for seed in range(20, 26):
        r = G.Rng(seed)
        w = np.frombuffer(RAND_FILLS[t](r, nb), np.uint8)
        a = np.frombuffer(ACT_FILLS[Q.act_kind(t)](r, nb), np.uint8)
        assert f32_bits(Q.dot(t, w, a, nb)) == f32_bits(Q.ref_dot(t, w, a, nb))
        assert np.array_equal(Q.dequantize(t, w, n).view(np.uint32), Q.ref_dequantize(t, w, n).view(np.uint32))
    rng = np.random.default_rng(t)
    x = (rng.standard_normal(4 * 256) * 3).astype(np.float32)
    x[7] = 0.0
    x[256:512] = 0.0  # an all-zero Q8_K block and Q8_0 blocks
    for kind in (0, 1, 2):
        assert np.array_equal(Q.quantize(kind, x), Q.ref_quantize(kind, x))


@pytest.mark.skipif(not oracle.have_ref(), reason="oracle/_ref not built")
@pytest.mark.parametrize("t", Q.QUANT_TYPES)
def test_matmul_q_bit_exact_vs_reference_backend(t):
    """CpuBackend::matmul on quantized weights (the production tier over the pool) equals the restatement."""
    in_ = 512 if Q.block_elems(t) == 256 else 160
    out_, n = 24, 5
    r = G.Rng(100 + t)
    w = np.frombuffer(RAND_FILLS[t](r, out_ * in_ // Q.block_elems(t)), np.uint8)
    x = (np.random.default_rng(t).standard_normal((n, in_)) * 2).astype(np.float32)
    got = Q.matmul_q(t, w, in_, out_, x)
    be = oracle.RefCpuBackend(4)
    try:
        ref = be.matmul_q(t, w, in_, out_, x)
    finally:
        be.close()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # and against the fp64 product of the dequantized weights and the dequantized activations: the block dots are
    # exact integer sums scaled once per block, so they agree to float rounding of the per-block terms (Q5_1 adds
    # m_w * s_a, whose s_a is the block sum rounded to fp16: 2^-11 relative)
    wd = Q.dequantize(t, w, out_ * in_).reshape(out_, in_).astype(np.float64)
    kind = Q.act_kind(t)
    xd = np.stack([Q.dequantize(Q.Q8_0, Q.quantize(0, x[i]), in_) if kind < 2 else _dequant_q8k(Q.quantize(2, x[i]), in_)
                   for i in range(n)]).astype(np.float64)
    exact = xd @ wd.T
    scale = np.abs(xd) @ np.abs(wd).T
    tol = 2.0 ** -10 if kind == 1 else 1e-5
    assert np.all(np.abs(got - exact) <= tol * scale + 1e-30)


def _dequant_q8k(raw, n):
    b = raw.reshape(-1, 292)
    d = b[:, :4].copy().view(np.float32)[:, 0]
    qs = b[:, 4:260].view(np.int8).astype(np.float32)
    return (qs * d[:, None]).reshape(n)
