"""Writes the golden vectors in tests/golden/*.npz from the reference's own CPU kernels.

Run in a container where oracle/_ref/libnibble_ref.so was built from the reference sources (oracle/Makefile,
target `ref`). The reference holds no RoPE or attention golden vectors of its own (its tests compute expected
values inline), so these are produced by its compiled code: cpu::rope (ref_ops.cpp:166-185),
cpu::attention_heads (ref_ops.cpp:188-214) and the AVX2 attention_heads (simd/ops.cpp:104-139).

Inputs come from nibble_amd.synth (counter-based, deterministic); each case stores its stream keys, its shape and
a SHA-256 of the input bytes (so a generator change is detected), plus the expected outputs. Large inputs are not
stored: the keys regenerate them.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from nibble_amd import synth  # noqa: E402

# (name, n, pos0, H, KV, D, qscale): the six shapes of the reference's SIMD-vs-scalar attention test
# (tests/test_ops.cpp:196-216) plus the BASELINE shapes at sizes a CPU finishes quickly.
ATTN_CASES = [
    ("ops_d8", 1, 0, 2, 1, 8, 1.0),
    ("ops_d16", 7, 3, 6, 2, 16, 1.0),
    ("ops_d64_pos300", 4, 300, 4, 2, 64, 1.0),
    ("ops_d13", 3, 40, 2, 2, 13, 1.0),
    ("ops_d128", 2, 20, 4, 1, 128, 1.0),
    ("ops_qscale30", 5, 60, 4, 2, 64, 30.0),
    ("backend_d16", 7, 3, 6, 2, 16, 1.0),           # test_cpu_backend.cpp:64-77 shape
    ("cfg1_qwen_decode", 1, 512, 14, 2, 64, 1.0),    # config 1 exactly
    ("qwen_prefill_96", 96, 0, 14, 2, 64, 1.0),      # config 2 shape, reduced length
    ("qwen_chunk", 40, 300, 14, 2, 64, 1.0),         # chunked prefill (pos0 > 0)
    ("tinyllama_decode", 1, 1792, 32, 4, 64, 1.0),   # config 3 first step
    ("llama_decode_2k", 1, 2047, 32, 8, 64, 1.0),    # config 4/5 shape, reduced context
    ("llama_prefill_300", 300, 0, 32, 8, 64, 1.0),   # crosses the fp32/MFMA prefill split at 128
    ("d128_prefill", 64, 200, 8, 2, 128, 1.0),
    # Large attention scores at prefill shapes (the reference's own large-q case, tests/test_ops.cpp:196-216, scales
    # q by 30): rows on both sides of the 128-row fp32 prefix, a chunk deep into a long cache, head_dim 128, and a
    # short chunk whose keys the MFMA route splits over several workgroups.
    ("prefill_qscale30", 320, 0, 4, 2, 64, 30.0),
    ("prefill_qscale5_pos4096", 512, 4096, 32, 8, 64, 5.0),
    ("prefill_d128_qscale30", 300, 100, 8, 2, 128, 30.0),
    ("prefill_qscale2", 600, 0, 14, 2, 64, 2.0),
    ("chunk_qscale30_pos1024", 64, 1024, 32, 8, 64, 30.0),
]

# (name, n, pos0, H, KV, D, qscale, rank, vmix): K and V projected from shared low-rank hidden states, as in a
# transformer (K = h Wk, V = h (vmix Wk + (1 - vmix) R), h of rank `rank` plus 10 % noise), with a random query per
# row and head. K and V correlate, so an error in the query that every key of a row shares does not average out over
# the keys. Chunks deep into a 4k cache (the MFMA route, key splits), Qwen and head_dim 128 shapes; "q05" keeps every
# row tile on the MFMA route, "r1_q1" sends every tile to the split-operand recomputation.
CORR_CASES = [
    ("prefill_corr_r2_q05", 256, 3840, 32, 8, 64, 0.5, 2, 0.8),
    ("prefill_corr_r8_q1", 256, 3840, 32, 8, 64, 1.0, 8, 0.6),
    ("prefill_corr_r1_q1", 256, 3840, 32, 8, 64, 1.0, 1, 1.0),
    ("prefill_corr_r2_qwen", 384, 1664, 14, 2, 64, 0.7, 2, 0.8),
    ("prefill_corr_d128", 192, 1856, 8, 2, 128, 0.7, 2, 0.8),
]

# (name, n, pos0, H, KV, D, kind, run_start, run_len): value rows that repeat, as the value rows of a token repeated
# in the prompt do (V carries no rotation). "const": every row of a KV head's V equal; "alt": two rows alternating
# over the whole window; "run": run_len rows from run_start equal, their keys equal too and aligned with the queries,
# so the run takes most of each row's weight. The repeated rows hold elements of 4-5 that sit just below the midpoint
# of two fp16 neighbours (fp16 rounding error 0.49 ulp = 1.9e-3, all towards zero): rounded to fp16 once per row,
# equal rows carry equal errors, and the output, a weighted mean of the rows, carries their mean whatever the number
# of keys. Deep chunks (the MFMA route), a short chunk whose keys are split over workgroups, Qwen's 7-to-1 grouping
# and head_dim 128.
REPEAT_CASES = [
    ("repeat_const_v", 256, 1792, 32, 8, 64, "const", 0, 0),
    ("repeat_run_attended", 256, 3840, 32, 8, 64, "run", 1000, 64),
    ("repeat_alt_d128", 192, 1856, 8, 2, 128, "alt", 0, 0),
    ("repeat_const_chunk", 64, 4032, 32, 8, 64, "const", 0, 0),
    ("repeat_run_qwen", 384, 1664, 14, 2, 64, "run", 200, 128),
]

# (name, n, heads, hd, pos0, base, neox, llama3)
ROPE_CASES = [
    ("qwen_q_pos512", 1, 14, 64, 512, 1e6, True, False),
    ("qwen_k_prefill", 2048, 2, 64, 0, 1e6, True, False),
    ("tinyllama_q_pos2047", 1, 32, 64, 2047, 1e4, False, False),
    ("llama_k_pos8191", 3, 8, 64, 8191, 5e5, False, True),
    ("llama_q_pos32768", 2, 32, 64, 32768, 5e5, False, True),
    ("llama_k_pos131071", 1, 8, 64, 131071, 5e5, False, True),
    ("neox_hd128_pos65536", 2, 4, 128, 65536, 1e4, True, False),
    ("hd4_pos1", 1, 1, 4, 1, 1e4, False, False),
]


def sha(*arrays) -> np.ndarray:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return np.frombuffer(h.digest(), dtype=np.uint8).copy()


FULL_LIMIT = 16384  # outputs larger than this many floats are stored as a SHA-256 plus sample rows


def put_output(out, key, y):
    """Stores y whole, or (when large) its SHA-256 with its first two and last rows, under key."""
    if y.size <= FULL_LIMIT:
        out[key] = y
    else:
        out[key + "_sha256"] = sha(y)
        out[key + "_head"] = y[:2].copy()
        out[key + "_tail"] = y[-1:].copy()


def attn_inputs(i, n, pos0, H, KV, D, qscale):
    ctx = pos0 + n
    q = synth.normal_array((n, H, D), 900, i, 1) * np.float32(qscale)
    k = synth.normal_array((ctx, KV, D), 900, i, 2)
    v = synth.normal_array((ctx, KV, D), 900, i, 3)
    return q.astype(np.float32), k, v


def corr_inputs(i, n, pos0, H, KV, D, qscale, rank, vmix):
    """q [n, H, D], k, v [pos0 + n, KV, D] of a CORR_CASES entry. The projections are exact int64 products of
    quantised normals (hidden states x 256, weights x 4096 / sqrt(4 D)), scaled by a power of two and rounded once to
    float32, so every machine regenerates the same bits whatever its BLAS."""
    ctx, dm = pos0 + n, 4 * D

    def ints(shape, tensor, scale):
        return np.rint(synth.normal_array(shape, 902, i, tensor).astype(np.float64) * scale).astype(np.int64)

    h = ints((ctx, rank), 1, 16) @ ints((rank, dm), 2, 16 / np.sqrt(rank)) + ints((ctx, dm), 3, 25.6)
    ws = 4096 / np.sqrt(dm)
    wk, r = ints((dm, KV * D), 4, ws), ints((dm, KV * D), 5, ws)
    wv = np.rint(vmix * wk + (1 - vmix) * r).astype(np.int64)
    sc = 1.0 / (256 * 4096)
    k = ((h @ wk) * sc).astype(np.float32).reshape(ctx, KV, D)
    v = ((h @ wv) * sc).astype(np.float32).reshape(ctx, KV, D)
    q = (synth.normal_array((n, H, D), 902, i, 7).astype(np.float64) * qscale).astype(np.float32)
    return q, k, v


def repeat_inputs(i, n, pos0, H, KV, D, kind, run_start, run_len):
    """q [n, H, D], k, v [pos0 + n, KV, D] of a REPEAT_CASES entry. A repeated value row is a N(0,1) row whose
    elements beyond 1.5 in magnitude become +-(4 + (m + 0.49) 2^-8), m in [0, 256): float32 values 0.49 fp16 ulps
    above a representable fp16 value."""
    ctx = pos0 + n
    q = synth.normal_array((n, H, D), 903, i, 1)
    k = synth.normal_array((ctx, KV, D), 903, i, 2)
    v = synth.normal_array((ctx, KV, D), 903, i, 3)

    def big_row(tensor, like=None):
        """like: a row whose large elements fix where this row's are, and their signs."""
        z = synth.normal_array((KV, D), 903, i, tensor).astype(np.float64)
        m = np.floor(np.abs(z) * 1e4) % 256
        mask, sign = (np.abs(z) > 1.5, np.sign(z)) if like is None else (np.abs(like) >= 4, np.sign(like))
        return np.where(mask, sign * (4.0 + (m + 0.49) / 256.0), z).astype(np.float32)
    a = big_row(4)
    if kind == "const":
        v[:] = a
    elif kind == "alt":
        b = big_row(5, like=a)
        v[0::2], v[1::2] = a, b
    elif kind == "run":
        s = slice(run_start, run_start + run_len)
        v[s] = a
        key = synth.normal_array((KV, D), 903, i, 6)
        k[s] = key
        g = H // KV  # query head h reads KV head h // g: aligned with that head's run key, plus noise
        q = (0.75 * np.repeat(key, g, axis=0)[None] + 0.5 * q).astype(np.float32)
    else:
        raise ValueError(kind)
    return q, k, v


def rope_input(i, n, heads, hd):
    return synth.normal_array((n, heads, hd), 901, i, 1)


def main():
    if not oracle.have_ref():
        sys.exit("oracle/_ref/libnibble_ref.so is not built; run `make -C oracle ref` first")
    out = {}
    for i, (name, n, pos0, H, KV, D, qs) in enumerate(ATTN_CASES):
        q, k, v = attn_inputs(i, n, pos0, H, KV, D, qs)
        out[f"attn/{name}/shape"] = np.array([i, n, pos0, H, KV, D], np.int64)
        out[f"attn/{name}/qscale"] = np.array([qs], np.float32)
        out[f"attn/{name}/input_sha256"] = sha(q, k, v)
        put_output(out, f"attn/{name}/scalar", oracle.ref_attention_scalar(q, k, v, pos0, KV))
        simd = oracle.ref_attention_simd(q, k, v, pos0, KV)
        if simd is None:
            sys.exit("the reference's SIMD tier is unavailable on this host; golden vectors need AVX2")
        put_output(out, f"attn/{name}/simd", simd)
    for i, (name, n, pos0, H, KV, D, qs, rank, vmix) in enumerate(CORR_CASES):
        q, k, v = corr_inputs(i, n, pos0, H, KV, D, qs, rank, vmix)
        out[f"attn/{name}/shape"] = np.array([i, n, pos0, H, KV, D], np.int64)
        out[f"attn/{name}/qscale"] = np.array([qs], np.float32)
        out[f"attn/{name}/input_sha256"] = sha(q, k, v)
        put_output(out, f"attn/{name}/scalar", oracle.ref_attention_scalar(q, k, v, pos0, KV))
        put_output(out, f"attn/{name}/simd", oracle.ref_attention_simd(q, k, v, pos0, KV))
    for i, (name, n, pos0, H, KV, D, kind, rs, rl) in enumerate(REPEAT_CASES):
        q, k, v = repeat_inputs(i, n, pos0, H, KV, D, kind, rs, rl)
        out[f"attn/{name}/shape"] = np.array([i, n, pos0, H, KV, D], np.int64)
        out[f"attn/{name}/input_sha256"] = sha(q, k, v)
        put_output(out, f"attn/{name}/scalar", oracle.ref_attention_scalar(q, k, v, pos0, KV))
        put_output(out, f"attn/{name}/simd", oracle.ref_attention_simd(q, k, v, pos0, KV))
    for i, (name, n, heads, hd, pos0, base, neox, l3) in enumerate(ROPE_CASES):
        x = rope_input(i, n, heads, hd)
        ff = synth.llama3_freq_factors(hd, base) if l3 else None
        y = oracle.ref_rope(x.copy(), pos0, base, neox, ff)
        out[f"rope/{name}/params"] = np.array([i, n, heads, hd, pos0, int(neox), int(l3)], np.int64)
        out[f"rope/{name}/base"] = np.array([base], np.float32)
        out[f"rope/{name}/input_sha256"] = sha(x)
        if ff is not None:
            out[f"rope/{name}/freq_factors"] = ff
        put_output(out, f"rope/{name}/out", y)
    # Known answers of test_ref_ops.cpp:73-95 / 130-135 evaluated by the reference itself.
    qkv = np.array([[[1, 0]], [[0, 1]]], np.float32)  # n=2, H=1, D=2
    out["kat/attention_2tok/out"] = oracle.ref_attention_scalar(qkv, qkv, qkv, 0, 1)
    path = os.path.join(HERE, "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes, kernel tier {oracle.ref_kernel_set()}")


if __name__ == "__main__":
    main()
