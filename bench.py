#!/usr/bin/env python3
"""Attention-path benchmark on one MI355X: BASELINE config 4 (Llama-3.2-1B shape, 16 layers).

Workload (inputs resident in HBM before any timed region; synthetic N(0,1) data generated on the device):
  * prefill: 8192 tokens per layer - KV append with RoPE (Llama-3 frequency factors) into the layer's cache, then
    causal GQA attention over the 8192 rows;
  * decode: cache rows 8192..32767 seeded, then `--steps` single-token steps at positions 32768 + s, each through
    all 16 layers (append with RoPE, then attention over 32769 + s rows). One "step" = one token through 16 layers.
Printed: one JSON line. `value` = decode attention HBM GB/s (algorithmic bytes 8*KV*hd*L_ctx per layer-step over the
timed wall time of the steps); `prefill` = prefill attention TFLOP/s (2*H*hd*n*(n+1) per layer). `roofline` is the
decode partial kernel (attn_decode_rows) alone: algorithmic bytes per launch / its average duration, read from
start/stop events that hipExtLaunchKernel stamps on each dispatch in one more pass over the same steps;
`prefill.roofline` is the MFMA kernel
alone, from one more prefill pass. `traffic` = HBM bytes per launch from two `rocprofv3 --pmc` child runs (FETCH_SIZE,
WRITE_SIZE) over `--probe`, scaled by what the counters read for a known-size copy; a third run reads the prefill
kernel's MFMA busy cycles (`prefill.roofline.mfma_busy_frac`). `cpu_baseline` is the reference's CpuBackend
(compiled from its sources, oracle/_ref) timed on this host on bounded samples.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import nibble_amd  # noqa: E402
from nibble_amd import KernelTiming, configs  # noqa: E402

METRIC = "decode attn HBM GB/s (%peak) @32k ctx; prefill attn TFLOP/s (%MFMA) @8k"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
FP32_PREFIX_ROWS = 128  # prefill rows below this position run in fp32, in the MFMA launch (hip_backend.cpp)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_bytes(kv, hd, ctx_len):
    return 8 * kv * hd * ctx_len  # fp32 K and V rows read once


def prefill_flops(h, hd, pos0, n):
    # 4*H*hd per (query, visible key): QK^T and PV, causal-unmasked pairs only
    t = np.arange(pos0, pos0 + n, dtype=np.float64)
    return float(4.0 * h * hd * np.sum(t + 1))


def _host_cpu_info():
    """Host CPU description for the baseline: the lscpu model name, the online CPU count (what
    std::thread::hardware_concurrency() returns), the CPUs this process may run on, and the cgroup CPU quota."""
    import subprocess

    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next((l.split(":", 1)[1].strip() for l in out.splitlines() if l.startswith("Model name")), None)
    except (OSError, subprocess.SubprocessError):
        pass
    if not model:
        try:
            model = next((l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name")),
                         "?")
        except OSError:
            model = "?"
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()
        if q != "max":
            quota = round(int(q) / int(period), 2)
    except (OSError, ValueError):
        pass
    return {"cpu_model": model, "host_cpus": os.cpu_count() or 1, "affinity_cpus": len(os.sched_getaffinity(0)),
            "cgroup_cpu_quota": quota}


def cpu_baseline(be, shape, ck0, cv0, dq_dec, ctx, q_pre, budget_s):
    """The reference's own CPU attention (ThreadPool + CpuBackend from oracle/_ref, AVX2 tier), timed on this host on
    bounded samples of the same workload; falls back to our C restatement (kind "port") without oracle/_ref.
    The pool has std::thread::hardware_concurrency() threads (the online CPU count), and the protocol is the
    reference's `nibble bench` (cli/cmd_bench.cpp:225-244): one untimed warm-up, then median, min and max."""
    import oracle

    H, KV, D = shape.n_heads, shape.n_kv_heads, shape.head_dim
    host = _host_cpu_info()
    threads = host["host_cpus"]
    L = ctx + 1
    k = be.download(ck0, (L, KV, D))
    v = be.download(cv0, (L, KV, D))
    q = be.download(dq_dec, (1, H, D))
    out = np.zeros((1, H, D), np.float32)
    ref = oracle.have_ref()
    if ref:
        cb = oracle.RefCpuBackend(threads)
        cb.reserve(L, H, 512, 8192)
        run = lambda qq, kk, vv, oo, n, p0: cb.attention(qq, kk, vv, oo, n, p0, H, KV, D)  # noqa: E731
        kind, tier = "reference", oracle.ref_kernel_set()
    else:
        def run(qq, kk, vv, oo, n, p0):
            oo[...] = oracle.attention_parallel(qq, kk[:p0 + n], vv[:p0 + n], p0, KV, threads,
                                                use_avx2=oracle.have_avx2())
        kind, tier = "port", ("avx2" if oracle.have_avx2() else "scalar")

    def timed(fn, min_reps, seconds):
        fn()  # warm-up (cmd_bench.cpp:225: rep -1 is untimed)
        times = []
        t_end = time.perf_counter() + seconds
        while len(times) < min_reps or time.perf_counter() < t_end:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
            if len(times) >= 200:
                break
        return np.array(times)

    def stats(work, times, scale):
        rate = work / times / scale  # per-rep throughput, as cmd_bench.cpp reports per-rep tok/s
        return {"value": round(float(np.median(rate)), 5), "min": round(float(rate.min()), 5),
                "max": round(float(rate.max()), 5), "reps": int(len(times))}

    dec = stats(decode_bytes(KV, D, L), timed(lambda: run(q, k, v, out, 1, ctx), 5, budget_s / 2), 1e9)
    # prefill sample: the last 256 query rows of the 8192-token prefill of layer 0 (pos0 = 7936)
    n_s, pos0_s = 256, 8192 - 256
    qs = np.ascontiguousarray(q_pre[pos0_s:8192])
    outp = np.zeros_like(qs)
    pre = stats(prefill_flops(H, D, pos0_s, n_s), timed(lambda: run(qs, k, v, outp, n_s, pos0_s), 3, budget_s / 2),
                1e12)
    return {
        "value": dec["value"], "unit": "GB/s", "cores": threads, "kind": kind,
        "min": dec["min"], "max": dec["max"], "reps": dec["reps"],
        "sample": f"layer-0 decode attention at {L} ctx (1 token, {H} heads), median of {dec['reps']} reps; "
                  f"reference CpuBackend::attention, tier {tier}, parallel_for over {H} heads (at most {H} busy "
                  f"threads)",
        "threads": threads, "tasks": H, **host,
        "prefill": {"value": pre["value"], "min": pre["min"], "max": pre["max"], "reps": pre["reps"],
                    "unit": "TFLOP/s",
                    "sample": f"layer-0 prefill rows {pos0_s}..8191 ({n_s} rows), median of {pre['reps']} reps"},
    }


def ragged_decode(be, steps, warmup):
    """BASELINE config 5 throughput: 16 Llama-3.2-1B-shape sequences with the ragged cache lengths of the parity
    test (log-uniform 1024..131072, seeded), 16 layers, N(0,1) caches with 1 % of K rows scaled x8 (in blocks of 16
    rows, one in a hundred), one token per sequence per step. Each layer of a step is one
    append_rope_attention_batch call for all 16 sequences; the same steps are then timed again as 16 single-sequence
    calls per layer. Returns the config-5 sub-object of the JSON line."""
    shape = configs.LLAMA32_1B
    H, KV, D = shape.n_heads, shape.n_kv_heads, shape.head_dim
    base, neox, ff = shape.rope_base, shape.neox, shape.freq_factors()
    NL, row = 16, KV * D
    lengths = configs.cfg5_lengths()
    n_seq = len(lengths)
    span = warmup + steps
    caches = []
    for l in range(NL):
        per = []
        for i, L in enumerate(lengths):
            k, v = be.alloc((L + span) * row), be.alloc((L + span) * row)
            be.fill_normal(k, L * row, seed=9000 + 64 * l + 2 * i)
            be.fill_normal(v, L * row, seed=9001 + 64 * l + 2 * i)
            for r0 in range(7 * 16, L, 1600):  # 1 % of K rows, x8
                nr = min(16, L - r0)
                be.fill_normal(k.at(r0 * row), nr * row, seed=7 + 131 * l + r0, scale=8.0)
            per.append((k, v))
        caches.append(per)
    qs = be.alloc(span * NL * n_seq * H * D)
    kn, vn = be.alloc(span * NL * n_seq * row), be.alloc(span * NL * n_seq * row)
    out = be.alloc(n_seq * H * D)
    be.fill_normal(qs, span * NL * n_seq * H * D, seed=31)
    be.fill_normal(kn, span * NL * n_seq * row, seed=32)
    be.fill_normal(vn, span * NL * n_seq * row, seed=33)
    be.reserve_rope(D, base, neox, ff)

    def args_of(s, l):
        j = (s * NL + l) * n_seq
        return ([qs.at((j + i) * H * D) for i in range(n_seq)], [c[0] for c in caches[l]], [c[1] for c in caches[l]],
                [kn.at((j + i) * row) for i in range(n_seq)], [vn.at((j + i) * row) for i in range(n_seq)],
                [out.at(i * H * D) for i in range(n_seq)], [L + s for L in lengths])

    def step_batched(s):
        for l in range(NL):
            q, k, v, a, b, o, p = args_of(s, l)
            be.append_rope_attention_batch(q, k, v, a, b, o, p, H, KV, D, base, neox, ff)

    def step_single(s):
        for l in range(NL):
            q, k, v, a, b, o, p = args_of(s, l)
            for i in range(n_seq):
                be.append_rope_attention(q[i], k[i], v[i], a[i], b[i], o[i], 1, p[i], H, KV, D, base, neox, ff)

    def timed(step):
        for s in range(warmup):
            step(s)
        be.sync()
        e0, e1 = be.event(), be.event()
        e0.record()
        for s in range(warmup, span):
            step(s)
        e1.record()
        return e0.elapsed_ms(e1)

    byts = sum(NL * decode_bytes(KV, D, L + s + 1) for s in range(warmup, span) for L in lengths)
    ms_b = timed(step_batched)
    ms_1 = timed(step_single)
    for per in caches:
        for k, v in per:
            be.free(k)
            be.free(v)
    for x in (qs, kn, vn, out):
        be.free(x)
    gbs_b, gbs_1 = byts / (ms_b * 1e-3) / 1e9, byts / (ms_1 * 1e-3) / 1e9
    log(f"config 5 (16 ragged sequences, {sum(lengths)} cache rows per layer): batched {ms_b / steps:.3f} ms/step -> "
        f"{gbs_b:.1f} GB/s ({gbs_b / HBM_PEAK_GBS:.1%}); 16 single calls per layer {ms_1 / steps:.3f} ms/step -> "
        f"{gbs_1:.1f} GB/s")
    return {"metric": "ragged batched decode attn HBM GB/s (BASELINE config 5)", "value": round(gbs_b, 1),
            "unit": "GB/s", "frac": round(gbs_b / HBM_PEAK_GBS, 4), "steps": steps, "warmup": warmup,
            "ms_per_step": round(ms_b / steps, 4), "sequences": n_seq, "layers": NL,
            "cache_rows_per_layer": sum(lengths), "lengths": lengths,
            "single_calls": {"value": round(gbs_1, 1), "ms_per_step": round(ms_1 / steps, 4),
                             "note": "the same steps as 16 single-sequence calls per layer"}}


FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 (MFMA)


def f16kv_decode(be, steps, warmup):
    """Decode steps over fp16 KV caches (an extension: the reference's cache is fp32), at the config-4 shape: 16
    layers at 32k context, one append_rope_attention_f16kv per layer (the new row rides in the attention launch).
    HBM GB/s of the fp16 K and V rows each step reads. Then the 8192-token prefill over the same caches
    (`prefill_8k`, TFLOP/s as the fp32-cache prefill counts them)."""
    shape, NL, ctx = configs.LLAMA32_1B, 16, 32768
    H, KV, D = shape.n_heads, shape.n_kv_heads, shape.head_dim
    stamped = 8  # steps whose partial launches carry start/stop events, after the timed ones
    rows = ctx + steps + warmup + stamped
    halves = rows * KV * D
    rng = np.random.default_rng(5)
    host = rng.standard_normal(halves).astype(np.float16).view(np.float32)
    ck, cv = [], []
    for l in range(NL):
        k, v = be.alloc(halves // 2), be.alloc(halves // 2)
        if l == 0:
            be.write(k, host)
            be.write(v, host[::-1].copy())
        else:
            be.copy(k, ck[0], halves // 2)
            be.copy(v, cv[0], halves // 2)
        ck.append(k)
        cv.append(v)
    q, kd, vd, out = be.alloc(H * D), be.alloc(KV * D), be.alloc(KV * D), be.alloc(H * D)
    for p_, n_ in ((q, H * D), (kd, KV * D), (vd, KV * D)):
        be.fill_normal(p_, n_, seed=n_)
    base, neox, ff = shape.rope_base, shape.neox, shape.freq_factors()

    def step(s):
        for l in range(NL):
            be.append_rope_attention_f16kv(q, ck[l], cv[l], kd, vd, out, 1, ctx + s, H, KV, D, base, neox, ff)

    for s in range(warmup):
        step(s)
    be.sync()
    e0, e1 = be.event(), be.event()
    e0.record()
    for s in range(warmup, warmup + steps):
        step(s)
    e1.record()
    ms = e0.elapsed_ms(e1) / steps
    byts = sum(NL * 4 * KV * D * (ctx + s + 1) for s in range(warmup, warmup + steps)) / steps
    KernelTiming.enable(True, only=KernelTiming.DECODE_PARTIAL)
    for s in range(warmup + steps, warmup + steps + stamped):
        step(s)
    be.sync()
    pm, pn = KernelTiming.read(KernelTiming.DECODE_PARTIAL)
    KernelTiming.enable(False)
    # The 8192-token prefill over the same fp16 caches: append fused with the staging, then the MFMA kernel (rows
    # below FP32_PREFIX_ROWS in fp32 from the fp16 cache) and the recomputation, as the fp32-cache prefill runs.
    n_pre = 8192
    qp, kp, vp, op_ = be.alloc(n_pre * H * D), be.alloc(n_pre * KV * D), be.alloc(n_pre * KV * D), be.alloc(n_pre * H * D)
    for p_, n_, sd in ((qp, n_pre * H * D, 11), (kp, n_pre * KV * D, 12), (vp, n_pre * KV * D, 13)):
        be.fill_normal(p_, n_, seed=sd)

    def prefill():
        for l in range(NL):
            be.append_rope_attention_f16kv(qp, ck[l], cv[l], kp, vp, op_, n_pre, 0, H, KV, D, base, neox, ff)

    for _ in range(4):
        prefill()
    be.sync()
    e0.record()
    for _ in range(3):
        prefill()
    e1.record()
    pre_ms = e0.elapsed_ms(e1) / 3
    pre_tflops = prefill_flops(H, D, 0, n_pre) * NL / (pre_ms * 1e-3) / 1e12
    for p_ in ck + cv + [q, kd, vd, out, qp, kp, vp, op_]:
        be.free(p_)
    gbs = byts / (ms * 1e-3) / 1e9
    part_us = pm / pn * 1e3
    part_rows = ctx + warmup + steps + (stamped + 1) / 2  # the stamped steps' mean context
    part_gbs = 4 * KV * D * part_rows / (part_us * 1e-6) / 1e9
    log(f"fp16 KV decode: {ms:.4f} ms/step over {NL} layers -> {gbs:.0f} GB/s of fp16 rows ({gbs / HBM_PEAK_GBS:.1%}); "
        f"partial kernel {part_us:.2f} us -> {part_gbs:.0f} GB/s; 8k prefill over fp16 caches {pre_ms:.3f} ms for "
        f"{NL} layers -> {pre_tflops:.1f} TFLOP/s")
    return {"metric": "decode attn over fp16 KV caches (extension), HBM GB/s of the fp16 rows read",
            "value": round(gbs, 1), "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "ms_per_step": round(ms, 4),
            "layers": NL, "ctx": ctx, "steps": steps,
            "partial_kernel": {"avg_launch_us": round(part_us, 3), "value": round(part_gbs, 1), "unit": "GB/s"},
            "prefill_8k": {"value": round(pre_tflops, 2), "unit": "TFLOP/s", "ms_per_prefill_16_layers": round(pre_ms, 4),
                           "note": "append_rope_attention_f16kv, 8192 rows per layer: the append fused with the "
                                   "staging, the MFMA kernel and the recomputation over fp16 caches"}}


def qkv_projection(be, steps, warmup, chunk=512, chunk_reps=3):
    """The QKV projection feeding the attention path (transformer.cpp:171-194) at the Llama-3.2-1B shape: F16
    weights wq [2048, 2048], wk and wv [512, 2048] per layer, 16 layers, one matmul_multi per layer writing q and the
    new K/V cache rows. Decode: one token per step (the gemv route: weight bytes streamed once per layer);
    prefill: chunks of `chunk` rows (the F16 GEMM route: each activation row split into fp16 hi + lo parts by one
    launch, then the three weights in one MFMA GEMM launch, fp32-grade results). Weights start in host memory and
    are copied to HBM on the first (untimed) call, as a model's are."""
    shape = configs.LLAMA32_1B
    E, Q, kvw, NL = shape.n_embd, shape.n_heads * shape.head_dim, shape.n_kv_heads * shape.head_dim, 16
    rng = np.random.default_rng(17)
    ws = [[(rng.standard_normal((r, E), dtype=np.float32) * 0.02).astype(np.float16) for r in (Q, kvw, kvw)]
          for _ in range(NL)]
    rows = warmup + steps
    x = be.alloc(max(rows, chunk) * E)
    be.fill_normal(x, max(rows, chunk) * E, seed=41)
    q = be.alloc(max(rows, chunk) * Q)
    kc = [be.alloc(max(rows, chunk) * kvw) for _ in range(NL)]
    vc = [be.alloc(max(rows, chunk) * kvw) for _ in range(NL)]

    def step(s, n):
        for l in range(NL):
            be.matmul_multi(ws[l], x.at(s * E), [q, kc[l].at(s * kvw), vc[l].at(s * kvw)], n)

    def timed(fn, reps):
        e0, e1 = be.event(), be.event()
        e0.record()
        for r in range(reps):
            fn(r)
        e1.record()
        return e0.elapsed_ms(e1)

    for s in range(warmup):
        step(s, 1)  # first call uploads the weights
    be.sync()
    dec_ms = timed(lambda r: step(warmup + r, 1), steps)
    KernelTiming.enable(True, only=KernelTiming.GEMV)
    timed(lambda r: step(warmup + r, 1), steps)
    be.sync()
    gemv_ms, gemv_n = KernelTiming.read(KernelTiming.GEMV)
    KernelTiming.enable(False)
    w_bytes = E * (Q + 2 * kvw) * 2
    alg_bytes = w_bytes + E * 4 + (Q + 2 * kvw) * 4  # weights, the x row, the q/k/v rows
    dec_gbs = NL * steps * alg_bytes / (dec_ms * 1e-3) / 1e9
    gemv_us = gemv_ms / gemv_n * 1e3
    gemv_gbs = alg_bytes / (gemv_us * 1e-6) / 1e9
    for r in range(2):
        step(0, chunk)  # the first GEMM calls load the kernels' code
    be.sync()
    pre_ms = timed(lambda r: step(0, chunk), chunk_reps)
    flops = 2 * chunk * E * (Q + 2 * kvw)
    pre_tflops = NL * chunk_reps * flops / (pre_ms * 1e-3) / 1e12
    # each kernel stamped alone in a pass of its own; per layer: the activation split, the GEMM launch(es) and, for
    # weights whose K is cut into ranges, the launch summing the ranges' partials
    layer_calls = chunk_reps * NL
    per_layer = {}
    for kern in (KernelTiming.GEMM, KernelTiming.GEMM_REDUCE, KernelTiming.SPLIT_ACTS):
        KernelTiming.enable(True, only=kern)
        timed(lambda r: step(0, chunk), chunk_reps)
        be.sync()
        ms, cnt = KernelTiming.read(kern)
        per_layer[kern] = (ms / layer_calls * 1e3, cnt)
    KernelTiming.enable(False)
    gemm_us, gemm_n = per_layer[KernelTiming.GEMM]
    reduce_us, reduce_n = per_layer[KernelTiming.GEMM_REDUCE]
    split_us = per_layer[KernelTiming.SPLIT_ACTS][0]
    gemm_tflops = flops / ((gemm_us + reduce_us) * 1e-6) / 1e12
    for p in [x, q] + kc + vc:
        be.free(p)
    be.release_weights()
    log(f"qkv projection: decode {dec_ms / steps * 1e3:.1f} us/step over {NL} layers -> {dec_gbs:.0f} GB/s; gemv "
        f"kernel {gemv_us:.2f} us -> {gemv_gbs:.0f} GB/s ({gemv_gbs / HBM_PEAK_GBS:.1%}); prefill chunk {chunk}: "
        f"{pre_ms / chunk_reps / NL * 1e3:.1f} us/layer -> {pre_tflops:.1f} TFLOP/s; F16 GEMM {gemm_us:.2f} us + "
        f"K-range sum {reduce_us:.2f} us per layer -> {gemm_tflops:.1f} TFLOP/s ({gemm_tflops / MFMA_F16_PEAK_TFLOPS:.1%} "
        f"of fp16 MFMA; two MFMA products per multiply-add), activation split {split_us:.2f} us")
    return {"metric": "QKV projection (matmul_multi, F16 weights, llama-3.2-1b shape, 16 layers)",
            "decode": {"value": round(dec_gbs, 1), "unit": "GB/s", "us_per_step": round(dec_ms / steps * 1e3, 2),
                       "steps": steps, "roofline": {"bound": "hbm", "kernel": "gemv_kernel",
                                                    "achieved": round(gemv_gbs, 1), "peak": HBM_PEAK_GBS,
                                                    "unit": "GB/s", "frac": round(gemv_gbs / HBM_PEAK_GBS, 4),
                                                    "avg_launch_us": round(gemv_us, 3), "launches": gemv_n,
                                                    "algorithmic_bytes_per_launch": alg_bytes}},
            "prefill_chunk": {"rows": chunk, "value": round(pre_tflops, 2), "unit": "TFLOP/s",
                              "us_per_layer": round(pre_ms / chunk_reps / NL * 1e3, 2),
                              "frac_of_fp32_peak": round(pre_tflops / FP32_PEAK_TFLOPS, 4),
                              "roofline": {"bound": "mfma", "kernel": "gemm_f16w_kernel",
                                           "achieved": round(gemm_tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                                           "unit": "TFLOP/s", "frac": round(gemm_tflops / MFMA_F16_PEAK_TFLOPS, 4),
                                           "gemm_us_per_layer": round(gemm_us, 3), "launches": gemm_n,
                                           "k_range_sum_us_per_layer": round(reduce_us, 3),
                                           "k_range_sum_launches": reduce_n,
                                           "algorithmic_flops_per_layer": flops,
                                           "mfma_flops_per_layer": 2 * flops,
                                           "duration_method": "GEMM and K-range-sum launches stamped (hipExtLaunchKernel"
                                                              " events), each in a pass of its own; achieved = "
                                                              "flops / (their per-layer sum)"},
                              "split_acts_us": round(split_us, 3),
                              "note": "per layer: one activation-split launch (fp16 hi + lo per row, power-of-two "
                                      "row scale) and one F16-weight MFMA GEMM launch for wq, wk, wv (64 x 64 tiles; "
                                      "K = 2048 is too short for K ranges, so no launch sums ranges; fp32-grade "
                                      "results; no fp32 copy of the weights)"}}


QUANT_NAMES = {2: "Q4_0", 8: "Q8_0", 12: "Q4_K", 14: "Q6_K"}


def quant_projection(be, steps, warmup, chunk=512, chunk_reps=2):
    """The same QKV projection with quantized weights (Llama-3.2-1B shape, 16 layers; synthetic blocks of each
    type): one launch per layer for the three weights, the activation row quantized inside it, bit-exact with the
    reference's quant.cpp. Decode (n = 1): HBM GB/s of the weight blocks (file bytes) streamed per launch, for the
    QKV launch and for the FFN's gate + up launch (2 x 8192 x 2048). Prefill chunks (n = 512): integer-op rate of
    the block dots."""
    from nibble_amd import synth
    shape = configs.LLAMA32_1B
    E, Q, kvw, NL = shape.n_embd, shape.n_heads * shape.head_dim, shape.n_kv_heads * shape.head_dim, 16
    out = {}
    x = be.alloc(chunk * E)
    be.fill_normal(x, chunk * E, seed=43)
    q, kc, vc = be.alloc(chunk * Q), be.alloc(chunk * kvw), be.alloc(chunk * kvw)
    for t, name in QUANT_NAMES.items():
        raws = [[synth.quant_weight(t, r, E, 1000 * l + i) for i, r in enumerate((Q, kvw, kvw))] for l in range(NL)]
        ws = [[nibble_amd.weight(raws[l][i], shape=(r, E), dtype=t) for i, r in enumerate((Q, kvw, kvw))]
              for l in range(NL)]
        w_bytes = sum(r.nbytes for r in raws[0])

        def step(n):
            for l in range(NL):
                be.matmul_multi(ws[l], x, [q, kc, vc], n)

        for _ in range(warmup):
            step(1)
        be.sync()
        e0, e1 = be.event(), be.event()
        e0.record()
        for _ in range(steps):
            step(1)
        e1.record()
        dec_ms = e0.elapsed_ms(e1)
        KernelTiming.enable(True, only=KernelTiming.QGEMV)
        for _ in range(steps):
            step(1)
        be.sync()
        g_ms, g_n = KernelTiming.read(KernelTiming.QGEMV)
        KernelTiming.enable(False)
        step(chunk)
        be.sync()
        e0.record()
        for _ in range(chunk_reps):
            step(chunk)
        e1.record()
        pre_ms = e0.elapsed_ms(e1) / chunk_reps
        alg = w_bytes + E * 4 + (Q + 2 * kvw) * 4
        us = g_ms / g_n * 1e3
        gbs = alg / (us * 1e-6) / 1e9
        tops = NL * 2 * chunk * E * (Q + 2 * kvw) / (pre_ms * 1e-3) / 1e12
        be.release_weights()
        # the FFN's gate + up projection (2 x 8192 x 2048) at decode: the largest single-row launch of a layer
        FF = 8192
        fraws = [[synth.quant_weight(t, FF, E, 7000 + 10 * l + i) for i in range(2)] for l in range(4)]
        fws = [[nibble_amd.weight(r, shape=(FF, E), dtype=t) for r in rl] for rl in fraws]
        g_buf, u_buf = be.alloc(FF), be.alloc(FF)
        for l in range(4):
            be.matmul_multi(fws[l], x, [g_buf, u_buf], 1)
        be.sync()
        KernelTiming.enable(True, only=KernelTiming.QGEMV)
        for _ in range(steps // 4):
            for l in range(4):
                be.matmul_multi(fws[l], x, [g_buf, u_buf], 1)
        be.sync()
        f_ms, f_n = KernelTiming.read(KernelTiming.QGEMV)
        KernelTiming.enable(False)
        be.free(g_buf)
        be.free(u_buf)
        f_alg = sum(r.nbytes for r in fraws[0]) + E * 4 + 2 * FF * 4
        f_us = f_ms / f_n * 1e3
        f_gbs = f_alg / (f_us * 1e-6) / 1e9
        out[name] = {"decode": {"avg_launch_us": round(us, 3), "value": round(gbs, 1), "unit": "GB/s",
                                "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_launch": alg,
                                "us_per_step_16_layers": round(dec_ms / steps * 1e3, 1)},
                     "ffn_gate_up_decode": {"avg_launch_us": round(f_us, 3), "value": round(f_gbs, 1), "unit": "GB/s",
                                            "frac": round(f_gbs / HBM_PEAK_GBS, 4),
                                            "algorithmic_bytes_per_launch": f_alg},
                     "prefill_chunk": {"rows": chunk, "us_per_layer": round(pre_ms / NL * 1e3, 1),
                                       "value": round(tops, 2), "unit": "TOPS (block-dot MACs x 2)"}}
        log(f"quant projection {name}: QKV decode launch {us:.2f} us -> {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%}) of "
            f"{alg / 1e6:.2f} MB; FFN gate+up decode {f_us:.2f} us -> {f_gbs:.0f} GB/s ({f_gbs / HBM_PEAK_GBS:.1%}) of "
            f"{f_alg / 1e6:.2f} MB; QKV prefill chunk {chunk}: {pre_ms / NL * 1e3:.1f} us/layer -> {tops:.1f} TOPS")
        be.release_weights()
    for p in (x, q, kc, vc):
        be.free(p)
    return {"metric": "QKV projection with quantized weights (bit-exact with quant.cpp), llama-3.2-1b shape",
            "types": out}


def mfma_loop_ceiling(be, waves_per_simd=3, iters=1 << 14, reps=5):
    """Sustained rate of the MFMA pipes on this GPU: a launch whose waves issue nothing but independent
    v_mfma_f32_32x32x16_f16 (the prefill kernel's instruction) at the prefill kernel's occupancy (3 waves per SIMD at
    its 168 VGPRs), timed from dispatch-stamped events. Under a sustained MFMA load the engine clock sits below the
    2.4 GHz the published peak assumes, so this is the rate the prefill kernel could reach with its softmax work
    fully hidden."""
    cus = be.cu_count()
    out = be.alloc(cus * waves_per_simd * 256)
    nibble_amd.mfma_loop(out, iters, waves_per_simd, cus)  # warm-up (clock ramp)
    nibble_amd.mfma_loop(out, iters, waves_per_simd, cus)
    be.sync()
    KernelTiming.enable(True, only=KernelTiming.CALIBRATION)
    flops = sum(nibble_amd.mfma_loop(out, iters, waves_per_simd, cus) for _ in range(reps))
    ms, n = KernelTiming.read(KernelTiming.CALIBRATION)
    KernelTiming.enable(False)
    be.free(out)
    assert n == reps
    return {"tflops": round(flops / (ms * 1e-3) / 1e12, 1), "waves_per_simd": waves_per_simd,
            "avg_launch_us": round(ms / n * 1e3, 1), "instruction": "v_mfma_f32_32x32x16_f16",
            "method": "nbhs_mfma_loop_f16: 8 independent MFMAs per iteration over 4 accumulator chains, nothing "
                      "else in the loop; dispatch-stamped events"}


COPY_CAL_BYTES = 1 << 30  # calibration copy for the HBM byte counters: 1 GiB read + 1 GiB written
PROBE_DECODE_STEPS = 8
# 8192-row prefills after the calibration copy; the counters are read from the last one, after the others have
# brought the engine clock up from the decode phase (a single cold launch under the profiler runs up to 25 % slower)
PROBE_PREFILLS = 4


def probe():
    """Short run for one `rocprofv3 --pmc` pass: layer 0 of config 4 only. Dispatch order: fill kernels, then
    PROBE_DECODE_STEPS decode steps at 32768+s ctx (split-context partial with the K/V append, combine), then one
    COPY_CAL_BYTES device copy (the calibration kernel of known size), then PROBE_PREFILLS 8192-row prefills into
    the same rows (K/V append fused with the fp16 staging, then the MFMA kernel with the fp32 rows in the same
    launch); the counters are taken from the last. Byte counts per dispatch do not depend on the data."""
    shape = configs.LLAMA32_1B
    H, KV, D = shape.n_heads, shape.n_kv_heads, shape.head_dim
    base, neox, ff = shape.rope_base, shape.neox, shape.freq_factors()
    n_pre, ctx = 8192, 32768
    cap, row = ctx + PROBE_DECODE_STEPS, KV * D
    be = nibble_amd.HipBackend(0)
    be.reserve(cap, H, n_pre, 8192)
    be.reserve_attention(KV, D)
    be.reserve_rope(D, base, neox, ff)
    ck, cv = be.alloc(cap * row), be.alloc(cap * row)
    be.fill_normal(ck, ctx * row, seed=1)
    be.fill_normal(cv, ctx * row, seed=2)
    qd, kd, vd = be.alloc(H * D), be.alloc(row), be.alloc(row)
    for p_, n_ in ((qd, H * D), (kd, row), (vd, row)):
        be.fill_normal(p_, n_, seed=3)
    out = be.alloc(n_pre * H * D)
    cal_floats = COPY_CAL_BYTES // 4
    src, dst = be.alloc(cal_floats), be.alloc(cal_floats)
    be.fill_normal(src, cal_floats, seed=4)
    q_pre, k_pre, v_pre = be.alloc(n_pre * H * D), be.alloc(n_pre * row), be.alloc(n_pre * row)
    for p_, n_ in ((q_pre, n_pre * H * D), (k_pre, n_pre * row), (v_pre, n_pre * row)):
        be.fill_normal(p_, n_, seed=5)
    be.sync()
    for s in range(PROBE_DECODE_STEPS):
        be.append_rope_attention(qd, ck, cv, kd, vd, out, 1, ctx + s, H, KV, D, base, neox, ff)
    be.copy(dst, src, cal_floats)
    for _ in range(PROBE_PREFILLS):
        be.append_rope_attention(q_pre, ck, cv, k_pre, v_pre, out, n_pre, 0, H, KV, D, base, neox, ff)
    be.sync()
    be.close()
    log("probe done")


def _counter_rows(csv_path):
    import csv
    with open(csv_path, newline="") as f:
        return [(int(r["Dispatch_Id"]), r["Kernel_Name"], r["Counter_Name"], float(r["Counter_Value"]))
                for r in csv.DictReader(f)]


def _gpu_agent(info_csv):
    """(XCD count, SIMD count) of the GPU agent, from rocprofv3's agent-info file."""
    import csv
    with open(info_csv, newline="") as f:
        for r in csv.DictReader(f):
            if r.get("Agent_Type") == "GPU":
                return int(r["Num_Xcc"]), int(r["Simd_Count"])
    return None


def _pmc_pass(prof, counters, d, timeout_s):
    """One `rocprofv3 --pmc` run over probe(): {(dispatch, kernel): {counter: value summed over its instances}} and
    the agent-info path, or None (reason logged)."""
    import subprocess

    cmd = [prof, "--pmc", *counters, "-f", "csv", "-d", d, "-o", "run", "--",
           sys.executable, "-u", os.path.abspath(__file__), "--probe"]
    log("counters: " + " ".join(cmd))
    try:
        r = subprocess.run(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"), timeout=timeout_s,
                           stdout=subprocess.DEVNULL, stderr=subprocess.PIPE, text=True)
    except subprocess.TimeoutExpired:
        log(f"counters: {' '.join(counters)} pass timed out")
        return None
    found = {f: os.path.join(dp, f) for dp, _, fs in os.walk(d) for f in fs
             if f.endswith("counter_collection.csv") or f.endswith("agent_info.csv")}
    data = next((p for f, p in found.items() if f.endswith("counter_collection.csv")), None)
    info = next((p for f, p in found.items() if f.endswith("agent_info.csv")), None)
    if not data or "probe done" not in (r.stderr or ""):
        log(f"counters: {' '.join(counters)} pass failed (rc {r.returncode}): {(r.stderr or '')[-400:]}")
        return None
    sums = {}
    for disp, name, counter, val in _counter_rows(data):
        per = sums.setdefault((disp, name), {})
        per[counter] = per.get(counter, 0.0) + val
    return sums, info


def measure_traffic(out_dir, timeout_s=150):
    """HBM bytes per launch of the decode partial kernel and the prefill MFMA kernel: two `rocprofv3 --pmc` passes
    over probe() (FETCH_SIZE, then WRITE_SIZE, each in KiB per dispatch, summed over the dispatch's counter
    instances), each scaled by the factor that makes the same counter read the known bytes of the calibration copy.
    A third pass reads the prefill kernel's MFMA busy cycles (SQ_VALU_MFMA_BUSY_CYCLES, summed over SIMDs) against
    its active cycles (GRBM_GUI_ACTIVE, summed over XCDs): the MFMA pipes' busy fraction, rocprofv3's MfmaUtil.
    Runs the profiler as child processes; returns a dict, or None with a logged reason."""
    import shutil

    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(prof):
        log("traffic: rocprofv3 not found")
        return None
    per = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        got = _pmc_pass(prof, [counter], os.path.join(out_dir, f"pmc_{counter.lower()}"), timeout_s)
        if got is None:
            return None
        rows = sorted((disp, name, v[counter]) for (disp, name), v in got[0].items() if counter in v)
        cal = [x for x in rows if "copy_kernel" in x[1]]
        if len(cal) != 1:
            log(f"traffic: expected one calibration copy dispatch, found {len(cal)}")
            return None
        cal_disp = cal[0][0]
        dec = [v for disp, name, v in rows if "attn_decode_rows" in name and disp < cal_disp]
        pre = [v for disp, name, v in rows if "attn_prefill_kernel" in name and disp > cal_disp]
        if len(dec) != PROBE_DECODE_STEPS or len(pre) != PROBE_PREFILLS:
            log(f"traffic: unexpected dispatch counts (decode {len(dec)}, prefill {len(pre)})")
            return None
        per[counter] = {"cal_kib": cal[0][2], "decode_kib": float(np.mean(dec)), "prefill_kib": pre[-1]}
    f_fetch = COPY_CAL_BYTES / 1024.0 / per["FETCH_SIZE"]["cal_kib"]
    f_write = COPY_CAL_BYTES / 1024.0 / per["WRITE_SIZE"]["cal_kib"]

    def traffic(key):
        return 1024.0 * (per["FETCH_SIZE"][key] * f_fetch + per["WRITE_SIZE"][key] * f_write)

    out = {"decode_bytes": traffic("decode_kib"), "prefill_bytes": traffic("prefill_kib"),
           "fetch_factor": f_fetch, "write_factor": f_write, "raw_kib": per, "prefill_mfma": None}
    counters = ["SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"]
    got = _pmc_pass(prof, counters, os.path.join(out_dir, "pmc_mfma_busy"), timeout_s)
    agent = _gpu_agent(got[1]) if got and got[1] else None
    pre = [v for (disp, name), v in sorted(got[0].items()) if "attn_prefill_kernel" in name] if got else []
    if agent and len(pre) == PROBE_PREFILLS and all(c in pre[-1] for c in counters) and pre[-1]["GRBM_GUI_ACTIVE"] > 0:
        n_xcc, n_simd = agent
        last = pre[-1]
        gui = last["GRBM_GUI_ACTIVE"] / n_xcc  # cycles the launch kept each XCD active
        out["prefill_mfma"] = {"mfma_busy_frac": last["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui * n_simd),
                               "active_cycles": gui, "busy_cycles_per_simd": last["SQ_VALU_MFMA_BUSY_CYCLES"] / n_simd,
                               "active_cycles_each": [round(p["GRBM_GUI_ACTIVE"] / n_xcc) for p in pre]}
    else:
        log("counters: no MFMA busy figure for the prefill kernel")
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64, help="timed decode steps (config 4 decodes 64 tokens)")
    ap.add_argument("--warmup", type=int, default=8, help="untimed decode steps before the timed ones")
    ap.add_argument("--prefill-reps", type=int, default=3)
    ap.add_argument("--prefill-warmup", type=int, default=8,
                    help="untimed prefill passes first: the compute clock takes some 20-40 ms of sustained MFMA load "
                         "to settle")
    ap.add_argument("--cpu-seconds", type=float, default=16.0, help="budget of the CPU baseline samples")
    ap.add_argument("--cfg5-steps", type=int, default=4,
                    help="timed steps of the config-5 ragged batch (0: skip; 2 untimed steps precede them)")
    ap.add_argument("--qkv-steps", type=int, default=32,
                    help="timed decode steps of the QKV projection figure (0: skip it)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc passes (child processes, about 10 s each) that measure HBM "
                         "bytes per launch for roofline.traffic")
    ap.add_argument("--traffic-dir", default=os.path.join(ROOT, "gpurun_out", "traffic"))
    ap.add_argument("--probe", action="store_true", help="internal: the short run the traffic passes profile")
    args = ap.parse_args()
    if args.probe:
        probe()
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "multi-GPU sharding is a design note of this repository, not run", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.steps > 64 or args.warmup < 0:
        sys.exit("--steps must be in 1..64 (config 4 decodes 64 tokens), --warmup >= 0")

    shape = configs.LLAMA32_1B
    H, KV, D, NL = shape.n_heads, shape.n_kv_heads, shape.head_dim, shape.n_layers
    base, neox, ff = shape.rope_base, shape.neox, shape.freq_factors()
    n_pre, ctx, max_steps = 8192, 32768, 64
    cap = ctx + max_steps
    row = KV * D

    be = nibble_amd.HipBackend(0)
    be.reserve(cap, H, n_pre, 8192)
    be.reserve_attention(KV, D)
    be.reserve_rope(D, base, neox, ff)
    log(f"device CUs: {be.cu_count()}; allocating caches for {NL} layers x {cap} rows")
    ck = [be.alloc(cap * row) for _ in range(NL)]
    cv = [be.alloc(cap * row) for _ in range(NL)]
    for l in range(NL):  # seeded rows 8192..32767 (the prefill writes rows 0..8191)
        be.fill_normal(ck[l].at(n_pre * row), (ctx - n_pre) * row, seed=(4 << 32) | (l << 8) | configs.T_KCACHE)
        be.fill_normal(cv[l].at(n_pre * row), (ctx - n_pre) * row, seed=(4 << 32) | (l << 8) | configs.T_VCACHE)
    q_pre = [be.alloc(n_pre * H * D) for _ in range(NL)]
    k_pre = [be.alloc(n_pre * row) for _ in range(NL)]
    v_pre = [be.alloc(n_pre * row) for _ in range(NL)]
    for l in range(NL):
        be.fill_normal(q_pre[l], n_pre * H * D, seed=(4 << 32) | (l << 8) | configs.T_Q)
        be.fill_normal(k_pre[l], n_pre * row, seed=(4 << 32) | (l << 8) | configs.T_K)
        be.fill_normal(v_pre[l], n_pre * row, seed=(4 << 32) | (l << 8) | configs.T_V)
    out_pre = be.alloc(n_pre * H * D)
    # decode inputs for every (step, layer)
    qd = be.alloc(max_steps * NL * H * D)
    kd = be.alloc(max_steps * NL * row)
    vd = be.alloc(max_steps * NL * row)
    be.fill_normal(qd, max_steps * NL * H * D, seed=(4 << 32) | (1 << 20) | configs.T_Q)
    be.fill_normal(kd, max_steps * NL * row, seed=(4 << 32) | (1 << 20) | configs.T_K)
    be.fill_normal(vd, max_steps * NL * row, seed=(4 << 32) | (1 << 20) | configs.T_V)
    out_dec = be.alloc(H * D)
    q_pre0_host = be.download(q_pre[0], (n_pre, H, D))  # layer-0 queries (CPU baseline sample)
    be.sync()

    # One layer = KV append with RoPE + attention, through the fused entry point (q rotated on load; on the prefill
    # route the append shares one pass with the fp16 staging).
    def prefill_pass():
        for l in range(NL):
            be.append_rope_attention(q_pre[l], ck[l], cv[l], k_pre[l], v_pre[l], out_pre, n_pre, 0, H, KV, D, base,
                                     neox, ff)

    def prefill_chunked_pass(chunk):
        # as nibble's Transformer runs a prompt: chunks of max_batch rows, each through every layer
        # (transformer.cpp:135-136; max_batch defaults to 512, transformer.h:24)
        row_q = H * D
        for p0 in range(0, n_pre, chunk):
            m = min(chunk, n_pre - p0)
            for l in range(NL):
                be.append_rope_attention(q_pre[l].at(p0 * row_q), ck[l], cv[l], k_pre[l].at(p0 * row),
                                         v_pre[l].at(p0 * row), out_pre.at(p0 * row_q), m, p0, H, KV, D, base, neox,
                                         ff)

    def decode_step(s):
        pos0 = ctx + s
        for l in range(NL):
            i = s * NL + l
            be.append_rope_attention(qd.at(i * H * D), ck[l], cv[l], kd.at(i * row), vd.at(i * row), out_dec, 1,
                                     pos0, H, KV, D, base, neox, ff)

    # ---------------- prefill (also fills cache rows 0..8191 of every layer)
    for _ in range(max(1, args.prefill_warmup)):
        prefill_pass()
    be.sync()
    e0, e1 = be.event(), be.event()
    pre_ms = []
    for _ in range(args.prefill_reps):
        e0.record()
        prefill_pass()
        e1.record()
        pre_ms.append(e0.elapsed_ms(e1))
    pre_ms_med = float(np.median(pre_ms))
    pre_flops = NL * prefill_flops(H, D, 0, n_pre)
    pre_tflops = pre_flops / (pre_ms_med * 1e-3) / 1e12
    log(f"prefill: {pre_ms_med:.3f} ms for {NL} layers -> {pre_tflops:.1f} TFLOP/s")

    # ---------------- per-kernel durations: one more pass of each phase, right after its timed region, whose launches
    # carry start/stop event pairs stamped from the dispatch itself (hipExtLaunchKernel on the launch's own stream;
    # the durations a kernel trace reads), kept out of the timed regions. A pass follows its own phase because the
    # compute clock moves with the load: the first prefill passes after a stretch of decode run several percent slower.
    def timed_pass(run, kernels, alone=None):
        # `alone`: one more pass that stamps only that kernel (the roofline kernel), so the event handling of its
        # neighbours' launches does not change what it is measured against; the others share one pass
        r = {}
        if alone is not None:
            KernelTiming.enable(True, only=alone)
            run()
            be.sync()
            r[alone] = KernelTiming.read(alone)
            KernelTiming.enable(False)
        KernelTiming.enable(True)
        run()
        be.sync()
        for k in kernels:
            got = KernelTiming.read(k)
            if k != alone:
                r[k] = got
        KernelTiming.enable(False)
        return [r[k] for k in kernels]

    (mfma_ms, mfma_n), (stage_ms, stage_n), (app2_ms, app2_n), (prec_ms, prec_n) = timed_pass(
        prefill_pass, [KernelTiming.PREFILL_MFMA, KernelTiming.STAGE_KV, KernelTiming.APPEND_ROPE,
                       KernelTiming.PREFILL_PRECISE], alone=KernelTiming.PREFILL_MFMA)
    # row tiles each layer's call sent to the split-operand recomputation (its rounding-error estimate over budget)
    recomputed = []
    for l in range(NL):
        be.append_rope_attention(q_pre[l], ck[l], cv[l], k_pre[l], v_pre[l], out_pre, n_pre, 0, H, KV, D, base, neox,
                                 ff)
        recomputed.append(be.prefill_recomputed())
    tiles_per_layer = (n_pre - FP32_PREFIX_ROWS) * (H // KV) // 128 * KV
    log(f"prefill: row tiles recomputed per layer {recomputed} of {tiles_per_layer}")

    # the same prefill in nibble's max_batch = 512 chunks (same rows, same results within rounding)
    prefill_chunked_pass(512)
    be.sync()
    ch_ms = []
    for _ in range(args.prefill_reps):
        e0.record()
        prefill_chunked_pass(512)
        e1.record()
        ch_ms.append(e0.elapsed_ms(e1))
    ch_ms_med = float(np.median(ch_ms))
    ch_tflops = pre_flops / (ch_ms_med * 1e-3) / 1e12
    log(f"prefill in 512-row chunks: {ch_ms_med:.3f} ms for {NL} layers -> {ch_tflops:.1f} TFLOP/s")

    # ---------------- decode: warm-up steps, then exactly K timed steps (re-appending the same positions)
    for s in range(args.warmup):
        decode_step(s % max_steps)
    be.sync()
    e0.record()
    for s in range(args.steps):
        decode_step(s)
    e1.record()
    dec_ms = e0.elapsed_ms(e1)
    be.sync()
    dec_bytes = sum(NL * decode_bytes(KV, D, ctx + s + 1) for s in range(args.steps))
    dec_gbs = dec_bytes / (dec_ms * 1e-3) / 1e9
    log(f"decode: {dec_ms:.3f} ms for {args.steps} steps -> {dec_gbs:.1f} GB/s ({dec_gbs / HBM_PEAK_GBS:.1%})")

    def decode_pass():
        for s in range(args.steps):
            decode_step(s)

    n_roof = args.steps
    (part_ms, part_n), (comb_ms, comb_n), (app_ms, app_n) = timed_pass(
        decode_pass, [KernelTiming.DECODE_PARTIAL, KernelTiming.DECODE_COMBINE, KernelTiming.APPEND_ROPE],
        alone=KernelTiming.DECODE_PARTIAL)
    roof_bytes = sum(NL * decode_bytes(KV, D, ctx + s + 1) for s in range(n_roof))
    dec_kernel_gbs = roof_bytes / (part_ms * 1e-3) / 1e9
    # Beside it, the in-situ figure: the timed region's time per layer-step less the combine's stamped duration (a
    # layer-step is exactly the partial launch and the combine launch), which the per-dispatch events do not inflate.
    assert app_n == 0 and part_n == comb_n, "decode layer-step is not partial + combine"
    part_insitu_us = dec_ms * 1e3 / args.steps / NL - comb_ms / comb_n * 1e3
    # the MFMA launch computes every row of the call: rows >= FP32_PREFIX_ROWS on MFMA, the others in fp32
    mfma_flops = prefill_flops(H, D, 0, n_pre)
    # A prefill layer is three back-to-back launches: K/V append + fp16 staging, the MFMA kernel, and the persistent
    # recomputation of listed row tiles. The roofline figure is the MFMA kernel's measured duration from the pass
    # whose launches carry dispatch-stamped events (the duration a kernel trace reads); beside it, the in-situ
    # figure derived from the timed region (time per layer less the other two kernels' stamped durations).
    assert app2_n == 0 and stage_n == mfma_n == prec_n == NL, "prefill layer is not staging + MFMA + recompute"
    mfma_stamped_us = mfma_ms / mfma_n * 1e3
    prec_us = prec_ms / prec_n * 1e3
    mfma_insitu_us = pre_ms_med * 1e3 / NL - stage_ms / stage_n * 1e3 - prec_us
    mfma_tflops = mfma_flops / (mfma_stamped_us * 1e-6) / 1e12
    log(f"kernels: decode partial avg {part_ms / part_n * 1e3:.2f} us ({dec_kernel_gbs:.0f} GB/s; in situ "
        f"{part_insitu_us:.2f} us), combine avg "
        f"{comb_ms / max(comb_n, 1) * 1e3:.2f} us, separate append launches {app_n}; "
        f"prefill mfma {mfma_stamped_us / 1e3:.3f} ms event-stamped ({mfma_tflops:.1f} TFLOP/s; in situ "
        f"{mfma_insitu_us / 1e3:.3f} ms), append+stage avg {stage_ms / max(stage_n, 1) * 1e3:.1f} us, "
        f"recompute avg {prec_us:.1f} us")

    result = {
        "metric": METRIC,
        "value": round(dec_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "BASELINE config 4: llama-3.2-1b shape (32 Q / 8 KV heads, hd 64, RoPE theta 5e5 with "
                               "llama3 factors), 16 layers; decode 1 token/step at 32768+s ctx after an 8192-token "
                               "prefill; value = decode", "layers": NL, "ctx": ctx, "prefill_tokens": n_pre,
                   "global_batch": 1, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(dec_kernel_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dec_kernel_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "attn_decode_rows<64,4,float>",
                     "avg_launch_us": round(part_ms / part_n * 1e3, 3), "launches": part_n,
                     "algorithmic_bytes_per_launch": int(roof_bytes / part_n),
                     "avg_launch_us_in_situ": round(part_insitu_us, 3),
                     "achieved_in_situ": round(roof_bytes / part_n / (part_insitu_us * 1e-6) / 1e9, 1),
                     "in_situ_method": "timed-region time per layer-step minus the combine's event-stamped duration"},
        "prefill": {"metric": "prefill attn TFLOP/s @8k", "value": round(pre_tflops, 2), "unit": "TFLOP/s",
                    "ms_per_prefill_16_layers": round(pre_ms_med, 4), "reps": args.prefill_reps,
                    "chunked_512": {"value": round(ch_tflops, 2), "unit": "TFLOP/s",
                                    "ms_per_prefill_16_layers": round(ch_ms_med, 4),
                                    "note": "the same 8192 rows as nibble's Transformer runs them: 16 chunks of "
                                            "max_batch = 512 rows, each through all 16 layers"},
                    "dtype": f"f16 MFMA operands, f32 accumulate and softmax (rows < {FP32_PREFIX_ROWS}: f32, in the same launch); "
                             "row tiles over the rounding-error budget recomputed with split (hi + lo) f16 operands",
                    "recomputed_tiles_per_layer": recomputed, "row_tiles_per_layer": tiles_per_layer,
                    "roofline": {"bound": "mfma", "achieved": round(mfma_tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                                 "unit": "TFLOP/s", "frac": round(mfma_tflops / MFMA_F16_PEAK_TFLOPS, 4),
                                 "traffic": None, "kernel": "attn_prefill_kernel<64>",
                                 "avg_launch_us": round(mfma_stamped_us, 2), "launches": mfma_n,
                                 "duration_method": "dispatch-stamped start/stop events of each launch "
                                                    "(hipExtLaunchKernel) in one untimed pass of 16 layers that "
                                                    "stamps this kernel alone",
                                 "avg_launch_us_in_situ": round(mfma_insitu_us, 2),
                                 "in_situ_method": "timed-region time per layer minus the staging and recompute "
                                                   "kernels' stamped durations",
                                 "algorithmic_flops_per_launch": mfma_flops,
                                 # fp32 Q rows read and output rows written, fp16 staged K and V^T read once,
                                 # fp32 cache K and V rows of the fp32 rows' window read once
                                 "algorithmic_bytes_per_launch": int(2 * 4 * n_pre * H * D + 2 * 2 * n_pre * KV * D
                                                                     + 2 * 4 * FP32_PREFIX_ROWS * KV * D)}},
        "kernels_us": {"decode_combine": round(comb_ms / max(comb_n, 1) * 1e3, 3),
                       # the decode step's K/V append rides in the partial kernel: no launches of its own
                       "append_rope_decode": round(app_ms / app_n * 1e3, 3) if app_n else None,
                       "append_rope_prefill": round(app2_ms / app2_n * 1e3, 2) if app2_n else None,
                       "append_stage_kv_f16": round(stage_ms / max(stage_n, 1) * 1e3, 2),
                       "prefill_recompute": round(prec_us, 2)},
    }
    ceil = mfma_loop_ceiling(be, waves_per_simd=3)
    result["prefill"]["roofline"]["mfma_loop_ceiling"] = dict(
        ceil, frac_of_ceiling=round(mfma_tflops / ceil["tflops"], 4))
    log(f"mfma loop ceiling: {ceil['tflops']:.1f} TFLOP/s at {ceil['waves_per_simd']} waves/SIMD; prefill mfma "
        f"kernel at {mfma_tflops / ceil['tflops']:.1%} of it")
    if args.cfg5_steps > 0:
        result["config5"] = ragged_decode(be, args.cfg5_steps, 2)
    if args.cfg5_steps > 0:
        result["decode_f16kv"] = f16kv_decode(be, 32, 4)
    if args.qkv_steps > 0:
        result["qkv_projection"] = qkv_projection(be, args.qkv_steps, 4)
        result["quant_projection"] = quant_projection(be, args.qkv_steps, 4)
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(be, shape, ck[0], cv[0], qd, ctx, q_pre0_host, args.cpu_seconds)
    be.close()
    if not args.no_traffic:
        t = measure_traffic(args.traffic_dir)
        if t is not None:
            note = (f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per dispatch x calibration factors {t['fetch_factor']:.4f} "
                    f"/ {t['write_factor']:.4f} (known-size {COPY_CAL_BYTES >> 20} MiB copy kernel)")
            result["roofline"]["traffic"] = int(t["decode_bytes"])
            result["roofline"]["traffic_method"] = note
            result["prefill"]["roofline"]["traffic"] = int(t["prefill_bytes"])
            log(f"traffic: decode partial {t['decode_bytes'] / 1e6:.2f} MB/launch (algorithmic "
                f"{result['roofline']['algorithmic_bytes_per_launch'] / 1e6:.2f} MB), prefill mfma "
                f"{t['prefill_bytes'] / 1e6:.2f} MB/launch; raw {json.dumps(t['raw_kib'])}")
            m = t["prefill_mfma"]
            if m is not None:
                # MFMA pipes' busy share of the launch's active cycles (rocprofv3 MfmaUtil), and the clock the
                # active cycles imply over the same launch in the probe (each launch alone under the profiler)
                result["prefill"]["roofline"]["mfma_busy_frac"] = round(m["mfma_busy_frac"], 4)
                result["prefill"]["roofline"]["mfma_busy_method"] = (
                    "rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x SIMDs), the last of the probe's prefill launches")
                log(f"counters: prefill mfma busy {m['mfma_busy_frac']:.1%} of {m['active_cycles']:.0f} active cycles "
                    f"(the last of {PROBE_PREFILLS} launches; each: {m['active_cycles_each']})")
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
