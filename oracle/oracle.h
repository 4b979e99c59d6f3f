/*
 * CPU oracle for nibble's attention path. TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's scalar and AVX2 attention-path kernels, used solely as the checker
 * for the HIP backend: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * never as the thing measured or shipped. The product path (nibble_amd/) does not link or call anything here.
 *
 * Each function names the reference file:line it restates (paths relative to the nibble source tree).
 * Pins (how each function is checked, see tests/test_oracle.py):
 *   orc_rope               bit-exact vs the compiled reference (oracle/_ref) and the committed fixtures;
 *                          known answers of tests/test_ref_ops.cpp:41-70; fp64 closed form.
 *   orc_softmax_inplace    known answer of test_ref_ops.cpp:130-135; bit-exact vs oracle/_ref through attention.
 *   orc_attention_scalar   bit-exact vs oracle/_ref and fixtures; known answers of test_ref_ops.cpp:73-95;
 *                          fp64 brute force within 2e-6.
 *   orc_attention_avx2     bit-exact vs oracle/_ref and fixtures; the 2e-6*qscale contract of
 *                          tests/test_ops.cpp:196-216 against orc_attention_scalar.
 *   orc_exp_ps             <= 2e-7 relative vs exp() over [-88, 88] (simd_helpers_test.cpp:92-137 contract).
 *   orc_attention_f64      independent fp64 brute force (tests/naive_llama.h:118-134 pattern); known answers.
 *   orc_matmul             bit-exact vs the compiled reference's scalar matmul_rows (oracle/_ref), F32 and F16
 *                          weights; fp64 brute force; the reference's AVX2 tier within float rounding.
 *   orc_fp16_to_fp32       every one of the 65536 halves (NaN payloads included) against numpy's exact conversion.
 *   orc_add_bias           bit-exact vs the compiled reference's cpu::add_bias.
 *   orc_embed              bit-exact vs the compiled reference's cpu::embed (F32 and F16 tables, bad ids rejected).
 *   orc_rmsnorm            bit-exact vs the compiled reference's scalar cpu::rmsnorm; its AVX2 tier within 1 ulp;
 *                          closed form for constant rows; fp64 brute force.
 *   orc_add                bit-exact vs the compiled reference's cpu::add and numpy.
 *   orc_silu_mul           bit-exact vs the compiled reference's scalar cpu::silu_mul (same libm expf); fp64 closed
 *                          form within 2 ulp; silu(0) = 0 and the large-|g| limits.
 *   orc_quantize_q8_0/_q8_1/_q8_k, orc_dequantize, orc_dot, orc_matmul_q (quant.c): the golden vectors of the
 *                          reference's tests/data/quant_golden.inc (llama.cpp's own outputs) and bit-exact vs the
 *                          compiled reference's quant.cpp and CpuBackend::matmul on random blocks of every type.
 *   orc_llama3_freq_factors  closed form of llama.cpp's Llama-3 rope scaling (third-party, not vendored):
 *                          checked against its defining properties (band limits, continuity at both edges,
 *                          monotonicity). Bit-level parity with the converter's float32 output is UNPINNED.
 */
#ifndef NIBBLE_ORACLE_H
#define NIBBLE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ref_ops.cpp:166-185 (cpu::rope). In place on x[n, n_heads, head_dim]; freq_factors is NULL or head_dim/2
 * floats. neox != 0 pairs (i, i + head_dim/2), else (2i, 2i+1) (config.cpp:24). */
void orc_rope(float* x, int64_t n, int64_t n_heads, int64_t head_dim, int64_t pos0, float freq_base, int neox,
              const float* freq_factors);

/* ref_ops.cpp:66-77 (cpu::softmax_inplace): float max, expf, double sum, float(1/sum) scaling. */
void orc_softmax_inplace(float* x, int64_t n);

/* ref_ops.cpp:188-214 (cpu::attention_heads): heads [head_begin, head_end); scratch holds pos0 + n floats. */
void orc_attention_scalar(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                          int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t head_begin,
                          int64_t head_end, float* scratch);

/* simd/ops.cpp:104-139 (simd::avx2::attention_heads) with exp_sub_sum (:31-51), exp_ps (simd.h:103-126) and
 * hsum_ps (simd.h:37-42). Returns -1 (and does nothing) when this build or CPU lacks AVX2/FMA. */
int orc_attention_avx2(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                       int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t head_begin, int64_t head_end,
                       float* scratch);

/* simd.h:103-126 (exp_ps), 8 lanes at a time over x[0..n) into y; -1 without AVX2. */
int orc_exp_ps(const float* x, float* y, int64_t n);

/* 1 when the AVX2 restatement is compiled in and the CPU supports AVX2+FMA+F16C. */
int orc_have_avx2(void);

/* cpu_backend.cpp:271-290 (CpuBackend::attention): one task per head on a pool of `threads` threads
 * (thread_pool.cpp:114-137 parallel_for with chunk 1, caller participates), scratch slot h*(pos0+n).
 * use_avx2 selects orc_attention_avx2 (the production tier, dispatch.cpp:123-136), else the scalar path.
 * scratch: n_heads*(pos0+n) floats. Returns 0, or -1 if use_avx2 is requested without AVX2. */
int orc_attention_heads_parallel(const float* q, const float* k, const float* v, float* out, int64_t n,
                                 int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int threads,
                                 int use_avx2, float* scratch);

/* Independent fp64 brute force (tests/naive_llama.h:118-134 pattern) on the same fp32 inputs; out is double. */
void orc_attention_f64(const float* q, const float* k, const float* v, double* out, int64_t n, int64_t pos0,
                       int64_t n_heads, int64_t n_kv_heads, int64_t head_dim);

/* IEEE binary16 -> binary32, exact (every half is a float), as fp16.h:18-41 converts F16 weights. */
float orc_fp16_to_fp32(uint16_t h);
/* The same over n halves into memory (a float return value can quiet a signalling NaN on its way out). */
void orc_fp16_to_fp32_n(const uint16_t* h, float* out, int64_t n);

/* ref_ops.cpp:109-135 (cpu::matmul_rows, float weights): y[t*out + r] = sum_k x[t*in + k] * w[r*in + k] for
 * t < n, r < out, each dot accumulated left to right in float with no FMA (this file is built with
 * -ffp-contract=off, as ref_ops.cpp is, CMakeLists.txt:72-73). w_type 0 = F32 (floats), 1 = F16 (halves, converted
 * exactly). Returns -1 for another w_type. */
int orc_matmul(int w_type, const void* w, int64_t in, int64_t out, const float* x, float* y, int64_t n);

/* ref_ops.cpp:154-160 (cpu::add_bias): x[t*d + i] += b[i] for t < n. */
void orc_add_bias(float* x, const float* b, int64_t d, int64_t n);

/* ref_ops.cpp:80-99 (cpu::embed, float tables): out[t*d ..] = row ids[t] of table [rows, d], type 0 = F32,
 * 1 = F16 (widened exactly). Returns -1 (writing nothing further) at the first id outside [0, rows). */
int orc_embed(int type, const void* table, int64_t rows, int64_t d, const int32_t* ids, int64_t n, float* out);

/* ref_ops.cpp:137-148 (cpu::rmsnorm): per row, ss = sum of double(x)^2 left to right, scale = 1 / sqrt(ss / d + eps)
 * in double, y = float(x * scale * w) with the two double products in that order. */
void orc_rmsnorm(const float* x, const float* w, float* y, int64_t n, int64_t d, float eps);

/* ref_ops.cpp:151-153 (cpu::add): x[i] += y[i]. */
void orc_add(float* x, const float* y, int64_t count);

/* ref_ops.cpp:217-222 (cpu::silu_mul): gate[i] = g / (1 + expf(-g)) * up[i] in float. */
void orc_silu_mul(float* gate, const float* up, int64_t count);

/* ---- quantized formats (quant.c, restating src/quant.cpp and src/fp16.h); type = ggml id ---- */
int64_t orc_block_bytes(int type); /* bytes per block, -1 for an unknown type */
int64_t orc_block_elems(int type); /* elements per block (1 for F32 / F16) */
uint16_t orc_fp32_to_fp16(float f);
int orc_quantize_q8_0(const float* x, void* y, int64_t n);
int orc_quantize_q8_1(const float* x, void* y, int64_t n);
int orc_quantize_q8_k(const float* x, void* y, int64_t n);
int orc_dequantize(int type, const void* src, float* dst, int64_t n);
float orc_dot(int type, const void* w, const void* a, int64_t n_blocks);
int orc_act_kind(int type); /* 0 = Q8_0, 1 = Q8_1, 2 = Q8_K activations, -1 = float weights */
int orc_matmul_q(int type, const void* w, int64_t in, int64_t out, const float* x, float* y, int64_t n);

/* Llama-3 rope frequency factors (llama.cpp convert_hf_to_gguf.py, rope_type "llama3"; not in the reference
 * tree, the reference only reads rope_freqs.weight, weights.cpp:56, and divides by it, ref_ops.cpp:175):
 * for freq_i = base^(-2i/head_dim) and wavelen = 2*pi/freq_i, factor_i = 1 if wavelen < orig/high,
 * `factor` if wavelen > orig/low, else 1/((1-s)/factor + s) with s = (orig/wavelen - low)/(high - low).
 * Computed in double, stored as float. */
void orc_llama3_freq_factors(float* out, int64_t head_dim, double base, double factor, double low_freq_factor,
                             double high_freq_factor, double orig_ctx);

#ifdef __cplusplus
}
#endif
#endif
