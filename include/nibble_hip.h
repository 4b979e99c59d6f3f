/*
 * nibble_hip.h - C ABI of the MI355X attention backend (libnibble_hip.so).
 *
 * This is the drop-in boundary for nibble's attention path. Each entry point wraps one member of
 * nibble::hip::HipBackend, which implements the reference's nibble::Backend operator interface
 * (src/backend/backend.h:36-71) on one gfx950 GPU; the citation on each declaration names the reference member it
 * replaces. A C++ caller (nibble's Transformer) uses HipBackend directly; FFI callers (ctypes, tests, benchmarks)
 * use these functions. Plain pointers and 64-bit sizes only.
 *
 * Buffers: nbh_backend_alloc() returns zeroed HBM. Every op that takes device pointers checks that each range it
 * will touch lies inside one buffer from this backend and fails with NBH_E_INPUT otherwise, before launching work.
 * Ops are asynchronous on the backend's HIP stream, in call order; read() and sync() wait for them.
 *
 * Errors: every function returns NBH_OK (0) or an NBH_E_* code; nbh_last_error() gives the message of the
 * calling thread's last failure. The reference throws nibble::Error for the same conditions
 * (include/nibble/error.h:11); HipBackend does too, and this layer converts it.
 * Threading: one caller thread per backend (like CpuBackend; src/model/transformer.h:7).
 */
#ifndef NIBBLE_HIP_H
#define NIBBLE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NBH_OK 0
#define NBH_E_INPUT 1    /* nibble::Error: bad argument, range outside a buffer, allocation or device failure */
#define NBH_E_INTERNAL 2 /* any other exception */

typedef struct nbh_backend nbh_backend;
typedef struct nbh_event nbh_event;

/* A weight view, field for field nibble::Tensor (src/tensor.h:21-66): type is the ggml type id (0 = F32, 1 = F16,
 * 2 = Q4_0, 6 = Q5_0, 7 = Q5_1, 8 = Q8_0, 12 = Q4_K, 13 = Q5_K, 14 = Q6_K), ne[1] * ne[2] * ne[3] rows of ne[0]
 * elements, row-major at data (quantized: rows of ggml blocks, src/quant.h). data is host memory (copied to HBM on
 * first use - quantized weights repacked into aligned planes - and kept until nbh_backend_release_weights; its
 * bytes must not change meanwhile) or, for F32 / F16, lies inside a buffer from nbh_backend_alloc (used in place). */
typedef struct nbh_tensor {
  uint32_t type;
  int32_t n_dims;
  int64_t ne[4];
  const void* data;
} nbh_tensor;

/* Message of the calling thread's last failed call ("" if none). */
const char* nbh_last_error(void);

/* Creates a backend on HIP device `device` (must be gfx950). Replaces CpuBackend(ThreadPool&)
 * (src/backend/cpu/cpu_backend.h:21, constructed at src/nibble.cpp:75-85). */
int nbh_backend_create(int device, nbh_backend** out);

/* Frees every buffer still allocated. Replaces CpuBackend::~CpuBackend (cpu_backend.cpp:70-72). */
void nbh_backend_destroy(nbh_backend* be);

/* Backend::supports (backend.h:41): whether weight type `dtype` (ggml id) can run matmul/embed: 1 for every type
 * the reference supports (F32, F16, Q4_0, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K). */
int nbh_backend_supports(const nbh_backend* be, uint32_t dtype, int* out);

/* Backend::reserve (backend.h:45; ReserveParams backend.h:24-26). */
int nbh_backend_reserve(nbh_backend* be, int64_t n_ctx, int64_t n_heads, int64_t max_rows, int64_t max_width);

/* Backend::alloc (backend.h:47): zeroed HBM for n_floats floats. */
int nbh_backend_alloc(nbh_backend* be, int64_t n_floats, float** out);

/* Backend::free (backend.h:51): NULL is a no-op; pointers this backend did not allocate are ignored. */
int nbh_backend_free(nbh_backend* be, float* p);

/* Backend::read (backend.h:53): device -> host copy of n floats; waits for queued work. */
int nbh_backend_read(nbh_backend* be, float* host_dst, const float* src, int64_t n);

/* Host -> device copy of n floats. No reference counterpart: CpuBackend buffers are host memory, so its callers
 * (e.g. tests/test_cpu_backend.cpp:69-74) write them directly. */
int nbh_backend_write(nbh_backend* be, float* dst, const float* host_src, int64_t n);

/* Backend::copy (backend.h:65; memmove semantics, cpu_backend.cpp:260-264). */
int nbh_backend_copy(nbh_backend* be, float* dst, const float* src, int64_t count);

/* Backend::rope (backend.h:64) with RopeParams (backend.h:16-20) passed field by field: freq_base, neox, and
 * freq_factors (NULL or head_dim/2 HOST floats). Bit-exact with ref_ops.cpp:166-185. */
int nbh_backend_rope(nbh_backend* be, float* x, int64_t n, int64_t n_heads, int64_t head_dim, int64_t pos0,
                     float freq_base, int neox, const float* freq_factors);

/* Backend::attention (backend.h:66-69): q,out [n, n_heads, head_dim]; k,v [>= pos0+n rows, n_kv_heads,
 * head_dim] (layer cache bases); row t attends to cache rows 0..pos0+t. */
int nbh_backend_attention(nbh_backend* be, const float* q, const float* k, const float* v, float* out, int64_t n,
                          int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim);

/* KV-cache append fused with RoPE: the per-layer sequence of src/model/transformer.cpp:171-198 (K/V rows written
 * into cache rows pos0.., rope(q) and rope(k rows) in place) for K/V rows that arrive in their own buffers
 * k_new/v_new [n, n_kv_heads, head_dim]. k_cache/v_cache are layer bases. Bit-identical to write + rope. */
int nbh_backend_append_rope(nbh_backend* be, float* q, float* k_cache, float* v_cache, const float* k_new,
                            const float* v_new, int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads,
                            int64_t head_dim, float freq_base, int neox, const float* freq_factors);

/* KV-cache append with RoPE fused into attention: the per-layer sequence of src/model/transformer.cpp:171-202
 * (K/V rows into cache rows pos0.., rope(q), rope(k rows), Backend::attention at backend.h:68-69) in one call.
 * Results are bit-identical to nbh_backend_append_rope followed by nbh_backend_attention, except that q is read
 * unrotated and left unchanged: it is rotated in registers as the attention kernels load it, and on the prefill
 * (MFMA) route the K/V append shares one pass with the fp16 operand staging. out [n, n_heads, head_dim]. */
int nbh_backend_append_rope_attention(nbh_backend* be, const float* q, float* k_cache, float* v_cache,
                                      const float* k_new, const float* v_new, float* out, int64_t n, int64_t pos0,
                                      int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, float freq_base, int neox,
                                      const float* freq_factors);

/* fp16 KV caches - an extension: the reference's cache is fp32 and its design defers an F16 KV cache
 * (docs/superpowers/specs/2026-10-17-nibble-design.md:181). k16, v16: layer bases of _Float16 [rows, n_kv_heads,
 * head_dim] caches in buffers from nbh_backend_alloc (a buffer of f floats holds 2f halves); head_dim 64 or 128.
 * nbh_backend_attention_f16kv is nbh_backend_attention over the cached values widened exactly (q already
 * rotated); nbh_backend_append_rope_attention_f16kv first writes rows pos0.. as fp16(rope(k_new)) and fp16(v_new)
 * (the fp32 rotation, then rounding to nearest even) and reads q unrotated, as nbh_backend_append_rope_attention.
 * Calls of at most 16 rows run on the decode kernels (a single row of the whole-row shapes on the whole-row kernel,
 * others on the split-context kernel); longer ones take the prefill route of
 * nbh_backend_attention (the fp16 cache rows staged unchanged - K and V carry no further rounding -, Q and the
 * softmax weights rounded to fp16 on MFMA, the rounding-error estimate and the split-operand recomputation; rows at
 * positions below 128 in fp32), with the append fused into the staging. Range: fp16 holds |x| <= 65504; a rotated
 * K or a V element
 * beyond that is stored as +-inf (IEEE conversion, not saturated), and attention over such a row is in general not
 * finite, where the fp32 cache would have stayed finite. */
int nbh_backend_attention_f16kv(nbh_backend* be, const float* q, const void* k16, const void* v16, float* out,
                                int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim);
int nbh_backend_append_rope_attention_f16kv(nbh_backend* be, const float* q, void* k16, void* v16,
                                            const float* k_new, const float* v_new, float* out, int64_t n,
                                            int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                            float freq_base, int neox, const float* freq_factors);

/* Ragged batch of single-token decodes. No counterpart in the reference, whose Backend serves one sequence: each
 * sequence i is Backend::attention (backend.h:68-69) with n = 1 - query row q[i] [n_heads, head_dim] at position
 * pos0[i] over its own layer caches k_cache[i], v_cache[i] - and equals that call within rounding. q, k_cache,
 * v_cache and out are host arrays of n_seq device pointers, pos0 a host array. One launch pair streams every
 * sequence's cache at once (head_dim 64 and 128; other sizes run one call per sequence). */
int nbh_backend_attention_batch(nbh_backend* be, int64_t n_seq, const float* const* q, const float* const* k_cache,
                                const float* const* v_cache, float* const* out, const int64_t* pos0, int64_t n_heads,
                                int64_t n_kv_heads, int64_t head_dim);

/* The batch with each sequence's new K/V row (k_new[i], v_new[i] [n_kv_heads, head_dim]) appended first at row
 * pos0[i] and q read unrotated: nbh_backend_append_rope_attention with n = 1 for every sequence (the per-layer
 * sequence of src/model/transformer.cpp:171-202), appended rows bit-identical. */
int nbh_backend_append_rope_attention_batch(nbh_backend* be, int64_t n_seq, const float* const* q,
                                            float* const* k_cache, float* const* v_cache, const float* const* k_new,
                                            const float* const* v_new, float* const* out, const int64_t* pos0,
                                            int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, float freq_base,
                                            int neox, const float* freq_factors);

/* Backend::matmul (backend.h:56): y[n, w.rows] = x[n, w.ne[0]] . W^T (ref_ops.cpp:109-135). F32/F16 weights: fp32
 * products and sums in another order than the reference's (equal within float rounding). Quantized weights: the
 * activation rows quantized to the type's companion format and the block dots of quant.cpp:305-419, bit-exact.
 * x, y device. */
int nbh_backend_matmul(nbh_backend* be, const nbh_tensor* w, const float* x, float* y, int64_t n);

/* Backend::matmul_multi (backend.h:57-60): ys[i] = matmul(ws[i], x, n) for n_w weights sharing the input x; the
 * QKV projection of src/model/transformer.cpp:177-180 passes ys = {q, k cache rows, v cache rows}. ws and ys are
 * host arrays. */
int nbh_backend_matmul_multi(nbh_backend* be, int64_t n_w, const nbh_tensor* const* ws, const float* x,
                             float* const* ys, int64_t n);

/* Backend::add_bias (backend.h:63, ref_ops.cpp:154-160): each of the n rows of x [n, bias.ne[0]] += bias (F32);
 * bit-exact. */
int nbh_backend_add_bias(nbh_backend* be, float* x, const nbh_tensor* bias, int64_t n);

/* Backend::embed (backend.h:55, ref_ops.cpp:80-99): out[t, :] = row ids[t] of table (F32 copied, F16 widened
 * exactly), t < n_ids. ids is HOST memory; an id outside [0, rows) fails with NBH_E_INPUT before any work. */
int nbh_backend_embed(nbh_backend* be, const nbh_tensor* table, const int32_t* ids, int64_t n_ids, float* out);

/* Backend::rmsnorm (backend.h:61, ref_ops.cpp:137-148): y[t] = x[t] * w / sqrt(mean(x[t]^2) + eps) for n rows of
 * weight.ne[0] floats (weight F32), the sum and scale in double as the reference computes them. */
int nbh_backend_rmsnorm(nbh_backend* be, const float* x, const nbh_tensor* weight, float* y, int64_t n, float eps);

/* Backend::add (backend.h:62, ref_ops.cpp:151-153): x[i] += y[i]; bit-exact. */
int nbh_backend_add(nbh_backend* be, float* x, const float* y, int64_t count);

/* Backend::silu_mul (backend.h:70, ref_ops.cpp:217-222): gate[i] = g / (1 + exp(-g)) * up[i]. */
int nbh_backend_silu_mul(nbh_backend* be, float* gate, const float* up, int64_t count);

/* Attention precision switch (no reference counterpart: the reference computes attention in float). on = 0
 * (default): calls of more than 16 rows with head_dim 64/128 run rows at positions >= 128 on the fp16-operand MFMA
 * kernel, whose per-row rounding-error estimate sends row tiles that could miss 1e-3 to a split-operand (fp16 high +
 * low) recomputation. on != 0: every row takes the fp32 split-context kernel, as decode does, at a much lower
 * prefill rate (a debugging aid). */
int nbh_backend_set_attention_fp32(nbh_backend* be, int on);

/* Batch invariance switch. The reference's kernels give a row the same bits however tokens are batched into calls
 * (its model tests demand it: tests/test_model.cpp:141-151, 253-263); this backend's default routes agree only
 * within rounding (fp16-operand MFMA prefill, keys split over workgroups by the call's shape, rocBLAS for long float
 * matmuls). on != 0: every attention row takes the ordered fp32 route (one workgroup per row over its whole window,
 * keys in position order) and every float-weight matmul the gemv kernel, so batch, token-by-token and chunked
 * evaluation agree bit for bit, at a much lower prefill rate (and a lower long-context decode rate: a row's keys are
 * no longer split over workgroups). Quantized matmuls are bit-exact either way. */
int nbh_backend_set_batch_invariant(nbh_backend* be, int on);

/* Decode attention that allocates nothing. No counterpart in the reference: for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops). It is the decode route of
 * nbh_backend_attention (n <= 16 query rows; q already rotated; results bit-identical to that call, which takes the
 * same kernel - a single row of the whole-row shapes runs the per-head split kernel here instead, equal within
 * rounding, when the whole-row kernel's partials would not fit the array) on the current device, over device pointers
 * the caller owns (they are not checked against any backend's buffers), enqueued on `stream` (a hipStream_t; NULL:
 * the null stream). Its partials go to a 4 MiB static device array each GPU holds until the process ends; a call
 * whose partials exceed it fails with NBH_E_INPUT (on a 256-CU MI355X no decode shape does). Every call on one GPU
 * shares that array: calls that overlap on one GPU (two streams) race. */
int nbh_attention_decode_noalloc(const float* q, const float* k, const float* v, float* out, int64_t n,
                                 int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, void* stream);

/* Row tiles (128 packed query rows x one KV head) the last MFMA prefill call recomputed with split operands; waits
 * for queued work. No reference counterpart: a diagnostic of the precision routing above. */
int nbh_backend_prefill_recomputed(nbh_backend* be, int64_t* tiles);

/* Drops every device copy of a host weight; no reference counterpart (CpuBackend reads weights in place). */
int nbh_backend_release_weights(nbh_backend* be);

/* Extension of Backend::reserve for shapes ReserveParams does not carry: sizes the prefill operand staging
 * (n_kv_heads x head_dim at the reserved n_ctx) so that the first prefill allocates nothing. */
int nbh_backend_reserve_attention(nbh_backend* be, int64_t n_kv_heads, int64_t head_dim);

/* Extension: builds the RoPE table for these parameters up to the reserved n_ctx ahead of the first rope(). */
int nbh_backend_reserve_rope(nbh_backend* be, int64_t head_dim, float freq_base, int neox, const float* freq_factors);

/* Waits for all queued work (no reference counterpart; CPU ops are synchronous). */
int nbh_backend_sync(nbh_backend* be);

/* Test hooks: buffers from alloc() still live (CpuBackend::live_allocations, cpu_backend.h:50); bytes of internal
 * workspaces and tables (must not grow after reserve for in-range calls); the device's compute-unit count. */
int nbh_backend_live_allocations(const nbh_backend* be, int64_t* out);
int nbh_backend_internal_bytes(const nbh_backend* be, int64_t* out);
int nbh_backend_cu_count(const nbh_backend* be, int* out);
int nbh_backend_weight_bytes(const nbh_backend* be, int64_t* out); /* HBM held by copies of host weights */

/* Synthetic N(0,1)*scale data generated on the device (benchmarks). No reference counterpart. */
int nbh_backend_fill_normal(nbh_backend* be, float* dst, int64_t count, uint64_t seed, float scale);

/* The hipStream_t the backend's ops run on, for ordering a caller's own work with them (for example
 * nbh_attention_decode_noalloc on the backend's buffers). No reference counterpart. */
int nbh_backend_stream(nbh_backend* be, void** stream);

/* HIP events on the backend's stream, for timing a span of queued ops. No reference counterpart. */
int nbh_event_create(nbh_backend* be, nbh_event** out);
int nbh_event_record(nbh_backend* be, nbh_event* e);
int nbh_event_elapsed_ms(nbh_event* start, nbh_event* end, float* ms); /* waits for `end` */
void nbh_event_destroy(nbh_event* e);

#ifdef __cplusplus
}
#endif
#endif
