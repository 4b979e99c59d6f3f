/*
 * nibble_hip_shim.h - the thin extern "C" layer between the C++20 HipBackend and HIP.
 *
 * These are the only entry points that touch HIP: device/stream/memory management and one launcher per
 * hand-written CDNA4 kernel. They take plain pointers and 64-bit sizes (byte offsets into a 131072-row,
 * 16-layer fp32 cache exceed 2^31), return 0 or a hipError_t value (nbhs_error_string() names it), and never
 * throw. Launchers only enqueue work on the given stream; they validate every size they are given before
 * launching (a launch that does not fit the kernel's assumptions returns NBHS_EINVAL and enqueues nothing), but
 * they cannot check that device pointers cover those sizes: HipBackend does that against its allocation table.
 *
 * The reference has no device code; each launcher names the reference operation it computes.
 */
#ifndef NIBBLE_HIP_SHIM_H
#define NIBBLE_HIP_SHIM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NBHS_EINVAL 1 /* hipErrorInvalidValue: a size or shape the launcher does not accept */
#define NBHS_EBLAS 100000 /* a rocBLAS call failed (outside hipError_t's range) */
#define NBHS_ETOOBIG 100001 /* the call needs more than a fixed static buffer holds */

typedef struct nbhs_stream_* nbhs_stream; /* a hipStream_t */
typedef struct nbhs_event_* nbhs_event;   /* a hipEvent_t */
typedef struct nbhs_blas_* nbhs_blas;     /* a rocblas_handle */

/* ---- device, streams, events, memory ---- */

/* Makes `device` current on the calling thread; fails unless it is a gfx950 (MI355X) device. Reports its
 * compute-unit count (for launch sizing). */
int nbhs_device_init(int device, int* cu_count);
const char* nbhs_error_string(int code);
int nbhs_stream_create(nbhs_stream* out); /* default priority, non-blocking */
int nbhs_stream_destroy(nbhs_stream s);
int nbhs_stream_sync(nbhs_stream s);
int nbhs_event_create(nbhs_event* out);
int nbhs_event_destroy(nbhs_event e);
int nbhs_event_record(nbhs_event e, nbhs_stream s);
int nbhs_event_elapsed_ms(nbhs_event start, nbhs_event end, float* ms); /* waits for `end` */
int nbhs_malloc(void** out, size_t bytes);
int nbhs_free(void* p);
/* Zero-fill with a kernel (never hipMemsetAsync, so the call is safe inside a captured graph). */
int nbhs_zero(void* p, size_t bytes, nbhs_stream s);
int nbhs_memcpy_h2d(void* dst, const void* host_src, size_t bytes, nbhs_stream s); /* returns when src is reusable */
int nbhs_memcpy_d2h(void* host_dst, const void* src, size_t bytes, nbhs_stream s); /* returns when dst is filled */
int nbhs_memcpy_d2d(void* dst, const void* src, size_t bytes, nbhs_stream s);      /* async; ranges must not overlap */

/* ---- kernels ---- */

/* RoPE in place (ref_ops.cpp:166-185 via Backend::rope, backend.h:64) on x[n, n_heads, head_dim] at positions
 * pos0..pos0+n-1. cs_table holds (cos, sin) float pairs [table_rows, head_dim/2] built on the host exactly as the
 * reference computes them; rows pos0..pos0+n-1 must exist (pos0 + n <= table_rows). The rotation is
 * a*c - b*s, a*s + b*c with every product and sum rounded separately (no FMA), so results are bit-exact. */
int nbhs_rope_f32(float* x, int64_t n, int64_t n_heads, int64_t head_dim, int64_t pos0, const float* cs_table,
                  int64_t table_rows, int neox, nbhs_stream s);

/* KV-cache append fused with RoPE (transformer.cpp:171-198: K/V rows land in cache rows pos0.., then rope(q) and
 * rope(k) in place): q[n, n_heads, head_dim] is rotated in place; cache_k rows pos0..pos0+n-1 receive
 * rope(k_new) and cache_v rows receive v_new, for caches laid out [rows, n_kv_heads, head_dim]. Bit-identical to
 * copying the rows and calling nbhs_rope_f32 on q and on the cache rows. q = NULL with n_heads = 0 appends the
 * K/V rows only. */
int nbhs_append_rope_f32(float* q, float* cache_k, float* cache_v, const float* k_new, const float* v_new, int64_t n,
                         int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, const float* cs_table,
                         int64_t table_rows, int neox, nbhs_stream s);

/* Causal GQA attention in fp32 (ref_ops.cpp:188-214 semantics via Backend::attention, backend.h:68-69) for n
 * query rows at positions pos0..pos0+n-1 over caches k, v [>= pos0+n rows, n_kv_heads, head_dim]; out is
 * [n, n_heads, head_dim]. Split-context ("flash-decoding"): each workgroup streams one chunk of one KV head for a
 * group of query heads and writes an online-softmax partial (max, sum, weighted V) to `workspace`; a second kernel
 * merges the partials with a log-sum-exp reduction. head_dim 64 or 128 take the tiled fast path, any other
 * head_dim in [1, 256] a generic path. A single row (n = 1) of the whole-row shapes (nbhs_attn_decode_rows_route)
 * takes the whole-row kernel instead: every wave reads whole cache rows (all KV heads, or a chunk of them) for all
 * their query heads, the grid's waves sweep the rows in lock-step, and each workgroup writes one partial per query
 * head for the same merge. workspace_floats must be >= nbhs_attn_decode_workspace(...) for the same arguments,
 * which returns the partial count the launcher will use. */
int64_t nbhs_attn_decode_workspace(int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                   int cu_count);
/* Upper bound of nbhs_attn_decode_workspace over every call shape with n_heads query heads (any context length,
 * row count, KV-head count and head_dim), for sizing the workspace once. */
int64_t nbhs_attn_decode_workspace_bound(int64_t n_heads, int cu_count);
/* 1 when a call of these arguments takes the whole-row kernel (n = 1, head_dim 64 with a multiple of 8 KV heads
 * or 128 with a multiple of 4, at most 8 such chunks of heads, GQA group 1, 2 or 4), else 0. */
int nbhs_attn_decode_rows_route(int64_t n, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim);
/* Rows nbhs_attn_decode_f32 and nbhs_attn_decode_noalloc take per call (the decode route of Backend::attention). */
#define NBHS_DECODE_MAX_ROWS 16
/* nbhs_attn_decode_f32 (no rotation, no append) on the current device with no allocation: the split partials go to
 * a 4 MiB static device array (nbhs_attn_decode_noalloc_capacity floats) that each GPU holds until the process ends.
 * It takes the kernel nbhs_attn_decode_f32 takes (then bit-identical to it) unless the whole-row kernel's partials
 * exceed the array, in which case it runs the per-head split kernel (equal within rounding). NBHS_ETOOBIG when
 * even those exceed it; calls overlapping on one GPU share the array and race. */
int nbhs_attn_decode_noalloc(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                             int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, nbhs_stream s);
int64_t nbhs_attn_decode_noalloc_capacity(void);
/* q_rope_cs: NULL when q is already rotated; otherwise the RoPE (cos, sin) table (as for nbhs_rope_f32, covering
 * positions pos0..pos0+n-1; q_rope_rows rows) and q is given unrotated and rotated on load, bit-identically to
 * rotating it first (head_dim 64 and 128 only). */
int nbhs_attn_decode_f32(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                         int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, float* workspace,
                         int64_t workspace_floats, int cu_count, const float* q_rope_cs, int64_t q_rope_rows,
                         int q_rope_neox, nbhs_stream s);
/* One decode step with its KV append (the single-row case of transformer.cpp:171-202: cache rows written, rope(q),
 * rope(kc), attention): cache row pos0 receives rope(k_new) and v_new (as nbhs_append_rope_f32 with no q), and
 * out receives the attention of the unrotated query row q, rotated on load, over rows 0..pos0 - bit-identical to
 * the append followed by nbhs_attn_decode_f32, in one launch fewer. head_dim 64 or 128; rope_cs covers pos0. */
int nbhs_append_attn_decode_f32(const float* q, float* k_cache, float* v_cache, const float* k_new,
                                const float* v_new, float* out, int64_t pos0, int64_t n_heads, int64_t n_kv_heads,
                                int64_t head_dim, float* workspace, int64_t workspace_floats, int cu_count,
                                const float* rope_cs, int64_t rope_rows, int neox, nbhs_stream s);

/* fp16 KV caches (an extension: the reference's cache is fp32, and its design defers an F16 KV cache,
 * docs/superpowers/specs/2026-10-17-nibble-design.md:181). k16, v16 hold _Float16 [rows, n_kv_heads, head_dim]; the
 * attention is the fp32 attention over the cached values widened exactly, head_dim 64 or 128 only, with the same
 * workspace as nbhs_attn_decode_f32. */
int nbhs_attn_decode_f16kv(const float* q, const void* k16, const void* v16, float* out, int64_t n, int64_t pos0,
                           int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, float* workspace,
                           int64_t workspace_floats, int cu_count, const float* q_rope_cs, int64_t q_rope_rows,
                           int q_rope_neox, nbhs_stream s);
/* The ordered route of nbhs_attn_decode_f32 / nbhs_attn_decode_f16kv: each query row (and head subgroup) in one
 * workgroup over its whole window, key groups in position order - no split of the keys over workgroups and no
 * whole-row kernel -, so a row's result depends on its own keys only: bitwise the same whichever call computes it,
 * however rows are batched into calls. Any head_dim the other routes take; no workspace. */
int nbhs_attn_decode_ordered_f32(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                                 int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, const float* q_rope_cs,
                                 int64_t q_rope_rows, int q_rope_neox, nbhs_stream s);
int nbhs_attn_decode_ordered_f16kv(const float* q, const void* k16, const void* v16, float* out, int64_t n,
                                   int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                   const float* q_rope_cs, int64_t q_rope_rows, int q_rope_neox, nbhs_stream s);
/* nbhs_append_attn_decode_f32 over fp16 caches: cache row pos0 receives fp16(rope(k_new)) and fp16(v_new) (rotated
 * in fp32 as the fp32 append does, then rounded to nearest even), and the attention uses the row as stored. */
int nbhs_append_attn_decode_f16kv(const float* q, void* k16, void* v16, const float* k_new, const float* v_new,
                                  float* out, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                  float* workspace, int64_t workspace_floats, int cu_count, const float* rope_cs,
                                  int64_t rope_rows, int neox, nbhs_stream s);
/* n fp32 rows k_new, v_new [n, n_kv_heads, head_dim] into fp16 cache rows pos0..pos0+n-1: K rotated by the table
 * (as nbhs_append_rope_f32), both rounded to fp16. */
int nbhs_append_rope_f16kv(void* k16, void* v16, const float* k_new, const float* v_new, int64_t n, int64_t pos0,
                           int64_t n_kv_heads, int64_t head_dim, const float* cs_table, int64_t table_rows, int neox,
                           nbhs_stream s);

/* Ragged batch of single-row decodes (one launch pair for all sequences; an extension the reference's single-session
 * Backend has no counterpart for - each sequence i is exactly Backend::attention with n = 1, backend.h:68-69):
 * query row q[i] [n_heads, head_dim] at position pos0[i] attends to rows 0..pos0[i] of its own caches k[i], v[i]
 * [>= pos0[i] + 1 rows, n_kv_heads, head_dim]; the result goes to out[i]. The arrays are host arrays of device
 * pointers. With k_new / v_new (host arrays, or both NULL), row pos0[i] of each cache first receives
 * rope(k_new[i]) and v_new[i], and q[i] is given unrotated and rotated on load (rope_cs required, covering every
 * pos0[i]) - as nbhs_append_attn_decode_f32 per sequence. head_dim 64 or 128. Sequences go 32 to a launch;
 * workspace_floats must be >= nbhs_attn_decode_batch_workspace(...) for the same positions. Results equal each
 * sequence's own nbhs_attn_decode_f32 call within rounding (the chunking differs); appended rows are bit-exact. */
int64_t nbhs_attn_decode_batch_workspace(int64_t n_seq, const int64_t* pos0, int64_t n_heads, int64_t n_kv_heads,
                                         int64_t head_dim, int cu_count);
int nbhs_attn_decode_batch_f32(int64_t n_seq, const float* const* q, const float* const* k, const float* const* v,
                               float* const* out, const float* const* k_new, const float* const* v_new,
                               const int64_t* pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                               float* workspace, int64_t workspace_floats, int cu_count, const float* rope_cs,
                               int64_t rope_rows, int neox, nbhs_stream s);

/* Operand staging for the MFMA prefill: cache rows [0, rows) of k and v [rows, n_kv_heads, head_dim] fp32 are
 * rounded to fp16 into k16 [n_kv_heads, rows_pad, head_dim] and vt16 [n_kv_heads, head_dim, rows_pad]
 * (transposed), rows_pad = rows rounded up to 64, padding zero-filled. After the transposed V, vt16 holds one
 * float2 per (KV head, 64-row tile): the tile's largest squared K row norm and largest |V| element, which the
 * prefill kernel's rounding-error estimate reads. aux (nbhs_prefill_aux_words words, zeroed when allocated) is
 * the prefill kernel's work list: staging empties it for the prefill launch that follows. */
int64_t nbhs_prefill_staging_halves(int64_t rows, int64_t n_kv_heads, int64_t head_dim); /* per tensor */
int64_t nbhs_prefill_aux_words(int64_t n, int64_t n_heads, int64_t n_kv_heads);
/* The largest nbhs_prefill_aux_words(m, n_heads, kv) over m <= max_rows and every kv dividing n_heads: the work list
 * that serves any prefill call of up to max_rows rows with n_heads query heads (what reserve() allocates). */
int64_t nbhs_prefill_aux_words_bound(int64_t max_rows, int64_t n_heads);
int nbhs_stage_kv_f16(const float* k, const float* v, void* k16, void* vt16, int64_t rows, int64_t n_kv_heads,
                      int64_t head_dim, uint32_t* aux, int64_t aux_words, nbhs_stream s);
/* KV append fused with the staging: cache rows pos0..pos0+n-1 receive rope(k_new) and v_new (as
 * nbhs_append_rope_f32 with no q), and k16 / vt16 are staged for rows [0, pos0+n) as nbhs_stage_kv_f16 would
 * after the append - one pass instead of two over the new rows. */
int nbhs_append_stage_kv_f16(float* cache_k, float* cache_v, const float* k_new, const float* v_new, int64_t n,
                             int64_t pos0, int64_t n_kv_heads, int64_t head_dim, const float* cs_table,
                             int64_t table_rows, int neox, void* k16, void* vt16, uint32_t* aux, int64_t aux_words,
                             nbhs_stream s);
/* The same two over fp16 caches (nbhs_attn_decode_f16kv's layout): rows are staged unchanged (already fp16); the
 * appended rows go into the caches rounded to fp16 (K after RoPE in fp32), exactly as nbhs_append_rope_f16kv stores
 * them, and are staged as stored. */
int nbhs_stage_kv_f16kv(const void* k_cache16, const void* v_cache16, void* k16, void* vt16, int64_t rows,
                        int64_t n_kv_heads, int64_t head_dim, uint32_t* aux, int64_t aux_words, nbhs_stream s);
int nbhs_append_stage_kv_f16kv(void* k_cache16, void* v_cache16, const float* k_new, const float* v_new, int64_t n,
                               int64_t pos0, int64_t n_kv_heads, int64_t head_dim, const float* cs_table,
                               int64_t table_rows, int neox, void* k16, void* vt16, uint32_t* aux,
                               int64_t aux_words, nbhs_stream s);

/* Causal GQA attention for n query rows at positions pos0.. (the prefill case of CpuBackend::attention,
 * cpu_backend.cpp:271-290). Rows [fp32_rows, n) run on gfx950 MFMA (v_mfma_f32_32x32x16_f16): Q rounded to fp16
 * after scaling by log2(e)/sqrt(head_dim), K/V from the staged fp16 copies, softmax and accumulators in fp32. Each
 * row's rounding error is estimated from its weights and the staged tile statistics; a row tile whose estimate
 * exceeds the budget is listed in aux and recomputed by a second launch with every operand split into fp16 high and
 * low parts, read from the fp32 caches k_cache / v_cache. Rows [0, fp32_rows) (0 <= fp32_rows < n) are computed in
 * fp32 from the caches, exactly as nbhs_attn_decode_f32 computes a single-chunk row, by workgroups of the same
 * launch. head_dim 64 or 128. The staged copies (and aux, by the staging call) must cover rows [0, pos0+n);
 * aux_words >= nbhs_prefill_aux_words(n - fp32_rows, ...); staged_rows_pad * head_dim * 2 <= INT32_MAX (the
 * staged K and V^T of one KV head are read through buffer resources with a 32-bit byte size: at most 16.7M
 * positions at head_dim 64, 8.3M at 128), else NBHS_EINVAL. q_rope_cs as for nbhs_attn_decode_f32. */
int nbhs_attn_prefill_mfma(const float* q, const void* k16, const void* vt16, float* out, int64_t n, int64_t pos0,
                           int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t staged_rows_pad,
                           const float* q_rope_cs, int64_t q_rope_rows, int q_rope_neox, const float* k_cache,
                           const float* v_cache, int64_t fp32_rows, float* workspace, int64_t workspace_floats,
                           uint32_t* aux, int64_t aux_words, int cu_count, nbhs_stream s);
/* nbhs_attn_prefill_mfma over fp16 caches: the fp32 rows and the recomputation read the fp16 cache values (widened
 * exactly), which are the values an fp16-cache attention attends to. */
int nbhs_attn_prefill_mfma_f16kv(const float* q, const void* k16, const void* vt16, float* out, int64_t n,
                                 int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                 int64_t staged_rows_pad, const float* q_rope_cs, int64_t q_rope_rows, int q_rope_neox,
                                 const void* k_cache16, const void* v_cache16, int64_t fp32_rows, float* workspace,
                                 int64_t workspace_floats, uint32_t* aux, int64_t aux_words, int cu_count,
                                 nbhs_stream s);
/* Workspace (floats) nbhs_attn_prefill_mfma needs for these arguments: when the MFMA rows' tiles cannot fill the
 * chip (short prefill chunks), each tile's key range is split over several workgroups whose partials a second,
 * log-sum-exp launch merges; 0 when no split is taken. */
int64_t nbhs_attn_prefill_workspace(int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                    int64_t fp32_rows, int cu_count);
/* Upper bound of nbhs_attn_prefill_workspace over every call shape, for sizing the workspace once. */
int64_t nbhs_attn_prefill_workspace_bound(int cu_count);

/* Synthetic N(0,1)*scale data for benchmarks: counter-based (SplitMix64 of seed and index), Box-Muller in fp32. */
int nbhs_fill_normal_f32(float* dst, int64_t count, uint64_t seed, float scale, nbhs_stream s);

/* MFMA calibration for benchmarks (no counterpart in the reference): cu_count * waves_per_simd workgroups of four
 * waves (one per SIMD of a CU), each wave issuing iters x 8 independent v_mfma_f32_32x32x16_f16 over 4 accumulator
 * chains and nothing else, so the launch runs at the sustained rate of the MFMA pipes at that occupancy (clock
 * included). FLOPs = cu_count * waves_per_simd * 4 * iters * 8 * 32768. out receives cu_count * waves_per_simd * 256
 * floats (the accumulators' sums, which keep the loop from being removed). 1 <= waves_per_simd <= 8,
 * 1 <= iters <= 1 << 24. Timed as NBHS_K_CALIBRATION. */
int nbhs_mfma_loop_f16(float* out, int64_t iters, int waves_per_simd, int cu_count, nbhs_stream s);

/* ---- float-weight projections (Backend::matmul / matmul_multi / add_bias, backend.h:56-62) ---- */

#define NBHS_GEMV_MAX_WEIGHTS 8
#define NBHS_GEMV_MAX_ROWS 16
/* Up to 8 weights sharing one input in one launch, for n <= 16 rows (decode, short appends): for each i,
 * y[i][t * rows[i] + r] = sum_k x[t * in + k] * w[i][r * in + k] (ref_ops.cpp:109-135 semantics; fp32 accumulation in
 * another order than the reference's, so equal within float rounding). w[i] is F32 (f16[i] = 0) or F16 (f16[i] = 1)
 * [rows[i], in] in device memory. */
int nbhs_gemv_multi(int n_w, const int* f16, const void* const* w, float* const* y, const int64_t* rows, int64_t in,
                    const float* x, int64_t n, nbhs_stream s);
/* Exact widening of count IEEE halves to floats. */
int nbhs_f16_to_f32(const void* src, float* dst, int64_t count, nbhs_stream s);
/* ref_ops.cpp:154-160 (cpu::add_bias): x[t * d + i] += bias[i] for t < n; bit-exact. */
int nbhs_add_bias_f32(float* x, const float* bias, int64_t d, int64_t n, nbhs_stream s);
/* A rocBLAS handle bound to stream s (its device workspace is allocated here, once). */
int nbhs_blas_create(nbhs_blas* out, nbhs_stream s);
int nbhs_blas_destroy(nbhs_blas h);
/* y[n, out] = x[n, in] . w[out, in]^T in fp32 (rocBLAS sgemm, full fp32 math), on the handle's stream: the same
 * product as nbhs_gemv_multi, for any n. */
int nbhs_sgemm_xwt(nbhs_blas h, const float* x, const float* w, float* y, int64_t n, int64_t in, int64_t out);

/* F16 weights on the fp16 MFMA pipes for any n (prefill chunks), up to NBHS_GEMM_MAX_WEIGHTS weights sharing x in
 * one launch: y[i][t * rows[i] + r] = sum_k x[t * in + k] * w[i][r * in + k], as nbhs_gemv_multi. Each activation
 * row is scaled by a power of two and split into fp16 hi + lo parts (x s = hi + lo to ~2^-22 relative); both are
 * multiplied by the exact fp16 weights with fp32 accumulation, so the result is fp32-grade (within the float
 * summation bound of the reference's sum). ws: device scratch of nbhs_gemm_f16w_workspace(n, in) bytes, 256-byte
 * aligned (the split rows and a fixed 64 MB area for K-range partial sums). Requires in % 8 == 0 and 16-byte aligned
 * weights. Deterministic; each weight's tile configuration and K ranges follow from its own shape, so its outputs do
 * not depend on the other weights of the call. */
#define NBHS_GEMM_MAX_WEIGHTS 8
int64_t nbhs_gemm_f16w_workspace(int64_t n, int64_t in);
int nbhs_gemm_f16w_multi(int n_w, const void* const* w, float* const* y, const int64_t* rows, int64_t in,
                         const float* x, int64_t n, void* ws, int64_t ws_bytes, nbhs_stream s);

/* ---- the other per-token ops (Backend::embed / rmsnorm / add / silu_mul, backend.h:55-70) ---- */

/* out[t, :] = row ids[t] of table [rows, d] (F32, or F16 widened exactly); ids in device memory, already checked
 * against the row count by the caller (ref_ops.cpp:80-99). */
int nbhs_embed(int f16, const void* table, const int32_t* ids, int64_t n, int64_t d, float* out, nbhs_stream s);
/* ref_ops.cpp:137-148: y[t] = float(x[t] * scale * w) with scale = 1 / sqrt(sum(x^2) / d + eps) in double. */
int nbhs_rmsnorm_f32(const float* x, const float* w, float* y, int64_t n, int64_t d, float eps, nbhs_stream s);
/* x[i] += y[i] (ref_ops.cpp:151-153). */
int nbhs_add_f32(float* x, const float* y, int64_t count, nbhs_stream s);
/* gate[i] = g / (1 + exp(-g)) * up[i] (ref_ops.cpp:217-222). */
int nbhs_silu_mul_f32(float* gate, const float* up, int64_t count, nbhs_stream s);

/* ---- quantized weights (Backend::matmul / embed for Q4_0 .. Q6_K; src/quant.h, ref_ops.cpp:109-135) ----
 * type is the ggml id. A weight lives on the device in the plane layout of kernels/quant_layout.h (the host repacks
 * the file's blocks on upload); activations are quantized into planes of the same header's ActLayout. */
int64_t nbhs_quant_weight_bytes(int type, int64_t rows, int64_t in); /* -1 when not a quant type / bad width */
int64_t nbhs_quant_act_bytes(int type, int64_t n, int64_t in);
/* The n x in activation rows x quantized to type's companion format (quant.cpp:37-49, 245-303), bit-exact. */
int nbhs_quantize_acts(int type, const float* x, int64_t n, int64_t in, void* acts, nbhs_stream s);
/* For each of n_w (<= 8) weights of one type sharing the input, y[i][t * rows[i] + r] for t < n (n <= 16): the
 * block dot of weight row r with activation row t0 + t (quant.cpp:305-419, same bits). The activations are the
 * n_acts rows quantized into acts by nbhs_quantize_acts; or, with acts NULL (n <= 4, t0 = 0, x 16-byte aligned),
 * rows of x quantized inside the launch (the same bits). */
int nbhs_qgemv_multi(int type, int n_w, const void* const* w, const int64_t* rows, float* const* y, int64_t in,
                     const float* x, const void* acts, int64_t n_acts, int64_t t0, int64_t n, nbhs_stream s);
/* nbhs_quantize_acts for the K types with each super-block's quants in residue-major order (byte 32 w + 4 k + i
 * holds element 32 k + w + 8 i), the layout nbhs_qgemm_multi reads for the K types. */
int nbhs_quantize_acts_rm(int type, const float* x, int64_t n, int64_t in, void* acts, nbhs_stream s);
/* The same products for any n (prefill chunks), tiled, in one launch for up to NBHS_GEMV_MAX_WEIGHTS weights of
 * one type: y[i][t * rows[i] + r] for t < n over all n quantized activation rows in acts; Q4_0, Q5_0, Q5_1, Q8_0
 * (acts from nbhs_quantize_acts) and Q4_K, Q5_K, Q6_K (acts from nbhs_quantize_acts_rm, int8 matrix cores). Same bits
 * as nbhs_qgemv_multi. */
int nbhs_qgemm_multi(int type, int n_w, const void* const* w, const int64_t* rows, float* const* y, int64_t in,
                     const void* acts, int64_t n, nbhs_stream s);
/* out[t, :] = dequantized row ids[t] (device ids) of the weight, quant.cpp:157-242 bit for bit. */
int nbhs_dequant_rows(int type, const void* w, int64_t rows, int64_t in, const int32_t* ids, int64_t n, float* out,
                      nbhs_stream s);

/* ---- per-kernel timing (measurement only) ----
 * While enabled for a kernel, its launcher launches it with a HIP event pair (hipExtLaunchKernel) stamped from the
 * dispatch itself, so the average device duration of that kernel can be read back live (bench.py's roofline
 * figures); the other kernels launch as usual. Timing a kernel alone keeps the event handling of its neighbours'
 * launches from changing what it is measured against. Off by default. Not thread-safe. */
enum nbhs_kernel_id {
  NBHS_K_ROPE = 0,
  NBHS_K_APPEND_ROPE = 1,
  NBHS_K_DECODE_PARTIAL = 2,
  NBHS_K_DECODE_COMBINE = 3,
  NBHS_K_GENERIC = 4,
  NBHS_K_STAGE_KV = 5,
  NBHS_K_PREFILL_MFMA = 6,
  NBHS_K_GEMV = 7,
  NBHS_K_CONVERT = 8,
  NBHS_K_ADD_BIAS = 9,
  NBHS_K_RMSNORM = 10,
  NBHS_K_ELEMENTWISE = 11, /* embed, add, silu_mul, dequantized embed */
  NBHS_K_QUANTIZE = 12,    /* activation quantization for quantized weights */
  NBHS_K_QGEMV = 13,
  NBHS_K_QGEMM = 14,
  NBHS_K_PREFILL_PRECISE = 15, /* split-operand recomputation of listed prefill row tiles */
  NBHS_K_CALIBRATION = 16,     /* nbhs_mfma_loop_f16 */
  NBHS_K_SPLIT_ACTS = 17,      /* activation rows split into fp16 hi + lo for the F16-weight GEMM */
  NBHS_K_GEMM = 18,            /* F16-weight GEMM (nbhs_gemm_f16w_multi) */
  NBHS_K_GEMM_REDUCE = 19,     /* the F16-weight GEMM's sum of K-range partials */
  NBHS_K_COUNT = 20
};
int nbhs_kernel_timing_enable(int on); /* on != 0: time every kernel; 0: none (clears what was recorded) */
int nbhs_kernel_timing_select(uint32_t kernel_mask); /* time the kernels whose bit (1 << id) is set; clears */
/* Waits for the recorded launches of `kernel` and returns their summed duration and count, then clears them. */
int nbhs_kernel_timing_read(int kernel, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif
#endif
