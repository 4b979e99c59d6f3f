#pragma once
// HipBackend: nibble's Backend (backend.h) on one MI355X (gfx950), the attention path in hand-written HIP.
// It replaces CpuBackend (reference src/backend/cpu/cpu_backend.h:18-91) for the ops the attention path uses:
// reserve/alloc/free/read/copy, rope and attention, plus HIP-only extensions (host upload, the fused KV append
// with RoPE, synthetic fill, events), the QKV projection that feeds it (matmul / matmul_multi and add_bias), and the
// remaining per-token ops (embed, rmsnorm, add, silu_mul), so a whole forward stays on the GPU. Weights may be F32,
// F16 or any of the reference's quantized types (Q4_0, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K): supports() is true for
// all of them. Quantized matmuls and embeds are bit-exact with the reference's quant.cpp.
//
// Weights: a Tensor's data is host memory (nibble maps the GGUF file), or memory from alloc(). Host weights are
// copied to HBM on first use and kept, keyed by their data pointer, until release_weights() or destruction; the
// caller must not change a weight's host bytes while its copy is kept (nibble's weights are read-only). Weights
// inside a buffer from alloc() are used in place.
//
// Memory: every buffer handed out is HBM, zeroed, tracked; every op checks that the device ranges it is given lie
// inside one tracked buffer before it launches anything, and throws Error otherwise (a bad range never reaches a
// kernel). Ops run asynchronously on the backend's own HIP stream in call order; read() and sync() wait.
// Not thread-safe (one caller thread, as for CpuBackend).
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "backend/backend.h"
#include "nibble/error.h"
#include "nibble_hip_shim.h"

namespace nibble::hip {

class HipBackend final : public Backend {
 public:
  // Selects `device` (must be gfx950) and creates the backend's stream. Throws Error on failure.
  explicit HipBackend(int device = 0);
  ~HipBackend() override;
  HipBackend(const HipBackend&) = delete;
  HipBackend& operator=(const HipBackend&) = delete;

  bool supports(DType t) const override;
  // Sizes every internal buffer so that afterwards ops with pos0 + n <= n_ctx, n_heads <= the reserved count,
  // n <= max_rows and matmul input width <= max_width allocate nothing (backend.h:42-45): the decode and split
  // workspaces, the quantized-activation and embed-id buffers, the copy bounce buffer, the fp16 prefill staging
  // (bounded by max_width >= n_heads * head_dim, since the KV width is not in ReserveParams) and the memory for the
  // first RoPE table. Device copies of host weights are made on a weight's first use, as model state, not here.
  void reserve(const ReserveParams&) override;
  float* alloc(int64_t n_floats) override;  // HBM, 64-byte granular, zeroed
  void free(float* p) override;
  void read(float* host_dst, const float* src, int64_t n) override;  // waits for queued work
  // out[t, :] = row ids[t] of the table (F32 copied, F16 widened; ref_ops.cpp:80-99); ids are host memory and are
  // checked against the row count before anything is queued (Error, as the reference throws).
  void embed(const Tensor& table, std::span<const int32_t> ids, float* out) override;
  // y[n, w.rows()] = x[n, w.ne[0]] . W^T for F32 and F16 weights (ref_ops.cpp:109-135): fp32 products and sums, in
  // another order than the reference's left-to-right one (equal within float rounding).
  void matmul(const Tensor& w, const float* x, float* y, int64_t n) override;
  // ys[i] = matmul(*ws[i], x, n); weights of one input width share one launch on the decode route (n <= 16).
  void matmul_multi(std::span<const Tensor* const> ws, const float* x, std::span<float* const> ys,
                    int64_t n) override;
  // ref_ops.cpp:137-148 with the sum of squares and the scale in double (weight F32 [d]).
  void rmsnorm(const float* x, const Tensor& weight, float* y, int64_t n, float eps) override;
  void add(float* x, const float* y, int64_t count) override;  // bit-exact
  void add_bias(float* x, const Tensor& bias, int64_t n) override;  // bias F32 [d]; bit-exact
  void rope(float* x, int64_t n, int64_t n_heads, int64_t head_dim, int64_t pos0, const RopeParams& p) override;
  void copy(float* dst, const float* src, int64_t count) override;  // memmove semantics
  void attention(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                 int64_t n_heads, int64_t n_kv_heads, int64_t head_dim) override;
  void silu_mul(float* gate, const float* up, int64_t count) override;  // within a few ulp (device expf)

  // ---- HIP-only extensions ----
  // Host -> device upload of n floats (the reference needs none: its buffers are host memory).
  void write(float* dst, const float* host_src, int64_t n);
  // Sizes the prefill operand staging exactly for caches of n_kv_heads x head_dim at up to the reserved n_ctx
  // rows, replacing the larger bound reserve() took from max_width.
  void reserve_attention(int64_t n_kv_heads, int64_t head_dim);
  // Prebuilds the RoPE (cos, sin) table for these parameters up to the reserved n_ctx positions.
  void reserve_rope(int64_t head_dim, const RopeParams& p);
  // KV-cache append fused with RoPE: the sequence matmul-into-cache, rope(q), rope(k rows) of
  // transformer.cpp:171-198 for K/V rows arriving in a separate buffer. k_cache/v_cache are layer bases.
  void append_rope(float* q, float* k_cache, float* v_cache, const float* k_new, const float* v_new, int64_t n,
                   int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, const RopeParams& p);
  // KV-cache append with RoPE fused into attention: the same results, bit for bit, as append_rope(q, ...) followed
  // by attention(q, ...), except that q is read unrotated and left unchanged (it is rotated on load). On the MFMA
  // route the append shares one pass with the fp16 operand staging, and q is never rewritten in memory.
  void append_rope_attention(const float* q, float* k_cache, float* v_cache, const float* k_new, const float* v_new,
                             float* out, int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads,
                             int64_t head_dim, const RopeParams& p);
  // fp16 KV caches (an extension; the reference's cache is fp32): k16 / v16 hold _Float16 [rows, n_kv_heads,
  // head_dim], head_dim 64 or 128. attention_f16kv is attention over the cached values widened exactly (q rotated
  // already); append_rope_attention_f16kv writes fp16(rope(k_new)) and fp16(v_new) into rows pos0.. first and
  // reads q unrotated. Every row runs on the split-context decode kernel (one launch with the append when n = 1).
  void attention_f16kv(const float* q, const void* k16, const void* v16, float* out, int64_t n, int64_t pos0,
                       int64_t n_heads, int64_t n_kv_heads, int64_t head_dim);
  void append_rope_attention_f16kv(const float* q, void* k16, void* v16, const float* k_new, const float* v_new,
                                   float* out, int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads,
                                   int64_t head_dim, const RopeParams& p);
  // Ragged batch of single-token decodes - an extension with no counterpart in the reference, whose Backend serves
  // one sequence: host arrays of n_seq device pointers and positions, sequence i being attention(q[i], k_cache[i],
  // v_cache[i], out[i], 1, pos0[i], ...) over its own caches (equal within rounding: the context split differs).
  // One launch pair streams every sequence's cache at once on the MFMA head sizes (64, 128); other head sizes run
  // one call per sequence.
  void attention_batch(int64_t n_seq, const float* const* q, const float* const* k_cache, const float* const* v_cache,
                       float* const* out, const int64_t* pos0, int64_t n_heads, int64_t n_kv_heads,
                       int64_t head_dim);
  // The same with each sequence's new K/V row appended first and q rotated on load: append_rope_attention with
  // n = 1 for every sequence (appended rows bit-identical).
  void append_rope_attention_batch(int64_t n_seq, const float* const* q, float* const* k_cache,
                                   float* const* v_cache, const float* const* k_new, const float* const* v_new,
                                   float* const* out, const int64_t* pos0, int64_t n_heads, int64_t n_kv_heads,
                                   int64_t head_dim, const RopeParams& p);
  // Attention precision. By default calls of more than 16 rows with head_dim 64/128 run their rows at positions
  // >= 256 on the fp16-operand MFMA kernel (fp32 accumulation and softmax). With fp32 set, every row takes the fp32
  // split-context kernel, as decode does: the reference's float arithmetic throughout, at a much lower prefill
  // rate. For models whose attention scores are large enough that fp16 rounding of Q and K moves the softmax.
  void set_attention_fp32(bool on) { attention_fp32_ = on; }
  // Batch invariance: the reference's CPU kernels compute each row with a fixed accumulation order, so how tokens
  // are batched into calls cannot change a bit (its model tests demand it: test_model.cpp:141-151, 253-263). By
  // default this backend trades that for speed (prefill rows on fp16-operand MFMA, keys split over workgroups by
  // the call's shape, rocBLAS for long float matmuls): results agree within rounding. With batch invariance on,
  // every attention row takes the ordered fp32 route (one workgroup per row over its whole window, keys in position
  // order) and float-weight matmuls of any row count the gemv kernel (16-row slices), so each row's results are
  // bitwise the same however rows are batched - at a much lower prefill rate and a lower decode rate.
  void set_batch_invariant(bool on) { batch_invariant_ = on; }
  bool batch_invariant() const { return batch_invariant_; }
  // Row tiles (128 packed query rows x one KV head) the last MFMA prefill call recomputed with split fp16 operands
  // because their rounding-error estimate exceeded the budget. Waits for queued work.
  int64_t prefill_recomputed();
  bool attention_fp32() const { return attention_fp32_; }
  // Drops every device copy of a host weight (after a caller changes or frees host weight memory).
  void release_weights();
  size_t weight_bytes() const;  // HBM held by weight copies
  void fill_normal(float* dst, int64_t count, uint64_t seed, float scale);
  void sync();
  nbhs_stream stream() const { return stream_; }
  int cu_count() const { return cu_count_; }
  size_t live_allocations() const { return allocs_.size(); }  // test hook (cpu_backend.h:50)
  // Internal device memory held for workspaces and tables, in bytes (test hook: must not grow after reserve).
  size_t internal_bytes() const;

 private:
  struct RopeTable {
    float base = 0;
    int64_t head_dim = 0;
    std::vector<float> factors;  // empty when no freq_factors
    int64_t rows = 0;
    float* dev = nullptr;  // [rows, head_dim/2] (cos, sin) float pairs
  };

  // A weight's device form: the F32/F16 bytes, plus (F16 only) an fp32 widening for the GEMM route.
  struct DeviceWeight {
    DType type = DType::F32;
    int64_t in = 0, rows = 0;
    const void* dev = nullptr;
    const void* key = nullptr;  // host data pointer of a kept copy; null for a weight used in place
    int64_t bytes = 0;          // device bytes of a kept copy (quantized weights: the repacked planes)
    float* f32 = nullptr;       // kept copies only: widening of an F16 weight for the GEMM route
  };
  struct AppendRows {
    const float* k_new;
    const float* v_new;
  };
  void run_decode_f16kv(const float* q, const void* k16, const void* v16, float* out, int64_t n, int64_t pos0,
                        int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, const float* rope_table,
                        int64_t rope_rows, bool neox, const char* op);
  // Prefill over fp16 caches (n > kDecodeMaxRows): staging (fused with the append when k_new is given), the MFMA
  // kernel with its fp32 rows and the recomputation, as run_attention does for fp32 caches. q is rotated on load
  // when rope_table is given.
  void run_prefill_f16kv(const float* q, void* k16, void* v16, float* out, int64_t n, int64_t pos0, int64_t n_heads,
                         int64_t n_kv_heads, int64_t head_dim, const float* rope_table, int64_t rope_rows, bool neox,
                         const float* k_new, const float* v_new, const char* op);
  // Shape and range checks of an attention call; the caches hold elements of cache_elem_bytes (4: fp32, 2: fp16).
  void check_attention_args(const float* q, const void* k, const void* v, const float* out, int64_t n, int64_t pos0,
                            int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, const char* op,
                            int cache_elem_bytes = 4) const;
  void run_attention(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                     int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, const float* rope_table,
                     int64_t rope_rows, bool neox, const AppendRows* app, const RopeParams* rp);
  void run_batch(int64_t n_seq, const float* const* q, const float* const* k, const float* const* v,
                 float* const* out, const float* const* k_new, const float* const* v_new, const int64_t* pos0,
                 int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, const RopeParams* p, const char* op);
  void check(int code, const char* what) const;
  // Throws unless [p, p + n_floats) lies inside one buffer from alloc().
  void check_range(const void* p, int64_t n_floats, const char* op, const char* arg) const;
  const float* rope_table(int64_t head_dim, int64_t rows_needed, const RopeParams& p, int64_t* rows_out);
  void ensure(float*& buf, size_t& cap_bytes, size_t need_bytes);
  void ensure_aux(size_t need_bytes);  // grows the prefill work list, zero-filled
  // The device form of w (copied to HBM on first use unless it lies in a buffer from alloc()).
  DeviceWeight device_weight(const Tensor& w, const char* op);
  // fp32 weights for the GEMM route: F32 as is; a kept F16 copy is widened once (in-place F16 weights take the
  // gemv route instead).
  const float* weight_f32(const DeviceWeight& d);
  bool in_buffer(const void* p, int64_t bytes) const;  // [p, p + bytes) inside one buffer from alloc()

  int device_ = 0;
  int cu_count_ = 0;
  nbhs_stream stream_ = nullptr;
  std::map<uintptr_t, size_t> allocs_;  // user buffers: start -> bytes
  ReserveParams reserved_{0, 0, 0, 0};
  std::vector<RopeTable> rope_tables_;
  float* decode_ws_ = nullptr;  // split-context partials
  size_t decode_ws_bytes_ = 0;
  float* k16_ = nullptr;  // prefill staging: fp16 K and transposed V
  float* vt16_ = nullptr;
  size_t k16_bytes_ = 0, vt16_bytes_ = 0;
  // Bounce buffer for overlapping copies (fixed size; larger copies go through it in chunks).
  static constexpr size_t kBounceBytes = size_t(4) << 20;
  float* copy_tmp_ = nullptr;
  size_t copy_tmp_bytes_ = 0;
  float* rope_slab_ = nullptr;  // device memory reserve() sets aside for the first RoPE table
  size_t rope_slab_bytes_ = 0;
  uint32_t* aux_ = nullptr;     // the MFMA prefill's work list of row tiles to recompute (zeroed on allocation)
  size_t aux_bytes_ = 0;
  std::map<const void*, DeviceWeight> weights_;  // host weight data -> its device form
  nbhs_blas blas_ = nullptr;
  bool attention_fp32_ = false;
  bool batch_invariant_ = false;
  float* ids_buf_ = nullptr;  // token ids of the last embed, on the device
  size_t ids_buf_bytes_ = 0;
  float* acts_buf_ = nullptr;  // activations quantized for quantized weights
  size_t acts_buf_bytes_ = 0;
  // matmul_multi's per-call lists (reused, so a warm call allocates nothing): the call's device weights (then its
  // float weights, compacted), their quantized types, one type's weight indices, the float weights' outputs
  std::vector<DeviceWeight> mm_dw_;
  std::vector<int> mm_types_;
  std::vector<size_t> mm_idx_;
  std::vector<float*> ys_float_;
};

}  // namespace nibble::hip
