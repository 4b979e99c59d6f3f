// HipBackend implementation: argument validation against the allocation table, the RoPE (cos, sin) tables, and
// the routing of attention calls to the decode (fp32, split-context) and prefill (fp16 MFMA) kernels.
// Host-side C++20 only; every device action goes through nibble_hip_shim.h.
#include "backend/hip/hip_backend.h"

#include "kernels/quant_layout.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>

namespace nibble::hip {
namespace {

// Calls with at most this many query rows take the fp32 split-context kernel (decode, short appends).
// K-type calls of more rows than these take the tiled kernels (the small-call one first): measured faster from
// there on at the QKV shape than the 16-row gemv launches
constexpr int64_t kKTiledMinRows = 8, kQ6KTiledMinRows = 4;
constexpr int64_t kDecodeMaxRows = NBHS_DECODE_MAX_ROWS;
constexpr size_t kGemmMaxWeights = NBHS_GEMM_MAX_WEIGHTS;
// Rows per launch of the ordered route (its grid holds one z index per row; a row's result is the same in any launch).
constexpr int64_t kOrderedMaxRows = 32768;
// Prefill rows at positions below this see so few keys that fp16 rounding of single V rows does not average out:
// nearly all of them would be listed for recomputation, so they take the fp32 kernel in the MFMA launch. Rows from
// here on take the MFMA kernel, whose rounding-error estimate lists the row tiles that need recomputing (at 128
// keys and more only a few do; a 256-row prefix made the launch 3 % longer than recomputing rows 128..255's).
constexpr int64_t kFp32PrefixRows = 128;
// matmul calls with at most this many rows take the weight-streaming gemv kernel; longer ones are GEMMs.
constexpr int64_t kGemvMaxRows = NBHS_GEMV_MAX_ROWS;
constexpr size_t kGemvMaxWeights = NBHS_GEMV_MAX_WEIGHTS;
// F16-weight calls of more rows than this take the fp16 MFMA GEMM where it applies, the rest stay on the gemv.
constexpr int64_t kF16GemmMinRows = 11;

std::string str(int64_t v) { return std::to_string(v); }

// Splits a quantized weight's file blocks (src/quant.h:34-110: rows x nb blocks of block_bytes) into the plane
// layout of kernels/quant_layout.h. Bytes are copied unchanged, only moved to aligned places.
std::vector<uint8_t> repack_quant(int t, const uint8_t* src, int64_t rows, int64_t nb) {
  using namespace nbh_quant;
  const WeightLayout l = weight_layout(t, rows, nb);
  std::vector<uint8_t> out(size_t(l.bytes), 0);
  const int64_t bb = block_bytes(t), qb = q_bytes(t), hb = h_bytes(t), sb = s_bytes(t);
  // field offsets inside a file block: d, m (or dmin), scales, qh, quants
  int od = 0, om = -1, os = -1, oh = -1, oq = 2;
  switch (t) {
    case kQ4_0: break;
    case kQ8_0: break;
    case kQ5_0: oh = 2, oq = 6; break;
    case kQ5_1: om = 2, oh = 4, oq = 8; break;
    case kQ4_K: om = 2, os = 4, oq = 16; break;
    case kQ5_K: om = 2, os = 4, oh = 16, oq = 48; break;
    case kQ6_K: od = 208, os = 192, oh = 128, oq = 0; break;
    default: break;
  }
  const int64_t s_len = t == kQ6_K ? 16 : 12;
  // K types: 32-byte groups indexed by the element's position in its sub-block go to residue order
  auto put = [&](uint8_t* dst, const uint8_t* from, int64_t len) {
    if (!is_k(t)) {
      std::memcpy(dst, from, size_t(len));
      return;
    }
    for (int64_t g = 0; g < len; g += 32)
      for (int j = 0; j < 32; ++j) dst[g + residue_pos(j)] = from[g + j];
  };
  for (int64_t i = 0; i < rows * nb; ++i) {
    const uint8_t* b = src + i * bb;
    put(&out[size_t(l.q_off + i * qb)], b + oq, qb);
    std::memcpy(&out[size_t(l.d_off + i * 2)], b + od, 2);
    if (om >= 0) std::memcpy(&out[size_t(l.m_off + i * 2)], b + om, 2);
    if (oh >= 0) put(&out[size_t(l.h_off + i * hb)], b + oh, hb);
    if (os >= 0) std::memcpy(&out[size_t(l.s_off + i * sb)], b + os, size_t(s_len));
  }
  return out;
}

bool overflow_mul(int64_t a, int64_t b, int64_t* out) { return __builtin_mul_overflow(a, b, out); }

}  // namespace

HipBackend::HipBackend(int device) : device_(device) {
  check(nbhs_device_init(device, &cu_count_), "device init");
  check(nbhs_stream_create(&stream_), "stream create");
}

HipBackend::~HipBackend() {
  if (stream_) nbhs_stream_sync(stream_);
  for (auto& [p, bytes] : allocs_) nbhs_free(reinterpret_cast<void*>(p));
  for (auto& t : rope_tables_)
    if (t.dev != rope_slab_) nbhs_free(t.dev);
  nbhs_free(decode_ws_);
  nbhs_free(k16_);
  nbhs_free(vt16_);
  nbhs_free(copy_tmp_);
  nbhs_free(rope_slab_);
  nbhs_free(aux_);
  nbhs_free(ids_buf_);
  nbhs_free(acts_buf_);
  for (auto& [key, d] : weights_) {
    nbhs_free(const_cast<void*>(d.dev));
    nbhs_free(d.f32);
  }
  if (blas_) nbhs_blas_destroy(blas_);
  if (stream_) nbhs_stream_destroy(stream_);
}

void HipBackend::check(int code, const char* what) const {
  if (code != 0) throw Error(std::string("HipBackend: ") + what + " failed: " + nbhs_error_string(code));
}

void HipBackend::check_range(const void* p, int64_t n_floats, const char* op, const char* arg) const {
  if (!p) throw Error(std::string(op) + ": " + arg + " is null");
  int64_t bytes;
  if (n_floats < 0 || overflow_mul(n_floats, int64_t(sizeof(float)), &bytes))
    throw Error(std::string(op) + ": " + arg + " size " + str(n_floats) + " floats is invalid");
  const auto a = reinterpret_cast<uintptr_t>(p);
  auto it = allocs_.upper_bound(a);
  if (it != allocs_.begin()) {
    --it;
    if (a >= it->first && a - it->first + uint64_t(bytes) <= it->second) return;
  }
  throw Error(std::string(op) + ": " + arg + " range of " + str(n_floats) +
              " floats is not inside one buffer allocated by this backend");
}

void HipBackend::ensure(float*& buf, size_t& cap_bytes, size_t need_bytes) {
  if (need_bytes <= cap_bytes) return;
  check(nbhs_stream_sync(stream_), "sync before workspace growth");
  check(nbhs_free(buf), "free workspace");
  buf = nullptr;
  cap_bytes = 0;
  void* p = nullptr;
  check(nbhs_malloc(&p, need_bytes), "workspace allocation");
  buf = static_cast<float*>(p);
  cap_bytes = need_bytes;
}

void HipBackend::ensure_aux(size_t need_bytes) {
  if (need_bytes <= aux_bytes_) return;
  float* p = reinterpret_cast<float*>(aux_);
  ensure(p, aux_bytes_, need_bytes);
  aux_ = reinterpret_cast<uint32_t*>(p);
  // a fresh list: no entry may carry a live epoch
  check(nbhs_zero(aux_, aux_bytes_, stream_), "prefill work list zero-fill");
}

size_t HipBackend::internal_bytes() const {
  size_t s = decode_ws_bytes_ + k16_bytes_ + vt16_bytes_ + copy_tmp_bytes_ + ids_buf_bytes_ + acts_buf_bytes_ +
             rope_slab_bytes_ + aux_bytes_;
  for (auto& t : rope_tables_)
    if (t.dev != rope_slab_) s += size_t(t.rows) * size_t(t.head_dim) * sizeof(float);
  return s;
}

void HipBackend::reserve(const ReserveParams& rp) {
  if (rp.n_ctx < 0 || rp.n_heads < 0 || rp.max_rows < 0 || rp.max_width < 0)
    throw Error("reserve: negative size (n_ctx=" + str(rp.n_ctx) + " n_heads=" + str(rp.n_heads) + " max_rows=" +
                str(rp.max_rows) + " max_width=" + str(rp.max_width) + ")");
  // Every size is computed (and overflow-checked) before anything is allocated, so a bad request changes nothing.
  // Split-context partials (decode chunks, and the key splits of short prefill chunks share the buffer), sized for
  // the worst split either kernel plans for this many query heads.
  const int64_t floats = nbhs_attn_decode_workspace_bound(std::max<int64_t>(rp.n_heads, 1), cu_count_);
  if (floats < 0) throw Error("reserve: invalid n_heads " + str(rp.n_heads));
  const int64_t ws_floats = std::max(floats, nbhs_attn_prefill_workspace_bound(cu_count_));
  // Quantized activations of up to max_rows rows of width up to max_width: the largest companion-format buffer
  // over the quantized types (their row-major and residue-major forms have one size).
  int64_t acts = 0;
  if (rp.max_rows > 0)
    for (const int t : {2, 6, 7, 8, 12, 13, 14}) {
      const int64_t be = nbh_quant::block_elems(t), w = rp.max_width / be * be;
      if (w > 0) {
        const int64_t b = nbhs_quant_act_bytes(t, rp.max_rows, w);
        if (b < 0) throw Error("reserve: activation scratch for max_rows=" + str(rp.max_rows) + " max_width=" +
                               str(rp.max_width) + " is too large");
        acts = std::max(acts, b);
      }
    }
  // The F16-weight GEMM's split activations share that buffer: max_rows rows of width up to max_width.
  if (rp.max_rows > 0 && rp.max_width > 0) {
    const int64_t g = nbhs_gemm_f16w_workspace(rp.max_rows, rp.max_width);
    if (g < 0) throw Error("reserve: GEMM scratch for max_rows=" + str(rp.max_rows) + " max_width=" +
                           str(rp.max_width) + " is too large");
    acts = std::max(acts, g);
  }
  // fp16 prefill staging for up to n_ctx rows. A cache row holds n_kv_heads * head_dim <= n_heads * head_dim <=
  // max_width floats (max_width is at least n_heads * head_dim, backend.h:22-23); the MFMA route's head_dim is at
  // least 64, so n_kv_heads <= max_width / 64 bounds the per-head tile statistics too.
  int64_t staging = 0;
  if (rp.n_ctx > 0 && rp.max_width >= 64) {
    staging = nbhs_prefill_staging_halves(rp.n_ctx, rp.max_width / 64, 64);
    if (staging < 0 || overflow_mul(staging, 2, &staging))
      throw Error("reserve: prefill staging for n_ctx=" + str(rp.n_ctx) + " is too large");
  }
  // RoPE (cos, sin) table: n_ctx rows of head_dim floats, head_dim <= max_width / n_heads.
  int64_t rope_floats = 0;
  if (rp.n_ctx > 0 && rp.n_heads > 0 && overflow_mul(rp.n_ctx, rp.max_width / rp.n_heads, &rope_floats))
    throw Error("reserve: RoPE table for n_ctx=" + str(rp.n_ctx) + " is too large");
  int64_t ids_bytes;
  if (overflow_mul(rp.max_rows, int64_t(sizeof(int32_t)), &ids_bytes)) throw Error("reserve: max_rows too large");
  // the prefill work list of a call of up to max_rows rows (one word per (row tile, KV head)), for any KV head count
  const int64_t aux_words = rp.max_rows > 0 && rp.n_heads > 0 ? nbhs_prefill_aux_words_bound(rp.max_rows, rp.n_heads) : 0;
  reserved_ = rp;
  ensure(decode_ws_, decode_ws_bytes_, size_t(ws_floats) * sizeof(float));
  ensure(acts_buf_, acts_buf_bytes_, size_t(acts));
  ensure(ids_buf_, ids_buf_bytes_, size_t(ids_bytes));
  ensure(k16_, k16_bytes_, size_t(staging));
  ensure(vt16_, vt16_bytes_, size_t(staging));
  ensure(copy_tmp_, copy_tmp_bytes_, kBounceBytes);
  ensure_aux(size_t(std::max<int64_t>(aux_words, 0)) * sizeof(uint32_t));
  if (size_t(rope_floats) * sizeof(float) > rope_slab_bytes_) {
    // The slab is about to be replaced: a table living in it is dropped and rebuilt into the new slab on next use.
    std::erase_if(rope_tables_, [&](const RopeTable& t) { return rope_slab_ && t.dev == rope_slab_; });
    ensure(rope_slab_, rope_slab_bytes_, size_t(rope_floats) * sizeof(float));
  }
}

void HipBackend::reserve_attention(int64_t n_kv_heads, int64_t head_dim) {
  if (head_dim != 64 && head_dim != 128) return;  // no staging on the generic path
  const int64_t halves = nbhs_prefill_staging_halves(std::max<int64_t>(reserved_.n_ctx, 1), n_kv_heads, head_dim);
  if (halves < 0) throw Error("reserve_attention: invalid n_kv_heads " + str(n_kv_heads));
  // exact size for these caches: replaces the bound reserve() took from max_width when that is larger
  const size_t need = size_t(halves) * 2;
  if (k16_bytes_ > need) {
    check(nbhs_stream_sync(stream_), "sync before staging resize");
    nbhs_free(k16_);
    nbhs_free(vt16_);
    k16_ = vt16_ = nullptr;
    k16_bytes_ = vt16_bytes_ = 0;
  }
  ensure(k16_, k16_bytes_, need);
  ensure(vt16_, vt16_bytes_, need);
}

void HipBackend::reserve_rope(int64_t head_dim, const RopeParams& p) {
  if (head_dim <= 0 || head_dim % 2 != 0) throw Error("reserve_rope: head_dim must be positive and even");
  int64_t rows;
  rope_table(head_dim, std::max<int64_t>(reserved_.n_ctx, 1), p, &rows);
}

float* HipBackend::alloc(int64_t n_floats) {
  if (n_floats < 0) throw Error("alloc: negative size " + str(n_floats) + " floats");
  int64_t bytes;
  if (overflow_mul(n_floats, int64_t(sizeof(float)), &bytes) || bytes > INT64_MAX - 63)
    throw Error("alloc: size of " + str(n_floats) + " floats overflows");
  bytes = std::max<int64_t>(64, (bytes + 63) & ~int64_t(63));
  void* p = nullptr;
  if (nbhs_malloc(&p, size_t(bytes)) != 0 || !p) throw Error("alloc: cannot allocate " + str(bytes) + " bytes of HBM");
  const int zr = nbhs_zero(p, size_t(bytes), stream_);
  if (zr != 0) {
    nbhs_free(p);
    check(zr, "alloc zero-fill");
  }
  allocs_.emplace(reinterpret_cast<uintptr_t>(p), size_t(bytes));
  return static_cast<float*>(p);
}

void HipBackend::free(float* p) {
  if (!p) return;
  auto it = allocs_.find(reinterpret_cast<uintptr_t>(p));
  if (it == allocs_.end()) return;  // not ours: ignore rather than risk a double free
  nbhs_stream_sync(stream_);        // queued work may still use it
  nbhs_free(p);
  allocs_.erase(it);
}

void HipBackend::read(float* host_dst, const float* src, int64_t n) {
  if (n < 0 || (n > 0 && !host_dst)) throw Error("read: invalid destination or size " + str(n));
  if (n == 0) return;
  check_range(src, n, "read", "src");
  check(nbhs_memcpy_d2h(host_dst, src, size_t(n) * sizeof(float), stream_), "read");
}

void HipBackend::write(float* dst, const float* host_src, int64_t n) {
  if (n < 0 || (n > 0 && !host_src)) throw Error("write: invalid source or size " + str(n));
  if (n == 0) return;
  check_range(dst, n, "write", "dst");
  check(nbhs_memcpy_h2d(dst, host_src, size_t(n) * sizeof(float), stream_), "write");
}

void HipBackend::copy(float* dst, const float* src, int64_t count) {
  if (count < 0) throw Error("copy: negative count " + str(count));
  if (count == 0 || dst == src) return;
  check_range(dst, count, "copy", "dst");
  check_range(src, count, "copy", "src");
  const size_t bytes = size_t(count) * sizeof(float);
  const auto d = reinterpret_cast<uintptr_t>(dst), s = reinterpret_cast<uintptr_t>(src);
  if (!(d < s + bytes && s < d + bytes)) {
    check(nbhs_memcpy_d2d(dst, src, bytes, stream_), "copy");
    return;
  }
  // Overlapping ranges (memmove semantics, cpu_backend.cpp:260-263): bounce through the fixed scratch, chunk by
  // chunk, front to back when moving down and back to front when moving up, so no chunk reads bytes an earlier
  // chunk has written. The scratch is allocated by reserve(), so copies of any size allocate nothing after it.
  ensure(copy_tmp_, copy_tmp_bytes_, std::min(bytes, kBounceBytes));
  const size_t chunk = copy_tmp_bytes_ / sizeof(float) * sizeof(float);
  auto* db = reinterpret_cast<uint8_t*>(dst);
  const auto* sb = reinterpret_cast<const uint8_t*>(src);
  auto piece = [&](size_t off, size_t len) {
    check(nbhs_memcpy_d2d(copy_tmp_, sb + off, len, stream_), "copy");
    check(nbhs_memcpy_d2d(db + off, copy_tmp_, len, stream_), "copy");
  };
  if (d < s) {
    for (size_t off = 0; off < bytes; off += chunk) piece(off, std::min(chunk, bytes - off));
  } else {
    for (size_t end = bytes; end > 0;) {
      const size_t len = std::min(chunk, end);
      end -= len;
      piece(end, len);
    }
  }
}

void HipBackend::sync() { check(nbhs_stream_sync(stream_), "sync"); }

int64_t HipBackend::prefill_recomputed() {
  if (!aux_) return 0;
  uint32_t n = 0;
  check(nbhs_memcpy_d2h(&n, aux_, sizeof(n), stream_), "prefill_recomputed");
  return int64_t(n);
}

void HipBackend::fill_normal(float* dst, int64_t count, uint64_t seed, float scale) {
  if (count == 0) return;
  check_range(dst, count, "fill_normal", "dst");
  check(nbhs_fill_normal_f32(dst, count, seed, scale, stream_), "fill_normal");
}

// ---- weights and the QKV projection (transformer.cpp:171-194) ----

bool HipBackend::in_buffer(const void* p, int64_t bytes) const {
  const auto a = reinterpret_cast<uintptr_t>(p);
  auto it = allocs_.upper_bound(a);
  if (it == allocs_.begin()) return false;
  --it;
  return a >= it->first && a - it->first + uint64_t(bytes) <= it->second;
}

HipBackend::DeviceWeight HipBackend::device_weight(const Tensor& w, const char* op) {
  if (!w.data) throw Error(std::string(op) + ": weight data is null");
  const bool quant = nbh_quant::is_quant(int(w.type));
  if (w.type != DType::F32 && w.type != DType::F16 && !quant)
    throw Error(std::string(op) + ": weight type " + str(int64_t(w.type)) + " is not supported by the GPU backend");
  const int64_t in = w.ne[0], rows = w.rows();
  int64_t count, bytes;
  if (in <= 0 || rows <= 0 || overflow_mul(in, rows, &count))
    throw Error(std::string(op) + ": invalid weight shape " + str(in) + " x " + str(rows));
  if (quant) {
    const int64_t be = nbh_quant::block_elems(int(w.type));
    if (in % be != 0)
      throw Error(std::string(op) + ": quantized weight width " + str(in) + " is not a multiple of " + str(be));
    if (overflow_mul(count / be, nbh_quant::block_bytes(int(w.type)), &bytes))
      throw Error(std::string(op) + ": weight size overflows");
  } else {
    const int64_t elem = w.type == DType::F32 ? 4 : 2;
    if (overflow_mul(count, elem, &bytes)) throw Error(std::string(op) + ": weight size overflows");
    if (reinterpret_cast<uintptr_t>(w.data) % size_t(elem) != 0)
      throw Error(std::string(op) + ": weight data is not aligned to its element size");
  }
  DeviceWeight d;
  d.type = w.type;
  d.in = in;
  d.rows = rows;
  if (in_buffer(w.data, bytes)) {  // already in HBM: use in place
    if (quant)
      throw Error(std::string(op) + ": a quantized weight must be host memory (it is repacked on upload)");
    d.dev = w.data;
    return d;
  }
  auto it = weights_.find(w.data);
  if (it != weights_.end()) {
    if (it->second.type == w.type && it->second.in == in && it->second.rows == rows) return it->second;
    // The same host address now describes another tensor: replace the copy.
    check(nbhs_stream_sync(stream_), "sync before weight replacement");
    nbhs_free(const_cast<void*>(it->second.dev));
    nbhs_free(it->second.f32);
    weights_.erase(it);
  }
  std::vector<uint8_t> planes;
  const void* src = w.data;
  if (quant) {
    planes = repack_quant(int(w.type), static_cast<const uint8_t*>(w.data), rows,
                          in / nbh_quant::block_elems(int(w.type)));
    src = planes.data();
    bytes = int64_t(planes.size());
  }
  void* p = nullptr;
  check(nbhs_malloc(&p, size_t(bytes)), "weight allocation");
  const int cr = nbhs_memcpy_h2d(p, src, size_t(bytes), stream_);
  if (cr != 0) {
    nbhs_free(p);
    check(cr, "weight upload");
  }
  d.dev = p;
  d.key = w.data;
  d.bytes = bytes;
  weights_.emplace(w.data, d);
  return d;
}

const float* HipBackend::weight_f32(const DeviceWeight& d) {
  if (d.type == DType::F32) return static_cast<const float*>(d.dev);
  const int64_t count = d.in * d.rows;
  DeviceWeight& kept = weights_.at(d.key);  // in-place F16 weights never get here (matmul_multi)
  if (!kept.f32) {
    void* p = nullptr;
    check(nbhs_malloc(&p, size_t(count) * sizeof(float)), "weight widening allocation");
    const int cr = nbhs_f16_to_f32(kept.dev, static_cast<float*>(p), count, stream_);
    if (cr != 0) {
      nbhs_free(p);
      check(cr, "weight widening");
    }
    kept.f32 = static_cast<float*>(p);
  }
  return kept.f32;
}

void HipBackend::release_weights() {
  if (weights_.empty()) return;
  check(nbhs_stream_sync(stream_), "sync before weight release");
  for (auto& [key, d] : weights_) {
    nbhs_free(const_cast<void*>(d.dev));
    nbhs_free(d.f32);
  }
  weights_.clear();
}

size_t HipBackend::weight_bytes() const {
  size_t s = 0;
  for (auto& [key, d] : weights_) s += size_t(d.bytes) + (d.f32 ? size_t(d.in) * size_t(d.rows) * 4 : 0);
  return s;
}

bool HipBackend::supports(DType t) const {
  return t == DType::F32 || t == DType::F16 || nbh_quant::is_quant(int(t));
}

void HipBackend::matmul(const Tensor& w, const float* x, float* y, int64_t n) {
  const Tensor* ws[] = {&w};
  float* ys[] = {y};
  matmul_multi(ws, x, ys, n);
}

void HipBackend::matmul_multi(std::span<const Tensor* const> ws, const float* x, std::span<float* const> ys,
                              int64_t n) {
  if (ws.empty() || ws.size() != ys.size())
    throw Error("matmul: " + str(int64_t(ws.size())) + " weights for " + str(int64_t(ys.size())) + " outputs");
  if (n <= 0) throw Error("matmul: n must be positive, got " + str(n));
  for (const Tensor* t : ws)
    if (!t) throw Error("matmul: null weight");
  const int64_t in = ws[0]->ne[0];
  for (const Tensor* t : ws)
    if (t->ne[0] != in) {  // different input widths: one call per weight (backend.h:58-60)
      for (size_t i = 0; i < ws.size(); ++i) matmul(*ws[i], x, ys[i], n);
      return;
    }
  int64_t x_count;
  if (overflow_mul(n, in, &x_count)) throw Error("matmul: n x width overflows");
  check_range(x, x_count, "matmul", "x");
  // Per-call lists live in member vectors that only grow: after the first call of a given weight count nothing
  // here allocates (alloc_tests.cpp:278-337 counts every operator new of a warm matmul).
  std::vector<DeviceWeight>& dw = mm_dw_;
  dw.clear();
  const auto xa = reinterpret_cast<uintptr_t>(x);
  for (size_t i = 0; i < ws.size(); ++i) {
    dw.push_back(device_weight(*ws[i], "matmul"));
    int64_t y_count;
    if (overflow_mul(n, dw.back().rows, &y_count)) throw Error("matmul: n x rows overflows");
    check_range(ys[i], y_count, "matmul", "y");
    const auto ya = reinterpret_cast<uintptr_t>(ys[i]);
    if (ya < xa + uint64_t(x_count) * 4 && xa < ya + uint64_t(y_count) * 4)
      throw Error("matmul: output " + str(int64_t(i)) + " overlaps the input");
  }
  // Quantized weights (ref_ops.cpp:109-135): the weights of one type share one launch per chunk of up to 16
  // activation rows. Up to 4 rows are quantized inside that launch; more are quantized once per activation format
  // first, as CpuBackend::matmul_multi quantizes the shared input once (cpu_backend.cpp:146-240).
  std::vector<int>& types = mm_types_;
  types.clear();
  for (size_t i = 0; i < dw.size(); ++i) {
    const int t = int(dw[i].type);
    if (nbh_quant::is_quant(t) && std::find(types.begin(), types.end(), t) == types.end()) types.push_back(t);
  }
  const bool fuse = n <= 4 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && in % 4 == 0;
  int done_act = -1;
  for (const int t : types) {
    // the tiled kernels from more than 16 rows on (K types: 8, Q6_K: 4), whose K-type activations are in
    // residue-major order
    const int64_t min_rows =
        t == nbh_quant::kQ6_K ? kQ6KTiledMinRows : nbh_quant::is_k(t) ? kKTiledMinRows : kGemvMaxRows;
    const bool tiled = n > min_rows;
    const bool rm = tiled && nbh_quant::is_k(t);
    const int act_key = 2 * nbh_quant::act_of(t) + (rm ? 1 : 0);
    if (!fuse && act_key != done_act) {
      const int64_t ab = nbhs_quant_act_bytes(t, n, in);
      if (ab < 0) throw Error("matmul: invalid quantized shape");
      ensure(acts_buf_, acts_buf_bytes_, size_t(ab));
      check(rm ? nbhs_quantize_acts_rm(t, x, n, in, acts_buf_, stream_)
               : nbhs_quantize_acts(t, x, n, in, acts_buf_, stream_),
            "matmul (activation quantization)");
      done_act = act_key;
    }
    std::vector<size_t>& idx = mm_idx_;
    idx.clear();
    for (size_t i = 0; i < dw.size(); ++i)
      if (int(dw[i].type) == t) idx.push_back(i);
    if (tiled) {  // up to 8 weights a launch
      for (size_t b = 0; b < idx.size(); b += kGemvMaxWeights) {
        const size_t cnt = std::min(idx.size() - b, kGemvMaxWeights);
        const void* wp[kGemvMaxWeights];
        int64_t rows[kGemvMaxWeights];
        float* yp[kGemvMaxWeights];
        for (size_t j = 0; j < cnt; ++j) {
          const size_t i = idx[b + j];
          wp[j] = dw[i].dev;
          rows[j] = dw[i].rows;
          yp[j] = ys[i];
        }
        check(nbhs_qgemm_multi(t, int(cnt), wp, rows, yp, in, acts_buf_, n, stream_), "matmul (quantized, tiled)");
      }
      continue;
    }
    for (size_t b = 0; b < idx.size(); b += kGemvMaxWeights) {
      const size_t cnt = std::min(idx.size() - b, kGemvMaxWeights);
      const void* wp[kGemvMaxWeights];
      int64_t rows[kGemvMaxWeights];
      float* yp[kGemvMaxWeights];
      for (int64_t t0 = 0; t0 < n; t0 += kGemvMaxRows) {
        for (size_t j = 0; j < cnt; ++j) {
          const size_t i = idx[b + j];
          wp[j] = dw[i].dev;
          rows[j] = dw[i].rows;
          yp[j] = ys[i] + t0 * dw[i].rows;
        }
        check(nbhs_qgemv_multi(t, int(cnt), wp, rows, yp, in, x, fuse ? nullptr : acts_buf_, n, t0,
                               std::min(kGemvMaxRows, n - t0), stream_),
              "matmul (quantized)");
      }
    }
  }
  // the float weights and their outputs, compacted to the front of the lists
  size_t nf = 0;
  ys_float_.clear();
  for (size_t i = 0; i < dw.size(); ++i)
    if (!nbh_quant::is_quant(int(dw[i].type))) {
      dw[nf++] = dw[i];
      ys_float_.push_back(ys[i]);
    }
  dw.resize(nf);
  if (dw.empty()) return;
  const std::vector<float*>& yv = ys_float_;
  // F16 weights the fp16 MFMA GEMM below can take (16-byte aligned rows of a multiple of 8 elements)
  const bool gemm_ok = !batch_invariant_ && in % 8 == 0;
  auto f16_gemm = [&](const DeviceWeight& w) {
    return gemm_ok && w.type == DType::F16 && reinterpret_cast<uintptr_t>(w.dev) % 16 == 0;
  };
  if (n <= kGemvMaxRows) {
    // Above kF16GemmMinRows rows those F16 weights take the GEMM (its K ranges fill the CUs sooner than the
    // gemv's per-row work grows); the others stay here.
    size_t ng = 0;
    if (n > kF16GemmMinRows)
      for (size_t i = 0; i < dw.size(); ++i)
        if (f16_gemm(dw[i])) {
          std::swap(dw[ng], dw[i]);
          std::swap(ys_float_[ng++], ys_float_[i]);
        }
    // One launch per (up to) eight weights: every weight row is read once for all n rows.
    for (size_t b = ng; b < dw.size(); b += kGemvMaxWeights) {
      const size_t cnt = std::min(dw.size() - b, kGemvMaxWeights);
      int f16[kGemvMaxWeights];
      const void* wp[kGemvMaxWeights];
      float* yp[kGemvMaxWeights];
      int64_t rows[kGemvMaxWeights];
      for (size_t j = 0; j < cnt; ++j) {
        f16[j] = dw[b + j].type == DType::F16;
        wp[j] = dw[b + j].dev;
        yp[j] = yv[b + j];
        rows[j] = dw[b + j].rows;
      }
      check(nbhs_gemv_multi(int(cnt), f16, wp, yp, rows, in, x, n, stream_), "matmul (gemv)");
    }
    if (ng == 0) return;
    dw.resize(ng);
    ys_float_.resize(ng);
  }
  // F16 weights on the fp16 MFMA GEMM (split activations, fp32-grade results, no fp32 copy of the weight): up to
  // eight per launch, sharing one split of x. Its scratch is the activation buffer (stream order keeps the
  // quantized launches above, which read that buffer, ahead of the split that overwrites it).
  if (gemm_ok) {
    size_t ng = 0;
    for (size_t i = 0; i < dw.size(); ++i)
      if (f16_gemm(dw[i])) ++ng;
    if (ng > 0) {
      const int64_t ws = nbhs_gemm_f16w_workspace(n, in);
      if (ws < 0) throw Error("matmul: invalid GEMM shape n=" + str(n) + " in=" + str(in));
      ensure(acts_buf_, acts_buf_bytes_, size_t(ws));
      const void* wp[kGemmMaxWeights];
      float* yp[kGemmMaxWeights];
      int64_t rows[kGemmMaxWeights];
      size_t cnt = 0, kept = 0;
      auto flush = [&]() {
        if (cnt == 0) return;
        check(nbhs_gemm_f16w_multi(int(cnt), wp, yp, rows, in, x, n, acts_buf_, int64_t(acts_buf_bytes_), stream_),
              "matmul (f16 GEMM)");
        cnt = 0;
      };
      for (size_t i = 0; i < dw.size(); ++i) {
        if (f16_gemm(dw[i])) {
          wp[cnt] = dw[i].dev;
          yp[cnt] = yv[i];
          rows[cnt] = dw[i].rows;
          if (++cnt == kGemmMaxWeights) flush();
        } else {  // the other weights stay for the routes below
          dw[kept] = dw[i];
          ys_float_[kept++] = yv[i];
        }
      }
      flush();
      dw.resize(kept);
      ys_float_.resize(kept);
    }
  }
  for (size_t i = 0; i < dw.size(); ++i) {
    if ((dw[i].type == DType::F16 && !dw[i].key) || batch_invariant_) {
      // An F16 weight in a caller's buffer: its bytes may change between calls, so no fp32 widening is kept; the
      // gemv kernel reads it as F16 in 16-row slices of x (no scratch, nothing allocated). With batch invariance
      // every float weight takes this route: the gemv computes each output from its own x row with one summation
      // order whatever the rows per launch, so batching cannot change its bits.
      const int f16 = dw[i].type == DType::F16 ? 1 : 0;
      const void* wp = dw[i].dev;
      const int64_t rows = dw[i].rows;
      for (int64_t t0 = 0; t0 < n; t0 += kGemvMaxRows) {
        float* yp = yv[i] + t0 * rows;
        check(nbhs_gemv_multi(1, &f16, &wp, &yp, &rows, in, x + t0 * in, std::min(kGemvMaxRows, n - t0), stream_),
              "matmul (gemv)");
      }
      continue;
    }
    if (!blas_) check(nbhs_blas_create(&blas_, stream_), "rocBLAS handle");
    check(nbhs_sgemm_xwt(blas_, x, weight_f32(dw[i]), yv[i], n, in, dw[i].rows), "matmul (sgemm)");
  }
}

void HipBackend::embed(const Tensor& table, std::span<const int32_t> ids, float* out) {
  if (ids.empty()) throw Error("embed: no token ids");
  const int64_t n = int64_t(ids.size()), d = table.ne[0], rows = table.rows();
  for (const int32_t id : ids)
    if (id < 0 || id >= rows)
      throw Error("embed: token id " + std::to_string(id) + " out of range (n_vocab " + std::to_string(rows) + ")");
  int64_t count;
  if (d <= 0 || overflow_mul(n, d, &count)) throw Error("embed: invalid table width " + str(d));
  check_range(out, count, "embed", "out");
  const DeviceWeight w = device_weight(table, "embed");
  ensure(ids_buf_, ids_buf_bytes_, size_t(n) * sizeof(int32_t));
  check(nbhs_memcpy_h2d(ids_buf_, ids.data(), size_t(n) * sizeof(int32_t), stream_), "embed ids upload");
  if (nbh_quant::is_quant(int(w.type))) {
    check(nbhs_dequant_rows(int(w.type), w.dev, w.rows, d, reinterpret_cast<const int32_t*>(ids_buf_), n, out,
                            stream_),
          "embed (dequantize)");
    return;
  }
  check(nbhs_embed(w.type == DType::F16, w.dev, reinterpret_cast<const int32_t*>(ids_buf_), n, d, out, stream_),
        "embed");
}

void HipBackend::rmsnorm(const float* x, const Tensor& weight, float* y, int64_t n, float eps) {
  if (n <= 0) throw Error("rmsnorm: n must be positive, got " + str(n));
  if (weight.type != DType::F32) throw Error("rmsnorm: weight type " + str(int64_t(weight.type)) + " (need F32)");
  const int64_t d = weight.ne[0];
  int64_t count;
  if (d <= 0 || overflow_mul(n, d, &count)) throw Error("rmsnorm: invalid weight width " + str(d));
  check_range(x, count, "rmsnorm", "x");
  check_range(y, count, "rmsnorm", "y");
  Tensor row = weight;
  row.n_dims = 1;
  row.ne = {d, 1, 1, 1};
  const DeviceWeight w = device_weight(row, "rmsnorm");
  check(nbhs_rmsnorm_f32(x, static_cast<const float*>(w.dev), y, n, d, eps, stream_), "rmsnorm");
}

void HipBackend::add(float* x, const float* y, int64_t count) {
  if (count <= 0) throw Error("add: count must be positive, got " + str(count));
  check_range(x, count, "add", "x");
  check_range(y, count, "add", "y");
  check(nbhs_add_f32(x, y, count, stream_), "add");
}

void HipBackend::silu_mul(float* gate, const float* up, int64_t count) {
  if (count <= 0) throw Error("silu_mul: count must be positive, got " + str(count));
  check_range(gate, count, "silu_mul", "gate");
  check_range(up, count, "silu_mul", "up");
  check(nbhs_silu_mul_f32(gate, up, count, stream_), "silu_mul");
}

void HipBackend::add_bias(float* x, const Tensor& bias, int64_t n) {
  if (n <= 0) throw Error("add_bias: n must be positive, got " + str(n));
  if (bias.type != DType::F32) throw Error("add_bias: bias type " + str(int64_t(bias.type)) + " (need F32)");
  const int64_t d = bias.ne[0];
  int64_t count;
  if (d <= 0 || overflow_mul(n, d, &count)) throw Error("add_bias: invalid bias width " + str(d));
  check_range(x, count, "add_bias", "x");
  Tensor row = bias;  // the bias is its first ne[0] floats
  row.n_dims = 1;
  row.ne = {d, 1, 1, 1};
  const DeviceWeight b = device_weight(row, "add_bias");
  check(nbhs_add_bias_f32(x, static_cast<const float*>(b.dev), d, n, stream_), "add_bias");
}

// The table holds, for every position `pos` and pair i, float(cos(theta)) and float(sin(theta)) with
// theta = double(pos) * pow(double(base), -2i/head_dim) [/ double(freq_factors[i])] - the reference's angle
// (ref_ops.cpp:169-176) computed by the same libm calls on the same doubles, so the device rotation that reads it is
// bit-exact. pow depends only on i, so it is evaluated once per pair; the product is the reference's own.
const float* HipBackend::rope_table(int64_t head_dim, int64_t rows_needed, const RopeParams& p, int64_t* rows_out) {
  const int64_t half = head_dim / 2;
  auto same = [&](const RopeTable& t) {
    if (std::memcmp(&t.base, &p.freq_base, sizeof(float)) != 0 || t.head_dim != head_dim) return false;
    if (!p.freq_factors) return t.factors.empty();
    return !t.factors.empty() && std::memcmp(t.factors.data(), p.freq_factors, size_t(half) * sizeof(float)) == 0;
  };
  auto it = std::find_if(rope_tables_.begin(), rope_tables_.end(), same);
  if (it != rope_tables_.end() && it->rows >= rows_needed) {
    *rows_out = it->rows;
    return it->dev;
  }
  // Past the reserved n_ctx a table at least doubles (in whole 1024-row blocks), so positions that creep up one
  // per decode step rebuild it a logarithmic number of times, not once per step.
  int64_t rows = std::max(rows_needed, reserved_.n_ctx);
  if (rows > reserved_.n_ctx) {
    if (it != rope_tables_.end()) rows = std::max(rows, 2 * it->rows);
    rows = (rows + 1023) / 1024 * 1024;
  }
  int64_t entries;
  if (overflow_mul(rows, head_dim, &entries)) throw Error("rope: table size overflows");
  std::vector<float> host(static_cast<size_t>(entries));
  std::vector<double> inv(static_cast<size_t>(half));
  for (int64_t i = 0; i < half; ++i)
    inv[size_t(i)] = std::pow(static_cast<double>(p.freq_base), -2.0 * static_cast<double>(i) / static_cast<double>(head_dim));
  const float* ff = p.freq_factors;
  auto fill = [&](int64_t r0, int64_t r1) {
    for (int64_t pos = r0; pos < r1; ++pos) {
      const double dpos = static_cast<double>(pos);
      float* row = host.data() + pos * head_dim;
      for (int64_t i = 0; i < half; ++i) {
        double theta = dpos * inv[size_t(i)];
        if (ff) theta /= ff[i];
        row[2 * i] = static_cast<float>(std::cos(theta));
        row[2 * i + 1] = static_cast<float>(std::sin(theta));
      }
    }
  };
  const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  const int64_t nt = entries > (int64_t(1) << 16) ? int64_t(hw) : 1;
  if (nt == 1) {
    fill(0, rows);
  } else {
    std::vector<std::thread> th;
    const int64_t step = (rows + nt - 1) / nt;
    for (int64_t r = 0; r < rows; r += step) th.emplace_back(fill, r, std::min(rows, r + step));
    for (auto& x : th) x.join();
  }
  // The first table whose rows fit goes into the slab reserve() sized from n_ctx and max_width (no allocation);
  // others, and tables grown past it, get their own buffer.
  const size_t tbytes = size_t(entries) * sizeof(float);
  const bool slab_free =
      std::none_of(rope_tables_.begin(), rope_tables_.end(), [&](const RopeTable& t) { return t.dev == rope_slab_; });
  bool was_slab = false;  // a growing table that held the slab may keep it
  if (it == rope_tables_.end()) {
    rope_tables_.push_back(RopeTable{});
    it = rope_tables_.end() - 1;
    it->base = p.freq_base;
    it->head_dim = head_dim;
    if (ff) it->factors.assign(ff, ff + half);
  } else {
    check(nbhs_stream_sync(stream_), "sync before rope table growth");  // queued work may still read it
    was_slab = rope_slab_ && it->dev == rope_slab_;
    if (!was_slab) check(nbhs_free(it->dev), "free rope table");
    it->dev = nullptr;
    it->rows = 0;
  }
  if (rope_slab_ && tbytes <= rope_slab_bytes_ && (slab_free || was_slab)) {
    it->dev = rope_slab_;
  } else {
    void* d = nullptr;
    check(nbhs_malloc(&d, tbytes), "rope table allocation");
    it->dev = static_cast<float*>(d);
  }
  it->rows = rows;
  check(nbhs_memcpy_h2d(it->dev, host.data(), tbytes, stream_), "rope table upload");
  *rows_out = rows;
  return it->dev;
}

void HipBackend::rope(float* x, int64_t n, int64_t n_heads, int64_t head_dim, int64_t pos0, const RopeParams& p) {
  if (n <= 0 || n_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0 || pos0 < 0)
    throw Error("rope: invalid shape n=" + str(n) + " n_heads=" + str(n_heads) + " head_dim=" + str(head_dim) +
                " (must be even) pos0=" + str(pos0));
  int64_t count;
  if (overflow_mul(n, n_heads, &count) || overflow_mul(count, head_dim, &count)) throw Error("rope: size overflows");
  check_range(x, count, "rope", "x");
  int64_t rows;
  const float* table = rope_table(head_dim, pos0 + n, p, &rows);
  check(nbhs_rope_f32(x, n, n_heads, head_dim, pos0, table, rows, p.neox ? 1 : 0, stream_), "rope");
}

void HipBackend::append_rope(float* q, float* k_cache, float* v_cache, const float* k_new, const float* v_new,
                             int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                             const RopeParams& p) {
  if (n <= 0 || n_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 2 != 0 || pos0 < 0)
    throw Error("append_rope: invalid shape n=" + str(n) + " n_heads=" + str(n_heads) + " n_kv_heads=" +
                str(n_kv_heads) + " head_dim=" + str(head_dim) + " pos0=" + str(pos0));
  int64_t qf, kvf, cachef;
  if (overflow_mul(n * n_heads, head_dim, &qf) || overflow_mul(n * n_kv_heads, head_dim, &kvf) ||
      overflow_mul((pos0 + n) * n_kv_heads, head_dim, &cachef))
    throw Error("append_rope: size overflows");
  check_range(q, qf, "append_rope", "q");
  check_range(k_new, kvf, "append_rope", "k_new");
  check_range(v_new, kvf, "append_rope", "v_new");
  check_range(k_cache, cachef, "append_rope", "k_cache");
  check_range(v_cache, cachef, "append_rope", "v_cache");
  int64_t rows;
  const float* table = rope_table(head_dim, pos0 + n, p, &rows);
  check(nbhs_append_rope_f32(q, k_cache, v_cache, k_new, v_new, n, pos0, n_heads, n_kv_heads, head_dim, table, rows,
                             p.neox ? 1 : 0, stream_),
        "append_rope");
}

void HipBackend::attention(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                           int64_t n_heads, int64_t n_kv_heads, int64_t head_dim) {
  check_attention_args(q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim, "attention");
  run_attention(q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim, nullptr, 0, false, nullptr, nullptr);
}

void HipBackend::append_rope_attention(const float* q, float* k_cache, float* v_cache, const float* k_new,
                                       const float* v_new, float* out, int64_t n, int64_t pos0, int64_t n_heads,
                                       int64_t n_kv_heads, int64_t head_dim, const RopeParams& p) {
  if (head_dim % 2 != 0) throw Error("append_rope_attention: head_dim must be even, got " + str(head_dim));
  check_attention_args(q, k_cache, v_cache, out, n, pos0, n_heads, n_kv_heads, head_dim, "append_rope_attention");
  int64_t kvf;
  if (overflow_mul(n * n_kv_heads, head_dim, &kvf)) throw Error("append_rope_attention: size overflows");
  check_range(k_new, kvf, "append_rope_attention", "k_new");
  check_range(v_new, kvf, "append_rope_attention", "v_new");
  int64_t rows;
  const float* table = rope_table(head_dim, pos0 + n, p, &rows);
  if (head_dim != 64 && head_dim != 128) {
    // No rotation-on-load for other head sizes: rotate a copy of q.
    int64_t qf = n * n_heads * head_dim;
    ensure(copy_tmp_, copy_tmp_bytes_, size_t(qf) * sizeof(float));
    check(nbhs_memcpy_d2d(copy_tmp_, q, size_t(qf) * sizeof(float), stream_), "append_rope_attention");
    check(nbhs_append_rope_f32(copy_tmp_, k_cache, v_cache, k_new, v_new, n, pos0, n_heads, n_kv_heads, head_dim,
                               table, rows, p.neox ? 1 : 0, stream_),
          "append_rope_attention (append)");
    run_attention(copy_tmp_, k_cache, v_cache, out, n, pos0, n_heads, n_kv_heads, head_dim, nullptr, 0, false,
                  nullptr, nullptr);
    return;
  }
  AppendRows app{k_new, v_new};
  run_attention(q, k_cache, v_cache, out, n, pos0, n_heads, n_kv_heads, head_dim, table, rows, p.neox, &app, &p);
}

void HipBackend::run_decode_f16kv(const float* q, const void* k16, const void* v16, float* out, int64_t n,
                                  int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                  const float* rope_table, int64_t rope_rows, bool neox, const char* op) {
  if (batch_invariant_) {
    const int64_t qw = n_heads * head_dim;
    for (int64_t t0 = 0; t0 < n; t0 += kOrderedMaxRows)
      check(nbhs_attn_decode_ordered_f16kv(q + t0 * qw, k16, v16, out + t0 * qw, std::min(kOrderedMaxRows, n - t0),
                                           pos0 + t0, n_heads, n_kv_heads, head_dim, rope_table, rope_rows,
                                           neox ? 1 : 0, stream_),
            op);
    return;
  }
  // rows in groups the decode kernel's workspace bound covers, q rotated on load when a table is given
  for (int64_t t0 = 0; t0 < n; t0 += kDecodeMaxRows) {
    const int64_t rows = std::min<int64_t>(kDecodeMaxRows, n - t0);
    const int64_t ws = nbhs_attn_decode_workspace(rows, pos0 + t0, n_heads, n_kv_heads, head_dim, cu_count_);
    if (ws < 0) throw Error(std::string(op) + ": invalid decode shape");
    ensure(decode_ws_, decode_ws_bytes_, size_t(ws) * sizeof(float));
    check(nbhs_attn_decode_f16kv(q + t0 * n_heads * head_dim, k16, v16, out + t0 * n_heads * head_dim, rows,
                                 pos0 + t0, n_heads, n_kv_heads, head_dim, decode_ws_,
                                 int64_t(decode_ws_bytes_ / sizeof(float)), cu_count_, rope_table, rope_rows,
                                 neox ? 1 : 0, stream_),
          op);
  }
}

void HipBackend::run_prefill_f16kv(const float* q, void* k16, void* v16, float* out, int64_t n, int64_t pos0,
                                   int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, const float* rope_table,
                                   int64_t rope_rows, bool neox, const float* k_new, const float* v_new,
                                   const char* op) {
  // rows below kFp32PrefixRows (all rows with set_attention_fp32 or batch invariance) take the fp32 kernel, as for
  // fp32 caches
  const int64_t split =
      attention_fp32_ || batch_invariant_ ? n : std::clamp<int64_t>(kFp32PrefixRows - pos0, 0, n);
  if (split == n) {
    if (k_new)
      check(nbhs_append_rope_f16kv(k16, v16, k_new, v_new, n, pos0, n_kv_heads, head_dim, rope_table, rope_rows,
                                   neox ? 1 : 0, stream_),
            op);
    run_decode_f16kv(q, k16, v16, out, n, pos0, n_heads, n_kv_heads, head_dim, rope_table, rope_rows, neox, op);
    return;
  }
  const int64_t rows = pos0 + n;
  const int64_t halves = nbhs_prefill_staging_halves(rows, n_kv_heads, head_dim);
  const int64_t words = nbhs_prefill_aux_words(n - split, n_heads, n_kv_heads);
  if (halves < 0 || words < 0) throw Error(std::string(op) + ": invalid prefill shape");
  ensure(k16_, k16_bytes_, size_t(halves) * 2);
  ensure(vt16_, vt16_bytes_, size_t(halves) * 2);
  ensure_aux(size_t(words) * sizeof(uint32_t));
  const int64_t aux_words = int64_t(aux_bytes_ / sizeof(uint32_t));
  if (k_new)
    check(nbhs_append_stage_kv_f16kv(k16, v16, k_new, v_new, n, pos0, n_kv_heads, head_dim, rope_table, rope_rows,
                                     neox ? 1 : 0, k16_, vt16_, aux_, aux_words, stream_),
          op);
  else
    check(nbhs_stage_kv_f16kv(k16, v16, k16_, vt16_, rows, n_kv_heads, head_dim, aux_, aux_words, stream_), op);
  const int64_t ws = nbhs_attn_prefill_workspace(n, pos0, n_heads, n_kv_heads, head_dim, split, cu_count_);
  if (ws < 0) throw Error(std::string(op) + ": invalid prefill shape");
  ensure(decode_ws_, decode_ws_bytes_, size_t(ws) * sizeof(float));
  check(nbhs_attn_prefill_mfma_f16kv(q, k16_, vt16_, out, n, pos0, n_heads, n_kv_heads, head_dim, (rows + 63) / 64 * 64,
                                     rope_table, rope_rows, neox ? 1 : 0, k16, v16, split, decode_ws_,
                                     int64_t(decode_ws_bytes_ / sizeof(float)), aux_, aux_words, cu_count_, stream_),
        op);
}

void HipBackend::attention_f16kv(const float* q, const void* k16, const void* v16, float* out, int64_t n,
                                 int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim) {
  if (head_dim != 64 && head_dim != 128)
    throw Error("attention_f16kv: head_dim must be 64 or 128, got " + str(head_dim));
  check_attention_args(q, k16, v16, out, n, pos0, n_heads, n_kv_heads, head_dim, "attention_f16kv", 2);
  if (n > kDecodeMaxRows) {  // prefill: the caches are only read (staging takes no new rows)
    run_prefill_f16kv(q, const_cast<void*>(k16), const_cast<void*>(v16), out, n, pos0, n_heads, n_kv_heads, head_dim,
                      nullptr, 0, false, nullptr, nullptr, "attention_f16kv");
    return;
  }
  run_decode_f16kv(q, k16, v16, out, n, pos0, n_heads, n_kv_heads, head_dim, nullptr, 0, false, "attention_f16kv");
}

void HipBackend::append_rope_attention_f16kv(const float* q, void* k16, void* v16, const float* k_new,
                                             const float* v_new, float* out, int64_t n, int64_t pos0,
                                             int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                             const RopeParams& p) {
  const char* op = "append_rope_attention_f16kv";
  if (head_dim != 64 && head_dim != 128) throw Error(std::string(op) + ": head_dim must be 64 or 128, got " + str(head_dim));
  check_attention_args(q, k16, v16, out, n, pos0, n_heads, n_kv_heads, head_dim, op, 2);
  int64_t kvf;
  if (overflow_mul(n * n_kv_heads, head_dim, &kvf)) throw Error(std::string(op) + ": size overflows");
  check_range(k_new, kvf, op, "k_new");
  check_range(v_new, kvf, op, "v_new");
  int64_t rows;
  const float* table = rope_table(head_dim, pos0 + n, p, &rows);
  if (n == 1 && !batch_invariant_) {  // decode step: the append rides in the attention launch
    const int64_t ws = nbhs_attn_decode_workspace(1, pos0, n_heads, n_kv_heads, head_dim, cu_count_);
    if (ws < 0) throw Error(std::string(op) + ": invalid decode shape");
    ensure(decode_ws_, decode_ws_bytes_, size_t(ws) * sizeof(float));
    check(nbhs_append_attn_decode_f16kv(q, k16, v16, k_new, v_new, out, pos0, n_heads, n_kv_heads, head_dim,
                                        decode_ws_, int64_t(decode_ws_bytes_ / sizeof(float)), cu_count_, table, rows,
                                        p.neox ? 1 : 0, stream_),
          op);
    return;
  }
  if (n > kDecodeMaxRows) {  // prefill: the append fused with the staging
    run_prefill_f16kv(q, k16, v16, out, n, pos0, n_heads, n_kv_heads, head_dim, table, rows, p.neox, k_new, v_new, op);
    return;
  }
  check(nbhs_append_rope_f16kv(k16, v16, k_new, v_new, n, pos0, n_kv_heads, head_dim, table, rows, p.neox ? 1 : 0,
                               stream_),
        op);
  run_decode_f16kv(q, k16, v16, out, n, pos0, n_heads, n_kv_heads, head_dim, table, rows, p.neox, op);
}

void HipBackend::attention_batch(int64_t n_seq, const float* const* q, const float* const* k_cache,
                                 const float* const* v_cache, float* const* out, const int64_t* pos0, int64_t n_heads,
                                 int64_t n_kv_heads, int64_t head_dim) {
  run_batch(n_seq, q, k_cache, v_cache, out, nullptr, nullptr, pos0, n_heads, n_kv_heads, head_dim, nullptr,
            "attention_batch");
}

void HipBackend::append_rope_attention_batch(int64_t n_seq, const float* const* q, float* const* k_cache,
                                             float* const* v_cache, const float* const* k_new,
                                             const float* const* v_new, float* const* out, const int64_t* pos0,
                                             int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                             const RopeParams& p) {
  if (n_seq > 0 && (!k_new || !v_new)) throw Error("append_rope_attention_batch: k_new / v_new arrays are null");
  run_batch(n_seq, q, k_cache, v_cache, out, k_new, v_new, pos0, n_heads, n_kv_heads, head_dim, &p,
            "append_rope_attention_batch");
}

void HipBackend::run_batch(int64_t n_seq, const float* const* q, const float* const* k, const float* const* v,
                           float* const* out, const float* const* k_new, const float* const* v_new,
                           const int64_t* pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                           const RopeParams* p, const char* op) {
  if (n_seq < 0) throw Error(std::string(op) + ": negative sequence count " + str(n_seq));
  if (n_seq == 0) return;
  if (!q || !k || !v || !out || !pos0) throw Error(std::string(op) + ": a pointer array is null");
  if (p && head_dim % 2 != 0) throw Error(std::string(op) + ": head_dim must be even, got " + str(head_dim));
  int64_t max_pos = 0;
  for (int64_t i = 0; i < n_seq; ++i) {
    check_attention_args(q[i], k[i], v[i], out[i], 1, pos0[i], n_heads, n_kv_heads, head_dim, op);
    if (p) {
      check_range(k_new[i], n_kv_heads * head_dim, op, "k_new");
      check_range(v_new[i], n_kv_heads * head_dim, op, "v_new");
    }
    max_pos = std::max(max_pos, pos0[i]);
  }
  // no batch kernel for these sizes, and none on the ordered route: one call per sequence
  if ((head_dim != 64 && head_dim != 128) || batch_invariant_) {
    for (int64_t i = 0; i < n_seq; ++i) {
      if (p)
        append_rope_attention(q[i], const_cast<float*>(k[i]), const_cast<float*>(v[i]), k_new[i], v_new[i], out[i],
                              1, pos0[i], n_heads, n_kv_heads, head_dim, *p);
      else
        attention(q[i], k[i], v[i], out[i], 1, pos0[i], n_heads, n_kv_heads, head_dim);
    }
    return;
  }
  const float* table = nullptr;
  int64_t rows = 0;
  if (p) table = rope_table(head_dim, max_pos + 1, *p, &rows);
  const int64_t ws = nbhs_attn_decode_batch_workspace(n_seq, pos0, n_heads, n_kv_heads, head_dim, cu_count_);
  if (ws < 0) throw Error(std::string(op) + ": invalid batch shape");
  ensure(decode_ws_, decode_ws_bytes_, size_t(ws) * sizeof(float));
  check(nbhs_attn_decode_batch_f32(n_seq, q, k, v, out, k_new, v_new, pos0, n_heads, n_kv_heads, head_dim,
                                   decode_ws_, int64_t(decode_ws_bytes_ / sizeof(float)), cu_count_, table, rows,
                                   p && p->neox ? 1 : 0, stream_),
        op);
}

void HipBackend::check_attention_args(const float* q, const void* k, const void* v, const float* out, int64_t n,
                                      int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                      const char* op, int cache_elem_bytes) const {
  if (n <= 0 || pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || head_dim <= 0 ||
      head_dim > 256)
    throw Error(std::string(op) + ": invalid shape n=" + str(n) + " pos0=" + str(pos0) + " n_heads=" + str(n_heads) +
                " n_kv_heads=" + str(n_kv_heads) + " head_dim=" + str(head_dim) +
                " (n_heads must be a multiple of n_kv_heads, head_dim at most 256)");
  int64_t qf, cache_elems, cache_bytes;
  if (overflow_mul(n * n_heads, head_dim, &qf) || overflow_mul((pos0 + n) * n_kv_heads, head_dim, &cache_elems) ||
      overflow_mul(cache_elems, int64_t(cache_elem_bytes), &cache_bytes))
    throw Error(std::string(op) + ": size overflows");
  check_range(q, qf, op, "q");
  check_range(out, qf, op, "out");
  // the caches' extent in whole floats (an fp16 cache of an odd element count ends inside its last float)
  const int64_t cache_floats = (cache_bytes + 3) / 4;
  check_range(k, cache_floats, op, "k");
  check_range(v, cache_floats, op, "v");
}

// Attention over cache rows 0..pos0+t for q rows t. With rope_table set, q is unrotated and rotated on load, and
// with `app` set the rows pos0..pos0+n-1 are appended first (rope(k_new), v_new) - fused with the fp16 staging
// on the MFMA route.
void HipBackend::run_attention(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                               int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, const float* rope_table,
                               int64_t rope_rows, bool neox, const AppendRows* app, const RopeParams* rp) {
  (void)rp;
  auto decode_rows = [&](const float* qq, float* oo, int64_t rows, int64_t p0) {
    const int64_t ws = nbhs_attn_decode_workspace(rows, p0, n_heads, n_kv_heads, head_dim, cu_count_);
    if (ws < 0) throw Error("attention: invalid decode shape");
    ensure(decode_ws_, decode_ws_bytes_, size_t(ws) * sizeof(float));
    check(nbhs_attn_decode_f32(qq, k, v, oo, rows, p0, n_heads, n_kv_heads, head_dim, decode_ws_,
                               int64_t(decode_ws_bytes_ / sizeof(float)), cu_count_, rope_table, rope_rows,
                               neox ? 1 : 0, stream_),
          "attention (decode kernel)");
  };
  // K/V rows only (q stays as given; it is rotated on load)
  auto append_kv = [&]() {
    check(nbhs_append_rope_f32(nullptr, const_cast<float*>(k), const_cast<float*>(v), app->k_new, app->v_new, n,
                               pos0, 0, n_kv_heads, head_dim, rope_table, rope_rows, neox ? 1 : 0, stream_),
          "attention (append)");
  };

  if (batch_invariant_) {  // every row on the ordered route: its result depends on its own keys only
    if (app) append_kv();
    const int64_t qw = n_heads * head_dim;
    for (int64_t t0 = 0; t0 < n; t0 += kOrderedMaxRows)
      check(nbhs_attn_decode_ordered_f32(q + t0 * qw, k, v, out + t0 * qw, std::min(kOrderedMaxRows, n - t0),
                                         pos0 + t0, n_heads, n_kv_heads, head_dim, rope_table, rope_rows,
                                         neox ? 1 : 0, stream_),
            "attention (ordered route)");
    return;
  }
  const bool mfma_shape = head_dim == 64 || head_dim == 128;
  if (app && mfma_shape && n == 1) {  // decode step: the append rides in the attention launch
    const int64_t ws = nbhs_attn_decode_workspace(1, pos0, n_heads, n_kv_heads, head_dim, cu_count_);
    if (ws < 0) throw Error("attention: invalid decode shape");
    ensure(decode_ws_, decode_ws_bytes_, size_t(ws) * sizeof(float));
    check(nbhs_append_attn_decode_f32(q, const_cast<float*>(k), const_cast<float*>(v), app->k_new, app->v_new, out,
                                      pos0, n_heads, n_kv_heads, head_dim, decode_ws_,
                                      int64_t(decode_ws_bytes_ / sizeof(float)), cu_count_, rope_table, rope_rows,
                                      neox ? 1 : 0, stream_),
          "attention (append and decode kernel)");
    return;
  }
  if (!mfma_shape || n <= kDecodeMaxRows) {
    if (app) append_kv();
    decode_rows(q, out, n, pos0);
    return;
  }
  const int64_t split = attention_fp32_ ? n : std::clamp<int64_t>(kFp32PrefixRows - pos0, 0, n);
  const int64_t rows = pos0 + n;
  const int64_t halves = nbhs_prefill_staging_halves(rows, n_kv_heads, head_dim);
  if (split < n) {
    ensure(k16_, k16_bytes_, size_t(halves) * 2);
    ensure(vt16_, vt16_bytes_, size_t(halves) * 2);
    const int64_t words = nbhs_prefill_aux_words(n - split, n_heads, n_kv_heads);
    if (words < 0) throw Error("attention: invalid prefill shape");
    ensure_aux(size_t(words) * sizeof(uint32_t));
  }
  if (app) {
    if (split < n)
      check(nbhs_append_stage_kv_f16(const_cast<float*>(k), const_cast<float*>(v), app->k_new, app->v_new, n, pos0,
                                     n_kv_heads, head_dim, rope_table, rope_rows, neox ? 1 : 0, k16_, vt16_, aux_,
                                     int64_t(aux_bytes_ / sizeof(uint32_t)), stream_),
            "attention (append and staging)");
    else
      append_kv();
  } else if (split < n) {
    check(nbhs_stage_kv_f16(k, v, k16_, vt16_, rows, n_kv_heads, head_dim, aux_, int64_t(aux_bytes_ / sizeof(uint32_t)),
                            stream_),
          "attention (staging)");
  }
  if (split == n) {
    decode_rows(q, out, split, pos0);
    return;
  }
  // rows [0, split) in fp32 and the rest on MFMA, in one launch (plus a merge when short chunks split their keys)
  const int64_t rows_pad = (rows + 63) / 64 * 64;
  const int64_t ws = nbhs_attn_prefill_workspace(n, pos0, n_heads, n_kv_heads, head_dim, split, cu_count_);
  if (ws < 0) throw Error("attention: invalid prefill shape");
  ensure(decode_ws_, decode_ws_bytes_, size_t(ws) * sizeof(float));
  check(nbhs_attn_prefill_mfma(q, k16_, vt16_, out, n, pos0, n_heads, n_kv_heads, head_dim, rows_pad, rope_table,
                               rope_rows, neox ? 1 : 0, k, v, split, decode_ws_,
                               int64_t(decode_ws_bytes_ / sizeof(float)), aux_,
                               int64_t(aux_bytes_ / sizeof(uint32_t)), cu_count_, stream_),
        "attention (prefill kernel)");
}

}  // namespace nibble::hip
