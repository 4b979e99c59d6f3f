// C entry points over the compiled reference CPU backend. TEST INFRASTRUCTURE ONLY: the real nibble sources are
// compiled where they lie under the reference tree (oracle/Makefile, target `ref`) into oracle/_ref/, and this
// file (our own code) exposes them to ctypes so tests can pin the C restatement against the reference itself and
// bench.py can time the reference's CPU attention as its baseline. Nothing of the reference is copied here.
#include <cstdint>
#include <exception>
#include <limits>
#include <new>
#include <span>

#include "backend/cpu/cpu_backend.h"
#include "backend/cpu/ref_ops.h"
#include "backend/cpu/simd/dispatch.h"
#include "quant.h"
#include "thread_pool.h"

namespace {
struct RefBackend {
  nibble::ThreadPool pool;
  nibble::cpu::CpuBackend be;
  explicit RefBackend(int threads) : pool(threads), be(pool) {}
};
}  // namespace

extern "C" {

// nibble::cpu::rope (ref_ops.cpp:166-185).
int ref_rope(float* x, int64_t n, int64_t n_heads, int64_t head_dim, int64_t pos0, float base, int neox,
             const float* freq_factors) {
  nibble::RopeParams p{base, neox != 0, freq_factors};
  nibble::cpu::rope(x, n, n_heads, head_dim, pos0, p);
  return 0;
}

// nibble::cpu::attention_heads (ref_ops.cpp:188-214).
int ref_attention_scalar(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                         int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t head_begin, int64_t head_end,
                         float* scratch) {
  nibble::cpu::attention_heads(q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim, head_begin, head_end, scratch);
  return 0;
}

// The selected SIMD tier's attention_heads (simd/ops.cpp:104-139 on AVX2 hosts); -1 when no tier is available.
int ref_attention_simd(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                       int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t head_begin, int64_t head_end,
                       float* scratch) {
  try {
    const nibble::simd::Kernels* ks = nibble::simd::select();
    if (!ks) return -1;
    ks->attention_heads(q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim, head_begin, head_end, scratch);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// "scalar", "avx2+fma+f16c", ...: the tier CpuBackend runs on this host (dispatch.cpp:150-153).
const char* ref_kernel_set() {
  try {
    return nibble::simd::kernel_set();
  } catch (const std::exception&) {
    return "error";
  }
}

namespace {
nibble::Tensor weight(int type, const void* w, int64_t in, int64_t out) {
  nibble::Tensor t;
  t.type = static_cast<nibble::DType>(type);  // ggml type id: 0 F32, 1 F16, 2 Q4_0, ... 14 Q6_K
  t.n_dims = 2;
  t.ne = {in, out, 1, 1};
  t.data = w;
  return t;
}
}  // namespace

// nibble::cpu::matmul_rows (ref_ops.cpp:109-135), all output rows, float weights (type 0 F32, 1 F16).
int ref_matmul_scalar(int type, const void* w, int64_t in, int64_t out, const float* x, float* y, int64_t n) {
  try {
    nibble::cpu::matmul_rows(weight(type, w, in, out), x, y, n, 0, out, nullptr);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// nibble::cpu::add_bias (ref_ops.cpp:154-160); the bias is an F32 vector of d floats.
int ref_add_bias(float* x, const float* b, int64_t d, int64_t n) {
  nibble::Tensor t;
  t.type = nibble::DType::F32;
  t.n_dims = 1;
  t.ne = {d, 1, 1, 1};
  t.data = b;
  nibble::cpu::add_bias(x, t, n);
  return 0;
}

namespace {
nibble::Tensor vec_f32(const float* v, int64_t d) {
  nibble::Tensor t;
  t.type = nibble::DType::F32;
  t.n_dims = 1;
  t.ne = {d, 1, 1, 1};
  t.data = v;
  return t;
}
}  // namespace

// nibble::cpu::embed (ref_ops.cpp:80-99) for F32 (type 0) and F16 (type 1) tables [rows, d]; -1 on a bad id.
int ref_embed(int type, const void* table, int64_t rows, int64_t d, const int32_t* ids, int64_t n, float* out) {
  try {
    nibble::cpu::embed(weight(type, table, d, rows), std::span<const int32_t>(ids, size_t(n)), out);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// nibble::cpu::rmsnorm (ref_ops.cpp:137-148), the scalar path.
int ref_rmsnorm(const float* x, const float* w, float* y, int64_t n, int64_t d, float eps) {
  nibble::cpu::rmsnorm(x, vec_f32(w, d), y, n, eps);
  return 0;
}

// nibble::cpu::add (ref_ops.cpp:151-153) and cpu::silu_mul (:217-222), the scalar paths.
int ref_add(float* x, const float* y, int64_t count) {
  nibble::cpu::add(x, y, count);
  return 0;
}
int ref_silu_mul(float* gate, const float* up, int64_t count) {
  nibble::cpu::silu_mul(gate, up, count);
  return 0;
}

// The selected SIMD tier's rmsnorm / silu_mul (simd/ops.cpp:64-100): -1 when no tier is available.
int ref_rmsnorm_simd(const float* x, const float* w, float* y, int64_t n, int64_t d, float eps) {
  const nibble::simd::Kernels* ks = nibble::simd::select();
  if (!ks) return -1;
  ks->rmsnorm(x, vec_f32(w, d), y, n, eps);
  return 0;
}
int ref_silu_mul_simd(float* gate, const float* up, int64_t count) {
  const nibble::simd::Kernels* ks = nibble::simd::select();
  if (!ks) return -1;
  ks->silu_mul(gate, up, count);
  return 0;
}

// src/quant.cpp: the activation quantizers (quant.h:120-133), dequantize_row (:117) and the block dots
// (:137-160), as the reference compiles them.
int ref_quantize(int kind, const float* x, void* y, int64_t n) {
  try {
    if (kind == 0) nibble::quantize_row_q8_0(x, static_cast<nibble::BlockQ8_0*>(y), n);
    else if (kind == 1) nibble::quantize_row_q8_1(x, static_cast<nibble::BlockQ8_1*>(y), n);
    else nibble::quantize_row_q8_K(x, static_cast<nibble::BlockQ8_K*>(y), n);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}
int ref_dequantize(int type, const void* src, float* dst, int64_t n) {
  try {
    nibble::dequantize_row(static_cast<nibble::DType>(type), src, dst, n);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}
float ref_dot(int type, const void* w, const void* a, int64_t nb) {
  using namespace nibble;
  switch (static_cast<DType>(type)) {
    case DType::Q4_0: return dot_q4_0_q8_0(static_cast<const BlockQ4_0*>(w), static_cast<const BlockQ8_0*>(a), nb);
    case DType::Q8_0: return dot_q8_0_q8_0(static_cast<const BlockQ8_0*>(w), static_cast<const BlockQ8_0*>(a), nb);
    case DType::Q5_0: return dot_q5_0_q8_0(static_cast<const BlockQ5_0*>(w), static_cast<const BlockQ8_0*>(a), nb);
    case DType::Q5_1: return dot_q5_1_q8_1(static_cast<const BlockQ5_1*>(w), static_cast<const BlockQ8_1*>(a), nb);
    case DType::Q4_K: return dot_q4_K_q8_K(static_cast<const BlockQ4_K*>(w), static_cast<const BlockQ8_K*>(a), nb);
    case DType::Q5_K: return dot_q5_K_q8_K(static_cast<const BlockQ5_K*>(w), static_cast<const BlockQ8_K*>(a), nb);
    case DType::Q6_K: return dot_q6_K_q8_K(static_cast<const BlockQ6_K*>(w), static_cast<const BlockQ8_K*>(a), nb);
    default: return std::numeric_limits<float>::quiet_NaN();
  }
}

// A ThreadPool of `threads` threads and a CpuBackend on it (nibble.cpp:75-85 builds the same pair).
void* ref_backend_create(int threads) {
  try {
    return new RefBackend(threads);
  } catch (const std::exception&) {
    return nullptr;
  }
}

void ref_backend_destroy(void* h) { delete static_cast<RefBackend*>(h); }

// CpuBackend::reserve (cpu_backend.cpp:24-67).
int ref_backend_reserve(void* h, int64_t n_ctx, int64_t n_heads, int64_t max_rows, int64_t max_width) {
  try {
    static_cast<RefBackend*>(h)->be.reserve({n_ctx, n_heads, max_rows, max_width});
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// CpuBackend::attention (cpu_backend.cpp:271-290): parallel_for over heads, chunk 1.
int ref_backend_attention(void* h, const float* q, const float* k, const float* v, float* out, int64_t n,
                          int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim) {
  try {
    static_cast<RefBackend*>(h)->be.attention(q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// CpuBackend::rope (cpu_backend.cpp:253-259): scalar, on the calling thread.
int ref_backend_rope(void* h, float* x, int64_t n, int64_t n_heads, int64_t head_dim, int64_t pos0, float base,
                     int neox, const float* freq_factors) {
  try {
    static_cast<RefBackend*>(h)->be.rope(x, n, n_heads, head_dim, pos0, {base, neox != 0, freq_factors});
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// CpuBackend::matmul (cpu_backend.cpp:134-138 -> matmul_multi :146-248): the production tier (AVX2 gemm_f /
// matmul_rows_f on this host) over the pool.
int ref_backend_matmul(void* h, int type, const void* w, int64_t in, int64_t out, const float* x, float* y,
                       int64_t n) {
  try {
    static_cast<RefBackend*>(h)->be.matmul(weight(type, w, in, out), x, y, n);
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

}  // extern "C"
