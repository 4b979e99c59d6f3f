// Float-weight projections on the GPU: Backend::matmul / matmul_multi (backend.h:56-60) for F32 and F16 weights
// with the semantics of ref_ops.cpp:109-135 (y[t, r] = sum_k x[t, k] w[r, k], fp32 accumulation; the order differs
// from the reference's left-to-right one, so results agree within float rounding), and Backend::add_bias
// (backend.h:62, ref_ops.cpp:154-160, bit-exact: one add per element).
//
// This is the Transformer's QKV projection (transformer.cpp:171-194): matmul_multi writes q and the new K/V rows
// straight into their cache rows, so the KV append of the attention path starts on the device.
//  * Decode and short appends (n <= 16 rows) are HBM-bound on the weights: gemv_kernel streams every weight row once
//    (one wave per output row, 16-byte loads, f16 weights read as f16) and keeps up to 16 rows' dot products in
//    registers; all the weights of a matmul_multi share one launch over their stacked output rows.
//  * Longer calls (prefill chunks) are plain GEMMs and go to rocBLAS sgemm on an fp32 copy of the weight (an f16
//    weight widens exactly), so products and sums stay fp32.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include "backend/hip/kernel_timing.h"
#include "nibble_hip_shim.h"

namespace {

constexpr int kGemvMaxRows = NBHS_GEMV_MAX_ROWS;  // activation rows one gemv launch serves
constexpr int kGemvMaxWeights = NBHS_GEMV_MAX_WEIGHTS;

struct GemvWeight {
  const void* w;  // [rows, in], F32 or F16
  float* y;       // [n, rows]
  int64_t rows;
  int64_t row0;   // first stacked row of this weight
  int f16;
};
struct GemvBatch {
  GemvWeight w[kGemvMaxWeights];
  int n_w;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// 8 weights from element k of a row, as floats.
template <bool F16>
__device__ __forceinline__ void load8(const void* row, int64_t k, float (&w)[8]) {
  if constexpr (F16) {
    typedef _Float16 half8 __attribute__((ext_vector_type(8)));
    const half8 h = *reinterpret_cast<const half8*>(static_cast<const _Float16*>(row) + k);
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = float(h[e]);
  } else {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(row) + k);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(row) + k + 4);
    w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = b.x, w[5] = b.y, w[6] = b.z, w[7] = b.w;
  }
}

template <bool F16>
__device__ __forceinline__ float load1(const void* row, int64_t k) {
  if constexpr (F16)
    return float(static_cast<const _Float16*>(row)[k]);
  else
    return static_cast<const float*>(row)[k];
}

// One wave per stacked output row; lanes take 8-element chunks of the row (16-byte loads when `vec`: in % 8 == 0
// and every weight and x 16-byte aligned, checked on the host).
template <bool F16>
__device__ __forceinline__ void gemv_row(const void* wrow, const float* __restrict__ x, int64_t in, int n, bool vec,
                                         float (&acc)[kGemvMaxRows]) {
  const int lane = threadIdx.x & 63;
  if (vec) {
    for (int64_t k = int64_t(lane) * 8; k < in; k += 64 * 8) {
      float w[8];
      load8<F16>(wrow, k, w);
#pragma unroll
      for (int t = 0; t < kGemvMaxRows; ++t) {
        if (t < n) {
          const float4 a = *reinterpret_cast<const float4*>(x + t * in + k);
          const float4 b = *reinterpret_cast<const float4*>(x + t * in + k + 4);
          acc[t] += a.x * w[0] + a.y * w[1] + a.z * w[2] + a.w * w[3] + b.x * w[4] + b.y * w[5] + b.z * w[6] +
                    b.w * w[7];
        }
      }
    }
  } else {
    for (int64_t k = lane; k < in; k += 64) {
      const float w = load1<F16>(wrow, k);
#pragma unroll
      for (int t = 0; t < kGemvMaxRows; ++t)
        if (t < n) acc[t] += x[t * in + k] * w;
    }
  }
}

__global__ __launch_bounds__(256) void gemv_kernel(GemvBatch b, const float* __restrict__ x, int64_t in, int n,
                                                   bool vec) {
  const int64_t r = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);  // stacked output row of this wave
  int i = 0;
  for (int j = 1; j < b.n_w; ++j)
    if (r >= b.w[j].row0) i = j;
  const GemvWeight& d = b.w[i];
  const int64_t rr = r - d.row0;
  if (rr >= d.rows) return;  // past the last weight's rows: the whole wave leaves
  float acc[kGemvMaxRows];
#pragma unroll
  for (int t = 0; t < kGemvMaxRows; ++t) acc[t] = 0.f;
  if (d.f16)
    gemv_row<true>(static_cast<const _Float16*>(d.w) + rr * in, x, in, n, vec, acc);
  else
    gemv_row<false>(static_cast<const float*>(d.w) + rr * in, x, in, n, vec, acc);
#pragma unroll
  for (int t = 0; t < kGemvMaxRows; ++t) {
    if (t < n) {
      const float s = wave_sum(acc[t]);
      if ((threadIdx.x & 63) == 0) d.y[t * d.rows + rr] = s;
    }
  }
}

__global__ __launch_bounds__(256) void f16_to_f32_kernel(const _Float16* __restrict__ src, float* __restrict__ dst,
                                                         int64_t count) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < count; i += int64_t(gridDim.x) * 256)
    dst[i] = float(src[i]);
}

__global__ __launch_bounds__(256) void add_bias_kernel(float* __restrict__ x, const float* __restrict__ b, int64_t d,
                                                       int64_t count) {
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < count; i += int64_t(gridDim.x) * 256)
    x[i] += b[i % d];
}

unsigned grid_for(int64_t count) {
  const int64_t blocks = (count + 255) / 256;
  return unsigned(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096);
}

}  // namespace

extern "C" {

int nbhs_gemv_multi(int n_w, const int* f16, const void* const* w, float* const* y, const int64_t* rows, int64_t in,
                    const float* x, int64_t n, nbhs_stream stream) {
  if (n_w <= 0 || n_w > kGemvMaxWeights || !f16 || !w || !y || !rows || in <= 0 || !x || n <= 0 ||
      n > kGemvMaxRows)
    return NBHS_EINVAL;
  GemvBatch b{};
  int64_t total = 0;
  bool vec = in % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
  for (int i = 0; i < n_w; ++i) {
    if (!w[i] || !y[i] || rows[i] <= 0) return NBHS_EINVAL;
    vec = vec && reinterpret_cast<uintptr_t>(w[i]) % 16 == 0;
    b.w[i] = GemvWeight{w[i], y[i], rows[i], total, f16[i] ? 1 : 0};
    total += rows[i];
  }
  b.n_w = n_w;
  const int64_t blocks = (total + 3) / 4;
  if (blocks >= (int64_t(1) << 31)) return NBHS_EINVAL;
  return nbhs_timing::launch(NBHS_K_GEMV, gemv_kernel, dim3(unsigned(blocks)), dim3(256),
                             reinterpret_cast<hipStream_t>(stream), b, x, in, int(n), vec);
}

int nbhs_f16_to_f32(const void* src, float* dst, int64_t count, nbhs_stream stream) {
  if (!src || !dst || count < 0) return NBHS_EINVAL;
  if (count == 0) return hipSuccess;
  return nbhs_timing::launch(NBHS_K_CONVERT, f16_to_f32_kernel, dim3(grid_for(count)), dim3(256),
                             reinterpret_cast<hipStream_t>(stream), static_cast<const _Float16*>(src), dst, count);
}

int nbhs_add_bias_f32(float* x, const float* bias, int64_t d, int64_t n, nbhs_stream stream) {
  if (!x || !bias || d <= 0 || n <= 0) return NBHS_EINVAL;
  return nbhs_timing::launch(NBHS_K_ADD_BIAS, add_bias_kernel, dim3(grid_for(d * n)), dim3(256),
                             reinterpret_cast<hipStream_t>(stream), x, bias, d, d * n);
}

int nbhs_blas_create(nbhs_blas* out, nbhs_stream stream) {
  if (!out) return NBHS_EINVAL;
  rocblas_handle h = nullptr;
  if (rocblas_create_handle(&h) != rocblas_status_success) return NBHS_EBLAS;
  if (rocblas_set_stream(h, reinterpret_cast<hipStream_t>(stream)) != rocblas_status_success) {
    rocblas_destroy_handle(h);
    return NBHS_EBLAS;
  }
  *out = reinterpret_cast<nbhs_blas>(h);
  return hipSuccess;
}

int nbhs_blas_destroy(nbhs_blas h) {
  if (h) rocblas_destroy_handle(reinterpret_cast<rocblas_handle>(h));
  return hipSuccess;
}

int nbhs_sgemm_xwt(nbhs_blas h, const float* x, const float* w, float* y, int64_t n, int64_t in, int64_t out) {
  if (!h || !x || !w || !y || n <= 0 || in <= 0 || out <= 0 || n > INT32_MAX || in > INT32_MAX || out > INT32_MAX)
    return NBHS_EINVAL;
  // Row-major y[n, out] = x[n, in] . w[out, in]^T is, column-major, y^T (out x n) = w^T^T (out x in) . x^T (in x n):
  // A = w viewed (in x out) transposed, B = x viewed (in x n), both with leading dimension in.
  const float one = 1.0f, zero = 0.0f;
  const rocblas_status st =
      rocblas_sgemm(reinterpret_cast<rocblas_handle>(h), rocblas_operation_transpose, rocblas_operation_none,
                    rocblas_int(out), rocblas_int(n), rocblas_int(in), &one, w, rocblas_int(in), x, rocblas_int(in),
                    &zero, y, rocblas_int(out));
  return st == rocblas_status_success ? hipSuccess : NBHS_EBLAS;
}

}  // extern "C"
