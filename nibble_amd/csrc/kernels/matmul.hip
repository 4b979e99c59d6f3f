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
//  * Longer calls (prefill chunks) are GEMMs. F16 weights take the split-activation MFMA GEMM of kernels/gemm.hip;
//    F32 weights, and F16 ones whose width is not a multiple of 8, go to rocBLAS sgemm (on an fp32 copy of an F16
//    weight, which widens exactly), so products and sums stay fp32.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include "backend/hip/kernel_timing.h"
#include "nibble_hip_shim.h"

namespace {

constexpr int kGemvMaxRows = NBHS_GEMV_MAX_ROWS;  // activation rows one gemv launch serves
constexpr int kGemvMaxWeights = NBHS_GEMV_MAX_WEIGHTS;
constexpr int kRowsPerWave = 4;  // weight rows one wave streams together (x chunks are read once for all four)

struct GemvWeight {
  const void* w;  // [rows, in], F32 or F16
  float* y;       // [n, rows]
  int64_t rows;
  int64_t wave0;  // first wave (block) of this weight
  int f16;
};
struct GemvBatch {
  GemvWeight w[kGemvMaxWeights];
  int n_w;
};

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

// Eight consecutive weights of a row as loaded: 16 bytes of halves or 32 bytes of floats.
template <bool F16>
struct Chunk;
template <>
struct Chunk<true> {
  half8 h;
  __device__ __forceinline__ void load(const void* row, int64_t k) {
    h = *reinterpret_cast<const half8*>(static_cast<const _Float16*>(row) + k);
  }
  __device__ __forceinline__ float operator[](int e) const { return float(h[e]); }
};
template <>
struct Chunk<false> {
  float4 a, b;
  __device__ __forceinline__ void load(const void* row, int64_t k) {
    a = *reinterpret_cast<const float4*>(static_cast<const float*>(row) + k);
    b = *reinterpret_cast<const float4*>(static_cast<const float*>(row) + k + 4);
  }
  __device__ __forceinline__ float operator[](int e) const {
    return e < 4 ? (e == 0 ? a.x : e == 1 ? a.y : e == 2 ? a.z : a.w) : (e == 4 ? b.x : e == 5 ? b.y : e == 6 ? b.z : b.w);
  }
};

// Sum of each of CNT values over the 64 lanes of the wave, halving the values held per lane at each butterfly step
// (a lane keeps the half its partner does not), so CNT - 1 + log2(64 / CNT) exchanges instead of 6 * CNT. Lane L
// ends with the full sum of value L >> (6 - log2 CNT) in v[0].
template <int CNT, int MASK, int M>
__device__ __forceinline__ void wave_reduce_scatter(float (&v)[M], int lane) {
  if constexpr (MASK >= 1) {
    if constexpr (CNT > 1) {
      constexpr int h = CNT / 2;
      const bool up = (lane & MASK) != 0;
#pragma unroll
      for (int j = 0; j < h; ++j) {
        const float send = up ? v[j] : v[j + h];
        const float keep = up ? v[j + h] : v[j];
        v[j] = keep + __shfl_xor(send, MASK, 64);
      }
      wave_reduce_scatter<h, MASK / 2>(v, lane);
    } else {
      v[0] += __shfl_xor(v[0], MASK, 64);
      wave_reduce_scatter<1, MASK / 2>(v, lane);
    }
  }
}

constexpr int ilog2(int v) { return v <= 1 ? 0 : 1 + ilog2(v / 2); }

// One wave: rows r0..r0+3 of one weight against NT (>= n) activation rows. Every chunk the wave needs of its four
// rows is loaded before any arithmetic (64 bytes per lane per row and pass), so a wave keeps 16 KB in flight.
// `vec`: 16-byte loads (in % 8 == 0, weight and x 16-byte aligned, checked on the host); otherwise one element per
// lane per step.
template <bool F16, int NT>
__device__ __forceinline__ void gemv_rows(const GemvWeight& d, const float* __restrict__ x, int64_t in, int n,
                                          bool vec, int64_t r0) {
  constexpr int R = kRowsPerWave;
  const int lane = threadIdx.x;
  const int nr = int(d.rows - r0 < R ? d.rows - r0 : R);
  const void* row[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {  // rows past the weight's end re-read its last row; their sums are dropped
    const int64_t rr = r0 + (r < nr ? r : nr - 1);
    row[r] = F16 ? static_cast<const void*>(static_cast<const _Float16*>(d.w) + rr * in)
                 : static_cast<const void*>(static_cast<const float*>(d.w) + rr * in);
  }
  float acc[R * NT];
#pragma unroll
  for (int j = 0; j < R * NT; ++j) acc[j] = 0.f;
  if (vec) {
    constexpr int U = F16 ? 4 : 2;  // chunks per lane per pass: 64 bytes of each row
    for (int64_t k0 = int64_t(lane) * 8; k0 < in; k0 += 64 * 8 * U) {
      Chunk<F16> w[R][U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t k = k0 + u * 512;
        if (k < in) {
#pragma unroll
          for (int r = 0; r < R; ++r) w[r][u].load(row[r], k);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t k = k0 + u * 512;
        if (k < in) {
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            if (t < n) {
              const float4 xa = *reinterpret_cast<const float4*>(x + t * in + k);
              const float4 xb = *reinterpret_cast<const float4*>(x + t * in + k + 4);
#pragma unroll
              for (int r = 0; r < R; ++r)
                acc[r * NT + t] += xa.x * w[r][u][0] + xa.y * w[r][u][1] + xa.z * w[r][u][2] + xa.w * w[r][u][3] +
                                   xb.x * w[r][u][4] + xb.y * w[r][u][5] + xb.z * w[r][u][6] + xb.w * w[r][u][7];
            }
          }
        }
      }
    }
  } else {
    for (int64_t k = lane; k < in; k += 64) {
      float w[R];
#pragma unroll
      for (int r = 0; r < R; ++r)
        w[r] = F16 ? float(static_cast<const _Float16*>(row[r])[k]) : static_cast<const float*>(row[r])[k];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (t < n) {
          const float xv = x[t * in + k];
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r * NT + t] += xv * w[r];
        }
      }
    }
  }
  constexpr int M = R * NT;
  static_assert(M <= 64 && (M & (M - 1)) == 0, "R * NT must be a power of two up to 64");
  wave_reduce_scatter<M, 32>(acc, lane);
  constexpr int shift = 6 - ilog2(M);
  if ((lane & ((1 << shift) - 1)) == 0) {
    const int idx = lane >> shift, r = idx / NT, t = idx % NT;
    if (r < nr && t < n) d.y[int64_t(t) * d.rows + r0 + r] = acc[0];
  }
}

// One 64-thread block (one wave) per four stacked weight rows.
template <int NT>
__global__ __launch_bounds__(64) void gemv_kernel(GemvBatch b, const float* __restrict__ x, int64_t in, int n,
                                                  bool vec) {
  int i = 0;
  for (int j = 1; j < b.n_w; ++j)
    if (int64_t(blockIdx.x) >= b.w[j].wave0) i = j;
  const GemvWeight& d = b.w[i];
  const int64_t r0 = (int64_t(blockIdx.x) - d.wave0) * kRowsPerWave;
  if (d.f16)
    gemv_rows<true, NT>(d, x, in, n, vec, r0);
  else
    gemv_rows<false, NT>(d, x, in, n, vec, r0);
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
  int64_t waves = 0;
  bool vec = in % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
  for (int i = 0; i < n_w; ++i) {
    if (!w[i] || !y[i] || rows[i] <= 0) return NBHS_EINVAL;
    vec = vec && reinterpret_cast<uintptr_t>(w[i]) % 16 == 0;
    b.w[i] = GemvWeight{w[i], y[i], rows[i], waves, f16[i] ? 1 : 0};
    waves += (rows[i] + kRowsPerWave - 1) / kRowsPerWave;
  }
  b.n_w = n_w;
  if (waves >= (int64_t(1) << 31)) return NBHS_EINVAL;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid{unsigned(waves), 1, 1}, block{64, 1, 1};
  if (n == 1) return nbhs_timing::launch(NBHS_K_GEMV, gemv_kernel<1>, grid, block, s, b, x, in, int(n), vec);
  if (n <= 4) return nbhs_timing::launch(NBHS_K_GEMV, gemv_kernel<4>, grid, block, s, b, x, in, int(n), vec);
  return nbhs_timing::launch(NBHS_K_GEMV, gemv_kernel<16>, grid, block, s, b, x, in, int(n), vec);
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
