// The rest of the Backend's per-token ops on the GPU, so that a whole forward (transformer.cpp:166-230) can stay in
// HBM: embed, rmsnorm, add and silu_mul (backend.h:55-70), with the semantics of ref_ops.cpp.
//  * embed (ref_ops.cpp:80-99): row copy for F32 tables, exact widening for F16; bit-exact.
//  * rmsnorm (ref_ops.cpp:137-148): sum of squares in double (float * float is exact in double, so only the order
//    of the sum differs from the reference), scale = 1 / sqrt(ss / d + eps) in double, y = float(x * scale * w)
//    with the reference's two double products in its order. The file is compiled with -ffp-contract=off, so no
//    multiply-add is fused (the reference's ref_ops.cpp is built the same way).
//  * add (ref_ops.cpp:151-153): one float add per element; bit-exact.
//  * silu_mul (ref_ops.cpp:217-222): gate = g / (1 + exp(-g)) * up in float; exp is the device library's expf,
//    so results match the reference within a few ulp (the reference's own SIMD tier uses its own exp too).
// All four are HBM-bound streams.
#include <hip/hip_runtime.h>

#include "backend/hip/kernel_timing.h"
#include "nibble_hip_shim.h"

namespace {

constexpr int kThreads = 256;

unsigned grid_for(int64_t count) {
  const int64_t blocks = (count + kThreads - 1) / kThreads;
  return unsigned(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192);
}

// out[t, :] = row ids[t] of the table, widened to float. One workgroup per output row.
template <bool F16>
__global__ __launch_bounds__(kThreads) void embed_kernel(const void* __restrict__ table, const int32_t* __restrict__ ids,
                                                         float* __restrict__ out, int64_t d) {
  const int64_t t = blockIdx.x;
  const int64_t id = ids[t];
  float* o = out + t * d;
  if constexpr (F16) {
    const _Float16* r = static_cast<const _Float16*>(table) + id * d;
    for (int64_t k = threadIdx.x; k < d; k += kThreads) o[k] = float(r[k]);
  } else {
    const float* r = static_cast<const float*>(table) + id * d;
    for (int64_t k = threadIdx.x; k < d; k += kThreads) o[k] = r[k];
  }
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// One workgroup per row of d elements.
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           float* __restrict__ y, int64_t d, float eps) {
  __shared__ double part[kThreads / 64];
  __shared__ double scale_sh;
  const int64_t t = blockIdx.x;
  const float* xt = x + t * d;
  double ss = 0.0;
  for (int64_t i = threadIdx.x; i < d; i += kThreads) {
    const double v = double(xt[i]);
    ss = __dadd_rn(ss, __dmul_rn(v, v));
  }
  ss = wave_sum_f64(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int i = 0; i < kThreads / 64; ++i) s = __dadd_rn(s, part[i]);
    scale_sh = __ddiv_rn(1.0, __dsqrt_rn(__dadd_rn(__ddiv_rn(s, double(d)), double(eps))));
  }
  __syncthreads();
  const double scale = scale_sh;
  float* yt = y + t * d;
  for (int64_t i = threadIdx.x; i < d; i += kThreads) yt[i] = float(__dmul_rn(__dmul_rn(double(xt[i]), scale), double(w[i])));
}

__global__ __launch_bounds__(kThreads) void add_kernel(float* __restrict__ x, const float* __restrict__ y,
                                                       int64_t count) {
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < count; i += int64_t(gridDim.x) * kThreads)
    x[i] = __fadd_rn(x[i], y[i]);
}

__global__ __launch_bounds__(kThreads) void silu_mul_kernel(float* __restrict__ gate, const float* __restrict__ up,
                                                            int64_t count) {
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < count; i += int64_t(gridDim.x) * kThreads) {
    const float g = gate[i];
    gate[i] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), up[i]);
  }
}

}  // namespace

extern "C" {

int nbhs_embed(int f16, const void* table, const int32_t* ids, int64_t n, int64_t d, float* out, nbhs_stream s) {
  if (!table || !ids || !out || n <= 0 || d <= 0 || n >= (int64_t(1) << 31)) return NBHS_EINVAL;
  const hipStream_t st = reinterpret_cast<hipStream_t>(s);
  if (f16)
    return nbhs_timing::launch(NBHS_K_ELEMENTWISE, embed_kernel<true>, dim3(unsigned(n)), dim3(kThreads), st, table,
                               ids, out, d);
  return nbhs_timing::launch(NBHS_K_ELEMENTWISE, embed_kernel<false>, dim3(unsigned(n)), dim3(kThreads), st, table,
                             ids, out, d);
}

int nbhs_rmsnorm_f32(const float* x, const float* w, float* y, int64_t n, int64_t d, float eps, nbhs_stream s) {
  if (!x || !w || !y || n <= 0 || d <= 0 || n >= (int64_t(1) << 31)) return NBHS_EINVAL;
  return nbhs_timing::launch(NBHS_K_RMSNORM, rmsnorm_kernel, dim3(unsigned(n)), dim3(kThreads),
                             reinterpret_cast<hipStream_t>(s), x, w, y, d, eps);
}

int nbhs_add_f32(float* x, const float* y, int64_t count, nbhs_stream s) {
  if (!x || !y || count <= 0) return NBHS_EINVAL;
  return nbhs_timing::launch(NBHS_K_ELEMENTWISE, add_kernel, dim3(grid_for(count)), dim3(kThreads),
                             reinterpret_cast<hipStream_t>(s), x, y, count);
}

int nbhs_silu_mul_f32(float* gate, const float* up, int64_t count, nbhs_stream s) {
  if (!gate || !up || count <= 0) return NBHS_EINVAL;
  return nbhs_timing::launch(NBHS_K_ELEMENTWISE, silu_mul_kernel, dim3(grid_for(count)), dim3(kThreads),
                             reinterpret_cast<hipStream_t>(s), gate, up, count);
}

}  // extern "C"
