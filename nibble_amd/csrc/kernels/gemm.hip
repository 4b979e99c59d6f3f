// F16-weight GEMM for prefill-sized projections: Backend::matmul / matmul_multi (backend.h:56-60) with n > 16
// activation rows and F16 weights, y[t, r] = sum_k x[t, k] w[r, k] (ref_ops.cpp:109-135) in fp32-grade arithmetic
// on the fp16 MFMA pipes.
//
// The weights are exact in fp16. The fp32 activations are not, so each activation row t is scaled by a power of two
// s_t (exact) that brings its largest element into [2^13, 2^14), and split into two fp16 parts, hi = fp16(x s_t)
// and lo = fp16(x s_t - hi): x s_t = hi + lo + r with |r| <= 2^-22 |x s_t| (2^-25 absolute where lo is an fp16
// subnormal, i.e. for elements below 2^-17 of the row's largest). fp16 x fp16 products are exact in fp32, and
// v_mfma_f32_32x32x16_f16 accumulates in fp32, so y = (sum_k lo_k w_k + hi_k w_k) / s_t carries an error of the
// order of an fp32 GEMM's (the classical bound in * 2^-24 * sum_k |x_k w_k| holds with a wide margin) at two fp16
// MFMAs per product instead of fp32 arithmetic - and without an fp32 copy of the weights.
//
//  * split_acts_kernel: one wave per activation row: the row's largest magnitude, then hi and lo written as fp16
//    rows padded with zeros to a multiple of the K slice (16-byte stores), and 1 / s_t.
//  * gemm_f16w_kernel: output tiles of 64 x 64 (64-deep K slices) or, for grids with many tiles, 128 x 128 (32-deep
//    slices), four waves each on a quarter, K slices through a 3-stage LDS ring filled by direct-to-LDS buffer loads
//    (rows past the activation count or a weight's row count, and columns past `in`, read as zeros). Per 16-deep
//    step a wave reads its hi, lo and weight fragments once and issues the lo then the hi MFMA into each
//    accumulator. Up to kMaxWeights weights sharing x run in one launch over their stacked tiles.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "backend/hip/kernel_timing.h"
#include "nibble_hip_shim.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kMaxWeights = NBHS_GEMM_MAX_WEIGHTS;
constexpr int kThreads = 256;

struct GemmWeight {
  const _Float16* w;  // [rows, in]
  float* y;           // [n, rows]
  int64_t rows;
  int tile0;          // first workgroup (blockIdx.x) of this weight
  int split;          // K ranges (1: the whole K; > 1: partial sums into part, merged by gemm_split_reduce_kernel)
  float* part;        // [split][n][rows] partial sums when split > 1
};
struct GemmBatch {
  GemmWeight w[kMaxWeights];
  int n_w;
};

// LDS position of 16-byte chunk x of tile row r (CPR chunks per row): chunks are permuted per row so that the 16
// lanes a ds_read_b128 serves per cycle (16 consecutive rows, one chunk) cover all 64 banks.
template <int CPR>
__device__ __forceinline__ int swz(int r) {
  if constexpr (CPR == 8) return (r ^ (r >> 3)) & 7;
  return (r >> 2) & 3;
}

constexpr int vmcnt_wait(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, void* lds_wave_base, uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds_wave_base, 16, voff, 0, 0, 0);
#endif
}

// (hi, lo) of x: the value is pinned to its fp32 rounding first, so that the compiler cannot fuse a producing
// multiply into hi's conversion while lo subtracts a differently rounded hi.
__device__ __forceinline__ void split_f16(float x, _Float16& hi, _Float16& lo) {
  asm("" : "+v"(x));
  hi = (_Float16)x;
  const float h = (float)hi;
  lo = __builtin_isfinite(h) ? (_Float16)(x - h) : (_Float16)0.f;  // an infinite or NaN hi carries the value alone
}

// One wave per activation row, each lane on runs of 8 consecutive elements: the row's largest magnitude (a wave
// reduction), then the hi and lo rows in 16-byte stores. Runs past `in` (up to in_pad) are written as zeros.
// in % 8 == 0; `vec`: x is 16-byte aligned, so a run is two 16-byte loads. Up to kHeld runs per lane stay in
// registers between the two passes (rows up to 4096 wide); longer rows read the rest again.
constexpr int kHeld = 8;
__global__ __launch_bounds__(64) void split_acts_kernel(const float* __restrict__ x, int64_t in, int64_t in_pad,
                                                        _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                        float* __restrict__ inv_scale, int vec) {
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x;
  const float* xr = x + t * in;
  auto load_run = [&](int64_t k, float (&v)[8]) {
    if (k >= in) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.f;
    } else if (vec) {
      const float4 a = *reinterpret_cast<const float4*>(xr + k), b = *reinterpret_cast<const float4*>(xr + k + 4);
      v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = xr[k + e];
    }
  };
  const int64_t runs = in_pad / 8;
  float held[kHeld][8];
  float m = 0.f;
#pragma unroll
  for (int c = 0; c < kHeld; ++c) {
    load_run(8 * (lane + int64_t(c) * 64), held[c]);  // runs past in read as zeros
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(held[c][e]));  // NaN elements are skipped
  }
  for (int64_t j = lane + kHeld * 64; j < runs; j += 64) {
    float v[8];
    load_run(8 * j, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[e]));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  // s = 2^e with m s in [2^13, 2^14): m in [2^(ex-1), 2^ex) gives e = 14 - ex. A zero or infinite row is not scaled;
  // e is capped so that s and 1 / s stay normal floats (x s is then exact unless it is an fp32 subnormal).
  int e = 0;
  if (m > 0.f && m <= 3.402823466e38f) {
    int ex;
    (void)frexpf(m, &ex);
    e = min(14 - ex, 120);
  }
  const float sc = ldexpf(1.0f, e);
  if (lane == 0) inv_scale[t] = ldexpf(1.0f, -e);
  auto store_run = [&](int64_t j, const float (&v)[8]) {
    half8_t h, l;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      _Float16 hi, lo;
      split_f16(v[q] * sc, hi, lo);
      h[q] = hi;
      l[q] = lo;
    }
    *reinterpret_cast<half8_t*>(xh + t * in_pad + 8 * j) = h;
    *reinterpret_cast<half8_t*>(xl + t * in_pad + 8 * j) = l;
  };
#pragma unroll
  for (int c = 0; c < kHeld; ++c) {
    const int64_t j = lane + int64_t(c) * 64;
    if (j < runs) store_run(j, held[c]);
  }
  for (int64_t j = lane + kHeld * 64; j < runs; j += 64) {
    float v[8];
    load_run(8 * j, v);
    store_run(j, v);
  }
}

// Tile configuration: BM activation rows x BN weight rows per tile (each of the four waves takes BM/2 x BN/2),
// BK-deep K slices, a STAGES-deep LDS ring. Two instances, chosen per weight: 128 x 128 tiles with 32-deep slices for
// a weight that alone makes at least kWideMinTiles of them (an FFN gate or up projection at 512 rows: each operand
// byte fetched from L2 serves twice the products), 64 x 64 tiles with 64-deep slices otherwise (a 512-row QKV or
// FFN-down projection: more workgroups to spread the operand traffic). Both keep 72 KB of LDS per workgroup.
constexpr int kSmallBM = 64, kSmallBN = 64, kSmallBK = 64, kSmallStages = 3;
constexpr int kWideBM = 128, kWideBN = 128, kWideBK = 32, kWideStages = 3;
constexpr int kPadK = 64;  // K padding of the split activation rows (a multiple of both slice depths)
constexpr int64_t kWideMinTiles = 256;
// K ranges of a weight with few 128 x 128 tiles: up to kMaxSplit, each at least kSplitMinKTiles 32-deep slices
// (1536 elements; measured at 512 rows: an FFN-down projection, K = 8192, 108 -> 80 us in 4 ranges; a QKV one, K =
// 2048, 38 -> 40 us in 4 ranges of 512, whose partial sums cost more than the halved operand traffic saves, so it is
// not cut); the partial sums live in a fixed area of the workspace (64 MB), which bounds a split weight's outputs.
constexpr int kMaxSplit = 4, kSplitMinKTiles = 48;
// K ranges of a weight's 64 x 64 tiles in calls of few rows, where the tiles are too few to fill the CUs and each
// walks the whole K: up to kFewMaxSplit ranges of at least kFewMinKTiles 64-deep slices, while the weight's tiles
// times its ranges stay within kFewMinWgs (measured at the QKV shape, K = 2048, 3072 output rows: 12-64 rows,
// 27-29 -> 15-19 us per call; 65-128 rows, 29-30 -> 19-22 us; FFN gate + up and down shapes unchanged. A target of
// 512 workgroups, up to 256 rows, gained 2-4 us at 192-256 QKV rows but cost gate + up 4-10 us at 32-128 rows).
// Such calls take these ranges rather than the wide tiles' ones above, whose few 128 x 128 tiles would leave most CUs
// idle (FFN down, K = 8192, 2048 output rows: 17-64 rows 61-64 -> 28-30 us, 96-128 rows 64-65 -> 40-41 us).
constexpr int kFewMaxRows = 128, kFewMaxSplit = 8, kFewMinKTiles = 4;
constexpr int64_t kFewMinWgs = 256;
constexpr int64_t kSplitPartFloats = int64_t(1) << 24;

template <int BM, int BN, int BK, int STAGES>
__global__ __launch_bounds__(kThreads) void gemm_f16w_kernel(GemmBatch b, const _Float16* __restrict__ xh,
                                                             const _Float16* __restrict__ xl,
                                                             const float* __restrict__ inv_scale, int64_t n,
                                                             int64_t in, int64_t in_pad) {
  constexpr int CPR = BK / 8;             // 16-byte chunks per tile row
  constexpr int XT = BM * BK, WT = BN * BK;  // halves per activation-part tile and per weight tile
  constexpr int XLD = BM * CPR / 256;     // loads per wave per activation part (1 KB pieces over 4 waves)
  constexpr int WLD = BN * CPR / 256;     // loads per wave for the weight tile
  constexpr int MB = BM / 64, NB = BN / 64;  // 32-wide activation-row and weight-row blocks per wave
  __shared__ __attribute__((aligned(16))) _Float16 lds[STAGES][2 * XT + WT];
  int wi = 0;
  for (int j = 1; j < b.n_w; ++j)
    if (int(blockIdx.x) >= b.w[j].tile0) wi = j;
  const GemmWeight& d = b.w[wi];
  // this workgroup's output tile and K range: workgroups of a split weight are tile-major within each range
  const int local = int(blockIdx.x) - d.tile0, tiles = int((d.rows + BN - 1) / BN);
  const int ks = local / tiles;
  const int64_t n0 = int64_t(local % tiles) * BN, m0 = int64_t(blockIdx.y) * BM;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // this wave's rows wm*BM/2.. and weight rows wn*BN/2..

  // Buffer resources over the valid rows only: reads past the activation count or the weight's row count return
  // zeros (their results are never stored), so no row index is clamped.
  const uint32_t xrows = uint32_t(min<int64_t>(n - m0, BM)), wrows = uint32_t(min<int64_t>(d.rows - n0, BN));
  const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<_Float16*>(xh + m0 * in_pad), 0, int(xrows * uint32_t(in_pad) * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<_Float16*>(xl + m0 * in_pad), 0, int(xrows * uint32_t(in_pad) * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(d.w + n0 * in), 0,
                                                                      int(wrows * uint32_t(in) * 2), 0x00020000);
  // A load fills one 1 KB piece: piece q of an operand is LDS slots 64 q .. 64 q + 63 (slot = row * CPR +
  // position); lane -> slot, and the lane loads the chunk that position holds. Load i of this wave is piece
  // i * 4 + wave of its operand.
  auto slot_chunk = [&](int q, int& r) {
    const int slot = q * 64 + lane;
    r = slot / CPR;
    return (slot % CPR) ^ swz<CPR>(r);
  };
  uint32_t xoff[XLD], woff[WLD];
  int wk[WLD];
#pragma unroll
  for (int i = 0; i < XLD; ++i) {
    int r;
    const int x = slot_chunk(i * 4 + wave, r);
    xoff[i] = uint32_t((r * int(in_pad) + 8 * x) * 2);
  }
#pragma unroll
  for (int i = 0; i < WLD; ++i) {
    int r;
    const int x = slot_chunk(i * 4 + wave, r);
    wk[i] = 8 * x;
    woff[i] = uint32_t((r * int(in) + 8 * x) * 2);
  }
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int nk_all = int(in_pad / BK), per = (nk_all + d.split - 1) / d.split;
  const int kb = ks * per;  // this range's first K tile
  auto fetch = [&](int kt, int st) {
    const uint32_t k0 = uint32_t(kb + kt) * BK;
#pragma unroll
    for (int i = 0; i < XLD; ++i) {
      buffer_load_lds16(rh, &lds[st][(i * 4 + wave_u) * 512], xoff[i] + k0 * 2);
      buffer_load_lds16(rl, &lds[st][XT + (i * 4 + wave_u) * 512], xoff[i] + k0 * 2);
    }
#pragma unroll
    for (int i = 0; i < WLD; ++i) {  // weight columns past `in` read as zeros (the offset is sent past the buffer)
      const bool ok = int64_t(k0) + wk[i] < in;
      buffer_load_lds16(rw, &lds[st][2 * XT + (i * 4 + wave_u) * 512], ok ? woff[i] + k0 * 2 : 0x80000000u);
    }
  };
  constexpr int kLoads = 2 * XLD + WLD;  // this wave's loads per stage
  // Fragment offsets (bytes within an operand tile) of this lane's reads for the BK / 16 steps of a slice.
  const int hf = lane >> 5;
  uint32_t fa[MB][BK / 16], fb[NB][BK / 16];
#pragma unroll
  for (int s = 0; s < BK / 16; ++s) {
    const int x = 2 * s + hf;
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const int ra = wm * (BM / 2) + 32 * i + (lane & 31);
      fa[i][s] = uint32_t((ra * BK + 8 * (x ^ swz<CPR>(ra))) * 2);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int rb = wn * (BN / 2) + 32 * j + (lane & 31);
      fb[j][s] = uint32_t((2 * XT + rb * BK + 8 * (x ^ swz<CPR>(rb))) * 2);
    }
  }
  auto frag = [&](int st, uint32_t off) {
    return *reinterpret_cast<const half8_t*>(reinterpret_cast<const char*>(&lds[st][0]) + off);
  };

  floatx16 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  const int nk = max(0, min(per, nk_all - kb));  // K tiles of this range
#pragma unroll
  for (int i = 0; i < STAGES - 1; ++i)
    if (i < nk) fetch(i, i);
  // Tile kt lives in stage kt % STAGES: wait for this wave's loads of it (the later tiles' may stay in flight), one
  // barrier publishes it and certifies every wave is done with tile kt - 1, whose stage then takes tile
  // kt + STAGES - 1.
  auto step = [&](int kt, auto cur_c) {
    constexpr int cur = decltype(cur_c)::value;
    const int ahead = min(nk - 1 - kt, STAGES - 2);  // tiles after kt already fetched
    if constexpr (STAGES >= 4) {
      if (ahead >= 2)
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(2 * kLoads));
      else if (ahead == 1)
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(kLoads));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(0));
    } else if constexpr (STAGES == 3) {
      if (ahead >= 1)
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(kLoads));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_wait(0));
    } else {
      __builtin_amdgcn_s_waitcnt(vmcnt_wait(0));
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + STAGES - 1 < nk) fetch(kt + STAGES - 1, (cur + STAGES - 1) % STAGES);
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      half8_t ah[MB], al[MB], bw[NB];
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        ah[i] = frag(cur, fa[i][s]);
        al[i] = frag(cur, uint32_t(XT * 2) + fa[i][s]);
      }
#pragma unroll
      for (int j = 0; j < NB; ++j) bw[j] = frag(cur, fb[j][s]);
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bw[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bw[j], acc[i][j], 0, 0, 0);
    }
  };
  for (int kt = 0; kt < nk; kt += STAGES) {
    step(kt, std::integral_constant<int, 0>{});
    if constexpr (STAGES > 1)
      if (kt + 1 < nk) step(kt + 1, std::integral_constant<int, 1>{});
    if constexpr (STAGES > 2)
      if (kt + 2 < nk) step(kt + 2, std::integral_constant<int, 2>{});
    if constexpr (STAGES > 3)
      if (kt + 3 < nk) step(kt + 3, std::integral_constant<int, 3 % STAGES>{});
  }

  // acc[i][j][r] holds activation row 8 (r / 4) + 4 hf + r % 4 of the wave's block i and weight row lane % 32 of
  // its block j. A K range's partial sums go unscaled to its slice of part.
  float* const dst = d.split > 1 ? d.part + int64_t(ks) * n * d.rows : d.y;
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int64_t col = n0 + wn * (BN / 2) + 32 * j + (lane & 31);
    if (col < d.rows) {
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t t = m0 + wm * (BM / 2) + 32 * i + 8 * (r / 4) + 4 * hf + (r % 4);
          if (t < n) dst[t * d.rows + col] = d.split > 1 ? acc[i][j][r] : acc[i][j][r] * inv_scale[t];
        }
    }
  }
}

// y = (sum of a split weight's K-range partials, in range order) * 1 / s_t, for every weight of the batch with
// split > 1: one thread per output, the weights' outputs laid end to end (`first` output of each, in weight order).
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(GemmBatch b, const float* __restrict__ inv_scale,
                                                                int64_t n, int64_t total) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  int64_t off = 0;
  for (int j = 0; j < b.n_w; ++j) {
    const GemmWeight& d = b.w[j];
    const int64_t cnt = n * d.rows;
    if (i < off + cnt) {
      const int64_t o = i - off;
      float acc = 0.f;
      for (int s = 0; s < d.split; ++s) acc += d.part[int64_t(s) * cnt + o];
      d.y[o] = acc * inv_scale[o / d.rows];
      return;
    }
    off += cnt;
  }
}

int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

}  // namespace

extern "C" {

int64_t nbhs_gemm_f16w_workspace(int64_t n, int64_t in) {
  if (n <= 0 || in <= 0 || n > (int64_t(1) << 31) || in > (int64_t(1) << 30)) return -1;
  const int64_t in_pad = round_up(in, kPadK);
  return round_up(2 * n * in_pad * 2, 256) + round_up(n * 4, 256) + kSplitPartFloats * 4;
}

int nbhs_gemm_f16w_multi(int n_w, const void* const* w, float* const* y, const int64_t* rows, int64_t in,
                         const float* x, int64_t n, void* ws, int64_t ws_bytes, nbhs_stream stream) {
  if (n_w <= 0 || n_w > kMaxWeights || !w || !y || !rows || !x || !ws || n <= 0 || in <= 0 || in % 8 != 0)
    return NBHS_EINVAL;
  const int64_t need = nbhs_gemm_f16w_workspace(n, in);
  if (need < 0 || ws_bytes < need || reinterpret_cast<uintptr_t>(ws) % 256 != 0) return NBHS_EINVAL;
  const int64_t in_pad = round_up(in, kPadK);
  // every operand a buffer resource addresses must fit 32-bit offsets
  if (kWideBM * in_pad * 2 > INT32_MAX || kWideBN * in * 2 > INT32_MAX || n > 65535 * int64_t(kSmallBM))
    return NBHS_EINVAL;
  // every weight is checked before anything is launched, so a rejected call writes no output
  for (int i = 0; i < n_w; ++i)
    if (!w[i] || !y[i] || rows[i] <= 0 || rows[i] > INT32_MAX || reinterpret_cast<uintptr_t>(w[i]) % 16 != 0)
      return NBHS_EINVAL;
  char* base = static_cast<char*>(ws);
  _Float16* xh = reinterpret_cast<_Float16*>(base);
  _Float16* xl = xh + n * in_pad;
  float* inv = reinterpret_cast<float*>(base + round_up(2 * n * in_pad * 2, 256));
  float* part = reinterpret_cast<float*>(base + round_up(2 * n * in_pad * 2, 256) + round_up(n * 4, 256));
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int vec = reinterpret_cast<uintptr_t>(x) % 16 == 0 ? 1 : 0;
  const unsigned wide_rows = unsigned((n + kWideBM - 1) / kWideBM), small_rows = unsigned((n + kSmallBM - 1) / kSmallBM);
  // Each weight's configuration follows from its own shape (so its results do not depend on the other weights of
  // the call: matmul_multi equals separate calls): 128 x 128 tiles when they alone are many; otherwise, when K is
  // long and the output fits the partial-sum area, 128 x 128 tiles over 2 or 4 K ranges (each range's workgroup
  // fetches half the operand bytes per product of a 64 x 64 tile's, and the ranges restore the workgroup count;
  // the partials are summed in range order); otherwise 64 x 64 tiles. The weights of each configuration share a
  // launch; split weights share one while their partials fit the area, then the next group starts.
  GemmBatch wide{}, small{}, split{}, fsplit{};
  int64_t wide_tiles = 0, small_tiles = 0, split_wgs = 0, split_out = 0, fsplit_wgs = 0, fsplit_out = 0,
          part_used = 0;
  hipError_t e = nbhs_timing::launch(NBHS_K_SPLIT_ACTS, split_acts_kernel, dim3(unsigned(n)), dim3(64), s, x, in,
                                     in_pad, xh, xl, inv, vec);
  // the weights taking K ranges (128 x 128 tiles, or 64 x 64 ones in calls of few rows), whose partial sums share
  // the partial-sum area: their launches and sums, then the area is free again
  auto flush_split = [&]() {
    if (e == hipSuccess && split.n_w > 0) {
      e = nbhs_timing::launch(NBHS_K_GEMM, gemm_f16w_kernel<kWideBM, kWideBN, kWideBK, kWideStages>,
                              dim3(unsigned(split_wgs), wide_rows), dim3(kThreads), s, split, xh, xl, inv, n, in,
                              in_pad);
      if (e == hipSuccess)
        e = nbhs_timing::launch(NBHS_K_GEMM_REDUCE, gemm_split_reduce_kernel,
                                dim3(unsigned((split_out + 255) / 256)), dim3(256), s, split, inv, n, split_out);
    }
    if (e == hipSuccess && fsplit.n_w > 0) {
      e = nbhs_timing::launch(NBHS_K_GEMM, gemm_f16w_kernel<kSmallBM, kSmallBN, kSmallBK, kSmallStages>,
                              dim3(unsigned(fsplit_wgs), small_rows), dim3(kThreads), s, fsplit, xh, xl, inv, n, in,
                              in_pad);
      if (e == hipSuccess)
        e = nbhs_timing::launch(NBHS_K_GEMM_REDUCE, gemm_split_reduce_kernel,
                                dim3(unsigned((fsplit_out + 255) / 256)), dim3(256), s, fsplit, inv, n, fsplit_out);
    }
    split = fsplit = GemmBatch{};
    split_wgs = split_out = fsplit_wgs = fsplit_out = part_used = 0;
  };
  for (int i = 0; i < n_w && e == hipSuccess; ++i) {
    const int64_t wt = (rows[i] + kWideBN - 1) / kWideBN * wide_rows;
    int sp = 1;
    if (wt < kWideMinTiles && n > kFewMaxRows && n * rows[i] * kMaxSplit <= kSplitPartFloats) {
      const int64_t nkt = in_pad / kWideBK;
      while (sp < kMaxSplit && wt * sp < kWideMinTiles && nkt / (2 * sp) >= kSplitMinKTiles) sp *= 2;
    }
    const _Float16* wd = static_cast<const _Float16*>(w[i]);
    if (wt >= kWideMinTiles) {
      wide.w[wide.n_w++] = GemmWeight{wd, y[i], rows[i], int(wide_tiles), 1, nullptr};
      wide_tiles += (rows[i] + kWideBN - 1) / kWideBN;
    } else if (sp > 1) {
      const int64_t cnt = n * rows[i] * sp;
      if (part_used + cnt > kSplitPartFloats) flush_split();
      split.w[split.n_w++] = GemmWeight{wd, y[i], rows[i], int(split_wgs), sp, part + part_used};
      split_wgs += (rows[i] + kWideBN - 1) / kWideBN * sp;
      split_out += n * rows[i];
      part_used += cnt;
    } else {
      const int64_t st = (rows[i] + kSmallBN - 1) / kSmallBN * small_rows;
      int fsp = 1;
      if (n <= kFewMaxRows && n * rows[i] * kFewMaxSplit <= kSplitPartFloats) {
        const int64_t nkt = in_pad / kSmallBK;
        while (fsp < kFewMaxSplit && st * fsp * 2 <= kFewMinWgs && nkt / (2 * fsp) >= kFewMinKTiles) fsp *= 2;
      }
      if (fsp > 1) {
        const int64_t cnt = n * rows[i] * fsp;
        if (part_used + cnt > kSplitPartFloats) flush_split();
        fsplit.w[fsplit.n_w++] = GemmWeight{wd, y[i], rows[i], int(fsplit_wgs), fsp, part + part_used};
        fsplit_wgs += (rows[i] + kSmallBN - 1) / kSmallBN * fsp;
        fsplit_out += n * rows[i];
        part_used += cnt;
      } else {
        small.w[small.n_w++] = GemmWeight{wd, y[i], rows[i], int(small_tiles), 1, nullptr};
        small_tiles += (rows[i] + kSmallBN - 1) / kSmallBN;
      }
    }
    if (wide_tiles > INT32_MAX || small_tiles > INT32_MAX || split_wgs > INT32_MAX || fsplit_wgs > INT32_MAX)
      return NBHS_EINVAL;
  }
  flush_split();
  if (e == hipSuccess && wide.n_w > 0)
    e = nbhs_timing::launch(NBHS_K_GEMM, gemm_f16w_kernel<kWideBM, kWideBN, kWideBK, kWideStages>,
                            dim3(unsigned(wide_tiles), wide_rows), dim3(kThreads), s, wide, xh, xl, inv, n, in, in_pad);
  if (e == hipSuccess && small.n_w > 0)
    e = nbhs_timing::launch(NBHS_K_GEMM, gemm_f16w_kernel<kSmallBM, kSmallBN, kSmallBK, kSmallStages>,
                            dim3(unsigned(small_tiles), small_rows), dim3(kThreads), s, small, xh, xl, inv, n, in,
                            in_pad);
  return e;
}

}  // extern "C"
