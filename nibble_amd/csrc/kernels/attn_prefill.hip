// Causal GQA prefill attention on gfx950 MFMA: Backend::attention (backend.h:68-69) for many query rows,
// semantics of ref_ops.cpp:188-214 (row t attends to cache rows 0..pos0+t; head h reads KV head h/(H/KV)).
//
// Numerics: Q is scaled by log2(e)/sqrt(d) and split into fp16 high and low parts (a rounding of the query would
// be shared by every key of its row), K and V come from fp16 copies of the fp32 cache (stage_kv), QK^T (K times
// both query parts) and PV run on v_mfma_f32_32x32x16_f16 with fp32 accumulation, and the online softmax (shift,
// exp2, running sums, rescaling) is fp32. The softmax shift is not the running max: it is set from the first tile
// and raised only when a tile's weights outgrow it (checked through their sum, see kPSumMax), so the per-tile
// max, the subtraction (folded into the MFMA accumulator init) and the O rescale all leave the common path; the
// result is the same normalised softmax, since any shift cancels. The host routes rows with fewer than 128
// visible keys to the fp32 decode kernel, where fp16 rounding of a few V rows is not averaged away.
//
// Layout (per wave, 32 query rows):
//  * S^T = K Q^T: A = K tile rows from LDS ([key][d], 16 B per lane), B = the wave's Q fragment held in
//    registers for the whole pass. The accumulator puts one query per lane column (lane % 32) and 16 keys per
//    lane, so the row max needs one cross-half shuffle and the running (m, l) are per-lane scalars.
//  * O^T = V^T P^T: B = P straight from the S^T accumulator registers (converted to fp16), A = V^T from LDS
//    ([d][key]), whose keys are staged in the accumulator's row interleave (vt_key) so that a lane's 8 keys are
//    one 16-byte read. O^T keeps one query per lane too, so rescaling O is a per-lane multiply.
//  * K and V^T tiles of 64 keys go from global memory straight into LDS (global_load_lds, no register staging),
//    XOR-swizzled instead of padded, through a 3-stage ring for head_dim 64: two tiles are in flight while one
//    is computed, with one barrier per tile.
//  * GQA packing: the G query heads sharing a KV head are interleaved into the row dimension (packed row
//    p = t*G + head), so a workgroup's 128 rows span only 128/G positions and each K/V tile in LDS serves all G
//    heads.
//  * Scheduling: workgroup b takes KV head b % KV and row tiles from the longest (last) to the shortest, so
//    long causal rows start first and, with workgroups dispatched round-robin over the 8 XCDs, one KV head's
//    tiles stay in one XCD's L2.
//  * Rows kept in fp32 (the first ones, whose few keys do not average out fp16 rounding of V) ride in the same
//    launch: workgroups after the MFMA tiles run the fp32 split-context body (nbh_decode::partial_block, one
//    chunk per row) from the fp32 cache, in the tail the shortest MFMA tiles leave.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "backend/hip/kernel_timing.h"
#include "kernels/decode_block.h"
#include "kernels/rope_device.h"
#include "nibble_hip_shim.h"

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kBN = 64;          // keys per tile
// Query column blocks of 32 per wave: with 2, every K and V^T fragment read from LDS feeds two MFMAs and each wave
// keeps twice the independent MFMA chains in flight (at twice the accumulator registers).
#ifndef NBH_PREFILL_QB
#define NBH_PREFILL_QB 1
#endif
constexpr int kQB = NBH_PREFILL_QB;
constexpr int kRowsPerWave = 32 * kQB;
#ifndef NBH_PREFILL_WAVES
#define NBH_PREFILL_WAVES 4
#endif
constexpr int kWaves = NBH_PREFILL_WAVES;
constexpr int kRowsPerBlock = kRowsPerWave * kWaves;
constexpr int kPad = 8;          // halves of LDS row padding of the staging transpose (spreads banks)
// Largest sum of one lane's 32 tile weights accepted without recomputing the tile against a raised shift: every
// weight is then <= 2^12, far inside fp16 (max 65504).
constexpr float kPSumMax = 4096.0f;
// Work list of row tiles the precise kernel recomputes, in a buffer of kAuxHead + 3 cap words: aux[0] = entries,
// aux[1] = the call's epoch, then one word per (row tile, KV head) holding the epoch of the last call that listed
// it, then the list itself, then one arrival counter per list entry (zeroed by the staging launch).
constexpr int kAuxHead = 16;
// Per key split of a prefill row tile, the record beside its partial output: shift, sum, sum of squared weights,
// the error estimate's score coefficient (est_c1 * |y|^2/d * largest |k|^2), the largest |v|^2 and the query
// residual's coefficient (est_c3 * |r| * sqrt(largest |k|^2)).
constexpr int kSplitRec = 6;

// Rounding-error estimate of a row computed with fp16 operands. The scaled query y = Q * log2(e)/sqrt(d) enters
// the scores as two fp16 parts, y = hi + lo + r (hi = fp16(y), lo = fp16(y - hi), |r| ~ 2^-22 |y|), so its
// rounding is not a per-row error shared by every key. K and V are staged with stochastic rounding (f16_sr): one
// independent, zero-mean error per element whatever the data, of variance at most u^2 x^2 (u = 2^-11); the weights
// P are rounded to nearest, one rounding per key modelled as independent with variance u^2/3; accumulation is fp32.
// To first order the output error of dimension d is
//   sum_j w_j [ln2 (e_j - e_mean)(v_jd - o_d) + eps_v,jd v_jd + (eps_p,j - eps_p,mean)(v_jd - o_d)] + c_d,
// w_j = p_j / l, with e_j the score error (log2 units) of key j from rounding k_j: variance about
// u^2 |y|^2/d |k_j|^2. Bounding |k_j|^2 by the largest row norm K, |v_jd| by the largest element V and
// (v - o)^2 by 2 (V^2 + O^2), O the row's largest output:
//   var <= (sum_j p_j^2 / l^2) [2 ln2^2 u^2 (|y|^2/d) K (V^2 + O^2) + (u^2/3) (5 V^2 + 2 O^2)].
// Over an fp16 cache K and V are staged exactly and only the weights' term (u^2/3) 2 (V^2 + O^2) remains.
// The query's residual r is common to every key of the row, so its term c_d = ln2 sum_j w_j (r.k_j)(v_jd - o_d)
// does not average out; it is bounded outright, |c_d| <= ln2 |r| sqrt(K) (V + O), with |r| computed exactly per row.
// The row is accepted when kEstZ * sqrt(var) + ln2 |r| sqrt(K) (V + O) <= kEstBudget (the 1e-3 parity bar).
// Checked against an exact emulation of this kernel's rounding (its stochastic rounding bit for bit) over N(0,1)
// data at score scales 0.5-30, keys with 1 % outlier rows x8, outlier V rows, a query aligned with one key,
// low-rank keys, a large common key or value component, q, K and V projected from shared low-rank hidden states (K
// and V correlated: the case where an unsplit query's rounding adds up coherently over the keys), 65-8192 keys,
// head_dim 64 and 128: the emulated error stayed within 0.62 sqrt(var) (tests/test_error_estimate.py). With value
// rows repeated - in runs, alternating or recurring at scattered positions, their large elements 0.1-0.49 ulp off
// the fp16 grid, where rounding to nearest erred by up to 1.97e-3 on rows this estimate keeps - it stayed within
// 1.3 sqrt(var), so an accepted row errs by at most 1.3 / 1.5 of the bar. The model is statistical: values placed
// on purpose at the largest stochastic-rounding variance in every dimension make sqrt(var) tight, and the largest
// of a row's dimensions can then exceed 1.5 sqrt(var) (emulated: up to 1.18e-3 on 4 of 300 such rows kept);
// set_attention_fp32 routes every row through fp32 for callers that need the bar for any input.
constexpr float kEstZ = 1.5f;
// A row whose weights are all (nearly) equal - keys * sum p^2 <= (sum p)^2 (1 + kFlatTol), equality exactly when
// every weight is the same - has lost its scores' differences to the weights' rounding (a near-zero query: every
// weight rounds to the same fp16 value), an error the variance model does not see and that does not shrink with the
// output when the values cancel. Such rows are recomputed. Rows of ordinary scores sit far above the threshold.
constexpr float kFlatTol = 1.0f / 4096.0f;
constexpr float kEstBudget = 1e-3f;
constexpr double kEstU = 1.0 / 2048.0;
constexpr double kLn2 = 0.6931471805599453;

__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }  // v_exp_f32; -inf -> 0

// (hi, lo) of x: hi = fp16(x), lo = fp16(x - hi). Both must start from the same x: a product passed in is pinned to
// its fp32 rounding first (the empty asm), or the compiler fuses the multiply into hi's conversion (v_fma_mixlo_f16,
// one rounding of the exact product) while lo subtracts a hi rounded from the fp32 product - at an fp16 tie the two
// disagree and hi + lo misses x by one fp16 ulp. x - hi is exact in fp32 (hi is x's nearest fp16).
__device__ __forceinline__ half2_t split_f16(float x) {
  asm("" : "+v"(x));
  const _Float16 hi = (_Float16)x;
  return half2_t{hi, (_Float16)(x - (float)hi)};
}

// Chunk swizzle of LDS tile rows with CPR 16-byte chunks: rows 0..7 (and 0..15) map a given chunk to distinct
// chunks, and for 8-chunk (128-byte) rows also the rows of equal parity among 16 consecutive ones (64-bank LDS
// serves 16 lanes per cycle, and rows r, r + 2 share banks there).
template <int CPR>
__device__ __forceinline__ int swz(int r) {
  if constexpr (CPR >= 16) return r & 15;
  return (r ^ (r >> 3)) & 7;
}

// 16 bytes from global memory into LDS without passing through registers: lane l of the wave writes bytes
// [16 l, 16 l + 16) after the wave-uniform LDS address (global_load_lds_dwordx4; completion counts in vmcnt). The
// builtin is left out of the host compilation pass, where its presence makes clang drop the kernel's launch stub.
__device__ __forceinline__ void load_lds16(const void* src, void* lds_wave_base) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(src, lds_wave_base, 16, 0, 0);
#endif
}

// The same 16-byte load through a buffer resource: byte offset voff (per lane) + soff (uniform) into the buffer.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, void* lds_wave_base, uint32_t voff,
                                                  uint32_t soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, lds_wave_base, 16, voff, soff, 0, 0);
#endif
}

// s_waitcnt immediate that waits for at most n outstanding vector-memory loads and nothing else (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int vmcnt_wait(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

// The S^T accumulator gives lane (query, half hf) the 8 keys {4hf .. 4hf+3, 8+4hf .. 8+4hf+3} of each 16-key step,
// and that register order is the B operand (P) of the PV MFMA, so its A operand (V^T) must hold the same keys at
// k = 8hf + e. Staged V^T rows store each 16-key group as keys [0-3, 8-11, 4-7, 12-15]: a lane's 8 keys are then
// 16 consecutive bytes. vt_key(p) is the key stored at position p of a 64-key tile row.
__device__ __forceinline__ int vt_key(int p) { return (p & ~15) + (p & 3) + ((p >> 2) & 1) * 8 + ((p >> 3) & 1) * 4; }

// Four consecutive cache elements as fp32, and back (an fp16 cache stores them rounded to nearest even, as the
// fp16-cache append kernels do).
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 ld4(const _Float16* p) {
  const half4_t h = *reinterpret_cast<const half4_t*>(p);
  return make_float4(float(h[0]), float(h[1]), float(h[2]), float(h[3]));
}
__device__ __forceinline__ void st4(float* p, float4 x) { *reinterpret_cast<float4*>(p) = x; }
__device__ __forceinline__ void st4(_Float16* p, float4 x) {
  *reinterpret_cast<half4_t*>(p) = half4_t{(_Float16)x.x, (_Float16)x.y, (_Float16)x.z, (_Float16)x.w};
}
// x as a cache of element type KVT stores it
template <typename KVT>
__device__ __forceinline__ float4 as_cached(float4 x) {
  if constexpr (sizeof(KVT) == 4) {
    return x;
  } else {
    return make_float4(float(_Float16(x.x)), float(_Float16(x.y)), float(_Float16(x.z)), float(_Float16(x.w)));
  }
}

// Stochastic rounding of the staged operands. Rounded to nearest, equal cache values round alike wherever they sit,
// so value rows that repeat (a token recurring in the prompt: V carries no rotation), key dimensions that RoPE
// barely turns over a window, or values that sit on a common offset from the fp16 grid carry one shared rounding
// error that the softmax's weighted mean does not average out (up to 1.95e-3 for elements of 4 to 8). Each element
// is instead rounded up or down with probability given by its distance to the two fp16 neighbours, with random bits
// hashed from its (position, KV head, dimension): the errors are zero-mean and independent from key to key whatever
// the data, which is what the error estimate's variance model takes them to be, and the staging repeats bit for bit
// (the same row is staged to the same fp16 values in every call). The variance of one such rounding is at most
// ulp^2/4 <= u^2 x^2 (u = 2^-11), three times the u^2 x^2 / 3 of a rounding to nearest modelled as uniform.
//
// sr_bits: lowbias32 (Chris Wellons' integer hash, public domain) of a key built from the element's coordinates.
__device__ __forceinline__ uint32_t sr_bits(int64_t row, int g, int d, int hd) {
  uint32_t x = uint32_t(row) * 0x9E3779B1u + uint32_t(g * hd + d) * 0x85EBCA77u + 0x27D4EB2Fu;
  x ^= x >> 16;
  x *= 0x7FEB352Du;
  x ^= x >> 15;
  x *= 0x846CA68Bu;
  x ^= x >> 16;
  return x;
}
// x to fp16, rounded up or down at random: r13 (13 uniform bits) is added below the 10 mantissa bits fp16 keeps,
// and the 13 bits below them are dropped, so the magnitude rounds up with probability (dropped part) / ulp. Applied
// where the result is an fp16 normal number below 2^15 (the truncated value is then exactly representable); other
// values (fp16 subnormals, whose rounding error is below 2^-25; magnitudes of 2^15 and more; inf and NaN) are
// rounded to nearest.
__device__ __forceinline__ _Float16 f16_sr(float x, uint32_t r13) {
  const uint32_t b = __float_as_uint(x), mag = b & 0x7FFFFFFFu;
  if (mag >= 0x38800000u && mag < 0x47000000u) return (_Float16)__uint_as_float((b + r13) & ~0x1FFFu);
  return (_Float16)x;
}

// ---- staging: cache rows -> fp16 K [KV][rows_pad][HD] and transposed V [KV][HD][rows_pad] ----
// The cache holds fp32 (KVT float) or fp16 (KVT _Float16) elements; an fp16 cache's rows are staged unchanged, an
// fp32 cache's are rounded to fp16 stochastically (f16_sr).
// Rows [0, pos0) come from the cache ck/cv; rows [pos0, rows), when kn/vn are given, are the appended rows: K
// rotated by RoPE at its position (cs, neox) in fp32, and both written into the cache (rounded to fp16 for an fp16
// cache) as well as staged - the KV append and the staging in one pass. A thread takes one row and dimensions [4 d4, 4 d4 + 4) and the same four
// HD/2 further on, so both RoPE pairings (adjacent, and NeoX's (j, j + HD/2)) stay within the thread. Rows past
// `rows` (padding up to rows_pad) are staged as zeros.
template <int HD, typename KVT>
__global__ __launch_bounds__(256) void stage_kv_kernel(KVT* ck, KVT* cv, const float* __restrict__ kn,
                                                       const float* __restrict__ vn, _Float16* __restrict__ k16,
                                                       _Float16* __restrict__ vt16, int64_t pos0, int64_t rows,
                                                       int64_t rows_pad, int n_kv, const float2* __restrict__ cs,
                                                       int neox, float2* __restrict__ kstats,
                                                       uint32_t* __restrict__ aux, int aux_cap) {
  __shared__ _Float16 tr[HD][kBN + kPad];
  __shared__ float red[2][4];
  const int g = blockIdx.y;
  const int64_t r0 = int64_t(blockIdx.x) * kBN;
  constexpr int H2 = HD / 2;
  constexpr int LPR = HD / 8;  // threads per row in the loop below (consecutive lanes)
  // The prefill launch that follows collects its flagged row tiles afresh (see attn_prefill_kernel): empty the
  // list and open a new epoch (never 0, the value of entries no call has written).
  if (aux) {
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
      aux[0] = 0;
      const uint32_t e = aux[1] + 1;
      aux[1] = e ? e : 1;
    }
    const int64_t nthreads = int64_t(gridDim.x) * gridDim.y * 256;
    for (int64_t w = (int64_t(blockIdx.y) * gridDim.x + blockIdx.x) * 256 + threadIdx.x; w < aux_cap; w += nthreads)
      aux[kAuxHead + 2 * aux_cap + w] = 0;  // the precise kernel's arrival counters
  }
  float k2max = 0.f, vmax = 0.f;  // this tile's largest |k row|^2 and |v| element, as the cache holds them
  for (int idx = threadIdx.x; idx < kBN * HD / 8; idx += 256) {
    const int r = idx / (HD / 8), d4 = idx % (HD / 8);
    const int64_t row = r0 + r;
    float4 k0 = make_float4(0.f, 0.f, 0.f, 0.f), k1 = k0, v0 = k0, v1 = k0;
    if (row < rows) {
      const int64_t at = (row * n_kv + g) * HD + 4 * d4;
      if (row < pos0 || !kn) {
        k0 = ld4(ck + at);
        k1 = ld4(ck + at + H2);
        v0 = ld4(cv + at);
        v1 = ld4(cv + at + H2);
      } else {
        const int64_t src = ((row - pos0) * n_kv + g) * HD + 4 * d4;
        k0 = *reinterpret_cast<const float4*>(kn + src);
        k1 = *reinterpret_cast<const float4*>(kn + src + H2);
        v0 = *reinterpret_cast<const float4*>(vn + src);
        v1 = *reinterpret_cast<const float4*>(vn + src + H2);
        const float2* c = cs + row * H2;
        if (neox) {
          rope_rotate(k0.x, k1.x, c[4 * d4 + 0]);
          rope_rotate(k0.y, k1.y, c[4 * d4 + 1]);
          rope_rotate(k0.z, k1.z, c[4 * d4 + 2]);
          rope_rotate(k0.w, k1.w, c[4 * d4 + 3]);
        } else {
          rope_rotate(k0.x, k0.y, c[2 * d4]);
          rope_rotate(k0.z, k0.w, c[2 * d4 + 1]);
          rope_rotate(k1.x, k1.y, c[H2 / 2 + 2 * d4]);
          rope_rotate(k1.z, k1.w, c[H2 / 2 + 2 * d4 + 1]);
        }
        k0 = as_cached<KVT>(k0);  // the values the cache holds from here on
        k1 = as_cached<KVT>(k1);
        v0 = as_cached<KVT>(v0);
        v1 = as_cached<KVT>(v1);
        st4(ck + at, k0);
        st4(ck + at + H2, k1);
        st4(cv + at, v0);
        st4(cv + at + H2, v1);
      }
    }
    float ss = k0.x * k0.x + k0.y * k0.y + k0.z * k0.z + k0.w * k0.w + k1.x * k1.x + k1.y * k1.y + k1.z * k1.z +
               k1.w * k1.w;
#pragma unroll
    for (int m = 1; m < LPR; m <<= 1) ss += __shfl_xor(ss, m, 64);  // the row's LPR lanes: its squared norm
    k2max = fmaxf(k2max, ss);
    vmax = fmaxf(vmax, fmaxf(fmaxf(fmaxf(fabsf(v0.x), fabsf(v0.y)), fmaxf(fabsf(v0.z), fabsf(v0.w))),
                             fmaxf(fmaxf(fabsf(v1.x), fabsf(v1.y)), fmaxf(fabsf(v1.z), fabsf(v1.w)))));
    const float kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    _Float16 kh[8], vh[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (sizeof(KVT) == 4) {
        // one hash per element: bits 0..12 round its K value, bits 13..25 its V value
        const uint32_t rb = sr_bits(row, g, (e < 4 ? 0 : H2) + 4 * d4 + (e & 3), HD);
        kh[e] = f16_sr(kk[e], rb & 0x1FFFu);
        vh[e] = f16_sr(vv[e], (rb >> 13) & 0x1FFFu);
      } else {
        kh[e] = (_Float16)kk[e];  // already fp16 values
        vh[e] = (_Float16)vv[e];
      }
    }
    _Float16* kd = k16 + (int64_t(g) * rows_pad + row) * HD + 4 * d4;
    *reinterpret_cast<half4_t*>(kd) = half4_t{kh[0], kh[1], kh[2], kh[3]};
    *reinterpret_cast<half4_t*>(kd + H2) = half4_t{kh[4], kh[5], kh[6], kh[7]};
#pragma unroll
    for (int e = 0; e < 8; ++e) tr[(e < 4 ? 0 : H2) + 4 * d4 + (e & 3)][r] = vh[e];
  }
  __syncthreads();
  // V^T: each d row of the tile is 64 keys (128 B), stored in the key order of the PV MFMA operand (vt_key).
  for (int idx = threadIdx.x; idx < HD * kBN / 8; idx += 256) {
    const int d = idx / (kBN / 8), c8 = idx % (kBN / 8);
    half8_t x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = tr[d][vt_key(8 * c8 + e)];
    *reinterpret_cast<half8_t*>(vt16 + (int64_t(g) * HD + d) * rows_pad + r0 + 8 * c8) = x;
  }
  if (kstats) {  // the tile's statistics for the prefill kernel's error estimate
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
      k2max = fmaxf(k2max, __shfl_xor(k2max, m, 64));
      vmax = fmaxf(vmax, __shfl_xor(vmax, m, 64));
    }
    if ((threadIdx.x & 63) == 0) {
      red[0][threadIdx.x >> 6] = k2max;
      red[1][threadIdx.x >> 6] = vmax;
    }
    __syncthreads();
    if (threadIdx.x == 0)
      kstats[int64_t(g) * (rows_pad / kBN) + blockIdx.x] =
          make_float2(fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3])),
                      fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3])));
  }
}

// Occupancy (waves per SIMD) the register allocator must reach. The kernel is built with MFMA accumulators in
// architectural VGPRs (-amdgpu-mfma-vgpr-form, see the Makefile), so the S^T and O^T accumulators both stay
// resident with no per-tile copies through accumulation registers. head_dim 64 is held to 3 waves per SIMD
// (<= 168 registers, measured fastest: 2 waves with more registers per wave lose more latency hiding than they
// gain); head_dim 128 is held to 2 (256 registers: its query's high and low parts alone take 64), where two
// values live across the key loop go to scratch outside it.
#ifndef NBH_PREFILL_WAVES_PER_EU
#define NBH_PREFILL_WAVES_PER_EU 3
#endif
#ifndef NBH_PREFILL_MIN_WAVES_PER_EU
#define NBH_PREFILL_MIN_WAVES_PER_EU 3
#endif
template <int HD, typename KVT>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(
    HD == 64 ? NBH_PREFILL_MIN_WAVES_PER_EU : 2, NBH_PREFILL_WAVES_PER_EU)))
void attn_prefill_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ k16, const _Float16* __restrict__ vt16,
    float* __restrict__ out, int64_t n, int64_t pos0, int n_heads, int n_kv, int group, int64_t rows_pad,
    int n_tiles, float qscale, const float2* __restrict__ q_rope, int q_rope_neox, const KVT* __restrict__ kc,
    const KVT* __restrict__ vc, int64_t fp32_rows, int fp32_n_sub, int n_split, float* __restrict__ ws_o,
    float* __restrict__ ws_ml, const float2* __restrict__ kstats, uint32_t* __restrict__ aux, int aux_cap,
    float est_c1, float est_cv, float est_co, float est_c3) {
  // Workgroups past the MFMA tiles: query row t < fp32_rows of the call (q and out start fp32_rows rows before
  // this launch's MFMA rows) for KV head x head subgroup `by`, in fp32 over its whole causal window.
  static_assert(kWaves * 64 == nbh_decode::kDecodeThreads, "the fp32 rows' body runs on the MFMA workgroup size");
  if (int64_t(blockIdx.x) >= int64_t(n_tiles) * n_kv * n_split) {
    const int64_t e = int64_t(blockIdx.x) - int64_t(n_tiles) * n_kv * n_split;
    const int streams = n_kv * fp32_n_sub;
    const int64_t p0 = pos0 - fp32_rows;
    constexpr int64_t kStepRows =
        (nbh_decode::kDecodeThreads / 64) * (64 / (HD / 8)) * nbh_decode::unroll_for(int(sizeof(KVT)));
    nbh_decode::partial_block<HD, 4, KVT>(q - fp32_rows * n_heads * HD, kc, vc, out - fp32_rows * n_heads * HD,
                                     nullptr, nullptr, p0, n_heads, n_kv, group, fp32_n_sub, 1,
                                     (p0 + fp32_rows + kStepRows - 1) / kStepRows, 0, qscale, q_rope, q_rope_neox,
                                     nullptr, nullptr, nullptr, nullptr, 0, int(e % streams),
                                     fp32_rows - 1 - e / streams);  // longest rows first
    return;
  }
  constexpr int DC = HD / 16;  // 16-wide d chunks of the S^T contraction
  constexpr int DT = HD / 32;  // 32-row d tiles of O^T
  // K and V^T tiles live in LDS unpadded, one row of 16-byte chunks per key (K) or per dimension (V^T), with chunk
  // x of row r stored at chunk x ^ swz(r). The fragment reads (16 B per lane, one row per lane) then hit distinct
  // bank groups for any 8 consecutive rows (32 banks) or 16 (64 banks), and the tiles can be filled by
  // global_load_lds, which writes each wave's 64 lanes x 16 B to one contiguous kilobyte of LDS: the swizzle is
  // applied on the global side, by choosing which chunk each lane fetches.
  constexpr int KCPR = HD / 8;    // 16-byte chunks per K row
  constexpr int VCPR = kBN / 8;   // 16-byte chunks per V^T row
  constexpr int THREADS = kWaves * 64;
  constexpr int K_LD = kBN * KCPR / THREADS;  // global_load_lds instructions per wave per K tile
  constexpr int V_LD = HD * VCPR / THREADS;   // ... per V^T tile
  static_assert(K_LD * THREADS == kBN * KCPR && V_LD * THREADS == HD * VCPR, "tiles split evenly over lanes");
  // Pipeline depth: tiles in LDS at once (the current one and those being fetched).
  constexpr int kStages = HD == 64 ? 3 : 2;
  __shared__ _Float16 ks[kStages][kBN * HD];
  __shared__ _Float16 vs[kStages][HD * kBN];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ql = lane & 31, hf = lane >> 5;
  // Workgroup b: KV head b % KV, key split (b / KV) % n_split of row tile n_tiles - 1 - b / (KV n_split).
  const int b = blockIdx.x;
  const int g = b % n_kv;
  const int split = (b / n_kv) % n_split;
  const int tile = n_tiles - 1 - b / (n_kv * n_split);
  const int64_t P = n * group;
  const int64_t pb0 = int64_t(tile) * kRowsPerBlock;
  const int64_t wp0 = pb0 + wave * kRowsPerWave;
  // The lane's query of column block qb: packed row wp0 + 32 qb + ql.
  bool active[kQB];
  int64_t t[kQB], qpos[kQB];
  int head[kQB];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const int64_t p = wp0 + 32 * qb + ql;
    active[qb] = p < P;
    t[qb] = active[qb] ? p / group : 0;
    head[qb] = g * group + (active[qb] ? int(p % group) : 0);
    qpos[qb] = pos0 + t[qb];
  }

  const int64_t p_last = min(pb0 + kRowsPerBlock, P) - 1;
  const int64_t kend = pos0 + p_last / group + 1;  // the block's keys: [0, kend)
  const int ntk = int((kend + kBN - 1) / kBN);
  // This workgroup's key tiles: split `split` of the block's ntk tiles in n_split contiguous ranges.
  const int per_split = (ntk + n_split - 1) / n_split;
  const int kt0 = min(ntk, split * per_split), kt1 = min(ntk, kt0 + per_split);
  const bool wave_active = wp0 < P;
  const int64_t wave_kend = wave_active ? pos0 + (min(wp0 + kRowsPerWave, P) - 1) / group + 1 : 0;
  const int64_t wave_kfull = wave_active ? pos0 + wp0 / group + 1 : 0;  // keys every row of the wave sees

  // Q fragments (B operand of S^T): query of block qb, d = 16c + 8hf .. +8. Unrotated q (q_rope = the
  // position-major (cos, sin) table) is rotated here, exactly as the RoPE kernel would have in memory: the lane
  // holds both members of every pair it needs - adjacent pairs within its 8 dimensions, NeoX pairs (j, j + HD/2)
  // in chunks c and c + DC/2.
  // qf / qlo: the scaled query's fp16 high and low parts (both multiply each K fragment, see split_f16); qr2: the
  // squared norm of what the two leave out, for the error estimate's query term.
  half8_t qf[kQB][DC], qlo[kQB][DC];
  float qn2[kQB], qr2[kQB];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const float* qrow = q + (t[qb] * n_heads + head[qb]) * HD;
    float x[DC][8];
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f), bb = a;
      if (active[qb]) {
        a = *reinterpret_cast<const float4*>(qrow + 16 * c + 8 * hf);
        bb = *reinterpret_cast<const float4*>(qrow + 16 * c + 8 * hf + 4);
      }
      x[c][0] = a.x, x[c][1] = a.y, x[c][2] = a.z, x[c][3] = a.w;
      x[c][4] = bb.x, x[c][5] = bb.y, x[c][6] = bb.z, x[c][7] = bb.w;
    }
    if (q_rope && active[qb]) {
      const float2* cs = q_rope + qpos[qb] * (HD / 2);
      if (q_rope_neox) {
#pragma unroll
        for (int c = 0; c < DC / 2; ++c)
#pragma unroll
          for (int e = 0; e < 8; ++e) rope_rotate(x[c][e], x[c + DC / 2][e], cs[16 * c + 8 * hf + e]);
      } else {
#pragma unroll
        for (int c = 0; c < DC; ++c)
#pragma unroll
          for (int e = 0; e < 8; e += 2) rope_rotate(x[c][e], x[c][e + 1], cs[(16 * c + 8 * hf + e) / 2]);
      }
    }
    float ss = 0.f, rr = 0.f;
#pragma unroll
    for (int c = 0; c < DC; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float y = x[c][e] * qscale;
        asm("" : "+v"(y));  // hi, lo and the norms all from y's fp32 rounding (see split_f16)
        ss += y * y;
        const half2_t hl = split_f16(y);
        qf[qb][c][e] = hl[0];
        qlo[qb][c][e] = hl[1];
        const float r = (y - float(hl[0])) - float(hl[1]);  // both differences exact in fp32
        rr += r * r;
      }
    qn2[qb] = (ss + __shfl_xor(ss, 32, 64)) * (1.0f / HD);  // mean square of the scaled query
    qr2[qb] = rr + __shfl_xor(rr, 32, 64);
  }

  floatx16 oacc[kQB][DT];
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) oacc[qb][dt][r] = 0.f;
  // m_sh: the query's softmax shift (log2 domain). With one query block the subtraction is folded into the S^T
  // MFMAs: their accumulator starts from mneg, 16 copies of -m_sh. With two blocks the registers are scarcer and
  // the shift is subtracted on the VALU instead, which has slack.
  constexpr bool kFold = kQB == 1;
  float m_sh[kQB], l_run[kQB], l2_run[kQB];  // l2_run: sum of the squared fp16 weights (the error estimate's)
  float kmx = 0.f, vmx = 0.f;  // largest |k row|^2 and |v| element over the key tiles this wave visits
  floatx16 mneg;
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    m_sh[qb] = 0.f;
    l_run[qb] = 0.f;
    l2_run[qb] = 0.f;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) mneg[r] = 0.f;

  const _Float16* kg = k16 + int64_t(g) * rows_pad * HD;
  const _Float16* vg = vt16 + int64_t(g) * HD * rows_pad;
  // The KV head's staged K [rows_pad][HD] and V^T [HD][rows_pad] as buffer resources: each lane's byte offset
  // within a tile is fixed for the whole pass (a VGPR computed once) and the tile's offset is a scalar, so a fetch
  // costs no vector instructions. Out-of-range reads would return zeros, not fault.
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(kg), 0,
                                                                      int(rows_pad * HD * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(vg), 0,
                                                                      int(HD * rows_pad * 2), 0x00020000);
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  uint32_t koff[K_LD], voff[V_LD];
#pragma unroll
  for (int i = 0; i < K_LD; ++i) {
    const int piece = i * kWaves + wave, slot = piece * 64 + lane;
    const int r = slot / KCPR, x = (slot % KCPR) ^ swz<KCPR>(r);
    koff[i] = uint32_t((r * HD + 8 * x) * 2);
  }
#pragma unroll
  for (int i = 0; i < V_LD; ++i) {
    const int piece = i * kWaves + wave, slot = piece * 64 + lane;
    const int d = slot / VCPR, x = (slot % VCPR) ^ swz<VCPR>(d);
    voff[i] = uint32_t((d * int(rows_pad) + 8 * x) * 2);
  }
  // Asynchronous fetch of key tile kt into LDS stage st: each wave fills its share of 1 KB pieces.
  auto fetch = [&](int kt, int st) {
#pragma unroll
    for (int i = 0; i < K_LD; ++i)
      buffer_load_lds16(rk, &ks[st][(i * kWaves + wave_u) * 512], koff[i], uint32_t(kt) * (kBN * HD * 2));
#pragma unroll
    for (int i = 0; i < V_LD; ++i)
      buffer_load_lds16(rv, &vs[st][(i * kWaves + wave_u) * 512], voff[i], uint32_t(kt) * (kBN * 2));
  };
  // Fragment reads: this lane's byte offset within a stage for each (32-row block, 16-wide chunk) it reads, computed
  // once; with the stage a compile-time constant, a read is one ds_read with an immediate offset.
  uint32_t kfo[2][DC], vfo[DT][4];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      const int r = kk * 32 + ql, x = 2 * c + hf;
      kfo[kk][c] = uint32_t((r * HD + 8 * (x ^ swz<KCPR>(r))) * 2);
    }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      const int d = 32 * dt + ql, x = 2 * kc + hf;
      vfo[dt][kc] = uint32_t((d * kBN + 8 * (x ^ swz<VCPR>(d))) * 2);
    }
  auto k_frag = [&](int st, int kk, int c) {
    return *reinterpret_cast<const half8_t*>(reinterpret_cast<const char*>(&ks[st][0]) + kfo[kk][c]);
  };
  auto v_frag = [&](int st, int dt, int kc) {
    return *reinterpret_cast<const half8_t*>(reinterpret_cast<const char*>(&vs[st][0]) + vfo[dt][kc]);
  };

  // Tile kt lives in stage (kt - kt0) % kStages. Tiles kt0 .. kt0+kStages-2 are fetched ahead; step kt waits for
  // its own tile (the later ones may still be in flight), then one barrier both publishes tile kt to every wave and
  // certifies that all waves are done with tile kt - 1, whose stage the fetch of tile kt + kStages - 1 then
  // refills. The barrier is the bare s_barrier: the LDS writes are ordered by the wait on vmcnt (a load to LDS
  // completes when its data is in LDS), and a fence here would also wait for the fetches meant to stay in flight.
  // The loop is unrolled by kStages so every stage index is a compile-time constant (an immediate LDS offset).
#pragma unroll
  for (int i = 0; i < kStages - 1; ++i)
    if (kt0 + i < kt1) fetch(kt0 + i, i);
  auto step = [&](int kt, auto cur_c) {
    constexpr int cur = decltype(cur_c)::value;
    constexpr int ahead = (kStages - 2) * (K_LD + V_LD);  // this wave's loads of the tiles after kt
    if (kStages > 2 && kt + 1 < kt1)
      __builtin_amdgcn_s_waitcnt(vmcnt_wait(ahead));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_wait(0));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + kStages - 1 < kt1) fetch(kt + kStages - 1, (cur + kStages - 1) % kStages);
    if (wave_active && int64_t(kt) * kBN < wave_kend) {
      const float2 tst = kstats[int64_t(g) * (rows_pad / kBN) + kt];  // the tile's statistics (stage_kv_kernel)
      kmx = fmaxf(kmx, tst.x);
      vmx = fmaxf(vmx, tst.y);
      // S^T for the tile's two 32-key halves and every query block, K times the query's high and then its low
      // part in one accumulator; each K fragment read from LDS serves both parts and all blocks, and the chains
      // are interleaved so consecutive MFMAs do not wait on each other's results. The raised wave priority keeps
      // the MFMA pipe fed while other waves of the SIMD run their softmax VALU work.
      floatx16 s[kQB][2];
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int c = 0; c < DC; ++c) {
        const half8_t a[2] = {k_frag(cur, 0, c), k_frag(cur, 1, c)};
#pragma unroll
        for (int part = 0; part < 2; ++part)
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int qb = 0; qb < kQB; ++qb) {
              floatx16 c0;
              if (c == 0 && part == 0) {
                if constexpr (kFold) {
                  c0 = mneg;
                } else {
#pragma unroll
                  for (int r = 0; r < 16; ++r) c0[r] = 0.f;
                }
              } else {
                c0 = s[qb][kk];
              }
              s[qb][kk] =
                  __builtin_amdgcn_mfma_f32_32x32x16_f16(a[kk], part == 0 ? qf[qb][c] : qlo[qb][c], c0, 0, 0, 0);
            }
      }
      __builtin_amdgcn_s_setprio(0);
      // Causal mask (and inactive rows) only where some key of the tile lies past the wave's first row.
      if (int64_t(kt) * kBN + kBN > wave_kfull) {
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
          // keys of this tile past the query's position (relative to the tile start; inactive rows mask all)
          const int64_t rel64 = active[qb] ? qpos[qb] - int64_t(kt) * kBN : -1;
          const int rel = int(rel64 < kBN ? rel64 : kBN);
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if (kk * 32 + 8 * (r / 4) + 4 * hf + (r % 4) > rel) s[qb][kk][r] = -INFINITY;
        }
      }
      // P = exp2(S - m_sh) in fp16 (the MFMA B operand) and the lane's sum of it, taken from the same fp16 values
      // with v_dot2 so the normaliser matches the weights the MFMA multiplies.
      half8_t pb[kQB][4];
      float l_tile[kQB], l2_tile[kQB];
      const half2_t ones = {(_Float16)1.0f, (_Float16)1.0f};
      auto exps = [&](int qb, float shift) {
        l_tile[qb] = 0.f;
        l2_tile[qb] = 0.f;
#pragma unroll
        for (int kc = 0; kc < 4; ++kc)
#pragma unroll
          for (int e = 0; e < 8; ++e)
            pb[qb][kc][e] = (_Float16)exp2_raw(s[qb][kc >> 1][8 * (kc & 1) + e] - shift);
#pragma unroll
        for (int kc = 0; kc < 4; ++kc)
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            const half2_t w = {pb[qb][kc][e], pb[qb][kc][e + 1]};
            l_tile[qb] = __builtin_amdgcn_fdot2(w, ones, l_tile[qb], false);
            l2_tile[qb] = __builtin_amdgcn_fdot2(w, w, l2_tile[qb], false);
          }
      };
      // The shift is not raised per tile: the weights are computed against the current one, and only when some
      // lane's sum leaves (0, kPSumMax] - a score grew past the shift by ~12 (log2), or inf/NaN from an fp16
      // overflow - does the wave take the slow path below (always on its first tile, where no shift exists yet).
      bool slow = kt == kt0;
      if (!slow) {
        bool bad = false;
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
          exps(qb, kFold ? 0.0f : m_sh[qb]);
          bad = bad || !(l_tile[qb] <= kPSumMax);
        }
        slow = __builtin_amdgcn_ballot_w64(bad) != 0;
      }
      if (slow) {
#pragma unroll
        for (int qb = 0; qb < kQB; ++qb) {
          const float base = kFold ? 0.0f : m_sh[qb];  // s holds S - base
          float mt = -INFINITY;
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[qb][kk][r]);
          mt = fmaxf(mt, __shfl_xor(mt, 32, 64)) - base;  // tile max relative to the current shift
          // first tile: shift to the tile max (0 if every key is masked); later: raise by the excess only
          const float d = kt == kt0 ? (mt == -INFINITY ? 0.0f : mt) : fmaxf(mt, 0.0f);
          exps(qb, base + d);
          if (kt != kt0) {
            const float corr = exp2_raw(-d);
            l_run[qb] *= corr;
            l2_run[qb] *= corr * corr;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
              for (int r = 0; r < 16; ++r) oacc[qb][dt][r] *= corr;
          }
          m_sh[qb] += d;
          if constexpr (kFold) {
#pragma unroll
            for (int r = 0; r < 16; ++r) mneg[r] = -m_sh[qb];
          }
        }
      }
#pragma unroll
      for (int qb = 0; qb < kQB; ++qb) {
        l_run[qb] += l_tile[qb];
        l2_run[qb] += l2_tile[qb];
      }
      // O^T += V^T P^T over 4 steps of 16 keys; each V^T fragment read from LDS serves every query block, and the
      // DT x kQB output tiles are independent chains.
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const half8_t a = v_frag(cur, dt, kc);
#pragma unroll
          for (int qb = 0; qb < kQB; ++qb)
            oacc[qb][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[qb][kc], oacc[qb][dt], 0, 0, 0);
        }
      }
      __builtin_amdgcn_s_setprio(0);
    }
  };
  static_assert(kStages == 2 || kStages == 3, "the unrolled key loop covers two or three stages");
  for (int kt = kt0; kt < kt1; kt += kStages) {
    step(kt, std::integral_constant<int, 0>{});
    if (kt + 1 < kt1) step(kt + 1, std::integral_constant<int, 1>{});
    if constexpr (kStages > 2) {
      if (kt + 2 < kt1) step(kt + 2, std::integral_constant<int, 2>{});
    }
  }

  // Rounding-error estimate of this workgroup's rows (see kEstZ): a row whose estimate exceeds the budget flags
  // the row tile, which the precise kernel then recomputes from the fp32 cache.
  bool flag = false;
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const float l_tot = l_run[qb] + __shfl_xor(l_run[qb], 32, 64);
    const float l2_tot = l2_run[qb] + __shfl_xor(l2_run[qb], 32, 64);
    float om = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) om = fmaxf(om, fabsf(oacc[qb][dt][r]));
    om = fmaxf(om, __shfl_xor(om, 32, 64)) / l_tot;
    const float om2 = om * om, vg2 = vmx * vmx;
    const float est =
        l2_tot / (l_tot * l_tot) * (est_c1 * qn2[qb] * kmx * (vg2 + om2) + est_cv * vg2 + est_co * om2);
    const float rk = est_c3 * sqrtf(qr2[qb] * kmx);  // the query residual's bound, per unit of (V + O)
    const bool flat = l2_tot * float(qpos[qb] + 1) <= l_tot * l_tot * (1.0f + kFlatTol);
    flag = flag || (n_split == 1 && active[qb] && l_tot > 0.f && (flat || !(sqrtf(est) + rk * (vmx + om) <= 1.0f)));
    if (n_split > 1 && active[qb] && hf == 0) {
      // a key split judges nothing alone (few keys look sharp): its terms go to the merge, which estimates the row
      float* rec = ws_ml + ((t[qb] * n_heads + head[qb]) * n_split + split) * kSplitRec;
      rec[2] = l2_tot;
      rec[3] = est_c1 * qn2[qb] * kmx;
      rec[4] = vg2;
      rec[5] = rk;
    }
  }
  if (__syncthreads_or(flag) && threadIdx.x == 0) {
    // Append the row tile once per call, however many of its key splits flag it: entries hold the epoch of the
    // call that last listed them (the staging launch opens a new epoch).
    const uint32_t ep = aux[1], slot = uint32_t(tile) * uint32_t(n_kv) + uint32_t(g);
    if (atomicExch(&aux[kAuxHead + slot], ep) != ep) aux[kAuxHead + aux_cap + atomicAdd(&aux[0], 1u)] = slot;
  }
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    const float l_tot = l_run[qb] + __shfl_xor(l_run[qb], 32, 64);
    if (active[qb] && n_split > 1) {
      // One of several key splits: the unnormalised partial (shift m_sh in the log2 domain, sum, weighted V) in
      // the split-context decode kernel's layout, merged by the same log-sum-exp combine. A split with no visible
      // key leaves l = 0 and contributes nothing.
      const int64_t slot = (t[qb] * n_heads + head[qb]) * n_split + split;
      float* orow = ws_o + slot * HD;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 32 * dt + 8 * i + 4 * hf;
          *reinterpret_cast<float4*>(orow + d) =
              make_float4(oacc[qb][dt][4 * i], oacc[qb][dt][4 * i + 1], oacc[qb][dt][4 * i + 2],
                          oacc[qb][dt][4 * i + 3]);
        }
      if (hf == 0) {
        ws_ml[kSplitRec * slot] = l_tot > 0.f ? m_sh[qb] : -INFINITY;  // an empty split must not raise the merged max
        ws_ml[kSplitRec * slot + 1] = l_tot;
      }
    } else if (active[qb]) {
      const float inv = 1.0f / l_tot;
      float* orow = out + (t[qb] * n_heads + head[qb]) * HD;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 32 * dt + 8 * i + 4 * hf;
          *reinterpret_cast<float4*>(orow + d) =
              make_float4(oacc[qb][dt][4 * i] * inv, oacc[qb][dt][4 * i + 1] * inv, oacc[qb][dt][4 * i + 2] * inv,
                          oacc[qb][dt][4 * i + 3] * inv);
        }
    }
  }
}

// Precise recomputation of the row tiles the prefill kernel (or its split merge) listed because their
// rounding-error estimate exceeded the budget: the same tiling (4 waves x 32 packed rows, 64-key tiles) with every
// fp16 operand split into a high and a low part, x = hi + lo with hi = fp16(x) and lo = fp16(x - hi), about 22 bits:
//   S^T = Kh Qh^T + Kl Qh^T + Kh Ql^T,   O^T = Vh P_h^T + Vl P_h^T + Vh P_l^T
// (the lo x lo products, of relative size 2^-22, are left out), fp32 accumulation, an exact running max and fp32
// row sums. K and V come straight from the fp32 cache: each tile is loaded into registers one tile ahead, split and
// written to LDS by the workgroup.
// Work units: list entry e and key range r < ps of its row tile (ps = ranges per entry for this launch, at most
// kPreciseMaxRanges, fewer when the list is long). A tile whose keys span more than one range writes per-range
// partials (shift, sum, weighted V for its 128 rows) to ws; the last unit of the tile to finish (an arrival
// counter per entry, an agent-scope release before counting and an acquire after) merges them into out, reading
// every range's shifts and sums at once, then the weighted rows range by range with all of a thread's columns in
// flight together. The launch is persistent: the units that exist are numbered densely (the kernel's schedule
// below) and workgroup b takes units b, b + grid, ...; with a short list every unit starts at once, and with an
// empty list every workgroup returns at once.
constexpr int kPreciseMaxRanges = 16;
#ifndef NBH_PRECISE_MIN_TILES
#define NBH_PRECISE_MIN_TILES 4
#endif
#ifndef NBH_PRECISE_WG_PER_CU
#define NBH_PRECISE_WG_PER_CU 1
#endif
constexpr int kPreciseMinTiles = NBH_PRECISE_MIN_TILES;  // key tiles per range at least: shorter ones merge more
constexpr int kPreciseBatch = 32;    // a workgroup's units located per pass over the work list
constexpr int kPreciseSlotRegs = 4;  // list entries per thread kept in registers between the schedule's passes

__device__ __forceinline__ int precise_ranges(uint32_t count, int64_t ws_floats, int hd, int max_key_tiles) {
  const int64_t per_unit = int64_t(kRowsPerBlock) * (hd + 2);
  int64_t ps = count ? ws_floats / (per_unit * int64_t(count)) : 1;
  ps = min<int64_t>(ps, min<int64_t>(kPreciseMaxRanges, max_key_tiles / kPreciseMinTiles));
  return int(max<int64_t>(ps, 1));
}

template <int HD, typename KVT>
__global__ __launch_bounds__(kWaves * 64) void attn_prefill_precise_kernel(
    const float* __restrict__ q, const KVT* __restrict__ kc, const KVT* __restrict__ vc, float* __restrict__ out,
    int64_t n, int64_t pos0, int n_heads, int n_kv, int group, float qscale, const float2* __restrict__ q_rope,
    int q_rope_neox, uint32_t* __restrict__ aux, int aux_cap, float* __restrict__ ws, int64_t ws_floats) {
  static_assert(kQB == 1, "one 32-query block per wave");
  constexpr int DC = HD / 16, DT = HD / 32;
  constexpr int KCPR = HD / 8, VCPR = kBN / 8;
  constexpr int THREADS = kWaves * 64;
  constexpr int K_F4 = kBN * HD / 4 / THREADS;            // K float4 loads per thread per tile
  constexpr int V_U = (kBN / 2) * (HD / 8) / THREADS;     // V units (2 keys x 8 dims) per thread per tile
  __shared__ _Float16 khi[kBN * HD], klo[kBN * HD], vhi[HD * kBN], vlo[HD * kBN];
  __shared__ uint32_t arrival;
  __shared__ float merge_w[kPreciseMaxRanges][kRowsPerBlock];  // the merge's per-row range weights
  const uint32_t count = aux[0];
  if (count == 0) return;  // nothing listed: most calls of a chunked prefill
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ql = lane & 31, hf = lane >> 5;
  const int64_t P = n * group, rows_valid = pos0 + n;
  const int64_t row_stride = int64_t(n_kv) * HD;
  const int max_key_tiles = int((pos0 + n + kBN - 1) / kBN);
  const int ps = precise_ranges(count, ws_floats, HD, max_key_tiles);
  uint32_t* const arrivals = aux + kAuxHead + 2 * aux_cap;
  const uint32_t* const list = aux + kAuxHead + aux_cap;
  // key tiles of list entry e's row tile (its causal window)
  auto slot_ntk = [&](uint32_t slot) -> int {
    const int64_t pb = int64_t(slot / uint32_t(n_kv)) * kRowsPerBlock;
    return int((pos0 + (min(pb + kRowsPerBlock, P) - 1) / group + 1 + kBN - 1) / kBN);
  };

  // Schedule. T = the listed tiles' key tiles in all; an entry of ntk key tiles is cut into max(1, ntk / per_all)
  // equal ranges (at most ps, the workspace's slots), per_all = max(kPreciseMinTiles, ceil(T / grid)): ranges of at
  // least per_all tiles (a short entry stays whole, with no merge), and at most T / per_all <= grid units, one round
  // when the list allows it. The units (entry e, range r) are numbered densely, entry after entry, through a
  // block-wide prefix sum of the entries' range counts, and workgroup b takes units b, b + grid, ...: no workgroup
  // waits on units that do not exist.
  const uint32_t G = gridDim.x, b = blockIdx.x;
  __shared__ uint32_t s_wsum[kWaves];
  __shared__ uint32_t s_mine_e[kPreciseBatch], s_mine_r[kPreciseBatch], s_mine_slot[kPreciseBatch];
  // the list's slots, read once: entries threadIdx.x + THREADS j for j < kPreciseSlotRegs in registers, the rest
  // (lists longer than THREADS * kPreciseSlotRegs) read again where needed
  uint32_t slot_reg[kPreciseSlotRegs];
  uint32_t tsum = 0;
#pragma unroll
  for (int j = 0; j < kPreciseSlotRegs; ++j) {
    const uint32_t e = threadIdx.x + THREADS * j;
    slot_reg[j] = e < count ? list[e] : 0u;
    tsum += e < count ? uint32_t(slot_ntk(slot_reg[j])) : 0u;
  }
  for (uint32_t e = threadIdx.x + THREADS * kPreciseSlotRegs; e < count; e += THREADS)
    tsum += uint32_t(slot_ntk(list[e]));
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) tsum += __shfl_xor(tsum, m, 64);
  if (lane == 0) s_wsum[wave] = tsum;
  __syncthreads();
  uint32_t T = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) T += s_wsum[w];
  __syncthreads();
  const int per_all = max(kPreciseMinTiles, int((T + G - 1) / G));
  // key tiles per range of an entry of ntk key tiles; its ranges are ceil(ntk / per) <= ps
  auto entry_per = [&](int ntk) {
    const int nr = min(ps, max(1, ntk / per_all));
    return (ntk + nr - 1) / nr;
  };

  for (uint32_t done = 0;;) {
    // this workgroup's units done .. done + kPreciseBatch - 1 (its k-th unit is unit b + k G)
    uint32_t base = 0;  // units of the entries before this chunk
    for (uint32_t c0 = 0, c = 0; c0 < count; c0 += THREADS, ++c) {
      const uint32_t e = c0 + threadIdx.x;
      uint32_t nr = 0, slot = 0;
      if (e < count) {
        slot = c < kPreciseSlotRegs ? slot_reg[0] : list[e];
#pragma unroll
        for (int j = 1; j < kPreciseSlotRegs; ++j) slot = c == uint32_t(j) ? slot_reg[j] : slot;
        const int ntk = slot_ntk(slot), per = entry_per(ntk);
        nr = uint32_t((ntk + per - 1) / per);
      }
      uint32_t x = nr;  // inclusive prefix sum over the chunk
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
      }
      if (lane == 63) s_wsum[wave] = x;
      __syncthreads();
      uint32_t off = 0, total = 0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        off += w < wave ? s_wsum[w] : 0u;
        total += s_wsum[w];
      }
      __syncthreads();
      const uint32_t u0 = base + off + x - nr;  // entry e's first unit
      for (uint32_t u = u0 + (b + G - u0 % G) % G; u < u0 + nr; u += G) {
        const uint32_t k = (u - b) / G;
        if (k >= done && k < done + kPreciseBatch) {
          s_mine_e[k - done] = e;
          s_mine_r[k - done] = u - u0;
          s_mine_slot[k - done] = slot;
        }
      }
      base += total;
    }
    __syncthreads();
    const uint32_t mine = base > b ? (base - b + G - 1) / G : 0u;  // this workgroup's units in all
    const uint32_t batch = mine > done ? min(mine - done, uint32_t(kPreciseBatch)) : 0u;
    for (uint32_t kb = 0; kb < batch; ++kb) {
      const uint32_t it = s_mine_e[kb];
      const int range = int(s_mine_r[kb]);
      const uint32_t slot = s_mine_slot[kb];
      const int tile = int(slot / uint32_t(n_kv)), g = int(slot % uint32_t(n_kv));
      const int64_t pb0 = int64_t(tile) * kRowsPerBlock, wp0 = pb0 + wave * kRowsPerWave;
      const int64_t p = wp0 + ql;
      const bool active = p < P;
      const int64_t t = active ? p / group : 0;
      const int head = g * group + (active ? int(p % group) : 0);
      const int64_t qpos = pos0 + t;
      const int64_t kend = pos0 + (min(pb0 + kRowsPerBlock, P) - 1) / group + 1;
      const int ntk = int((kend + kBN - 1) / kBN);
      // this unit's key tiles: range `range` of the tile's ntk tiles in n_ranges contiguous ranges of at least
      // kPreciseMinTiles tiles (a short tile is one range)
      const int per = entry_per(ntk), n_ranges = (ntk + per - 1) / per;
      const int kt0 = range * per, kt1 = min(ntk, kt0 + per);
      const bool wave_active = wp0 < P;
      const int64_t wave_kend = wave_active ? pos0 + (min(wp0 + kRowsPerWave, P) - 1) / group + 1 : 0;
      const int64_t wave_kfull = wave_active ? pos0 + wp0 / group + 1 : 0;

      // Q (rotated on load when q_rope is given, as the prefill kernel does), scaled, split.
      half8_t qh[DC], qlw[DC];
      {
        const float* qrow = q + (t * n_heads + head) * HD;
        float x[DC][8];
  #pragma unroll
        for (int c = 0; c < DC; ++c) {
          float4 a = make_float4(0.f, 0.f, 0.f, 0.f), bb = a;
          if (active) {
            a = *reinterpret_cast<const float4*>(qrow + 16 * c + 8 * hf);
            bb = *reinterpret_cast<const float4*>(qrow + 16 * c + 8 * hf + 4);
          }
          x[c][0] = a.x, x[c][1] = a.y, x[c][2] = a.z, x[c][3] = a.w;
          x[c][4] = bb.x, x[c][5] = bb.y, x[c][6] = bb.z, x[c][7] = bb.w;
        }
        if (q_rope && active) {
          const float2* cs = q_rope + qpos * (HD / 2);
          if (q_rope_neox) {
  #pragma unroll
            for (int c = 0; c < DC / 2; ++c)
  #pragma unroll
              for (int e = 0; e < 8; ++e) rope_rotate(x[c][e], x[c + DC / 2][e], cs[16 * c + 8 * hf + e]);
          } else {
  #pragma unroll
            for (int c = 0; c < DC; ++c)
  #pragma unroll
              for (int e = 0; e < 8; e += 2) rope_rotate(x[c][e], x[c][e + 1], cs[(16 * c + 8 * hf + e) / 2]);
          }
        }
  #pragma unroll
        for (int c = 0; c < DC; ++c)
  #pragma unroll
          for (int e = 0; e < 8; ++e) {
            const half2_t hl = split_f16(x[c][e] * qscale);
            qh[c][e] = hl[0];
            qlw[c][e] = hl[1];
          }
      }

      floatx16 oacc[DT];
  #pragma unroll
      for (int dt = 0; dt < DT; ++dt)
  #pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
      float m = -INFINITY, l = 0.f;

      // One key tile's fp32 K rows (float4 (key, 4 dims)) and V pairs (keys 2j, 2j+1 x 8 dims), held in registers one
      // tile ahead of the compute; rows past the call's last valid row are zeros (and masked).
      float4 kr[K_F4], va[V_U][2], vb[V_U][2];
      auto fetch = [&](int kt) {
        const int64_t r0 = int64_t(kt) * kBN;
  #pragma unroll
        for (int i = 0; i < K_F4; ++i) {
          const int f = threadIdx.x + THREADS * i, r = f / (HD / 4), c4 = f % (HD / 4);
          kr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (r0 + r < rows_valid) kr[i] = ld4(kc + (r0 + r) * row_stride + g * HD + 4 * c4);
        }
  #pragma unroll
        for (int i = 0; i < V_U; ++i) {
          const int uu = threadIdx.x + THREADS * i, db = uu % (HD / 8), j = uu / (HD / 8);
          const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
          va[i][0] = va[i][1] = vb[i][0] = vb[i][1] = z;
          const int64_t ra = r0 + 2 * j;
          if (ra < rows_valid) {
            const KVT* src = vc + ra * row_stride + g * HD + 8 * db;
            va[i][0] = ld4(src);
            va[i][1] = ld4(src + 4);
          }
          if (ra + 1 < rows_valid) {
            const KVT* src = vc + (ra + 1) * row_stride + g * HD + 8 * db;
            vb[i][0] = ld4(src);
            vb[i][1] = ld4(src + 4);
          }
        }
      };
      // The fetched tile, split, into LDS: K rows at their swizzled chunks, V^T as key pairs in the vt_key order
      // (vt_key is its own inverse: the position of key 2j, with 2j + 1 next to it).
      auto stage = [&]() {
  #pragma unroll
        for (int i = 0; i < K_F4; ++i) {
          const int f = threadIdx.x + THREADS * i, r = f / (HD / 4), c4 = f % (HD / 4);
          const half2_t sx = split_f16(kr[i].x), sy = split_f16(kr[i].y), sz = split_f16(kr[i].z), sw = split_f16(kr[i].w);
          const int at = r * HD + 8 * ((c4 >> 1) ^ swz<KCPR>(r)) + 4 * (c4 & 1);
          *reinterpret_cast<half4_t*>(&khi[at]) = half4_t{sx[0], sy[0], sz[0], sw[0]};
          *reinterpret_cast<half4_t*>(&klo[at]) = half4_t{sx[1], sy[1], sz[1], sw[1]};
        }
  #pragma unroll
        for (int i = 0; i < V_U; ++i) {
          const int uu = threadIdx.x + THREADS * i, db = uu % (HD / 8), j = uu / (HD / 8);
          const int pos = vt_key(2 * j);
          const float a8[8] = {va[i][0].x, va[i][0].y, va[i][0].z, va[i][0].w, va[i][1].x, va[i][1].y, va[i][1].z,
                               va[i][1].w};
          const float b8[8] = {vb[i][0].x, vb[i][0].y, vb[i][0].z, vb[i][0].w, vb[i][1].x, vb[i][1].y, vb[i][1].z,
                               vb[i][1].w};
  #pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int d = 8 * db + e;
            const half2_t sa = split_f16(a8[e]), sb = split_f16(b8[e]);
            const int at = d * kBN + 8 * ((pos >> 3) ^ swz<VCPR>(d)) + (pos & 7);
            *reinterpret_cast<half2_t*>(&vhi[at]) = half2_t{sa[0], sb[0]};
            *reinterpret_cast<half2_t*>(&vlo[at]) = half2_t{sa[1], sb[1]};
          }
        }
      };
      auto kfrag = [&](const _Float16* base, int r, int x) {
        return *reinterpret_cast<const half8_t*>(&base[r * HD + 8 * (x ^ swz<KCPR>(r))]);
      };
      auto vfrag = [&](const _Float16* base, int d, int x) {
        return *reinterpret_cast<const half8_t*>(&base[d * kBN + 8 * (x ^ swz<VCPR>(d))]);
      };

      fetch(kt0);
      for (int kt = kt0; kt < kt1; ++kt) {
        __syncthreads();  // every wave is done with the previous tile (or unit) in LDS
        stage();
        __syncthreads();
        if (kt + 1 < kt1) fetch(kt + 1);  // in flight while this tile is computed
        const int64_t r0 = int64_t(kt) * kBN;
        if (!(wave_active && r0 < wave_kend)) continue;
        floatx16 sacc[2];
  #pragma unroll
        for (int kk = 0; kk < 2; ++kk)
  #pragma unroll
          for (int r = 0; r < 16; ++r) sacc[kk][r] = 0.f;
        // consecutive MFMAs go to the two halves' independent accumulators
  #pragma unroll
        for (int c = 0; c < DC; ++c) {
          half8_t ah[2], al[2];
  #pragma unroll
          for (int kk = 0; kk < 2; ++kk) {
            ah[kk] = kfrag(khi, kk * 32 + ql, 2 * c + hf);
            al[kk] = kfrag(klo, kk * 32 + ql, 2 * c + hf);
          }
  #pragma unroll
          for (int kk = 0; kk < 2; ++kk) sacc[kk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[kk], qh[c], sacc[kk], 0, 0, 0);
  #pragma unroll
          for (int kk = 0; kk < 2; ++kk) sacc[kk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[kk], qlw[c], sacc[kk], 0, 0, 0);
  #pragma unroll
          for (int kk = 0; kk < 2; ++kk) sacc[kk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[kk], qh[c], sacc[kk], 0, 0, 0);
        }
        if (r0 + kBN > wave_kfull) {
          const int64_t rel64 = active ? qpos - r0 : -1;
          const int rel = int(rel64 < kBN ? rel64 : kBN);
  #pragma unroll
          for (int kk = 0; kk < 2; ++kk)
  #pragma unroll
            for (int r = 0; r < 16; ++r)
              if (kk * 32 + 8 * (r / 4) + 4 * hf + (r % 4) > rel) sacc[kk][r] = -INFINITY;
        }
        float mt = -INFINITY;
  #pragma unroll
        for (int kk = 0; kk < 2; ++kk)
  #pragma unroll
          for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sacc[kk][r]);
        const float mn = fmaxf(m, fmaxf(mt, __shfl_xor(mt, 32, 64)));
        const float ms = mn == -INFINITY ? 0.0f : mn;
        if (__builtin_amdgcn_ballot_w64(mn > m) != 0) {
          const float corr = exp2_raw(m - ms);  // m = -inf: 0, and o, l are still 0
          l *= corr;
  #pragma unroll
          for (int dt = 0; dt < DT; ++dt)
  #pragma unroll
            for (int r = 0; r < 16; ++r) oacc[dt][r] *= corr;
        }
        m = mn;
  #pragma unroll
        for (int kk = 0; kk < 2; ++kk)
  #pragma unroll
          for (int r = 0; r < 16; ++r) {
            sacc[kk][r] = exp2_raw(sacc[kk][r] - ms);
            l += sacc[kk][r];
          }
  #pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
          half8_t ph, pl;
  #pragma unroll
          for (int e = 0; e < 8; ++e) {
            const half2_t hl = split_f16(sacc[kc >> 1][8 * (kc & 1) + e]);
            ph[e] = hl[0];
            pl[e] = hl[1];
          }
          half8_t ah[DT], al[DT];
  #pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            ah[dt] = vfrag(vhi, 32 * dt + ql, 2 * kc + hf);
            al[dt] = vfrag(vlo, 32 * dt + ql, 2 * kc + hf);
          }
  #pragma unroll
          for (int dt = 0; dt < DT; ++dt) oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[dt], ph, oacc[dt], 0, 0, 0);
  #pragma unroll
          for (int dt = 0; dt < DT; ++dt) oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[dt], pl, oacc[dt], 0, 0, 0);
  #pragma unroll
          for (int dt = 0; dt < DT; ++dt) oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[dt], ph, oacc[dt], 0, 0, 0);
        }
      }
      const float l_tot = l + __shfl_xor(l, 32, 64);
      if (n_ranges == 1) {  // the whole key range: the output directly
        if (active) {
          const float inv = 1.0f / l_tot;
          float* orow = out + (t * n_heads + head) * HD;
  #pragma unroll
          for (int dt = 0; dt < DT; ++dt)
  #pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int d = 32 * dt + 8 * i + 4 * hf;
              *reinterpret_cast<float4*>(orow + d) = make_float4(oacc[dt][4 * i] * inv, oacc[dt][4 * i + 1] * inv,
                                                                 oacc[dt][4 * i + 2] * inv, oacc[dt][4 * i + 3] * inv);
            }
        }
        continue;
      }
      // A partial: rows of the tile as [128][HD + 2] (weighted V, then shift and sum) in the unit's workspace slot.
      float* part = ws + (int64_t(it) * ps + range) * kRowsPerBlock * (HD + 2);
      {
        float* prow = part + int64_t(wave * kRowsPerWave + ql) * (HD + 2);
  #pragma unroll
        for (int dt = 0; dt < DT; ++dt)
  #pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int d = 32 * dt + 8 * i + 4 * hf;
            *reinterpret_cast<float4*>(prow + d) =
                make_float4(oacc[dt][4 * i], oacc[dt][4 * i + 1], oacc[dt][4 * i + 2], oacc[dt][4 * i + 3]);
          }
        if (hf == 0) {
          prow[HD] = l_tot > 0.f ? m : -INFINITY;  // a range with no visible key must not raise the merged max
          prow[HD + 1] = l_tot;
        }
      }
      // Arrive; the last range of the tile merges. Release the partial before counting, acquire the others after.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      __syncthreads();
      if (threadIdx.x == 0) arrival = atomicAdd(&arrivals[it], 1u);
      __syncthreads();
      if (arrival != uint32_t(n_ranges - 1)) continue;
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      const float* p0 = ws + int64_t(it) * ps * kRowsPerBlock * (HD + 2);
      // Each row's weights 2^(m_r - M) / L over the ranges, every range's (m, l) loaded at once (one row per thread).
      if (threadIdx.x < kRowsPerBlock) {
        const int r = threadIdx.x;
        float2 ml[kPreciseMaxRanges];
  #pragma unroll
        for (int rg = 0; rg < kPreciseMaxRanges; ++rg)
          ml[rg] = rg < n_ranges ? *reinterpret_cast<const float2*>(p0 + (int64_t(rg) * kRowsPerBlock + r) * (HD + 2) + HD)
                                 : make_float2(-INFINITY, 0.f);
        float mx = -INFINITY;
  #pragma unroll
        for (int rg = 0; rg < kPreciseMaxRanges; ++rg) mx = fmaxf(mx, ml[rg].x);
        const float msh = mx == -INFINITY ? 0.0f : mx;
        float lsum = 0.f;
  #pragma unroll
        for (int rg = 0; rg < kPreciseMaxRanges; ++rg) {
          ml[rg].x = exp2_raw(ml[rg].x - msh);
          lsum += ml[rg].y * ml[rg].x;
        }
        const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;  // 0: a row past the call's last (never written out)
  #pragma unroll
        for (int rg = 0; rg < kPreciseMaxRanges; ++rg)
          if (rg < n_ranges) merge_w[rg][r] = ml[rg].x * inv;
      }
      __syncthreads();
      // The weighted rows: every thread's ITEMS (row, float4 column) pairs, one range after another, the items' loads
      // of a range in flight together.
      constexpr int V4 = HD / 4, ITEMS = kRowsPerBlock * V4 / THREADS;
      static_assert(ITEMS * THREADS == kRowsPerBlock * V4, "merge items split evenly over the threads");
      float4 acc[ITEMS];
  #pragma unroll
      for (int j = 0; j < ITEMS; ++j) acc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int rg = 0; rg < n_ranges; ++rg) {
        float4 o[ITEMS];
  #pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
          const int idx = int(threadIdx.x) + THREADS * j, r = idx / V4, c4 = idx % V4;
          o[j] = *reinterpret_cast<const float4*>(p0 + (int64_t(rg) * kRowsPerBlock + r) * (HD + 2) + 4 * c4);
        }
  #pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
          const int idx = int(threadIdx.x) + THREADS * j, r = idx / V4;
          const float w = merge_w[rg][r];
          acc[j].x += o[j].x * w;
          acc[j].y += o[j].y * w;
          acc[j].z += o[j].z * w;
          acc[j].w += o[j].w * w;
        }
      }
  #pragma unroll
      for (int j = 0; j < ITEMS; ++j) {
        const int idx = int(threadIdx.x) + THREADS * j, r = idx / V4, c4 = idx % V4;
        const int64_t pp = pb0 + r;
        if (pp >= P) continue;
        const int64_t tt = pp / group;
        const int hh = g * group + int(pp % group);
        reinterpret_cast<float4*>(out + (tt * n_heads + hh) * HD)[c4] = acc[j];
      }
    }
    __syncthreads();  // the batch's slots are read; the next batch may overwrite them
    done += batch;
    if (done >= mine) break;
  }
}

// Merges the key splits of the MFMA rows (partials in the decode kernel's layout: slot rh * n_split + s holds the
// weighted V row and a kSplitRec record - shift m in the log2 domain, sum l, ...). One thread per (row x head rh,
// float4 column): out = sum_s O_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), M = max_s m_s, the splits taken in order. The
// row's rounding-error estimate (the prefill kernel's, over the merged weights) is evaluated here, and a row over
// budget lists its row tile for the precise kernel. SPM >= n_split: every split's record and partial are loaded at
// once, in registers.
template <int HD, int SPM>
__global__ __launch_bounds__(256) void prefill_split_merge(const float* __restrict__ ws_o,
                                                           const float* __restrict__ ws_ml, float* __restrict__ out,
                                                           int64_t rows_heads, int n_split, int n_heads, int group,
                                                           uint32_t* __restrict__ aux, int aux_cap, float est_cv,
                                                           float est_co, int64_t row_pos0) {
  constexpr int V4 = HD / 4;
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows_heads * V4) return;  // whole rows only: rows_heads * V4 is a multiple of V4, and V4 divides 256
  const int64_t rh = i / V4;
  const int c4 = int(i % V4);
  const float* ml = ws_ml + rh * n_split * kSplitRec;
  const float4* po = reinterpret_cast<const float4*>(ws_o + rh * n_split * HD) + c4;
  float2 ml01[SPM], ml23[SPM];  // (shift, sum), (sum of squared weights, score coefficient)
  float2 ml45[SPM];             // (largest |v|^2, query residual coefficient)
  float4 o[SPM];
#pragma unroll
  for (int sp = 0; sp < SPM; ++sp) {
    ml01[sp] = make_float2(-INFINITY, 0.f);
    ml23[sp] = make_float2(0.f, 0.f);
    ml45[sp] = make_float2(0.f, 0.f);
    o[sp] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (sp < n_split) {
      const float* rec = ml + kSplitRec * sp;
      ml01[sp] = *reinterpret_cast<const float2*>(rec);
      ml23[sp] = *reinterpret_cast<const float2*>(rec + 2);
      ml45[sp] = *reinterpret_cast<const float2*>(rec + 4);
      o[sp] = po[int64_t(sp) * V4];
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int sp = 0; sp < SPM; ++sp) mx = fmaxf(mx, ml01[sp].x);
  const float ms = mx == -INFINITY ? 0.0f : mx;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float l = 0.f, l2 = 0.f, a = 0.f, b = 0.f, rk = 0.f;
#pragma unroll
  for (int sp = 0; sp < SPM; ++sp) {
    const float w = sp < n_split ? exp2_raw(ml01[sp].x - ms) : 0.f;  // the missing splits' partials are zeros
    acc.x += o[sp].x * w;
    acc.y += o[sp].y * w;
    acc.z += o[sp].z * w;
    acc.w += o[sp].w * w;
    l += ml01[sp].y * w;
    if (ml01[sp].y > 0.f) {  // splits that saw keys (the others' records are not written)
      l2 += ml23[sp].x * w * w;
      a = fmaxf(a, ml23[sp].y);
      b = fmaxf(b, ml45[sp].x);
      rk = fmaxf(rk, ml45[sp].y);
    }
  }
  const float inv = 1.0f / l;
  const float4 r = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
  reinterpret_cast<float4*>(out + rh * HD)[c4] = r;
  float om = fmaxf(fmaxf(fabsf(r.x), fabsf(r.y)), fmaxf(fabsf(r.z), fabsf(r.w)));
#pragma unroll
  for (int m = 1; m < V4; m <<= 1) om = fmaxf(om, __shfl_xor(om, m, 64));  // over the row's V4 lanes
  const float om2 = om * om;
  const float est = l2 * inv * inv * (a * (b + om2) + est_cv * b + est_co * om2);
  const int64_t t = rh / n_heads;
  const bool flat = l2 * float(row_pos0 + t + 1) <= l * l * (1.0f + kFlatTol);  // see kFlatTol
  if (c4 == 0 && l > 0.f && (flat || !(sqrtf(est) + rk * (sqrtf(b) + om) <= 1.0f))) {
    const int head = int(rh % n_heads), g = head / group;
    const int64_t p = t * group + head % group;
    const uint32_t ep = aux[1], slot = uint32_t(p / kRowsPerBlock) * uint32_t(n_heads / group) + uint32_t(g);
    if (atomicExch(&aux[kAuxHead + slot], ep) != ep) aux[kAuxHead + aux_cap + atomicAdd(&aux[0], 1u)] = slot;
  }
}

// The merge instantiation whose register window holds n_split (at most 16) splits.
template <int HD>
auto split_merge_for(int n_split) {
  return n_split <= 4 ? prefill_split_merge<HD, 4> : n_split <= 8 ? prefill_split_merge<HD, 8>
                                                                   : prefill_split_merge<HD, 16>;
}

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Key splits per row tile for a launch of n_mfma MFMA rows at positions pos0..: 1 when the row tiles alone fill
// the workgroup slots of the chip (3 per CU at head_dim 64, 2 at 128), otherwise enough to fill them, at most 16
// and keeping at least two key tiles per split. Short prefill chunks - nibble's Transformer runs a prompt in
// chunks of max_batch = 512 rows - would otherwise leave most CUs idle.
int prefill_splits(int64_t n_mfma, int64_t pos0, int64_t group, int64_t n_kv, int64_t head_dim, int cu_count) {
  const int64_t tiles = (n_mfma * group + kRowsPerBlock - 1) / kRowsPerBlock;
  const int64_t blocks = tiles * n_kv;
  // two workgroups per CU: a chunk of 512 rows at Llama-3.2 shape then splits its keys 4 ways rather than 6, and
  // the fewer, longer splits write and merge a third fewer partials for the same work (measured 3 % faster per call)
  const int64_t target = int64_t(cu_count > 0 ? cu_count : 256) * 2;
  if (blocks >= target) return 1;
  const int64_t key_tiles = (pos0 + n_mfma + kBN - 1) / kBN;  // the longest row tile's
  int64_t sp = (target + blocks - 1) / blocks;
  sp = std::min<int64_t>(sp, std::min<int64_t>(16, std::max<int64_t>(1, key_tiles / 2)));
  return int(std::max<int64_t>(1, sp));
}

}  // namespace

extern "C" {

int64_t nbhs_prefill_staging_halves(int64_t rows, int64_t n_kv_heads, int64_t head_dim) {
  if (rows < 0 || n_kv_heads <= 0 || head_dim <= 0) return -1;
  // the operands, then (in the V^T buffer) one float2 of statistics per (KV head, 64-row tile)
  const int64_t rows_pad = round_up(rows, kBN);
  return n_kv_heads * rows_pad * head_dim + n_kv_heads * (rows_pad / kBN) * 4;
}

int64_t nbhs_prefill_aux_words(int64_t n, int64_t n_heads, int64_t n_kv_heads) {
  if (n <= 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0) return -1;
  const int64_t tiles = (n * (n_heads / n_kv_heads) + kRowsPerBlock - 1) / kRowsPerBlock;
  return kAuxHead + 3 * tiles * n_kv_heads;
}

int64_t nbhs_prefill_aux_words_bound(int64_t max_rows, int64_t n_heads) {
  if (max_rows <= 0 || n_heads <= 0) return -1;
  // n_kv ceil(m G / 128) tiles, G = n_heads / n_kv: not monotone in n_kv (the rounding), so every divisor is tried;
  // it is monotone in m
  int64_t words = 0;
  for (int64_t kv = 1; kv <= n_heads; ++kv)
    if (n_heads % kv == 0) words = std::max(words, nbhs_prefill_aux_words(max_rows, n_heads, kv));
  return words;
}

namespace {
float2* stats_of(void* vt16, int64_t rows_pad, int64_t n_kv, int64_t head_dim) {
  return reinterpret_cast<float2*>(static_cast<_Float16*>(vt16) + n_kv * rows_pad * head_dim);
}
// list entries a work-list buffer of aux_words words holds (its layout follows this capacity)
int aux_cap_of(int64_t aux_words) { return aux_words > kAuxHead ? int((aux_words - kAuxHead) / 3) : 0; }
}  // namespace

}  // extern "C"

namespace {

template <typename KVT>
int stage_impl(const KVT* k, const KVT* v, void* k16, void* vt16, int64_t rows, int64_t n_kv_heads,
               int64_t head_dim, uint32_t* aux, int64_t aux_words, hipStream_t s) {
  if (!k || !v || !k16 || !vt16 || rows <= 0 || n_kv_heads <= 0 || n_kv_heads > 65535 ||
      (head_dim != 64 && head_dim != 128))
    return NBHS_EINVAL;
  const int64_t rows_pad = round_up(rows, kBN);
  const dim3 grid(unsigned(rows_pad / kBN), unsigned(n_kv_heads));
  // read-only use of the cache: no new rows (kn = vn = NULL), so ck/cv are only read
  return nbhs_timing::launch(NBHS_K_STAGE_KV, head_dim == 64 ? stage_kv_kernel<64, KVT> : stage_kv_kernel<128, KVT>,
                             grid, dim3(256), s, const_cast<KVT*>(k), const_cast<KVT*>(v),
                             static_cast<const float*>(nullptr), static_cast<const float*>(nullptr),
                             static_cast<_Float16*>(k16), static_cast<_Float16*>(vt16), rows, rows, rows_pad,
                             int(n_kv_heads), static_cast<const float2*>(nullptr), 0,
                             stats_of(vt16, rows_pad, n_kv_heads, head_dim), aux, aux_cap_of(aux_words));
}

template <typename KVT>
int append_stage_impl(KVT* cache_k, KVT* cache_v, const float* k_new, const float* v_new, int64_t n, int64_t pos0,
                      int64_t n_kv_heads, int64_t head_dim, const float* cs_table, int64_t table_rows, int neox,
                      void* k16, void* vt16, uint32_t* aux, int64_t aux_words, hipStream_t s) {
  if (!cache_k || !cache_v || !k_new || !v_new || !cs_table || !k16 || !vt16 || n <= 0 || pos0 < 0 ||
      n_kv_heads <= 0 || n_kv_heads > 65535 || (head_dim != 64 && head_dim != 128) || pos0 + n > table_rows)
    return NBHS_EINVAL;
  const int64_t rows = pos0 + n, rows_pad = round_up(rows, kBN);
  const dim3 grid(unsigned(rows_pad / kBN), unsigned(n_kv_heads));
  return nbhs_timing::launch(NBHS_K_STAGE_KV, head_dim == 64 ? stage_kv_kernel<64, KVT> : stage_kv_kernel<128, KVT>,
                             grid, dim3(256), s, cache_k, cache_v, k_new, v_new, static_cast<_Float16*>(k16),
                             static_cast<_Float16*>(vt16), pos0, rows, rows_pad, int(n_kv_heads),
                             reinterpret_cast<const float2*>(cs_table), neox,
                             stats_of(vt16, rows_pad, n_kv_heads, head_dim), aux, aux_cap_of(aux_words));
}

}  // namespace

extern "C" {

int nbhs_stage_kv_f16(const float* k, const float* v, void* k16, void* vt16, int64_t rows, int64_t n_kv_heads,
                      int64_t head_dim, uint32_t* aux, int64_t aux_words, nbhs_stream stream) {
  return stage_impl(k, v, k16, vt16, rows, n_kv_heads, head_dim, aux, aux_words,
                    reinterpret_cast<hipStream_t>(stream));
}

int nbhs_stage_kv_f16kv(const void* k_cache16, const void* v_cache16, void* k16, void* vt16, int64_t rows,
                        int64_t n_kv_heads, int64_t head_dim, uint32_t* aux, int64_t aux_words, nbhs_stream stream) {
  return stage_impl(static_cast<const _Float16*>(k_cache16), static_cast<const _Float16*>(v_cache16), k16, vt16, rows,
                    n_kv_heads, head_dim, aux, aux_words, reinterpret_cast<hipStream_t>(stream));
}

int nbhs_append_stage_kv_f16(float* cache_k, float* cache_v, const float* k_new, const float* v_new, int64_t n,
                             int64_t pos0, int64_t n_kv_heads, int64_t head_dim, const float* cs_table,
                             int64_t table_rows, int neox, void* k16, void* vt16, uint32_t* aux,
                             int64_t aux_words, nbhs_stream stream) {
  return append_stage_impl(cache_k, cache_v, k_new, v_new, n, pos0, n_kv_heads, head_dim, cs_table, table_rows, neox,
                           k16, vt16, aux, aux_words, reinterpret_cast<hipStream_t>(stream));
}

int nbhs_append_stage_kv_f16kv(void* k_cache16, void* v_cache16, const float* k_new, const float* v_new, int64_t n,
                               int64_t pos0, int64_t n_kv_heads, int64_t head_dim, const float* cs_table,
                               int64_t table_rows, int neox, void* k16, void* vt16, uint32_t* aux,
                               int64_t aux_words, nbhs_stream stream) {
  return append_stage_impl(static_cast<_Float16*>(k_cache16), static_cast<_Float16*>(v_cache16), k_new, v_new, n,
                           pos0, n_kv_heads, head_dim, cs_table, table_rows, neox, k16, vt16, aux, aux_words,
                           reinterpret_cast<hipStream_t>(stream));
}

int64_t nbhs_attn_prefill_workspace_bound(int cu_count) {
  // A split is taken only when blocks = tiles * KV < target, with sp <= ceil(target / blocks) and
  // n_mfma <= 128 tiles / G, so n_mfma * n_heads * sp < 256 target: the bound is 256 target (head_dim + kSplitRec)
  // at the larger head size (target 2 workgroups per CU).
  const int64_t cus = cu_count > 0 ? cu_count : 256;
  return 256 * 2 * cus * (128 + kSplitRec);
}

int64_t nbhs_attn_prefill_workspace(int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                    int64_t fp32_rows, int cu_count) {
  if (n <= 0 || pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || fp32_rows < 0 ||
      fp32_rows >= n || (head_dim != 64 && head_dim != 128))
    return -1;
  const int64_t n_mfma = n - fp32_rows;
  const int sp = prefill_splits(n_mfma, pos0 + fp32_rows, n_heads / n_kv_heads, n_kv_heads, head_dim, cu_count);
  return sp == 1 ? 0 : n_mfma * n_heads * sp * (head_dim + kSplitRec);
}

}  // extern "C"

namespace {
template <typename KVT>
int prefill_impl(const float* q, const void* k16, const void* vt16, float* out, int64_t n, int64_t pos0,
                 int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t staged_rows_pad,
                 const float* q_rope_cs, int64_t q_rope_rows, int q_rope_neox, const KVT* k_cache, const KVT* v_cache,
                 int64_t fp32_rows, float* workspace, int64_t workspace_floats, uint32_t* aux, int64_t aux_words,
                 int cu_count, hipStream_t s) {
  if (!q || !k16 || !vt16 || !out || !k_cache || !v_cache || !aux || n <= 0 || pos0 < 0 || n_heads <= 0 ||
      n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || (head_dim != 64 && head_dim != 128) ||
      staged_rows_pad % kBN != 0 || staged_rows_pad < round_up(pos0 + n, kBN) || (q_rope_cs && pos0 + n > q_rope_rows) ||
      fp32_rows < 0 || fp32_rows >= n)
    return NBHS_EINVAL;
  // the kernel reads each KV head's staged K and V^T through buffer resources with a 32-bit byte size
  if (staged_rows_pad * head_dim * 2 > int64_t(INT32_MAX)) return NBHS_EINVAL;
  const int64_t group = n_heads / n_kv_heads;
  const int64_t n_mfma = n - fp32_rows;
  const int64_t tiles = (n_mfma * group + kRowsPerBlock - 1) / kRowsPerBlock;
  // the work list's layout follows the buffer's capacity (stable across calls), which must hold every row tile
  const int64_t aux_cap = aux_cap_of(aux_words);
  if (aux_cap < tiles * n_kv_heads || aux_words > int64_t(1) << 30) return NBHS_EINVAL;
  const int sp = prefill_splits(n_mfma, pos0 + fp32_rows, group, n_kv_heads, head_dim, cu_count);
  if (sp > 16) return NBHS_EINVAL;  // the split merge holds at most 16 splits in registers
  const int64_t need = sp == 1 ? 0 : n_mfma * n_heads * sp * (head_dim + kSplitRec);
  if (need > 0 && (!workspace || workspace_floats < need)) return NBHS_EINVAL;
  float* ws_o = need > 0 ? workspace : nullptr;
  float* ws_ml = need > 0 ? workspace + n_mfma * n_heads * sp * head_dim : nullptr;  // kSplitRec floats per split
  const int64_t fp32_sub = (group + 3) / 4;  // head subgroups of the fp32 rows' workgroups (4 query heads each)
  const int64_t blocks = tiles * n_kv_heads * sp + fp32_rows * n_kv_heads * fp32_sub;
  if (blocks >= int64_t(1) << 31) return NBHS_EINVAL;
  const float qscale = (1.0f / std::sqrt(float(head_dim))) * kLog2e;
  const int64_t off = fp32_rows * n_heads * head_dim;  // the MFMA rows start fp32_rows rows in
  const float2* kstats = stats_of(const_cast<void*>(vt16), staged_rows_pad, n_kv_heads, head_dim);
  // error-estimate coefficients, with the acceptance test folded in: flag when
  // sqrt(var * Z^2 / budget^2) + (ln2 / budget) |r| sqrt(K) (V + O) > 1
  const double u2 = kEstU * kEstU, zb = double(kEstZ) * kEstZ / (double(kEstBudget) * kEstBudget);
  // Per unit variance of a rounding (u^2 / 3 to nearest, u^2 stochastic): an fp32 cache's K and V are staged with
  // stochastic rounding (score term 2 ln2^2 u^2 (|y|^2/d) K (V^2 + O^2), V's own rounding u^2 V^2); an fp16 cache's
  // are staged exactly, leaving the weights' rounding alone, (u^2/3) 2 (V^2 + O^2).
  constexpr bool kRoundedKV = sizeof(KVT) == 4;
  const float est_c1 = kRoundedKV ? float(2.0 * kLn2 * kLn2 * u2 * zb) : 0.f;
  const float est_cv = float((kRoundedKV ? 5.0 : 2.0) * u2 / 3.0 * zb), est_co = float(2.0 * u2 / 3.0 * zb);
  const float est_c3 = float(kLn2 / kEstBudget);
  const float2* q_rope = reinterpret_cast<const float2*>(q_rope_cs);
  hipError_t e = nbhs_timing::launch(
      NBHS_K_PREFILL_MFMA, head_dim == 64 ? attn_prefill_kernel<64, KVT> : attn_prefill_kernel<128, KVT>,
      dim3(unsigned(blocks)),
      dim3(kWaves * 64), s, q + off, static_cast<const _Float16*>(k16), static_cast<const _Float16*>(vt16), out + off,
      n_mfma, pos0 + fp32_rows, int(n_heads), int(n_kv_heads), int(group), staged_rows_pad, int(tiles), qscale,
      q_rope, q_rope_neox, k_cache, v_cache, fp32_rows, int(fp32_sub), sp, ws_o, ws_ml, kstats, aux, int(aux_cap),
      est_c1, est_cv, est_co, est_c3);
  if (e != hipSuccess) return e;
  if (sp > 1) {
    const int64_t threads = n_mfma * n_heads * (head_dim / 4);
    e = nbhs_timing::launch(NBHS_K_DECODE_COMBINE, head_dim == 64 ? split_merge_for<64>(sp) : split_merge_for<128>(sp),
                            dim3(unsigned((threads + 255) / 256)), dim3(256), s, ws_o, ws_ml, out + off,
                            n_mfma * n_heads, sp, int(n_heads), int(group), aux, int(aux_cap), est_cv,
                            est_co, pos0 + fp32_rows);
    if (e != hipSuccess) return e;
  }
  // The listed row tiles, recomputed with split operands (a persistent launch; nothing to do when none was listed).
  // Key-range partials use the workspace, whose split partials the merge above has consumed.
  const int64_t grid = std::min<int64_t>(tiles * n_kv_heads * kPreciseMaxRanges,
                                         int64_t(cu_count > 0 ? cu_count : 256) * NBH_PRECISE_WG_PER_CU);
  return nbhs_timing::launch(NBHS_K_PREFILL_PRECISE,
                             head_dim == 64 ? attn_prefill_precise_kernel<64, KVT> : attn_prefill_precise_kernel<128, KVT>,
                             dim3(unsigned(grid)), dim3(kWaves * 64), s, q + off, k_cache, v_cache, out + off, n_mfma,
                             pos0 + fp32_rows, int(n_heads), int(n_kv_heads), int(group), qscale, q_rope, q_rope_neox,
                             aux, int(aux_cap), workspace, workspace ? workspace_floats : int64_t(0));
}

}  // namespace

extern "C" {

int nbhs_attn_prefill_mfma(const float* q, const void* k16, const void* vt16, float* out, int64_t n, int64_t pos0,
                           int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t staged_rows_pad,
                           const float* q_rope_cs, int64_t q_rope_rows, int q_rope_neox, const float* k_cache,
                           const float* v_cache, int64_t fp32_rows, float* workspace, int64_t workspace_floats,
                           uint32_t* aux, int64_t aux_words, int cu_count, nbhs_stream stream) {
  return prefill_impl(q, k16, vt16, out, n, pos0, n_heads, n_kv_heads, head_dim, staged_rows_pad, q_rope_cs,
                      q_rope_rows, q_rope_neox, k_cache, v_cache, fp32_rows, workspace, workspace_floats, aux,
                      aux_words, cu_count, reinterpret_cast<hipStream_t>(stream));
}

int nbhs_attn_prefill_mfma_f16kv(const float* q, const void* k16, const void* vt16, float* out, int64_t n,
                                 int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                 int64_t staged_rows_pad, const float* q_rope_cs, int64_t q_rope_rows, int q_rope_neox,
                                 const void* k_cache16, const void* v_cache16, int64_t fp32_rows, float* workspace,
                                 int64_t workspace_floats, uint32_t* aux, int64_t aux_words, int cu_count,
                                 nbhs_stream stream) {
  return prefill_impl(q, k16, vt16, out, n, pos0, n_heads, n_kv_heads, head_dim, staged_rows_pad, q_rope_cs,
                      q_rope_rows, q_rope_neox, static_cast<const _Float16*>(k_cache16),
                      static_cast<const _Float16*>(v_cache16), fp32_rows, workspace, workspace_floats, aux, aux_words,
                      cu_count, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
