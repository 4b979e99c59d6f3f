// Causal GQA prefill attention on gfx950 MFMA: Backend::attention (backend.h:68-69) for many query rows,
// semantics of ref_ops.cpp:188-214 (row t attends to cache rows 0..pos0+t; head h reads KV head h/(H/KV)).
//
// Numerics: Q is scaled by log2(e)/sqrt(d) and rounded to fp16, K and V come from fp16 copies of the fp32 cache
// (stage_kv), QK^T and PV run on v_mfma_f32_32x32x16_f16 with fp32 accumulation, and the online softmax (shift,
// exp2, running sums, rescaling) is fp32. The softmax shift is not the running max: it is set from the first tile
// and raised only when a tile's weights outgrow it (checked through their sum, see kPSumMax), so the per-tile
// max, the subtraction (folded into the MFMA accumulator init) and the O rescale all leave the common path; the
// result is the same normalised softmax, since any shift cancels. The host routes rows with fewer than 256
// visible keys to the fp32 decode kernel, where fp16 rounding of a few V rows is not averaged away.
//
// Layout (per wave, 32 query rows):
//  * S^T = K Q^T: A = K tile rows from LDS ([key][d], 16 B per lane), B = the wave's Q fragment held in
//    registers for the whole pass. The accumulator puts one query per lane column (lane % 32) and 16 keys per
//    lane, so the row max needs one cross-half shuffle and the running (m, l) are per-lane scalars.
//  * O^T = V^T P^T: B = P straight from the S^T accumulator registers (converted to fp16), A = V^T from LDS
//    ([d][key]), with the key order inside each 16-key MFMA step permuted identically on both operands to match
//    the accumulator's row interleave. O^T keeps one query per lane too, so rescaling O is a per-lane multiply.
//  * GQA packing: the G query heads sharing a KV head are interleaved into the row dimension (packed row
//    p = t*G + head), so a workgroup's 128 rows span only 128/G positions and each K/V tile in LDS serves all G
//    heads.
//  * Scheduling: workgroup b takes KV head b % KV and row tiles from the longest (last) to the shortest, so
//    long causal rows start first and, with workgroups dispatched round-robin over the 8 XCDs, one KV head's
//    tiles stay in one XCD's L2.
#include <hip/hip_runtime.h>

#include <cmath>

#include "backend/hip/kernel_timing.h"
#include "nibble_hip_shim.h"

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kBN = 64;          // keys per tile
constexpr int kRowsPerWave = 32;
#ifndef NBH_PREFILL_WAVES
#define NBH_PREFILL_WAVES 4
#endif
constexpr int kWaves = NBH_PREFILL_WAVES;
constexpr int kRowsPerBlock = kRowsPerWave * kWaves;
constexpr int kPad = 8;          // halves of LDS row padding (keeps rows 16-byte aligned, spreads banks)
// Largest sum of one lane's 32 tile weights accepted without recomputing the tile against a raised shift: every
// weight is then <= 2^12, far inside fp16 (max 65504).
constexpr float kPSumMax = 4096.0f;

__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }  // v_exp_f32; -inf -> 0

// ---- staging: fp32 cache rows -> fp16 K [KV][rows_pad][HD] and transposed V [KV][HD][rows_pad] ----
template <int HD>
__global__ __launch_bounds__(256) void stage_kv_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                       _Float16* __restrict__ k16, _Float16* __restrict__ vt16,
                                                       int64_t rows, int64_t rows_pad, int n_kv) {
  __shared__ _Float16 tr[HD][kBN + kPad];
  const int g = blockIdx.y;
  const int64_t r0 = int64_t(blockIdx.x) * kBN;
  // K: straight conversion, 4 floats per thread step.
  for (int idx = threadIdx.x; idx < kBN * HD / 4; idx += 256) {
    const int r = idx / (HD / 4), d4 = idx % (HD / 4);
    const int64_t row = r0 + r;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f), y = x;
    if (row < rows) {
      x = *reinterpret_cast<const float4*>(k + (row * n_kv + g) * HD + 4 * d4);
      y = *reinterpret_cast<const float4*>(v + (row * n_kv + g) * HD + 4 * d4);
    }
    half4_t hk = {(_Float16)x.x, (_Float16)x.y, (_Float16)x.z, (_Float16)x.w};
    *reinterpret_cast<half4_t*>(k16 + (int64_t(g) * rows_pad + row) * HD + 4 * d4) = hk;
    tr[4 * d4 + 0][r] = (_Float16)y.x;
    tr[4 * d4 + 1][r] = (_Float16)y.y;
    tr[4 * d4 + 2][r] = (_Float16)y.z;
    tr[4 * d4 + 3][r] = (_Float16)y.w;
  }
  __syncthreads();
  // V^T: each d row of the tile is 64 consecutive keys (128 B).
  for (int idx = threadIdx.x; idx < HD * kBN / 8; idx += 256) {
    const int d = idx / (kBN / 8), c8 = idx % (kBN / 8);
    *reinterpret_cast<half8_t*>(vt16 + (int64_t(g) * HD + d) * rows_pad + r0 + 8 * c8) =
        *reinterpret_cast<const half8_t*>(&tr[d][8 * c8]);
  }
}

// Occupancy cap (waves per SIMD) the register allocator plans for. The kernel is built with MFMA accumulators in
// architectural VGPRs (-amdgpu-mfma-vgpr-form, see the Makefile), so the S^T and O^T accumulators both stay
// resident with no per-tile copies through accumulation registers; head_dim 64 fits 3 waves per SIMD.
#ifndef NBH_PREFILL_WAVES_PER_EU
#define NBH_PREFILL_WAVES_PER_EU 3
#endif
#ifndef NBH_PREFILL_MIN_WAVES_PER_EU
#define NBH_PREFILL_MIN_WAVES_PER_EU 1
#endif
template <int HD>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(NBH_PREFILL_MIN_WAVES_PER_EU, NBH_PREFILL_WAVES_PER_EU)))
void attn_prefill_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ k16, const _Float16* __restrict__ vt16,
    float* __restrict__ out, int64_t n, int64_t pos0, int n_heads, int n_kv, int group, int64_t rows_pad,
    int n_tiles, float qscale) {
  constexpr int DC = HD / 16;  // 16-wide d chunks of the S^T contraction
  constexpr int DT = HD / 32;  // 32-row d tiles of O^T
  // Row strides (halves). K rows are read 16 B per lane, 36 dwords apart: 8 (or 16) consecutive rows cover
  // distinct 4-bank groups. V^T rows are read 8 B per lane, 34 dwords apart: 17 is odd, so any 16 (or 32)
  // consecutive rows land on distinct even bank pairs - a 36-dword stride would put rows r and r + 8 on the same
  // banks and serialise half of every V read.
  constexpr int KLD = HD + kPad;
  constexpr int VLD = kBN + 4;
  constexpr int K_VECS = kBN * HD / 8;  // 16-byte vectors per K tile
  constexpr int V_VECS = HD * kBN / 8;
  constexpr int THREADS = kWaves * 64;
  constexpr int K_PER_T = K_VECS / THREADS;
  constexpr int V_PER_T = V_VECS / THREADS;
  __shared__ _Float16 ks[2][kBN][KLD];
  __shared__ _Float16 vs[2][HD][VLD];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ql = lane & 31, hf = lane >> 5;
  const int b = blockIdx.x;
  const int g = b % n_kv;
  const int tile = n_tiles - 1 - b / n_kv;
  const int64_t P = n * group;
  const int64_t pb0 = int64_t(tile) * kRowsPerBlock;
  const int64_t wp0 = pb0 + wave * kRowsPerWave;
  const int64_t p = wp0 + ql;
  const bool active = p < P;
  const int64_t t = active ? p / group : 0;
  const int head = g * group + (active ? int(p % group) : 0);
  const int64_t qpos = pos0 + t;

  const int64_t p_last = min(pb0 + kRowsPerBlock, P) - 1;
  const int64_t kend = pos0 + p_last / group + 1;  // the block's keys: [0, kend)
  const int ntk = int((kend + kBN - 1) / kBN);
  const bool wave_active = wp0 < P;
  const int64_t wave_kend = wave_active ? pos0 + (min(wp0 + kRowsPerWave, P) - 1) / group + 1 : 0;
  const int64_t wave_kfull = wave_active ? pos0 + wp0 / group + 1 : 0;  // keys every row of the wave sees

  // Q fragment (B operand of S^T): query ql, d = 16c + 8hf .. +8.
  half8_t qf[DC];
  {
    const float* qrow = q + (t * n_heads + head) * HD;
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f), bb = a;
      if (active) {
        a = *reinterpret_cast<const float4*>(qrow + 16 * c + 8 * hf);
        bb = *reinterpret_cast<const float4*>(qrow + 16 * c + 8 * hf + 4);
      }
      qf[c] = half8_t{(_Float16)(a.x * qscale), (_Float16)(a.y * qscale), (_Float16)(a.z * qscale),
                      (_Float16)(a.w * qscale), (_Float16)(bb.x * qscale), (_Float16)(bb.y * qscale),
                      (_Float16)(bb.z * qscale), (_Float16)(bb.w * qscale)};
    }
  }

  floatx16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
  // m_sh: the query's softmax shift (log2 domain); mneg: 16 copies of -m_sh, the accumulator block S^T starts from.
  float m_sh = 0.f, l_run = 0.f;
  floatx16 mneg;
#pragma unroll
  for (int r = 0; r < 16; ++r) mneg[r] = 0.f;

  const _Float16* kg = k16 + int64_t(g) * rows_pad * HD;
  const _Float16* vg = vt16 + int64_t(g) * HD * rows_pad;
  half8_t kreg[K_PER_T], vreg[V_PER_T];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < K_PER_T; ++i) {
      const int ci = threadIdx.x + THREADS * i;
      kreg[i] = *reinterpret_cast<const half8_t*>(kg + (int64_t(kt) * kBN) * HD + int64_t(ci) * 8);
    }
#pragma unroll
    for (int i = 0; i < V_PER_T; ++i) {
      const int ci = threadIdx.x + THREADS * i;
      const int d = ci / (kBN / 8), c8 = ci % (kBN / 8);
      vreg[i] = *reinterpret_cast<const half8_t*>(vg + int64_t(d) * rows_pad + int64_t(kt) * kBN + 8 * c8);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < K_PER_T; ++i) {
      const int ci = threadIdx.x + THREADS * i;
      const int r = ci / (HD / 8), c8 = ci % (HD / 8);
      *reinterpret_cast<half8_t*>(&ks[buf][r][8 * c8]) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < V_PER_T; ++i) {
      const int ci = threadIdx.x + THREADS * i;
      const int d = ci / (kBN / 8), c8 = ci % (kBN / 8);
      // V^T rows are 8-byte aligned (VLD = 68 halves): two 8-byte stores
      *reinterpret_cast<half4_t*>(&vs[buf][d][8 * c8]) = half4_t{vreg[i][0], vreg[i][1], vreg[i][2], vreg[i][3]};
      *reinterpret_cast<half4_t*>(&vs[buf][d][8 * c8 + 4]) = half4_t{vreg[i][4], vreg[i][5], vreg[i][6], vreg[i][7]};
    }
  };

  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int kt = 0; kt < ntk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ntk) load_tile(kt + 1);
    if (wave_active && int64_t(kt) * kBN < wave_kend) {
      // S^T - m for the tile's two 32-key halves: the first MFMA of each chain starts from the accumulator block
      // mneg (every entry -m_sh, the lane's query shift), so the subtraction costs no instruction. The two chains
      // are interleaved so consecutive MFMAs do not wait on each other's results.
      floatx16 s[2];
#pragma unroll
      for (int c = 0; c < DC; ++c)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const half8_t a = *reinterpret_cast<const half8_t*>(&ks[cur][kk * 32 + ql][16 * c + 8 * hf]);
          s[kk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[c], c == 0 ? mneg : s[kk], 0, 0, 0);
        }
      // Causal mask (and inactive rows) only where some key of the tile lies past the wave's first row.
      if (int64_t(kt) * kBN + kBN > wave_kfull) {
        // keys of this tile past the query's position (relative to the tile start; inactive rows mask all)
        const int64_t rel64 = active ? qpos - int64_t(kt) * kBN : -1;
        const int rel = int(rel64 < kBN ? rel64 : kBN);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (kk * 32 + 8 * (r / 4) + 4 * hf + (r % 4) > rel) s[kk][r] = -INFINITY;
      }
      // P = exp2(S - m_sh) in fp16 (the MFMA B operand) and the lane's sum of it, taken from the same fp16 values
      // with v_dot2 so the normaliser matches the weights the MFMA multiplies.
      half8_t pb[4];
      float l_tile = 0.f;
      const half2_t ones = {(_Float16)1.0f, (_Float16)1.0f};
      auto exps = [&](float shift) {
        l_tile = 0.f;
#pragma unroll
        for (int kc = 0; kc < 4; ++kc)
#pragma unroll
          for (int e = 0; e < 8; ++e) pb[kc][e] = (_Float16)exp2_raw(s[kc >> 1][8 * (kc & 1) + e] - shift);
#pragma unroll
        for (int kc = 0; kc < 4; ++kc)
#pragma unroll
          for (int e = 0; e < 8; e += 2)
            l_tile = __builtin_amdgcn_fdot2(half2_t{pb[kc][e], pb[kc][e + 1]}, ones, l_tile, false);
      };
      // The shift is not raised per tile: the weights are computed against the current one, and only when some
      // lane's sum leaves (0, kPSumMax] - a score grew past the shift by ~12 (log2), or inf/NaN from an fp16
      // overflow - does the wave take the slow path below (always on its first tile, where no shift exists yet).
      bool slow = kt == 0;
      if (!slow) {
        exps(0.0f);
        slow = __builtin_amdgcn_ballot_w64(!(l_tile <= kPSumMax)) != 0;
      }
      if (slow) {
        float mt = -INFINITY;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[kk][r]);
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        // first tile: shift to the tile max (0 if every key is masked); later: raise by the excess only
        const float d = kt == 0 ? (mt == -INFINITY ? 0.0f : mt) : fmaxf(mt, 0.0f);
        exps(d);
        if (kt != 0) {
          const float corr = exp2_raw(-d);
          l_run *= corr;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[dt][r] *= corr;
        }
        m_sh += d;
#pragma unroll
        for (int r = 0; r < 16; ++r) mneg[r] = -m_sh;
      }
      l_run += l_tile;
      // O^T += V^T P^T over 4 steps of 16 keys; the DT output tiles are independent chains.
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const _Float16* vrow = &vs[cur][32 * dt + ql][16 * kc + 4 * hf];
          const half4_t lo = *reinterpret_cast<const half4_t*>(vrow);
          const half4_t hi = *reinterpret_cast<const half4_t*>(vrow + 8);
          const half8_t a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[kc], oacc[dt], 0, 0, 0);
        }
      }
    }
    if (kt + 1 < ntk) store_tile(cur ^ 1);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
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
}

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

}  // namespace

extern "C" {

int64_t nbhs_prefill_staging_halves(int64_t rows, int64_t n_kv_heads, int64_t head_dim) {
  if (rows < 0 || n_kv_heads <= 0 || head_dim <= 0) return -1;
  return n_kv_heads * round_up(rows, kBN) * head_dim;
}

int nbhs_stage_kv_f16(const float* k, const float* v, void* k16, void* vt16, int64_t rows, int64_t n_kv_heads,
                      int64_t head_dim, nbhs_stream stream) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (!k || !v || !k16 || !vt16 || rows <= 0 || n_kv_heads <= 0 || n_kv_heads > 65535 ||
      (head_dim != 64 && head_dim != 128))
    return NBHS_EINVAL;
  const int64_t rows_pad = round_up(rows, kBN);
  const dim3 grid(unsigned(rows_pad / kBN), unsigned(n_kv_heads));
  auto* const kh = static_cast<_Float16*>(k16);
  auto* const vh = static_cast<_Float16*>(vt16);
  return nbhs_timing::launch(NBHS_K_STAGE_KV, head_dim == 64 ? stage_kv_kernel<64> : stage_kv_kernel<128>, grid,
                             dim3(256), s, k, v, kh, vh, rows, rows_pad, int(n_kv_heads));
}

int nbhs_attn_prefill_mfma(const float* q, const void* k16, const void* vt16, float* out, int64_t n, int64_t pos0,
                           int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t staged_rows_pad,
                           nbhs_stream stream) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (!q || !k16 || !vt16 || !out || n <= 0 || pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 ||
      n_heads % n_kv_heads != 0 || (head_dim != 64 && head_dim != 128) || staged_rows_pad % kBN != 0 ||
      staged_rows_pad < round_up(pos0 + n, kBN))
    return NBHS_EINVAL;
  const int64_t group = n_heads / n_kv_heads;
  const int64_t tiles = (n * group + kRowsPerBlock - 1) / kRowsPerBlock;
  if (tiles * n_kv_heads > int64_t(1) << 31) return NBHS_EINVAL;
  const float qscale = (1.0f / std::sqrt(float(head_dim))) * kLog2e;
  const unsigned blocks = unsigned(tiles * n_kv_heads);
  return nbhs_timing::launch(NBHS_K_PREFILL_MFMA, head_dim == 64 ? attn_prefill_kernel<64> : attn_prefill_kernel<128>,
                             dim3(blocks), dim3(kWaves * 64), s, q, static_cast<const _Float16*>(k16),
                             static_cast<const _Float16*>(vt16), out, n, pos0, int(n_heads), int(n_kv_heads),
                             int(group), staged_rows_pad, int(tiles), qscale);
}

}  // extern "C"
