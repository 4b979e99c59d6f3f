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

__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }  // v_exp_f32; -inf -> 0

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

// s_waitcnt immediate that waits for at most n outstanding vector-memory loads and nothing else (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int vmcnt_wait(int n) { return (n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14); }

// The S^T accumulator gives lane (query, half hf) the 8 keys {4hf .. 4hf+3, 8+4hf .. 8+4hf+3} of each 16-key step,
// and that register order is the B operand (P) of the PV MFMA, so its A operand (V^T) must hold the same keys at
// k = 8hf + e. Staged V^T rows store each 16-key group as keys [0-3, 8-11, 4-7, 12-15]: a lane's 8 keys are then
// 16 consecutive bytes. vt_key(p) is the key stored at position p of a 64-key tile row.
__device__ __forceinline__ int vt_key(int p) { return (p & ~15) + (p & 3) + ((p >> 2) & 1) * 8 + ((p >> 3) & 1) * 4; }

// ---- staging: fp32 cache rows -> fp16 K [KV][rows_pad][HD] and transposed V [KV][HD][rows_pad] ----
// Rows [0, pos0) come from the cache ck/cv; rows [pos0, rows), when kn/vn are given, are the appended rows: K
// rotated by RoPE at its position (cs, neox), and both written into the fp32 cache as well as staged - the KV
// append and the staging in one pass. A thread takes one row and dimensions [4 d4, 4 d4 + 4) and the same four
// HD/2 further on, so both RoPE pairings (adjacent, and NeoX's (j, j + HD/2)) stay within the thread. Rows past
// `rows` (padding up to rows_pad) are staged as zeros.
template <int HD>
__global__ __launch_bounds__(256) void stage_kv_kernel(float* ck, float* cv, const float* __restrict__ kn,
                                                       const float* __restrict__ vn, _Float16* __restrict__ k16,
                                                       _Float16* __restrict__ vt16, int64_t pos0, int64_t rows,
                                                       int64_t rows_pad, int n_kv, const float2* __restrict__ cs,
                                                       int neox) {
  __shared__ _Float16 tr[HD][kBN + kPad];
  const int g = blockIdx.y;
  const int64_t r0 = int64_t(blockIdx.x) * kBN;
  constexpr int H2 = HD / 2;
  for (int idx = threadIdx.x; idx < kBN * HD / 8; idx += 256) {
    const int r = idx / (HD / 8), d4 = idx % (HD / 8);
    const int64_t row = r0 + r;
    float4 k0 = make_float4(0.f, 0.f, 0.f, 0.f), k1 = k0, v0 = k0, v1 = k0;
    if (row < rows) {
      const int64_t at = (row * n_kv + g) * HD + 4 * d4;
      if (row < pos0 || !kn) {
        k0 = *reinterpret_cast<const float4*>(ck + at);
        k1 = *reinterpret_cast<const float4*>(ck + at + H2);
        v0 = *reinterpret_cast<const float4*>(cv + at);
        v1 = *reinterpret_cast<const float4*>(cv + at + H2);
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
        *reinterpret_cast<float4*>(ck + at) = k0;
        *reinterpret_cast<float4*>(ck + at + H2) = k1;
        *reinterpret_cast<float4*>(cv + at) = v0;
        *reinterpret_cast<float4*>(cv + at + H2) = v1;
      }
    }
    _Float16* kd = k16 + (int64_t(g) * rows_pad + row) * HD + 4 * d4;
    *reinterpret_cast<half4_t*>(kd) = half4_t{(_Float16)k0.x, (_Float16)k0.y, (_Float16)k0.z, (_Float16)k0.w};
    *reinterpret_cast<half4_t*>(kd + H2) = half4_t{(_Float16)k1.x, (_Float16)k1.y, (_Float16)k1.z, (_Float16)k1.w};
    tr[4 * d4 + 0][r] = (_Float16)v0.x;
    tr[4 * d4 + 1][r] = (_Float16)v0.y;
    tr[4 * d4 + 2][r] = (_Float16)v0.z;
    tr[4 * d4 + 3][r] = (_Float16)v0.w;
    tr[H2 + 4 * d4 + 0][r] = (_Float16)v1.x;
    tr[H2 + 4 * d4 + 1][r] = (_Float16)v1.y;
    tr[H2 + 4 * d4 + 2][r] = (_Float16)v1.z;
    tr[H2 + 4 * d4 + 3][r] = (_Float16)v1.w;
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
}

// Occupancy (waves per SIMD) the register allocator must reach. The kernel is built with MFMA accumulators in
// architectural VGPRs (-amdgpu-mfma-vgpr-form, see the Makefile), so the S^T and O^T accumulators both stay
// resident with no per-tile copies through accumulation registers. head_dim 64 is held to 3 waves per SIMD
// (<= 168 registers, measured fastest: 2 waves with more registers per wave lose more latency hiding than they
// gain); head_dim 128 needs more registers and runs at what fits.
#ifndef NBH_PREFILL_WAVES_PER_EU
#define NBH_PREFILL_WAVES_PER_EU 3
#endif
#ifndef NBH_PREFILL_MIN_WAVES_PER_EU
#define NBH_PREFILL_MIN_WAVES_PER_EU 3
#endif
template <int HD>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(
    HD == 64 ? NBH_PREFILL_MIN_WAVES_PER_EU : 1, NBH_PREFILL_WAVES_PER_EU)))
void attn_prefill_kernel(
    const float* __restrict__ q, const _Float16* __restrict__ k16, const _Float16* __restrict__ vt16,
    float* __restrict__ out, int64_t n, int64_t pos0, int n_heads, int n_kv, int group, int64_t rows_pad,
    int n_tiles, float qscale, const float2* __restrict__ q_rope, int q_rope_neox, const float* __restrict__ kc,
    const float* __restrict__ vc, int64_t fp32_rows, int fp32_n_sub, int n_split, float* __restrict__ ws_o,
    float* __restrict__ ws_ml) {
  // Workgroups past the MFMA tiles: query row t < fp32_rows of the call (q and out start fp32_rows rows before
  // this launch's MFMA rows) for KV head x head subgroup `by`, in fp32 over its whole causal window.
  static_assert(kWaves * 64 == nbh_decode::kDecodeThreads, "the fp32 rows' body runs on the MFMA workgroup size");
  if (int64_t(blockIdx.x) >= int64_t(n_tiles) * n_kv * n_split) {
    const int64_t e = int64_t(blockIdx.x) - int64_t(n_tiles) * n_kv * n_split;
    const int streams = n_kv * fp32_n_sub;
    const int64_t p0 = pos0 - fp32_rows;
    constexpr int64_t kStepRows = (nbh_decode::kDecodeThreads / 64) * (64 / (HD / 8)) * nbh_decode::kUnroll;
    nbh_decode::partial_block<HD, 4, float>(q - fp32_rows * n_heads * HD, kc, vc, out - fp32_rows * n_heads * HD,
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
  half8_t qf[kQB][DC];
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
#pragma unroll
    for (int c = 0; c < DC; ++c)
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[qb][c][e] = (_Float16)(x[c][e] * qscale);
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
  float m_sh[kQB], l_run[kQB];
  floatx16 mneg;
#pragma unroll
  for (int qb = 0; qb < kQB; ++qb) {
    m_sh[qb] = 0.f;
    l_run[qb] = 0.f;
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) mneg[r] = 0.f;

  const _Float16* kg = k16 + int64_t(g) * rows_pad * HD;
  const _Float16* vg = vt16 + int64_t(g) * HD * rows_pad;
  // Asynchronous fetch of key tile kt into LDS stage kt % kStages: each wave fills its share of 1 KB pieces.
  auto fetch = [&](int kt) {
    const int st = kt % kStages;
#pragma unroll
    for (int i = 0; i < K_LD; ++i) {
      const int piece = i * kWaves + wave, slot = piece * 64 + lane;  // 16-byte slot of the tile
      const int r = slot / KCPR, x = (slot % KCPR) ^ swz<KCPR>(r);
      load_lds16(kg + (int64_t(kt) * kBN + r) * HD + 8 * x, &ks[st][piece * 512]);
    }
#pragma unroll
    for (int i = 0; i < V_LD; ++i) {
      const int piece = i * kWaves + wave, slot = piece * 64 + lane;
      const int d = slot / VCPR, x = (slot % VCPR) ^ swz<VCPR>(d);
      load_lds16(vg + int64_t(d) * rows_pad + int64_t(kt) * kBN + 8 * x, &vs[st][piece * 512]);
    }
  };
  // Fragment reads: row r, logical chunk x of a stage.
  auto k_frag = [&](int st, int r, int x) {
    return *reinterpret_cast<const half8_t*>(&ks[st][r * HD + 8 * (x ^ swz<KCPR>(r))]);
  };
  auto v_frag = [&](int st, int d, int x) {
    return *reinterpret_cast<const half8_t*>(&vs[st][d * kBN + 8 * (x ^ swz<VCPR>(d))]);
  };

  // Tiles 0 .. kStages-2 are fetched ahead; step kt waits for its own tile (the later ones may still be in flight),
  // then one barrier both publishes tile kt to every wave and certifies that all waves are done with tile kt - 1,
  // whose stage the fetch of tile kt + kStages - 1 then refills. The barrier is the bare s_barrier: the LDS writes
  // are ordered by the wait on vmcnt (global_load_lds completes when its data is in LDS), and a fence here would
  // also wait for the fetches that are meant to stay in flight.
#pragma unroll
  for (int i = 0; i < kStages - 1; ++i)
    if (kt0 + i < kt1) fetch(kt0 + i);
  for (int kt = kt0; kt < kt1; ++kt) {
    const int cur = kt % kStages;
    constexpr int ahead = (kStages - 2) * (K_LD + V_LD);  // this wave's loads of the tiles after kt
    if (kStages > 2 && kt + 1 < kt1)
      __builtin_amdgcn_s_waitcnt(vmcnt_wait(ahead));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_wait(0));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + kStages - 1 < kt1) fetch(kt + kStages - 1);
    if (wave_active && int64_t(kt) * kBN < wave_kend) {
      // S^T for the tile's two 32-key halves and every query block; each K fragment read from LDS serves all
      // blocks, and the chains are interleaved so consecutive MFMAs do not wait on each other's results. The
      // raised wave priority keeps the MFMA pipe fed while other waves of the SIMD run their softmax VALU work.
      floatx16 s[kQB][2];
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int c = 0; c < DC; ++c)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const half8_t a = k_frag(cur, kk * 32 + ql, 2 * c + hf);
#pragma unroll
          for (int qb = 0; qb < kQB; ++qb) {
            floatx16 c0;
            if (c == 0) {
              if constexpr (kFold) {
                c0 = mneg;
              } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) c0[r] = 0.f;
              }
            } else {
              c0 = s[qb][kk];
            }
            s[qb][kk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[qb][c], c0, 0, 0, 0);
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
      float l_tile[kQB];
      const half2_t ones = {(_Float16)1.0f, (_Float16)1.0f};
      auto exps = [&](int qb, float shift) {
        l_tile[qb] = 0.f;
#pragma unroll
        for (int kc = 0; kc < 4; ++kc)
#pragma unroll
          for (int e = 0; e < 8; ++e)
            pb[qb][kc][e] = (_Float16)exp2_raw(s[qb][kc >> 1][8 * (kc & 1) + e] - shift);
#pragma unroll
        for (int kc = 0; kc < 4; ++kc)
#pragma unroll
          for (int e = 0; e < 8; e += 2)
            l_tile[qb] = __builtin_amdgcn_fdot2(half2_t{pb[qb][kc][e], pb[qb][kc][e + 1]}, ones, l_tile[qb], false);
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
      for (int qb = 0; qb < kQB; ++qb) l_run[qb] += l_tile[qb];
      // O^T += V^T P^T over 4 steps of 16 keys; each V^T fragment read from LDS serves every query block, and the
      // DT x kQB output tiles are independent chains.
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int kc = 0; kc < 4; ++kc) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const half8_t a = v_frag(cur, 32 * dt + ql, 2 * kc + hf);
#pragma unroll
          for (int qb = 0; qb < kQB; ++qb)
            oacc[qb][dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[qb][kc], oacc[qb][dt], 0, 0, 0);
        }
      }
      __builtin_amdgcn_s_setprio(0);
    }
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
        ws_ml[2 * slot] = l_tot > 0.f ? m_sh[qb] : -INFINITY;  // an empty split must not raise the merged max
        ws_ml[2 * slot + 1] = l_tot;
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

// Merges the key splits of the MFMA rows (partials in the decode kernel's layout: slot rh * n_split + s holds the
// shift m in the log2 domain, the sum l and the weighted V row). One thread per (row x head rh, float4 column):
// out = sum_s O_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), M = max_s m_s, the splits taken in order.
template <int HD>
__global__ __launch_bounds__(256) void prefill_split_merge(const float* __restrict__ ws_o,
                                                           const float* __restrict__ ws_ml, float* __restrict__ out,
                                                           int64_t rows_heads, int n_split) {
  constexpr int V4 = HD / 4;
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows_heads * V4) return;
  const int64_t rh = i / V4;
  const int c4 = int(i % V4);
  const float* ml = ws_ml + rh * n_split * 2;
  float mx = -INFINITY;
  for (int sp = 0; sp < n_split; ++sp) mx = fmaxf(mx, ml[2 * sp]);
  const float ms = mx == -INFINITY ? 0.0f : mx;
  const float4* po = reinterpret_cast<const float4*>(ws_o + rh * n_split * HD) + c4;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float l = 0.f;
  for (int sp = 0; sp < n_split; ++sp) {
    const float w = exp2_raw(ml[2 * sp] - ms);
    const float4 o = po[int64_t(sp) * V4];
    acc.x += o.x * w;
    acc.y += o.y * w;
    acc.z += o.z * w;
    acc.w += o.w * w;
    l += ml[2 * sp + 1] * w;
  }
  const float inv = 1.0f / l;
  reinterpret_cast<float4*>(out + rh * HD)[c4] = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
}

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Key splits per row tile for a launch of n_mfma MFMA rows at positions pos0..: 1 when the row tiles alone fill
// the workgroup slots of the chip (3 per CU at head_dim 64, 2 at 128), otherwise enough to fill them, at most 16
// and keeping at least two key tiles per split. Short prefill chunks - nibble's Transformer runs a prompt in
// chunks of max_batch = 512 rows - would otherwise leave most CUs idle.
int prefill_splits(int64_t n_mfma, int64_t pos0, int64_t group, int64_t n_kv, int64_t head_dim, int cu_count) {
  const int64_t tiles = (n_mfma * group + kRowsPerBlock - 1) / kRowsPerBlock;
  const int64_t blocks = tiles * n_kv;
  const int64_t target = int64_t(cu_count > 0 ? cu_count : 256) * (head_dim == 64 ? 3 : 2);
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
  // read-only use of the cache: no new rows (kn = vn = NULL), so ck/cv are only read
  return nbhs_timing::launch(NBHS_K_STAGE_KV, head_dim == 64 ? stage_kv_kernel<64> : stage_kv_kernel<128>, grid,
                             dim3(256), s, const_cast<float*>(k), const_cast<float*>(v),
                             static_cast<const float*>(nullptr), static_cast<const float*>(nullptr), kh, vh, rows,
                             rows, rows_pad, int(n_kv_heads), static_cast<const float2*>(nullptr), 0);
}

int nbhs_append_stage_kv_f16(float* cache_k, float* cache_v, const float* k_new, const float* v_new, int64_t n,
                             int64_t pos0, int64_t n_kv_heads, int64_t head_dim, const float* cs_table,
                             int64_t table_rows, int neox, void* k16, void* vt16, nbhs_stream stream) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (!cache_k || !cache_v || !k_new || !v_new || !cs_table || !k16 || !vt16 || n <= 0 || pos0 < 0 ||
      n_kv_heads <= 0 || n_kv_heads > 65535 || (head_dim != 64 && head_dim != 128) || pos0 + n > table_rows)
    return NBHS_EINVAL;
  const int64_t rows = pos0 + n, rows_pad = round_up(rows, kBN);
  const dim3 grid(unsigned(rows_pad / kBN), unsigned(n_kv_heads));
  return nbhs_timing::launch(NBHS_K_STAGE_KV, head_dim == 64 ? stage_kv_kernel<64> : stage_kv_kernel<128>, grid,
                             dim3(256), s, cache_k, cache_v, k_new, v_new, static_cast<_Float16*>(k16),
                             static_cast<_Float16*>(vt16), pos0, rows, rows_pad, int(n_kv_heads),
                             reinterpret_cast<const float2*>(cs_table), neox);
}

int64_t nbhs_attn_prefill_workspace_bound(int cu_count) {
  // A split is taken only when blocks = tiles * KV < target, with sp <= ceil(target / blocks) and
  // n_mfma <= 128 tiles / G, so n_mfma * n_heads * sp < 256 target: the bound is 256 target (head_dim + 2),
  // largest over the two head sizes (targets 3 and 2 workgroups per CU).
  const int64_t cus = cu_count > 0 ? cu_count : 256;
  return std::max<int64_t>(256 * 3 * cus * (64 + 2), 256 * 2 * cus * (128 + 2));
}

int64_t nbhs_attn_prefill_workspace(int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                    int64_t fp32_rows, int cu_count) {
  if (n <= 0 || pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || fp32_rows < 0 ||
      fp32_rows >= n || (head_dim != 64 && head_dim != 128))
    return -1;
  const int64_t n_mfma = n - fp32_rows;
  const int sp = prefill_splits(n_mfma, pos0 + fp32_rows, n_heads / n_kv_heads, n_kv_heads, head_dim, cu_count);
  return sp == 1 ? 0 : n_mfma * n_heads * sp * (head_dim + 2);
}

int nbhs_attn_prefill_mfma(const float* q, const void* k16, const void* vt16, float* out, int64_t n, int64_t pos0,
                           int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t staged_rows_pad,
                           const float* q_rope_cs, int64_t q_rope_rows, int q_rope_neox, const float* k_cache,
                           const float* v_cache, int64_t fp32_rows, float* workspace, int64_t workspace_floats,
                           int cu_count, nbhs_stream stream) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (!q || !k16 || !vt16 || !out || n <= 0 || pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 ||
      n_heads % n_kv_heads != 0 || (head_dim != 64 && head_dim != 128) || staged_rows_pad % kBN != 0 ||
      staged_rows_pad < round_up(pos0 + n, kBN) || (q_rope_cs && pos0 + n > q_rope_rows) || fp32_rows < 0 ||
      fp32_rows >= n || (fp32_rows > 0 && (!k_cache || !v_cache)))
    return NBHS_EINVAL;
  const int64_t group = n_heads / n_kv_heads;
  const int64_t n_mfma = n - fp32_rows;
  const int64_t tiles = (n_mfma * group + kRowsPerBlock - 1) / kRowsPerBlock;
  const int sp = prefill_splits(n_mfma, pos0 + fp32_rows, group, n_kv_heads, head_dim, cu_count);
  const int64_t need = sp == 1 ? 0 : n_mfma * n_heads * sp * (head_dim + 2);
  if (need > 0 && (!workspace || workspace_floats < need)) return NBHS_EINVAL;
  float* ws_o = need > 0 ? workspace : nullptr;
  float* ws_ml = need > 0 ? workspace + n_mfma * n_heads * sp * head_dim : nullptr;
  const int64_t fp32_sub = (group + 3) / 4;  // head subgroups of the fp32 rows' workgroups (4 query heads each)
  const int64_t blocks = tiles * n_kv_heads * sp + fp32_rows * n_kv_heads * fp32_sub;
  if (blocks >= int64_t(1) << 31) return NBHS_EINVAL;
  const float qscale = (1.0f / std::sqrt(float(head_dim))) * kLog2e;
  const int64_t off = fp32_rows * n_heads * head_dim;  // the MFMA rows start fp32_rows rows in
  const hipError_t e = nbhs_timing::launch(
      NBHS_K_PREFILL_MFMA, head_dim == 64 ? attn_prefill_kernel<64> : attn_prefill_kernel<128>, dim3(unsigned(blocks)),
      dim3(kWaves * 64), s, q + off, static_cast<const _Float16*>(k16), static_cast<const _Float16*>(vt16), out + off,
      n_mfma, pos0 + fp32_rows, int(n_heads), int(n_kv_heads), int(group), staged_rows_pad, int(tiles), qscale,
      reinterpret_cast<const float2*>(q_rope_cs), q_rope_neox, k_cache, v_cache, fp32_rows, int(fp32_sub), sp, ws_o,
      ws_ml);
  if (e != hipSuccess || sp == 1) return e;
  const int64_t threads = n_mfma * n_heads * (head_dim / 4);
  return nbhs_timing::launch(NBHS_K_DECODE_COMBINE, head_dim == 64 ? prefill_split_merge<64> : prefill_split_merge<128>,
                             dim3(unsigned((threads + 255) / 256)), dim3(256), s, ws_o, ws_ml, out + off,
                             n_mfma * n_heads, sp);
}

}  // extern "C"
