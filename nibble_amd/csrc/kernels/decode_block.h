// Split-context fp32 causal GQA attention, one workgroup's share: the body of the decode kernel
// (attn_decode.hip), also run by the prefill kernel for the rows it keeps in fp32. Semantics of
// ref_ops.cpp:188-214 - row t attends to cache rows 0..pos0+t, query head h reads KV head h / (H/KV).
//
// Design (CDNA4, wave64; HBM-bound: arithmetic intensity H/(2*KV) FLOP/B, far below the fp32 ridge). Measured on
// MI355X: a pure read of this access pattern streams at ~6 TB/s; what separates the kernel from that is VALU work
// per byte, so the loop is built to spend as few instructions per K/V byte as possible.
//  * Grid = (context chunk, KV head x head subgroup, query row), sized to the workgroups that fit on the chip at
//    once. A workgroup streams one chunk of one KV head - row groups c, c + n_chunks, ..., so that all workgroups
//    sweep the cache together - and serves every query head of its GQA group from registers: each K/V byte is read
//    from HBM once per step, not once per query head.
//  * A 64-float K/V row is 8 lanes x 2 float4 (lane dl holds float4 columns dl and dl + 8, so each load
//    instruction reads whole contiguous 128-byte halves of 8 rows); a wave covers 8 rows per load pair and keeps
//    NBH_DECODE_UNROLL such row slots of K and of V in flight per lane, with non-temporal (streaming) loads; the
//    next group's loads are issued right after the current group is consumed. Dot products reduce over the 8 lanes
//    with 3 DPP steps.
//  * Online softmax in the log2 domain (queries pre-scaled by log2(e)/sqrt(d)) with raw v_exp_f32 and one running
//    max per wave and query head, raised only when some score exceeds it by more than kLazy (log2 units) - a rare,
//    wave-uniform branch - so unnormalised weights stay <= 2^kLazy and the wave's 8 row groups share one scale: at
//    the end they are combined by plain sums (DPP), and only the workgroup's 4 waves need exp-weighted merges.
//  * Row validity is only tested in a chunk's last, partial iteration.
//  * Each workgroup writes an unnormalised partial (max, sum, weighted V) per query head; attn_decode_combine
//    merges the chunks with a log-sum-exp reduction. With a single chunk the partial kernel writes the output.
//  * Single-row append (decode step of the fused append + attention op): the new K/V row is not in the cache yet.
//    The workgroup whose chunk ends with row pos0 loads it from k_new / v_new, rotates K in registers and uses it
//    in place of cache row pos0; it writes the row into the cache in its epilogue. No other workgroup reads that
//    row, so the separate append launch disappears.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

#include "kernels/rope_device.h"

namespace nbh_decode {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kDecodeThreads = 256;  // 4 waves
// Row slots in flight per lane per tensor, and the split targets in workgroups per CU: short contexts use
// NBH_DECODE_WG_PER_CU, long ones (at least kLongGroups row groups per chunk at the higher count) up to
// NBH_DECODE_WG_PER_CU_LONG. Compile-time so that tuning sweeps can build variants; the defaults are the measured
// best on MI355X (3 per CU streams 128k contexts 6 % faster, is even at 32k and 7 % slower at 8k).
#ifndef NBH_DECODE_UNROLL
#define NBH_DECODE_UNROLL 1
#endif
#ifndef NBH_DECODE_WG_PER_CU
#define NBH_DECODE_WG_PER_CU 2
#endif
#ifndef NBH_DECODE_WG_PER_CU_LONG
#define NBH_DECODE_WG_PER_CU_LONG 3
#endif
constexpr int64_t kLongGroups = 12;
// K/V rows are read exactly once per step: stream them past the caches (non-temporal loads) unless disabled.
#ifndef NBH_DECODE_NT
#define NBH_DECODE_NT 1
#endif
// Chunk c of a head takes row groups c, c + n_chunks, c + 2 n_chunks, ... (1) instead of one contiguous range (0):
// all workgroups then sweep the cache together, front to back.
#ifndef NBH_DECODE_INTERLEAVE
#define NBH_DECODE_INTERLEAVE 1
#endif
constexpr int kUnroll = NBH_DECODE_UNROLL;
// Row slots per lane per iteration for a cache element of `bytes` bytes: fp16 caches take twice the rows, so that
// an iteration moves as many bytes as with fp32 (the kernel is bound by iterations, one memory round trip each).
constexpr int unroll_for(int bytes) { return bytes == 4 ? kUnroll : 2 * kUnroll; }
constexpr int kMaxChunks = 4096;  // partials per (row, head); bounds the combine kernel's LDS table
constexpr float kLazy = 8.0f;     // allowed growth of scores over the running max before a rescale

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of LPR lanes (8 or 16); every lane of the group gets the bit-identical sum
// (each step adds a lane's value to its partner's, and a + b == b + a).
template <int LPR>
__device__ __forceinline__ float group_sum(float x) {
  x += dpp<0xB1>(x);   // quad_perm(1,0,3,2): lane ^ 1
  x += dpp<0x4E>(x);   // quad_perm(2,3,0,1): lane ^ 2
  x += dpp<0x141>(x);  // row_half_mirror: lane i <-> 7 - i within 8 (joins the two quads)
  if constexpr (LPR == 16) x += dpp<0x140>(x);  // row_mirror: lane i <-> 15 - i within 16
  return x;
}

// Sum of the values held by lanes l, l + LPR, l + 2 LPR, ... (the wave's row groups), in every lane.
template <int LPR>
__device__ __forceinline__ float row_group_sum(float x) {
  if constexpr (LPR == 8) x += dpp<0x128>(x);  // row_ror:8 within 16 lanes: lane ^ 8
  x += __shfl_xor(x, 16, 64);
  x += __shfl_xor(x, 32, 64);
  return x;
}

__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }  // v_exp_f32; -inf -> 0

// One 16-byte K/V load.
__device__ __forceinline__ f32x4 load4(const float* p) {
#if NBH_DECODE_NT
  return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
#else
  return *reinterpret_cast<const f32x4*>(p);
#endif
}

// Four consecutive cache elements as floats: fp32 caches (the reference's) or fp16 caches (8-byte loads, exact
// widening).
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
template <typename KV>
__device__ __forceinline__ f32x4 load_kv4(const KV* p) {
  if constexpr (sizeof(KV) == 4) {
    return load4(reinterpret_cast<const float*>(p));
  } else {
#if NBH_DECODE_NT
    const f16x4 h = __builtin_nontemporal_load(reinterpret_cast<const f16x4*>(p));
#else
    const f16x4 h = *reinterpret_cast<const f16x4*>(p);
#endif
    return f32x4{float(h[0]), float(h[1]), float(h[2]), float(h[3])};
  }
}
template <typename KV>
__device__ __forceinline__ void store_kv4(KV* p, f32x4 x) {
  if constexpr (sizeof(KV) == 4)
    *reinterpret_cast<f32x4*>(p) = x;
  else
    *reinterpret_cast<f16x4*>(p) = f16x4{_Float16(x[0]), _Float16(x[1]), _Float16(x[2]), _Float16(x[3])};
}
// x as the cache will hold it (fp16 caches: rounded to nearest even).
template <typename KV>
__device__ __forceinline__ f32x4 as_stored(f32x4 x) {
  if constexpr (sizeof(KV) == 4)
    return x;
  else
    return f32x4{float(_Float16(x[0])), float(_Float16(x[1])), float(_Float16(x[2])), float(_Float16(x[3]))};
}

// Online-softmax state of one query head over some rows, as held by one lane: running max m (log2 domain), sum of
// weights l, weighted V slice o (VPL float4 of the lane's dimensions).
template <int VPL>
struct State {
  float m, l;
  f32x4 o[VPL];
};

// Merges state b into a: the result covers the rows of both.
template <int VPL>
__device__ __forceinline__ void merge(State<VPL>& a, float bm, float bl, const f32x4* bo) {
  const float mn = fmaxf(a.m, bm);
  const float ms = mn == -INFINITY ? 0.0f : mn;
  const float wa = exp2_raw(a.m - ms), wb = exp2_raw(bm - ms);
  a.l = a.l * wa + bl * wb;
#pragma unroll
  for (int i = 0; i < VPL; ++i) a.o[i] = a.o[i] * wa + bo[i] * wb;
  a.m = mn;
}

// One workgroup of the split-context kernel: chunk `chunk` of query row t for KV head x head subgroup `by`
// (by / n_sub, by % n_sub). HD: head_dim (64 or 128). GB: query heads per workgroup (the GQA group, or a slice of
// it). KV: the cache element type (float, or _Float16 for an fp16 cache). Needs kDecodeThreads threads.
template <int HD, int GB, typename KV = float>
__device__ __forceinline__ void partial_block(
    const float* __restrict__ q, const KV* __restrict__ k, const KV* __restrict__ v, float* __restrict__ out,
    float* __restrict__ ws_o, float* __restrict__ ws_ml, int64_t pos0, int n_heads, int n_kv, int group, int n_sub,
    int n_chunks, int64_t groups_per_chunk, int64_t extra_groups, float qscale, const float2* __restrict__ q_rope,
    int q_rope_neox, const float* __restrict__ k_new, const float* __restrict__ v_new, KV* __restrict__ k_dst,
    KV* __restrict__ v_dst, int chunk, int by, int64_t t) {
  constexpr int VPL = 2;                            // float4 per lane per row
  constexpr int LPR = HD / (4 * VPL);               // lanes per K/V row: 8 (hd 64) or 16 (hd 128)
  constexpr int RPS = 64 / LPR;                     // rows per wave load
  constexpr int KU = unroll_for(int(sizeof(KV)));   // row slots per lane per iteration
  constexpr int WAVE_ROWS = RPS * KU;               // rows per wave iteration
  constexpr int NW = kDecodeThreads / 64;           // waves per workgroup
  constexpr int64_t kStep = NW * WAVE_ROWS;         // rows the workgroup covers per iteration
  __shared__ float sm_m[NW][GB], sm_l[NW][GB];
  __shared__ f32x4 sm_o[NW][GB][LPR * VPL];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, dl = lane % LPR;
  const int g = by / n_sub, sg = by % n_sub;
  const int h0 = g * group + sg * GB;
  const int gcount = min(GB, group - sg * GB);
  const int64_t len = pos0 + t + 1;
  // The chunk's row groups (kStep consecutive rows each), clipped to this row's causal length: iteration i takes
  // group g0 + i * gstride, for i < gcnt. The first extra_groups chunks hold one group more than the others (the
  // remainder of the even split).
  const int64_t n_groups = (len + kStep - 1) / kStep;
  const bool extra = chunk < extra_groups;
#if NBH_DECODE_INTERLEAVE
  const int64_t g0 = chunk, gstride = n_chunks;
  const int64_t gcnt = g0 < n_groups ? min(groups_per_chunk + (extra ? 1 : 0), (n_groups - 1 - g0) / gstride + 1) : 0;
#else
  const int64_t g0 = int64_t(chunk) * groups_per_chunk + min(int64_t(chunk), extra_groups), gstride = 1;
  const int64_t gcnt = max(int64_t(0), min(groups_per_chunk + (extra ? 1 : 0), n_groups - g0));
#endif

  const int64_t row_stride = int64_t(n_kv) * HD;
  const KV* kb = k + int64_t(g) * HD + 4 * dl;  // float4 column dl + LPR * i of the row
  const KV* vb = v + int64_t(g) * HD + 4 * dl;

  // Single-row append: the workgroup whose last row group holds row pos0 (= len - 1, n is 1) owns the new row.
  const bool append = k_new != nullptr;
  const int64_t new_grp = pos0 / kStep;
  const bool owner = append && gcnt > 0 && g0 + (gcnt - 1) * gstride == new_grp;
  const float* knb = append ? k_new + int64_t(g) * HD + 4 * dl : nullptr;  // the new row's lane slice
  const float* vnb = append ? v_new + int64_t(g) * HD + 4 * dl : nullptr;

  // One iteration's rows: KU row slots, VPL float4 of K and of V each. Rows past the causal window are
  // clamped to the last valid row (never read out of range) and masked in the partial iteration. When appending,
  // lanes on row pos0 (and those clamped to it) read k_new / v_new instead of the cache row, which this kernel
  // writes; compute() replaces those values with the rotated row.
  struct Rows {
    f32x4 k[KU][VPL], v[KU][VPL];
  };
  auto row_of = [&](int64_t grp, int u) { return grp * kStep + wave * WAVE_ROWS + u * RPS + sub; };
  auto load = [&](int64_t grp, Rows& r) {
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int64_t j = min(row_of(grp, u), len - 1);
      const bool fresh = append && j >= pos0;
      if constexpr (sizeof(KV) == 4) {
        const float* kr = fresh ? knb : reinterpret_cast<const float*>(kb) + j * row_stride;
        const float* vr = fresh ? vnb : reinterpret_cast<const float*>(vb) + j * row_stride;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          r.k[u][i] = load4(kr + 4 * LPR * i);
          r.v[u][i] = load4(vr + 4 * LPR * i);
        }
      } else {  // the appended row's lanes read cache row 0 instead (their values are replaced in compute)
        const KV* kr = kb + (fresh ? 0 : j) * row_stride;
        const KV* vr = vb + (fresh ? 0 : j) * row_stride;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          r.k[u][i] = load_kv4(kr + 4 * LPR * i);
          r.v[u][i] = load_kv4(vr + 4 * LPR * i);
        }
      }
    }
  };

  Rows ra, rb;
  // The first K/V loads go out before the query loads, so the first HBM round trip is not spent on q alone. A
  // chunk holding an extra group loads its first two groups together: the extra group's round trip overlaps the
  // first one instead of adding one, so every chunk takes groups_per_chunk round trips.
  int64_t it = 0;  // iterations done
  if (gcnt > 0) load(g0, ra);
  const bool two = extra && gcnt > 1;
  if (two) load(g0 + gstride, rb);

  // Rotates a lane's slice of a row at position pos (cs = the position-major (cos, sin) table), exactly as the RoPE
  // kernel does in memory. The lane holds both members of each of its pairs: adjacent pairs sit in one float4, and
  // with NeoX pairing (j, j + HD/2) float4 i = 1 is float4 i = 0 shifted by 4 LPR = HD/2 floats.
  auto rotate = [&](f32x4 (&x)[VPL], int64_t pos) {
    const float2* cs = q_rope + pos * (HD / 2);
    if (q_rope_neox) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float2 r = rope_pair(x[0][e], x[1][e], cs[4 * dl + e]);
        x[0][e] = r.x;
        x[1][e] = r.y;
      }
    } else {
#pragma unroll
      for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          const float2 r = rope_pair(x[i][2 * pr], x[i][2 * pr + 1], cs[2 * (dl + LPR * i) + pr]);
          x[i][2 * pr] = r.x;
          x[i][2 * pr + 1] = r.y;
        }
    }
  };

  // The appended row, rotated (owner only; consumed in the chunk's last iteration and the epilogue).
  f32x4 nk[VPL], nv[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) nk[i] = nv[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (owner) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      nk[i] = *reinterpret_cast<const f32x4*>(knb + 4 * LPR * i);
      nv[i] = *reinterpret_cast<const f32x4*>(vnb + 4 * LPR * i);
    }
    rotate(nk, pos0);
    // attend to the row as the cache will hold it
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      nk[i] = as_stored<KV>(nk[i]);
      nv[i] = as_stored<KV>(nv[i]);
    }
  }

  f32x4 qv[GB][VPL];
  State<VPL> st[GB];
#pragma unroll
  for (int h = 0; h < GB; ++h) {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      qv[h][i] = f32x4{0.f, 0.f, 0.f, 0.f};
      st[h].o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (h < gcount) qv[h][i] = *reinterpret_cast<const f32x4*>(q + (t * n_heads + h0 + h) * HD + 4 * (dl + LPR * i));
    }
    if (q_rope && h < gcount) rotate(qv[h], pos0 + t);  // unrotated q: rotate on load
#pragma unroll
    for (int i = 0; i < VPL; ++i) qv[h][i] *= qscale;
    st[h].m = -INFINITY;
    st[h].l = 0.f;
  }

  auto compute = [&](Rows& r, int64_t grp_idx) {
    // Wave-uniform: does this iteration reach past the causal window?
    const bool partial = grp_idx * kStep + wave * WAVE_ROWS + WAVE_ROWS > len;
    // Wave-uniform: does it hold the appended row? Then its lanes take the rotated row from registers.
    if (owner && grp_idx == new_grp && grp_idx * kStep + wave * WAVE_ROWS + WAVE_ROWS > pos0) {
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const bool fresh = row_of(grp_idx, u) >= pos0;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
          r.k[u][i] = fresh ? nk[i] : r.k[u][i];
          r.v[u][i] = fresh ? nv[i] : r.v[u][i];
        }
      }
    }
#pragma unroll
    for (int h = 0; h < GB; ++h) {
      if (h >= gcount) continue;
      float sc[KU];
      float mloc = -INFINITY;
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        f32x4 prod = qv[h][0] * r.k[u][0];
#pragma unroll
        for (int i = 1; i < VPL; ++i) prod += qv[h][i] * r.k[u][i];
        float d = (prod[0] + prod[1]) + (prod[2] + prod[3]);
        d = group_sum<LPR>(d);
        if (partial && row_of(grp_idx, u) >= len) d = -INFINITY;
        sc[u] = d;
        mloc = fmaxf(mloc, d);
      }
      // The wave's reference max (identical in every lane) is raised only when some score outgrew it by more
      // than kLazy; the first iteration always sets it (m = -inf).
      if (__builtin_amdgcn_ballot_w64(mloc > st[h].m + kLazy)) {
#pragma unroll
        for (int mask = LPR; mask < 64; mask <<= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, mask, 64));
        const float mn = fmaxf(st[h].m, mloc);
        const float corr = exp2_raw(st[h].m - (mn == -INFINITY ? 0.0f : mn));
        st[h].l *= corr;
#pragma unroll
        for (int i = 0; i < VPL; ++i) st[h].o[i] *= corr;
        st[h].m = mn;
      }
      const float ms = st[h].m == -INFINITY ? 0.0f : st[h].m;
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const float p = exp2_raw(sc[u] - ms);
        st[h].l += p;
#pragma unroll
        for (int i = 0; i < VPL; ++i) st[h].o[i] += p * r.v[u][i];
      }
    }
  };

  if (two) {
    compute(ra, g0);
    compute(rb, g0 + gstride);
    it = 2;
    if (it < gcnt) load(g0 + it * gstride, ra);
  }
  while (it < gcnt) {
    compute(ra, g0 + it * gstride);
    ++it;
    if (it < gcnt) load(g0 + it * gstride, ra);
  }

  // The appended row goes into its cache row once per KV head (head subgroup 0 of the owner).
  if (owner && sg == 0 && wave == 0 && lane < LPR) {
    KV* kd = k_dst + pos0 * row_stride + int64_t(g) * HD + 4 * dl;
    KV* vd = v_dst + pos0 * row_stride + int64_t(g) * HD + 4 * dl;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      store_kv4(kd + 4 * LPR * i, nk[i]);
      store_kv4(vd + 4 * LPR * i, nv[i]);
    }
  }

  // The wave's row groups (lanes dl, dl + LPR, ...) share the wave's max: sum them, then merge the waves
  // through LDS.
#pragma unroll
  for (int h = 0; h < GB; ++h) {
    st[h].l = row_group_sum<LPR>(st[h].l);
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int c = 0; c < 4; ++c) st[h].o[i][c] = row_group_sum<LPR>(st[h].o[i][c]);
    if (lane < LPR) {
#pragma unroll
      for (int i = 0; i < VPL; ++i) sm_o[wave][h][dl + LPR * i] = st[h].o[i];
      if (lane == 0) {
        sm_m[wave][h] = st[h].m;
        sm_l[wave][h] = st[h].l;
      }
    }
  }
  __syncthreads();
  constexpr int V4 = HD / 4;  // float4 columns of a head row
  for (int idx = threadIdx.x; idx < GB * V4; idx += kDecodeThreads) {
    const int h = idx / V4, c4 = idx % V4;
    if (h >= gcount) continue;
    State<1> acc;
    acc.m = sm_m[0][h];
    acc.l = sm_l[0][h];
    acc.o[0] = sm_o[0][h][c4];
#pragma unroll
    for (int w = 1; w < NW; ++w) merge<1>(acc, sm_m[w][h], sm_l[w][h], &sm_o[w][h][c4]);
    const int64_t head = h0 + h;
    if (n_chunks == 1) {
      reinterpret_cast<f32x4*>(out + (t * n_heads + head) * HD)[c4] = acc.o[0] * (1.0f / acc.l);
    } else {
      const int64_t slot = (t * n_heads + head) * n_chunks + chunk;
      reinterpret_cast<f32x4*>(ws_o + slot * HD)[c4] = acc.o[0];
      if (c4 == 0) {
        ws_ml[2 * slot] = acc.m;
        ws_ml[2 * slot + 1] = acc.l;
      }
    }
  }
}

// Block-wide reduction of one float per thread (kDecodeThreads threads); every thread gets the result.
template <bool MAX>
__device__ __forceinline__ float block_reduce(float x, float* scratch) {
#pragma unroll
  for (int mask = 1; mask < 64; mask <<= 1) {
    const float y = __shfl_xor(x, mask, 64);
    x = MAX ? fmaxf(x, y) : x + y;
  }
  __syncthreads();  // scratch may still be read from a previous reduction
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = x;
  __syncthreads();
  float r = scratch[0];
#pragma unroll
  for (int w = 1; w < kDecodeThreads / 64; ++w) r = MAX ? fmaxf(r, scratch[w]) : r + scratch[w];
  return r;
}

// Log-sum-exp merge of the chunk partials of one (row, head) per workgroup. Thread (chunk group cg, float4 column
// c4) loads the max, sum and partial-output column of its chunks cg, cg + CG, ... all at once (one memory round
// trip for up to kPer chunks each), the global max comes from a block reduction, and the weighted sums of the
// chunk groups are added through LDS.
template <int HD>
__device__ __forceinline__ void combine_block(const float* __restrict__ ws_o, const float* __restrict__ ws_ml,
                                              float* __restrict__ out, int n_chunks, int64_t rh) {
  constexpr int V4 = HD / 4;                // float4 columns of one head row
  constexpr int CG = kDecodeThreads / V4;   // chunk groups
  constexpr int kPer = 16;                  // chunks per thread held in registers
  __shared__ float red[kDecodeThreads / 64];
  __shared__ f32x4 acc_s[CG][V4];
  __shared__ float l_s[CG];
  const int tid = threadIdx.x;
  const int cg = tid / V4, c4 = tid % V4;
  const float* ml = ws_ml + rh * n_chunks * 2;
  const f32x4* po = reinterpret_cast<const f32x4*>(ws_o + rh * n_chunks * HD) + c4;
  float mv[kPer], lv[kPer];
  f32x4 ov[kPer];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int c = cg + i * CG;
    mv[i] = -INFINITY;
    lv[i] = 0.f;
    ov[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (c < n_chunks) {
      mv[i] = ml[2 * c];
      lv[i] = ml[2 * c + 1];
      ov[i] = po[int64_t(c) * V4];
    }
    mx = fmaxf(mx, mv[i]);
  }
  for (int c = cg + kPer * CG; c < n_chunks; c += CG) mx = fmaxf(mx, ml[2 * c]);  // beyond the register window
  mx = block_reduce<true>(mx, red);
  const float ms = mx == -INFINITY ? 0.0f : mx;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float lsum = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const float wc = exp2_raw(mv[i] - ms);
    acc += ov[i] * wc;
    lsum += lv[i] * wc;
  }
  for (int c = cg + kPer * CG; c < n_chunks; c += CG) {
    const float wc = exp2_raw(ml[2 * c] - ms);
    acc += po[int64_t(c) * V4] * wc;
    lsum += ml[2 * c + 1] * wc;
  }
  acc_s[cg][c4] = acc;
  if (c4 == 0) l_s[cg] = lsum;
  __syncthreads();
  if (tid < V4) {
    f32x4 r = acc_s[0][tid];
    float l = l_s[0];
#pragma unroll
    for (int i = 1; i < CG; ++i) {
      r += acc_s[i][tid];
      l += l_s[i];
    }
    reinterpret_cast<f32x4*>(out + rh * HD)[tid] = r * (1.0f / l);
  }
}

}  // namespace nbh_decode
