// fp32 causal GQA attention for few query rows (decode): Backend::attention (backend.h:68-69) with the semantics
// of ref_ops.cpp:188-214 - row t attends to cache rows 0..pos0+t, query head h reads KV head h / (H/KV).
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
#include <hip/hip_runtime.h>

#include <cmath>

#include "backend/hip/kernel_timing.h"
#include "kernels/rope_device.h"
#include "nibble_hip_shim.h"

namespace {

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

// HD: head_dim (64 or 128). GB: query heads per workgroup (the GQA group, or a slice of it).
template <int HD, int GB>
__global__ __launch_bounds__(kDecodeThreads) void attn_decode_partial(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ out,
    float* __restrict__ ws_o, float* __restrict__ ws_ml, int64_t pos0, int n_heads, int n_kv, int group, int n_sub,
    int n_chunks, int64_t groups_per_chunk, int64_t extra_groups, float qscale, const float2* __restrict__ q_rope,
    int q_rope_neox, const float* __restrict__ k_new, const float* __restrict__ v_new, float* __restrict__ k_dst,
    float* __restrict__ v_dst) {
  constexpr int VPL = 2;                            // float4 per lane per row
  constexpr int LPR = HD / (4 * VPL);               // lanes per K/V row: 8 (hd 64) or 16 (hd 128)
  constexpr int RPS = 64 / LPR;                     // rows per wave load
  constexpr int WAVE_ROWS = RPS * kUnroll;          // rows per wave iteration
  constexpr int NW = kDecodeThreads / 64;           // waves per workgroup
  constexpr int64_t kStep = NW * WAVE_ROWS;         // rows the workgroup covers per iteration
  __shared__ float sm_m[NW][GB], sm_l[NW][GB];
  __shared__ f32x4 sm_o[NW][GB][LPR * VPL];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, dl = lane % LPR;
  const int chunk = blockIdx.x;
  const int g = blockIdx.y / n_sub, sg = blockIdx.y % n_sub;
  const int64_t t = blockIdx.z;
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
  const float* kb = k + int64_t(g) * HD + 4 * dl;  // float4 column dl + LPR * i of the row
  const float* vb = v + int64_t(g) * HD + 4 * dl;

  // Single-row append: the workgroup whose last row group holds row pos0 (= len - 1, n is 1) owns the new row.
  const bool append = k_new != nullptr;
  const int64_t new_grp = pos0 / kStep;
  const bool owner = append && gcnt > 0 && g0 + (gcnt - 1) * gstride == new_grp;
  const float* knb = append ? k_new + int64_t(g) * HD + 4 * dl : kb;  // the new row's lane slice
  const float* vnb = append ? v_new + int64_t(g) * HD + 4 * dl : vb;

  // One iteration's rows: kUnroll row slots, VPL float4 of K and of V each. Rows past the causal window are
  // clamped to the last valid row (never read out of range) and masked in the partial iteration. When appending,
  // lanes on row pos0 (and those clamped to it) read k_new / v_new instead of the cache row, which this kernel
  // writes; compute() replaces those values with the rotated row.
  struct Rows {
    f32x4 k[kUnroll][VPL], v[kUnroll][VPL];
  };
  auto row_of = [&](int64_t grp, int u) { return grp * kStep + wave * WAVE_ROWS + u * RPS + sub; };
  auto load = [&](int64_t grp, Rows& r) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = min(row_of(grp, u), len - 1);
      const bool fresh = append && j >= pos0;
      const float* kr = fresh ? knb : kb + j * row_stride;
      const float* vr = fresh ? vnb : vb + j * row_stride;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        r.k[u][i] = load4(kr + 4 * LPR * i);
        r.v[u][i] = load4(vr + 4 * LPR * i);
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
      for (int u = 0; u < kUnroll; ++u) {
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
      float sc[kUnroll];
      float mloc = -INFINITY;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
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
      for (int u = 0; u < kUnroll; ++u) {
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
    float* kd = k_dst + pos0 * row_stride + int64_t(g) * HD + 4 * dl;
    float* vd = v_dst + pos0 * row_stride + int64_t(g) * HD + 4 * dl;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      *reinterpret_cast<f32x4*>(kd + 4 * LPR * i) = nk[i];
      *reinterpret_cast<f32x4*>(vd + 4 * LPR * i) = nv[i];
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
__global__ __launch_bounds__(kDecodeThreads) void attn_decode_combine(const float* __restrict__ ws_o,
                                                                      const float* __restrict__ ws_ml,
                                                                      float* __restrict__ out, int n_chunks) {
  constexpr int V4 = HD / 4;                // float4 columns of one head row
  constexpr int CG = kDecodeThreads / V4;   // chunk groups
  constexpr int kPer = 16;                  // chunks per thread held in registers
  __shared__ float red[kDecodeThreads / 64];
  __shared__ f32x4 acc_s[CG][V4];
  __shared__ float l_s[CG];
  const int tid = threadIdx.x;
  const int cg = tid / V4, c4 = tid % V4;
  const int64_t rh = blockIdx.x;  // t * n_heads + head
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

// Any head_dim in [1, 256]: one wave per (row, head), one key per step, lanes over dimensions. Slow, exact
// semantics; serves head sizes without a tiled kernel.
__global__ __launch_bounds__(64) void attn_generic(const float* __restrict__ q, const float* __restrict__ k,
                                                   const float* __restrict__ v, float* __restrict__ out,
                                                   int64_t pos0, int n_heads, int n_kv, int hd, float qscale) {
  const int lane = threadIdx.x;
  const int h = blockIdx.x;
  const int64_t t = blockIdx.y;
  const int g = h / (n_heads / n_kv);
  const int64_t len = pos0 + t + 1;
  float qr[4], o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int d = lane + 64 * r;
    qr[r] = d < hd ? q[(t * n_heads + h) * hd + d] * qscale : 0.f;
    o[r] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  for (int64_t j = 0; j < len; ++j) {
    const float* kj = k + (j * n_kv + g) * hd;
    const float* vj = v + (j * n_kv + g) * hd;
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = lane + 64 * r;
      if (d < hd) s = fmaf(qr[r], kj[d], s);
    }
#pragma unroll
    for (int mask = 1; mask < 64; mask <<= 1) s += __shfl_xor(s, mask, 64);
    const float mn = fmaxf(m, s);
    const float corr = exp2f(m - mn), p = exp2f(s - mn);
    l = l * corr + p;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = lane + 64 * r;
      o[r] = o[r] * corr + (d < hd ? p * vj[d] : 0.f);
    }
    m = mn;
  }
  const float inv = 1.0f / l;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int d = lane + 64 * r;
    if (d < hd) out[(t * n_heads + h) * hd + d] = o[r] * inv;
  }
}

// Chunking plan shared by the workspace query and the launcher.
struct Plan {
  int gb;                     // query heads per workgroup (1, 2, 4 or 8)
  int n_sub;                  // head subgroups per KV head
  int n_chunks;               // chunks per (row, head subgroup); each writes one partial per query head
  int64_t groups_per_chunk;   // row groups per chunk
  int64_t extra_groups;       // the first extra_groups chunks take one group more
};

// Workgroups of attn_decode_partial<HD, GB> that fit on one CU at once (register and LDS limits), capped at
// NBH_DECODE_WG_PER_CU_LONG; queried from the runtime once per instance.
template <int HD, int GB>
int resident_per_cu() {
  static const int n = [] {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, attn_decode_partial<HD, GB>, kDecodeThreads, 0) !=
            hipSuccess ||
        b < 1)
      b = 1;
    return b < NBH_DECODE_WG_PER_CU_LONG ? b : NBH_DECODE_WG_PER_CU_LONG;
  }();
  return n;
}

int resident_per_cu(int64_t head_dim, int gb) {
  if (head_dim == 64)
    return gb == 1 ? resident_per_cu<64, 1>() : gb == 2 ? resident_per_cu<64, 2>()
         : gb == 4 ? resident_per_cu<64, 4>() : resident_per_cu<64, 8>();
  return gb == 1 ? resident_per_cu<128, 1>() : gb == 2 ? resident_per_cu<128, 2>()
       : gb == 4 ? resident_per_cu<128, 4>() : resident_per_cu<128, 8>();
}

// As many workgroups as fit on the chip at once: one round, no tail of late starters. The row groups are split
// evenly over min(slots, groups) chunks; the remainder goes one group each to the first chunks, which load that
// group together with their first one (see attn_decode_partial), so a context one row past a round size costs no
// workgroup an extra HBM round trip and no workgroup waits for a free slot.
Plan make_plan(int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv, int64_t head_dim, int cu_count) {
  Plan p;
  const int64_t group = n_heads / n_kv;
  p.gb = group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 ? 4 : 8;
  p.n_sub = int((group + p.gb - 1) / p.gb);
  const int64_t max_len = pos0 + n;
  const int64_t lpr = head_dim / 8;
  const int64_t step = (64 / lpr) * kUnroll * (kDecodeThreads / 64);  // rows a workgroup covers per iteration
  const int64_t units = (max_len + step - 1) / step;
  const int64_t cus = cu_count > 0 ? cu_count : 256;
  const int64_t streams = n * n_kv * p.n_sub;  // workgroups per chunk index
  const int resident = resident_per_cu(head_dim, p.gb);
  int64_t slots = cus * resident / streams;
  if (resident > NBH_DECODE_WG_PER_CU && units < kLongGroups * slots)
    slots = cus * NBH_DECODE_WG_PER_CU / streams;  // short context: fewer, longer workgroups
  if (slots < 1) slots = 1;
  int64_t chunks = units < slots ? units : slots;
  if (chunks > kMaxChunks) chunks = kMaxChunks;
  p.n_chunks = int(chunks);
  p.groups_per_chunk = units / chunks;
  p.extra_groups = units % chunks;
  return p;
}

// Appended row of a single-row call: new K/V rows in, cache rows out (all null when nothing is appended).
struct Append {
  const float* k_new = nullptr;
  const float* v_new = nullptr;
  float* k_dst = nullptr;
  float* v_dst = nullptr;
};

template <int HD>
int launch_decode(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0, int64_t H,
                  int64_t KV, float* ws, const Plan& p, float qscale, const float2* q_rope, int q_rope_neox,
                  const Append& app, hipStream_t s) {
  float* ws_o = ws;
  float* ws_ml = ws ? ws + n * H * p.n_chunks * HD : nullptr;
  const int group = int(H / KV);
  const dim3 grid(p.n_chunks, unsigned(KV * p.n_sub), unsigned(n));
  hipError_t e;
#define NBH_DECODE(GB)                                                                                             \
  e = nbhs_timing::launch(NBHS_K_DECODE_PARTIAL, attn_decode_partial<HD, GB>, grid, dim3(kDecodeThreads), s, q, k, \
                          v, out, ws_o, ws_ml, pos0, int(H), int(KV), group, p.n_sub, p.n_chunks,                   \
                          p.groups_per_chunk, p.extra_groups, qscale, q_rope, q_rope_neox, app.k_new, app.v_new,  \
                          app.k_dst, app.v_dst)
  switch (p.gb) {
    case 1: NBH_DECODE(1); break;
    case 2: NBH_DECODE(2); break;
    case 4: NBH_DECODE(4); break;
    default: NBH_DECODE(8); break;
  }
#undef NBH_DECODE
  if (e != hipSuccess || p.n_chunks == 1) return e;
  return nbhs_timing::launch(NBHS_K_DECODE_COMBINE, attn_decode_combine<HD>, dim3(unsigned(n * H)),
                             dim3(kDecodeThreads), s, ws_o, ws_ml, out, p.n_chunks);
}

bool tiled_head_dim(int64_t hd) { return hd == 64 || hd == 128; }

int decode(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0, int64_t n_heads,
           int64_t n_kv_heads, int64_t head_dim, float* workspace, int64_t workspace_floats, int cu_count,
           const float* q_rope_cs, int64_t q_rope_rows, int q_rope_neox, const Append& app, hipStream_t s) {
  if (!q || !k || !v || !out || n <= 0 || n > 65535 || pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 ||
      n_heads % n_kv_heads != 0 || head_dim <= 0 || head_dim > 256 || n_heads > 65535)
    return NBHS_EINVAL;
  // q rotation on load is implemented for the tiled head sizes only, over table rows covering pos0 .. pos0+n-1
  if (q_rope_cs && (!tiled_head_dim(head_dim) || pos0 + n > q_rope_rows)) return NBHS_EINVAL;
  const float2* q_rope = reinterpret_cast<const float2*>(q_rope_cs);
  const float qscale = (1.0f / std::sqrt(float(head_dim))) * kLog2e;
  if (!tiled_head_dim(head_dim)) {
    return nbhs_timing::launch(NBHS_K_GENERIC, attn_generic, dim3(unsigned(n_heads), unsigned(n)), dim3(64), s, q, k,
                               v, out, pos0, int(n_heads), int(n_kv_heads), int(head_dim), qscale);
  }
  const Plan p = make_plan(n, pos0, n_heads, n_kv_heads, head_dim, cu_count);
  const int64_t need = p.n_chunks == 1 ? 0 : n * n_heads * p.n_chunks * (head_dim + 2);
  if (need > 0 && (!workspace || workspace_floats < need)) return NBHS_EINVAL;
  if (n_kv_heads * p.n_sub > 65535) return NBHS_EINVAL;
  if (head_dim == 64)
    return launch_decode<64>(q, k, v, out, n, pos0, n_heads, n_kv_heads, workspace, p, qscale, q_rope, q_rope_neox,
                             app, s);
  return launch_decode<128>(q, k, v, out, n, pos0, n_heads, n_kv_heads, workspace, p, qscale, q_rope, q_rope_neox,
                            app, s);
}

}  // namespace

extern "C" {

int64_t nbhs_attn_decode_workspace(int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                   int cu_count) {
  if (n <= 0 || pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0) return -1;
  if (!tiled_head_dim(head_dim)) return 0;
  const Plan p = make_plan(n, pos0, n_heads, n_kv_heads, head_dim, cu_count);
  if (p.n_chunks == 1) return 0;
  return n * n_heads * p.n_chunks * (head_dim + 2);
}

int64_t nbhs_attn_decode_workspace_bound(int64_t n_heads, int cu_count) {
  // With T = the workgroup target, a call with n rows that splits at all uses at most T / n chunks per query head,
  // so n * chunks <= T (the bound keeps twice that); each partial holds at most 128 + 2 floats per query head.
  if (n_heads <= 0) return -1;
  const int64_t slots = int64_t(cu_count > 0 ? cu_count : 256) *
                        (NBH_DECODE_WG_PER_CU_LONG > NBH_DECODE_WG_PER_CU ? NBH_DECODE_WG_PER_CU_LONG
                                                                         : NBH_DECODE_WG_PER_CU);
  return n_heads * (2 * slots + 16) * (128 + 2);
}

int nbhs_attn_decode_f32(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                         int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, float* workspace,
                         int64_t workspace_floats, int cu_count, const float* q_rope_cs, int64_t q_rope_rows,
                         int q_rope_neox, nbhs_stream stream) {
  return decode(q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim, workspace, workspace_floats, cu_count,
                q_rope_cs, q_rope_rows, q_rope_neox, Append{}, reinterpret_cast<hipStream_t>(stream));
}

int nbhs_append_attn_decode_f32(const float* q, float* k_cache, float* v_cache, const float* k_new,
                                const float* v_new, float* out, int64_t pos0, int64_t n_heads, int64_t n_kv_heads,
                                int64_t head_dim, float* workspace, int64_t workspace_floats, int cu_count,
                                const float* rope_cs, int64_t rope_rows, int neox, nbhs_stream stream) {
  // One query row, tiled head sizes, RoPE table required (it rotates q and the new K row alike).
  if (!k_new || !v_new || !rope_cs || !tiled_head_dim(head_dim)) return NBHS_EINVAL;
  Append app;
  app.k_new = k_new;
  app.v_new = v_new;
  app.k_dst = k_cache;
  app.v_dst = v_cache;
  return decode(q, k_cache, v_cache, out, 1, pos0, n_heads, n_kv_heads, head_dim, workspace, workspace_floats,
                cu_count, rope_cs, rope_rows, neox, app, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
