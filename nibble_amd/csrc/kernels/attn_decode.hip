// fp32 causal GQA attention for few query rows (decode): Backend::attention (backend.h:68-69) with the semantics
// of ref_ops.cpp:188-214 - row t attends to cache rows 0..pos0+t, query head h reads KV head h / (H/KV).
//
// Design (CDNA4, wave64, HBM-bound: arithmetic intensity H/(2*KV) FLOP/B, far below the fp32 ridge):
//  * Grid = (context chunk, KV head x head subgroup, query row). A workgroup streams one chunk of one KV head
//    and serves every query head of its GQA group from registers, so each K/V byte is read from HBM once per
//    step, not once per query head.
//  * A 64-float K/V row is 16 lanes x float4 (256 B, one coalesced segment); a wave covers 4 rows per load and
//    keeps 4 loads of K and 4 of V in flight per lane. Dot products reduce over the 16 lanes with DPP (no LDS).
//  * Online softmax in the log2 domain per lane (queries pre-scaled by log2(e)/sqrt(d)), merged across the
//    wave's row groups with shuffles and across the workgroup's waves through LDS.
//  * Each workgroup writes an unnormalised partial (max, sum, weighted V) per query head; attn_decode_combine
//    merges the chunks with a log-sum-exp reduction. With a single chunk the partial kernel writes the output.
#include <hip/hip_runtime.h>

#include <cmath>

#include "backend/hip/kernel_timing.h"
#include "nibble_hip_shim.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kDecodeThreads = 256;  // 4 waves
constexpr int kUnroll = 4;           // row loads in flight per lane per tensor
constexpr int kMaxChunks = 4096;     // partials per (row, head); bounds the combine kernel's LDS table

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of LPR lanes (16 or 32); every lane of the group gets the bit-identical sum
// (each step adds a lane's value to its partner's, and a + b == b + a).
template <int LPR>
__device__ __forceinline__ float group_sum(float x) {
  x += dpp<0xB1>(x);   // quad_perm(1,0,3,2): lane ^ 1
  x += dpp<0x4E>(x);   // quad_perm(2,3,0,1): lane ^ 2
  x += dpp<0x141>(x);  // row_half_mirror: lane i <-> 7 - i within 8 (joins the two quads)
  x += dpp<0x140>(x);  // row_mirror: lane i <-> 15 - i within 16 (joins the two halves)
  if constexpr (LPR == 32) x += __shfl_xor(x, 16, 64);
  return x;
}

// Merge (m, l, o) online-softmax states: the result describes the union of the rows both covered.
__device__ __forceinline__ void merge_state(float& m, float& l, float4& o, float mo, float lo, float4 oo) {
  const float mn = fmaxf(m, mo);
  const float ms = mn == -INFINITY ? 0.0f : mn;
  const float a = exp2f(m - ms), b = exp2f(mo - ms);
  l = l * a + lo * b;
  o.x = o.x * a + oo.x * b;
  o.y = o.y * a + oo.y * b;
  o.z = o.z * a + oo.z * b;
  o.w = o.w * a + oo.w * b;
  m = mn;
}

__device__ __forceinline__ float4 shfl_xor4(float4 v, int mask) {
  return make_float4(__shfl_xor(v.x, mask, 64), __shfl_xor(v.y, mask, 64), __shfl_xor(v.z, mask, 64),
                     __shfl_xor(v.w, mask, 64));
}

// HD: head_dim (64 or 128). GB: query heads per workgroup (the GQA group, or a slice of it).
template <int HD, int GB>
__global__ __launch_bounds__(kDecodeThreads) void attn_decode_partial(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ out,
    float* __restrict__ ws_o, float* __restrict__ ws_ml, int64_t pos0, int n_heads, int n_kv, int group, int n_sub,
    int64_t chunk_len, int n_chunks, float qscale) {
  constexpr int LPR = HD / 4;                      // lanes per K/V row
  constexpr int RPS = 64 / LPR;                    // rows per wave load
  constexpr int WAVE_ROWS = RPS * kUnroll;         // rows per wave iteration
  constexpr int NW = kDecodeThreads / 64;          // waves per workgroup
  __shared__ float sm_m[NW][GB], sm_l[NW][GB];
  __shared__ float4 sm_o[NW][GB][LPR];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, dl = lane % LPR;
  const int chunk = blockIdx.x;
  const int g = blockIdx.y / n_sub, sg = blockIdx.y % n_sub;
  const int64_t t = blockIdx.z;
  const int h0 = g * group + sg * GB;
  const int gcount = min(GB, group - sg * GB);
  const int64_t len = pos0 + t + 1;
  const int64_t c0 = int64_t(chunk) * chunk_len;
  const int64_t c1 = min(c0 + chunk_len, len);

  float4 qv[GB];
  float m[GB], l[GB];
  float4 o[GB];
#pragma unroll
  for (int h = 0; h < GB; ++h) {
    qv[h] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (h < gcount) {
      const float4 x = *reinterpret_cast<const float4*>(q + (t * n_heads + h0 + h) * HD + 4 * dl);
      qv[h] = make_float4(x.x * qscale, x.y * qscale, x.z * qscale, x.w * qscale);
    }
    m[h] = -INFINITY;
    l[h] = 0.f;
    o[h] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  const int64_t row_stride = int64_t(n_kv) * HD;
  const float* kb = k + int64_t(g) * HD + 4 * dl;
  const float* vb = v + int64_t(g) * HD + 4 * dl;
  for (int64_t base = c0 + wave * WAVE_ROWS; base < c1; base += NW * WAVE_ROWS) {
    float4 kr[kUnroll], vr[kUnroll];
    bool valid[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = base + u * RPS + sub;
      valid[u] = j < c1;
      const int64_t jj = valid[u] ? j : c0;  // rows past the chunk are never read: clamp to a valid row
      kr[u] = *reinterpret_cast<const float4*>(kb + jj * row_stride);
      vr[u] = *reinterpret_cast<const float4*>(vb + jj * row_stride);
    }
#pragma unroll
    for (int h = 0; h < GB; ++h) {
      if (h >= gcount) continue;
      float s[kUnroll];
      float mloc = -INFINITY;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        float d = qv[h].x * kr[u].x;
        d = fmaf(qv[h].y, kr[u].y, d);
        d = fmaf(qv[h].z, kr[u].z, d);
        d = fmaf(qv[h].w, kr[u].w, d);
        d = group_sum<LPR>(d);
        s[u] = valid[u] ? d : -INFINITY;
        mloc = fmaxf(mloc, s[u]);
      }
      const float mn = fmaxf(m[h], mloc);
      const float ms = mn == -INFINITY ? 0.0f : mn;
      const float corr = exp2f(m[h] - ms);
      float lh = l[h] * corr;
      float4 oh = make_float4(o[h].x * corr, o[h].y * corr, o[h].z * corr, o[h].w * corr);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const float p = exp2f(s[u] - ms);
        lh += p;
        oh.x = fmaf(p, vr[u].x, oh.x);
        oh.y = fmaf(p, vr[u].y, oh.y);
        oh.z = fmaf(p, vr[u].z, oh.z);
        oh.w = fmaf(p, vr[u].w, oh.w);
      }
      m[h] = mn;
      l[h] = lh;
      o[h] = oh;
    }
  }

  // Merge the wave's row groups (lanes dl, dl + LPR, ...), then the waves through LDS.
#pragma unroll
  for (int h = 0; h < GB; ++h) {
#pragma unroll
    for (int mask = LPR; mask < 64; mask <<= 1) {
      const float mo = __shfl_xor(m[h], mask, 64), lo = __shfl_xor(l[h], mask, 64);
      const float4 oo = shfl_xor4(o[h], mask);
      merge_state(m[h], l[h], o[h], mo, lo, oo);
    }
    if (lane < LPR) {
      sm_o[wave][h][dl] = o[h];
      if (lane == 0) {
        sm_m[wave][h] = m[h];
        sm_l[wave][h] = l[h];
      }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < GB * LPR; idx += kDecodeThreads) {
    const int h = idx / LPR, d4 = idx % LPR;
    if (h >= gcount) continue;
    float mm = sm_m[0][h], ll = sm_l[0][h];
    float4 oo = sm_o[0][h][d4];
#pragma unroll
    for (int w = 1; w < NW; ++w) merge_state(mm, ll, oo, sm_m[w][h], sm_l[w][h], sm_o[w][h][d4]);
    const int64_t head = h0 + h;
    if (n_chunks == 1) {
      const float inv = 1.0f / ll;
      *reinterpret_cast<float4*>(out + (t * n_heads + head) * HD + 4 * d4) =
          make_float4(oo.x * inv, oo.y * inv, oo.z * inv, oo.w * inv);
    } else {
      const int64_t slot = (t * n_heads + head) * n_chunks + chunk;
      *reinterpret_cast<float4*>(ws_o + slot * HD + 4 * d4) = oo;
      if (d4 == 0) {
        ws_ml[2 * slot] = mm;
        ws_ml[2 * slot + 1] = ll;
      }
    }
  }
}

// Log-sum-exp merge of the chunk partials: one wave per (row, head).
template <int HD>
__global__ __launch_bounds__(64) void attn_decode_combine(const float* __restrict__ ws_o,
                                                          const float* __restrict__ ws_ml, float* __restrict__ out,
                                                          int n_chunks) {
  __shared__ float w[kMaxChunks];
  const int lane = threadIdx.x;
  const int64_t rh = blockIdx.x;  // t * n_heads + head
  const float* ml = ws_ml + rh * n_chunks * 2;
  float mx = -INFINITY;
  for (int c = lane; c < n_chunks; c += 64) mx = fmaxf(mx, ml[2 * c]);
#pragma unroll
  for (int mask = 1; mask < 64; mask <<= 1) mx = fmaxf(mx, __shfl_xor(mx, mask, 64));
  const float ms = mx == -INFINITY ? 0.0f : mx;
  float lsum = 0.f;
  for (int c = lane; c < n_chunks; c += 64) {
    const float wc = exp2f(ml[2 * c] - ms);
    w[c] = wc;
    lsum += ml[2 * c + 1] * wc;
  }
#pragma unroll
  for (int mask = 1; mask < 64; mask <<= 1) lsum += __shfl_xor(lsum, mask, 64);
  __syncthreads();
  const float inv = 1.0f / lsum;
  const float* po = ws_o + rh * n_chunks * HD;
#pragma unroll
  for (int d = lane; d < HD; d += 64) {
    float acc = 0.f;
    for (int c = 0; c < n_chunks; ++c) acc = fmaf(po[int64_t(c) * HD + d], w[c], acc);
    out[rh * HD + d] = acc * inv;
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
  int gb;            // heads per workgroup (1, 2, 4 or 8)
  int n_sub;         // head subgroups per KV head
  int n_chunks;
  int64_t chunk_len;
};

Plan make_plan(int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv, int cu_count) {
  Plan p;
  const int64_t group = n_heads / n_kv;
  p.gb = group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 ? 4 : 8;
  p.n_sub = int((group + p.gb - 1) / p.gb);
  const int64_t max_len = pos0 + n;
  // Aim for ~4 workgroups per CU in total; chunks shorter than 64 rows do not pay for their partial.
  const int64_t target = int64_t(cu_count > 0 ? cu_count : 256) * 4;
  const int64_t per_chunk_groups = n * n_kv * p.n_sub;
  int64_t chunks = (target + per_chunk_groups - 1) / per_chunk_groups;
  const int64_t max_by_len = (max_len + 63) / 64;
  if (chunks > max_by_len) chunks = max_by_len;
  if (chunks < 1) chunks = 1;
  if (chunks > kMaxChunks) chunks = kMaxChunks;
  p.chunk_len = (max_len + chunks - 1) / chunks;
  p.n_chunks = int((max_len + p.chunk_len - 1) / p.chunk_len);
  return p;
}

template <int HD>
int launch_decode(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0, int64_t H,
                  int64_t KV, float* ws, const Plan& p, float qscale, hipStream_t s) {
  const dim3 grid(p.n_chunks, unsigned(KV * p.n_sub), unsigned(n));
  float* ws_o = ws;
  float* ws_ml = ws ? ws + n * H * p.n_chunks * HD : nullptr;
  const int group = int(H / KV);
#define NBH_DECODE(GB)                                                                                              \
  attn_decode_partial<HD, GB><<<grid, kDecodeThreads, 0, s>>>(q, k, v, out, ws_o, ws_ml, pos0, int(H), int(KV), \
                                                               group, p.n_sub, p.chunk_len, p.n_chunks, qscale)
  {
  nbhs_timing::KernelTimer timer(NBHS_K_DECODE_PARTIAL, s);
  switch (p.gb) {
    case 1: NBH_DECODE(1); break;
    case 2: NBH_DECODE(2); break;
    case 4: NBH_DECODE(4); break;
    default: NBH_DECODE(8); break;
  }
  }
#undef NBH_DECODE
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.n_chunks == 1) return e;
  nbhs_timing::KernelTimer timer(NBHS_K_DECODE_COMBINE, s);
  attn_decode_combine<HD><<<unsigned(n * H), 64, 0, s>>>(ws_o, ws_ml, out, p.n_chunks);
  return hipGetLastError();
}

bool tiled_head_dim(int64_t hd) { return hd == 64 || hd == 128; }

}  // namespace

extern "C" {

int64_t nbhs_attn_decode_workspace(int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                   int cu_count) {
  if (n <= 0 || pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0) return -1;
  if (!tiled_head_dim(head_dim)) return 0;
  const Plan p = make_plan(n, pos0, n_heads, n_kv_heads, cu_count);
  if (p.n_chunks == 1) return 0;
  return n * n_heads * p.n_chunks * (head_dim + 2);
}

int nbhs_attn_decode_f32(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                         int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, float* workspace,
                         int64_t workspace_floats, int cu_count, nbhs_stream stream) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (!q || !k || !v || !out || n <= 0 || n > 65535 || pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 ||
      n_heads % n_kv_heads != 0 || head_dim <= 0 || head_dim > 256 || n_heads > 65535)
    return NBHS_EINVAL;
  const float qscale = (1.0f / std::sqrt(float(head_dim))) * kLog2e;
  if (!tiled_head_dim(head_dim)) {
    nbhs_timing::KernelTimer timer(NBHS_K_GENERIC, s);
    attn_generic<<<dim3(unsigned(n_heads), unsigned(n)), 64, 0, s>>>(q, k, v, out, pos0, int(n_heads),
                                                                     int(n_kv_heads), int(head_dim), qscale);
    return hipGetLastError();
  }
  const Plan p = make_plan(n, pos0, n_heads, n_kv_heads, cu_count);
  const int64_t need = p.n_chunks == 1 ? 0 : n * n_heads * p.n_chunks * (head_dim + 2);
  if (need > 0 && (!workspace || workspace_floats < need)) return NBHS_EINVAL;
  if (n_kv_heads * p.n_sub > 65535) return NBHS_EINVAL;
  if (head_dim == 64) return launch_decode<64>(q, k, v, out, n, pos0, n_heads, n_kv_heads, workspace, p, qscale, s);
  return launch_decode<128>(q, k, v, out, n, pos0, n_heads, n_kv_heads, workspace, p, qscale, s);
}

}  // extern "C"
