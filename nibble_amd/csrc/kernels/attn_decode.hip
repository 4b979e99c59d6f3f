// fp32 causal GQA attention for few query rows (decode): Backend::attention (backend.h:68-69) with the semantics
// of ref_ops.cpp:188-214 - row t attends to cache rows 0..pos0+t, query head h reads KV head h / (H/KV).
//
// The per-workgroup body is partial_block (kernels/decode_block.h), shared with the prefill kernel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>

#include "backend/hip/kernel_timing.h"
#include "kernels/decode_block.h"
#include "kernels/decode_rows.h"
#include "nibble_hip_shim.h"

namespace {

using namespace nbh_decode;

template <int HD, int GB, typename KV>
__global__ __launch_bounds__(kDecodeThreads) void attn_decode_partial(
    const float* __restrict__ q, const KV* __restrict__ k, const KV* __restrict__ v, float* __restrict__ out,
    float* __restrict__ ws_o, float* __restrict__ ws_ml, int64_t pos0, int n_heads, int n_kv, int group, int n_sub,
    int n_chunks, int64_t groups_per_chunk, int64_t extra_groups, float qscale, const float2* __restrict__ q_rope,
    int q_rope_neox, const float* __restrict__ k_new, const float* __restrict__ v_new, KV* __restrict__ k_dst,
    KV* __restrict__ v_dst) {
  partial_block<HD, GB, KV>(q, k, v, out, ws_o, ws_ml, pos0, n_heads, n_kv, group, n_sub, n_chunks, groups_per_chunk,
                        extra_groups, qscale, q_rope, q_rope_neox, k_new, v_new, k_dst, v_dst, blockIdx.x, blockIdx.y,
                        blockIdx.z);
}

// One workgroup per (row, head): rh = t * n_heads + head.
template <int HD>
__global__ __launch_bounds__(kDecodeThreads) void attn_decode_combine(const float* __restrict__ ws_o,
                                                                      const float* __restrict__ ws_ml,
                                                                      float* __restrict__ out, int n_chunks) {
  combine_block<HD>(ws_o, ws_ml, out, n_chunks, blockIdx.x);
}

// ---- ragged batch: one query row per sequence, each over its own cache and context length ----
// The launch's sequences travel by value in the kernel arguments (no device-side table to upload). Workgroup x of
// the partial kernel belongs to the sequence whose chunk range [chunk0, chunk0 + n_chunks) holds x; the chunks are
// shared out over the sequences in proportion to their lengths, so one launch streams every cache at once.
constexpr int kMaxBatch = 32;
struct SeqDesc {
  const float* q;      // [n_heads, HD], the sequence's query row
  const float* k;      // the sequence's caches [>= pos0 + 1 rows, n_kv, HD]
  const float* v;
  float* out;          // [n_heads, HD]
  const float* k_new;  // appended row [n_kv, HD] (null: nothing appended)
  const float* v_new;
  float* ws_o;         // partials [n_heads, n_chunks, HD] and [n_heads, n_chunks, 2] (n_chunks > 1)
  float* ws_ml;
  int64_t pos0;        // position of the query row; it attends to rows 0..pos0
  int64_t groups_per_chunk, extra_groups;
  int chunk0, n_chunks;
};
struct Batch {
  SeqDesc s[kMaxBatch];
  int n_seq;
};

__device__ __forceinline__ int batch_seq_of(const Batch& b, int x) {
  int s = 0;
  for (int i = 1; i < b.n_seq; ++i)
    if (x >= b.s[i].chunk0) s = i;
  return s;
}

template <int HD, int GB>
__global__ __launch_bounds__(kDecodeThreads) void attn_decode_batch_partial(Batch b, int n_heads, int n_kv, int group,
                                                                            int n_sub, float qscale,
                                                                            const float2* __restrict__ q_rope,
                                                                            int q_rope_neox) {
  const SeqDesc& d = b.s[batch_seq_of(b, blockIdx.x)];
  partial_block<HD, GB>(d.q, d.k, d.v, d.out, d.ws_o, d.ws_ml, d.pos0, n_heads, n_kv, group, n_sub, d.n_chunks,
                        d.groups_per_chunk, d.extra_groups, qscale, q_rope, q_rope_neox, d.k_new, d.v_new,
                        const_cast<float*>(d.k), const_cast<float*>(d.v), int(blockIdx.x) - d.chunk0, blockIdx.y, 0);
}

// One workgroup per (sequence, head); sequences that took a single chunk were written by the partial kernel.
template <int HD>
__global__ __launch_bounds__(kDecodeThreads) void attn_decode_batch_combine(Batch b, int n_heads) {
  const SeqDesc& d = b.s[blockIdx.x / n_heads];
  if (d.n_chunks == 1) return;
  combine_block<HD>(d.ws_o, d.ws_ml, d.out, d.n_chunks, blockIdx.x % n_heads);
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

// Workgroups of attn_decode_partial<HD, GB, KV> that fit on one CU at once (register and LDS limits), capped at
// NBH_DECODE_WG_PER_CU_LONG; queried from the runtime once per instance. The fp16-cache instance holds twice the row
// slots per lane, so its register count, and with it the fit, can differ from the fp32 one.
template <int HD, int GB, typename KV>
int resident_per_cu() {
  static const int n = [] {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, attn_decode_partial<HD, GB, KV>, kDecodeThreads, 0) !=
            hipSuccess ||
        b < 1)
      b = 1;
    return b < NBH_DECODE_WG_PER_CU_LONG ? b : NBH_DECODE_WG_PER_CU_LONG;
  }();
  return n;
}

template <typename KV>
int resident_per_cu(int64_t head_dim, int gb) {
  if (head_dim == 64)
    return gb == 1 ? resident_per_cu<64, 1, KV>() : gb == 2 ? resident_per_cu<64, 2, KV>()
         : gb == 4 ? resident_per_cu<64, 4, KV>() : resident_per_cu<64, 8, KV>();
  return gb == 1 ? resident_per_cu<128, 1, KV>() : gb == 2 ? resident_per_cu<128, 2, KV>()
       : gb == 4 ? resident_per_cu<128, 4, KV>() : resident_per_cu<128, 8, KV>();
}

// As many workgroups as fit on the chip at once: one round, no tail of late starters. The row groups are split
// evenly over min(slots, groups) chunks; the remainder goes one group each to the first chunks, which load that
// group together with their first one (see attn_decode_partial), so a context one row past a round size costs no
// workgroup an extra HBM round trip and no workgroup waits for a free slot.
//
// single_chunk: every (row, head subgroup) in one workgroup over its whole window, key groups in position order (the
// ordered route): a row's summation then depends on its own keys only, not on the call's other rows or its length.
template <typename KV = float>
Plan make_plan(int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv, int64_t head_dim, int cu_count,
               bool single_chunk = false) {
  const int unroll = unroll_for(int(sizeof(KV)));
  Plan p;
  const int64_t group = n_heads / n_kv;
  p.gb = group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 ? 4 : 8;
  p.n_sub = int((group + p.gb - 1) / p.gb);
  const int64_t max_len = pos0 + n;
  const int64_t lpr = head_dim / 8;
  const int64_t step = (64 / lpr) * unroll * (kDecodeThreads / 64);  // rows a workgroup covers per iteration
  const int64_t units = (max_len + step - 1) / step;
  const int64_t cus = cu_count > 0 ? cu_count : 256;
  const int64_t streams = n * n_kv * p.n_sub;  // workgroups per chunk index
  const int resident = resident_per_cu<KV>(head_dim, p.gb);
  int64_t slots = cus * resident / streams;
  if (resident > NBH_DECODE_WG_PER_CU && units < kLongGroups * slots)
    slots = cus * NBH_DECODE_WG_PER_CU / streams;  // short context: fewer, longer workgroups
  if (slots < 1 || single_chunk) slots = 1;
  int64_t chunks = units < slots ? units : slots;
  if (chunks > kMaxChunks) chunks = kMaxChunks;
  p.n_chunks = int(chunks);
  p.groups_per_chunk = units / chunks;
  p.extra_groups = units % chunks;
  return p;
}

// Appended row of a single-row call: new K/V rows in (fp32), cache rows out (all null when nothing is appended).
template <typename KVT>
struct Append {
  const float* k_new = nullptr;
  const float* v_new = nullptr;
  KVT* k_dst = nullptr;
  KVT* v_dst = nullptr;
};

template <int HD, typename KVT>
int launch_decode(const float* q, const KVT* k, const KVT* v, float* out, int64_t n, int64_t pos0, int64_t H,
                  int64_t KV, float* ws, const Plan& p, float qscale, const float2* q_rope, int q_rope_neox,
                  const Append<KVT>& app, hipStream_t s) {
  float* ws_o = ws;
  float* ws_ml = ws ? ws + n * H * p.n_chunks * HD : nullptr;
  const int group = int(H / KV);
  const dim3 grid(p.n_chunks, unsigned(KV * p.n_sub), unsigned(n));
  hipError_t e;
#define NBH_DECODE(GB)                                                                                             \
  e = nbhs_timing::launch(NBHS_K_DECODE_PARTIAL, attn_decode_partial<HD, GB, KVT>, grid, dim3(kDecodeThreads), s, q, \
                          k,                                                                                        \
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

// n appended rows into fp16 caches: K rotated exactly as the fp32 append does (rope_rotate in fp32, the table of
// the RoPE kernel), then both K and V rounded to fp16. One thread per rotation pair (and the matching V pair).
__global__ __launch_bounds__(256) void append_rope_f16_kernel(_Float16* __restrict__ k16, _Float16* __restrict__ v16,
                                                              const float* __restrict__ kn,
                                                              const float* __restrict__ vn, int64_t n, int64_t pos0,
                                                              int64_t n_kv, int64_t hd,
                                                              const float2* __restrict__ cs, int neox) {
  const int64_t h2 = hd / 2, pairs = n * n_kv * h2;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < pairs; i += int64_t(gridDim.x) * 256) {
    const int64_t row = i / (n_kv * h2), rem = i % (n_kv * h2), g = rem / h2, j = rem % h2;
    const int64_t a = neox ? j : 2 * j, b = neox ? j + h2 : 2 * j + 1;  // the pair's two dimensions
    const int64_t src = (row * n_kv + g) * hd, dst = ((pos0 + row) * n_kv + g) * hd;
    float x = kn[src + a], y = kn[src + b];
    rope_rotate(x, y, cs[(pos0 + row) * h2 + j]);
    k16[dst + a] = _Float16(x);
    k16[dst + b] = _Float16(y);
    v16[dst + a] = _Float16(vn[src + a]);
    v16[dst + b] = _Float16(vn[src + b]);
  }
}

bool tiled_head_dim(int64_t hd) { return hd == 64 || hd == 128; }

// The whole-row route (attn_decode_rows, kernels/decode_rows.h): one query row, head_dim 64 or 128, a KV-head count
// that whole waves cover (a multiple of 8 at hd 64, of 4 at hd 128, in at most kRowsWaves head chunks), GQA group
// 1, 2 or 4. Other single-row shapes, and calls of several rows, take the per-head split kernel.
bool rows_route(int64_t n, int64_t n_heads, int64_t n_kv, int64_t hd) {
  if (n != 1 || !tiled_head_dim(hd) || n_kv <= 0 || n_heads % n_kv != 0) return false;
  const int64_t hpw = 64 / (hd / 8), group = n_heads / n_kv;
  if (n_kv % hpw != 0 || kRowsWaves % (n_kv / hpw) != 0) return false;
  return group == 1 || group == 2 || group == 4;
}

// Workgroups of a whole-row launch: one per CU, fewer for short contexts so that every wave stream holds at least
// kRowsMinBlocks row blocks.
constexpr int64_t kRowsMinBlocks = 4;
// Positions the whole-row kernel takes (its row-block bookkeeping is 32-bit); later ones go to the per-head kernel.
constexpr int64_t kRowsMaxPos = int64_t(1) << 30;
template <typename KV>
int64_t rows_grid(int64_t pos0, int64_t n_kv, int64_t hd, int cu_count) {
  const int64_t hc = n_kv / (64 / (hd / 8));
  const int64_t nblk = (pos0 + rows_per_block<KV>()) / rows_per_block<KV>();  // blocks of rows 0..pos0
  const int64_t want = (nblk * hc + kRowsWaves * kRowsMinBlocks - 1) / (kRowsWaves * kRowsMinBlocks);
  return std::clamp<int64_t>(want, 1, cu_count > 0 ? cu_count : 256);
}

// Workspace floats of a whole-row call (the partials of its workgroups; 0 with one workgroup).
template <typename KV>
int64_t rows_workspace(int64_t pos0, int64_t n_heads, int64_t n_kv, int64_t hd, int cu_count) {
  const int64_t G = rows_grid<KV>(pos0, n_kv, hd, cu_count);
  return G == 1 ? 0 : n_heads * G * (hd + 2);
}

template <int HD, typename KVT>
int launch_rows(const float* q, const KVT* k, const KVT* v, float* out, int64_t pos0, int64_t H, int64_t KV,
                float* ws, int64_t G, float qscale, const float2* q_rope, int q_rope_neox, const Append<KVT>& app,
                hipStream_t s) {
  float* ws_o = ws;
  float* ws_ml = ws ? ws + H * G * HD : nullptr;
  hipError_t e;
#define NBH_ROWS(GRP)                                                                                              \
  e = nbhs_timing::launch(NBHS_K_DECODE_PARTIAL,                                                                   \
                          q_rope ? attn_decode_rows<HD, GRP, KVT, true> : attn_decode_rows<HD, GRP, KVT, false>,   \
                          dim3(unsigned(G)), dim3(kRowsWaves * 64), s, q, k, v, out, ws_o, ws_ml, pos0, int(KV),   \
                          qscale, q_rope, q_rope_neox, app.k_new, app.v_new, app.k_dst, app.v_dst)
  switch (H / KV) {
    case 1: NBH_ROWS(1); break;
    case 2: NBH_ROWS(2); break;
    default: NBH_ROWS(4); break;
  }
#undef NBH_ROWS
  if (e != hipSuccess || G == 1) return e;
  return nbhs_timing::launch(NBHS_K_DECODE_COMBINE, attn_decode_combine<HD>, dim3(unsigned(H)), dim3(kDecodeThreads),
                             s, ws_o, ws_ml, out, int(G));
}

// allow_rows: single-row calls of the whole-row shapes take attn_decode_rows (off: the per-head split kernel, for
// callers whose workspace is sized for it alone).
template <typename KVT>
int decode(const float* q, const KVT* k, const KVT* v, float* out, int64_t n, int64_t pos0, int64_t n_heads,
           int64_t n_kv_heads, int64_t head_dim, float* workspace, int64_t workspace_floats, int cu_count,
           const float* q_rope_cs, int64_t q_rope_rows, int q_rope_neox, const Append<KVT>& app, hipStream_t s,
           bool allow_rows = true, bool single_chunk = false) {
  if (!q || !k || !v || !out || n <= 0 || n > 65535 || pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 ||
      n_heads % n_kv_heads != 0 || head_dim <= 0 || head_dim > 256 || n_heads > 65535)
    return NBHS_EINVAL;
  // q rotation on load is implemented for the tiled head sizes only, over table rows covering pos0 .. pos0+n-1
  if (q_rope_cs && (!tiled_head_dim(head_dim) || pos0 + n > q_rope_rows)) return NBHS_EINVAL;
  const float2* q_rope = reinterpret_cast<const float2*>(q_rope_cs);
  const float qscale = (1.0f / std::sqrt(float(head_dim))) * kLog2e;
  if (!tiled_head_dim(head_dim)) {
    if constexpr (sizeof(KVT) != 4) {
      return NBHS_EINVAL;  // fp16 caches: the tiled head sizes only
    } else {
      return nbhs_timing::launch(NBHS_K_GENERIC, attn_generic, dim3(unsigned(n_heads), unsigned(n)), dim3(64), s, q,
                                 k, v, out, pos0, int(n_heads), int(n_kv_heads), int(head_dim), qscale);
    }
  }
  if (allow_rows && !single_chunk && rows_route(n, n_heads, n_kv_heads, head_dim) && pos0 < kRowsMaxPos) {
    const int64_t G = rows_grid<KVT>(pos0, n_kv_heads, head_dim, cu_count);
    const int64_t need = G == 1 ? 0 : n_heads * G * (head_dim + 2);
    if (need > 0 && (!workspace || workspace_floats < need)) return NBHS_EINVAL;
    if (head_dim == 64)
      return launch_rows<64>(q, k, v, out, pos0, n_heads, n_kv_heads, workspace, G, qscale, q_rope, q_rope_neox, app,
                             s);
    return launch_rows<128>(q, k, v, out, pos0, n_heads, n_kv_heads, workspace, G, qscale, q_rope, q_rope_neox, app,
                            s);
  }
  // (nbhs_attn_decode_workspace covers the plans of both cache types)
  const Plan p = make_plan<KVT>(n, pos0, n_heads, n_kv_heads, head_dim, cu_count, single_chunk);
  const int64_t need = p.n_chunks == 1 ? 0 : n * n_heads * p.n_chunks * (head_dim + 2);
  if (need > 0 && (!workspace || workspace_floats < need)) return NBHS_EINVAL;
  if (n_kv_heads * p.n_sub > 65535) return NBHS_EINVAL;
  if (head_dim == 64)
    return launch_decode<64>(q, k, v, out, n, pos0, n_heads, n_kv_heads, workspace, p, qscale, q_rope, q_rope_neox,
                             app, s);
  return launch_decode<128>(q, k, v, out, n, pos0, n_heads, n_kv_heads, workspace, p, qscale, q_rope, q_rope_neox,
                            app, s);
}

// Workspace floats of the per-head split kernel for either cache type.
int64_t perhead_workspace(int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                          int cu_count) {
  const int chunks = std::max(make_plan<float>(n, pos0, n_heads, n_kv_heads, head_dim, cu_count).n_chunks,
                              make_plan<_Float16>(n, pos0, n_heads, n_kv_heads, head_dim, cu_count).n_chunks);
  return chunks == 1 ? 0 : n * n_heads * chunks * (head_dim + 2);
}

// Chunk layout of one batch launch (sequences pos0[0..n) with n <= kMaxBatch): the workgroup slots that fit on the
// chip (as make_plan counts them) are shared out over the sequences so that the largest number of row groups any
// one chunk streams - what the launch's duration follows - is as small as the slots allow: the least T for which
// chunks of at most T groups (sum over sequences of ceil(groups / T)) fit the slots, by bisection. Fills the
// scheduling fields of b and returns the workspace floats the launch needs.
int64_t batch_layout(int64_t n, const int64_t* pos0, int64_t n_heads, int64_t n_kv, int64_t head_dim, int cu_count,
                     Batch* b, int* gb, int* n_sub) {
  const int64_t group = n_heads / n_kv;
  *gb = group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 ? 4 : 8;
  *n_sub = int((group + *gb - 1) / *gb);
  const int64_t step = (64 / (head_dim / 8)) * kUnroll * (kDecodeThreads / 64);
  int64_t total = 0;
  for (int64_t i = 0; i < n; ++i) total += (pos0[i] + 1 + step - 1) / step;
  const int64_t cus = cu_count > 0 ? cu_count : 256;
  const int64_t streams = n_kv * *n_sub;
  const int resident = resident_per_cu<float>(head_dim, *gb);
  int64_t slots = cus * resident / streams;
  if (resident > NBH_DECODE_WG_PER_CU && total < kLongGroups * slots) slots = cus * NBH_DECODE_WG_PER_CU / streams;
  if (slots < n) slots = n;  // every sequence takes at least one chunk
  auto chunks_of = [&](int64_t units, int64_t t) {
    return std::min<int64_t>((units + t - 1) / t, kMaxChunks);
  };
  auto fits = [&](int64_t t) {
    int64_t c = 0;
    for (int64_t i = 0; i < n; ++i) c += chunks_of((pos0[i] + 1 + step - 1) / step, t);
    return c <= slots;
  };
  int64_t lo = std::max<int64_t>(1, (total + slots - 1) / slots), hi = 1;
  for (int64_t i = 0; i < n; ++i) hi = std::max(hi, (pos0[i] + 1 + step - 1) / step);
  while (lo < hi) {  // least T that fits (T = the longest sequence's groups always does)
    const int64_t mid = lo + (hi - lo) / 2;
    if (fits(mid))
      hi = mid;
    else
      lo = mid + 1;
  }
  int64_t ws = 0;
  int chunk0 = 0;
  b->n_seq = int(n);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t units = (pos0[i] + 1 + step - 1) / step;
    const int64_t c = chunks_of(units, lo);
    SeqDesc& d = b->s[i];
    d.pos0 = pos0[i];
    d.chunk0 = chunk0;
    d.n_chunks = int(c);
    d.groups_per_chunk = units / c;
    d.extra_groups = units % c;
    chunk0 += int(c);
    if (c > 1) ws += n_heads * c * (head_dim + 2);
  }
  return ws;
}

template <int HD>
int launch_batch(Batch& b, int gb, int n_sub, int64_t H, int64_t KV, float* ws, float qscale, const float2* q_rope,
                 int q_rope_neox, hipStream_t s) {
  int64_t off = 0;
  bool merge = false;
  int chunks = 0;
  for (int i = 0; i < b.n_seq; ++i) {
    SeqDesc& d = b.s[i];
    chunks += d.n_chunks;
    if (d.n_chunks > 1) {
      d.ws_o = ws + off;
      d.ws_ml = d.ws_o + H * d.n_chunks * HD;
      off += H * d.n_chunks * (HD + 2);
      merge = true;
    } else {
      d.ws_o = d.ws_ml = nullptr;
    }
  }
  const int group = int(H / KV);
  const dim3 grid(unsigned(chunks), unsigned(KV * n_sub));
  hipError_t e;
#define NBH_BATCH(GB)                                                                                             \
  e = nbhs_timing::launch(NBHS_K_DECODE_PARTIAL, attn_decode_batch_partial<HD, GB>, grid, dim3(kDecodeThreads), s, \
                          b, int(H), int(KV), group, n_sub, qscale, q_rope, q_rope_neox)
  switch (gb) {
    case 1: NBH_BATCH(1); break;
    case 2: NBH_BATCH(2); break;
    case 4: NBH_BATCH(4); break;
    default: NBH_BATCH(8); break;
  }
#undef NBH_BATCH
  if (e != hipSuccess || !merge) return e;
  return nbhs_timing::launch(NBHS_K_DECODE_COMBINE, attn_decode_batch_combine<HD>, dim3(unsigned(b.n_seq * H)),
                             dim3(kDecodeThreads), s, b, int(H));
}

// ---- allocation-free decode: the split partials in a static device array ----
// Some callers cannot allocate device memory (code under HIP graph capture, tight serving loops). For them
// nbhs_attn_decode_noalloc runs the decode route with its split-context partials in `scratch`, a file-scope array
// every GPU the library runs on holds until the process ends. Kernels take its per-device address as an argument;
// in host code the array's name is only a stand-in for it, taken once per device with hipGetSymbolAddress.
constexpr int64_t kNoAllocScratchFloats = int64_t(1) << 20;  // 4 MiB per GPU
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];
constexpr int kNoAllocMaxDevices = 64;
struct NoAllocDevice {
  float* ptr = nullptr;  // this device's copy of `scratch`
  int cu_count = 0;
};
std::mutex g_noalloc_mu;
NoAllocDevice g_noalloc[kNoAllocMaxDevices];

// The current device's scratch address and CU count, taken at the first call on that device (with it current).
int noalloc_device(NoAllocDevice* out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kNoAllocMaxDevices) return NBHS_EINVAL;
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  NoAllocDevice& d = g_noalloc[dev];
  if (!d.ptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    int cus = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    d.cu_count = cus;
    d.ptr = static_cast<float*>(p);
  }
  *out = d;
  return hipSuccess;
}

}  // namespace

extern "C" {

int nbhs_attn_decode_noalloc(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                             int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, nbhs_stream stream) {
  if (!q || !k || !v || !out || n <= 0 || n > NBHS_DECODE_MAX_ROWS || pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 ||
      n_heads % n_kv_heads != 0 || head_dim <= 0 || head_dim > 256)
    return NBHS_EINVAL;
  NoAllocDevice d;
  const int e = noalloc_device(&d);
  if (e != hipSuccess) return e;
  if (!tiled_head_dim(head_dim)) {
    const nbhs_timing::Suppress no_events;  // a timed launch would create events
    return decode(q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim, d.ptr, kNoAllocScratchFloats, d.cu_count,
                  nullptr, 0, 0, Append<float>{}, reinterpret_cast<hipStream_t>(stream));
  }
  // The route nbh_backend_attention takes (the whole-row kernel for its shapes) when its partials fit the array,
  // else the per-head split kernel.
  const bool rows = rows_route(n, n_heads, n_kv_heads, head_dim) && pos0 < kRowsMaxPos &&
                    rows_workspace<float>(pos0, n_heads, n_kv_heads, head_dim, d.cu_count) <= kNoAllocScratchFloats;
  if (!rows && perhead_workspace(n, pos0, n_heads, n_kv_heads, head_dim, d.cu_count) > kNoAllocScratchFloats)
    return NBHS_ETOOBIG;
  const nbhs_timing::Suppress no_events;  // a timed launch would create events
  return decode(q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim, d.ptr, kNoAllocScratchFloats, d.cu_count,
                nullptr, 0, 0, Append<float>{}, reinterpret_cast<hipStream_t>(stream), rows);
}

int64_t nbhs_attn_decode_noalloc_capacity(void) { return kNoAllocScratchFloats; }

int nbhs_attn_decode_rows_route(int64_t n, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim) {
  return rows_route(n, n_heads, n_kv_heads, head_dim) ? 1 : 0;
}


int64_t nbhs_attn_decode_batch_workspace(int64_t n_seq, const int64_t* pos0, int64_t n_heads, int64_t n_kv_heads,
                                         int64_t head_dim, int cu_count) {
  if (n_seq <= 0 || !pos0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0) return -1;
  if (!tiled_head_dim(head_dim)) return -1;
  int64_t need = 0;
  for (int64_t i0 = 0; i0 < n_seq; i0 += kMaxBatch) {
    for (int64_t i = i0; i < std::min<int64_t>(n_seq, i0 + kMaxBatch); ++i)
      if (pos0[i] < 0) return -1;
    Batch b;
    int gb, n_sub;
    need = std::max(need, batch_layout(std::min<int64_t>(kMaxBatch, n_seq - i0), pos0 + i0, n_heads, n_kv_heads,
                                       head_dim, cu_count, &b, &gb, &n_sub));
  }
  return need;
}

int nbhs_attn_decode_batch_f32(int64_t n_seq, const float* const* q, const float* const* k, const float* const* v,
                               float* const* out, const float* const* k_new, const float* const* v_new,
                               const int64_t* pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                               float* workspace, int64_t workspace_floats, int cu_count, const float* rope_cs,
                               int64_t rope_rows, int neox, nbhs_stream stream) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (n_seq <= 0 || !q || !k || !v || !out || !pos0 || n_heads <= 0 || n_heads > 65535 || n_kv_heads <= 0 ||
      n_heads % n_kv_heads != 0 || !tiled_head_dim(head_dim) || (!k_new) != (!v_new) || (k_new && !rope_cs))
    return NBHS_EINVAL;
  for (int64_t i = 0; i < n_seq; ++i) {
    if (!q[i] || !k[i] || !v[i] || !out[i] || pos0[i] < 0 || (k_new && (!k_new[i] || !v_new[i])) ||
        (rope_cs && pos0[i] + 1 > rope_rows))
      return NBHS_EINVAL;
  }
  const float2* q_rope = reinterpret_cast<const float2*>(rope_cs);
  const float qscale = (1.0f / std::sqrt(float(head_dim))) * kLog2e;
  for (int64_t i0 = 0; i0 < n_seq; i0 += kMaxBatch) {  // launches of up to kMaxBatch sequences, in stream order
    const int64_t n = std::min<int64_t>(kMaxBatch, n_seq - i0);
    Batch b;
    int gb, n_sub;
    const int64_t need = batch_layout(n, pos0 + i0, n_heads, n_kv_heads, head_dim, cu_count, &b, &gb, &n_sub);
    if (need > 0 && (!workspace || workspace_floats < need)) return NBHS_EINVAL;
    if (n_kv_heads * n_sub > 65535) return NBHS_EINVAL;
    for (int64_t i = 0; i < n; ++i) {
      SeqDesc& d = b.s[i];
      d.q = q[i0 + i];
      d.k = k[i0 + i];
      d.v = v[i0 + i];
      d.out = out[i0 + i];
      d.k_new = k_new ? k_new[i0 + i] : nullptr;
      d.v_new = v_new ? v_new[i0 + i] : nullptr;
    }
    const int e = head_dim == 64
                      ? launch_batch<64>(b, gb, n_sub, n_heads, n_kv_heads, workspace, qscale, q_rope, neox, s)
                      : launch_batch<128>(b, gb, n_sub, n_heads, n_kv_heads, workspace, qscale, q_rope, neox, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

int64_t nbhs_attn_decode_workspace(int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                   int cu_count) {
  if (n <= 0 || pos0 < 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0) return -1;
  if (!tiled_head_dim(head_dim)) return 0;
  // the larger of the fp32- and fp16-cache plans (their occupancy, and so their chunk counts, can differ), of the
  // per-head split kernel and, for the whole-row shapes, of the whole-row route
  int64_t need = perhead_workspace(n, pos0, n_heads, n_kv_heads, head_dim, cu_count);
  if (rows_route(n, n_heads, n_kv_heads, head_dim))
    need = std::max({need, rows_workspace<float>(pos0, n_heads, n_kv_heads, head_dim, cu_count),
                     rows_workspace<_Float16>(pos0, n_heads, n_kv_heads, head_dim, cu_count)});
  return need;
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
                q_rope_cs, q_rope_rows, q_rope_neox, Append<float>{}, reinterpret_cast<hipStream_t>(stream));
}

int nbhs_attn_decode_f16kv(const float* q, const void* k16, const void* v16, float* out, int64_t n, int64_t pos0,
                           int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, float* workspace,
                           int64_t workspace_floats, int cu_count, const float* q_rope_cs, int64_t q_rope_rows,
                           int q_rope_neox, nbhs_stream stream) {
  return decode(q, static_cast<const _Float16*>(k16), static_cast<const _Float16*>(v16), out, n, pos0, n_heads,
                n_kv_heads, head_dim, workspace, workspace_floats, cu_count, q_rope_cs, q_rope_rows, q_rope_neox,
                Append<_Float16>{}, reinterpret_cast<hipStream_t>(stream));
}

int nbhs_attn_decode_ordered_f32(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                                 int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, const float* q_rope_cs,
                                 int64_t q_rope_rows, int q_rope_neox, nbhs_stream stream) {
  return decode(q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim, nullptr, 0, 0, q_rope_cs, q_rope_rows,
                q_rope_neox, Append<float>{}, reinterpret_cast<hipStream_t>(stream), false, true);
}

int nbhs_attn_decode_ordered_f16kv(const float* q, const void* k16, const void* v16, float* out, int64_t n,
                                   int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                   const float* q_rope_cs, int64_t q_rope_rows, int q_rope_neox,
                                   nbhs_stream stream) {
  return decode(q, static_cast<const _Float16*>(k16), static_cast<const _Float16*>(v16), out, n, pos0, n_heads,
                n_kv_heads, head_dim, nullptr, 0, 0, q_rope_cs, q_rope_rows, q_rope_neox, Append<_Float16>{},
                reinterpret_cast<hipStream_t>(stream), false, true);
}

int nbhs_append_attn_decode_f32(const float* q, float* k_cache, float* v_cache, const float* k_new,
                                const float* v_new, float* out, int64_t pos0, int64_t n_heads, int64_t n_kv_heads,
                                int64_t head_dim, float* workspace, int64_t workspace_floats, int cu_count,
                                const float* rope_cs, int64_t rope_rows, int neox, nbhs_stream stream) {
  // One query row, tiled head sizes, RoPE table required (it rotates q and the new K row alike).
  if (!k_new || !v_new || !rope_cs || !tiled_head_dim(head_dim)) return NBHS_EINVAL;
  Append<float> app;
  app.k_new = k_new;
  app.v_new = v_new;
  app.k_dst = k_cache;
  app.v_dst = v_cache;
  return decode(q, k_cache, v_cache, out, 1, pos0, n_heads, n_kv_heads, head_dim, workspace, workspace_floats,
                cu_count, rope_cs, rope_rows, neox, app, reinterpret_cast<hipStream_t>(stream));
}

int nbhs_append_attn_decode_f16kv(const float* q, void* k16, void* v16, const float* k_new, const float* v_new,
                                  float* out, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                  float* workspace, int64_t workspace_floats, int cu_count, const float* rope_cs,
                                  int64_t rope_rows, int neox, nbhs_stream stream) {
  if (!k_new || !v_new || !rope_cs || !tiled_head_dim(head_dim)) return NBHS_EINVAL;
  Append<_Float16> app;
  app.k_new = k_new;
  app.v_new = v_new;
  app.k_dst = static_cast<_Float16*>(k16);
  app.v_dst = static_cast<_Float16*>(v16);
  return decode(q, static_cast<const _Float16*>(k16), static_cast<const _Float16*>(v16), out, 1, pos0, n_heads,
                n_kv_heads, head_dim, workspace, workspace_floats, cu_count, rope_cs, rope_rows, neox, app,
                reinterpret_cast<hipStream_t>(stream));
}

int nbhs_append_rope_f16kv(void* k16, void* v16, const float* k_new, const float* v_new, int64_t n, int64_t pos0,
                           int64_t n_kv_heads, int64_t head_dim, const float* cs_table, int64_t table_rows, int neox,
                           nbhs_stream stream) {
  if (!k16 || !v16 || !k_new || !v_new || !cs_table || n <= 0 || pos0 < 0 || n_kv_heads <= 0 || head_dim <= 0 ||
      head_dim % 2 != 0 || pos0 + n > table_rows)
    return NBHS_EINVAL;
  const int64_t pairs = n * n_kv_heads * (head_dim / 2);
  const int64_t blocks = (pairs + 255) / 256;
  return nbhs_timing::launch(NBHS_K_ROPE, append_rope_f16_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)),
                             dim3(256), reinterpret_cast<hipStream_t>(stream), static_cast<_Float16*>(k16),
                             static_cast<_Float16*>(v16), k_new, v_new, n, pos0, n_kv_heads, head_dim,
                             reinterpret_cast<const float2*>(cs_table), neox);
}

}  // extern "C"
