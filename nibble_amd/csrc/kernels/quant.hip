// Quantized weight matmuls and dequantization on gfx950: Backend::matmul / matmul_multi / embed for the ggml block
// formats Q4_0, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K (src/quant.h), bit-exact with the reference's scalar kernels
// src/quant.cpp (itself llama.cpp's generic code) and hence with its AVX2 tier.
//
// A matmul never dequantizes the weights (ref_ops.cpp:109-135): each activation row is quantized to the weight
// type's companion format (Q8_0, Q8_1 or Q8_K), and y[t, r] = sum over blocks b of a per-block term, summed in block
// order. The integer part of every term is exact, so it is computed in any order (here with v_dot4 where it
// applies); the float part - the scale products and the running sum over blocks - is the reference's expression,
// in its order, with no multiply-add contraction (this file is compiled with -ffp-contract=off, as the reference's
// quant.cpp is; the __f*_rn spellings only mark the rounding points):
//   Q4_0  sum += (float(isum) * d_w) * d_a          quant.cpp:309-325
//   Q8_0  sum += float(isum) * (d_w * d_a)          :329-342
//   Q5_0  sum += (d_w * d_a) * float(isum)          :346-365
//   Q5_1  sum += (d_w * d_a) * float(isum) + m_w * s_a  :369-390
//   Q4_K / Q5_K (quant.cpp:118-144) and Q6_K (:394-416): eight int32 lanes (element e feeds lane e % 8) per
//   super-block, sums[l] += (d_w * d_a) * float(aux[l]) in super-block order, Q4_K / Q5_K also sumf -= (dmin_w *
//   d_a) * float(sumi) per super-block, and the eight sums added to sumf last.
//
// qgemv_kernel (n <= 16 activation rows): a 64-lane wave takes RW weight rows; its lanes take (row, block) pairs -
// a legacy block or a whole K super-block each - and write each pair's float term(s) to LDS; then one lane per
// (row, activation row) adds its terms in block order. K quants are stored in residue order (quant_layout.h), so a
// sub-block's eight integer lanes are eight v_dot4. With up to 4 activation rows the rows are quantized inside the
// launch (into LDS, once per wave and block), with the same bits as the standalone quantizer.
#include <hip/hip_runtime.h>


#include "backend/hip/kernel_timing.h"
#include "kernels/quant_layout.h"
#include "nibble_hip_shim.h"

namespace {

using namespace nbh_quant;

struct QW {
  const uint8_t* q;
  const uint8_t* h;
  const uint8_t* s;
  const uint16_t* d;
  const uint16_t* m;
  int64_t rows, nb;
};
struct QA {
  const int8_t* qs;
  const float* d;
  const float* s;
  const int16_t* bsums;
  int64_t nb;
};

__device__ __forceinline__ float h2f(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, _Float16(f)); }  // RNE

// v as a float in a register, opaque to the optimizer. fp16(a * b) is otherwise compiled to one v_fma_mix, which
// rounds the exact product to fp16 once; the reference rounds to float first and then to fp16, and the two differ
// when the float product lands on an fp16 tie.
__device__ __forceinline__ float opaque(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4(int(a), int(b), c, false);
}

// ---- activation quantizers (quant.cpp:37-49, 245-303) ----

// One thread per 32-element block of row t: Q8_0 (and Q8_1's sum term when Q81).
template <bool Q81>
__global__ __launch_bounds__(256) void quantize_q8_kernel(const float* __restrict__ x, int64_t in, int64_t n,
                                                          int8_t* __restrict__ qs, float* __restrict__ dq,
                                                          float* __restrict__ sq) {
  const int64_t nb = in / 32;
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n * nb) return;
  const float* xb = x + (i / nb) * in + (i % nb) * 32;
  float v[32];
  float amax = 0.f;
  bool nan = false;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    v[j] = xb[j];
    amax = fmaxf(amax, fabsf(v[j]));
    nan |= v[j] != v[j];
  }
  const float d = nan ? __builtin_nanf("") : __fdiv_rn(amax, 127.f);
  const float id = d != 0.f ? __fdiv_rn(1.0f, d) : 0.0f;
  int sum = 0;
  uint32_t packed[8];
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float r = roundf(__fmul_rn(v[4 * w + e], id));
      const int q = r != r ? 0 : int(fminf(127.f, fmaxf(-127.f, r)));
      sum += q;
      word |= uint32_t(q & 0xFF) << (8 * e);
    }
    packed[w] = word;
  }
  uint4* o = reinterpret_cast<uint4*>(qs + i * 32);
  o[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  o[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
  dq[i] = h2f(f2h(d));
  if constexpr (Q81) sq[i] = h2f(f2h(opaque(__fmul_rn(float(sum), d))));
}

// ggml nearest_int (quant.cpp:146-152): round half to even through the float mantissa.
__device__ __forceinline__ int nearest_int(float f) {
  const float val = __fadd_rn(f, 12582912.f);
  return (__float_as_int(val) & 0x007fffff) - 0x00400000;
}

// One wave per 256-element super-block; lane l = 8k + w holds elements 32k + w + 8i (i < 4) of sub-block k: the four
// elements of residue word w, which it stores as word w of the sub-block (residue order, quant_layout.h).
// RM: the super-block's quants in residue-major order instead (byte 32 w + 4 k + i = element 32 k + w + 8 i), so
// that residue w's 32 quants - the ones that feed the reference's integer lane w - are contiguous (the order
// qgemm_k_kernel reads).
template <bool RM>
__global__ __launch_bounds__(64) void quantize_q8k_kernel(const float* __restrict__ x, int64_t in,
                                                          int8_t* __restrict__ qs, float* __restrict__ dq,
                                                          int16_t* __restrict__ bsums) {
  const int64_t nb = in / 256, i = blockIdx.x;
  const int lane = threadIdx.x, k = lane >> 3, w = lane & 7;
  const float* xb = x + (i / nb) * in + (i % nb) * 256 + 32 * k + w;
  const float v[4] = {xb[0], xb[8], xb[16], xb[24]};
  // the first element of largest magnitude (strictly greater replaces; NaN never does)
  float amax = 0.f, mx = 0.f;
  int idx = 1 << 30;
  bool nan = false;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float ax = fabsf(v[e]);
    if (ax > amax) amax = ax, mx = v[e], idx = 32 * k + w + 8 * e;
    nan |= v[e] != v[e];
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const float oa = __shfl_xor(amax, m, 64), om = __shfl_xor(mx, m, 64);
    const int oi = __shfl_xor(idx, m, 64);
    if (oa > amax || (oa == amax && oi < idx)) amax = oa, mx = om, idx = oi;
  }
  nan = __builtin_amdgcn_ballot_w64(nan) != 0;
  uint32_t word = 0;
  int b0 = 0, b1 = 0;  // this lane's share of the sub-block's two 16-sums (elements w, w + 8 | w + 16, w + 24)
  float d = 0.f;
  if (amax != 0.f) {
    const float iscale = __fdiv_rn(-127.f, mx);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float sv = __fmul_rn(iscale, v[e]);
      const int q = sv != sv ? 0 : nearest_int(fminf(127.f, fmaxf(-127.f, sv)));
      if (e < 2) b0 += q; else b1 += q;
      word |= uint32_t(q & 0xFF) << (8 * e);
    }
    d = __fdiv_rn(1.f, iscale);
  }
#pragma unroll
  for (int m = 1; m < 8; m <<= 1) b0 += __shfl_xor(b0, m, 64), b1 += __shfl_xor(b1, m, 64);
  reinterpret_cast<uint32_t*>(qs + i * 256)[RM ? 8 * w + k : lane] = word;
  if (w == 0) bsums[i * 16 + 2 * k] = int16_t(b0), bsums[i * 16 + 2 * k + 1] = int16_t(b1);
  if (lane == 0) dq[i] = nan ? __builtin_nanf("") : d;
}

// ---- activation blocks ----

// One legacy activation block: 32 quants as 8 words, the scale d (fp16-rounded, widened), Q8_1's s, and the sum
// of the quants (for the Q4_0 / Q5_0 offsets).
struct ActL {
  uint32_t a[8];
  float d, s;
  int sum;
};

__device__ __forceinline__ ActL load_act_l(const QA& A, int64_t t, int64_t b) {
  ActL r;
  const int64_t ab = t * A.nb + b;
  const uint4* ap = reinterpret_cast<const uint4*>(A.qs + ab * 32);
  const uint4 a0 = ap[0], a1 = ap[1];
  r.a[0] = a0.x, r.a[1] = a0.y, r.a[2] = a0.z, r.a[3] = a0.w, r.a[4] = a1.x, r.a[5] = a1.y, r.a[6] = a1.z,
  r.a[7] = a1.w;
  r.d = A.d[ab];
  r.s = A.s ? A.s[ab] : 0.f;
  r.sum = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) r.sum = sdot4(r.a[i], 0x01010101u, r.sum);
  return r;
}

// quantize_block_q8 (quant.cpp:37-49) of the 32 floats at xb (16-byte aligned), in registers: the same bits
// quantize_q8_kernel writes.
template <bool Q81>
__device__ __forceinline__ ActL quant_act_l(const float* xb) {
  float v[32];
  float amax = 0.f;
  bool nan = false;
#pragma unroll
  for (int j = 0; j < 32; j += 4) {
    const float4 f = *reinterpret_cast<const float4*>(xb + j);
    v[j] = f.x, v[j + 1] = f.y, v[j + 2] = f.z, v[j + 3] = f.w;
  }
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    amax = fmaxf(amax, fabsf(v[j]));
    nan |= v[j] != v[j];
  }
  const float d = nan ? __builtin_nanf("") : __fdiv_rn(amax, 127.f);
  const float id = d != 0.f ? __fdiv_rn(1.0f, d) : 0.0f;
  ActL r;
  r.sum = 0;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float q = roundf(__fmul_rn(v[4 * w + e], id));
      const int qi = q != q ? 0 : int(fminf(127.f, fmaxf(-127.f, q)));
      r.sum += qi;
      word |= uint32_t(qi & 0xFF) << (8 * e);
    }
    r.a[w] = word;
  }
  r.d = h2f(f2h(d));
  r.s = Q81 ? h2f(f2h(opaque(__fmul_rn(float(r.sum), d)))) : 0.f;
  return r;
}

// quantize_row_q8_K (quant.cpp:273-303) of one super-block spread over the 8 lanes of this lane's group (lane k
// holds elements 32k..32k+31 at xs, 16-byte aligned): the first element of largest magnitude sets the scale.
// Returns sub-block k's words in residue order and its two 16-sums; every lane of the wave must call it.
__device__ __forceinline__ void quant_act_k(const float* xs, int k, uint32_t (&aw)[8], int& bs0, int& bs1, float& d) {
  float v[32];
#pragma unroll
  for (int j = 0; j < 32; j += 4) {
    const float4 f = *reinterpret_cast<const float4*>(xs + j);
    v[j] = f.x, v[j + 1] = f.y, v[j + 2] = f.z, v[j + 3] = f.w;
  }
  float amax = 0.f, mx = 0.f;
  int idx = 1 << 30, nanf = 0;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const float ax = fabsf(v[e]);
    if (ax > amax) amax = ax, mx = v[e], idx = 32 * k + e;
    nanf |= v[e] != v[e];
  }
#pragma unroll
  for (int m = 1; m < 8; m <<= 1) {
    const float oa = __shfl_xor(amax, m, 64), om = __shfl_xor(mx, m, 64);
    const int oi = __shfl_xor(idx, m, 64);
    if (oa > amax || (oa == amax && oi < idx)) amax = oa, mx = om, idx = oi;
    nanf |= __shfl_xor(nanf, m, 64);
  }
  int q[32];
  d = 0.f;
  bs0 = bs1 = 0;
  if (amax != 0.f) {
    const float iscale = __fdiv_rn(-127.f, mx);
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const float sv = __fmul_rn(iscale, v[e]);
      q[e] = sv != sv ? 0 : nearest_int(fminf(127.f, fmaxf(-127.f, sv)));
      if (e < 16) bs0 += q[e]; else bs1 += q[e];
    }
    d = __fdiv_rn(1.f, iscale);
  } else {
#pragma unroll
    for (int e = 0; e < 32; ++e) q[e] = 0;
  }
#pragma unroll
  for (int w = 0; w < 8; ++w)
    aw[w] = uint32_t(q[w] & 0xFF) | uint32_t(q[w + 8] & 0xFF) << 8 | uint32_t(q[w + 16] & 0xFF) << 16 |
            uint32_t(q[w + 24] & 0xFF) << 24;
  if (nanf) d = __builtin_nanf("");
}

// ---- block terms ----

// Legacy block b of weight row rr against one activation block: the block's float term (header comment).
template <int T>
__device__ __forceinline__ float legacy_term(const QW& W, int64_t rr, int64_t b, const ActL& A) {
  const int64_t wb = rr * W.nb + b;
  const float dw = h2f(W.d[wb]), da = A.d;
  if constexpr (T == kQ8_0) {
    const uint4* wp = reinterpret_cast<const uint4*>(W.q + wb * 32);
    const uint4 w0 = wp[0], w1 = wp[1];
    int s = sdot4(w0.x, A.a[0], 0);
    s = sdot4(w0.y, A.a[1], s), s = sdot4(w0.z, A.a[2], s), s = sdot4(w0.w, A.a[3], s);
    s = sdot4(w1.x, A.a[4], s), s = sdot4(w1.y, A.a[5], s), s = sdot4(w1.z, A.a[6], s), s = sdot4(w1.w, A.a[7], s);
    return __fmul_rn(float(s), __fmul_rn(dw, da));
  } else {
    const uint4 wv = *reinterpret_cast<const uint4*>(W.q + wb * 16);
    const uint32_t w[4] = {wv.x, wv.y, wv.z, wv.w};
    // element j of the block: low nibble of byte j (j < 16), high nibble of byte j - 16 (j >= 16)
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) lo[i] = w[i] & 0x0F0F0F0Fu, hi[i] = (w[i] >> 4) & 0x0F0F0F0Fu;
    if constexpr (T == kQ5_0 || T == kQ5_1) {
      const uint32_t qh = *reinterpret_cast<const uint32_t*>(W.h + wb * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 4 * i + e;
          lo[i] |= ((qh >> j) & 1u) << (8 * e + 4);
          hi[i] |= ((qh >> (j + 16)) & 1u) << (8 * e + 4);
        }
    }
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) s = sdot4(lo[i], A.a[i], s), s = sdot4(hi[i], A.a[i + 4], s);
    if constexpr (T == kQ4_0) return __fmul_rn(__fmul_rn(float(s - 8 * A.sum), dw), da);
    if constexpr (T == kQ5_0) return __fmul_rn(__fmul_rn(dw, da), float(s - 16 * A.sum));
    if constexpr (T == kQ5_1) return __fadd_rn(__fmul_rn(__fmul_rn(dw, da), float(s)), __fmul_rn(h2f(W.m[wb]), A.s));
  }
  return 0.f;
}

// A legacy weight block in registers (loaded ahead of the activation work that hides its latency).
struct WBlk {
  uint4 q0, q1;  // quants (q1: Q8_0's second half)
  uint32_t h;    // Q5_0 / Q5_1 high bits
  uint16_t d, m;
};

template <int T>
__device__ __forceinline__ WBlk load_wblk(const QW& W, int64_t rr, int64_t b) {
  const int64_t wb = rr * W.nb + b;
  WBlk k;
  if constexpr (T == kQ8_0) {
    const uint4* wp = reinterpret_cast<const uint4*>(W.q + wb * 32);
    k.q0 = wp[0], k.q1 = wp[1];
  } else {
    k.q0 = *reinterpret_cast<const uint4*>(W.q + wb * 16);
  }
  if constexpr (T == kQ5_0 || T == kQ5_1) k.h = reinterpret_cast<const uint32_t*>(W.h)[wb];
  k.d = W.d[wb];
  if constexpr (T == kQ5_1) k.m = W.m[wb];
  return k;
}

// legacy_term on a preloaded weight block.
template <int T>
__device__ __forceinline__ float wblk_term(const WBlk& k, const ActL& A) {
  const float dw = h2f(k.d), da = A.d;
  if constexpr (T == kQ8_0) {
    int s = sdot4(k.q0.x, A.a[0], 0);
    s = sdot4(k.q0.y, A.a[1], s), s = sdot4(k.q0.z, A.a[2], s), s = sdot4(k.q0.w, A.a[3], s);
    s = sdot4(k.q1.x, A.a[4], s), s = sdot4(k.q1.y, A.a[5], s), s = sdot4(k.q1.z, A.a[6], s), s = sdot4(k.q1.w, A.a[7], s);
    return __fmul_rn(float(s), __fmul_rn(dw, da));
  } else {
    const uint32_t w[4] = {k.q0.x, k.q0.y, k.q0.z, k.q0.w};
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) lo[i] = w[i] & 0x0F0F0F0Fu, hi[i] = (w[i] >> 4) & 0x0F0F0F0Fu;
    if constexpr (T == kQ5_0 || T == kQ5_1) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 4 * i + e;
          lo[i] |= ((k.h >> j) & 1u) << (8 * e + 4);
          hi[i] |= ((k.h >> (j + 16)) & 1u) << (8 * e + 4);
        }
    }
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) s = sdot4(lo[i], A.a[i], s), s = sdot4(hi[i], A.a[i + 4], s);
    if constexpr (T == kQ4_0) return __fmul_rn(__fmul_rn(float(s - 8 * A.sum), dw), da);
    if constexpr (T == kQ5_0) return __fmul_rn(__fmul_rn(dw, da), float(s - 16 * A.sum));
    if constexpr (T == kQ5_1) return __fadd_rn(__fmul_rn(__fmul_rn(dw, da), float(s)), __fmul_rn(h2f(k.m), A.s));
  }
  return 0.f;
}

// ggml get_scale_min_k4 (quant.cpp:52-61)
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t* q, int& d, int& m) {
  if (j < 4) {
    d = q[j] & 63;
    m = q[j + 4] & 63;
  } else {
    d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

__device__ __forceinline__ void load32(const uint8_t* p, uint32_t (&w)[8]) {
  const uint4 a = reinterpret_cast<const uint4*>(p)[0], b = reinterpret_cast<const uint4*>(p)[1];
  w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = b.x, w[5] = b.y, w[6] = b.z, w[7] = b.w;
}

// The integer lanes of super-block sb of row rr against an activation super-block whose sub-block k words are
// act(k, w) (residue order) and 16-sums bsum(g): aux[w] = sum over the block's elements e with e % 8 == w of
// scale(e) * (a_e * q_e) (quant.cpp:118-144, 394-416), and for Q4_K / Q5_K sumi = sum_k (bsums) * m_k.
// SPL > 1: this lane takes part `part` of SPL equal shares of the sub-blocks (the same code for every part, only
// the data offsets differ, so lanes of different parts do not diverge); the integer results of the parts add up
// to the whole block's (exactly: integer sums).
template <int T, int SPL = 1, class ActW, class BSum>
__device__ __forceinline__ void k_lanes(const QW& W, int64_t rr, int64_t sb, ActW act, BSum bsum, int (&aux)[8],
                                        int& sumi, int part = 0) {
  const int64_t wb = rr * W.nb + sb;
#pragma unroll
  for (int w = 0; w < 8; ++w) aux[w] = 0;
  sumi = 0;
  const uint8_t* sc = W.s + wb * 16;
  if constexpr (T == kQ4_K || T == kQ5_K) {
    uint32_t hw[8];
    if constexpr (T == kQ5_K) load32(W.h + wb * 32, hw);
#pragma unroll
    for (int cc = 0; cc < 4 / SPL; ++cc) {
      const int c = cc + (4 / SPL) * part;
      uint32_t qw[8];
      load32(W.q + wb * 128 + 32 * c, qw);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int k = 2 * c + half;
        int s, m;
        scale_min_k4(k, sc, s, m);
        sumi += (bsum(2 * k) + bsum(2 * k + 1)) * m;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          uint32_t v = (qw[w] >> (4 * half)) & 0x0F0F0F0Fu;
          if constexpr (T == kQ5_K) v |= ((hw[w] >> k) & 0x01010101u) << 4;
          aux[w] += s * sdot4(v, act(k, w), 0);
        }
      }
    }
  } else {  // Q6_K: sub-block k = 4h + g of the 128-element half h; values 0..63 less 32 (quant.cpp:84-96)
    const int8_t* scl = reinterpret_cast<const int8_t*>(sc);
#pragma unroll
    for (int hh = 0; hh < 2 / SPL; ++hh) {
      const int h = hh + (2 / SPL) * part;
      uint32_t hw[8];
      load32(W.h + wb * 64 + 32 * h, hw);
#pragma unroll
      for (int lg = 0; lg < 2; ++lg) {  // ql group: bytes 64h + 32lg .. +31 (sub-blocks g = lg and lg + 2)
        uint32_t lw[8];
        load32(W.q + wb * 128 + 64 * h + 32 * lg, lw);
#pragma unroll
        for (int sel = 0; sel < 2; ++sel) {
          const int g = lg + 2 * sel, k = 4 * h + g;
          const int s_lo = scl[2 * k], s_hi = scl[2 * k + 1];
#pragma unroll
          for (int w = 0; w < 8; ++w) {
            const uint32_t v = ((lw[w] >> (4 * sel)) & 0x0F0F0F0Fu) | (((hw[w] >> (2 * g)) & 0x03030303u) << 4);
            const uint32_t a = act(k, w);
            // bytes 0, 1 of a residue word are elements w, w + 8 (the first 16: scale s_lo); bytes 2, 3 the rest
            const int dlo = sdot4(v & 0x0000FFFFu, a, 0) - 32 * sdot4(0x00000101u, a, 0);
            const int dhi = sdot4(v & 0xFFFF0000u, a, 0) - 32 * sdot4(0x01010000u, a, 0);
            aux[w] += s_lo * dlo + s_hi * dhi;
          }
        }
      }
    }
  }
}

// ---- the matmul ----

constexpr int kMaxQWeights = NBHS_GEMV_MAX_WEIGHTS;
struct QBatch {  // weights of one type sharing one input; wave0: first wave of each weight's rows
  QW w[kMaxQWeights];
  float* y[kMaxQWeights];
  int64_t wave0[kMaxQWeights];
  int n_w;
};

// Weight rows per wave: a legacy row has a block per lane (in = 2048: 64 blocks), a K row a super-block per lane
// (in = 2048: 8), so K waves take twice the rows; with 16 activation rows a wave's outputs are capped at 64. A
// single-row launch over many rows (an FFN's 16384) takes 16 rows per wave: the activation row each wave quantizes
// is then shared by more weight rows, and there are still a thousand or more waves.
constexpr int rows_per_wave(bool k, int NT, bool wide) {
  return NT > 4 ? 4 : k ? (NT == 1 && !wide ? 4 : 8) : wide && NT == 1 ? 16 : 4;
}
// K types with one activation row in a launch of QKV size: each (row, super-block) pair is split over two adjacent
// lanes (half the sub-blocks each), which halves the serial integer chain per lane and doubles the waves. Wide
// launches (an FFN's 16384 rows) have waves enough and lose more to the activation quantization each wave repeats.
constexpr int k_split(bool k, int NT, bool wide) { return k && NT == 1 && !wide ? 2 : 1; }
constexpr int64_t kWideRows = 16384;  // total rows of a launch from which single-row launches go wide

// A K activation super-block staged in LDS on the fused path: 256 quants in residue order, d, the 16-sums.
struct LdsActK {
  uint32_t a[64];
  float d;
  int bs[16];
};

// FUSED: the activation rows are quantized here, from x (NT <= 4), instead of read from A.
template <int T, int NT, bool FUSED, bool WIDE>
__global__ __launch_bounds__(64) void qgemv_kernel(QBatch B, QA A, const float* __restrict__ x, int64_t in, int n) {
  constexpr bool K = T == kQ4_K || T == kQ5_K || T == kQ6_K;
  constexpr int RW = rows_per_wave(K, NT, WIDE);
  constexpr int O = RW * NT;  // outputs of this wave
  constexpr int CH = K ? 8 : 64;  // blocks per chunk
  constexpr int TERMS = K ? 9 : 1;
  static_assert(O <= 64, "one lane per output in the ordered sum");
  static_assert(!FUSED || NT <= 4, "fused activation quantization stages at most 4 rows");
  __shared__ float terms[O][CH][TERMS];
  __shared__ LdsActK acts[K && FUSED ? NT : 1][K ? CH : 1];
  const int lane = threadIdx.x;
  int wi = 0;
  for (int j = 1; j < B.n_w; ++j)
    if (int64_t(blockIdx.x) >= B.wave0[j]) wi = j;
  const QW& W = B.w[wi];
  float* __restrict__ y = B.y[wi];
  const int64_t r0 = (int64_t(blockIdx.x) - B.wave0[wi]) * RW;
  const int nr = int(W.rows - r0 < RW ? W.rows - r0 : RW);
  float acc = 0.f, sums[8];
#pragma unroll
  for (int l = 0; l < 8; ++l) sums[l] = 0.f;
  for (int64_t c0 = 0; c0 < W.nb; c0 += CH) {
    const int nc = int(W.nb - c0 < CH ? W.nb - c0 : CH);
    if constexpr (FUSED && K) {  // quantize this chunk's activation super-blocks once, into LDS
      const int sbl = lane >> 3, k = lane & 7;
      const int64_t sb = c0 + (sbl < nc ? sbl : 0);
      for (int t = 0; t < NT; ++t) {
        if (t >= n) break;
        uint32_t aw[8];
        int bs0, bs1;
        float d;
        quant_act_k(x + int64_t(t) * in + sb * 256 + 32 * k, k, aw, bs0, bs1, d);
        if (sbl < nc) {
          LdsActK& o = acts[t][sbl];
#pragma unroll
          for (int w = 0; w < 8; ++w) o.a[8 * k + w] = aw[w];
          o.bs[2 * k] = bs0, o.bs[2 * k + 1] = bs1;
          if (k == 0) o.d = d;
        }
      }
      __syncthreads();
    }
    // phase 1: the term(s) of every (row, block) pair, for each activation row
    if constexpr (!K) {  // a block per lane; its activation block (quantized here when fused) serves every row
      if (lane < nc) {
        const int64_t b = c0 + lane;
        // every row's weight block is requested before the activation work, which hides the loads' latency
        WBlk wk[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) wk[r] = load_wblk<T>(W, r0 + (r < nr ? r : nr - 1), b);
        for (int t = 0; t < NT; ++t) {
          if (t >= n) break;
          ActL a;
          if constexpr (FUSED)
            a = quant_act_l<T == kQ5_1>(x + int64_t(t) * in + b * 32);
          else
            a = load_act_l(A, t, b);
#pragma unroll
          for (int r = 0; r < RW; ++r) terms[r * NT + t][lane][0] = wblk_term<T>(wk[r], a);
        }
      }
    } else {
      constexpr int SPL = k_split(K, NT, WIDE);
      // RW * nc * SPL <= 64 (nc <= 8), so the two lanes of a split pair are always in the same pass
      for (int p = lane; p < RW * nc * SPL; p += 64) {
        const int pair = p / SPL, part = p % SPL;
        const int r = pair / nc, bl = pair % nc;
        const int64_t rr = r0 + (r < nr ? r : nr - 1), b = c0 + bl;
        for (int t = 0; t < NT; ++t) {
          if (t >= n) break;
          int aux[8], sumi;
          float da;
          if constexpr (FUSED) {
            const LdsActK& s = acts[t][bl];
            k_lanes<T, SPL>(W, rr, b, [&](int k, int w) { return s.a[8 * k + w]; }, [&](int g) { return s.bs[g]; },
                            aux, sumi, part);
            da = s.d;
          } else {
            const int64_t ab = int64_t(t) * A.nb + b;
            const uint32_t* aq = reinterpret_cast<const uint32_t*>(A.qs + ab * 256);
            const int16_t* bs = A.bsums + ab * 16;
            k_lanes<T, SPL>(W, rr, b, [&](int k, int w) { return aq[8 * k + w]; }, [&](int g) { return int(bs[g]); },
                            aux, sumi, part);
            da = A.d[ab];
          }
          if constexpr (SPL == 2) {  // the partner lane (p ^ 1) holds the other half
#pragma unroll
            for (int l = 0; l < 8; ++l) aux[l] += __shfl_xor(aux[l], 1, 64);
            sumi += __shfl_xor(sumi, 1, 64);
            if (part != 0) continue;
          }
          const int64_t wb = rr * W.nb + b;
          const float d = __fmul_rn(h2f(W.d[wb]), da);
#pragma unroll
          for (int l = 0; l < 8; ++l) terms[r * NT + t][bl][l] = __fmul_rn(d, float(aux[l]));
          terms[r * NT + t][bl][8] = T == kQ6_K ? 0.f : __fmul_rn(__fmul_rn(h2f(W.m[wb]), da), float(sumi));
        }
      }
    }
    __syncthreads();
    // phase 2: each output adds its terms in block order
    if (lane < O) {
      if constexpr (!K) {
        for (int b = 0; b < nc; ++b) acc = __fadd_rn(acc, terms[lane][b][0]);
      } else {
        for (int b = 0; b < nc; ++b) {
#pragma unroll
          for (int l = 0; l < 8; ++l) sums[l] = __fadd_rn(sums[l], terms[lane][b][l]);
          if constexpr (T != kQ6_K) acc = __fsub_rn(acc, terms[lane][b][8]);
        }
      }
    }
    __syncthreads();
  }
  if (lane < O) {
    if constexpr (K) {
#pragma unroll
      for (int l = 0; l < 8; ++l) acc = __fadd_rn(acc, sums[l]);
    }
    const int r = lane / NT, t = lane % NT;
    if (r < nr && t < n) y[int64_t(t) * W.rows + r0 + r] = acc;
  }
}

// ---- the tiled matmul for longer calls (prefill chunks) ----
//
// qgemm_legacy_kernel: a 256-thread workgroup computes 64 weight rows x 16 TJ activation rows on the int8 matrix
// cores. A legacy block is 32 elements, exactly the contraction of one v_mfma_i32_16x16x32_i8, so each (16 weight
// rows, 16 activation rows, block) is one MFMA from zero: the block's exact integer dots (Q4_0 / Q5_0 as
// sum q_w q_a, the offset term -8 or -16 times the activation block's quant sum applied after, exactly). Every output
// then adds its block's float term - the reference's expression, in block order - so the outputs are bit-exact with
// the v_dot4 path and with quant.cpp. Waves: 2 x 2 over 64 x 64 (TJ = 4), 4 x 1 over 64 x 32 (TJ = 2) or, with
// WRT = 32 weight rows, 2 x 2 over 32 x 32; each lane holds the MFMA result layout's 4 weight rows of one
// activation row per 16 x 16 pair. Chunks of 8 blocks of
// both operands are staged in LDS (one 16-byte pad per row: conflict-free fragment reads); the next chunk's share of
// each thread is loaded into registers while the current one is computed, the weight scales are widened to float
// and an activation block's quant sum taken once at staging. One launch covers the weights of one type that share
// the input (a layer's Q, K and V): grid x runs over the row tiles of all of them, so small weights do not leave
// most CUs idle; TJ = 2 doubles the workgroups of a launch that would otherwise leave most SIMDs with one wave.
constexpr int kGemmCB = 8;  // blocks per staged chunk

struct QGemmBatch {  // weights of one type sharing one input; tile0[i]: first row tile of weight i
  QW w[kMaxQWeights];
  float* y[kMaxQWeights];
  int tile0[kMaxQWeights];
  int n_w;
};

// Staged quant words as a native vector type (a uint4 copy is a memcpy that keeps the staging share in scratch).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));  // an integer MFMA result

template <int T, int TJ, int WRT = 64>
__global__ __launch_bounds__(256) void qgemm_legacy_kernel(QGemmBatch B, QA A, int64_t n) {
  int wi = 0;
  for (int i = 1; i < B.n_w; ++i)
    if (int(blockIdx.x) >= B.tile0[i]) wi = i;
  const QW W = B.w[wi];
  float* __restrict__ y = B.y[wi];
  constexpr int QB = T == kQ8_0 ? 32 : 16;           // quant bytes per block
  constexpr int QW4 = QB / 16;                        // u32x4_t per block
  constexpr int WROW = kGemmCB * QW4 + 1;             // u32x4_t per staged weight row (one of padding: spreads banks)
  constexpr int AROW = 2 * kGemmCB + 1;               // u32x4_t per staged activation row (likewise)
  constexpr int AR = 16 * TJ;                         // activation rows per workgroup
  constexpr int NWQ = WRT * kGemmCB * QW4 / 256;       // weight u32x4_t a thread stages per chunk
  constexpr int NWM = WRT * kGemmCB / 256;             // weight block headers a thread stages per chunk
  constexpr int NA = (AR * kGemmCB + 255) / 256;      // activation blocks a thread stages per chunk (at most)
  static_assert(NWQ * 256 == WRT * kGemmCB * QW4 && NWM * 256 == WRT * kGemmCB, "chunks split evenly");
  // Per wave: WM 16-row weight groups x 2 16-row activation groups, one v_mfma_i32_16x16x32_i8 per pair and block
  // (a legacy block is exactly the MFMA's 32-deep contraction). TJ = 4: waves 2 x 2 over 64 x 64; TJ = 2: waves
  // 4 x 1 over 64 x 32.
  constexpr int WM = TJ == 4 && WRT == 64 ? 2 : 1;
  constexpr int WN = WRT == 64 ? 2 : 1;  // 16-row activation groups per wave (32 x 32 tiles: waves 2 x 2 of 16 x 16)
  __shared__ u32x4_t wq[WRT * WROW];
  __shared__ float wdf[kGemmCB][WRT], wmf[kGemmCB][WRT];
  __shared__ uint32_t wh[WRT][kGemmCB];
  __shared__ u32x4_t aq[AR * AROW];
  __shared__ float ad[kGemmCB][AR], as_[kGemmCB][AR];
  __shared__ int asum[kGemmCB][AR];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ml = lane & 15, kg = lane >> 4;  // operand row / column of the lane and its 8-deep k group
  const int wr0 = WRT == 32 ? 16 * (wave & 1) : TJ == 4 ? 32 * (wave & 1) : 16 * wave;
  const int ac0 = WRT == 32 ? 16 * (wave >> 1) : TJ == 4 ? 32 * (wave >> 1) : 0;
  const int64_t row0 = int64_t(int(blockIdx.x) - B.tile0[wi]) * WRT, t0 = int64_t(blockIdx.y) * AR;
  // acc[i][j][v]: weight row wr0 + 16 i + 4 kg + v, activation row ac0 + 16 j + ml (the MFMA's result layout)
  float acc[WM][WN][4];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0.f;
  // A thread's share of one chunk, in registers: rows and activation rows past the ends, and blocks past the
  // chunk's end, load clamped (staged but never used).
  struct Share {
    u32x4_t q[NWQ];
    uint32_t d[NWM], m[NWM], h[NWM];
    u32x4_t a0[NA], a1[NA];
    float ad[NA], as[NA];
  };
  auto load_share = [&](int64_t c0, Share& sh) __attribute__((always_inline)) {
    const int nc = int(W.nb - c0 < kGemmCB ? W.nb - c0 : kGemmCB);
#pragma unroll
    for (int u = 0; u < NWQ; ++u) {
      const int e = tid + 256 * u;
      const int r = e / (kGemmCB * QW4), rem = e % (kGemmCB * QW4), b = rem / QW4, part = rem % QW4;
      const int64_t rr = min(row0 + r, W.rows - 1), bb = c0 + min(b, nc - 1);
      sh.q[u] = reinterpret_cast<const u32x4_t*>(W.q + (rr * W.nb + bb) * QB)[part];
    }
#pragma unroll
    for (int u = 0; u < NWM; ++u) {
      const int e = tid + 256 * u;
      const int r = e / kGemmCB, b = e % kGemmCB;
      const int64_t wb = min(row0 + r, W.rows - 1) * W.nb + c0 + min(b, nc - 1);
      sh.d[u] = W.d[wb];
      if constexpr (T == kQ5_1) sh.m[u] = W.m[wb];
      if constexpr (T == kQ5_0 || T == kQ5_1) sh.h[u] = reinterpret_cast<const uint32_t*>(W.h)[wb];
    }
#pragma unroll
    for (int u = 0; u < NA; ++u) {
      const int e = tid + 256 * u;
      if (e < AR * kGemmCB) {
        const int r = e / kGemmCB, b = e % kGemmCB;
        const int64_t ab = min(t0 + r, n - 1) * A.nb + c0 + min(b, nc - 1);
        sh.ad[u] = A.d[ab];
        if constexpr (T == kQ5_1) sh.as[u] = A.s[ab];
        const u32x4_t* ap = reinterpret_cast<const u32x4_t*>(A.qs + ab * 32);
        sh.a0[u] = ap[0];
        sh.a1[u] = ap[1];
      }
    }
  };
  auto store_share = [&](const Share& sh) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < NWQ; ++u) {
      const int e = tid + 256 * u;
      const int r = e / (kGemmCB * QW4), rem = e % (kGemmCB * QW4);
      wq[r * WROW + rem] = sh.q[u];
    }
#pragma unroll
    for (int u = 0; u < NWM; ++u) {
      const int e = tid + 256 * u;
      const int r = e / kGemmCB, b = e % kGemmCB;
      wdf[b][r] = h2f(uint16_t(sh.d[u]));
      if constexpr (T == kQ5_1) wmf[b][r] = h2f(uint16_t(sh.m[u]));
      if constexpr (T == kQ5_0 || T == kQ5_1) wh[r][b] = sh.h[u];
    }
#pragma unroll
    for (int u = 0; u < NA; ++u) {
      const int e = tid + 256 * u;
      if (e < AR * kGemmCB) {
        const int r = e / kGemmCB, b = e % kGemmCB;
        ad[b][r] = sh.ad[u];
        if constexpr (T == kQ5_1) as_[b][r] = sh.as[u];
        aq[r * AROW + 2 * b] = sh.a0[u];
        aq[r * AROW + 2 * b + 1] = sh.a1[u];
        if constexpr (T == kQ4_0 || T == kQ5_0) {
          int sum = 0;
#pragma unroll
          for (int w = 0; w < 4; ++w) sum = sdot4(sh.a0[u][w], 0x01010101u, sum);
#pragma unroll
          for (int w = 0; w < 4; ++w) sum = sdot4(sh.a1[u][w], 0x01010101u, sum);
          asum[b][r] = sum;
        }
      }
    }
  };
  // The lane's A operand (weight row wr0 + 16 i + ml, block elements 8 kg .. 8 kg + 7) as int8 values: element e of
  // a 4/5-bit block is the low nibble of byte e (e < 16) or the high nibble of byte e - 16, plus bit e of qh as
  // bit 4 for the 5-bit types; Q8_0 bytes are the values.
  auto a_operand = [&](int r, int b) __attribute__((always_inline)) {
    const uint32_t* wr = reinterpret_cast<const uint32_t*>(&wq[r * WROW + QW4 * b]);
    uint32_t lo, hi;
    if constexpr (T == kQ8_0) {
      lo = wr[2 * kg], hi = wr[2 * kg + 1];
    } else {
      const int sh = 4 * (kg >> 1);
      lo = (wr[2 * (kg & 1)] >> sh) & 0x0F0F0F0Fu;
      hi = (wr[2 * (kg & 1) + 1] >> sh) & 0x0F0F0F0Fu;
      if constexpr (T == kQ5_0 || T == kQ5_1) {
        const uint32_t bits = (wh[r][b] >> (8 * kg)) & 0xFFu;  // qh bits of elements 8 kg .. 8 kg + 7
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo |= ((bits >> e) & 1u) << (8 * e + 4);
          hi |= ((bits >> (e + 4)) & 1u) << (8 * e + 4);
        }
      }
    }
    return long((uint64_t(hi) << 32) | uint64_t(lo));
  };
  Share cur;
  load_share(0, cur);
  for (int64_t c0 = 0; c0 < W.nb; c0 += kGemmCB) {
    const int nc = int(W.nb - c0 < kGemmCB ? W.nb - c0 : kGemmCB);
    store_share(cur);
    __syncthreads();
    // the next chunk's share, in flight while this one is computed (the last chunk loads itself again, unused)
    load_share(c0 + kGemmCB < W.nb ? c0 + kGemmCB : c0, cur);
    for (int b = 0; b < nc; ++b) {
      long bop[WN];
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const uint32_t* ar = reinterpret_cast<const uint32_t*>(&aq[(ac0 + 16 * j + ml) * AROW + 2 * b]);
        bop[j] = long((uint64_t(ar[2 * kg + 1]) << 32) | uint64_t(ar[2 * kg]));
      }
#pragma unroll
      for (int i = 0; i < WM; ++i) {
        const int rb = wr0 + 16 * i;
        const long aop = a_operand(rb + ml, b);
        const float4 dw4 = *reinterpret_cast<const float4*>(&wdf[b][rb + 4 * kg]);
        const float dw[4] = {dw4.x, dw4.y, dw4.z, dw4.w};
        float mw[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (T == kQ5_1) {
          const float4 m4 = *reinterpret_cast<const float4*>(&wmf[b][rb + 4 * kg]);
          mw[0] = m4.x, mw[1] = m4.y, mw[2] = m4.z, mw[3] = m4.w;
        }
#pragma unroll
        for (int j = 0; j < WN; ++j) {
          const i32x4_t c = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop[j], i32x4_t{0, 0, 0, 0}, 0, 0, 0);
          const int t = ac0 + 16 * j + ml;
          const float da = ad[b][t];
          const int sum = T == kQ4_0 || T == kQ5_0 ? asum[b][t] : 0;
          const float sa = T == kQ5_1 ? as_[b][t] : 0.f;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int s = c[v];
            float term;
            if constexpr (T == kQ8_0) term = __fmul_rn(float(s), __fmul_rn(dw[v], da));
            if constexpr (T == kQ4_0) term = __fmul_rn(__fmul_rn(float(s - 8 * sum), dw[v]), da);
            if constexpr (T == kQ5_0) term = __fmul_rn(__fmul_rn(dw[v], da), float(s - 16 * sum));
            if constexpr (T == kQ5_1) term = __fadd_rn(__fmul_rn(__fmul_rn(dw[v], da), float(s)), __fmul_rn(mw[v], sa));
            acc[i][j][v] = __fadd_rn(acc[i][j][v], term);
          }
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t r = row0 + wr0 + 16 * i + 4 * kg + v, t = t0 + ac0 + 16 * j + ml;
        if (r < W.rows && t < n) y[t * W.rows + r] = acc[i][j][v];
      }
}

// The legacy kernel's tile for a launch: 64 x 64 while 64 x 64 tiles give at least kLegacyMinWgs workgroups
// (two per CU); else 64 x 32 while those do; else 32 x 32 (more, smaller workgroups: at the QKV shape 16-80 rows
// run 10-20 % faster than with 64 x 32, and 512 rows 3-5 % slower).
constexpr int64_t kLegacyMinWgs = 512;
enum LegacyTile { kTile64x64, kTile64x32, kTile32x32 };
template <int T>
hipError_t launch_legacy(LegacyTile tile, unsigned tiles, int64_t n, hipStream_t s, const QGemmBatch& B,
                         const QA& A) {
  if (tile == kTile64x64)
    return nbhs_timing::launch(NBHS_K_QGEMM, qgemm_legacy_kernel<T, 4>, dim3(tiles, unsigned((n + 63) / 64)),
                               dim3(256), s, B, A, n);
  const dim3 grid{tiles, unsigned((n + 31) / 32)};
  if (tile == kTile64x32)
    return nbhs_timing::launch(NBHS_K_QGEMM, qgemm_legacy_kernel<T, 2>, grid, dim3(256), s, B, A, n);
  return nbhs_timing::launch(NBHS_K_QGEMM, qgemm_legacy_kernel<T, 2, 32>, grid, dim3(256), s, B, A, n);
}

// qgemm_k_kernel: the tiled matmul for the K types on the int8 matrix cores (v_mfma_i32_16x16x32_i8).
// The reference's integer lane w of a super-block is aux[w] = sum over the 32 elements e of residue w (four per
// sub-block) of s(e) * q(e) * a(e), with the sub-block scale s varying along it. s * q is split into slices small
// enough that each slice's per-element product fits int8, each slice is one exact integer MFMA over the residue
// (K = 32), and aux[w] = sum_i c_i C_i, exactly:
//   Q4_K: s = 8 s1 + s0 (s0, s1 < 8), q < 16                        -> s0 q, s1 q            (c = 1, 8)
//   Q5_K: s = 16 s2 + 4 s1 + s0 (each < 4), q < 32                   -> s0 q, s1 q, s2 q      (c = 1, 4, 16)
//   Q6_K: s signed 8-bit per 16 elements = 16 s1 + s0 (s0 < 16, -8 <= s1 < 8), q - 32 = 8 u1 + u0 (u0 < 8,
//         -4 <= u1 < 4)                                              -> s1 u1, s1 u0, s0 u1, s0 u0 (c = 128, 16, 8, 1)
// The float arithmetic that follows is the reference's per output and block: d = fp16(d_w) * d_a, sums[w] +=
// d * aux[w], for Q4_K / Q5_K acc -= (fp16(dmin_w) * d_a) * sumi, result acc + sums[0] + ... + sums[7] - the same
// operations in the same order as qgemv_kernel, so the same bits.
// A workgroup (4 waves) takes 64 weight rows and 32 activation rows; each wave 16 weight rows against both 16-row
// activation groups. Per super-block the raw weight words (quants, high bits), the sub-block scales and minimums
// (taken out of their packing once, at staging), d / dmin widened, and the activation rows (residue-major Q8_K
// quants, d, the sub-block sums of the 16-sums) are staged in LDS with 16-byte loads, the next super-block's share
// of each thread loaded into registers while the current one is computed. A lane (weight row ml, k group kg of the
// MFMA operand layout) builds its slice operands for residue w from its row's quant word 8 kg + w (the elements of
// residue w in sub-blocks 2 kg and 2 kg + 1) and the two sub-blocks' scales; the result layout gives it weight rows
// 4 kg + v (v < 4) of activation row ml of each group: 8 outputs and their 9 float accumulators per lane.
template <int T>
constexpr int k_slices() { return T == kQ4_K ? 2 : T == kQ5_K ? 3 : 4; }
constexpr int kKTileRows = 64, kKTileActs = 32;

typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));

// Bytes b of the result hold lo16(x_b * y_b) & 0xFF for the four bytes of a word, with x_b, y_b small signed
// values given as 16-bit lanes: ex / ox the even / odd bytes' x, sy the y of bytes 0 and 1 (lane 0) and of bytes 2
// and 3 (lane 1). Every product here fits int8, so its low byte is its two's complement.
__device__ __forceinline__ uint32_t byte_products(u16x2_t ex, u16x2_t ox, u16x2_t sy) {
  const u16x2_t pe = ex * sy, po = ox * sy;
  return (__builtin_bit_cast(uint32_t, pe) & 0x00FF00FFu) | ((__builtin_bit_cast(uint32_t, po) & 0x00FF00FFu) << 8);
}

template <int T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void qgemm_k_kernel(QGemmBatch B, QA A,
                                                                                             int64_t n) {
  static_assert(T == kQ4_K || T == kQ5_K || T == kQ6_K, "K types");
  constexpr int NS = k_slices<T>();
  constexpr int WR = kKTileRows, AR = kKTileActs;
  constexpr int QS = 33;                                 // words per staged quant row (32 and one of padding)
  constexpr int HW = T == kQ5_K ? 8 : T == kQ6_K ? 16 : 0;  // high-bit words per row
  constexpr int HS = HW + 1;
  constexpr int AS = 68;                                 // words per staged activation row (64 and 4 of padding)
  __shared__ uint32_t wq[WR * QS];
  __shared__ uint32_t wh[HW > 0 ? WR * HS : 1];
  __shared__ int wsc[WR][8], wmn[WR][8];                 // Q4_K / Q5_K: 6-bit scale and minimum per sub-block
  __shared__ uint32_t wsq[WR][4];                        // Q6_K: the 16 int8 scales
  __shared__ float wdm[WR][2];
  __shared__ __align__(16) uint32_t aq[AR * AS];
  __shared__ float ad[AR];
  __shared__ int abs_[AR][8];                            // sum of the 16-sums of each sub-block (Q4_K / Q5_K)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ml = lane & 15, kg = lane >> 4;
  int wi = 0;
  for (int i = 1; i < B.n_w; ++i)
    if (int(blockIdx.x) >= B.tile0[i]) wi = i;
  const QW W = B.w[wi];
  float* __restrict__ y = B.y[wi];
  const int64_t row0 = int64_t(int(blockIdx.x) - B.tile0[wi]) * WR, t0 = int64_t(blockIdx.y) * AR;
  // A thread's share of one super-block: 2 quant u32x4 (64 rows x 128 bytes), its high-bit part, the scales and
  // d / dmin of one row (threads < 64), 2 activation u32x4 (32 rows x 256 bytes) and one row's d and 16-sums
  // (threads < 32). Rows and activation rows past the ends load clamped (staged, never stored).
  struct Share {
    u32x4_t q[2], h, sc, a[2], bs[2];
    uint32_t d, m;
    float da;
  };
  auto load_share = [&](int64_t sb, Share& sh) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = tid + 256 * u, r = e >> 3, part = e & 7;
      const int64_t rr = min(row0 + r, W.rows - 1);
      sh.q[u] = reinterpret_cast<const u32x4_t*>(W.q + (rr * W.nb + sb) * 128)[part];
    }
    if constexpr (T == kQ5_K) {
      if (tid < WR * 2) {
        const int64_t rr = min(row0 + (tid >> 1), W.rows - 1);
        sh.h = reinterpret_cast<const u32x4_t*>(W.h + (rr * W.nb + sb) * 32)[tid & 1];
      }
    }
    if constexpr (T == kQ6_K) {
      const int64_t rr = min(row0 + (tid >> 2), W.rows - 1);
      sh.h = reinterpret_cast<const u32x4_t*>(W.h + (rr * W.nb + sb) * 64)[tid & 3];
    }
    if (tid < WR) {
      const int64_t wb = min(row0 + tid, W.rows - 1) * W.nb + sb;
      sh.sc = *reinterpret_cast<const u32x4_t*>(W.s + wb * 16);
      sh.d = W.d[wb];
      sh.m = T == kQ6_K ? 0u : uint32_t(W.m[wb]);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = tid + 256 * u, r = e >> 4, part = e & 15;
      const int64_t ab = min(t0 + r, n - 1) * A.nb + sb;
      sh.a[u] = reinterpret_cast<const u32x4_t*>(A.qs + ab * 256)[part];
    }
    if (tid < AR) {
      const int64_t ab = min(t0 + tid, n - 1) * A.nb + sb;
      sh.da = A.d[ab];
      if constexpr (T != kQ6_K) {
        const u32x4_t* bp = reinterpret_cast<const u32x4_t*>(A.bsums + ab * 16);
        sh.bs[0] = bp[0];
        sh.bs[1] = bp[1];
      }
    }
  };
  auto store_share = [&](const Share& sh) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = tid + 256 * u, r = e >> 3, part = e & 7;
#pragma unroll
      for (int c = 0; c < 4; ++c) wq[r * QS + 4 * part + c] = sh.q[u][c];
    }
    if constexpr (T == kQ5_K) {
      if (tid < WR * 2) {
#pragma unroll
        for (int c = 0; c < 4; ++c) wh[(tid >> 1) * HS + 4 * (tid & 1) + c] = sh.h[c];
      }
    }
    if constexpr (T == kQ6_K) {
#pragma unroll
      for (int c = 0; c < 4; ++c) wh[(tid >> 2) * HS + 4 * (tid & 3) + c] = sh.h[c];
    }
    if (tid < WR) {
      const uint32_t scw[4] = {sh.sc[0], sh.sc[1], sh.sc[2], sh.sc[3]};
      auto sbyte = [&](int i) { return int((scw[i >> 2] >> (8 * (i & 3))) & 0xFFu); };
      if constexpr (T == kQ6_K) {
#pragma unroll
        for (int c = 0; c < 4; ++c) wsq[tid][c] = scw[c];
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {  // ggml get_scale_min_k4 (quant.cpp:52-61), compile-time byte indices
          int sk, mk;
          if (k < 4) {
            sk = sbyte(k) & 63;
            mk = sbyte(k + 4) & 63;
          } else {
            sk = (sbyte(k + 4) & 0xF) | ((sbyte(k - 4) >> 6) << 4);
            mk = (sbyte(k + 4) >> 4) | ((sbyte(k) >> 6) << 4);
          }
          wsc[tid][k] = sk;
          wmn[tid][k] = mk;
        }
      }
      wdm[tid][0] = h2f(uint16_t(sh.d));
      wdm[tid][1] = h2f(uint16_t(sh.m));
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = tid + 256 * u, r = e >> 4, part = e & 15;
      *reinterpret_cast<u32x4_t*>(&aq[r * AS + 4 * part]) = sh.a[u];
    }
    if (tid < AR) {
      ad[tid] = sh.da;
      if constexpr (T != kQ6_K) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {  // 16-sums 2k and 2k + 1: the two int16 halves of word k
          const uint32_t wk = sh.bs[k >> 2][k & 3];
          abs_[tid][k] = int(int16_t(wk & 0xFFFFu)) + int(int16_t(wk >> 16));
        }
      }
    }
  };
  // acc[j][v], sums[w][j][v]: weight row 16 wave + 4 kg + v, activation row 16 j + ml
  float sums[8][2][4], acc[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      acc[j][v] = 0.f;
#pragma unroll
      for (int w = 0; w < 8; ++w) sums[w][j][v] = 0.f;
    }
  const int ra = 16 * wave + ml;  // this lane's operand row
  Share cur;
  load_share(0, cur);
  for (int64_t sb = 0; sb < W.nb; ++sb) {
    store_share(cur);
    __syncthreads();
    load_share(sb + 1 < W.nb ? sb + 1 : sb, cur);  // in flight while this super-block is computed
    float dv[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) dv[j][v] = __fmul_rn(wdm[16 * wave + 4 * kg + v][0], ad[16 * j + ml]);
    // the lane's two sub-blocks' scales: 2 kg and 2 kg + 1 (Q4_K / Q5_K), or their int8 pairs (Q6_K)
    int s_a = 0, s_b = 0;
    uint32_t s6 = 0;
    if constexpr (T == kQ6_K)
      s6 = wsq[ra][kg];  // bytes 4 kg .. 4 kg + 3: scales 2k, 2k + 1 of sub-blocks k = 2 kg, 2 kg + 1
    else
      s_a = wsc[ra][2 * kg], s_b = wsc[ra][2 * kg + 1];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      long aop[NS];
      if constexpr (T == kQ6_K) {
        // sub-block k = 2 kg + b: half h = kg >> 1, g = 2 (kg & 1) + b; ql group lg = b at word 16 h + 8 lg + w,
        // nibble 4 (kg & 1); qh word 8 h + w at bits 2 g
        const int h = kg >> 1, sel = kg & 1;
        const uint32_t hq = wh[ra * HS + 8 * h + w];
        uint32_t sl[4][2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const int g = 2 * sel + b;
          const uint32_t lw = wq[ra * QS + 16 * h + 8 * b + w];
          const uint32_t v = ((lw >> (4 * sel)) & 0x0F0F0F0Fu) | (((hq >> (2 * g)) & 0x03030303u) << 4);
          const u16x2_t u0e = __builtin_bit_cast(u16x2_t, v & 0x00070007u);
          const u16x2_t u0o = __builtin_bit_cast(u16x2_t, (v >> 8) & 0x00070007u);
          const u16x2_t four = {4, 4};
          const u16x2_t u1e = __builtin_bit_cast(u16x2_t, (v >> 3) & 0x00070007u) - four;
          const u16x2_t u1o = __builtin_bit_cast(u16x2_t, (v >> 11) & 0x00070007u) - four;
          const int slo = int(int8_t((s6 >> (16 * b)) & 0xFFu)), shi = int(int8_t((s6 >> (16 * b + 8)) & 0xFFu));
          const u16x2_t s0 = {uint16_t(slo & 15), uint16_t(shi & 15)};
          const u16x2_t s1 = {uint16_t(slo >> 4), uint16_t(shi >> 4)};
          sl[0][b] = byte_products(u1e, u1o, s1);
          sl[1][b] = byte_products(u0e, u0o, s1);
          sl[2][b] = byte_products(u1e, u1o, s0);
          sl[3][b] = byte_products(u0e, u0o, s0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) aop[i] = long((uint64_t(sl[i][1]) << 32) | uint64_t(sl[i][0]));
      } else {
        const uint32_t qw = wq[ra * QS + 8 * kg + w];
        uint32_t qa = qw & 0x0F0F0F0Fu, qb = (qw >> 4) & 0x0F0F0F0Fu;  // sub-blocks 2 kg and 2 kg + 1
        if constexpr (T == kQ5_K) {
          const uint32_t hb = wh[ra * HS + w];
          qa |= ((hb >> (2 * kg)) & 0x01010101u) << 4;
          qb |= ((hb >> (2 * kg + 1)) & 0x01010101u) << 4;
        }
        if constexpr (T == kQ4_K) {
          aop[0] = long((uint64_t(qb * uint32_t(s_b & 7)) << 32) | uint64_t(qa * uint32_t(s_a & 7)));
          aop[1] = long((uint64_t(qb * uint32_t(s_b >> 3)) << 32) | uint64_t(qa * uint32_t(s_a >> 3)));
        } else {
          aop[0] = long((uint64_t(qb * uint32_t(s_b & 3)) << 32) | uint64_t(qa * uint32_t(s_a & 3)));
          aop[1] = long((uint64_t(qb * uint32_t((s_b >> 2) & 3)) << 32) | uint64_t(qa * uint32_t((s_a >> 2) & 3)));
          aop[2] = long((uint64_t(qb * uint32_t(s_b >> 4)) << 32) | uint64_t(qa * uint32_t(s_a >> 4)));
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint2 bw = *reinterpret_cast<const uint2*>(&aq[(16 * j + ml) * AS + 8 * w + 2 * kg]);
        const long bop = long((uint64_t(bw.y) << 32) | uint64_t(bw.x));
        i32x4_t c[NS];
#pragma unroll
        for (int sl = 0; sl < NS; ++sl)
          c[sl] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop[sl], bop, i32x4_t{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          int aux;
          if constexpr (T == kQ6_K)
            aux = 128 * c[0][v] + 16 * c[1][v] + 8 * c[2][v] + c[3][v];
          else if constexpr (T == kQ5_K)
            aux = c[0][v] + 4 * c[1][v] + 16 * c[2][v];
          else
            aux = c[0][v] + 8 * c[1][v];
          sums[w][j][v] = __fadd_rn(sums[w][j][v], __fmul_rn(dv[j][v], float(aux)));
        }
      }
    }
    if constexpr (T != kQ6_K) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int t = 16 * j + ml;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int rv = 16 * wave + 4 * kg + v;
          int sumi = 0;
#pragma unroll
          for (int k = 0; k < 8; ++k) sumi += abs_[t][k] * wmn[rv][k];
          acc[j][v] = __fsub_rn(acc[j][v], __fmul_rn(__fmul_rn(wdm[rv][1], ad[t]), float(sumi)));
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float o = acc[j][v];
#pragma unroll
      for (int w = 0; w < 8; ++w) o = __fadd_rn(o, sums[w][j][v]);
      const int64_t r = row0 + 16 * wave + 4 * kg + v, t = t0 + 16 * j + ml;
      if (r < W.rows && t < n) y[t * W.rows + r] = o;
    }
}

// qgemm_k_small_kernel: the K types for calls of few activation rows, where 64-row weight tiles leave most CUs
// idle and each workgroup would walk every super-block alone. A workgroup takes 16 weight rows x 32 activation
// rows and its 4 waves split the super-blocks (wave w: w, w + 4, ...): each computes its super-block's float terms
// - d * aux[l] for the eight lanes and, for Q4_K / Q5_K, the minimum term, with the operands, slices and
// expressions of qgemm_k_kernel, its operands read straight from global memory - and writes them to LDS; per round
// of four super-blocks the 256 threads, two outputs each, add them to their running sums in super-block order:
// the reference's order, so the same bits.
template <int T>
__global__ __launch_bounds__(256) void qgemm_k_small_kernel(QGemmBatch B, QA A, int64_t n) {
  static_assert(T == kQ4_K || T == kQ5_K || T == kQ6_K, "K types");
  constexpr int NS = k_slices<T>();
  constexpr int NTM = T == kQ6_K ? 8 : 9;  // float terms per output and super-block
  __shared__ float terms[4][NTM][16][33];  // [wave][term][weight row][activation row], one column of padding
  __shared__ float rowd[4][16][2];         // per wave: d, dmin of its super-block's 16 rows
  __shared__ int rowm[4][16][8], rows6[4][16][8];  // minimums and 6-bit scales (Q4_K / Q5_K)
  __shared__ uint32_t rowq6[4][16][4];     // Q6_K: the 16 int8 scales
  __shared__ float actd[4][32];
  __shared__ int actb[4][32][8];           // sums of the 16-sums per sub-block (Q4_K / Q5_K)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ml = lane & 15, kg = lane >> 4;
  int wi = 0;
  for (int i = 1; i < B.n_w; ++i)
    if (int(blockIdx.x) >= B.tile0[i]) wi = i;
  const QW W = B.w[wi];
  float* __restrict__ y = B.y[wi];
  const int64_t row0 = int64_t(int(blockIdx.x) - B.tile0[wi]) * 16, t0 = int64_t(blockIdx.y) * 32;
  // owner sums: outputs (weight row tid & 15, activation rows (tid >> 4) and (tid >> 4) + 16)
  float sums[2][8], acc[2];
#pragma unroll
  for (int o = 0; o < 2; ++o) {
    acc[o] = 0.f;
#pragma unroll
    for (int l = 0; l < 8; ++l) sums[o][l] = 0.f;
  }
  const int64_t ra = min(row0 + ml, W.rows - 1);  // this lane's operand row
  for (int64_t s0 = 0; s0 < W.nb; s0 += 4) {
    const int64_t sb = s0 + wave;
    const bool has = sb < W.nb;
    const int64_t sbc = has ? sb : W.nb - 1;
    // this wave's super-block: per-row and per-activation-row values into its LDS slices
    if (lane < 16) {
      const int64_t wb = min(row0 + lane, W.rows - 1) * W.nb + sbc;
      const u32x4_t sc = *reinterpret_cast<const u32x4_t*>(W.s + wb * 16);
      const uint32_t scw[4] = {sc[0], sc[1], sc[2], sc[3]};
      auto sbyte = [&](int i) { return int((scw[i >> 2] >> (8 * (i & 3))) & 0xFFu); };
      rowd[wave][lane][0] = h2f(W.d[wb]);
      if constexpr (T == kQ6_K) {
        rowd[wave][lane][1] = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) rowq6[wave][lane][c] = scw[c];
      } else {
        rowd[wave][lane][1] = h2f(W.m[wb]);
#pragma unroll
        for (int k = 0; k < 8; ++k) {  // ggml get_scale_min_k4 (quant.cpp:52-61), compile-time byte indices
          int sk, mk;
          if (k < 4) {
            sk = sbyte(k) & 63;
            mk = sbyte(k + 4) & 63;
          } else {
            sk = (sbyte(k + 4) & 0xF) | ((sbyte(k - 4) >> 6) << 4);
            mk = (sbyte(k + 4) >> 4) | ((sbyte(k) >> 6) << 4);
          }
          rows6[wave][lane][k] = sk;
          rowm[wave][lane][k] = mk;
        }
      }
    } else if (lane < 48) {
      const int a = lane - 16;
      const int64_t ab = min(t0 + a, n - 1) * A.nb + sbc;
      actd[wave][a] = A.d[ab];
      if constexpr (T != kQ6_K) {
        const u32x4_t* bp = reinterpret_cast<const u32x4_t*>(A.bsums + ab * 16);
        const u32x4_t b0 = bp[0], b1 = bp[1];
#pragma unroll
        for (int k = 0; k < 8; ++k) {  // 16-sums 2k and 2k + 1: the two int16 halves of word k
          const uint32_t wk = k < 4 ? b0[k] : b1[k - 4];
          actb[wave][a][k] = int(int16_t(wk & 0xFFFFu)) + int(int16_t(wk >> 16));
        }
      }
    }
    // the lane's operand words: its row's quant words of its k group (and their high bits), every residue
    const int64_t wb = ra * W.nb + sbc;
    u32x4_t qv[T == kQ6_K ? 4 : 2], hv[2];
    if constexpr (T == kQ6_K) {
      const u32x4_t* q = reinterpret_cast<const u32x4_t*>(W.q + wb * 128 + 64 * (kg >> 1));
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = q[i];
      const u32x4_t* h = reinterpret_cast<const u32x4_t*>(W.h + wb * 64 + 32 * (kg >> 1));
      hv[0] = h[0], hv[1] = h[1];
    } else {
      const u32x4_t* q = reinterpret_cast<const u32x4_t*>(W.q + wb * 128 + 32 * kg);
      qv[0] = q[0], qv[1] = q[1];
      if constexpr (T == kQ5_K) {
        const u32x4_t* h = reinterpret_cast<const u32x4_t*>(W.h + wb * 32);
        hv[0] = h[0], hv[1] = h[1];
      }
    }
    uint2 bw[2][8];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t ab = min(t0 + 16 * j + ml, n - 1) * A.nb + sbc;
      const uint8_t* aq = reinterpret_cast<const uint8_t*>(A.qs) + ab * 256;
#pragma unroll
      for (int w = 0; w < 8; ++w) bw[j][w] = *reinterpret_cast<const uint2*>(aq + 32 * w + 8 * kg);
    }
    __syncthreads();  // this round's row and activation values are in LDS
    if (has) {
      float dv[2][4];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) dv[j][v] = __fmul_rn(rowd[wave][4 * kg + v][0], actd[wave][16 * j + ml]);
      int s_a = 0, s_b = 0;
      uint32_t s6 = 0;
      if constexpr (T == kQ6_K)
        s6 = rowq6[wave][ml][kg];
      else
        s_a = rows6[wave][ml][2 * kg], s_b = rows6[wave][ml][2 * kg + 1];
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        long aop[NS];
        if constexpr (T == kQ6_K) {
          const int sel = kg & 1;
          const uint32_t hq = hv[w >> 2][w & 3];
          uint32_t sl[4][2];
#pragma unroll
          for (int b = 0; b < 2; ++b) {
            const int g = 2 * sel + b;
            const uint32_t lw = qv[(8 * b + w) >> 2][(8 * b + w) & 3];
            const uint32_t v = ((lw >> (4 * sel)) & 0x0F0F0F0Fu) | (((hq >> (2 * g)) & 0x03030303u) << 4);
            const u16x2_t u0e = __builtin_bit_cast(u16x2_t, v & 0x00070007u);
            const u16x2_t u0o = __builtin_bit_cast(u16x2_t, (v >> 8) & 0x00070007u);
            const u16x2_t four = {4, 4};
            const u16x2_t u1e = __builtin_bit_cast(u16x2_t, (v >> 3) & 0x00070007u) - four;
            const u16x2_t u1o = __builtin_bit_cast(u16x2_t, (v >> 11) & 0x00070007u) - four;
            const int slo = int(int8_t((s6 >> (16 * b)) & 0xFFu)), shi = int(int8_t((s6 >> (16 * b + 8)) & 0xFFu));
            const u16x2_t s0 = {uint16_t(slo & 15), uint16_t(shi & 15)};
            const u16x2_t s1 = {uint16_t(slo >> 4), uint16_t(shi >> 4)};
            sl[0][b] = byte_products(u1e, u1o, s1);
            sl[1][b] = byte_products(u0e, u0o, s1);
            sl[2][b] = byte_products(u1e, u1o, s0);
            sl[3][b] = byte_products(u0e, u0o, s0);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) aop[i] = long((uint64_t(sl[i][1]) << 32) | uint64_t(sl[i][0]));
        } else {
          const uint32_t qw = qv[w >> 2][w & 3];
          uint32_t qa = qw & 0x0F0F0F0Fu, qb = (qw >> 4) & 0x0F0F0F0Fu;  // sub-blocks 2 kg and 2 kg + 1
          if constexpr (T == kQ5_K) {
            const uint32_t hb = hv[w >> 2][w & 3];
            qa |= ((hb >> (2 * kg)) & 0x01010101u) << 4;
            qb |= ((hb >> (2 * kg + 1)) & 0x01010101u) << 4;
          }
          if constexpr (T == kQ4_K) {
            aop[0] = long((uint64_t(qb * uint32_t(s_b & 7)) << 32) | uint64_t(qa * uint32_t(s_a & 7)));
            aop[1] = long((uint64_t(qb * uint32_t(s_b >> 3)) << 32) | uint64_t(qa * uint32_t(s_a >> 3)));
          } else {
            aop[0] = long((uint64_t(qb * uint32_t(s_b & 3)) << 32) | uint64_t(qa * uint32_t(s_a & 3)));
            aop[1] = long((uint64_t(qb * uint32_t((s_b >> 2) & 3)) << 32) | uint64_t(qa * uint32_t((s_a >> 2) & 3)));
            aop[2] = long((uint64_t(qb * uint32_t(s_b >> 4)) << 32) | uint64_t(qa * uint32_t(s_a >> 4)));
          }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const long bop = long((uint64_t(bw[j][w].y) << 32) | uint64_t(bw[j][w].x));
          i32x4_t c[NS];
#pragma unroll
          for (int sl = 0; sl < NS; ++sl)
            c[sl] = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop[sl], bop, i32x4_t{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            int aux;
            if constexpr (T == kQ6_K)
              aux = 128 * c[0][v] + 16 * c[1][v] + 8 * c[2][v] + c[3][v];
            else if constexpr (T == kQ5_K)
              aux = c[0][v] + 4 * c[1][v] + 16 * c[2][v];
            else
              aux = c[0][v] + 8 * c[1][v];
            terms[wave][w][4 * kg + v][16 * j + ml] = __fmul_rn(dv[j][v], float(aux));
          }
        }
      }
      if constexpr (T != kQ6_K) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int t = 16 * j + ml;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int rv = 4 * kg + v;
            int sumi = 0;
#pragma unroll
            for (int k = 0; k < 8; ++k) sumi += actb[wave][t][k] * rowm[wave][rv][k];
            terms[wave][8][rv][t] = __fmul_rn(__fmul_rn(rowd[wave][rv][1], actd[wave][t]), float(sumi));
          }
        }
      }
    }
    __syncthreads();  // every wave's terms are in LDS
    const int orow = tid & 15;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s0 + s < W.nb) {
#pragma unroll
        for (int o = 0; o < 2; ++o) {
          const int ot = (tid >> 4) + 16 * o;
#pragma unroll
          for (int l = 0; l < 8; ++l) sums[o][l] = __fadd_rn(sums[o][l], terms[s][l][orow][ot]);
          if constexpr (T != kQ6_K) acc[o] = __fsub_rn(acc[o], terms[s][8][orow][ot]);
        }
      }
    }
    __syncthreads();  // the terms are consumed before the next round overwrites them
  }
#pragma unroll
  for (int o = 0; o < 2; ++o) {
    float r = acc[o];
#pragma unroll
    for (int l = 0; l < 8; ++l) r = __fadd_rn(r, sums[o][l]);
    const int64_t row = row0 + (tid & 15), t = t0 + (tid >> 4) + 16 * o;
    if (row < W.rows && t < n) y[t * W.rows + row] = r;
  }
}

// The small-call K kernel runs while 64 x 32 tiles would give fewer than this many workgroups (measured at the QKV
// shape, 48 such row tiles: Q4_K faster up to 64 rows, Q5_K / Q6_K up to 128-160; beyond, the 64 x 32 kernel).
template <int T>
constexpr int64_t k_small_max_wgs() { return T == kQ4_K ? 128 : 256; }
template <int T>
hipError_t launch_k(bool small, dim3 grid32, hipStream_t s, const QGemmBatch& B, const QA& A, int64_t n) {
  if (small) return nbhs_timing::launch(NBHS_K_QGEMM, qgemm_k_small_kernel<T>, grid32, dim3(256), s, B, A, n);
  return nbhs_timing::launch(NBHS_K_QGEMM, qgemm_k_kernel<T>, grid32, dim3(256), s, B, A, n);
}

// ---- dequantization (quant.cpp:157-242), one thread per block of one output row ----

template <int T>
__global__ __launch_bounds__(256) void dequant_rows_kernel(QW W, const int32_t* __restrict__ ids, int64_t n,
                                                           float* __restrict__ out) {
  const int64_t be = block_elems(T), d_ = W.nb * be;
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n * W.nb) return;
  const int64_t t = i / W.nb, b = i % W.nb, wb = int64_t(ids[t]) * W.nb + b;
  float* o = out + t * d_ + b * be;
  const float d = h2f(W.d[wb]);
  if constexpr (T == kQ8_0) {
    const int8_t* q = reinterpret_cast<const int8_t*>(W.q + wb * 32);
    for (int j = 0; j < 32; ++j) o[j] = __fmul_rn(float(q[j]), d);
  } else if constexpr (T == kQ4_0 || T == kQ5_0 || T == kQ5_1) {
    const uint8_t* q = W.q + wb * 16;
    const uint32_t qh = T == kQ4_0 ? 0u : *reinterpret_cast<const uint32_t*>(W.h + wb * 4);
    const float m = T == kQ5_1 ? h2f(W.m[wb]) : 0.f;
    for (int j = 0; j < 16; ++j) {
      int x0 = q[j] & 0x0F, x1 = q[j] >> 4;
      if constexpr (T != kQ4_0) x0 |= ((qh >> j) & 1) << 4, x1 |= ((qh >> (j + 16)) & 1) << 4;
      if constexpr (T == kQ5_1) {
        o[j] = __fadd_rn(__fmul_rn(float(x0), d), m);
        o[j + 16] = __fadd_rn(__fmul_rn(float(x1), d), m);
      } else {
        constexpr int bias = T == kQ4_0 ? 8 : 16;
        o[j] = __fmul_rn(float(x0 - bias), d);
        o[j + 16] = __fmul_rn(float(x1 - bias), d);
      }
    }
  } else if constexpr (T == kQ4_K || T == kQ5_K) {
    const uint8_t* qs = W.q + wb * 128;
    const float mn = h2f(W.m[wb]);
    for (int k = 0; k < 8; ++k) {
      int sc, m;
      scale_min_k4(k, W.s + wb * 16, sc, m);
      const float d1 = __fmul_rn(d, float(sc)), m1 = __fmul_rn(mn, float(m));
      for (int e = 0; e < 32; ++e) {
        const int p = residue_pos(e);
        int q = (qs[32 * (k >> 1) + p] >> (4 * (k & 1))) & 0xF;
        if constexpr (T == kQ5_K) q += ((W.h[wb * 32 + p] >> k) & 1) ? 16 : 0;
        o[32 * k + e] = __fsub_rn(__fmul_rn(d1, float(q)), m1);
      }
    }
  } else {  // Q6_K
    const int8_t* scl = reinterpret_cast<const int8_t*>(W.s + wb * 16);
    for (int k = 0; k < 8; ++k) {
      const int h = k >> 2, g = k & 3;
      const uint8_t* ql = W.q + wb * 128 + 64 * h + 32 * (g & 1);
      const uint8_t* qh = W.h + wb * 64 + 32 * h;
      for (int e = 0; e < 32; ++e) {
        const int p = residue_pos(e);
        const int q = (((ql[p] >> ((g >> 1) * 4)) & 0xF) | (((qh[p] >> (2 * g)) & 3) << 4)) - 32;
        const float dk = __fmul_rn(d, float(scl[2 * k + (e >> 4)]));
        o[32 * k + e] = __fmul_rn(dk, float(q));
      }
    }
  }
}

QW weight_of(int type, const void* w, int64_t rows, int64_t in) {
  const int64_t nb = in / block_elems(type);
  const WeightLayout l = weight_layout(type, rows, nb);
  const uint8_t* base = static_cast<const uint8_t*>(w);
  return QW{base + l.q_off, base + l.h_off, base + l.s_off, reinterpret_cast<const uint16_t*>(base + l.d_off),
            reinterpret_cast<const uint16_t*>(base + l.m_off), rows, nb};
}

template <int T>
int launch_gemv(const QBatch& B, const int64_t* rows, int n_w, const QA& A, const float* x, int64_t in, int64_t n,
                bool fused, hipStream_t s) {
  int64_t total = 0;
  for (int i = 0; i < n_w; ++i) total += rows[i];
  const bool wide = fused && n == 1 && total >= kWideRows;
  const int rw = rows_per_wave(is_k(T), fused ? (n == 1 ? 1 : 4) : (n <= 4 ? 4 : 16), wide);
  QBatch b = B;
  int64_t waves = 0;
  for (int i = 0; i < n_w; ++i) b.wave0[i] = waves, waves += (rows[i] + rw - 1) / rw;
  if (waves >= (int64_t(1) << 31)) return NBHS_EINVAL;
  const dim3 grid{unsigned(waves), 1, 1}, block{64, 1, 1};
  if (fused) {
    if (wide)
      return nbhs_timing::launch(NBHS_K_QGEMV, qgemv_kernel<T, 1, true, true>, grid, block, s, b, A, x, in, int(n));
    if (n == 1)
      return nbhs_timing::launch(NBHS_K_QGEMV, qgemv_kernel<T, 1, true, false>, grid, block, s, b, A, x, in, int(n));
    return nbhs_timing::launch(NBHS_K_QGEMV, qgemv_kernel<T, 4, true, false>, grid, block, s, b, A, x, in, int(n));
  }
  if (n <= 4)
    return nbhs_timing::launch(NBHS_K_QGEMV, qgemv_kernel<T, 4, false, false>, grid, block, s, b, A, x, in, int(n));
  return nbhs_timing::launch(NBHS_K_QGEMV, qgemv_kernel<T, 16, false, false>, grid, block, s, b, A, x, in, int(n));
}

template <int T>
int launch_dequant(const QW& W, const int32_t* ids, int64_t n, float* out, hipStream_t s) {
  const int64_t blocks = (n * W.nb + 255) / 256;
  return nbhs_timing::launch(NBHS_K_ELEMENTWISE, dequant_rows_kernel<T>, dim3(unsigned(blocks)), dim3(256), s, W, ids,
                             n, out);
}

}  // namespace

extern "C" {

int64_t nbhs_quant_weight_bytes(int type, int64_t rows, int64_t in) {
  if (!is_quant(type) || rows <= 0 || in <= 0 || in % block_elems(type)) return -1;
  return weight_layout(type, rows, in / block_elems(type)).bytes;
}

int64_t nbhs_quant_act_bytes(int type, int64_t n, int64_t in) {
  if (!is_quant(type) || n <= 0 || in <= 0 || in % block_elems(type)) return -1;
  return act_layout(act_of(type), n, in / block_elems(type)).bytes;
}

int nbhs_quantize_acts(int type, const float* x, int64_t n, int64_t in, void* acts, nbhs_stream stream) {
  if (!is_quant(type) || !x || !acts || n <= 0 || in <= 0 || in % block_elems(type)) return NBHS_EINVAL;
  const int act = act_of(type);
  const int64_t nb = in / block_elems(type), blocks = n * nb;
  const ActLayout l = act_layout(act, n, nb);
  uint8_t* base = static_cast<uint8_t*>(acts);
  int8_t* qs = reinterpret_cast<int8_t*>(base + l.qs_off);
  float* d = reinterpret_cast<float*>(base + l.d_off);
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (act == kActQ8_K) {
    if (blocks >= (int64_t(1) << 31)) return NBHS_EINVAL;
    return nbhs_timing::launch(NBHS_K_QUANTIZE, quantize_q8k_kernel<false>, dim3(unsigned(blocks)), dim3(64), s, x, in,
                               qs, d, reinterpret_cast<int16_t*>(base + l.bsums_off));
  }
  const dim3 grid{unsigned((blocks + 255) / 256), 1, 1};
  if (act == kActQ8_1)
    return nbhs_timing::launch(NBHS_K_QUANTIZE, quantize_q8_kernel<true>, grid, dim3(256), s, x, in, n, qs, d,
                               reinterpret_cast<float*>(base + l.s_off));
  return nbhs_timing::launch(NBHS_K_QUANTIZE, quantize_q8_kernel<false>, grid, dim3(256), s, x, in, n, qs, d,
                             static_cast<float*>(nullptr));
}

int nbhs_quantize_acts_rm(int type, const float* x, int64_t n, int64_t in, void* acts, nbhs_stream stream) {
  if (!is_k(type) || !x || !acts || n <= 0 || in <= 0 || in % 256) return NBHS_EINVAL;
  const int64_t nb = in / 256, blocks = n * nb;
  if (blocks >= (int64_t(1) << 31)) return NBHS_EINVAL;
  const ActLayout l = act_layout(kActQ8_K, n, nb);
  uint8_t* base = static_cast<uint8_t*>(acts);
  return nbhs_timing::launch(NBHS_K_QUANTIZE, quantize_q8k_kernel<true>, dim3(unsigned(blocks)), dim3(64),
                             reinterpret_cast<hipStream_t>(stream), x, in, reinterpret_cast<int8_t*>(base + l.qs_off),
                             reinterpret_cast<float*>(base + l.d_off), reinterpret_cast<int16_t*>(base + l.bsums_off));
}

int nbhs_qgemv_multi(int type, int n_w, const void* const* w, const int64_t* rows, float* const* y, int64_t in,
                     const float* x, const void* acts, int64_t n_acts, int64_t t0, int64_t n, nbhs_stream stream) {
  if (!is_quant(type) || n_w <= 0 || n_w > kMaxQWeights || !w || !rows || !y || in <= 0 ||
      in % block_elems(type) || n <= 0 || n > NBHS_GEMV_MAX_ROWS)
    return NBHS_EINVAL;
  const bool fused = acts == nullptr;
  if (fused ? (!x || n > 4 || t0 != 0 || reinterpret_cast<uintptr_t>(x) % 16 || in % 4) : (t0 < 0 || t0 + n > n_acts))
    return NBHS_EINVAL;
  QBatch B{};
  for (int i = 0; i < n_w; ++i) {
    if (!w[i] || !y[i] || rows[i] <= 0) return NBHS_EINVAL;
    B.w[i] = weight_of(type, w[i], rows[i], in);
    B.y[i] = y[i];
  }
  B.n_w = n_w;
  const int64_t nb = in / block_elems(type);
  QA A{};
  A.nb = nb;
  if (!fused) {
    const int act = act_of(type);
    const ActLayout l = act_layout(act, n_acts, nb);
    const uint8_t* base = static_cast<const uint8_t*>(acts);
    const int64_t b0 = t0 * nb;  // first block of activation row t0
    A.qs = reinterpret_cast<const int8_t*>(base + l.qs_off) + b0 * (act == kActQ8_K ? 256 : 32);
    A.d = reinterpret_cast<const float*>(base + l.d_off) + b0;
    A.s = act == kActQ8_1 ? reinterpret_cast<const float*>(base + l.s_off) + b0 : nullptr;
    A.bsums = reinterpret_cast<const int16_t*>(base + l.bsums_off) + b0 * 16;
  }
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (type) {
    case kQ4_0: return launch_gemv<kQ4_0>(B, rows, n_w, A, x, in, n, fused, s);
    case kQ5_0: return launch_gemv<kQ5_0>(B, rows, n_w, A, x, in, n, fused, s);
    case kQ5_1: return launch_gemv<kQ5_1>(B, rows, n_w, A, x, in, n, fused, s);
    case kQ8_0: return launch_gemv<kQ8_0>(B, rows, n_w, A, x, in, n, fused, s);
    case kQ4_K: return launch_gemv<kQ4_K>(B, rows, n_w, A, x, in, n, fused, s);
    case kQ5_K: return launch_gemv<kQ5_K>(B, rows, n_w, A, x, in, n, fused, s);
    case kQ6_K: return launch_gemv<kQ6_K>(B, rows, n_w, A, x, in, n, fused, s);
    default: return NBHS_EINVAL;
  }
}

int nbhs_qgemm_multi(int type, int n_w, const void* const* w, const int64_t* rows, float* const* y, int64_t in,
                     const void* acts, int64_t n, nbhs_stream stream) {
  if (!is_quant(type) || n_w <= 0 || n_w > kMaxQWeights || !w || !rows || !y || !acts ||
      in <= 0 || in % block_elems(type) || n <= 0 || (n + 31) / 32 > 65535)
    return NBHS_EINVAL;
  // weight-row tiles of every weight at 64 rows (each weight's tiles start at its tile0 in grid x) and, for the
  // legacy types' smallest launches, at 32
  QGemmBatch B{};
  int64_t tiles64 = 0, tiles32 = 0;
  for (int i = 0; i < n_w; ++i) {
    if (!w[i] || !y[i] || rows[i] <= 0) return NBHS_EINVAL;
    B.w[i] = weight_of(type, w[i], rows[i], in);
    B.y[i] = y[i];
    tiles64 += (rows[i] + 63) / 64;
    tiles32 += (rows[i] + 31) / 32;
    if ((tiles32 + 1) * 2 >= (int64_t(1) << 31)) return NBHS_EINVAL;  // 16-row tiles fit too
  }
  B.n_w = n_w;
  LegacyTile tile = kTile64x64;
  if (!is_k(type)) {
    if (tiles64 * ((n + 63) / 64) >= kLegacyMinWgs && n > 32)
      tile = kTile64x64;
    else if (tiles64 * ((n + 31) / 32) >= kLegacyMinWgs)
      tile = kTile64x32;
    else
      tile = kTile32x32;
  }
  // K types: the small-call kernel (16-row weight tiles, super-blocks split over the waves) when 64-row tiles
  // would give fewer than kKSmallMaxWgs workgroups
  const bool small = is_k(type) && tiles64 * ((n + 31) / 32) < (type == kQ4_K ? k_small_max_wgs<kQ4_K>()
                                                                                 : k_small_max_wgs<kQ6_K>());
  const int64_t tile_rows = small ? 16 : tile == kTile32x32 ? 32 : 64;
  int64_t tiles = 0;
  for (int i = 0; i < n_w; ++i) {
    B.tile0[i] = int(tiles);
    tiles += (rows[i] + tile_rows - 1) / tile_rows;
  }
  const int act = act_of(type);
  const ActLayout l = act_layout(act, n, B.w[0].nb);
  const uint8_t* base = static_cast<const uint8_t*>(acts);
  const QA A{reinterpret_cast<const int8_t*>(base + l.qs_off), reinterpret_cast<const float*>(base + l.d_off),
             act == kActQ8_1 ? reinterpret_cast<const float*>(base + l.s_off) : nullptr,
             act == kActQ8_K ? reinterpret_cast<const int16_t*>(base + l.bsums_off) : nullptr, B.w[0].nb};
  const dim3 grid32{unsigned(tiles), unsigned((n + 31) / 32), 1}, block{256, 1, 1};
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (type) {
    case kQ4_K: return launch_k<kQ4_K>(small, grid32, s, B, A, n);
    case kQ5_K: return launch_k<kQ5_K>(small, grid32, s, B, A, n);
    case kQ6_K: return launch_k<kQ6_K>(small, grid32, s, B, A, n);
    case kQ4_0: return launch_legacy<kQ4_0>(tile, unsigned(tiles), n, s, B, A);
    case kQ5_0: return launch_legacy<kQ5_0>(tile, unsigned(tiles), n, s, B, A);
    case kQ5_1: return launch_legacy<kQ5_1>(tile, unsigned(tiles), n, s, B, A);
    case kQ8_0: return launch_legacy<kQ8_0>(tile, unsigned(tiles), n, s, B, A);
    default: return NBHS_EINVAL;
  }
}

int nbhs_dequant_rows(int type, const void* w, int64_t rows, int64_t in, const int32_t* ids, int64_t n, float* out,
                      nbhs_stream stream) {
  if (!is_quant(type) || !w || !ids || !out || rows <= 0 || in <= 0 || in % block_elems(type) || n <= 0)
    return NBHS_EINVAL;
  const QW W = weight_of(type, w, rows, in);
  if ((n * W.nb + 255) / 256 >= (int64_t(1) << 31)) return NBHS_EINVAL;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (type) {
    case kQ4_0: return launch_dequant<kQ4_0>(W, ids, n, out, s);
    case kQ5_0: return launch_dequant<kQ5_0>(W, ids, n, out, s);
    case kQ5_1: return launch_dequant<kQ5_1>(W, ids, n, out, s);
    case kQ8_0: return launch_dequant<kQ8_0>(W, ids, n, out, s);
    case kQ4_K: return launch_dequant<kQ4_K>(W, ids, n, out, s);
    case kQ5_K: return launch_dequant<kQ5_K>(W, ids, n, out, s);
    case kQ6_K: return launch_dequant<kQ6_K>(W, ids, n, out, s);
    default: return NBHS_EINVAL;
  }
}

}  // extern "C"
