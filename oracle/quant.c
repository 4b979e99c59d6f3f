/*
 * CPU oracle for nibble's quantized weight formats. TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Restates src/quant.cpp (the reference's scalar oracle, itself ggml's generic code with its floating-point
 * operation order) and the fp16 conversions of src/fp16.h: the Q8_0 / Q8_1 / Q8_K activation quantizers,
 * dequantization of every block format, and every block dot product. Block layouts are those of src/quant.h
 * (llama.cpp's, byte for byte); blocks are read through memcpy since they may sit at any byte offset.
 * Pinned in tests/test_quant_oracle.py against the golden vectors of tests/data/quant_golden.inc (produced by
 * llama.cpp itself) and bit for bit against the compiled reference (oracle/_ref).
 */
#include <math.h>
#include <stdlib.h>
#include <stdint.h>
#include <string.h>

#include "oracle.h"

enum { QK = 32, QK_K = 256 };
enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14 };

typedef struct { uint16_t d; uint8_t qs[16]; } q4_0_t;                                  /* 18 bytes */
typedef struct { uint16_t d; int8_t qs[32]; } q8_0_t;                                   /* 34 */
typedef struct { uint16_t d; uint8_t qh[4]; uint8_t qs[16]; } q5_0_t;                    /* 22 */
typedef struct { uint16_t d, m; uint8_t qh[4]; uint8_t qs[16]; } q5_1_t;                 /* 24 */
typedef struct { uint16_t d, s; int8_t qs[32]; } q8_1_t;                                 /* 36 */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } q4_k_t;        /* 144 */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } q5_k_t; /* 176 */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } q6_k_t; /* 210 */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } q8_k_t;                   /* 292 */

_Static_assert(sizeof(q4_0_t) == 18 && sizeof(q8_0_t) == 34 && sizeof(q5_0_t) == 22 && sizeof(q5_1_t) == 24 &&
                   sizeof(q8_1_t) == 36 && sizeof(q4_k_t) == 144 && sizeof(q5_k_t) == 176 &&
                   sizeof(q6_k_t) == 210 && sizeof(q8_k_t) == 292,
               "block layouts of src/quant.h:34-110");

int64_t orc_block_bytes(int type) {
  switch (type) {
    case T_F32: return 4;
    case T_F16: return 2;
    case T_Q4_0: return 18;
    case T_Q5_0: return 22;
    case T_Q5_1: return 24;
    case T_Q8_0: return 34;
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q6_K: return 210;
    default: return -1;
  }
}

int64_t orc_block_elems(int type) {
  switch (type) {
    case T_F32:
    case T_F16: return 1;
    case T_Q4_0:
    case T_Q5_0:
    case T_Q5_1:
    case T_Q8_0: return QK;
    case T_Q4_K:
    case T_Q5_K:
    case T_Q6_K: return QK_K;
    default: return -1;
  }
}

/* fp16.h:45-70: float to the nearest half, ties to even; overflow to infinity, underflow to signed zero; NaN stays
 * NaN with the quiet bit set and the top payload bits kept. */
uint16_t orc_fp32_to_fp16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, e = (x >> 23) & 0xFFu;
  uint32_t m = x & 0x7FFFFFu;
  if (e == 0xFFu) return (uint16_t)(sign | 0x7C00u | (m ? (0x200u | (m >> 13)) : 0u));
  const int exp = (int)e - 127 + 15; /* rebias */
  if (exp >= 31) return (uint16_t)(sign | 0x7C00u);
  if (exp <= 0) { /* half subnormal (or zero): shift the full significand into place, round to even */
    if (exp < -10) return (uint16_t)sign;
    m |= 0x800000u;
    const int shift = 14 - exp;
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)exp << 10) | (m >> 13);
  const uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h; /* a carry into the exponent is correct rounding */
  return (uint16_t)(sign | h);
}

static float h2f(uint16_t h) { return orc_fp16_to_fp32(h); }

/* quant.cpp:37-49 (quantize_block_q8): amax by fmax (NaN skipped, flagged), d = amax / 127, id = 1 / d (0 for
 * d = 0), q = roundf(x * id) clamped to [-127, 127], NaN to 0; returns d before fp16 rounding. */
static float quantize_block_q8(const float* x, int8_t* qs) {
  float amax = 0.f;
  int has_nan = 0;
  for (int j = 0; j < QK; ++j) {
    amax = fmaxf(amax, fabsf(x[j]));
    has_nan |= isnan(x[j]);
  }
  const float d = has_nan ? NAN : amax / 127.f;
  const float id = d != 0.f ? 1.0f / d : 0.0f;
  for (int j = 0; j < QK; ++j) {
    const float r = roundf(x[j] * id);
    qs[j] = r != r ? 0 : (int8_t)fminf(127.f, fmaxf(-127.f, r));
  }
  return d;
}

/* quant.cpp:245-253 */
int orc_quantize_q8_0(const float* x, void* y, int64_t n) {
  if (n < 0 || n % QK) return -1;
  for (int64_t b = 0; b < n / QK; ++b) {
    q8_0_t blk;
    blk.d = orc_fp32_to_fp16(quantize_block_q8(x + b * QK, blk.qs));
    memcpy((uint8_t*)y + b * sizeof blk, &blk, sizeof blk);
  }
  return 0;
}

/* quant.cpp:256-268: Q8_0 plus s = fp16(float(sum(qs)) * d) from the unrounded d. */
int orc_quantize_q8_1(const float* x, void* y, int64_t n) {
  if (n < 0 || n % QK) return -1;
  for (int64_t b = 0; b < n / QK; ++b) {
    q8_1_t blk;
    const float d = quantize_block_q8(x + b * QK, blk.qs);
    blk.d = orc_fp32_to_fp16(d);
    int sum = 0;
    for (int j = 0; j < QK; ++j) sum += blk.qs[j];
    blk.s = orc_fp32_to_fp16((float)sum * d);
    memcpy((uint8_t*)y + b * sizeof blk, &blk, sizeof blk);
  }
  return 0;
}

/* quant.cpp:146-152 (ggml nearest_int): round half to even by adding 1.5 * 2^23 and reading the mantissa. */
static int nearest_int(float fval) {
  const float val = fval + 12582912.f;
  int32_t i;
  memcpy(&i, &val, 4);
  return (i & 0x007fffff) - 0x00400000;
}

/* quant.cpp:273-303: the scale comes from the first element of largest magnitude, iscale = -127 / max, q =
 * nearest_int of iscale * x clamped to [-127, 127] (NaN to 0), bsums per 16, d = 1 / iscale; all-zero blocks
 * stay zero; a NaN anywhere makes d NaN. */
int orc_quantize_q8_k(const float* x, void* y, int64_t n) {
  if (n < 0 || n % QK_K) return -1;
  for (int64_t b = 0; b < n / QK_K; ++b, x += QK_K) {
    q8_k_t blk;
    memset(&blk, 0, sizeof blk);
    float max = 0.f, amax = 0.f;
    int has_nan = 0;
    for (int j = 0; j < QK_K; ++j) {
      const float ax = fabsf(x[j]);
      if (ax > amax) {
        amax = ax;
        max = x[j];
      }
      has_nan |= isnan(x[j]);
    }
    if (amax != 0.f) {
      const float iscale = -127.f / max;
      for (int j = 0; j < QK_K; ++j) {
        const float v = iscale * x[j];
        blk.qs[j] = (int8_t)(v != v ? 0 : nearest_int(fminf(127.f, fmaxf(-127.f, v))));
      }
      for (int g = 0; g < 16; ++g) {
        int sum = 0;
        for (int i = 0; i < 16; ++i) sum += blk.qs[g * 16 + i];
        blk.bsums[g] = (int16_t)sum;
      }
      blk.d = 1 / iscale;
    }
    if (has_nan) blk.d = NAN;
    memcpy((uint8_t*)y + b * sizeof blk, &blk, sizeof blk);
  }
  return 0;
}

/* quant.cpp:52-61 (ggml get_scale_min_k4) */
static void scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* quant.cpp:66-96: a super-block's 256 quants as integers in element order. */
static void expand_q4_k(const q4_k_t* b, int8_t a[256]) {
  for (int c = 0; c < 4; ++c)
    for (int l = 0; l < 32; ++l) {
      a[64 * c + l] = (int8_t)(b->qs[32 * c + l] & 0xF);
      a[64 * c + 32 + l] = (int8_t)(b->qs[32 * c + l] >> 4);
    }
}
static void expand_q5_k(const q5_k_t* b, int8_t a[256]) {
  for (int c = 0; c < 4; ++c)
    for (int l = 0; l < 32; ++l) {
      a[64 * c + l] = (int8_t)((b->qs[32 * c + l] & 0xF) + ((b->qh[l] & (1 << (2 * c))) ? 16 : 0));
      a[64 * c + 32 + l] = (int8_t)((b->qs[32 * c + l] >> 4) + ((b->qh[l] & (2 << (2 * c))) ? 16 : 0));
    }
}
static void expand_q6_k(const q6_k_t* b, int8_t a[256]) {
  for (int h = 0; h < 2; ++h)
    for (int l = 0; l < 32; ++l) {
      const uint8_t* ql = b->ql + 64 * h;
      const uint8_t qh = b->qh[32 * h + l];
      a[128 * h + l] = (int8_t)(((ql[l] & 0xF) | (((qh >> 0) & 3) << 4)) - 32);
      a[128 * h + 32 + l] = (int8_t)(((ql[32 + l] & 0xF) | (((qh >> 2) & 3) << 4)) - 32);
      a[128 * h + 64 + l] = (int8_t)(((ql[l] >> 4) | (((qh >> 4) & 3) << 4)) - 32);
      a[128 * h + 96 + l] = (int8_t)(((ql[32 + l] >> 4) | (((qh >> 6) & 3) << 4)) - 32);
    }
}

/* quant.cpp:157-242 (dequantize_row) for the quantized types; F32 / F16 as copies / exact widening. */
int orc_dequantize(int type, const void* src, float* dst, int64_t n) {
  const uint8_t* p = (const uint8_t*)src;
  const int64_t be = orc_block_elems(type), bb = orc_block_bytes(type);
  if (be < 0 || n < 0 || n % be) return -1;
  for (int64_t b = 0; b < n / be; ++b) {
    const uint8_t* q = p + b * bb;
    float* o = dst + b * be;
    switch (type) {
      case T_F32: memcpy(o, q, 4); break;
      case T_F16: {
        uint16_t h;
        memcpy(&h, q, 2);
        o[0] = h2f(h);
        break;
      }
      case T_Q4_0: {
        q4_0_t k;
        memcpy(&k, q, sizeof k);
        const float d = h2f(k.d);
        for (int j = 0; j < 16; ++j) {
          o[j] = (float)((k.qs[j] & 0x0F) - 8) * d;
          o[j + 16] = (float)((k.qs[j] >> 4) - 8) * d;
        }
        break;
      }
      case T_Q8_0: {
        q8_0_t k;
        memcpy(&k, q, sizeof k);
        const float d = h2f(k.d);
        for (int j = 0; j < 32; ++j) o[j] = (float)k.qs[j] * d;
        break;
      }
      case T_Q5_0:
      case T_Q5_1: {
        uint16_t dh, mh = 0;
        uint32_t qh;
        const uint8_t* qs;
        if (type == T_Q5_0) {
          q5_0_t k;
          memcpy(&k, q, sizeof k);
          dh = k.d;
          memcpy(&qh, k.qh, 4);
          qs = q + 6;
        } else {
          q5_1_t k;
          memcpy(&k, q, sizeof k);
          dh = k.d;
          mh = k.m;
          memcpy(&qh, k.qh, 4);
          qs = q + 8;
        }
        const float d = h2f(dh), m = h2f(mh);
        for (int j = 0; j < 16; ++j) {
          const int x0 = (qs[j] & 0x0F) | (int)(((qh >> j) << 4) & 0x10);
          const int x1 = (qs[j] >> 4) | (int)((qh >> (j + 12)) & 0x10);
          if (type == T_Q5_0) {
            o[j] = (float)(x0 - 16) * d;
            o[j + 16] = (float)(x1 - 16) * d;
          } else {
            o[j] = (float)x0 * d + m;
            o[j + 16] = (float)x1 * d + m;
          }
        }
        break;
      }
      case T_Q4_K:
      case T_Q5_K: {
        int8_t a[256];
        uint16_t dh, mh;
        const uint8_t* sc;
        q4_k_t k4;
        q5_k_t k5;
        if (type == T_Q4_K) {
          memcpy(&k4, q, sizeof k4);
          expand_q4_k(&k4, a);
          dh = k4.d, mh = k4.dmin, sc = k4.scales;
        } else {
          memcpy(&k5, q, sizeof k5);
          expand_q5_k(&k5, a);
          dh = k5.d, mh = k5.dmin, sc = k5.scales;
        }
        const float d = h2f(dh), mn = h2f(mh);
        for (int j = 0; j < 8; ++j) { /* x = (d * sc) * q - (dmin * m), quant.cpp:102-116 */
          uint8_t s, m;
          scale_min_k4(j, sc, &s, &m);
          const float d1 = d * s, m1 = mn * m;
          for (int l = 0; l < 32; ++l) o[32 * j + l] = d1 * (float)a[32 * j + l] - m1;
        }
        break;
      }
      case T_Q6_K: {
        q6_k_t k;
        memcpy(&k, q, sizeof k);
        int8_t a[256];
        expand_q6_k(&k, a);
        const float d = h2f(k.d);
        for (int j = 0; j < 16; ++j) {
          const float dk = d * (float)k.scales[j];
          for (int l = 0; l < 16; ++l) o[16 * j + l] = dk * (float)a[16 * j + l];
        }
        break;
      }
      default: return -1;
    }
  }
  return 0;
}

/* ---- block dot products (quant.cpp:305-419), each in ggml's generic evaluation order ---- */

static float dot_q4_0(const uint8_t* w, const uint8_t* a, int64_t nb) { /* ((float)isum * d_w) * d_a */
  float sum = 0.f;
  for (int64_t b = 0; b < nb; ++b) {
    q4_0_t bw;
    q8_0_t ba;
    memcpy(&bw, w + b * sizeof bw, sizeof bw);
    memcpy(&ba, a + b * sizeof ba, sizeof ba);
    int s0 = 0, s1 = 0;
    for (int j = 0; j < 16; ++j) {
      s0 += ((bw.qs[j] & 0x0F) - 8) * ba.qs[j];
      s1 += ((bw.qs[j] >> 4) - 8) * ba.qs[j + 16];
    }
    sum += (float)(s0 + s1) * h2f(bw.d) * h2f(ba.d);
  }
  return sum;
}

static float dot_q8_0(const uint8_t* w, const uint8_t* a, int64_t nb) { /* (float)isum * (d_w * d_a) */
  float sum = 0.f;
  for (int64_t b = 0; b < nb; ++b) {
    q8_0_t bw, ba;
    memcpy(&bw, w + b * sizeof bw, sizeof bw);
    memcpy(&ba, a + b * sizeof ba, sizeof ba);
    int s = 0;
    for (int j = 0; j < 32; ++j) s += bw.qs[j] * ba.qs[j];
    sum += (float)s * (h2f(bw.d) * h2f(ba.d));
  }
  return sum;
}

static float dot_q5(int type, const uint8_t* w, const uint8_t* a, int64_t nb) {
  float sum = 0.f;
  const int64_t wb = type == T_Q5_0 ? 22 : 24, ab = type == T_Q5_0 ? 34 : 36;
  for (int64_t b = 0; b < nb; ++b) {
    const uint8_t* pw = w + b * wb;
    const uint8_t* pa = a + b * ab;
    uint16_t dw, mw = 0, da, sa = 0;
    uint32_t qh;
    memcpy(&dw, pw, 2);
    if (type == T_Q5_1) memcpy(&mw, pw + 2, 2);
    const uint8_t* qhp = pw + (type == T_Q5_0 ? 2 : 4);
    memcpy(&qh, qhp, 4);
    const uint8_t* qs = qhp + 4;
    memcpy(&da, pa, 2);
    if (type == T_Q5_1) memcpy(&sa, pa + 2, 2);
    const int8_t* aq = (const int8_t*)(pa + (type == T_Q5_0 ? 2 : 4));
    const int bias = type == T_Q5_0 ? 16 : 0;
    int s0 = 0, s1 = 0;
    for (int j = 0; j < 16; ++j) {
      s0 += (((qs[j] & 0x0F) | (int)(((qh >> j) << 4) & 0x10)) - bias) * aq[j];
      s1 += (((qs[j] >> 4) | (int)((qh >> (j + 12)) & 0x10)) - bias) * aq[j + 16];
    }
    if (type == T_Q5_0)
      sum += (h2f(dw) * h2f(da)) * (float)(s0 + s1);
    else
      sum += (h2f(dw) * h2f(da)) * (float)(s0 + s1) + h2f(mw) * h2f(sa); /* block term first */
  }
  return sum;
}

/* quant.cpp:118-144 (dot_k45): eight int32 lanes (element e feeds lane e % 8), one float partial per lane,
 * the min term subtracted into sumf per block, the lane partials added to sumf last. */
static float dot_k45(int type, const uint8_t* w, const uint8_t* a, int64_t nb) {
  float sums[8] = {0};
  float sumf = 0;
  const int64_t wb = type == T_Q4_K ? 144 : 176;
  for (int64_t b = 0; b < nb; ++b) {
    int8_t q[256];
    uint16_t dh, mh;
    uint8_t scales[12];
    if (type == T_Q4_K) {
      q4_k_t k;
      memcpy(&k, w + b * wb, sizeof k);
      expand_q4_k(&k, q);
      dh = k.d, mh = k.dmin;
      memcpy(scales, k.scales, 12);
    } else {
      q5_k_t k;
      memcpy(&k, w + b * wb, sizeof k);
      expand_q5_k(&k, q);
      dh = k.d, mh = k.dmin;
      memcpy(scales, k.scales, 12);
    }
    q8_k_t ba;
    memcpy(&ba, a + b * sizeof ba, sizeof ba);
    int32_t aux32[8] = {0};
    int sumi = 0;
    for (int k = 0; k < 8; ++k) {
      uint8_t sc, m;
      scale_min_k4(k, scales, &sc, &m);
      sumi += (ba.bsums[2 * k] + ba.bsums[2 * k + 1]) * m;
      for (int e = 0; e < 32; ++e) aux32[e & 7] += sc * (ba.qs[32 * k + e] * q[32 * k + e]);
    }
    const float d = h2f(dh) * ba.d;
    for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
    const float dmin = h2f(mh) * ba.d;
    sumf -= dmin * (float)sumi;
  }
  for (int l = 0; l < 8; ++l) sumf += sums[l];
  return sumf;
}

/* quant.cpp:394-419 */
static float dot_q6_k(const uint8_t* w, const uint8_t* a, int64_t nb) {
  float sums[8] = {0};
  for (int64_t b = 0; b < nb; ++b) {
    q6_k_t bw;
    q8_k_t ba;
    memcpy(&bw, w + b * sizeof bw, sizeof bw);
    memcpy(&ba, a + b * sizeof ba, sizeof ba);
    int8_t q[256];
    expand_q6_k(&bw, q);
    int32_t aux32[8] = {0};
    for (int e = 0; e < 256; ++e) aux32[e & 7] += bw.scales[e / 16] * (ba.qs[e] * q[e]);
    const float d = h2f(bw.d) * ba.d;
    for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
  }
  float sumf = 0;
  for (int l = 0; l < 8; ++l) sumf += sums[l];
  return sumf;
}

/* The block dot of weight type `type` against its activation type's blocks (quant.h's vec_dot_type table:
 * Q4_0 / Q5_0 / Q8_0 with Q8_0, Q5_1 with Q8_1, the K types with Q8_K). */
float orc_dot(int type, const void* w, const void* a, int64_t n_blocks) {
  const uint8_t* pw = (const uint8_t*)w;
  const uint8_t* pa = (const uint8_t*)a;
  switch (type) {
    case T_Q4_0: return dot_q4_0(pw, pa, n_blocks);
    case T_Q8_0: return dot_q8_0(pw, pa, n_blocks);
    case T_Q5_0:
    case T_Q5_1: return dot_q5(type, pw, pa, n_blocks);
    case T_Q4_K:
    case T_Q5_K: return dot_k45(type, pw, pa, n_blocks);
    case T_Q6_K: return dot_q6_k(pw, pa, n_blocks);
    default: return NAN;
  }
}

int orc_act_kind(int type) { /* 0 = Q8_0, 1 = Q8_1, 2 = Q8_K, -1 = none */
  switch (type) {
    case T_Q4_0:
    case T_Q5_0:
    case T_Q8_0: return 0;
    case T_Q5_1: return 1;
    case T_Q4_K:
    case T_Q5_K:
    case T_Q6_K: return 2;
    default: return -1;
  }
}

/* ref_ops.cpp:109-135 for quantized weights: each activation row quantized to the weight's activation type, then
 * y[t * out + r] = block dot of weight row r with activation row t. */
int orc_matmul_q(int type, const void* w, int64_t in, int64_t out, const float* x, float* y, int64_t n) {
  const int kind = orc_act_kind(type);
  const int64_t be = orc_block_elems(type), bb = orc_block_bytes(type);
  if (kind < 0 || in % be) return -1;
  const int64_t nb = in / be;
  const int64_t ab = kind == 0 ? 34 : kind == 1 ? 36 : 292;
  uint8_t* acts = (uint8_t*)malloc((size_t)(n * nb * ab));
  if (!acts) return -1;
  for (int64_t t = 0; t < n; ++t) {
    uint8_t* at = acts + t * nb * ab;
    if (kind == 0) orc_quantize_q8_0(x + t * in, at, in);
    else if (kind == 1) orc_quantize_q8_1(x + t * in, at, in);
    else orc_quantize_q8_k(x + t * in, at, in);
  }
  for (int64_t t = 0; t < n; ++t)
    for (int64_t r = 0; r < out; ++r)
      y[t * out + r] = orc_dot(type, (const uint8_t*)w + r * nb * bb, acts + t * nb * ab, nb);
  free(acts);
  return 0;
}
