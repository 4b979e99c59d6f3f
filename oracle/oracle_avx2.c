/*
 * AVX2 restatement of nibble's production CPU attention tier. TEST INFRASTRUCTURE ONLY (see oracle.h).
 * Built with -mavx2 -mfma -mf16c -ffp-contract=off like the reference's tier sources (CMakeLists.txt:83-95),
 * so the scalar tails round exactly as the reference's do.
 */
#include <math.h>
#include <stdint.h>

#include "oracle.h"

#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>

/* simd.h:37-42: fold the high 128 bits onto the low, then the high pair, then lane 1 onto lane 0. */
static inline float hsum8(__m256 v) {
  __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
  return _mm_cvtss_f32(s);
}

/* simd.h:103-126: clamp to [-104, 89], n = round(x*log2e), r = x - n*ln2 in two exact-product steps
 * (ln2_hi = 0.693359375, ln2_lo = -2.12194440e-4), e^r - 1 by a degree-7 Taylor polynomial in Horner form,
 * then (t*2^m + 2^m) * 2^(n-m) with m = min(n, 127) and 2^m built as a normal or subnormal bit pattern. */
static inline __m256 exp8(__m256 x) {
  x = _mm256_max_ps(_mm256_set1_ps(-104.0f), _mm256_min_ps(_mm256_set1_ps(89.0f), x));
  const __m256 fn =
      _mm256_round_ps(_mm256_mul_ps(x, _mm256_set1_ps(1.44269504f)), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  __m256 r = _mm256_fnmadd_ps(fn, _mm256_set1_ps(0.693359375f), x);
  r = _mm256_fnmadd_ps(fn, _mm256_set1_ps(-2.12194440e-4f), r);
  static const float taylor[6] = {1.0f / 720, 1.0f / 120, 1.0f / 24, 1.0f / 6, 0.5f, 1.0f};
  __m256 poly = _mm256_set1_ps(1.0f / 5040);
  for (int i = 0; i < 6; ++i) poly = _mm256_fmadd_ps(poly, r, _mm256_set1_ps(taylor[i]));
  const __m256 em1 = _mm256_mul_ps(poly, r);
  const __m256i ni = _mm256_cvtps_epi32(fn);
  const __m256i nc = _mm256_min_epi32(ni, _mm256_set1_epi32(127));
  const __m256i normal_bits = _mm256_slli_epi32(_mm256_add_epi32(nc, _mm256_set1_epi32(127)), 23);
  const __m256i subnormal_bits = _mm256_sllv_epi32(_mm256_set1_epi32(1), _mm256_add_epi32(nc, _mm256_set1_epi32(149)));
  const __m256 scale1 = _mm256_castsi256_ps(
      _mm256_blendv_epi8(subnormal_bits, normal_bits, _mm256_cmpgt_epi32(nc, _mm256_set1_epi32(-127))));
  const __m256 scale2 = _mm256_castsi256_ps(
      _mm256_slli_epi32(_mm256_add_epi32(_mm256_sub_epi32(ni, nc), _mm256_set1_epi32(127)), 23));
  return _mm256_mul_ps(_mm256_fmadd_ps(em1, scale1, scale1), scale2);
}

/* simd/ops.cpp:31-51: x[i] = e^(x[i]-m) eight at a time; the ragged tail goes through one vector padded with
 * -inf; returns hsum of the lane accumulator. */
static float exp_sub_sum(float* x, int64_t len, float m) {
  const __m256 mv = _mm256_set1_ps(m);
  __m256 acc = _mm256_setzero_ps();
  int64_t j = 0;
  for (; j + 8 <= len; j += 8) {
    const __m256 e = exp8(_mm256_sub_ps(_mm256_loadu_ps(x + j), mv));
    _mm256_storeu_ps(x + j, e);
    acc = _mm256_add_ps(acc, e);
  }
  if (j < len) {
    float pad[8] __attribute__((aligned(32)));
    for (int i = 0; i < 8; ++i) pad[i] = j + i < len ? x[j + i] : -INFINITY;
    const __m256 e = exp8(_mm256_sub_ps(_mm256_load_ps(pad), mv));
    _mm256_store_ps(pad, e);
    for (int64_t i = 0; j + i < len; ++i) x[j + i] = pad[i];
    acc = _mm256_add_ps(acc, e);
  }
  return hsum8(acc);
}

int orc_have_avx2(void) {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c");
}

int orc_exp_ps(const float* x, float* y, int64_t n) {
  if (!orc_have_avx2()) return -1;
  int64_t i = 0;
  for (; i + 8 <= n; i += 8) _mm256_storeu_ps(y + i, exp8(_mm256_loadu_ps(x + i)));
  if (i < n) {
    float buf[8] = {0};
    for (int64_t j = 0; i + j < n; ++j) buf[j] = x[i + j];
    _mm256_storeu_ps(buf, exp8(_mm256_loadu_ps(buf)));
    for (int64_t j = 0; i + j < n; ++j) y[i + j] = buf[j];
  }
  return 0;
}

/* simd/ops.cpp:104-139: per key an 8-lane FMA dot over the multiple-of-8 part of head_dim, hsum8, then a
 * scalar tail; the running max is tracked in the score loop; probabilities are e^(s-m) * (1/sum) applied on the
 * fly; the output row accumulates p*v with FMA over the vector part and a scalar tail. */
int orc_attention_avx2(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                       int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t head_begin, int64_t head_end,
                       float* scratch) {
  if (!orc_have_avx2()) return -1;
  const int64_t group = n_heads / n_kv_heads, vec = head_dim & ~(int64_t)7;
  const float scale = 1.0f / sqrtf((float)head_dim);
  for (int64_t h = head_begin; h < head_end; ++h) {
    const int64_t kvh = h / group;
    for (int64_t t = 0; t < n; ++t) {
      const float* qh = q + (t * n_heads + h) * head_dim;
      const int64_t len = pos0 + t + 1;
      float m = -INFINITY;
      for (int64_t j = 0; j < len; ++j) {
        const float* kj = k + (j * n_kv_heads + kvh) * head_dim;
        __m256 acc = _mm256_setzero_ps();
        int64_t d = 0;
        for (; d < vec; d += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(qh + d), _mm256_loadu_ps(kj + d), acc);
        float dot = hsum8(acc);
        for (; d < head_dim; ++d) dot += qh[d] * kj[d];
        scratch[j] = dot * scale;
        m = (m < scratch[j]) ? scratch[j] : m;
      }
      const float inv = 1.0f / exp_sub_sum(scratch, len, m);
      float* o = out + (t * n_heads + h) * head_dim;
      for (int64_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
      for (int64_t j = 0; j < len; ++j) {
        const float* vj = v + (j * n_kv_heads + kvh) * head_dim;
        const float pj = scratch[j] * inv;
        const __m256 p = _mm256_set1_ps(pj);
        int64_t d = 0;
        for (; d < vec; d += 8)
          _mm256_storeu_ps(o + d, _mm256_fmadd_ps(p, _mm256_loadu_ps(vj + d), _mm256_loadu_ps(o + d)));
        for (; d < head_dim; ++d) o[d] += pj * vj[d];
      }
    }
  }
  return 0;
}

#else /* no AVX2 in this build: report it, compute nothing */

int orc_have_avx2(void) { return 0; }
int orc_exp_ps(const float* x, float* y, int64_t n) {
  (void)x, (void)y, (void)n;
  return -1;
}
int orc_attention_avx2(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                       int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t head_begin, int64_t head_end,
                       float* scratch) {
  (void)q, (void)k, (void)v, (void)out, (void)n, (void)pos0, (void)n_heads, (void)n_kv_heads, (void)head_dim;
  (void)head_begin, (void)head_end, (void)scratch;
  return -1;
}

#endif
