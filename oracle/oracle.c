/*
 * CPU oracle for nibble's attention path: scalar kernels, fp64 brute force, Llama-3 factors and the
 * head-parallel driver. TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP backend, never the
 * product path. Built with -ffp-contract=off, mirroring the reference's flags for ref_ops.cpp
 * (CMakeLists.txt:72-73), so every float multiply and add rounds on its own as in the reference.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ref_ops.cpp:166-185. The angle is pos * base^(-2i/hd) in double (divided by the optional per-pair factor,
 * promoted to double), cos/sin are rounded to float, and the rotation is four float products and two float
 * sums with no fused multiply-add. */
void orc_rope(float* x, int64_t n, int64_t n_heads, int64_t head_dim, int64_t pos0, float freq_base, int neox,
              const float* freq_factors) {
  const int64_t half = head_dim / 2;
  for (int64_t t = 0; t < n; ++t) {
    const double pos = (double)(pos0 + t);
    for (int64_t h = 0; h < n_heads; ++h) {
      float* row = x + (t * n_heads + h) * head_dim;
      for (int64_t i = 0; i < half; ++i) {
        double theta = pos * pow((double)freq_base, -2.0 * (double)i / (double)head_dim);
        if (freq_factors) theta /= (double)freq_factors[i];
        const float c = (float)cos(theta), s = (float)sin(theta);
        float* a = neox ? &row[i] : &row[2 * i];
        float* b = neox ? &row[i + half] : &row[2 * i + 1];
        const float a0 = *a, b0 = *b;
        *a = a0 * c - b0 * s;
        *b = a0 * s + b0 * c;
      }
    }
  }
}

/* ref_ops.cpp:66-77. std::max(m, x) keeps m unless m < x. */
void orc_softmax_inplace(float* x, int64_t n) {
  if (n <= 0) return;
  float m = x[0];
  for (int64_t i = 1; i < n; ++i) m = (m < x[i]) ? x[i] : m;
  double sum = 0;
  for (int64_t i = 0; i < n; ++i) {
    x[i] = expf(x[i] - m);
    sum += x[i];
  }
  const float inv = (float)(1.0 / sum);
  for (int64_t i = 0; i < n; ++i) x[i] *= inv;
}

/* ref_ops.cpp:188-214. Query head h reads K/V head h / (n_heads / n_kv_heads); row t attends to cache rows
 * 0..pos0+t; scores are float dots scaled by the float 1/sqrt(head_dim). */
void orc_attention_scalar(const float* q, const float* k, const float* v, float* out, int64_t n, int64_t pos0,
                          int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int64_t head_begin,
                          int64_t head_end, float* scratch) {
  const int64_t group = n_heads / n_kv_heads;
  const float scale = 1.0f / sqrtf((float)head_dim);
  for (int64_t h = head_begin; h < head_end; ++h) {
    const int64_t kvh = h / group;
    for (int64_t t = 0; t < n; ++t) {
      const float* qh = q + (t * n_heads + h) * head_dim;
      const int64_t len = pos0 + t + 1;
      for (int64_t j = 0; j < len; ++j) {
        const float* kj = k + (j * n_kv_heads + kvh) * head_dim;
        float dot = 0;
        for (int64_t d = 0; d < head_dim; ++d) dot += qh[d] * kj[d];
        scratch[j] = dot * scale;
      }
      orc_softmax_inplace(scratch, len);
      float* o = out + (t * n_heads + h) * head_dim;
      for (int64_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
      for (int64_t j = 0; j < len; ++j) {
        const float* vj = v + (j * n_kv_heads + kvh) * head_dim;
        const float pj = scratch[j];
        for (int64_t d = 0; d < head_dim; ++d) o[d] += pj * vj[d];
      }
    }
  }
}

/* fp64 brute force over the same fp32 inputs: scores, max-subtracted exp and the weighted sum all in double
 * (tests/naive_llama.h:118-134 computes attention the same way). */
void orc_attention_f64(const float* q, const float* k, const float* v, double* out, int64_t n, int64_t pos0,
                       int64_t n_heads, int64_t n_kv_heads, int64_t head_dim) {
  const int64_t group = n_heads / n_kv_heads, ctx = pos0 + n;
  double* sc = (double*)malloc((size_t)(ctx > 0 ? ctx : 1) * sizeof(double));
  if (!sc) abort();
  const double inv_sqrt = 1.0 / sqrt((double)head_dim);
  for (int64_t t = 0; t < n; ++t) {
    const int64_t len = pos0 + t + 1;
    for (int64_t h = 0; h < n_heads; ++h) {
      const int64_t kvh = h / group;
      const float* qh = q + (t * n_heads + h) * head_dim;
      double mx = -INFINITY;
      for (int64_t j = 0; j < len; ++j) {
        const float* kj = k + (j * n_kv_heads + kvh) * head_dim;
        double d = 0;
        for (int64_t i = 0; i < head_dim; ++i) d += (double)qh[i] * (double)kj[i];
        sc[j] = d * inv_sqrt;
        if (sc[j] > mx) mx = sc[j];
      }
      double sum = 0;
      for (int64_t j = 0; j < len; ++j) sum += (sc[j] = exp(sc[j] - mx));
      double* o = out + (t * n_heads + h) * head_dim;
      for (int64_t i = 0; i < head_dim; ++i) o[i] = 0;
      for (int64_t j = 0; j < len; ++j) {
        const float* vj = v + (j * n_kv_heads + kvh) * head_dim;
        const double p = sc[j] / sum;
        for (int64_t i = 0; i < head_dim; ++i) o[i] += p * (double)vj[i];
      }
    }
  }
  free(sc);
}

void orc_llama3_freq_factors(float* out, int64_t head_dim, double base, double factor, double low_freq_factor,
                             double high_freq_factor, double orig_ctx) {
  const double low_wavelen = orig_ctx / low_freq_factor, high_wavelen = orig_ctx / high_freq_factor;
  for (int64_t i = 0; i < head_dim / 2; ++i) {
    const double freq = pow(base, -2.0 * (double)i / (double)head_dim);
    const double wavelen = 2.0 * M_PI / freq;
    double f;
    if (wavelen < high_wavelen) {
      f = 1.0;
    } else if (wavelen > low_wavelen) {
      f = factor;
    } else {
      const double s = (orig_ctx / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor);
      f = 1.0 / ((1.0 - s) / factor + s);
    }
    out[i] = (float)f;
  }
}

/* ---- head-parallel driver (cpu_backend.cpp:271-290 over thread_pool.cpp:114-137) ---- */

typedef struct {
  const float *q, *k, *v;
  float* out;
  int64_t n, pos0, n_heads, n_kv_heads, head_dim;
  int use_avx2;
  float* scratch;
  atomic_llong next; /* the shared chunk cursor (thread_pool.cpp:136-138) */
} HeadJob;

static void run_heads(HeadJob* j) {
  const int64_t ctx = j->pos0 + j->n;
  for (;;) {
    const int64_t h = atomic_fetch_add_explicit(&j->next, 1, memory_order_relaxed);
    if (h >= j->n_heads) break;
    if (j->use_avx2)
      orc_attention_avx2(j->q, j->k, j->v, j->out, j->n, j->pos0, j->n_heads, j->n_kv_heads, j->head_dim, h, h + 1,
                         j->scratch + h * ctx);
    else
      orc_attention_scalar(j->q, j->k, j->v, j->out, j->n, j->pos0, j->n_heads, j->n_kv_heads, j->head_dim, h,
                           h + 1, j->scratch + h * ctx);
  }
}

static void* worker(void* arg) {
  run_heads((HeadJob*)arg);
  return NULL;
}

int orc_attention_heads_parallel(const float* q, const float* k, const float* v, float* out, int64_t n,
                                 int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, int threads,
                                 int use_avx2, float* scratch) {
  if (use_avx2 && !orc_have_avx2()) return -1;
  HeadJob job = {q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim, use_avx2, scratch, 0};
  if (threads < 1) threads = 1;
  pthread_t* tids = threads > 1 ? (pthread_t*)malloc(sizeof(pthread_t) * (size_t)(threads - 1)) : NULL;
  int started = 0;
  for (int i = 0; i + 1 < threads; ++i)
    if (pthread_create(&tids[started], NULL, worker, &job) == 0) ++started;
  run_heads(&job); /* the caller is worker 0, as in ThreadPool::parallel_for */
  for (int i = 0; i < started; ++i) pthread_join(tids[i], NULL);
  free(tids);
  return 0;
}

/* ---- float matmul and bias (the Transformer's QKV projection into the cache, transformer.cpp:171-194) ---- */

float orc_fp16_to_fp32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  union {
    uint32_t u;
    float f;
  } r;
  if (e == 0x1Fu) {
    r.u = sign | 0x7F800000u | (m << 13); /* inf, NaN (payload kept) */
  } else if (e != 0) {
    r.u = sign | ((e + 112u) << 23) | (m << 13); /* rebias 15 -> 127 */
  } else {
    r.f = (float)m * 0x1p-24f; /* zero and subnormals: m * 2^-24, exact */
    r.u |= sign;
  }
  return r.f;
}

void orc_fp16_to_fp32_n(const uint16_t* h, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = orc_fp16_to_fp32(h[i]);
}

int orc_matmul(int w_type, const void* w, int64_t in, int64_t out, const float* x, float* y, int64_t n) {
  if (w_type != 0 && w_type != 1) return -1;
  for (int64_t t = 0; t < n; ++t) {
    const float* xt = x + t * in;
    for (int64_t r = 0; r < out; ++r) {
      float acc = 0.0f;
      if (w_type == 0) {
        const float* wr = (const float*)w + r * in;
        for (int64_t k = 0; k < in; ++k) acc += xt[k] * wr[k];
      } else {
        const uint16_t* wr = (const uint16_t*)w + r * in;
        for (int64_t k = 0; k < in; ++k) acc += xt[k] * orc_fp16_to_fp32(wr[k]);
      }
      y[t * out + r] = acc;
    }
  }
  return 0;
}

void orc_add_bias(float* x, const float* b, int64_t d, int64_t n) {
  for (int64_t t = 0; t < n; ++t)
    for (int64_t i = 0; i < d; ++i) x[t * d + i] += b[i];
}

/* ---- the other per-token ops of the forward (transformer.cpp:166-230) ---- */

int orc_embed(int type, const void* table, int64_t rows, int64_t d, const int32_t* ids, int64_t n, float* out) {
  if (type != 0 && type != 1) return -1;
  for (int64_t t = 0; t < n; ++t) {
    const int64_t id = ids[t];
    if (id < 0 || id >= rows) return -1;
    float* o = out + t * d;
    if (type == 0) {
      const float* r = (const float*)table + id * d;
      for (int64_t k = 0; k < d; ++k) o[k] = r[k];
    } else {
      const uint16_t* r = (const uint16_t*)table + id * d;
      for (int64_t k = 0; k < d; ++k) o[k] = orc_fp16_to_fp32(r[k]);
    }
  }
  return 0;
}

void orc_rmsnorm(const float* x, const float* w, float* y, int64_t n, int64_t d, float eps) {
  for (int64_t t = 0; t < n; ++t) {
    const float* xt = x + t * d;
    double ss = 0.0;
    for (int64_t i = 0; i < d; ++i) ss += (double)xt[i] * (double)xt[i];
    const double scale = 1.0 / sqrt(ss / (double)d + (double)eps);
    for (int64_t i = 0; i < d; ++i) y[t * d + i] = (float)((double)xt[i] * scale * (double)w[i]);
  }
}

void orc_add(float* x, const float* y, int64_t count) {
  for (int64_t i = 0; i < count; ++i) x[i] += y[i];
}

void orc_silu_mul(float* gate, const float* up, int64_t count) {
  for (int64_t i = 0; i < count; ++i) {
    const float g = gate[i];
    gate[i] = g / (1.0f + expf(-g)) * up[i];
  }
}
