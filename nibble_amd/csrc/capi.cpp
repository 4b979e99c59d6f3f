// The C ABI of include/nibble_hip.h over nibble::hip::HipBackend: exceptions become NBH_E_* codes plus a
// thread-local message.
#include <exception>
#include <new>
#include <string>
#include <vector>

#include "backend/hip/hip_backend.h"
#include "nibble_hip.h"

using nibble::RopeParams;
using nibble::hip::HipBackend;

struct nbh_backend {
  HipBackend impl;
  explicit nbh_backend(int device) : impl(device) {}
};

struct nbh_event {
  nbhs_event ev = nullptr;
};

namespace {

thread_local std::string g_last_error;

template <class F>
int guarded(F&& f) {
  try {
    f();
    g_last_error.clear();
    return NBH_OK;
  } catch (const nibble::Error& e) {
    g_last_error = e.what();
    return NBH_E_INPUT;
  } catch (const std::bad_alloc&) {
    g_last_error = "out of host memory";
    return NBH_E_INPUT;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return NBH_E_INTERNAL;
  } catch (...) {
    g_last_error = "unknown exception";
    return NBH_E_INTERNAL;
  }
}

nibble::Tensor tensor_of(const nbh_tensor* t) {
  if (!t) throw nibble::Error("null tensor");
  nibble::Tensor r;
  r.type = static_cast<nibble::DType>(t->type);
  r.n_dims = t->n_dims;
  for (int i = 0; i < 4; ++i) r.ne[size_t(i)] = t->ne[i];
  r.data = t->data;
  return r;
}

HipBackend& B(nbh_backend* be) {
  if (!be) throw nibble::Error("null backend handle");
  return be->impl;
}
const HipBackend& B(const nbh_backend* be) {
  if (!be) throw nibble::Error("null backend handle");
  return be->impl;
}

}  // namespace

extern "C" {

const char* nbh_last_error(void) { return g_last_error.c_str(); }

int nbh_backend_create(int device, nbh_backend** out) {
  return guarded([&] {
    if (!out) throw nibble::Error("null output handle");
    *out = nullptr;
    *out = new nbh_backend(device);
  });
}

void nbh_backend_destroy(nbh_backend* be) { delete be; }

int nbh_backend_supports(const nbh_backend* be, uint32_t dtype, int* out) {
  return guarded([&] { *out = B(be).supports(static_cast<nibble::DType>(dtype)) ? 1 : 0; });
}

int nbh_backend_reserve(nbh_backend* be, int64_t n_ctx, int64_t n_heads, int64_t max_rows, int64_t max_width) {
  return guarded([&] { B(be).reserve({n_ctx, n_heads, max_rows, max_width}); });
}

int nbh_backend_alloc(nbh_backend* be, int64_t n_floats, float** out) {
  return guarded([&] {
    if (!out) throw nibble::Error("alloc: null output pointer");
    *out = B(be).alloc(n_floats);
  });
}

int nbh_backend_free(nbh_backend* be, float* p) {
  return guarded([&] { B(be).free(p); });
}

int nbh_backend_read(nbh_backend* be, float* host_dst, const float* src, int64_t n) {
  return guarded([&] { B(be).read(host_dst, src, n); });
}

int nbh_backend_write(nbh_backend* be, float* dst, const float* host_src, int64_t n) {
  return guarded([&] { B(be).write(dst, host_src, n); });
}

int nbh_backend_copy(nbh_backend* be, float* dst, const float* src, int64_t count) {
  return guarded([&] { B(be).copy(dst, src, count); });
}

int nbh_backend_rope(nbh_backend* be, float* x, int64_t n, int64_t n_heads, int64_t head_dim, int64_t pos0,
                     float freq_base, int neox, const float* freq_factors) {
  return guarded([&] { B(be).rope(x, n, n_heads, head_dim, pos0, RopeParams{freq_base, neox != 0, freq_factors}); });
}

int nbh_backend_matmul(nbh_backend* be, const nbh_tensor* w, const float* x, float* y, int64_t n) {
  return guarded([&] { B(be).matmul(tensor_of(w), x, y, n); });
}

int nbh_backend_matmul_multi(nbh_backend* be, int64_t n_w, const nbh_tensor* const* ws, const float* x,
                             float* const* ys, int64_t n) {
  return guarded([&] {
    if (n_w <= 0 || !ws || !ys) throw nibble::Error("matmul_multi: need n_w > 0 weights and outputs");
    // The views on the stack for up to kStack weights (a layer's QKV or gate + up: nothing allocated per call).
    constexpr int64_t kStack = 16;
    nibble::Tensor ts[kStack];
    const nibble::Tensor* tps[kStack];
    std::vector<nibble::Tensor> tv;
    std::vector<const nibble::Tensor*> tpv;
    const nibble::Tensor** tp = tps;
    if (n_w > kStack) {
      tv.resize(size_t(n_w));
      tpv.resize(size_t(n_w));
      tp = tpv.data();
    }
    for (int64_t i = 0; i < n_w; ++i) {
      nibble::Tensor& t = n_w > kStack ? tv[size_t(i)] : ts[i];
      t = tensor_of(ws[i]);
      tp[i] = &t;
    }
    B(be).matmul_multi(std::span<const nibble::Tensor* const>(tp, size_t(n_w)), x,
                       std::span<float* const>(ys, size_t(n_w)), n);
  });
}

int nbh_backend_add_bias(nbh_backend* be, float* x, const nbh_tensor* bias, int64_t n) {
  return guarded([&] { B(be).add_bias(x, tensor_of(bias), n); });
}

int nbh_backend_embed(nbh_backend* be, const nbh_tensor* table, const int32_t* ids, int64_t n_ids, float* out) {
  return guarded([&] {
    if (n_ids <= 0 || !ids) throw nibble::Error("embed: need n_ids > 0 host token ids");
    B(be).embed(tensor_of(table), std::span<const int32_t>(ids, size_t(n_ids)), out);
  });
}

int nbh_backend_rmsnorm(nbh_backend* be, const float* x, const nbh_tensor* weight, float* y, int64_t n, float eps) {
  return guarded([&] { B(be).rmsnorm(x, tensor_of(weight), y, n, eps); });
}

int nbh_backend_add(nbh_backend* be, float* x, const float* y, int64_t count) {
  return guarded([&] { B(be).add(x, y, count); });
}

int nbh_backend_silu_mul(nbh_backend* be, float* gate, const float* up, int64_t count) {
  return guarded([&] { B(be).silu_mul(gate, up, count); });
}

int nbh_backend_set_attention_fp32(nbh_backend* be, int on) {
  return guarded([&] { B(be).set_attention_fp32(on != 0); });
}

int nbh_backend_set_batch_invariant(nbh_backend* be, int on) {
  return guarded([&] { B(be).set_batch_invariant(on != 0); });
}

int nbh_attention_decode_noalloc(const float* q, const float* k, const float* v, float* out, int64_t n,
                                 int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, void* stream) {
  return guarded([&] {
    const int e = nbhs_attn_decode_noalloc(q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim,
                                           static_cast<nbhs_stream>(stream));
    if (e == NBHS_ETOOBIG)
      throw nibble::Error("attention_decode_noalloc: the call's split partials exceed the " +
                          std::to_string(nbhs_attn_decode_noalloc_capacity() * 4 >> 20) + " MiB static scratch");
    if (e == NBHS_EINVAL)
      throw nibble::Error("attention_decode_noalloc: invalid shape n=" + std::to_string(n) + " (1.." +
                          std::to_string(NBHS_DECODE_MAX_ROWS) + ") pos0=" + std::to_string(pos0) + " n_heads=" +
                          std::to_string(n_heads) + " n_kv_heads=" + std::to_string(n_kv_heads) + " head_dim=" +
                          std::to_string(head_dim) + " (or a null pointer)");
    if (e != 0) throw nibble::Error(std::string("attention_decode_noalloc: ") + nbhs_error_string(e));
  });
}

int nbh_backend_stream(nbh_backend* be, void** stream) {
  return guarded([&] {
    if (!stream) throw nibble::Error("stream: null output");
    *stream = B(be).stream();
  });
}

int nbh_backend_prefill_recomputed(nbh_backend* be, int64_t* tiles) {
  return guarded([&] {
    if (!tiles) throw nibble::Error("prefill_recomputed: null output");
    *tiles = B(be).prefill_recomputed();
  });
}

int nbh_backend_release_weights(nbh_backend* be) {
  return guarded([&] { B(be).release_weights(); });
}

int nbh_backend_attention(nbh_backend* be, const float* q, const float* k, const float* v, float* out, int64_t n,
                          int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim) {
  return guarded([&] { B(be).attention(q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim); });
}

int nbh_backend_append_rope(nbh_backend* be, float* q, float* k_cache, float* v_cache, const float* k_new,
                            const float* v_new, int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads,
                            int64_t head_dim, float freq_base, int neox, const float* freq_factors) {
  return guarded([&] {
    B(be).append_rope(q, k_cache, v_cache, k_new, v_new, n, pos0, n_heads, n_kv_heads, head_dim,
                      RopeParams{freq_base, neox != 0, freq_factors});
  });
}

int nbh_backend_append_rope_attention(nbh_backend* be, const float* q, float* k_cache, float* v_cache,
                                      const float* k_new, const float* v_new, float* out, int64_t n, int64_t pos0,
                                      int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, float freq_base, int neox,
                                      const float* freq_factors) {
  return guarded([&] {
    B(be).append_rope_attention(q, k_cache, v_cache, k_new, v_new, out, n, pos0, n_heads, n_kv_heads, head_dim,
                                RopeParams{freq_base, neox != 0, freq_factors});
  });
}

int nbh_backend_attention_f16kv(nbh_backend* be, const float* q, const void* k16, const void* v16, float* out,
                                int64_t n, int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim) {
  return guarded([&] { B(be).attention_f16kv(q, k16, v16, out, n, pos0, n_heads, n_kv_heads, head_dim); });
}

int nbh_backend_append_rope_attention_f16kv(nbh_backend* be, const float* q, void* k16, void* v16,
                                            const float* k_new, const float* v_new, float* out, int64_t n,
                                            int64_t pos0, int64_t n_heads, int64_t n_kv_heads, int64_t head_dim,
                                            float freq_base, int neox, const float* freq_factors) {
  return guarded([&] {
    B(be).append_rope_attention_f16kv(q, k16, v16, k_new, v_new, out, n, pos0, n_heads, n_kv_heads, head_dim,
                                      RopeParams{freq_base, neox != 0, freq_factors});
  });
}

int nbh_backend_attention_batch(nbh_backend* be, int64_t n_seq, const float* const* q, const float* const* k_cache,
                                const float* const* v_cache, float* const* out, const int64_t* pos0, int64_t n_heads,
                                int64_t n_kv_heads, int64_t head_dim) {
  return guarded([&] { B(be).attention_batch(n_seq, q, k_cache, v_cache, out, pos0, n_heads, n_kv_heads, head_dim); });
}

int nbh_backend_append_rope_attention_batch(nbh_backend* be, int64_t n_seq, const float* const* q,
                                            float* const* k_cache, float* const* v_cache, const float* const* k_new,
                                            const float* const* v_new, float* const* out, const int64_t* pos0,
                                            int64_t n_heads, int64_t n_kv_heads, int64_t head_dim, float freq_base,
                                            int neox, const float* freq_factors) {
  return guarded([&] {
    B(be).append_rope_attention_batch(n_seq, q, k_cache, v_cache, k_new, v_new, out, pos0, n_heads, n_kv_heads,
                                      head_dim, RopeParams{freq_base, neox != 0, freq_factors});
  });
}

int nbh_backend_reserve_attention(nbh_backend* be, int64_t n_kv_heads, int64_t head_dim) {
  return guarded([&] { B(be).reserve_attention(n_kv_heads, head_dim); });
}

int nbh_backend_reserve_rope(nbh_backend* be, int64_t head_dim, float freq_base, int neox, const float* freq_factors) {
  return guarded([&] { B(be).reserve_rope(head_dim, RopeParams{freq_base, neox != 0, freq_factors}); });
}

int nbh_backend_sync(nbh_backend* be) {
  return guarded([&] { B(be).sync(); });
}

int nbh_backend_live_allocations(const nbh_backend* be, int64_t* out) {
  return guarded([&] { *out = int64_t(B(be).live_allocations()); });
}

int nbh_backend_internal_bytes(const nbh_backend* be, int64_t* out) {
  return guarded([&] { *out = int64_t(B(be).internal_bytes()); });
}

int nbh_backend_cu_count(const nbh_backend* be, int* out) {
  return guarded([&] { *out = B(be).cu_count(); });
}

int nbh_backend_weight_bytes(const nbh_backend* be, int64_t* out) {
  return guarded([&] { *out = int64_t(B(be).weight_bytes()); });
}

int nbh_backend_fill_normal(nbh_backend* be, float* dst, int64_t count, uint64_t seed, float scale) {
  return guarded([&] { B(be).fill_normal(dst, count, seed, scale); });
}

int nbh_event_create(nbh_backend* be, nbh_event** out) {
  return guarded([&] {
    if (!out) throw nibble::Error("null output handle");
    B(be);
    auto* e = new nbh_event;
    const int rc = nbhs_event_create(&e->ev);
    if (rc != 0) {
      delete e;
      throw nibble::Error(std::string("event create failed: ") + nbhs_error_string(rc));
    }
    *out = e;
  });
}

int nbh_event_record(nbh_backend* be, nbh_event* e) {
  return guarded([&] {
    if (!e) throw nibble::Error("null event");
    const int rc = nbhs_event_record(e->ev, B(be).stream());
    if (rc != 0) throw nibble::Error(std::string("event record failed: ") + nbhs_error_string(rc));
  });
}

int nbh_event_elapsed_ms(nbh_event* start, nbh_event* end, float* ms) {
  return guarded([&] {
    if (!start || !end || !ms) throw nibble::Error("null event or output");
    const int rc = nbhs_event_elapsed_ms(start->ev, end->ev, ms);
    if (rc != 0) throw nibble::Error(std::string("event elapsed failed: ") + nbhs_error_string(rc));
  });
}

void nbh_event_destroy(nbh_event* e) {
  if (!e) return;
  nbhs_event_destroy(e->ev);
  delete e;
}

}  // extern "C"
