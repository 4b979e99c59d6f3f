// Heap-allocation accounting of the HIP backend's warm paths, in the manner of the reference's
// tests/alloc_tests.cpp:38-106 (a replaced global operator new counts every allocation while armed) and its
// no-allocation cases (:278-380: decode, short and long prefill and a direct matmul after warm-up allocate nothing).
// Every call goes through the C ABI (include/nibble_hip.h) at Llama-3.2-1B's attention shape (32 query heads, 8 KV
// heads, head_dim 64, width 2048) over a 1024-row cache.
//
// The HIP runtime and rocBLAS allocate through the same operator new inside the backend's calls, so each counted
// allocation is charged to the shared object of its first caller frame outside the C/C++ runtime (backtrace +
// dladdr; libstdc++/libc frames and standard-library template code are skipped): libnibble_hip.so is the backend's
// own code, anything else (libamdhip64, librocblas, ...) is a library it calls. One phase measures the runtime alone: a call that is one kernel launch and nothing else.
//
// Prints one JSON object: per armed phase, the backend calls made, the allocations in the backend's own code and
// the allocations by library.
#include <dlfcn.h>
#include <execinfo.h>

#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "nibble_hip.h"

namespace {
std::atomic<bool> g_armed{false};
constexpr int kLibs = 16;
struct Tally {
  std::atomic<int64_t> own{0};                 // charged to libnibble_hip.so
  std::atomic<int64_t> unknown{0};             // no frame outside the C/C++ runtime and this program
  const char* lib[kLibs] = {};                 // other shared objects (dli_fname, stable while loaded)
  std::atomic<int64_t> lib_count[kLibs] = {};
  const char* site[kLibs] = {};                // the backend's own allocating functions (dli_sname)
  std::atomic<int64_t> site_count[kLibs] = {};
};
Tally g_tally;
thread_local bool g_in_hook = false;

bool is_runtime_lib(const char* f) {
  const char* b = std::strrchr(f, '/');
  b = b ? b + 1 : f;
  return std::strncmp(b, "libstdc++", 9) == 0 || std::strncmp(b, "libc.so", 7) == 0 ||
         std::strncmp(b, "libgcc_s", 8) == 0 || std::strncmp(b, "libc++", 6) == 0;
}

void charge() {
  void* frames[24];
  const int n = backtrace(frames, 24);
  Dl_info self{};
  dladdr(reinterpret_cast<void*>(&charge), &self);
  for (int i = 1; i < n; ++i) {
    Dl_info info{};
    if (!dladdr(frames[i], &info) || !info.dli_fname) continue;
    if (info.dli_fbase == self.dli_fbase || is_runtime_lib(info.dli_fname)) continue;  // the hook, libstdc++, libc
    // Standard-library template code instantiated in a library (std::string, std::vector members) can serve other
    // libraries too: the dynamic linker binds every library's call of such a weak symbol to the first copy it
    // finds. Such a frame is the C++ runtime's, whichever object holds it; the caller is further up.
    if (info.dli_sname && (std::strncmp(info.dli_sname, "_ZNSt", 5) == 0 || std::strncmp(info.dli_sname, "_ZNKSt", 6) == 0 ||
                           std::strncmp(info.dli_sname, "_ZSt", 4) == 0))
      continue;
    if (std::strstr(info.dli_fname, "libnibble_hip")) {
      g_tally.own.fetch_add(1);
      const char* name = info.dli_sname ? info.dli_sname : "?";
      for (int k = 0; k < kLibs; ++k) {
        if (!g_tally.site[k]) g_tally.site[k] = name;
        if (g_tally.site[k] == name || std::strcmp(g_tally.site[k], name) == 0) {
          g_tally.site_count[k].fetch_add(1);
          break;
        }
      }
      return;
    }
    for (int k = 0; k < kLibs; ++k) {
      if (!g_tally.lib[k]) g_tally.lib[k] = info.dli_fname;  // one thread arms the hook at a time
      if (g_tally.lib[k] == info.dli_fname || std::strcmp(g_tally.lib[k], info.dli_fname) == 0) {
        g_tally.lib_count[k].fetch_add(1);
        return;
      }
    }
    break;
  }
  g_tally.unknown.fetch_add(1);
}

void* counted_alloc(std::size_t n, std::size_t align = 0) {
  if (g_armed.load(std::memory_order_relaxed) && !g_in_hook) {
    g_in_hook = true;
    charge();
    g_in_hook = false;
  }
  void* p = align ? std::aligned_alloc(align, (n + align - 1) / align * align) : std::malloc(n ? n : 1);
  if (!p) throw std::bad_alloc();
  return p;
}

struct Armed {
  Armed() {
    g_tally.own = 0;
    g_tally.unknown = 0;
    for (int k = 0; k < kLibs; ++k) g_tally.lib_count[k] = 0, g_tally.site_count[k] = 0;
    g_armed = true;
  }
  ~Armed() { g_armed = false; }
};

void check(int rc, const char* what) {
  if (rc != NBH_OK) {
    std::fprintf(stderr, "%s failed (%d): %s\n", what, rc, nbh_last_error());
    std::exit(2);
  }
}
}  // namespace

void* operator new(std::size_t n) { return counted_alloc(n); }
void* operator new[](std::size_t n) { return counted_alloc(n); }
void* operator new(std::size_t n, const std::nothrow_t&) noexcept {
  try {
    return counted_alloc(n);
  } catch (...) {
    return nullptr;
  }
}
void* operator new[](std::size_t n, const std::nothrow_t&) noexcept {
  try {
    return counted_alloc(n);
  } catch (...) {
    return nullptr;
  }
}
void* operator new(std::size_t n, std::align_val_t a) { return counted_alloc(n, static_cast<std::size_t>(a)); }
void* operator new[](std::size_t n, std::align_val_t a) { return counted_alloc(n, static_cast<std::size_t>(a)); }
void operator delete(void* p, std::align_val_t) noexcept { std::free(p); }
void operator delete[](void* p, std::align_val_t) noexcept { std::free(p); }
void operator delete(void* p, std::size_t, std::align_val_t) noexcept { std::free(p); }
void operator delete[](void* p, std::size_t, std::align_val_t) noexcept { std::free(p); }
void operator delete(void* p) noexcept { std::free(p); }
void operator delete[](void* p) noexcept { std::free(p); }
void operator delete(void* p, std::size_t) noexcept { std::free(p); }
void operator delete[](void* p, std::size_t) noexcept { std::free(p); }
void operator delete(void* p, const std::nothrow_t&) noexcept { std::free(p); }
void operator delete[](void* p, const std::nothrow_t&) noexcept { std::free(p); }

namespace {
constexpr int64_t H = 32, KV = 8, D = 64, W = 2048, CTX = 1024, ROWS = 64;
constexpr float kBase = 5e5f;

// A weight of `rows` x W in host memory: F16 (ggml id 1) halves near +-0.02, or Q8_0 (id 8: fp16 scale + 32 int8
// per block) / Q4_K (id 12: 144-byte super-blocks) blocks with small fp16 scales and pseudo-random quants.
struct HostWeight {
  std::vector<uint8_t> bytes;
  nbh_tensor t{};
};

HostWeight make_weight(uint32_t type, int64_t rows, uint32_t seed) {
  HostWeight w;
  uint64_t s = 0x9E3779B97F4A7C15ull * (seed + 1);
  auto next = [&] {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    return s;
  };
  int64_t row_bytes = type == 1 ? W * 2 : type == 8 ? (W / 32) * 34 : (W / 256) * 144;
  w.bytes.resize(size_t(rows * row_bytes));
  for (auto& b : w.bytes) b = uint8_t(next());
  if (type == 1) {  // fp16 with exponent 2^-6..2^-5 and random sign/mantissa
    for (size_t i = 0; i + 1 < w.bytes.size(); i += 2) w.bytes[i + 1] = uint8_t((w.bytes[i + 1] & 0x83) | 0x24);
  } else if (type == 8) {
    for (int64_t b = 0; b < rows * (W / 32); ++b) {
      w.bytes[size_t(b * 34)] = 0x00;
      w.bytes[size_t(b * 34 + 1)] = 0x20;  // scale 2^-7
    }
  } else {
    for (int64_t b = 0; b < rows * (W / 256); ++b) {
      uint8_t* p = &w.bytes[size_t(b * 144)];
      p[0] = 0x00, p[1] = 0x20, p[2] = 0x00, p[3] = 0x1c;  // d = 2^-7, dmin = 2^-8
    }
  }
  w.t.type = type;
  w.t.n_dims = 2;
  w.t.ne[0] = W;
  w.t.ne[1] = rows;
  w.t.ne[2] = w.t.ne[3] = 1;
  w.t.data = w.bytes.data();
  return w;
}
}  // namespace

int main() {
  nbh_backend* be = nullptr;
  check(nbh_backend_create(0, &be), "create");
  check(nbh_backend_reserve(be, CTX, H, ROWS, W), "reserve");
  auto alloc = [&](int64_t n) {
    float* p = nullptr;
    check(nbh_backend_alloc(be, n, &p), "alloc");
    check(nbh_backend_fill_normal(be, p, n, uint64_t(n) * 7 + 1, 1.0f), "fill_normal");
    return p;
  };
  float* x = alloc(ROWS * W);
  float* q = alloc(ROWS * H * D);
  float* kn = alloc(ROWS * KV * D);
  float* vn = alloc(ROWS * KV * D);
  float* out = alloc(ROWS * H * D);
  float* ck = alloc(CTX * KV * D);
  float* cv = alloc(CTX * KV * D);
  float* y = alloc(ROWS * 4 * W);
  constexpr int kSeq = 4;
  float* bk[kSeq];
  float* bv[kSeq];
  for (int i = 0; i < kSeq; ++i) bk[i] = alloc(CTX * KV * D), bv[i] = alloc(CTX * KV * D);

  HostWeight f16[3] = {make_weight(1, H * D, 1), make_weight(1, KV * D, 2), make_weight(1, KV * D, 3)};
  HostWeight qw[3] = {make_weight(8, H * D, 4), make_weight(12, KV * D, 5), make_weight(8, KV * D, 6)};
  const nbh_tensor* wf[3] = {&f16[0].t, &f16[1].t, &f16[2].t};
  const nbh_tensor* wq[3] = {&qw[0].t, &qw[1].t, &qw[2].t};
  float* ys[3] = {q, kn, vn};
  float* ysq[3] = {y, y + ROWS * H * D, y + ROWS * (H + KV) * D};

  auto decode_step = [&](int64_t pos) {
    check(nbh_backend_matmul_multi(be, 3, wf, x, ys, 1), "matmul_multi f16 n=1");
    check(nbh_backend_append_rope_attention(be, q, ck, cv, kn, vn, out, 1, pos, H, KV, D, kBase, 0, nullptr),
          "append_rope_attention n=1");
    check(nbh_backend_attention(be, q, ck, cv, out, 1, pos, H, KV, D), "attention n=1");
  };
  auto prefill_chunk = [&](int64_t pos0, int64_t n) {
    check(nbh_backend_matmul_multi(be, 3, wf, x, ys, n), "matmul_multi f16 chunk");
    check(nbh_backend_append_rope_attention(be, q, ck, cv, kn, vn, out, n, pos0, H, KV, D, kBase, 0, nullptr),
          "append_rope_attention chunk");
    check(nbh_backend_rope(be, q, n, H, D, pos0, kBase, 0, nullptr), "rope chunk");
    check(nbh_backend_attention(be, q, ck, cv, out, n, pos0, H, KV, D), "attention chunk");
  };
  auto quant = [&](int64_t n) { check(nbh_backend_matmul_multi(be, 3, wq, x, ysq, n), "matmul_multi quantized"); };
  const float* bq[kSeq];
  const float* bkn[kSeq];
  const float* bvn[kSeq];
  float* bo[kSeq];
  int64_t bpos[kSeq];
  for (int i = 0; i < kSeq; ++i) {
    bq[i] = q + i * H * D;
    bkn[i] = kn + i * KV * D;
    bvn[i] = vn + i * KV * D;
    bo[i] = out + i * H * D;
  }
  auto batch_step = [&](int64_t pos) {
    for (int i = 0; i < kSeq; ++i) bpos[i] = pos + 37 * i;
    check(nbh_backend_append_rope_attention_batch(be, kSeq, bq, bk, bv, bkn, bvn, bo, bpos, H, KV, D, kBase, 0,
                                                  nullptr),
          "append_rope_attention_batch");
  };

  // The first calls after reserve() that need no weight: a prefill chunk's attention and decode steps (the RoPE
  // table is built on first use of each (base, head_dim, factors); reserve_rope() builds it ahead, as here).
  check(nbh_backend_reserve_rope(be, D, kBase, 0, nullptr), "reserve_rope");
  check(nbh_backend_sync(be), "sync");
  {  // the unwinder loads on first use; not inside an armed phase
    void* f[4];
    backtrace(f, 4);
  }
  // One armed phase's tally, written out as JSON at the end (the strings are formatted after disarming).
  struct Phase {
    const char* name;
    int64_t calls, own, unknown;
    const char* lib[kLibs];
    int64_t lib_count[kLibs];
    const char* site[kLibs];
    int64_t site_count[kLibs];
  };
  std::vector<Phase> phases;
  phases.reserve(8);
  auto snapshot = [&](const char* name, int64_t calls) {
    Phase p{name, calls, g_tally.own.load(), g_tally.unknown.load(), {}, {}, {}, {}};
    for (int k = 0; k < kLibs; ++k) {
      p.lib[k] = g_tally.lib[k], p.lib_count[k] = g_tally.lib_count[k].load();
      p.site[k] = g_tally.site[k], p.site_count[k] = g_tally.site_count[k].load();
    }
    phases.push_back(p);
  };
  auto run = [&](const char* name, int64_t calls, auto&& body) {
    {
      Armed a;
      body();
      check(nbh_backend_sync(be), "sync");
    }
    snapshot(name, calls);
  };
  run("first_calls_after_reserve", 5, [&] {
    check(nbh_backend_append_rope_attention(be, q, ck, cv, kn, vn, out, ROWS, 256, H, KV, D, kBase, 0, nullptr),
          "first prefill");
    for (int64_t i = 0; i < 4; ++i)
      check(nbh_backend_append_rope_attention(be, q, ck, cv, kn, vn, out, 1, 320 + i, H, KV, D, kBase, 0, nullptr),
            "first decode");
  });

  // Warm-up: every path once (weights copied to HBM on first use, rocBLAS handle, widenings).
  decode_step(100);
  prefill_chunk(128, ROWS);
  prefill_chunk(512, 40);
  for (int64_t n : {int64_t(1), int64_t(8), int64_t(17), ROWS}) quant(n);
  batch_step(300);
  check(nbh_backend_sync(be), "sync");

  constexpr int kLaunches = 64;
  run("runtime_fill_normal_launches", kLaunches, [&] {
    for (int i = 0; i < kLaunches; ++i) check(nbh_backend_fill_normal(be, out, H * D, uint64_t(i), 1.0f), "fill");
  });
  run("decode_steps", 16 * 3, [&] {
    for (int64_t i = 0; i < 16; ++i) decode_step(600 + i);
  });
  run("prefill_chunks", 4 * 4, [&] {
    prefill_chunk(192, ROWS);
    prefill_chunk(640, ROWS);
    prefill_chunk(900, 30);
    prefill_chunk(CTX - ROWS, ROWS);
  });
  run("matmul_quantized", 4, [&] {
    for (int64_t n : {int64_t(1), int64_t(8), int64_t(17), ROWS}) quant(n);
  });
  run("batch_decode", 8, [&] {
    for (int64_t i = 0; i < 8; ++i) batch_step(700 + i);
  });

  std::printf("{");
  for (size_t i = 0; i < phases.size(); ++i) {
    const Phase& p = phases[i];
    std::printf("%s\"%s\": {\"calls\": %lld, \"own\": %lld, \"unattributed\": %lld, \"libraries\": {", i ? ", " : "",
                p.name, static_cast<long long>(p.calls), static_cast<long long>(p.own),
                static_cast<long long>(p.unknown));
    bool first_lib = true;
    for (int k = 0; k < kLibs; ++k)
      if (p.lib[k] && p.lib_count[k]) {
        const char* b = std::strrchr(p.lib[k], '/');
        std::printf("%s\"%s\": %lld", first_lib ? "" : ", ", b ? b + 1 : p.lib[k],
                    static_cast<long long>(p.lib_count[k]));
        first_lib = false;
      }
    std::printf("}, \"own_sites\": {");
    bool first_site = true;
    for (int k = 0; k < kLibs; ++k)
      if (p.site[k] && p.site_count[k]) {
        std::printf("%s\"%s\": %lld", first_site ? "" : ", ", p.site[k], static_cast<long long>(p.site_count[k]));
        first_site = false;
      }
    std::printf("}}");
  }
  std::printf("}\n");
  nbh_backend_destroy(be);
  return 0;
}
