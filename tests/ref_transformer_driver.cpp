// Runs nibble's own model::Transformer (src/model/transformer.cpp, compiled from the reference's sources) over a
// chosen Backend: the reference's CpuBackend (src/backend/cpu/cpu_backend.h) or this repository's HipBackend, the
// drop-in. TEST INFRASTRUCTURE: built by oracle/Makefile (`make transformer`) into oracle/_ref/, run by
// tests/test_gpu_ref_transformer.py.
//
//   transformer_driver <model_dir> <cpu|hip> <n_ctx> <batch_invariant 0|1> <tokens,comma,separated> <run>...
//
// model_dir/model.txt holds the LlamaConfig fields (one "key value" line each) and one line per tensor,
// "tensor <name> <dtype> <n_dims> <ne0> <ne1> <offset> <bytes>", locating its bytes in model_dir/weights.bin. The
// Weights are bound by name here (Weights::bind reads a GGUF file, which the test does not write). Each <run> builds
// a fresh Transformer (empty KV cache): "b<max_batch>" feeds every token in one forward() call, chunked by
// max_batch as Transformer::forward chunks a prompt; "i" feeds one token per forward() call at positions 0, 1, ...
// For each run one JSON line is printed: {"run": "...", "bits": "<8 hex digits per logit>"}.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <span>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "backend/cpu/cpu_backend.h"
#include "backend/hip/hip_backend.h"
#include "model/transformer.h"
#include "nibble/error.h"
#include "thread_pool.h"

namespace {

using nibble::DType;
using nibble::Tensor;
using nibble::model::LayerWeights;
using nibble::model::LlamaConfig;
using nibble::model::Weights;

struct Model {
  LlamaConfig cfg;
  std::vector<char> bytes;
  std::map<std::string, Tensor> tensors;
};

Model load(const std::string& dir) {
  Model m;
  std::ifstream bin(dir + "/weights.bin", std::ios::binary);
  if (!bin) throw std::runtime_error("cannot open " + dir + "/weights.bin");
  m.bytes.assign(std::istreambuf_iterator<char>(bin), std::istreambuf_iterator<char>());
  std::ifstream txt(dir + "/model.txt");
  if (!txt) throw std::runtime_error("cannot open " + dir + "/model.txt");
  std::string line;
  while (std::getline(txt, line)) {
    std::istringstream ls(line);
    std::string key;
    ls >> key;
    if (key == "tensor") {
      std::string name;
      uint32_t type;
      int n_dims;
      int64_t ne0, ne1, off, nbytes;
      ls >> name >> type >> n_dims >> ne0 >> ne1 >> off >> nbytes;
      if (!ls || off < 0 || nbytes < 0 || off + nbytes > int64_t(m.bytes.size()))
        throw std::runtime_error("bad tensor line: " + line);
      Tensor t;
      t.type = DType(type);
      t.n_dims = n_dims;
      t.ne = {ne0, ne1, 1, 1};
      t.data = m.bytes.data() + off;
      m.tensors[name] = t;
    } else if (key == "arch") {
      ls >> m.cfg.arch;
    } else if (key == "n_layers") {
      ls >> m.cfg.n_layers;
    } else if (key == "n_embd") {
      ls >> m.cfg.n_embd;
    } else if (key == "n_ff") {
      ls >> m.cfg.n_ff;
    } else if (key == "n_heads") {
      ls >> m.cfg.n_heads;
    } else if (key == "n_kv_heads") {
      ls >> m.cfg.n_kv_heads;
    } else if (key == "head_dim") {
      ls >> m.cfg.head_dim;
    } else if (key == "n_vocab") {
      ls >> m.cfg.n_vocab;
    } else if (key == "rope_base") {
      ls >> m.cfg.rope_base;
    } else if (key == "rms_eps") {
      ls >> m.cfg.rms_eps;
    } else if (key == "rope_neox") {
      int v;
      ls >> v;
      m.cfg.rope_neox = v != 0;
    } else if (key == "qkv_bias") {
      int v;
      ls >> v;
      m.cfg.qkv_bias = v != 0;
    } else if (!key.empty()) {
      throw std::runtime_error("unknown key in model.txt: " + key);
    }
  }
  return m;
}

const Tensor& need(const Model& m, const std::string& name) {
  auto it = m.tensors.find(name);
  if (it == m.tensors.end()) throw std::runtime_error("missing tensor " + name);
  return it->second;
}

Weights bind(const Model& m) {
  Weights w;
  w.token_embd = need(m, "token_embd");
  w.output_norm = need(m, "output_norm");
  w.output = m.tensors.count("output") ? need(m, "output") : w.token_embd;  // tied, as the loader ties them
  if (m.tensors.count("rope_freqs")) w.rope_freqs = need(m, "rope_freqs");
  for (int64_t l = 0; l < m.cfg.n_layers; ++l) {
    const std::string p = "blk." + std::to_string(l) + ".";
    LayerWeights L;
    L.attn_norm = need(m, p + "attn_norm");
    L.wq = need(m, p + "wq");
    L.wk = need(m, p + "wk");
    L.wv = need(m, p + "wv");
    L.wo = need(m, p + "wo");
    L.ffn_norm = need(m, p + "ffn_norm");
    L.w_gate = need(m, p + "w_gate");
    L.w_up = need(m, p + "w_up");
    L.w_down = need(m, p + "w_down");
    if (m.cfg.qkv_bias) {
      L.bq = need(m, p + "bq");
      L.bk = need(m, p + "bk");
      L.bv = need(m, p + "bv");
    }
    w.layers.push_back(L);
  }
  return w;
}

std::vector<int32_t> parse_tokens(const std::string& s) {
  std::vector<int32_t> out;
  std::istringstream ss(s);
  std::string tok;
  while (std::getline(ss, tok, ',')) out.push_back(int32_t(std::stol(tok)));
  return out;
}

std::string hex_bits(const std::vector<float>& v) {
  std::string s;
  s.reserve(v.size() * 8);
  char buf[9];
  for (float f : v) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    std::snprintf(buf, sizeof buf, "%08x", u);
    s += buf;
  }
  return s;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 7) {
    std::fprintf(stderr, "usage: %s <model_dir> <cpu|hip> <n_ctx> <batch_invariant> <tokens> <run>...\n", argv[0]);
    return 2;
  }
  try {
    const Model m = load(argv[1]);
    const Weights w = bind(m);
    const std::string kind = argv[2];
    const int64_t n_ctx = std::stoll(argv[3]);
    const bool invariant = std::atoi(argv[4]) != 0;
    const std::vector<int32_t> toks = parse_tokens(argv[5]);
    std::unique_ptr<nibble::ThreadPool> pool;
    std::unique_ptr<nibble::Backend> be;
    if (kind == "cpu") {
      pool = std::make_unique<nibble::ThreadPool>(4);
      be = std::make_unique<nibble::cpu::CpuBackend>(*pool);
    } else if (kind == "hip") {
      auto hb = std::make_unique<nibble::hip::HipBackend>(0);
      hb->set_batch_invariant(invariant);
      be = std::move(hb);
    } else {
      std::fprintf(stderr, "unknown backend %s\n", kind.c_str());
      return 2;
    }
    std::vector<float> logits(size_t(m.cfg.n_vocab));
    for (int a = 6; a < argc; ++a) {
      const std::string run = argv[a];
      if (run == "i") {
        nibble::model::Transformer t(m.cfg, w, *be, n_ctx, 512);
        for (size_t i = 0; i < toks.size(); ++i)
          t.forward(std::span<const int32_t>(toks).subspan(i, 1), int64_t(i), logits.data());
      } else if (run.size() > 1 && run[0] == 'b') {
        nibble::model::Transformer t(m.cfg, w, *be, n_ctx, std::stoll(run.substr(1)));
        t.forward(toks, 0, logits.data());
      } else {
        std::fprintf(stderr, "unknown run %s\n", run.c_str());
        return 2;
      }
      std::printf("{\"run\": \"%s\", \"bits\": \"%s\"}\n", run.c_str(), hex_bits(logits).c_str());
      std::fflush(stdout);
    }
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
  }
  return 0;
}
