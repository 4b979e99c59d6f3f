"""Synthetic tiny models and the two forward drivers the model tests compare.

* tiny_model: a random qwen2 / llama model of the shape family of the reference's tests/tiny_model.h:177-260
  (2 layers, 4 heads, 2 KV heads; n_embd 16 / n_ff 32 by default, 256 / 512 for the head_dim-64 variant), weights
  uniform in [-0.5, 0.5], norms in [0.9, 1.1]; generated here with numpy (the reference's generator is C++).
* cpu_forward: the reference's Transformer::forward (src/model/transformer.cpp:128-220) restated as the same
  sequence of the oracle's float ops (each pinned to the compiled reference), one chunk of all tokens.
* gpu_forward: the same sequence through HipBackend (the C ABI), chunked by max_batch as the reference's forward
  chunks a prompt.
"""
from __future__ import annotations

import numpy as np

import oracle


def tiny_model(seed, wtype=np.float32, arch="qwen2", rope_freqs=False, E=16, FF=32, H=4, KV=2, V=261, L=2,
               eps=1e-6, base=10000.0, explicit_output=False, scale=1.0):
    """`scale` multiplies every weight matrix (uniform in [-0.5 scale, 0.5 scale])."""
    rng = np.random.default_rng(seed)

    def mat(out, inp):
        return (rng.uniform(-0.5, 0.5, (out, inp)) * scale).astype(np.float32).astype(wtype)

    def vec(n, lo, hi):
        return rng.uniform(lo, hi, n).astype(np.float32)

    HD = E // H
    m = {"arch": arch, "eps": eps, "base": base, "n_heads": H, "n_kv_heads": KV, "token_embd": mat(V, E),
         "output_norm": vec(E, 0.9, 1.1), "output": mat(V, E) if explicit_output else None,
         "rope_freqs": vec(HD // 2, 1.0, 8.0) if rope_freqs else None, "layers": []}
    for _ in range(L):
        lay = {"attn_norm": vec(E, 0.9, 1.1), "wq": mat(H * HD, E), "wk": mat(KV * HD, E), "wv": mat(KV * HD, E),
               "wo": mat(E, H * HD), "ffn_norm": vec(E, 0.9, 1.1), "w_gate": mat(FF, E), "w_up": mat(FF, E),
               "w_down": mat(E, FF)}
        if arch == "qwen2":
            lay.update(bq=vec(H * HD, -0.5, 0.5), bk=vec(KV * HD, -0.5, 0.5), bv=vec(KV * HD, -0.5, 0.5))
        m["layers"].append(lay)
    return m


def _dims(m):
    E = m["token_embd"].shape[1]
    H, KV = m["n_heads"], m["n_kv_heads"]
    return E, H, KV, E // H, m["layers"][0]["w_gate"].shape[0], m["token_embd"].shape[0]


def cpu_forward(m, tokens):
    """Transformer::forward restated with the oracle's float ops (all tokens as one chunk at position 0)."""
    E, H, KV, HD, FF, V = _dims(m)
    n = len(tokens)
    neox = m["arch"] == "qwen2"
    x = oracle.embed(m["token_embd"], tokens)
    for L in m["layers"]:
        h = oracle.rmsnorm(x, L["attn_norm"], m["eps"])
        q, k, v = oracle.matmul(L["wq"], h), oracle.matmul(L["wk"], h), oracle.matmul(L["wv"], h)
        if "bq" in L:
            q, k, v = oracle.add_bias(q, L["bq"]), oracle.add_bias(k, L["bk"]), oracle.add_bias(v, L["bv"])
        q = oracle.rope(q.reshape(n, H, HD), 0, m["base"], neox, m["rope_freqs"])
        k = oracle.rope(k.reshape(n, KV, HD), 0, m["base"], neox, m["rope_freqs"])
        att = oracle.attention_scalar(q, k, v.reshape(n, KV, HD), 0, KV).reshape(n, H * HD)
        x = oracle.add(x, oracle.matmul(L["wo"], att))
        h = oracle.rmsnorm(x, L["ffn_norm"], m["eps"])
        g = oracle.silu_mul(oracle.matmul(L["w_gate"], h), oracle.matmul(L["w_up"], h))
        x = oracle.add(x, oracle.matmul(L["w_down"], g))
    last = oracle.rmsnorm(x[n - 1:n], m["output_norm"], m["eps"])
    out = m["output"] if m["output"] is not None else m["token_embd"]
    return oracle.matmul(out, last)[0]


class GpuModel:
    """Device state of one model on a HipBackend: activation buffers for max_batch rows and per-layer K/V caches
    of n_ctx rows (Transformer's constructor, transformer.cpp:59-100). forward() follows Transformer::forward."""

    def __init__(self, be, m, n_ctx, max_batch=512):
        self.be, self.m, self.n_ctx, self.max_batch = be, m, n_ctx, max_batch
        E, H, KV, HD, FF, V = _dims(m)
        self.dims = (E, H, KV, HD, FF, V)
        be.reserve(n_ctx, H, max_batch, max(E, H * HD, FF))
        self.bufs = []

        def alloc(nf):
            p = be.alloc(nf)
            self.bufs.append(p)
            return p

        B = max_batch
        self.x, self.h, self.q, self.attn = alloc(B * E), alloc(B * E), alloc(B * H * HD), alloc(B * H * HD)
        self.gate, self.up, self.last, self.logits = alloc(B * FF), alloc(B * FF), alloc(E), alloc(V)
        self.k = [alloc(n_ctx * KV * HD) for _ in m["layers"]]
        self.v = [alloc(n_ctx * KV * HD) for _ in m["layers"]]
        self.ff = None if m["rope_freqs"] is None else np.ascontiguousarray(m["rope_freqs"], np.float32)

    def run_chunk(self, tokens, pos0):
        be, m = self.be, self.m
        E, H, KV, HD, FF, V = self.dims
        n, kvw, neox, base = len(tokens), KV * HD, m["arch"] == "qwen2", m["base"]
        be.embed(m["token_embd"], tokens, self.x)
        for li, L in enumerate(m["layers"]):
            kc, vc = self.k[li].at(pos0 * kvw), self.v[li].at(pos0 * kvw)
            be.rmsnorm(self.x, L["attn_norm"], self.h, n, m["eps"])
            be.matmul_multi([L["wq"], L["wk"], L["wv"]], self.h, [self.q, kc, vc], n)
            if "bq" in L:
                be.add_bias(self.q, L["bq"], n)
                be.add_bias(kc, L["bk"], n)
                be.add_bias(vc, L["bv"], n)
            be.rope(self.q, n, H, HD, pos0, base, neox, self.ff)
            be.rope(kc, n, KV, HD, pos0, base, neox, self.ff)
            be.attention(self.q, self.k[li], self.v[li], self.attn, n, pos0, H, KV, HD)
            be.matmul(L["wo"], self.attn, self.h, n)
            be.add(self.x, self.h, n * E)
            be.rmsnorm(self.x, L["ffn_norm"], self.h, n, m["eps"])
            be.matmul_multi([L["w_gate"], L["w_up"]], self.h, [self.gate, self.up], n)
            be.silu_mul(self.gate, self.up, n * FF)
            be.matmul(L["w_down"], self.gate, self.h, n)
            be.add(self.x, self.h, n * E)

    def forward(self, tokens, pos0=0):
        """Logits of the last token (transformer.cpp:128-143)."""
        E, H, KV, HD, FF, V = self.dims
        n = len(tokens)
        for off in range(0, n, self.max_batch):
            self.run_chunk(tokens[off:off + self.max_batch], pos0 + off)
        rows = (n - 1) % self.max_batch
        m = self.m
        self.be.rmsnorm(self.x.at(rows * E), m["output_norm"], self.last, 1, m["eps"])
        out = m["output"] if m["output"] is not None else m["token_embd"]
        self.be.matmul(out, self.last, self.logits, 1)
        return self.be.read(self.logits, V).copy()

    def close(self):
        for p in self.bufs:
            self.be.free(p)
        self.bufs.clear()
        self.be.release_weights()


def write_model_dir(m, path):
    """Writes model m for tests/ref_transformer_driver.cpp: model.txt (the LlamaConfig fields and one line per tensor)
    and weights.bin (every tensor's bytes, 64-byte aligned). Matrices are [in, out] Tensors (ne[0] = input width) of
    their array's type (F32, F16, or a quantized QMat's raw blocks); norms, biases and rope_freqs are F32 vectors."""
    import os

    E, H, KV, HD, FF, V = _dims(m)
    blobs, lines, off = [], [], 0

    def add(name, a):
        nonlocal off
        if hasattr(a, "raw"):  # tests.quant_util.QMat
            t, data, dims, ne0, ne1 = a.t, a.raw.tobytes(), 2, a.cols, a.rows
        else:
            a = np.ascontiguousarray(a)
            t = {np.dtype(np.float32): 0, np.dtype(np.float16): 1}[a.dtype]
            data, dims = a.tobytes(), a.ndim
            ne0, ne1 = a.shape[-1], (a.shape[0] if a.ndim == 2 else 1)
        pad = (-off) % 64
        blobs.append(b"\0" * pad + data)
        off += pad
        lines.append(f"tensor {name} {t} {dims} {ne0} {ne1} {off} {len(data)}")
        off += len(data)

    add("token_embd", m["token_embd"])
    add("output_norm", m["output_norm"])
    if m["output"] is not None:
        add("output", m["output"])
    if m["rope_freqs"] is not None:
        add("rope_freqs", m["rope_freqs"])
    for i, L in enumerate(m["layers"]):
        for k in ("attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w_gate", "w_up", "w_down", "bq", "bk", "bv"):
            if k in L:
                add(f"blk.{i}.{k}", L[k])
    qwen = m["arch"] == "qwen2"
    cfg = [f"arch {m['arch']}", f"n_layers {len(m['layers'])}", f"n_embd {E}", f"n_ff {FF}", f"n_heads {H}",
           f"n_kv_heads {KV}", f"head_dim {HD}", f"n_vocab {V}", f"rope_base {m['base']!r}", f"rms_eps {m['eps']!r}",
           f"rope_neox {int(qwen)}", f"qkv_bias {int('bq' in m['layers'][0])}"]
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "model.txt"), "w") as f:
        f.write("\n".join(cfg + lines) + "\n")
    with open(os.path.join(path, "weights.bin"), "wb") as f:
        for b in blobs:
            f.write(b)
