"""An independent fp64 forward pass of the qwen2 / llama transformer. TEST INFRASTRUCTURE ONLY.

Restates the reference's own second-opinion model, tests/naive_llama.h:63-150 (naive::naive_logits): plain
double-precision loops with no KV cache, no Backend and nothing of src/model. The reference's model tests require
its production forward to agree with it on logits (tests/test_model.cpp:110-131, max difference 1e-4); the GPU
forward is held to the same bar. Only tests/ use this module.

The model is a dict: "arch" ("qwen2" or "llama"), "eps", "base", "n_heads", "n_kv_heads", optional "rope_freqs"
[HD/2], "token_embd" [V, E], "output_norm" [E], optional "output" [V, E] (tied to token_embd otherwise), and
"layers": dicts with attn_norm, wq [H*HD, E], wk, wv [KV*HD, E], optional bq, bk, bv, wo [E, H*HD], ffn_norm,
w_gate, w_up [FF, E], w_down [E, FF]. Matrices may be float32 or float16; they are widened exactly.
"""
from __future__ import annotations

import numpy as np


def _d(a):
    return np.asarray(a, dtype=np.float64)


def _rms(x, w, eps):
    """naive_llama.h:53-60: x * w / sqrt(mean(x^2) + eps), all double; x [T, E]."""
    ss = np.sum(x * x, axis=-1, keepdims=True)
    return x * (1.0 / np.sqrt(ss / x.shape[-1] + eps)) * w


def _rope(v, heads, hd, positions, base, ff, llama):
    """naive_llama.h:78-90: angle pos * base^(-2i/hd) (/ ff[i]); llama pairs (2i, 2i+1), qwen2 (i, i+hd/2)."""
    i = np.arange(hd // 2, dtype=np.float64)
    theta = positions[:, None].astype(np.float64) * np.power(float(base), -2.0 * i / hd)[None, :]
    if ff is not None:
        theta = theta / _d(ff)[None, :]
    c, s = np.cos(theta)[:, None, :], np.sin(theta)[:, None, :]
    v = v.reshape(v.shape[0], heads, hd).copy()
    if llama:
        a, b = v[:, :, 0::2].copy(), v[:, :, 1::2].copy()
        v[:, :, 0::2], v[:, :, 1::2] = a * c - b * s, a * s + b * c
    else:
        a, b = v[:, :, : hd // 2].copy(), v[:, :, hd // 2:].copy()
        v[:, :, : hd // 2], v[:, :, hd // 2:] = a * c - b * s, a * s + b * c
    return v.reshape(v.shape[0], heads * hd)


def naive_logits(model, tokens):
    """Logits of the last token (naive_llama.h:63-150), fp64."""
    llama = model["arch"] == "llama"
    H, KV = model["n_heads"], model["n_kv_heads"]
    emb = _d(model["token_embd"])
    E = emb.shape[1]
    HD = E // H
    eps, base, ff = float(model["eps"]), float(model["base"]), model.get("rope_freqs")
    tokens = np.asarray(tokens, np.int64)
    T = tokens.size
    x = emb[tokens].copy()
    pos = np.arange(T)
    causal = np.tril(np.ones((T, T), bool))
    for L in model["layers"]:
        h = _rms(x, _d(L["attn_norm"]), eps)
        q, k, v = h @ _d(L["wq"]).T, h @ _d(L["wk"]).T, h @ _d(L["wv"]).T
        if "bq" in L:
            q, k, v = q + _d(L["bq"]), k + _d(L["bk"]), v + _d(L["bv"])
        q, k = _rope(q, H, HD, pos, base, ff, llama), _rope(k, KV, HD, pos, base, ff, llama)
        att = np.zeros((T, H * HD))
        for hh in range(H):
            g = hh // (H // KV)
            sc = q[:, hh * HD:(hh + 1) * HD] @ k[:, g * HD:(g + 1) * HD].T / np.sqrt(float(HD))
            sc = np.where(causal, sc, -np.inf)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            att[:, hh * HD:(hh + 1) * HD] = p @ v[:, g * HD:(g + 1) * HD]
        x = x + att @ _d(L["wo"]).T
        h = _rms(x, _d(L["ffn_norm"]), eps)
        gt, up = h @ _d(L["w_gate"]).T, h @ _d(L["w_up"]).T
        x = x + (gt / (1.0 + np.exp(-gt)) * up) @ _d(L["w_down"]).T
    h = _rms(x[T - 1:T], _d(model["output_norm"]), eps)
    out = _d(model["output"]) if model.get("output") is not None else emb
    return (h @ out.T)[0]
