"""Model shapes and workloads of the attention-path benchmark configurations.

Head geometry and RoPE settings follow the reference's LlamaConfig (src/model/config.h:14-33): NeoX pairing for
qwen2 (config.cpp:24), base theta from `<arch>.rope.freq_base`, Llama-3 frequency factors from rope_freqs.weight.
"""
from __future__ import annotations

import dataclasses

import numpy as np

from . import synth


@dataclasses.dataclass(frozen=True)
class Shape:
    name: str
    n_heads: int
    n_kv_heads: int
    head_dim: int
    n_layers: int
    rope_base: float
    neox: bool
    llama3: bool = False  # Llama-3 frequency scaling: factor 32, low 1, high 4, original context 8192
    n_embd: int = 0  # model width: the QKV projection's input width
    qkv_bias: bool = False  # q/k/v projections carry biases (qwen2)

    def freq_factors(self):
        return synth.llama3_freq_factors(self.head_dim, self.rope_base) if self.llama3 else None


QWEN25_05B = Shape("qwen2.5-0.5b", 14, 2, 64, 24, 1e6, True, n_embd=896, qkv_bias=True)
TINYLLAMA_11B = Shape("tinyllama-1.1b", 32, 4, 64, 22, 1e4, False, n_embd=2048)
LLAMA32_1B = Shape("llama-3.2-1b", 32, 8, 64, 16, 5e5, False, llama3=True, n_embd=2048)

# Stream-key tensor ids for synth.stream_key(config, layer, sequence, tensor, ...).
T_Q, T_K, T_V, T_KCACHE, T_VCACHE, T_SCALE = 1, 2, 3, 4, 5, 6

# Config 1: one Qwen layer, one new token at position 512 over 512 cached rows.
CFG1 = dict(id=1, shape=QWEN25_05B, layers=1, pos0=512)
# Config 2: Qwen prefill of 2048 tokens through all 24 layers.
CFG2 = dict(id=2, shape=QWEN25_05B, layers=24, n=2048)
# Config 3: TinyLlama, 256 single-token steps from a 1792-row cache to 2048, all 22 layers.
CFG3 = dict(id=3, shape=TINYLLAMA_11B, layers=22, start=1792, steps=256)
# Config 4: Llama-3.2 prefill 8192 then 64 decode steps against a 32768-row cache, all 16 layers. Chosen layout
# (the wording "first 8192 ... remaining earlier" is ambiguous): cache rows 0..8191 are the prefilled rows, rows
# 8192..32767 are seeded N(0,1), and decode step s appends at position 32768 + s (capacity 32832).
CFG4 = dict(id=4, shape=LLAMA32_1B, layers=16, prefill=8192, ctx=32768, steps=64)
# Config 5: 16 independent Llama-3.2 sequences, cache lengths log-uniform in [1024, 131072], 1% of K rows x8.
CFG5 = dict(id=5, shape=LLAMA32_1B, layers=16, n_seq=16, lo=1024, hi=131072, scaled_frac=0.01, scale=8.0)


def cfg5_lengths(seed_parts=(5, 0)) -> list[int]:
    """The 16 ragged cache lengths of config 5: round(exp(U(ln 1024, ln 131072))) from the seeded stream."""
    key = synth.stream_key(*seed_parts, 99)
    u = synth.normal(key, 2 * CFG5["n_seq"])  # two normals per draw -> a uniform via the normal CDF
    from math import erf, exp, log, sqrt
    lo, hi = log(CFG5["lo"]), log(CFG5["hi"])
    out = []
    for i in range(CFG5["n_seq"]):
        uu = 0.5 * (1.0 + erf(float(u[2 * i]) / sqrt(2.0)))
        out.append(int(round(exp(lo + (hi - lo) * uu))))
    return out


def cfg5_scaled_rows(seq: int, length: int) -> np.ndarray:
    """Sorted cache rows of sequence `seq` whose K rows are scaled x8 (1% of the rows, seeded)."""
    key = synth.stream_key(5, seq, 77)
    z = synth.normal(key, length)
    k = max(1, int(round(CFG5["scaled_frac"] * length)))
    return np.sort(np.argsort(z, kind="stable")[:k])
