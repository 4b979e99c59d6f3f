"""Seeded synthetic inputs for the benchmark configurations (host side, numpy).

A counter-based generator so that any element can be produced independently and identically on any host:
SplitMix64 of (stream key, element pair index) gives two 53-bit uniforms, a Box-Muller transform in double gives
two N(0,1) values, rounded to float32. Stream keys fold (config, layer, sequence, tensor, ...) integers. This is
deliberately not std::normal_distribution / numpy's Generator, whose streams are implementation-defined.

The device fill (HipBackend.fill_normal) uses the same hashing with fp32 Box-Muller; its values are not bit-equal to
these and are only used where the consumer reads the device data back (benchmarks, full-size parity checks).
"""
from __future__ import annotations

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_MASK = (1 << 64) - 1


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _mix_int(x: int) -> int:
    with np.errstate(over="ignore"):
        return int(_mix(np.array([x & _MASK], dtype=np.uint64))[0])


def stream_key(*parts: int) -> int:
    """Folds integers (config, layer, sequence, tensor id, ...) into one 64-bit stream key."""
    k = 0x6A09E667F3BCC909
    for p in parts:
        k = _mix_int((k + (int(p) + 1) * 0x9E3779B97F4A7C15) & _MASK)
    return k


def normal(key: int, count: int, offset: int = 0) -> np.ndarray:
    """Elements [offset, offset + count) of the N(0,1) stream `key`, as float32. offset must be even."""
    assert offset % 2 == 0 and count >= 0
    if count == 0:
        return np.zeros(0, np.float32)
    p0 = offset // 2
    pairs = (count + 1) // 2
    with np.errstate(over="ignore"):
        p = np.arange(p0, p0 + pairs, dtype=np.uint64)
        k = np.uint64(key & _MASK)
        h1 = _mix(k + (np.uint64(2) * p + np.uint64(1)) * _GAMMA)
        h2 = _mix(k + (np.uint64(2) * p + np.uint64(2)) * _GAMMA)
    u1 = ((h1 >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)  # (0, 1]
    u2 = (h2 >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)          # [0, 1)
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * pairs, np.float64)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return out[:count].astype(np.float32)


def normal_array(shape, *key_parts: int) -> np.ndarray:
    return normal(stream_key(*key_parts), int(np.prod(shape))).reshape(shape)


def llama3_freq_factors(head_dim: int, base: float, factor: float = 32.0, low: float = 1.0, high: float = 4.0,
                        orig_ctx: float = 8192.0) -> np.ndarray:
    """Llama-3 RoPE frequency factors (the rope_freqs.weight tensor llama.cpp's converter writes; the reference
    only reads it, weights.cpp:56, and divides angles by it, ref_ops.cpp:175). Closed form in double, float32."""
    i = np.arange(head_dim // 2, dtype=np.float64)
    freq = base ** (-2.0 * i / head_dim)
    wavelen = 2.0 * np.pi / freq
    s = (orig_ctx / wavelen - low) / (high - low)
    f = np.where(wavelen < orig_ctx / high, 1.0,
                 np.where(wavelen > orig_ctx / low, factor, 1.0 / ((1.0 - s) / factor + s)))
    return f.astype(np.float32)


# ggml block layouts (reference src/quant.h:34-110): block bytes, elements per block, and the byte offsets of the
# fp16 scale fields (d and, where present, the minimum) inside a block.
QUANT_BLOCKS = {2: (18, 32, (0,)), 6: (22, 32, (0,)), 7: (24, 32, (0, 2)), 8: (34, 32, (0,)),
                12: (144, 256, (0, 2)), 13: (176, 256, (0, 2)), 14: (210, 256, (208,))}


def quant_weight(t: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """Synthetic raw blocks of ggml type t for a rows x cols weight (benchmarks): random quant bytes and fp16 scales
    of magnitude 2^-9..2^-6, as trained weights' per-block scales are. Returns the uint8 block array."""
    bb, be, offs = QUANT_BLOCKS[t]
    nb = rows * cols // be
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, (nb, bb), dtype=np.uint8)
    for o in offs:
        mag = rng.uniform(2.0 ** -9, 2.0 ** -6, nb).astype(np.float16)
        sign = np.where(rng.random(nb) < 0.5, -1, 1).astype(np.float16) if o == 0 and t in (2, 6, 8) else 1
        raw[:, o:o + 2] = (mag * sign).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)
