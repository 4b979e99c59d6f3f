"""Quantized weight matrices for the GPU tests: raw ggml block bytes (src/quant.h layouts) with their type and shape.

QMat.nbh_tensor() gives the C ABI view; np.asarray(QMat) gives the dequantized float32 matrix (the oracle's
restatement of quant.cpp's dequantize_row), so the fp64 naive model reads the same weights."""
from __future__ import annotations

import numpy as np

import nibble_amd
import oracle
from tests.golden import quant_gen as G

FILLS = {oracle.Q4_0: G.fill_q4_0, oracle.Q5_0: G.fill_q5_0, oracle.Q5_1: G.fill_q5_1, oracle.Q8_0: G.fill_q8_0,
         oracle.Q4_K: G.fill_q4_k, oracle.Q5_K: G.fill_q5_k, oracle.Q6_K: G.fill_q6_k}
NAMES = {oracle.Q4_0: "Q4_0", oracle.Q5_0: "Q5_0", oracle.Q5_1: "Q5_1", oracle.Q8_0: "Q8_0", oracle.Q4_K: "Q4_K",
         oracle.Q5_K: "Q5_K", oracle.Q6_K: "Q6_K"}


class QMat:
    def __init__(self, t, raw, rows, cols):
        self.t, self.raw, self.rows, self.cols = t, np.ascontiguousarray(raw, np.uint8), rows, cols
        self.shape = (rows, cols)

    def nbh_tensor(self):
        return nibble_amd.weight(self.raw, shape=(self.rows, self.cols), dtype=self.t)

    def __array__(self, dtype=None, copy=None):
        d = oracle.dequantize(self.t, self.raw, self.rows * self.cols).reshape(self.rows, self.cols)
        return d.astype(dtype) if dtype is not None else d


def random_qmat(t, rows, cols, seed):
    """Random blocks from the golden generator (random quants and scales)."""
    nb = rows * cols // oracle.block_elems(t)
    return QMat(t, np.frombuffer(bytes(FILLS[t](G.Rng(seed), nb)), np.uint8), rows, cols)


def quantize_q4_0(w):
    """ggml's quantize_row_q4_0_ref: per block d = max / -8 with max the signed value of largest magnitude,
    q = min(15, int(x / d + 8.5)); used only to make Q4_0 test weights from float ones."""
    w = np.asarray(w, np.float32).reshape(-1, 32)
    out = np.zeros((w.shape[0], 18), np.uint8)
    for i, blk in enumerate(w):
        j = int(np.argmax(np.abs(blk)))
        mx = blk[j]
        d = np.float32(mx / np.float32(-8.0))
        idv = np.float32(1.0) / d if d != 0 else np.float32(0.0)
        dh = np.float16(d)
        out[i, :2] = np.frombuffer(dh.tobytes(), np.uint8)
        q = np.minimum(15, (blk * idv + np.float32(8.5)).astype(np.int8)).astype(np.uint8)
        out[i, 2:] = (q[:16] & 0xF) | ((q[16:] & 0xF) << 4)
    return out.reshape(-1)


def quantize_matrix(w, t):
    """Q8_0 (the oracle's Q8_0 quantizer, which makes valid Q8_0 blocks) or Q4_0 bytes of a float matrix."""
    w = np.asarray(w, np.float32)
    raw = oracle.quantize(0, w) if t == oracle.Q8_0 else quantize_q4_0(w)
    return QMat(t, raw, w.shape[0], w.shape[1])
