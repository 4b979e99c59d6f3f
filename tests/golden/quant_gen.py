"""Deterministic raw-block generator of the reference's quantization golden tests, restated in Python
(tests/quant_golden_gen.h in the reference: splitmix64 Rng, the fill_* block fillers, q8k_rows, crafted_q8k_row,
FNV-1a). The golden file records an FNV-1a hash of every generated input, so a slip here fails loudly. Integer-only,
like the original, so the bytes are identical everywhere."""
from __future__ import annotations

import math

import numpy as np

M64 = (1 << 64) - 1
Q4, Q8, Q5_0, Q5_1, Q8_1, Q4_K, Q5_K, Q6_K, Q8_K = 18, 34, 22, 24, 36, 144, 176, 210, 292


class Rng:
    def __init__(self, seed):
        self.s = seed & M64

    def next(self):  # splitmix64
        self.s = (self.s + 0x9E3779B97F4A7C15) & M64
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> 31)


def rand_d(r):
    """fp16 scale bits: random sign and mantissa, exponent field 8..15, or 0 one time in 16."""
    v = r.next()
    sign = (v & 1) << 15
    exp = 0 if ((v >> 1) & 15) == 0 else 8 + ((v >> 5) & 7)
    man = (v >> 8) & 0x3FF
    return sign | (exp << 10) | man


def put_d(buf, off, d):
    buf[off] = d & 0xFF
    buf[off + 1] = (d >> 8) & 0xFF


def fill_q8_0(r, nb):
    b = bytearray(nb * Q8)
    for k in range(nb):
        p = k * Q8
        put_d(b, p, rand_d(r))
        for j in range(32):
            b[p + 2 + j] = r.next() & 0xFF
    return b


def fill_q4_0(r, nb):
    b = bytearray(nb * Q4)
    for k in range(nb):
        p = k * Q4
        put_d(b, p, rand_d(r))
        for j in range(16):
            b[p + 2 + j] = r.next() & 0xFF
    return b


def fill_q5_0(r, nb):
    b = bytearray(nb * Q5_0)
    for k in range(nb):
        p = k * Q5_0
        put_d(b, p, rand_d(r))
        for j in range(20):
            b[p + 2 + j] = r.next() & 0xFF
    return b


def fill_q5_1(r, nb):
    b = bytearray(nb * Q5_1)
    for k in range(nb):
        p = k * Q5_1
        put_d(b, p, rand_d(r))
        put_d(b, p + 2, rand_d(r))
        for j in range(20):
            b[p + 4 + j] = r.next() & 0xFF
    return b


def fp16_mul_int(s, d):
    """fp16 bits of s * fp16(d), truncated toward zero (integer-only)."""
    sign = (d & 0x8000) ^ (0x8000 if s < 0 else 0)
    e = (d >> 10) & 31
    p = abs(s) * ((0x400 | (d & 0x3FF)) if e else (d & 0x3FF))
    ex = e if e else 1
    if p == 0:
        return sign
    while p >= 2048:
        p >>= 1
        ex += 1
    while p < 1024 and ex > 1:
        p <<= 1
        ex -= 1
    return sign | (((ex << 10) | (p & 0x3FF)) if p >= 1024 else p)


def fill_q8_1(r, nb):
    b = bytearray(nb * Q8_1)
    for k in range(nb):
        p = k * Q8_1
        d = rand_d(r)
        s = 0
        for j in range(32):
            q = (r.next() % 255) - 127
            b[p + 4 + j] = q & 0xFF
            s += q
        put_d(b, p, d)
        put_d(b, p + 2, fp16_mul_int(s, d))
    return b


def _fill_k(r, nb, size):
    b = bytearray(nb * size)
    for k in range(nb):
        p = k * size
        put_d(b, p, rand_d(r))
        put_d(b, p + 2, rand_d(r))
        for j in range(4, size):
            b[p + j] = r.next() & 0xFF
    return b


def fill_q4_k(r, nb):
    return _fill_k(r, nb, Q4_K)


def fill_q5_k(r, nb):
    return _fill_k(r, nb, Q5_K)


def fill_q6_k(r, nb):
    b = bytearray(nb * Q6_K)
    for k in range(nb):
        p = k * Q6_K
        for j in range(Q6_K - 2):
            b[p + j] = r.next() & 0xFF
        put_d(b, p + Q6_K - 2, rand_d(r))
    return b


def fill_q8_k(r, nb):
    b = bytearray(nb * Q8_K)
    for k in range(nb):
        p = k * Q8_K
        v = r.next()
        bits = ((v & 1) << 31) | ((120 + ((v >> 1) & 15)) << 23) | ((v >> 8) & 0x7FFFFF)
        b[p:p + 4] = bits.to_bytes(4, "little")
        for j in range(256):
            b[p + 4 + j] = ((r.next() % 255) - 127) & 0xFF
        for g in range(16):
            s = sum(int(np.int8(b[p + 4 + g * 16 + i] - 256 if b[p + 4 + g * 16 + i] > 127 else b[p + 4 + g * 16 + i]))
                    for i in range(16))
            put_d(b, p + 260 + g * 2, s & 0xFFFF)
    return b


def q8k_rows(r, n):
    """Float rows: per block a power-of-two scale, elements are 21-bit integers times it, an occasional 8x."""
    x = np.zeros(n, np.float32)
    for b in range(n // 256):
        e = (r.next() % 20) - 10 - 20
        for j in range(256):
            v = r.next()
            k = (v % (1 << 21)) - (1 << 20)
            if ((v >> 32) & 63) == 0:
                k *= 8
            x[b * 256 + j] = np.float32(math.ldexp(float(k), e))
    return x


def crafted_q8k_row(cid):
    x = np.zeros(256, np.float32)
    if cid == 1:
        x[3], x[10] = -5.0, 5.0
    elif cid == 2:
        x[0] = -127.0
        for j in range(1, 256):
            x[j] = float((j % 61) - 30) + 0.5
    elif cid == 3:
        x[0] = 127.0
        for j in range(1, 256):
            x[j] = float((j % 5) - 2) * 3.0
    return x


def fnv1a(data, h=0xCBF29CE484222325):
    for c in bytes(data):
        h = ((h ^ c) * 0x100000001B3) & M64
    return h
