"""ctypes bindings for the CPU oracle. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as the
checker or the reported CPU baseline. The product path (nibble_amd/) never imports it.

Two libraries:
  liboracle.so            our C restatement of nibble's attention path (oracle.c, oracle_avx2.c)
  _ref/libnibble_ref.so   the reference's own CPU backend compiled from its sources (absent when the reference
                          tree was not available at build time; `have_ref()` says which)
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int64, c_void_p

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
_F = POINTER(c_float)
_D = POINTER(c_double)
_I = c_int64

_lib = None
_ref = None
_ref_tried = False


def _load():
    global _lib
    if _lib is None:
        path = os.path.join(_DIR, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run __graft_entry__.build())")
        lib = ctypes.CDLL(path)
        lib.orc_rope.argtypes = [_F, _I, _I, _I, _I, c_float, c_int, _F]
        lib.orc_rope.restype = None
        lib.orc_softmax_inplace.argtypes = [_F, _I]
        lib.orc_softmax_inplace.restype = None
        attn = [_F, _F, _F, _F, _I, _I, _I, _I, _I, _I, _I, _F]
        lib.orc_attention_scalar.argtypes = attn
        lib.orc_attention_scalar.restype = None
        lib.orc_attention_avx2.argtypes = attn
        lib.orc_attention_avx2.restype = c_int
        lib.orc_exp_ps.argtypes = [_F, _F, _I]
        lib.orc_exp_ps.restype = c_int
        lib.orc_have_avx2.argtypes = []
        lib.orc_have_avx2.restype = c_int
        lib.orc_attention_heads_parallel.argtypes = [_F, _F, _F, _F, _I, _I, _I, _I, _I, c_int, c_int, _F]
        lib.orc_attention_heads_parallel.restype = c_int
        lib.orc_attention_f64.argtypes = [_F, _F, _F, _D, _I, _I, _I, _I, _I]
        lib.orc_attention_f64.restype = None
        lib.orc_llama3_freq_factors.argtypes = [_F, _I, c_double, c_double, c_double, c_double, c_double]
        lib.orc_llama3_freq_factors.restype = None
        lib.orc_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        lib.orc_fp16_to_fp32.restype = c_float
        lib.orc_fp16_to_fp32_n.argtypes = [c_void_p, _F, _I]
        lib.orc_fp16_to_fp32_n.restype = None
        lib.orc_matmul.argtypes = [c_int, c_void_p, _I, _I, _F, _F, _I]
        lib.orc_matmul.restype = c_int
        lib.orc_add_bias.argtypes = [_F, _F, _I, _I]
        lib.orc_add_bias.restype = None
        lib.orc_embed.argtypes = [c_int, c_void_p, _I, _I, c_void_p, _I, _F]
        lib.orc_rmsnorm.argtypes = [_F, _F, _F, _I, _I, c_float]
        lib.orc_rmsnorm.restype = None
        lib.orc_add.argtypes = [_F, _F, _I]
        lib.orc_add.restype = None
        lib.orc_silu_mul.argtypes = [_F, _F, _I]
        lib.orc_silu_mul.restype = None
        lib.orc_block_bytes.argtypes = [c_int]
        lib.orc_block_bytes.restype = _I
        lib.orc_block_elems.argtypes = [c_int]
        lib.orc_block_elems.restype = _I
        lib.orc_fp32_to_fp16.argtypes = [c_float]
        lib.orc_fp32_to_fp16.restype = ctypes.c_uint16
        for q in ("orc_quantize_q8_0", "orc_quantize_q8_1", "orc_quantize_q8_k"):
            getattr(lib, q).argtypes = [_F, c_void_p, _I]
        lib.orc_dequantize.argtypes = [c_int, c_void_p, _F, _I]
        lib.orc_dot.argtypes = [c_int, c_void_p, c_void_p, _I]
        lib.orc_dot.restype = c_float
        lib.orc_act_kind.argtypes = [c_int]
        lib.orc_matmul_q.argtypes = [c_int, c_void_p, _I, _I, _F, _F, _I]
        _lib = lib
    return _lib


def _load_ref():
    global _ref, _ref_tried
    if not _ref_tried:
        _ref_tried = True
        path = os.path.join(_DIR, "_ref", "libnibble_ref.so")
        if os.path.exists(path):
            lib = ctypes.CDLL(path)
            lib.ref_rope.argtypes = [_F, _I, _I, _I, _I, c_float, c_int, _F]
            attn = [_F, _F, _F, _F, _I, _I, _I, _I, _I, _I, _I, _F]
            lib.ref_attention_scalar.argtypes = attn
            lib.ref_attention_simd.argtypes = attn
            lib.ref_kernel_set.restype = c_char_p
            lib.ref_backend_create.argtypes = [c_int]
            lib.ref_backend_create.restype = c_void_p
            lib.ref_backend_destroy.argtypes = [c_void_p]
            lib.ref_backend_destroy.restype = None
            lib.ref_backend_reserve.argtypes = [c_void_p, _I, _I, _I, _I]
            lib.ref_backend_attention.argtypes = [c_void_p, _F, _F, _F, _F, _I, _I, _I, _I, _I]
            lib.ref_backend_rope.argtypes = [c_void_p, _F, _I, _I, _I, _I, c_float, c_int, _F]
            lib.ref_matmul_scalar.argtypes = [c_int, c_void_p, _I, _I, _F, _F, _I]
            lib.ref_add_bias.argtypes = [_F, _F, _I, _I]
            lib.ref_embed.argtypes = [c_int, c_void_p, _I, _I, c_void_p, _I, _F]
            lib.ref_rmsnorm.argtypes = [_F, _F, _F, _I, _I, c_float]
            lib.ref_rmsnorm_simd.argtypes = [_F, _F, _F, _I, _I, c_float]
            lib.ref_add.argtypes = [_F, _F, _I]
            lib.ref_silu_mul.argtypes = [_F, _F, _I]
            lib.ref_silu_mul_simd.argtypes = [_F, _F, _I]
            lib.ref_quantize.argtypes = [c_int, _F, c_void_p, _I]
            lib.ref_dequantize.argtypes = [c_int, c_void_p, _F, _I]
            lib.ref_dot.argtypes = [c_int, c_void_p, c_void_p, _I]
            lib.ref_dot.restype = c_float
            lib.ref_backend_matmul.argtypes = [c_void_p, c_int, c_void_p, _I, _I, _F, _F, _I]
            _ref = lib
    return _ref


def have_ref() -> bool:
    return _load_ref() is not None


def have_avx2() -> bool:
    return bool(_load().orc_have_avx2())


def _fp(a):
    return a.ctypes.data_as(_F) if a is not None else None


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


# ---- our restatement ----

def rope(x, pos0, freq_base, neox, freq_factors=None):
    """In-place restatement of cpu::rope on x[n, heads, hd] (returns x)."""
    assert x.dtype == np.float32 and x.flags.c_contiguous and x.ndim == 3
    n, h, hd = x.shape
    ff = _f32(freq_factors) if freq_factors is not None else None
    _load().orc_rope(_fp(x), n, h, hd, pos0, freq_base, int(bool(neox)), _fp(ff))
    return x


def softmax_inplace(x):
    assert x.dtype == np.float32 and x.flags.c_contiguous
    _load().orc_softmax_inplace(_fp(x), x.size)
    return x


def _attn_args(q, k, v, pos0, n_kv_heads):
    q, k, v = _f32(q), _f32(k), _f32(v)
    n, h, hd = q.shape
    ctx = pos0 + n
    assert k.size >= ctx * n_kv_heads * hd and v.size >= ctx * n_kv_heads * hd
    return q, k, v, n, h, hd, ctx


def attention_scalar(q, k, v, pos0, n_kv_heads):
    """cpu::attention_heads restated (all heads). q[n,H,hd]; k,v[>=pos0+n, KV, hd]."""
    q, k, v, n, h, hd, ctx = _attn_args(q, k, v, pos0, n_kv_heads)
    out = np.zeros_like(q)
    sc = np.zeros(ctx, np.float32)
    _load().orc_attention_scalar(_fp(q), _fp(k), _fp(v), _fp(out), n, pos0, h, n_kv_heads, hd, 0, h, _fp(sc))
    return out


def attention_avx2(q, k, v, pos0, n_kv_heads):
    """simd::avx2::attention_heads restated (all heads); None when AVX2 is unavailable."""
    q, k, v, n, h, hd, ctx = _attn_args(q, k, v, pos0, n_kv_heads)
    out = np.zeros_like(q)
    sc = np.zeros(ctx, np.float32)
    rc = _load().orc_attention_avx2(_fp(q), _fp(k), _fp(v), _fp(out), n, pos0, h, n_kv_heads, hd, 0, h, _fp(sc))
    return out if rc == 0 else None


def attention_parallel(q, k, v, pos0, n_kv_heads, threads, use_avx2=True):
    """CpuBackend::attention restated: one task per head over `threads` threads."""
    q, k, v, n, h, hd, ctx = _attn_args(q, k, v, pos0, n_kv_heads)
    out = np.zeros_like(q)
    sc = np.zeros(ctx * h, np.float32)
    rc = _load().orc_attention_heads_parallel(_fp(q), _fp(k), _fp(v), _fp(out), n, pos0, h, n_kv_heads, hd,
                                              threads, int(use_avx2), _fp(sc))
    if rc != 0:
        raise RuntimeError("AVX2 requested but unavailable")
    return out


def attention_f64(q, k, v, pos0, n_kv_heads):
    q, k, v, n, h, hd, ctx = _attn_args(q, k, v, pos0, n_kv_heads)
    out = np.zeros(q.shape, np.float64)
    _load().orc_attention_f64(_fp(q), _fp(k), _fp(v), out.ctypes.data_as(_D), n, pos0, h, n_kv_heads, hd)
    return out


def exp_ps(x):
    x = _f32(x)
    y = np.empty_like(x)
    if _load().orc_exp_ps(_fp(x), _fp(y), x.size) != 0:
        return None
    return y


def llama3_freq_factors(head_dim, base, factor=32.0, low=1.0, high=4.0, orig_ctx=8192.0):
    out = np.zeros(head_dim // 2, np.float32)
    _load().orc_llama3_freq_factors(_fp(out), head_dim, base, factor, low, high, orig_ctx)
    return out


# ---- the compiled reference (oracle/_ref) ----

def ref_rope(x, pos0, freq_base, neox, freq_factors=None):
    lib = _load_ref()
    assert lib is not None and x.dtype == np.float32 and x.flags.c_contiguous
    n, h, hd = x.shape
    ff = _f32(freq_factors) if freq_factors is not None else None
    lib.ref_rope(_fp(x), n, h, hd, pos0, freq_base, int(bool(neox)), _fp(ff))
    return x


def ref_attention_scalar(q, k, v, pos0, n_kv_heads):
    lib = _load_ref()
    q, k, v, n, h, hd, ctx = _attn_args(q, k, v, pos0, n_kv_heads)
    out = np.zeros_like(q)
    sc = np.zeros(ctx, np.float32)
    lib.ref_attention_scalar(_fp(q), _fp(k), _fp(v), _fp(out), n, pos0, h, n_kv_heads, hd, 0, h, _fp(sc))
    return out


def ref_attention_simd(q, k, v, pos0, n_kv_heads):
    lib = _load_ref()
    q, k, v, n, h, hd, ctx = _attn_args(q, k, v, pos0, n_kv_heads)
    out = np.zeros_like(q)
    sc = np.zeros(ctx, np.float32)
    rc = lib.ref_attention_simd(_fp(q), _fp(k), _fp(v), _fp(out), n, pos0, h, n_kv_heads, hd, 0, h, _fp(sc))
    return out if rc == 0 else None


def _w_type(w) -> int:
    if w.dtype == np.float32:
        return 0
    if w.dtype == np.float16:
        return 1
    raise TypeError("float weights are float32 (F32) or float16 (F16)")


def matmul(w, x):
    """ref_ops.cpp:109-135 restated: y[n, out] = x[n, in] . W^T for W [out, in] float32 or float16, each dot
    accumulated left to right in float."""
    w = np.ascontiguousarray(w)
    x = _f32(x)
    out_, in_ = w.shape
    n = x.size // in_
    y = np.zeros((n, out_), np.float32)
    if _load().orc_matmul(_w_type(w), w.ctypes.data, in_, out_, _fp(x), _fp(y), n) != 0:
        raise ValueError("orc_matmul: bad weight type")
    return y


def matmul_f64(w, x):
    """Independent fp64 product of the same float32 / float16 inputs."""
    return np.asarray(x, np.float64).reshape(-1, w.shape[1]) @ np.asarray(w, np.float64).T


def fp16_to_fp32(h):
    """IEEE halves (uint16 array) to float32, bit-exact (NaN payloads kept)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.zeros(h.shape, np.float32)
    _load().orc_fp16_to_fp32_n(h.ctypes.data, _fp(out), h.size)
    return out


def add_bias(x, b):
    """ref_ops.cpp:154-160 restated: every row of x [n, d] += b [d], in place on a copy."""
    y = _f32(x).copy()
    b = _f32(b)
    _load().orc_add_bias(_fp(y), _fp(b), b.size, y.size // b.size)
    return y


def ref_matmul_scalar(w, x):
    """The compiled reference's cpu::matmul_rows (scalar float path)."""
    w = np.ascontiguousarray(w)
    x = _f32(x)
    out_, in_ = w.shape
    n = x.size // in_
    y = np.zeros((n, out_), np.float32)
    if _load_ref().ref_matmul_scalar(_w_type(w), w.ctypes.data, in_, out_, _fp(x), _fp(y), n) != 0:
        raise RuntimeError("ref_matmul_scalar failed")
    return y


def ref_add_bias(x, b):
    y = _f32(x).copy()
    b = _f32(b)
    _load_ref().ref_add_bias(_fp(y), _fp(b), b.size, y.size // b.size)
    return y


def embed(table, ids):
    """ref_ops.cpp:80-99 restated: rows ids of a float32 / float16 table [rows, d] as float32 [n, d]."""
    table = np.ascontiguousarray(table)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    rows, d = table.shape
    out = np.zeros((ids.size, d), np.float32)
    if _load().orc_embed(_w_type(table), table.ctypes.data, rows, d, ids.ctypes.data, ids.size, _fp(out)) != 0:
        raise ValueError("embed: token id out of range")
    return out


def rmsnorm(x, w, eps):
    """ref_ops.cpp:137-148 restated: rows of x [n, d] normalised with the double sum and scale, times w [d]."""
    x = _f32(x)
    w = _f32(w)
    y = np.zeros_like(x)
    _load().orc_rmsnorm(_fp(x), _fp(w), _fp(y), x.size // w.size, w.size, eps)
    return y


def add(x, y):
    """ref_ops.cpp:151-153 restated: x + y elementwise in float, on a copy of x."""
    out = _f32(x).copy()
    _load().orc_add(_fp(out), _fp(_f32(y)), out.size)
    return out


def silu_mul(gate, up):
    """ref_ops.cpp:217-222 restated: g / (1 + expf(-g)) * up, on a copy of gate."""
    out = _f32(gate).copy()
    _load().orc_silu_mul(_fp(out), _fp(_f32(up)), out.size)
    return out


def ref_embed(table, ids):
    table = np.ascontiguousarray(table)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    rows, d = table.shape
    out = np.zeros((ids.size, d), np.float32)
    if _load_ref().ref_embed(_w_type(table), table.ctypes.data, rows, d, ids.ctypes.data, ids.size, _fp(out)) != 0:
        raise ValueError("ref_embed: token id out of range")
    return out


def ref_rmsnorm(x, w, eps, simd=False):
    x = _f32(x)
    w = _f32(w)
    y = np.zeros_like(x)
    fn = _load_ref().ref_rmsnorm_simd if simd else _load_ref().ref_rmsnorm
    if fn(_fp(x), _fp(w), _fp(y), x.size // w.size, w.size, eps) != 0:
        raise RuntimeError("the reference has no SIMD tier on this host")
    return y


def ref_add(x, y):
    out = _f32(x).copy()
    _load_ref().ref_add(_fp(out), _fp(_f32(y)), out.size)
    return out


def ref_silu_mul(gate, up, simd=False):
    out = _f32(gate).copy()
    fn = _load_ref().ref_silu_mul_simd if simd else _load_ref().ref_silu_mul
    if fn(_fp(out), _fp(_f32(up)), out.size) != 0:
        raise RuntimeError("the reference has no SIMD tier on this host")
    return out


def ref_kernel_set() -> str:
    return _load_ref().ref_kernel_set().decode()


class RefCpuBackend:
    """The reference's ThreadPool + CpuBackend (compiled from its sources), for the CPU baseline."""

    def __init__(self, threads: int):
        lib = _load_ref()
        if lib is None:
            raise RuntimeError("oracle/_ref is not built")
        self._lib = lib
        self._h = lib.ref_backend_create(threads)
        if not self._h:
            raise RuntimeError("ref_backend_create failed")
        self.threads = threads

    def reserve(self, n_ctx, n_heads, max_rows, max_width):
        if self._lib.ref_backend_reserve(self._h, n_ctx, n_heads, max_rows, max_width) != 0:
            raise RuntimeError("reserve failed")

    def attention(self, q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim):
        rc = self._lib.ref_backend_attention(self._h, _fp(q), _fp(k), _fp(v), _fp(out), n, pos0, n_heads,
                                             n_kv_heads, head_dim)
        if rc != 0:
            raise RuntimeError("attention failed")

    def rope(self, x, n, n_heads, head_dim, pos0, base, neox, freq_factors=None):
        rc = self._lib.ref_backend_rope(self._h, _fp(x), n, n_heads, head_dim, pos0, base, int(bool(neox)),
                                        _fp(freq_factors))
        if rc != 0:
            raise RuntimeError("rope failed")

    def matmul(self, w, x):
        """CpuBackend::matmul: the production tier over the pool."""
        w = np.ascontiguousarray(w)
        x = _f32(x)
        out_, in_ = w.shape
        n = x.size // in_
        y = np.zeros((n, out_), np.float32)
        if self._lib.ref_backend_matmul(self._h, _w_type(w), w.ctypes.data, in_, out_, _fp(x), _fp(y), n) != 0:
            raise RuntimeError("matmul failed")
        return y

    def matmul_q(self, t, w, in_, out_, x):
        """CpuBackend::matmul for a quantized weight (raw row bytes): the production tier over the pool."""
        w = np.ascontiguousarray(w, np.uint8)
        x = _f32(x).reshape(-1, in_)
        y = np.zeros((x.shape[0], out_), np.float32)
        if self._lib.ref_backend_matmul(self._h, t, w.ctypes.data, in_, out_, _fp(x), _fp(y), x.shape[0]) != 0:
            raise RuntimeError("matmul failed")
        return y

    def close(self):
        if self._h:
            self._lib.ref_backend_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------- quantized formats (quant.c; src/quant.cpp)

# ggml type ids (src/tensor.h) and the activation kind each weight type pairs with (quant.h:7-12)
F32, F16, Q4_0, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 6, 7, 8, 12, 13, 14
QUANT_TYPES = (Q4_0, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K)
ACT_BYTES = {0: 34, 1: 36, 2: 292}  # Q8_0, Q8_1, Q8_K block bytes


def block_bytes(t):
    return int(_load().orc_block_bytes(t))


def block_elems(t):
    return int(_load().orc_block_elems(t))


def act_kind(t):
    return int(_load().orc_act_kind(t))


def fp32_to_fp16(f):
    return int(_load().orc_fp32_to_fp16(float(f)))


def quantize(kind, x):
    """quant.cpp:245-303: float row(s) x to Q8_0 (kind 0), Q8_1 (1) or Q8_K (2) block bytes (uint8 array)."""
    x = _f32(x).reshape(-1)
    per = 32 if kind < 2 else 256
    out = np.zeros(x.size // per * ACT_BYTES[kind], np.uint8)
    fn = (_load().orc_quantize_q8_0, _load().orc_quantize_q8_1, _load().orc_quantize_q8_k)[kind]
    if fn(_fp(x), out.ctypes.data, x.size) != 0:
        raise ValueError("quantize: length is not a multiple of the block size")
    return out


def dequantize(t, raw, n):
    """quant.cpp:157-242: n elements of type t from raw bytes."""
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.zeros(n, np.float32)
    if _load().orc_dequantize(t, raw.ctypes.data, _fp(out), n) != 0:
        raise ValueError("dequantize: bad type or length")
    return out


def dot(t, w, a, nb):
    """quant.cpp:305-419: block dot of weight blocks w (type t) with activation blocks a, nb blocks."""
    w = np.ascontiguousarray(w, np.uint8)
    a = np.ascontiguousarray(a, np.uint8)
    return np.float32(_load().orc_dot(t, w.ctypes.data, a.ctypes.data, nb))


def matmul_q(t, w, in_, out_, x):
    """ref_ops.cpp:109-135 for quantized weights: y[n, out] from raw weight rows (out rows of in_ elements)."""
    w = np.ascontiguousarray(w, np.uint8)
    x = _f32(x).reshape(-1, in_)
    y = np.zeros((x.shape[0], out_), np.float32)
    if _load().orc_matmul_q(t, w.ctypes.data, in_, out_, _fp(x), _fp(y), x.shape[0]) != 0:
        raise ValueError("matmul_q: bad type or width")
    return y


def ref_quantize(kind, x):
    x = _f32(x).reshape(-1)
    per = 32 if kind < 2 else 256
    out = np.zeros(x.size // per * ACT_BYTES[kind], np.uint8)
    if _load_ref().ref_quantize(kind, _fp(x), out.ctypes.data, x.size) != 0:
        raise ValueError("ref_quantize failed")
    return out


def ref_dequantize(t, raw, n):
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.zeros(n, np.float32)
    if _load_ref().ref_dequantize(t, raw.ctypes.data, _fp(out), n) != 0:
        raise ValueError("ref_dequantize failed")
    return out


def ref_dot(t, w, a, nb):
    w = np.ascontiguousarray(w, np.uint8)
    a = np.ascontiguousarray(a, np.uint8)
    return np.float32(_load_ref().ref_dot(t, w.ctypes.data, a.ctypes.data, nb))
