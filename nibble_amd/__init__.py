"""nibble_amd: nibble's attention path (QKV projection, RoPE, KV-cache append, causal GQA attention) on one MI355X.

The product is libnibble_hip.so: hand-written HIP kernels for gfx950 behind a C++20 HipBackend that implements
nibble's Backend operator interface (reference src/backend/backend.h:36-71), exported through the C ABI in
include/nibble_hip.h. This module binds that ABI with ctypes for Python callers (tests, benchmarks). There is no
fallback: if the library is missing or a call fails, it raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, byref, c_char_p, c_float, c_int, c_int64, c_uint32, c_uint64, c_void_p

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "libnibble_hip.so")

_F = POINTER(c_float)
_I = c_int64

# ggml type ids of the weight types the GPU backend takes (src/tensor.h:21-31 in the reference).
F32, F16, Q4_0, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 6, 7, 8, 12, 13, 14
QUANT_TYPES = (Q4_0, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K)


class NbhTensor(ctypes.Structure):
    """nbh_tensor: a weight view, field for field nibble::Tensor."""
    _fields_ = [("type", c_uint32), ("n_dims", ctypes.c_int32), ("ne", c_int64 * 4), ("data", c_void_p)]

# Every function the C ABI exports, with its ctypes signature (restype, argtypes).
_SIGNATURES = {
    "nbh_last_error": (c_char_p, []),
    "nbh_backend_create": (c_int, [c_int, POINTER(c_void_p)]),
    "nbh_backend_destroy": (None, [c_void_p]),
    "nbh_backend_supports": (c_int, [c_void_p, c_uint32, POINTER(c_int)]),
    "nbh_backend_reserve": (c_int, [c_void_p, _I, _I, _I, _I]),
    "nbh_backend_alloc": (c_int, [c_void_p, _I, POINTER(c_void_p)]),
    "nbh_backend_free": (c_int, [c_void_p, c_void_p]),
    "nbh_backend_read": (c_int, [c_void_p, c_void_p, c_void_p, _I]),
    "nbh_backend_write": (c_int, [c_void_p, c_void_p, c_void_p, _I]),
    "nbh_backend_copy": (c_int, [c_void_p, c_void_p, c_void_p, _I]),
    "nbh_backend_rope": (c_int, [c_void_p, c_void_p, _I, _I, _I, _I, c_float, c_int, c_void_p]),
    "nbh_backend_attention": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, _I, _I, _I, _I, _I]),
    "nbh_backend_append_rope": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, _I, _I, _I, _I,
                                        _I, c_float, c_int, c_void_p]),
    "nbh_backend_append_rope_attention": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                                  c_void_p, _I, _I, _I, _I, _I, c_float, c_int, c_void_p]),
    "nbh_backend_attention_f16kv": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, _I, _I, _I, _I, _I]),
    "nbh_backend_append_rope_attention_f16kv": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                                        c_void_p, _I, _I, _I, _I, _I, c_float, c_int, c_void_p]),
    "nbh_backend_attention_batch": (c_int, [c_void_p, _I, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, _I, _I,
                                            _I]),
    "nbh_backend_append_rope_attention_batch": (c_int, [c_void_p, _I, c_void_p, c_void_p, c_void_p, c_void_p,
                                                        c_void_p, c_void_p, c_void_p, _I, _I, _I, c_float, c_int,
                                                        c_void_p]),
    "nbh_backend_matmul": (c_int, [c_void_p, POINTER(NbhTensor), c_void_p, c_void_p, _I]),
    "nbh_backend_matmul_multi": (c_int, [c_void_p, _I, c_void_p, c_void_p, c_void_p, _I]),
    "nbh_backend_add_bias": (c_int, [c_void_p, c_void_p, POINTER(NbhTensor), _I]),
    "nbh_backend_release_weights": (c_int, [c_void_p]),
    "nbh_backend_set_attention_fp32": (c_int, [c_void_p, c_int]),
    "nbh_backend_set_batch_invariant": (c_int, [c_void_p, c_int]),
    "nbh_backend_prefill_recomputed": (c_int, [c_void_p, POINTER(c_int64)]),
    "nbh_backend_stream": (c_int, [c_void_p, POINTER(c_void_p)]),
    "nbh_attention_decode_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, _I, _I, _I, _I, _I, c_void_p]),
    "nbh_backend_embed": (c_int, [c_void_p, POINTER(NbhTensor), c_void_p, _I, c_void_p]),
    "nbh_backend_rmsnorm": (c_int, [c_void_p, c_void_p, POINTER(NbhTensor), c_void_p, _I, c_float]),
    "nbh_backend_add": (c_int, [c_void_p, c_void_p, c_void_p, _I]),
    "nbh_backend_silu_mul": (c_int, [c_void_p, c_void_p, c_void_p, _I]),
    "nbh_backend_weight_bytes": (c_int, [c_void_p, POINTER(c_int64)]),
    "nbh_backend_reserve_attention": (c_int, [c_void_p, _I, _I]),
    "nbh_backend_reserve_rope": (c_int, [c_void_p, _I, c_float, c_int, c_void_p]),
    "nbh_backend_sync": (c_int, [c_void_p]),
    "nbh_backend_live_allocations": (c_int, [c_void_p, POINTER(c_int64)]),
    "nbh_backend_internal_bytes": (c_int, [c_void_p, POINTER(c_int64)]),
    "nbh_backend_cu_count": (c_int, [c_void_p, POINTER(c_int)]),
    "nbh_backend_fill_normal": (c_int, [c_void_p, c_void_p, _I, c_uint64, c_float]),
    "nbh_event_create": (c_int, [c_void_p, POINTER(c_void_p)]),
    "nbh_event_record": (c_int, [c_void_p, c_void_p]),
    "nbh_event_elapsed_ms": (c_int, [c_void_p, c_void_p, POINTER(c_float)]),
    "nbh_event_destroy": (None, [c_void_p]),
}

_lib = None


def _batch_arrays(pointer_lists, pos0):
    """Host arrays for a batch call: one c_void_p array per list of device pointers, and the positions as int64.
    The arrays are returned so that they outlive the call."""
    n = len(pos0)
    if any(len(x) != n for x in pointer_lists):
        raise BackendError("batch: every pointer list must hold one entry per position")
    arrs = [(c_void_p * max(n, 1))(*[int(x) for x in lst]) for lst in pointer_lists]
    pa = (c_int64 * max(n, 1))(*[int(x) for x in pos0])
    return n, arrs, pa


class BackendError(RuntimeError):
    """A call into libnibble_hip.so failed (nibble::Error on the C++ side)."""


def lib():
    """The loaded libnibble_hip.so. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                               "(there is no CPU fallback for the HIP backend)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(rc: int):
    if rc != 0:
        raise BackendError(lib().nbh_last_error().decode(errors="replace"))


def _host_ptr(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(c_void_p)


class DevicePtr(int):
    """A device address handed out by HipBackend.alloc (float*); supports pointer arithmetic in floats via +."""

    def at(self, floats: int) -> "DevicePtr":
        return DevicePtr(int(self) + 4 * int(floats))


def weight(w, shape=None, dtype=None) -> NbhTensor:
    """An nbh_tensor for a weight: a 2-D (or 1-D) float32/float16 host array; raw block bytes (a uint8 host array)
    with the (rows, ne0) shape and a quantized type id; or a DevicePtr into a buffer of this backend with its shape
    and type (F32 or F16)."""
    if isinstance(w, NbhTensor):
        return w
    if hasattr(w, "nbh_tensor"):
        return w.nbh_tensor()
    if isinstance(w, np.ndarray) and dtype is not None:
        assert w.flags.c_contiguous and shape is not None
        ne = [int(shape[-1]), int(shape[0]) if len(shape) > 1 else 1, 1, 1]
        t = NbhTensor(dtype, len(shape), (c_int64 * 4)(*ne), c_void_p(w.ctypes.data))
        t._host = w  # the view points into w: the array lives as long as the tensor (uploads happen at first use)
        return t
    if isinstance(w, np.ndarray):
        if w.dtype == np.float32:
            t = F32
        elif w.dtype == np.float16:
            t = F16
        else:
            raise BackendError(f"weight dtype {w.dtype}: the GPU matmul takes float32 and float16")
        assert w.flags.c_contiguous
        shape, data = w.shape, w.ctypes.data
    else:
        if shape is None or dtype is None:
            raise BackendError("a device weight needs its shape and type")
        t, data = dtype, int(w)
    ne = [int(shape[-1]), int(shape[0]) if len(shape) > 1 else 1, 1, 1]
    out = NbhTensor(t, len(shape), (c_int64 * 4)(*ne), c_void_p(data))
    if isinstance(w, np.ndarray):
        out._host = w  # as above: a host view keeps its array alive
    return out


class HipBackend:
    """Python face of nibble::hip::HipBackend (the reference's Backend interface on one gfx950 GPU)."""

    def __init__(self, device: int = 0):
        h = c_void_p()
        _check(lib().nbh_backend_create(device, byref(h)))
        self._h = h
        # Host weight arrays whose device copies the backend keeps (by address): held here so that no other array
        # takes their address while the copy is live.
        self._kept = {}

    # -- Backend members (backend.h:36-71) --
    def supports(self, dtype: int) -> bool:
        out = c_int()
        _check(lib().nbh_backend_supports(self._h, dtype, byref(out)))
        return bool(out.value)

    def reserve(self, n_ctx: int, n_heads: int, max_rows: int, max_width: int):
        _check(lib().nbh_backend_reserve(self._h, n_ctx, n_heads, max_rows, max_width))

    def alloc(self, n_floats: int) -> DevicePtr:
        p = c_void_p()
        _check(lib().nbh_backend_alloc(self._h, n_floats, byref(p)))
        return DevicePtr(p.value)

    def free(self, p):
        _check(lib().nbh_backend_free(self._h, c_void_p(int(p)) if p else None))

    def read(self, src, n: int, out: np.ndarray | None = None) -> np.ndarray:
        if out is None:
            out = np.empty(n, np.float32)
        assert out.dtype == np.float32 and out.size >= n
        _check(lib().nbh_backend_read(self._h, _host_ptr(out), c_void_p(int(src)), n))
        return out

    def write(self, dst, host: np.ndarray):
        host = np.ascontiguousarray(host, dtype=np.float32)
        _check(lib().nbh_backend_write(self._h, c_void_p(int(dst)), _host_ptr(host), host.size))

    def copy(self, dst, src, count: int):
        _check(lib().nbh_backend_copy(self._h, c_void_p(int(dst)), c_void_p(int(src)), count))

    def rope(self, x, n, n_heads, head_dim, pos0, freq_base, neox, freq_factors=None):
        ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)
        _check(lib().nbh_backend_rope(self._h, c_void_p(int(x)), n, n_heads, head_dim, pos0, freq_base, int(bool(neox)),
                                      None if ff is None else _host_ptr(ff)))

    def attention(self, q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim):
        _check(lib().nbh_backend_attention(self._h, c_void_p(int(q)), c_void_p(int(k)), c_void_p(int(v)),
                                           c_void_p(int(out)), n, pos0, n_heads, n_kv_heads, head_dim))

    # -- HIP-only extensions --
    def append_rope(self, q, k_cache, v_cache, k_new, v_new, n, pos0, n_heads, n_kv_heads, head_dim, freq_base,
                    neox, freq_factors=None):
        ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)
        _check(lib().nbh_backend_append_rope(self._h, c_void_p(int(q)), c_void_p(int(k_cache)),
                                             c_void_p(int(v_cache)), c_void_p(int(k_new)), c_void_p(int(v_new)), n,
                                             pos0, n_heads, n_kv_heads, head_dim, freq_base, int(bool(neox)),
                                             None if ff is None else _host_ptr(ff)))

    def append_rope_attention(self, q, k_cache, v_cache, k_new, v_new, out, n, pos0, n_heads, n_kv_heads, head_dim,
                              freq_base, neox, freq_factors=None):
        """append_rope then attention in one call, q read unrotated and left unchanged (bit-identical results)."""
        ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)
        _check(lib().nbh_backend_append_rope_attention(
            self._h, c_void_p(int(q)), c_void_p(int(k_cache)), c_void_p(int(v_cache)), c_void_p(int(k_new)),
            c_void_p(int(v_new)), c_void_p(int(out)), n, pos0, n_heads, n_kv_heads, head_dim, freq_base,
            int(bool(neox)), None if ff is None else _host_ptr(ff)))

    def attention_f16kv(self, q, k16, v16, out, n, pos0, n_heads, n_kv_heads, head_dim):
        """attention over fp16 caches k16, v16 (_Float16 [rows, n_kv_heads, head_dim] in buffers from alloc; a
        buffer of f floats holds 2f halves), q already rotated. head_dim 64 or 128."""
        _check(lib().nbh_backend_attention_f16kv(self._h, c_void_p(int(q)), c_void_p(int(k16)), c_void_p(int(v16)),
                                                 c_void_p(int(out)), n, pos0, n_heads, n_kv_heads, head_dim))

    def append_rope_attention_f16kv(self, q, k16, v16, k_new, v_new, out, n, pos0, n_heads, n_kv_heads, head_dim,
                                    freq_base, neox, freq_factors=None):
        """append_rope_attention over fp16 caches: rows pos0.. receive fp16(rope(k_new)) and fp16(v_new)."""
        ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)
        _check(lib().nbh_backend_append_rope_attention_f16kv(
            self._h, c_void_p(int(q)), c_void_p(int(k16)), c_void_p(int(v16)), c_void_p(int(k_new)),
            c_void_p(int(v_new)), c_void_p(int(out)), n, pos0, n_heads, n_kv_heads, head_dim, freq_base,
            int(bool(neox)), None if ff is None else _host_ptr(ff)))

    def attention_batch(self, q, k_cache, v_cache, out, pos0, n_heads, n_kv_heads, head_dim):
        """Ragged batch of single-token decodes: sequence i is attention(q[i], k_cache[i], v_cache[i], out[i], 1,
        pos0[i], ...) over its own caches; the lists hold device pointers, pos0 positions."""
        n, arrs, pa = _batch_arrays([q, k_cache, v_cache, out], pos0)
        _check(lib().nbh_backend_attention_batch(self._h, n, *arrs, pa, n_heads, n_kv_heads, head_dim))

    def append_rope_attention_batch(self, q, k_cache, v_cache, k_new, v_new, out, pos0, n_heads, n_kv_heads,
                                    head_dim, freq_base, neox, freq_factors=None):
        """append_rope_attention with n = 1 for every sequence of a ragged batch, in one launch pair."""
        n, arrs, pa = _batch_arrays([q, k_cache, v_cache, k_new, v_new, out], pos0)
        ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)
        _check(lib().nbh_backend_append_rope_attention_batch(self._h, n, *arrs, pa, n_heads, n_kv_heads, head_dim,
                                                             freq_base, int(bool(neox)),
                                                             None if ff is None else _host_ptr(ff)))

    def _tensor(self, w, shape=None, dtype=None) -> NbhTensor:
        if isinstance(w, np.ndarray):
            self._kept[w.ctypes.data] = w
        elif hasattr(w, "nbh_tensor"):  # an object holding raw blocks (keeps its array alive through us)
            self._kept[id(w)] = w
        return weight(w, shape, dtype)

    def matmul(self, w, x, y, n: int, shape=None, dtype=None):
        """y[n, rows] = x[n, ne0] . W^T; w a host array (float32/float16) or a DevicePtr with shape and dtype."""
        t = self._tensor(w, shape, dtype)
        _check(lib().nbh_backend_matmul(self._h, byref(t), c_void_p(int(x)), c_void_p(int(y)), n))

    def matmul_multi(self, ws, x, ys, n: int):
        """ys[i] = matmul(ws[i], x, n) for host weight arrays (or NbhTensor views) sharing the input x."""
        ts = [w if isinstance(w, NbhTensor) else self._tensor(w) for w in ws]
        tp = (c_void_p * len(ts))(*[ctypes.addressof(t) for t in ts])
        yp = (c_void_p * len(ys))(*[int(y) for y in ys])
        _check(lib().nbh_backend_matmul_multi(self._h, len(ts), tp, c_void_p(int(x)), yp, n))

    def add_bias(self, x, bias, n: int):
        """Each of the n rows of x += bias (a float32 host array or an NbhTensor)."""
        t = bias if isinstance(bias, NbhTensor) else self._tensor(np.ascontiguousarray(bias, dtype=np.float32))
        _check(lib().nbh_backend_add_bias(self._h, c_void_p(int(x)), byref(t), n))

    def embed(self, table, ids, out):
        """out[t, :] = row ids[t] of table (a float32/float16 host array or an NbhTensor); ids host int32."""
        t = table if isinstance(table, NbhTensor) else self._tensor(table)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        _check(lib().nbh_backend_embed(self._h, byref(t), _host_ptr(ids), ids.size, c_void_p(int(out))))

    def rmsnorm(self, x, weight, y, n: int, eps: float):
        t = weight if isinstance(weight, NbhTensor) else self._tensor(np.ascontiguousarray(weight, dtype=np.float32))
        _check(lib().nbh_backend_rmsnorm(self._h, c_void_p(int(x)), byref(t), c_void_p(int(y)), n, eps))

    def add(self, x, y, count: int):
        _check(lib().nbh_backend_add(self._h, c_void_p(int(x)), c_void_p(int(y)), count))

    def silu_mul(self, gate, up, count: int):
        _check(lib().nbh_backend_silu_mul(self._h, c_void_p(int(gate)), c_void_p(int(up)), count))

    def set_attention_fp32(self, on: bool):
        """Every attention row on the fp32 kernels (on) or the default fp16-operand MFMA prefill (off)."""
        _check(lib().nbh_backend_set_attention_fp32(self._h, int(bool(on))))

    def set_batch_invariant(self, on: bool):
        """Results bitwise independent of how rows are batched into calls (on): the ordered fp32 attention route and
        the gemv kernel for every float matmul; off (default): the faster routes, equal within rounding."""
        _check(lib().nbh_backend_set_batch_invariant(self._h, int(bool(on))))

    def stream_handle(self) -> int:
        """The hipStream_t (as an integer) the backend's ops run on."""
        v = c_void_p(None)
        _check(lib().nbh_backend_stream(self._h, ctypes.byref(v)))
        return int(v.value or 0)

    def prefill_recomputed(self) -> int:
        """Row tiles the last MFMA prefill call recomputed with split operands (waits for queued work)."""
        v = c_int64(0)
        _check(lib().nbh_backend_prefill_recomputed(self._h, ctypes.byref(v)))
        return int(v.value)

    def release_weights(self):
        _check(lib().nbh_backend_release_weights(self._h))
        self._kept.clear()

    def weight_bytes(self) -> int:
        out = c_int64()
        _check(lib().nbh_backend_weight_bytes(self._h, byref(out)))
        return out.value

    def reserve_attention(self, n_kv_heads: int, head_dim: int):
        _check(lib().nbh_backend_reserve_attention(self._h, n_kv_heads, head_dim))

    def reserve_rope(self, head_dim, freq_base, neox, freq_factors=None):
        ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)
        _check(lib().nbh_backend_reserve_rope(self._h, head_dim, freq_base, int(bool(neox)),
                                              None if ff is None else _host_ptr(ff)))

    def sync(self):
        _check(lib().nbh_backend_sync(self._h))

    def live_allocations(self) -> int:
        out = c_int64()
        _check(lib().nbh_backend_live_allocations(self._h, byref(out)))
        return out.value

    def internal_bytes(self) -> int:
        out = c_int64()
        _check(lib().nbh_backend_internal_bytes(self._h, byref(out)))
        return out.value

    def cu_count(self) -> int:
        out = c_int()
        _check(lib().nbh_backend_cu_count(self._h, byref(out)))
        return out.value

    def fill_normal(self, dst, count: int, seed: int, scale: float = 1.0):
        _check(lib().nbh_backend_fill_normal(self._h, c_void_p(int(dst)), count, seed & (2**64 - 1), scale))

    # -- convenience --
    def upload(self, host: np.ndarray) -> DevicePtr:
        host = np.ascontiguousarray(host, dtype=np.float32)
        p = self.alloc(host.size)
        self.write(p, host)
        return p

    def download(self, src, shape) -> np.ndarray:
        n = int(np.prod(shape))
        return self.read(src, n).reshape(shape)

    def event(self) -> "Event":
        return Event(self)

    def close(self):
        if getattr(self, "_h", None):
            lib().nbh_backend_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def attention_decode_noalloc(q, k, v, out, n, pos0, n_heads, n_kv_heads, head_dim, stream=None):
    """The decode route of HipBackend.attention with no allocation (nbh_attention_decode_noalloc): device pointers,
    the current device, `stream` a hipStream_t handle or None for the null stream."""
    _check(lib().nbh_attention_decode_noalloc(c_void_p(int(q)), c_void_p(int(k)), c_void_p(int(v)),
                                              c_void_p(int(out)), n, pos0, n_heads, n_kv_heads, head_dim,
                                              c_void_p(stream) if stream else None))


def mfma_loop(out, iters: int, waves_per_simd: int, cu_count: int):
    """MFMA calibration launch (nbhs_mfma_loop_f16) on the null stream: cu_count * waves_per_simd workgroups of four
    waves, each wave issuing iters x 8 independent 32x32x16 fp16 MFMAs; `out` holds cu_count * waves_per_simd * 256
    floats. Returns the launch's FLOPs."""
    L = lib()
    L.nbhs_mfma_loop_f16.argtypes = [c_void_p, c_int64, c_int, c_int, c_void_p]
    L.nbhs_mfma_loop_f16.restype = c_int
    _check(L.nbhs_mfma_loop_f16(c_void_p(int(out)), iters, waves_per_simd, cu_count, None))
    return cu_count * waves_per_simd * 4 * iters * 8 * 32768


class KernelTiming:
    """Live per-kernel device durations from the shim's launch bracketing (nbhs_kernel_timing_*,
    include/nibble_hip_shim.h). Used by the benchmark for roofline figures."""

    (ROPE, APPEND_ROPE, DECODE_PARTIAL, DECODE_COMBINE, GENERIC, STAGE_KV, PREFILL_MFMA, GEMV, CONVERT, ADD_BIAS, RMSNORM,
     ELEMENTWISE, QUANTIZE, QGEMV, QGEMM, PREFILL_PRECISE, CALIBRATION, SPLIT_ACTS, GEMM, GEMM_REDUCE) = range(20)

    @staticmethod
    def enable(on: bool = True, only: int | None = None):
        """Time every kernel (on), none (not on), or - with `only` - that one kernel alone."""
        L = lib()
        L.nbhs_kernel_timing_select.argtypes = [ctypes.c_uint32]
        L.nbhs_kernel_timing_select.restype = c_int
        mask = 0 if not on else (1 << only if only is not None else 0xFFFFFFFF)
        if L.nbhs_kernel_timing_select(mask) != 0:
            raise BackendError("nbhs_kernel_timing_select failed")

    @staticmethod
    def read(kernel: int) -> tuple[float, int]:
        """(total milliseconds, launches) recorded for `kernel` since the last read; clears them."""
        L = lib()
        L.nbhs_kernel_timing_read.argtypes = [c_int, POINTER(ctypes.c_double), POINTER(c_int64)]
        L.nbhs_kernel_timing_read.restype = c_int
        total, count = ctypes.c_double(), c_int64()
        rc = L.nbhs_kernel_timing_read(kernel, byref(total), byref(count))
        if rc != 0:
            raise BackendError(f"nbhs_kernel_timing_read failed ({rc})")
        return total.value, count.value


class Event:
    """A HIP event on the backend's stream."""

    def __init__(self, be: HipBackend):
        h = c_void_p()
        _check(lib().nbh_event_create(be._h, byref(h)))
        self._be = be
        self._h = h

    def record(self):
        _check(lib().nbh_event_record(self._be._h, self._h))
        return self

    def elapsed_ms(self, end: "Event") -> float:
        ms = c_float()
        _check(lib().nbh_event_elapsed_ms(self._h, end._h, byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self._h:
                lib().nbh_event_destroy(self._h)
        except Exception:
            pass
