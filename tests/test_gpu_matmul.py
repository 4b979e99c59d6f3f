"""GPU parity of the QKV projection (Backend::matmul / matmul_multi / add_bias) against the CPU oracle.

The reference's float matmul (ref_ops.cpp:109-135) accumulates each dot product left to right in float; the GPU
sums the same float products in another order (lane partials and a wave tree on the gemv route; on the F16-weight
GEMM route each activation row is scaled by a power of two and split into fp16 hi + lo parts whose exact products
with the fp16 weights accumulate in fp32 on MFMA; rocBLAS sgemm's blocking for F32 weights). Both stay within the classical bound for float summation of the same terms, so the test bound
is, per output element,
    |gpu - exact| <= in * 2^-24 * sum_k |x_k w_k|      (exact = fp64 product of the same float inputs)
    |gpu - ref|   <= 2 * in * 2^-24 * sum_k |x_k w_k|  (ref = the restated reference, bit-exact to it on the CPU)
A dropped, repeated or misplaced term moves an element by about one term, |x_k w_k| ~ sum/in, several times the
bound at these widths. add_bias is one float add per element and is compared bitwise, as are results that must be
the same computation (matmul_multi against separate calls, device-resident against host weights).
"""
import numpy as np
import pytest

import nibble_amd
import oracle
from nibble_amd import configs
from tests.gpu_util import Buffers, bits

pytestmark = pytest.mark.gpu
U = 2.0 ** -24


def rand(rng, shape, dtype=np.float32, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(dtype)


def assert_matmul_close(got, w, x, what=""):
    """got [n, out] against the exact product and the restated reference, within the summation bound."""
    in_ = w.shape[1]
    x2 = np.asarray(x, np.float32).reshape(-1, in_)
    exact = oracle.matmul_f64(w, x2)
    ref = oracle.matmul(w, x2)
    absdot = np.abs(x2.astype(np.float64)) @ np.abs(np.asarray(w, np.float64)).T
    bound = in_ * U * absdot + 1e-37
    e_exact = np.abs(got.astype(np.float64) - exact)
    e_ref = np.abs(got.astype(np.float64) - ref)
    worst = float(np.max(e_exact / bound))
    print(f"matmul {what}: max |gpu-exact|/bound = {worst:.3f}, max |gpu-ref| = {float(e_ref.max()):.3e}", flush=True)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    assert np.all(e_exact <= bound), f"{what}: {int(np.sum(e_exact > bound))} elements beyond the summation bound"
    assert np.all(e_ref <= 2 * bound), f"{what}: {int(np.sum(e_ref > 2 * bound))} elements beyond 2x the bound vs ref"


def gpu_matmul(be, w, x, n):
    out_ = w.shape[0]
    with Buffers(be) as B:
        dx, dy = B.upload(x), B.alloc(n * out_)
        be.matmul(w, dx, dy, n)
        return be.download(dy, (n, out_))


@pytest.mark.parametrize("dtype", [np.float32, np.float16], ids=["f32", "f16"])
@pytest.mark.parametrize("in_out", [(256, 96), (200, 40), (100, 33)], ids=["256x96", "200x40", "100x33-unaligned"])
@pytest.mark.parametrize("n", [1, 2, 7, 16, 17, 64, 65, 200])
def test_matmul_matches_reference(backend, dtype, in_out, n):
    """Both routes (gemv for n <= 16, n <= 11 for F16 weights; GEMM above) and both weight types, aligned
    (in % 8 == 0) and not; partial row, output and K tiles of the F16 GEMM (64 x 64 tiles, 64-deep slices: in 200 ends mid-slice, in 100 is not a
    multiple of 8 and takes the fp32 route)."""
    in_, out_ = in_out
    rng = np.random.default_rng(1000 * n + in_ + out_)
    w = rand(rng, (out_, in_), dtype, 0.5)
    x = rand(rng, (n, in_))
    got = gpu_matmul(backend, w, x, n)
    assert_matmul_close(got, w, x, f"{np.dtype(dtype).name} {in_}x{out_} n={n}")
    backend.release_weights()


@pytest.mark.parametrize("shape", [configs.LLAMA32_1B, configs.QWEN25_05B, configs.TINYLLAMA_11B],
                         ids=lambda s: s.name)
@pytest.mark.parametrize("n", [1, 5, 16, 300])
def test_qkv_projection_into_cache_rows(backend, shape, n):
    """transformer.cpp:171-194: q, and K/V projected straight into cache rows pos0..pos0+n-1 (+ biases for qwen2),
    F16 weights at the model's real widths. Cache rows outside the window keep their bits."""
    E, Q, kvw = shape.n_embd, shape.n_heads * shape.head_dim, shape.n_kv_heads * shape.head_dim
    pos0, n_ctx = 37, 400
    rng = np.random.default_rng(n + E)
    wq, wk, wv = (rand(rng, (r, E), np.float16, 0.05) for r in (Q, kvw, kvw))
    bq, bk, bv = (rand(rng, (r,), np.float32, 0.1) for r in (Q, kvw, kvw))
    x = rand(rng, (n, E))
    kc0, vc0 = rand(rng, (n_ctx, kvw)), rand(rng, (n_ctx, kvw))
    with Buffers(backend) as B:
        dx, dq, dk, dv = B.upload(x), B.alloc(n * Q), B.upload(kc0), B.upload(vc0)
        kc, vc = dk.at(pos0 * kvw), dv.at(pos0 * kvw)
        backend.matmul_multi([wq, wk, wv], dx, [dq, kc, vc], n)
        q_mm = backend.download(dq, (n, Q))
        k_all, v_all = backend.download(dk, (n_ctx, kvw)), backend.download(dv, (n_ctx, kvw))
        if shape.qkv_bias:
            backend.add_bias(dq, bq, n)
            backend.add_bias(kc, bk, n)
            backend.add_bias(vc, bv, n)
            q_b = backend.download(dq, (n, Q))
            k_b, v_b = backend.download(dk, (n_ctx, kvw)), backend.download(dv, (n_ctx, kvw))
        # matmul_multi equals separate matmul calls (backend.h:57), bit for bit
        dq2, dk2, dv2 = B.alloc(n * Q), B.alloc(n * kvw), B.alloc(n * kvw)
        for w, y in ((wq, dq2), (wk, dk2), (wv, dv2)):
            backend.matmul(w, dx, y, n)
        sep = [backend.download(dq2, (n, Q)), backend.download(dk2, (n, kvw)), backend.download(dv2, (n, kvw))]
    win = slice(pos0, pos0 + n)
    for got, w, name in ((q_mm, wq, "q"), (k_all[win], wk, "k"), (v_all[win], wv, "v")):
        assert_matmul_close(got, w, x, f"{shape.name} n={n} {name}")
    for a, b, name in ((q_mm, sep[0], "q"), (k_all[win], sep[1], "k"), (v_all[win], sep[2], "v")):
        assert np.array_equal(bits(a), bits(b)), f"matmul_multi {name} differs from a separate matmul"
    outside = np.ones(n_ctx, bool)
    outside[win] = False
    assert np.array_equal(bits(k_all[outside]), bits(kc0[outside])), "K cache rows outside the window changed"
    assert np.array_equal(bits(v_all[outside]), bits(vc0[outside])), "V cache rows outside the window changed"
    if shape.qkv_bias:
        assert np.array_equal(bits(q_b), bits(oracle.add_bias(q_mm, bq))), "add_bias q not bit-exact"
        assert np.array_equal(bits(k_b[win]), bits(oracle.add_bias(k_all[win], bk))), "add_bias k not bit-exact"
        assert np.array_equal(bits(v_b[win]), bits(oracle.add_bias(v_all[win], bv))), "add_bias v not bit-exact"
        assert np.array_equal(bits(k_b[outside]), bits(kc0[outside])), "add_bias touched rows outside the window"
    backend.release_weights()


@pytest.mark.parametrize("n", [3, 16, 40, 512])
def test_device_resident_weights_match_host_weights(backend, n):
    """Weights inside a buffer from alloc() are used in place. F32 ones run the same kernels on the same bytes as
    host weights, so the same bits; so do F16 ones, the gemv for n <= 11 and the F16 GEMM above (which reads the
    weight as fp16, so an in-place weight needs no widened copy)."""
    rng = np.random.default_rng(77 + n)
    in_, out_ = 256, 72
    w32 = rand(rng, (out_, in_), np.float32, 0.3)
    w16 = rand(rng, (out_, in_), np.float16, 0.3)
    x = rand(rng, (n, in_))
    with Buffers(backend) as B:
        dx = B.upload(x)
        dw32 = B.upload(w32)
        dw16 = B.upload(w16.view(np.float32))  # the halves' bytes, carried as floats
        y = [B.alloc(n * out_) for _ in range(4)]
        backend.matmul(w32, dx, y[0], n)
        backend.matmul(dw32, dx, y[1], n, shape=w32.shape, dtype=nibble_amd.F32)
        backend.matmul(w16, dx, y[2], n)
        backend.matmul(dw16, dx, y[3], n, shape=w16.shape, dtype=nibble_amd.F16)
        got = [backend.download(p, (n, out_)) for p in y]
    assert np.array_equal(bits(got[0]), bits(got[1])), "F32: device-resident weight differs from host weight"
    assert np.array_equal(bits(got[2]), bits(got[3])), "F16: device-resident weight differs from host weight"
    assert_matmul_close(got[2], w16, x, f"host f16 n={n}")
    assert_matmul_close(got[3], w16, x, f"device f16 n={n}")
    backend.release_weights()


@pytest.mark.parametrize("n", [4, 40])
def test_matmul_multi_mixed_widths_and_many_weights(backend, n):
    """Weights of different input widths fall back to one call each (backend.h:58-60); more than eight weights of
    one width take several launches (gemv at n = 4; at n = 40 the F16 ones share F16-GEMM launches and the F32 ones
    take sgemm)."""
    rng = np.random.default_rng(5)
    x = rand(rng, (n, 192))
    ws = [rand(rng, (16 + i, 192), np.float16 if i % 2 else np.float32, 0.4) for i in range(11)]
    narrow = rand(rng, (24, 96), np.float32, 0.4)
    with Buffers(backend) as B:
        dx = B.upload(x)
        ys = [B.alloc(n * w.shape[0]) for w in ws]
        backend.matmul_multi(ws, dx, ys, n)
        got = [backend.download(y, (n, w.shape[0])) for y, w in zip(ys, ws)]
        dn, dw0 = B.alloc(n * 24), B.alloc(n * ws[0].shape[0])
        backend.matmul_multi([ws[0], narrow], dx, [dw0, dn], n)
        got_n = backend.download(dn, (n, 24))
        got_0 = backend.download(dw0, (n, ws[0].shape[0]))
    for i, (g, w) in enumerate(zip(got, ws)):
        assert_matmul_close(g, w, x, f"weight {i}")
    assert np.array_equal(bits(got_0), bits(got[0]))
    # the narrow weight reads x as [n, 96]: the first n*96 floats of the buffer
    assert_matmul_close(got_n, narrow, x.reshape(-1)[: n * 96], "narrow")
    backend.release_weights()


def test_weight_copies_are_kept_and_released(backend):
    rng = np.random.default_rng(9)
    backend.release_weights()
    assert backend.weight_bytes() == 0
    w = rand(rng, (64, 128), np.float16)
    w_odd = rand(rng, (64, 100), np.float16)  # in % 8 != 0: the fp32 GEMM on a widened copy
    x = rand(rng, (20, 128))
    with Buffers(backend) as B:
        dx, dy = B.upload(x), B.alloc(20 * 64)
        backend.matmul(w, dx, dy, 1)
        assert backend.weight_bytes() == w.nbytes  # one F16 copy
        backend.matmul(w, dx, dy, 1)
        assert backend.weight_bytes() == w.nbytes  # reused, not copied again
        backend.matmul(w, dx, dy, 20)
        assert backend.weight_bytes() == w.nbytes  # the F16 GEMM reads the fp16 copy itself
        backend.matmul(w_odd, dx, dy, 20)
        assert backend.weight_bytes() == w.nbytes + w_odd.nbytes + 4 * w_odd.size  # plus the fp32 widening
    backend.release_weights()
    assert backend.weight_bytes() == 0


def test_matmul_rejects_bad_arguments(backend):
    rng = np.random.default_rng(3)
    w = rand(rng, (32, 64))
    with Buffers(backend) as B:
        dx, dy = B.alloc(4 * 64), B.alloc(4 * 32)
        with pytest.raises(nibble_amd.BackendError, match="not supported"):
            q3k = nibble_amd.weight(dx, shape=(2, 256), dtype=11)  # Q3_K: a ggml type the reference does not load
            backend.matmul_multi([q3k], dx, [dy], 1)
        with pytest.raises(nibble_amd.BackendError, match="overlaps the input"):
            backend.matmul(w, dx, dx.at(64), 2)
        with pytest.raises(nibble_amd.BackendError, match="not inside one buffer"):
            backend.matmul(w, dx, dy, 5)  # y holds 4 rows
        with pytest.raises(nibble_amd.BackendError, match="positive"):
            backend.matmul(w, dx, dy, 0)
        with pytest.raises(nibble_amd.BackendError, match="need F32"):
            backend.add_bias(dy, nibble_amd.weight(np.zeros(32, np.float16)), 1)
    backend.release_weights()


def test_f16_gemm_rows_of_any_magnitude(backend):
    """The F16 GEMM scales each activation row by its own power of two before splitting it into fp16 parts: rows
    whose largest elements range from 1e-30 to 3e30 (and an all-zero row, and a row mixing 1e-6 and 1e4 elements)
    all stay within the summation bound, as the fp32 product does."""
    rng = np.random.default_rng(21)
    in_, out_ = 320, 80
    w = rand(rng, (out_, in_), np.float16, 0.5)
    scales = [1e-30, 1e-12, 1e-3, 1.0, 7.0, 3e4, 1e12, 3e30]
    x = np.concatenate([rand(rng, (3, in_)) * np.float32(s) for s in scales] + [np.zeros((1, in_), np.float32)])
    mixed = rand(rng, (1, in_)) * np.float32(1e-6)
    mixed[0, ::17] *= np.float32(1e10)
    x = np.ascontiguousarray(np.concatenate([x, mixed]), np.float32)
    got = gpu_matmul(backend, w, x, x.shape[0])
    assert_matmul_close(got, w, x, "rows of any magnitude")
    assert np.all(bits(got[-2]) == 0), "an all-zero row gives +0"
    backend.release_weights()


def test_f16_gemm_nonfinite_activations(backend):
    """Infinite and NaN activations give the reference's non-finite outputs (an infinite element is carried by its
    fp16 high part alone, so it does not turn into NaN through hi - lo); the other rows are unaffected."""
    rng = np.random.default_rng(22)
    in_, out_, n = 64, 48, 24
    w = rand(rng, (out_, in_), np.float16, 0.5)
    w[5, 3] = 0.0  # inf * 0 = NaN in that output of the infinite row, as in the reference
    x = rand(rng, (n, in_))
    x[2, 3] = np.inf
    x[7, 10] = -np.inf
    x[9, 0] = np.nan
    got = gpu_matmul(backend, w, x, n)
    ref = oracle.matmul(w, x)
    for t in (2, 7, 9):
        assert np.array_equal(np.isnan(got[t]), np.isnan(ref[t])), f"row {t}: NaN pattern"
        fin = ~np.isnan(ref[t])
        assert np.array_equal(got[t][fin], ref[t][fin]), f"row {t}: infinities"
    ok = [t for t in range(n) if t not in (2, 7, 9)]
    assert_matmul_close(got[ok], w, x[ok], "finite rows beside non-finite ones")
    backend.release_weights()


def test_f16_gemm_wide_tiles(backend):
    """A weight with many output tiles takes the 128 x 128 tile configuration (32-deep K slices): 300 rows (a partial
    last row tile), weights of 11000 rows (partial last weight tiles), in = 200 (a partial last slice), within the
    summation bound. The configuration follows from each weight's own shape, so a call mixing two such weights and a
    500-row one (64 x 64 tiles; the two configurations in two launches) equals separate calls bit for bit
    (backend.h:57)."""
    rng = np.random.default_rng(23)
    n, in_ = 300, 200
    ws = [rand(rng, (r, in_), np.float16, 0.3) for r in (11000, 500, 11000)]
    x = rand(rng, (n, in_))
    with Buffers(backend) as B:
        dx = B.upload(x)
        ys = [B.alloc(n * w.shape[0]) for w in ws]
        backend.matmul_multi(ws, dx, ys, n)
        got = [backend.download(y, (n, w.shape[0])) for y, w in zip(ys, ws)]
        sep = []
        for w in ws:
            y1 = B.alloc(n * w.shape[0])
            backend.matmul(w, dx, y1, n)
            sep.append(backend.download(y1, (n, w.shape[0])))
    for i, (g, w) in enumerate(zip(got, ws)):
        assert_matmul_close(g, w, x, f"weight {i} ({w.shape[0]} rows)")
        assert np.array_equal(bits(g), bits(sep[i])), f"weight {i}: matmul_multi differs from a separate call"
    backend.release_weights()


def multi_vs_separate(backend, ws, x, n):
    with Buffers(backend) as B:
        dx = B.upload(x)
        ys = [B.alloc(n * w.shape[0]) for w in ws]
        backend.matmul_multi(ws, dx, ys, n)
        got = [backend.download(y, (n, w.shape[0])) for y, w in zip(ys, ws)]
        sep = []
        for w in ws:
            y1 = B.alloc(n * w.shape[0])
            backend.matmul(w, dx, y1, n)
            sep.append(backend.download(y1, (n, w.shape[0])))
    return got, sep


def assert_within_bound(got, w, x, what=""):
    """got [n, out] within the float-summation bound of the exact product (float64 reference only: for weights too
    large for the restated reference's scalar loop to run in a test)."""
    in_ = w.shape[1]
    x2 = np.asarray(x, np.float64).reshape(-1, in_)
    w64 = np.asarray(w, np.float64)
    bound = in_ * U * (np.abs(x2) @ np.abs(w64).T) + 1e-37
    err = np.abs(got.astype(np.float64) - x2 @ w64.T)
    print(f"matmul {what}: max |gpu-exact|/bound = {float(np.max(err / bound)):.3f}", flush=True)
    assert np.all(np.isfinite(got)) and np.all(err <= bound), what


def test_f16_gemm_split_k(backend):
    """Weights with few 128 x 128 tiles and a long K take K ranges (partials summed in range order): 700 and 90 rows at
    n = 300, in = 8200 (4 ranges of 65, 65, 65 and 63 slices; partial activation, weight and K tiles), in one call
    with a 12000-row weight (128 x 128 tiles, no ranges). Within the summation bound (the split weights also against
    the restated reference), and matmul_multi equals separate calls bit for bit (each weight's configuration follows
    from its own shape, backend.h:57)."""
    rng = np.random.default_rng(29)
    n, in_ = 300, 8200
    ws = [rand(rng, (r, in_), np.float16, 0.3) for r in (700, 90, 12000)]
    x = rand(rng, (n, in_))
    got, sep = multi_vs_separate(backend, ws, x, n)
    for i, (g, w) in enumerate(zip(got, ws)):
        if w.shape[0] < 1000:
            assert_matmul_close(g, w, x, f"weight {i} ({w.shape[0]} rows)")
        else:
            assert_within_bound(g, w, x, f"weight {i} ({w.shape[0]} rows)")
        assert np.array_equal(bits(g), bits(sep[i])), f"weight {i}: matmul_multi differs from a separate call"
    backend.release_weights()


def test_f16_gemm_split_k_groups(backend):
    """Three 9000-row weights at n = 300, in = 4160, each in 2 K ranges: their partial sums (5.4M floats each) exceed
    the 16M-float partial area together, so the call runs them as two groups (two weights, then one). Within the
    summation bound, and equal to separate calls bit for bit."""
    rng = np.random.default_rng(31)
    n, in_ = 300, 4160
    ws = [rand(rng, (9000, in_), np.float16, 0.3) for _ in range(3)]
    x = rand(rng, (n, in_))
    got, sep = multi_vs_separate(backend, ws, x, n)
    for i, (g, w) in enumerate(zip(got, ws)):
        assert_within_bound(g, w, x, f"weight {i}")
        assert np.array_equal(bits(g), bits(sep[i])), f"weight {i}: matmul_multi differs from a separate call"
    backend.release_weights()


@pytest.mark.parametrize("n", [9, 12, 16, 17, 40, 64, 96, 128])
def test_f16_gemm_few_rows_k_ranges(backend, n):
    """Calls of few activation rows (at most 64) give few 64 x 64 tiles, so each weight takes K ranges of 64 x 64
    tiles (up to 8, partials summed in range order): 300 and 40 rows at in = 2048 (8 ranges of 4 slices), and a
    100-row weight at in = 1000 (K padded to 1024: ranges of 4 slices, the last one partial), in one call. Within the
    summation bound and against the restated reference, and matmul_multi equals separate calls bit for bit."""
    rng = np.random.default_rng(37 + n)
    for in_, rows in ((2048, (300, 40)), (1000, (100,)), (8200, (130,))):
        ws = [rand(rng, (r, in_), np.float16, 0.3) for r in rows]
        x = rand(rng, (n, in_))
        got, sep = multi_vs_separate(backend, ws, x, n)
        for i, (g, w) in enumerate(zip(got, ws)):
            assert_matmul_close(g, w, x, f"in {in_}, weight {i} ({w.shape[0]} rows), n {n}")
            assert np.array_equal(bits(g), bits(sep[i])), f"weight {i}: matmul_multi differs from a separate call"
    backend.release_weights()
