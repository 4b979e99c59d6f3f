"""GPU quantized weights: Backend::matmul / matmul_multi / embed for Q4_0, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K and Q6_K,
through the C ABI, bit for bit against the oracle's restatement of quant.cpp (itself pinned to the reference's
golden vectors and to the compiled reference, tests/test_quant_oracle.py), and a quantized tiny model against the
fp64 naive model on the dequantized weights with the reference's own bar (tests/test_model.cpp:206-233: cosine >=
0.999 and the same argmax)."""
import numpy as np
import pytest

import nibble_amd
import oracle
from oracle import naive_model
from tests import model_util
from tests import quant_util as U
from tests.gpu_util import Buffers, bits

pytestmark = pytest.mark.gpu
TYPES = list(U.NAMES)


@pytest.mark.parametrize("t", TYPES, ids=[U.NAMES[t] for t in TYPES])
@pytest.mark.parametrize("n", [1, 3, 16, 17, 40, 96])
def test_quant_matmul_bit_exact(backend, t, n):
    """Activation quantization and the block dots, every activation-row chunking: n <= 16 (one row-chunked
    launch; K types above 8 rows, Q6_K above 4, take the small-call tiled kernel), 17, 40 and 96 (the tiled
    kernels: the legacy types' 32-row activation tiles, the K types' small-call kernel)."""
    be_ = oracle.block_elems(t)
    in_ = 2 * 256 if be_ == 256 else 7 * 32 + 32 * 64  # two super-blocks / 71 legacy blocks (a partial chunk)
    rows = 37  # not a multiple of the 4 rows per wave
    w = U.random_qmat(t, rows, in_, seed=1000 + t)
    x = (np.random.default_rng(n + t).standard_normal((n, in_)) * 3).astype(np.float32)
    x[0, :5] = [0.0, 1e-3, -7.0, 2.5, -2.5]
    with Buffers(backend) as B:
        dx, dy = B.upload(x), B.alloc(n * rows)
        backend.matmul(w, dx, dy, n)
        got = backend.download(dy, (n, rows))
        if n <= 4:  # x not 16-byte aligned: the activations are quantized by their own launch instead of fused
            dxu = B.alloc(n * in_ + 1)
            backend.write(dxu.at(1), x)
            backend.matmul(w, dxu.at(1), dy, n)
            assert np.array_equal(bits(backend.download(dy, (n, rows))), bits(got))
    ref = oracle.matmul_q(t, w.raw, in_, rows, x)
    diff = int(np.sum(bits(got) != bits(ref)))
    print(f"{U.NAMES[t]} n={n}: {diff} of {got.size} outputs differ from the restated reference", flush=True)
    assert diff == 0
    backend.release_weights()


def test_quant_matmul_multi_mixed_types(backend):
    """A Q4_K_M-style projection: wq, wk Q4_K and wv Q6_K sharing one quantized input, plus an F16 and a Q8_0
    weight in the same call (their own paths), into separate outputs."""
    in_, n = 512, 5
    ws = [U.random_qmat(oracle.Q4_K, 64, in_, 1), U.random_qmat(oracle.Q4_K, 16, in_, 2),
          U.random_qmat(oracle.Q6_K, 16, in_, 3), U.random_qmat(oracle.Q8_0, 8, in_, 4)]
    w16 = (np.random.default_rng(1).standard_normal((24, in_)) * 0.1).astype(np.float16)
    x = np.random.default_rng(2).standard_normal((n, in_)).astype(np.float32)
    with Buffers(backend) as B:
        dx = B.upload(x)
        ys = [B.alloc(n * w.rows) for w in ws] + [B.alloc(n * 24)]
        backend.matmul_multi(ws + [w16], dx, ys, n)
        got = [backend.download(y, (n, w.rows)) for y, w in zip(ys, ws)]
        got16 = backend.download(ys[-1], (n, 24))
    for g, w in zip(got, ws):
        assert np.array_equal(bits(g), bits(oracle.matmul_q(w.t, w.raw, in_, w.rows, x))), U.NAMES[w.t]
    exact = x.astype(np.float64) @ w16.astype(np.float64).T
    assert np.all(np.abs(got16 - exact) <= in_ * 2.0 ** -24 * (np.abs(x) @ np.abs(w16.astype(np.float64)).T) + 1e-30)
    backend.release_weights()


@pytest.mark.parametrize("t", TYPES, ids=[U.NAMES[t] for t in TYPES])
def test_quant_embed_bit_exact(backend, t):
    d = 512 if oracle.block_elems(t) == 256 else 96
    table = U.random_qmat(t, 50, d, seed=77 + t)
    ids = np.array([0, 49, 3, 3, 17], np.int32)
    with Buffers(backend) as B:
        out = B.alloc(ids.size * d)
        backend.embed(table, ids, out)
        got = backend.download(out, (ids.size, d))
    ref = np.asarray(table)[ids]
    assert np.array_equal(bits(got), bits(ref))
    backend.release_weights()


@pytest.mark.parametrize("n", [2, 100])
def test_quant_non_finite_activations(backend, n):
    """A NaN in an activation block makes its scale NaN (quant.cpp:37-49, 273-303): every output that reads the
    block is NaN, as in the reference; rows without it stay finite and exact. n = 2 runs the row-chunked kernel,
    n = 100 the tiled ones."""
    for t in (oracle.Q8_0, oracle.Q4_K, oracle.Q6_K):
        in_ = 512
        w = U.random_qmat(t, 8, in_, seed=5)
        x = np.random.default_rng(0).standard_normal((n, in_)).astype(np.float32)
        x[1, 300] = np.nan
        with Buffers(backend) as B:
            dx, dy = B.upload(x), B.alloc(n * 8)
            backend.matmul(w, dx, dy, n)
            got = backend.download(dy, (n, 8))
        ref = oracle.matmul_q(t, w.raw, in_, 8, x)
        assert np.all(np.isnan(got[1])) and np.all(np.isnan(ref[1]))
        keep = [i for i in range(n) if i != 1]
        assert np.array_equal(bits(got[keep]), bits(ref[keep])), U.NAMES[t]
    backend.release_weights()


def test_quant_rejects_bad_shapes(backend):
    with Buffers(backend) as B:
        dx, dy = B.alloc(64), B.alloc(64)
        bad = U.QMat(oracle.Q4_0, np.zeros(18 * 4, np.uint8), 2, 48)  # 48 is not a multiple of 32
        with pytest.raises(nibble_amd.BackendError, match="not a multiple"):
            backend.matmul(bad, dx, dy, 1)
        dev = B.alloc(64)
        with pytest.raises(nibble_amd.BackendError, match="host memory"):
            backend.matmul(nibble_amd.weight(dev, shape=(1, 32), dtype=oracle.Q8_0), dx, dy, 1)
    assert all(backend.supports(t) for t in TYPES + [0, 1])


LEGACY = [oracle.Q4_0, oracle.Q5_0, oracle.Q5_1, oracle.Q8_0]


@pytest.mark.parametrize("t", LEGACY, ids=[U.NAMES[t] for t in LEGACY])
def test_quant_tiled_many_weights_one_type(backend, t):
    """Prefill-sized calls (n > 16) over nine weights of one legacy type: a tiled launch takes up to eight weights,
    its grid runs over the row tiles of all of them (row counts that end inside a tile), and the ninth weight goes
    to a second launch. Every output bit-exact."""
    in_, n = 256, 100
    rows = [70, 33, 130, 64, 1, 65, 7, 128, 40]
    ws = [U.random_qmat(t, r, in_, seed=50 + i) for i, r in enumerate(rows)]
    x = np.random.default_rng(9).standard_normal((n, in_)).astype(np.float32)
    with Buffers(backend) as B:
        dx = B.upload(x)
        ys = [B.alloc(n * r) for r in rows]
        backend.matmul_multi(ws, dx, ys, n)
        got = [backend.download(y, (n, r)) for y, r in zip(ys, rows)]
    for i, (g, w) in enumerate(zip(got, ws)):
        assert np.array_equal(bits(g), bits(oracle.matmul_q(t, w.raw, in_, w.rows, x))), (U.NAMES[t], i)
    backend.release_weights()


@pytest.mark.parametrize("t", LEGACY, ids=[U.NAMES[t] for t in LEGACY])
def test_quant_tiled_legacy_every_tile_shape(backend, t):
    """The legacy tiled kernel in each of its tile shapes, chosen by the launch's size: 64 x 64 tiles when those
    give at least 512 workgroups (4100 rows = 65 row tiles x 9 activation tiles at n = 520), 64 x 32 when those do
    (n = 250: 65 x 8), 32 x 32 below (the same weight at n = 100, and a 70-row weight at n = 100). Rows and
    activation rows end inside a tile; three blocks per row: a partial chunk. Every output bit-exact."""
    in_ = 96
    w_big = U.random_qmat(t, 4100, in_, seed=700 + t)
    w_small = U.random_qmat(t, 70, in_, seed=800 + t)
    rng = np.random.default_rng(31 + t)
    x_big = (rng.standard_normal((520, in_)) * 2).astype(np.float32)
    cases = [(w_big, 520), (w_big, 250), (w_big, 100), (w_small, 100)]
    with Buffers(backend) as B:
        dx = B.upload(x_big)
        outs = []
        for w, n in cases:
            dy = B.alloc(n * w.rows)
            backend.matmul(w, dx, dy, n)
            outs.append(backend.download(dy, (n, w.rows)))
    for (w, n), g in zip(cases, outs):
        ref = oracle.matmul_q(t, w.raw, in_, w.rows, x_big[:n])
        diff = int(np.sum(bits(g) != bits(ref)))
        assert diff == 0, (U.NAMES[t], w.rows, n, diff)
    backend.release_weights()


KTYPES = [oracle.Q4_K, oracle.Q5_K, oracle.Q6_K]


@pytest.mark.parametrize("t", KTYPES, ids=[U.NAMES[t] for t in KTYPES])
def test_quant_tiled_k_both_kernels(backend, t):
    """The K types' two tiled kernels, chosen by the launch's size: a large call (4100 rows = 65 row tiles of 64 x
    17 activation tiles of 32 at n = 520) takes the 64 x 32 kernel; a small one (40 rows, n = 24) takes the
    small-call kernel, whose waves split the super-blocks - six of them here, so two rounds, the second one partial.
    Rows and activation rows end inside a tile. Every output bit-exact."""
    cases = [(U.random_qmat(t, 4100, 256, seed=900 + t), 256, 520),
             (U.random_qmat(t, 40, 1536, seed=950 + t), 1536, 24)]
    rng = np.random.default_rng(77 + t)
    for w, in_, n in cases:
        x = (rng.standard_normal((n, in_)) * 2).astype(np.float32)
        with Buffers(backend) as B:
            dx, dy = B.upload(x), B.alloc(n * w.rows)
            backend.matmul(w, dx, dy, n)
            got = backend.download(dy, (n, w.rows))
        ref = oracle.matmul_q(t, w.raw, in_, w.rows, x)
        diff = int(np.sum(bits(got) != bits(ref)))
        assert diff == 0, (U.NAMES[t], w.rows, n, diff)
    backend.release_weights()


@pytest.mark.parametrize("n", [17, 80, 130])
def test_quant_tiled_k_types_mixed(backend, n):
    """Prefill-sized calls over K-type weights, which run the int8 matrix-core kernel on residue-major Q8_K
    activations, mixed in one call with a Q8_0 weight (the legacy tiled kernel on Q8_0 activations): the
    activations are quantized once per layout, in the order the types come. Row counts that end inside a 16-row
    tile, three super-blocks per row, activation rows that end inside a 64-row tile. Every output bit-exact."""
    in_ = 768
    spec = [(oracle.Q4_K, 70), (oracle.Q6_K, 33), (oracle.Q8_0, 20), (oracle.Q5_K, 16), (oracle.Q4_K, 1),
            (oracle.Q5_K, 45), (oracle.Q6_K, 130)]
    ws = [U.random_qmat(t, r, in_, seed=300 + i) for i, (t, r) in enumerate(spec)]
    x = (np.random.default_rng(n).standard_normal((n, in_)) * 2).astype(np.float32)
    with Buffers(backend) as B:
        dx = B.upload(x)
        ys = [B.alloc(n * r) for _, r in spec]
        backend.matmul_multi(ws, dx, ys, n)
        got = [backend.download(y, (n, r)) for y, (_, r) in zip(ys, spec)]
    for i, (g, w) in enumerate(zip(got, ws)):
        ref = oracle.matmul_q(w.t, w.raw, in_, w.rows, x)
        diff = int(np.sum(bits(g) != bits(ref)))
        assert diff == 0, (U.NAMES[w.t], i, diff)
    backend.release_weights()


@pytest.mark.parametrize("n", [1, 5, 100])
def test_quant_q8_1_sum_term_tie(backend, n):
    """Q5_1 against activations holding a block whose Q8_1 sum term float(sum) * d is an exact fp16 tie (the
    reference rounds the product to float, then to fp16: down to the even neighbour here). Every activation path:
    quantized inside the launch (n = 1), by the quantizer launch (n = 5) and under the tiled kernel (n = 100)."""
    from tests.test_quant_oracle import tie_block
    in_, rows = 256, 24
    x = np.random.default_rng(3).standard_normal((n, in_)).astype(np.float32)
    x[-1, 96:128] = tie_block()
    w = U.random_qmat(oracle.Q5_1, rows, in_, seed=77)
    with Buffers(backend) as B:
        dx, dy = B.upload(x), B.alloc(n * rows)
        backend.matmul(w, dx, dy, n)
        got = backend.download(dy, (n, rows))
    assert np.array_equal(bits(got), bits(oracle.matmul_q(oracle.Q5_1, w.raw, in_, rows, x)))
    backend.release_weights()


@pytest.mark.parametrize("t", [oracle.Q8_0, oracle.Q4_0], ids=["Q8_0", "Q4_0"])
def test_quantized_tiny_model_matches_naive(backend, t):
    """tests/test_model.cpp:206-233 on the GPU: the reference's quant_dims tiny model (n_embd 32, n_ff 64, head_dim
    8) with every matrix quantized, against the fp64 naive model on the dequantized weights."""
    m = model_util.tiny_model(7, np.float32, "qwen2", False, E=32, FF=64)
    m["token_embd"] = U.quantize_matrix(m["token_embd"], t)
    for L in m["layers"]:
        for k in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            L[k] = U.quantize_matrix(L[k], t)
    toks = [1, 50, 257, 3, 99]
    g = model_util.GpuModel(backend, m, n_ctx=64)
    try:
        got = g.forward(toks)
        inc = None
        g2 = model_util.GpuModel(backend, m, n_ctx=64)
        try:
            for i, tok in enumerate(toks):
                inc = g2.forward([tok], pos0=i)
        finally:
            g2.close()
    finally:
        g.close()
    ref = naive_model.naive_logits(m, toks)
    cos = float(np.dot(got, ref) / np.sqrt(np.dot(got, got) * np.dot(ref, ref)))
    print(f"{U.NAMES[t]} tiny model: cosine vs naive {cos:.6f}, argmax {int(np.argmax(got))} vs "
          f"{int(np.argmax(ref))}; incremental max |diff| {np.max(np.abs(inc - got)):.2e}", flush=True)
    assert cos >= 0.999
    assert int(np.argmax(got)) == int(np.argmax(ref))
    assert np.all(np.isfinite(inc))


@pytest.mark.parametrize("t", [oracle.Q4_0, oracle.Q5_1, oracle.Q8_0, oracle.Q4_K], ids=["Q4_0", "Q5_1", "Q8_0", "Q4_K"])
def test_quant_single_row_over_many_rows(backend, t):
    """A single activation row against 16400 weight rows in one call (an FFN-sized launch, which takes 16 rows per
    wave for the legacy types), bit-exact."""
    in_ = 256
    rows = 16400
    w = U.random_qmat(t, rows, in_, seed=31 + t)
    x = np.random.default_rng(t).standard_normal((1, in_)).astype(np.float32)
    with Buffers(backend) as B:
        dx, dy = B.upload(x), B.alloc(rows)
        backend.matmul(w, dx, dy, 1)
        got = backend.download(dy, (1, rows))
    ref = oracle.matmul_q(t, w.raw, in_, rows, x)
    assert np.array_equal(bits(got), bits(ref))
    backend.release_weights()
