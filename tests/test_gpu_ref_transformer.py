"""nibble's own model::Transformer (src/model/transformer.cpp, compiled from the reference's sources) running over
HipBackend: the drop-in as the reference's model code sees it, with no restatement of the forward in between.

oracle/_ref/transformer_driver (built by `make -C oracle transformer` from transformer.cpp where it lies, linked with
the reference's CpuBackend in oracle/_ref/libnibble_ref.so and with nibble_amd/libnibble_hip.so) binds a model
written by tests/model_util.write_model_dir and runs Transformer::forward over either backend, printing the last
token's logits bit for bit. The bars are the reference's own model tests: logits within 1e-4 of the fp64 naive model
(test_model.cpp:110-131), and batch, one-token-at-a-time and 2-token-chunk runs bitwise equal (test_model.cpp:141-151,
253-263) - here with HipBackend's batch invariance on, the mode that gives that guarantee. Each HIP run is also held
against the same Transformer over the reference's CpuBackend.

The CPU-only test pins the driver and the model writer: over CpuBackend the compiled reference must pass its own
two tests. Skipped where the driver is not built (it needs the reference sources at build time).
"""
import json
import os
import subprocess

import numpy as np
import pytest

from oracle import naive_model
from tests import model_util
from tests import quant_util as U
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "oracle", "_ref", "transformer_driver")
TOKS = [1, 50, 257, 3, 99]

needs_driver = pytest.mark.skipif(not os.path.exists(DRIVER),
                                  reason="oracle/_ref/transformer_driver not built (make -C oracle ref transformer)")


def run(m, tmp_path, backend, toks, runs, n_ctx=64, invariant=False):
    d = str(tmp_path / "model")
    if not os.path.exists(os.path.join(d, "model.txt")):
        model_util.write_model_dir(m, d)
    print(f"driver: {backend} invariant={int(invariant)} runs={runs} tokens={len(toks)}", flush=True)
    r = subprocess.run([DRIVER, d, backend, str(n_ctx), str(int(invariant)), ",".join(map(str, toks)), *runs],
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-3000:]
    out = {}
    for line in r.stdout.splitlines():
        j = json.loads(line)
        out[j["run"]] = np.frombuffer(bytes.fromhex(j["bits"]), dtype=">u4").astype(np.uint32).view(np.float32)
    assert list(out) == list(runs)
    return out


def bitwise_equal(a, b):
    return np.array_equal(a.view(np.uint32), b.view(np.uint32))


MODELS = [("qwen2", np.float32, False), ("qwen2", np.float16, False), ("llama", np.float32, False),
          ("llama", np.float32, True), ("llama", np.float16, True)]
MODEL_IDS = ["qwen2-f32", "qwen2-f16", "llama-f32", "llama-f32-freqs", "llama-f16-freqs"]


@needs_driver
@pytest.mark.parametrize("arch,rf", [("llama", True), ("qwen2", False)], ids=["llama-freqs", "qwen2"])
def test_driver_over_cpu_backend_passes_the_reference_tests(tmp_path, arch, rf):
    """Over the reference's own CpuBackend: within 1e-4 of the naive model, and batch = incremental = 2-token chunks
    bit for bit (the reference's tests, seed 3, tokens {1, 50, 257, 3, 99})."""
    m = model_util.tiny_model(3, np.float32, arch, rf)
    out = run(m, tmp_path, "cpu", TOKS, ["b512", "i", "b2"])
    assert bitwise_equal(out["i"], out["b512"]) and bitwise_equal(out["b2"], out["b512"])
    assert float(np.max(np.abs(out["b512"] - naive_model.naive_logits(m, TOKS)))) <= 1e-4


@needs_driver
@pytest.mark.gpu
@pytest.mark.parametrize("arch,wtype,rf", MODELS, ids=MODEL_IDS)
def test_reference_transformer_over_hip_backend(tmp_path, arch, wtype, rf):
    """test_model.cpp:110-131 with HipBackend dropped in: the reference's forward over the GPU backend within 1e-4
    of the naive model and of the same forward over CpuBackend."""
    m = model_util.tiny_model(7, wtype, arch, rf)
    hip = run(m, tmp_path, "hip", TOKS, ["b512"])["b512"]
    cpu = run(m, tmp_path, "cpu", TOKS, ["b512"])["b512"]
    naive = naive_model.naive_logits(m, TOKS)
    print(f"{arch} {np.dtype(wtype).name} freqs={rf}: |hip-naive| {np.max(np.abs(hip - naive)):.2e}, "
          f"|hip-cpu| {np.max(np.abs(hip - cpu)):.2e}", flush=True)
    assert np.all(np.isfinite(hip))
    assert float(np.max(np.abs(hip - naive))) <= 1e-4
    assert float(np.max(np.abs(hip - cpu))) <= 1e-4


@needs_driver
@pytest.mark.gpu
@pytest.mark.parametrize("arch,rf", [("llama", True), ("qwen2", False)], ids=["llama-freqs", "qwen2"])
def test_reference_transformer_incremental_and_chunked_equal_batch(tmp_path, arch, rf):
    """test_model.cpp:141-151 (llama with rope freqs) and 253-263 (qwen2) over HipBackend with batch invariance:
    batch, one-by-one and 2-token chunks give identical bits."""
    m = model_util.tiny_model(3, np.float32, arch, rf)
    out = run(m, tmp_path, "hip", TOKS, ["b512", "i", "b2"], invariant=True)
    for name in ("i", "b2"):
        assert bitwise_equal(out[name], out["b512"]), name
    assert float(np.max(np.abs(out["b512"] - naive_model.naive_logits(m, TOKS)))) <= 1e-4


def cosine(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.dot(a, b) / np.sqrt(np.dot(a, a) * np.dot(b, b)))


@needs_driver
@pytest.mark.gpu
@pytest.mark.parametrize("t", [oracle.Q8_0, oracle.Q4_0], ids=["Q8_0", "Q4_0"])
def test_reference_transformer_quantized(tmp_path, t):
    """test_model.cpp:206-233 over HipBackend: the quant_dims model (n_embd 32, n_ff 64, head_dim 8) with every
    matrix quantized; logits with cosine >= 0.999 against the naive model on the dequantized weights and the same
    argmax, and (batch invariance on) batch equal to incremental bit for bit. Against the same forward over
    CpuBackend (quantized matmuls bit-exact on both; the activations' Q8 rounding can turn a last-bit difference
    from attention into one quantization step) the cosine is held to 0.9999."""
    m = model_util.tiny_model(7, np.float32, "qwen2", False, E=32, FF=64)
    m["token_embd"] = U.quantize_matrix(m["token_embd"], t)
    for L in m["layers"]:
        for k in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            L[k] = U.quantize_matrix(L[k], t)
    hip = run(m, tmp_path, "hip", TOKS, ["b512"])["b512"]
    inv = run(m, tmp_path, "hip", TOKS, ["b512", "i"], invariant=True)
    cpu = run(m, tmp_path, "cpu", TOKS, ["b512"])["b512"]
    naive = naive_model.naive_logits(m, TOKS)
    print(f"{U.NAMES[t]}: cosine vs naive {cosine(hip, naive):.6f}, vs cpu {cosine(hip, cpu):.8f}, "
          f"|hip-cpu| {np.max(np.abs(hip - cpu)):.2e}", flush=True)
    assert cosine(hip, naive) >= 0.999
    assert int(np.argmax(hip)) == int(np.argmax(naive))
    assert cosine(hip, cpu) >= 0.9999
    assert bitwise_equal(inv["i"], inv["b512"])


@needs_driver
@pytest.mark.gpu
def test_reference_transformer_head_dim_64(tmp_path):
    """n_embd 256, 4 heads of 64, llama with rope freqs, F16 weights, 150 tokens. Default route: the batch call
    runs rows 128.. on the MFMA prefill, within 1e-3 of the logits' scale of the CpuBackend forward. Batch
    invariance: batch, one-by-one, 2- and 17-token chunks bitwise equal, within 1e-4 of the CpuBackend forward."""
    m = model_util.tiny_model(11, np.float16, "llama", True, E=256, FF=512, scale=0.25)
    toks = np.random.default_rng(5).integers(0, 261, 150).tolist()
    cpu = run(m, tmp_path, "cpu", toks, ["b512"], n_ctx=160)["b512"]
    scale = max(1.0, float(np.max(np.abs(cpu))))
    hip = run(m, tmp_path, "hip", toks, ["b512", "i"], n_ctx=160)
    for name, o in hip.items():
        d = float(np.max(np.abs(o - cpu)))
        print(f"hd64 default route {name}: |hip-cpu| {d:.2e} (max |logit| {scale:.2f})", flush=True)
        assert d <= 1e-3 * scale
    inv = run(m, tmp_path, "hip", toks, ["b512", "i", "b2", "b17"], n_ctx=160, invariant=True)
    for name, o in inv.items():
        assert bitwise_equal(o, inv["b512"]), name
    d = float(np.max(np.abs(inv["b512"] - cpu)))
    print(f"hd64 batch-invariant: |hip-cpu| {d:.2e}", flush=True)
    assert d <= 1e-4 * scale


@needs_driver
@pytest.mark.gpu
def test_reference_transformer_repeated_phrase(tmp_path):
    """The head_dim-64 model (n_embd 256, llama with rope freqs, F16 weights) on a 600-token prompt that repeats one
    20-token phrase 30 times: a first layer's value rows repeat exactly wherever a token recurs, and rows 128..599
    take the MFMA prefill route (one call of 600 rows, and 512-row chunks as the Transformer cuts a prompt). Logits
    within 1e-3 of the logits' scale of the same forward over the reference's CpuBackend."""
    m = model_util.tiny_model(11, np.float16, "llama", True, E=256, FF=512, scale=0.25)
    phrase = np.random.default_rng(8).integers(0, 261, 20).tolist()
    toks = phrase * 30
    cpu = run(m, tmp_path, "cpu", toks, ["b1024"], n_ctx=640)["b1024"]
    scale = max(1.0, float(np.max(np.abs(cpu))))
    hip = run(m, tmp_path, "hip", toks, ["b1024", "b512"], n_ctx=640)
    for name, o in hip.items():
        d = float(np.max(np.abs(o - cpu)))
        print(f"repeated phrase {name}: |hip-cpu| {d:.2e} (max |logit| {scale:.2f})", flush=True)
        assert np.all(np.isfinite(o))
        assert d <= 1e-3 * scale
