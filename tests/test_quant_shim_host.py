"""Host-side contract of the quantized-matmul entry points of libnibble_hip.so, on the CPU: the device layout sizes
and the argument checks that reject a call before anything is launched (no GPU call is made here)."""
import ctypes

import pytest

import nibble_amd
import oracle

EINVAL = 1
QTYPES = [oracle.Q4_0, oracle.Q5_0, oracle.Q5_1, oracle.Q8_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K]
# bytes of one block in the file (quant.h) and elements per block
FILE_BLOCK = {oracle.Q4_0: (18, 32), oracle.Q5_0: (22, 32), oracle.Q5_1: (24, 32), oracle.Q8_0: (34, 32),
              oracle.Q4_K: (144, 256), oracle.Q5_K: (176, 256), oracle.Q6_K: (210, 256)}


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(nibble_amd.LIB_PATH)
    i64, vp, cint = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
    L.nbhs_quant_weight_bytes.restype = i64
    L.nbhs_quant_weight_bytes.argtypes = [cint, i64, i64]
    L.nbhs_quant_act_bytes.restype = i64
    L.nbhs_quant_act_bytes.argtypes = [cint, i64, i64]
    L.nbhs_qgemm_multi.restype = cint
    L.nbhs_qgemm_multi.argtypes = [cint, cint, vp, vp, vp, i64, vp, i64, vp]
    L.nbhs_quantize_acts_rm.restype = cint
    L.nbhs_quantize_acts_rm.argtypes = [cint, vp, i64, i64, vp, vp]
    return L


@pytest.mark.parametrize("t", QTYPES)
def test_weight_layout_holds_the_file_bytes(lib, t):
    """The repacked planes hold every byte of the file's blocks (Q4_K / Q5_K's 12 scale bytes padded to 16), each
    plane 256-byte aligned: at least the file size, at most one 256-byte pad per plane more, and it grows with the
    rows."""
    bb, be = FILE_BLOCK[t]
    for rows, nb in [(1, 1), (37, 3), (2048, 2048 // be if be == 32 else 8), (3, 17)]:
        got = lib.nbhs_quant_weight_bytes(t, rows, nb * be)
        pad_scales = 4 * rows * nb if t in (oracle.Q4_K, oracle.Q5_K) else 0
        assert rows * nb * bb + pad_scales <= got <= rows * nb * bb + pad_scales + 5 * 256, (t, rows, nb)
        assert got % 256 == 0
        assert lib.nbhs_quant_weight_bytes(t, rows + 1, nb * be) >= got


@pytest.mark.parametrize("t", QTYPES)
def test_bad_widths_are_rejected(lib, t):
    _, be = FILE_BLOCK[t]
    assert lib.nbhs_quant_weight_bytes(t, 4, be + 1) == -1
    assert lib.nbhs_quant_weight_bytes(t, 0, be) == -1
    assert lib.nbhs_quant_act_bytes(t, 4, be // 2) == -1
    assert lib.nbhs_quant_weight_bytes(1, 4, 256) == -1  # F16 is not a quantized type


@pytest.mark.parametrize("t", QTYPES)
def test_activation_planes(lib, t):
    """Q8_0 / Q8_1 / Q8_K planes: one int8 per element, a float scale per block (and Q8_1's sum term, Q8_K's 16
    16-bit sums), each plane 256-byte aligned."""
    _, be = FILE_BLOCK[t]
    n, nb = 5, 3
    per_block = 32 + 4 + (4 if t == oracle.Q5_1 else 0) if be == 32 else 256 + 4 + 32
    got = lib.nbhs_quant_act_bytes(t, n, nb * be)
    assert n * nb * per_block <= got <= n * nb * per_block + 4 * 256 and got % 256 == 0


def test_tiled_matmul_rejects_before_launching(lib):
    """Every shape the tiled kernels do not take returns EINVAL without touching the device (all pointers here
    are dummies that a launch would fault on)."""
    dummy = ctypes.c_void_p(0x1000)
    ws = (ctypes.c_void_p * 9)(*([0x1000] * 9))
    rows = (ctypes.c_int64 * 9)(*([64] * 9))
    ys = (ctypes.c_void_p * 9)(*([0x1000] * 9))
    q = lib.nbhs_qgemm_multi
    assert q(oracle.Q8_0, 0, ws, rows, ys, 256, dummy, 32, None) == EINVAL        # no weights
    assert q(oracle.Q8_0, 9, ws, rows, ys, 256, dummy, 32, None) == EINVAL        # more than 8 in one launch
    assert q(oracle.Q4_K, 2, ws, rows, ys, 300, dummy, 32, None) == EINVAL        # width not whole super-blocks
    assert q(oracle.Q8_0, 2, ws, rows, ys, 256, None, 32, None) == EINVAL         # no activations
    assert q(oracle.Q8_0, 2, ws, rows, ys, 256, dummy, 0, None) == EINVAL         # no rows
    assert q(oracle.Q8_0, 2, ws, rows, ys, 256, dummy, 64 * 65536, None) == EINVAL  # grid y beyond 65535
    assert q(1, 2, ws, rows, ys, 256, dummy, 32, None) == EINVAL                  # F16: not a quantized type
    bad_rows = (ctypes.c_int64 * 2)(64, 0)
    assert q(oracle.Q8_0, 2, ws, bad_rows, ys, 256, dummy, 32, None) == EINVAL    # an empty weight
    no_y = (ctypes.c_void_p * 2)(0x1000, 0)
    assert q(oracle.Q6_K, 2, ws, rows, no_y, 256, dummy, 32, None) == EINVAL      # a missing output
    rm = lib.nbhs_quantize_acts_rm
    assert rm(oracle.Q8_0, dummy, 4, 256, dummy, None) == EINVAL  # residue-major order is for the K types only
    assert rm(oracle.Q4_K, dummy, 4, 200, dummy, None) == EINVAL
    assert rm(oracle.Q4_K, None, 4, 256, dummy, None) == EINVAL
