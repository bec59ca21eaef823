"""GPU parity for Q5_K weights (GGML block_q5_K), through the C ABI, against the oracle.

Q5_K holds the projections of GGUF Q5_K_M files; the reference hands it to candle's
QMatMul like every other type (weight_loader_core.rs:569-571).  Bars as for Q4_K:
dequant bit-exact with GGML's dequantize_row_q5_K (oracle restatement, pinned in
tests/test_oracle.py); GEMV, batched decode and the f16 MFMA prefill within 1e-3
normwise of the f64 matmul of the exactly dequantized weights, and the fused
epilogues against the same f64 formulas as the other types.  Test weights are
random valid blocks (random codes, fifth bits and 6-bit scales / mins under f16
super-block scales): GGML's Q5_K quantizer is not on the path and is not restated.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import Q5_K
from unillm_amd import PATH_DECODE_MFMA, PATH_GEMV, PATH_PREFILL_MFMA, HipError, QuantLinear

pytestmark = pytest.mark.gpu


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _dequant_check(blocks: np.ndarray, n: int, k: int):
    # bit-exact; NaNs (d or dmin inf / nan) only need to be NaN on both sides
    got = QuantLinear.from_blocks(Q5_K, n, k, blocks).dequantize().cpu().numpy()
    want = oracle.dequant(Q5_K, blocks, n, k)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(_bits(got)[~nan], _bits(want)[~nan])


def test_q5k_dequant_bit_exact_every_d():
    # one block per f16 d value (all 65536, inf / nan included); every 5-bit code
    # in every sub-block position, random scales, mins and dmin
    rng = np.random.default_rng(1)
    blocks = oracle.random_q5_k(65536, 256, seed=2).reshape(65536, 176)
    blocks[:, 0:2] = np.arange(65536, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    blocks[:, 4:16] = rng.integers(0, 256, size=(65536, 12), dtype=np.uint8)
    # weight l of sub-block j: code (l + j) % 32 -> nibble and fifth bit
    qs = np.zeros((4, 32), np.uint8)
    qh = np.zeros(32, np.uint8)
    for j in range(8):
        for l in range(32):
            q = (l + j) % 32
            qs[j // 2, l] |= (q & 15) << (4 * (j % 2))
            qh[l] |= (q >> 4) << j
    blocks[:, 16:48] = qh
    blocks[:, 48:] = qs.reshape(-1)
    _dequant_check(blocks, 65536, 256)


def test_q5k_dequant_bit_exact_every_dmin():
    blocks = oracle.random_q5_k(65536, 256, seed=3).reshape(65536, 176)
    blocks[:, 2:4] = np.arange(65536, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    _dequant_check(blocks, 65536, 256)


@pytest.mark.parametrize("n,k", [(1, 256), (37, 512), (300, 4096), (64, 11008)])
def test_q5k_dequant_bit_exact_random(n, k):
    _dequant_check(oracle.random_q5_k(n, k, seed=n + k), n, k)


def test_q5k_device_bytes_and_layout_limits():
    ql = QuantLinear.from_blocks(Q5_K, 3, 512, oracle.random_q5_k(3, 512, seed=4))
    # per row: 32 payload + 2 (sc, m) bytes per 32 weights, 4 header bytes per 256
    assert ql.device_bytes >= 3 * (32 * 16 + 2 * 16 + 4 * 2)
    with pytest.raises(HipError):  # k must be a multiple of 256
        QuantLinear.from_blocks(Q5_K, 1, 288, np.zeros(9 * 22, np.uint8))


def _case(m, n, k, seed, scale=1.0):
    blocks = oracle.random_q5_k(n, k, seed=seed)
    x = (oracle.normal(m * k, seed=seed + 1) * scale).reshape(m, k).astype(np.float32)
    return blocks, x


@pytest.mark.parametrize("m,n,k", [(1, 37, 256), (1, 300, 4096), (2, 300, 4096), (3, 129, 2048),
                                   (4, 257, 4096), (1, 4096, 4096), (1, 12288, 4096),
                                   (1, 5632, 2048), (2, 512, 2048), (2, 300, 11008)])
def test_q5k_gemv_parity(m, n, k):
    blocks, x = _case(m, n, k, seed=7 * n + k)
    ql = QuantLinear.from_blocks(Q5_K, n, k, blocks)
    print(f"q5k gemv m={m} n={n} k={k}", flush=True)
    y = ql.forward(_dev(x), path=PATH_GEMV)
    torch.cuda.synchronize()
    ref = oracle.qmatmul_f64(Q5_K, blocks, x, n, k)
    assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3


def test_q5k_gemv_limits_and_auto_path():
    # byte codes: the GEMV takes k <= 16384 at one row (past 8192 with k split over
    # wave pairs, the down projections' k 11008 and 14336 among them), like Q8_0;
    # longer rows go to the batched decode
    ql = QuantLinear.from_blocks(Q5_K, 64, 16640, oracle.random_q5_k(64, 16640, seed=5))
    assert ql.select_path(1) == PATH_DECODE_MFMA
    with pytest.raises(HipError, match="GEMV path"):
        ql.forward(torch.zeros(1, 16640, device="cuda"), path=PATH_GEMV)
    _gemv_deep_k(1, 300, 11008)
    _gemv_deep_k(1, 257, 14336)


def _gemv_deep_k(m, n, k):
    blocks, x = _case(m, n, k, seed=9)
    ql = QuantLinear.from_blocks(Q5_K, n, k, blocks)
    assert ql.select_path(1) == PATH_GEMV
    ref = oracle.qmatmul_f64(Q5_K, blocks, x, n, k)
    xd = _dev(x)
    y = ql.forward(xd).cpu().numpy()
    assert oracle.normwise_error(y, ref) < 1e-3
    y0 = oracle.normal(n, seed=3).reshape(1, n).astype(np.float32)
    ya = _dev(y0)
    ql.forward_add(xd, ya)
    assert np.array_equal(ya.cpu().numpy(), y0 + y)
    y = ql.forward(xd, path=PATH_DECODE_MFMA).cpu().numpy()
    assert oracle.normwise_error(y, ref) < 1e-3


def test_q5k_gemv_x_range_and_zero_mins():
    # x spanning many binades (the per-block x scale and the block sum follow it),
    # and dmin = 0 (the min term vanishes)
    m, n, k = 2, 200, 2048
    blocks, x = _case(m, n, k, seed=31)
    x[0, :256] *= 1e4
    x[1, 256:512] *= 1e-4
    ql = QuantLinear.from_blocks(Q5_K, n, k, blocks)
    assert ql.select_path(m) == PATH_GEMV
    y = ql.forward(_dev(x))
    assert oracle.normwise_error(y.cpu().numpy(), oracle.qmatmul_f64(Q5_K, blocks, x, n, k)) < 1e-3
    blocks = blocks.reshape(-1, 176).copy()
    blocks[:, 2:4] = 0
    y = QuantLinear.from_blocks(Q5_K, n, k, blocks).forward(_dev(x), path=PATH_GEMV)
    assert oracle.normwise_error(y.cpu().numpy(), oracle.qmatmul_f64(Q5_K, blocks, x, n, k)) < 1e-3


# ---- batched decode (f16 MFMA): per-block f16 (d sc 2^-E, dmin m 2^-E) ---------------------

@pytest.mark.parametrize("m,n,k", [(5, 257, 256), (8, 300, 4096), (16, 4096, 4096),
                                   (33, 129, 2048), (64, 512, 4096), (16, 257, 11008),
                                   (12, 1024, 14336), (16, 14336, 4096)])
def test_q5k_decode_parity(m, n, k):
    blocks, x = _case(m, n, k, seed=5 * m + n + k)
    ql = QuantLinear.from_blocks(Q5_K, n, k, blocks)
    assert ql.select_path(m) == PATH_DECODE_MFMA
    print(f"q5k decode m={m} n={n} k={k}", flush=True)
    y = ql.forward(_dev(x))
    torch.cuda.synchronize()
    ref = oracle.qmatmul_f64(Q5_K, blocks, x, n, k)
    assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3


def test_q5k_decode_scale_range():
    # d, dmin far from 1: the weight's f16 exponent offset keeps d sc and dmin m normal
    m, n, k = 16, 128, 2048
    x = oracle.normal(m * k, seed=61).reshape(m, k)
    for mult in (2.0 ** -14, 2.0 ** 12):
        blocks = oracle.random_q5_k(n, k, seed=62).reshape(-1, 176)
        for off in (0, 2):
            v = blocks[:, off:off + 2].copy().view(np.float16).astype(np.float32) * mult
            blocks[:, off:off + 2] = v.astype(np.float16).view(np.uint8)
        y = QuantLinear.from_blocks(Q5_K, n, k, blocks).forward(_dev(x), path=PATH_DECODE_MFMA)
        ref = oracle.qmatmul_f64(Q5_K, blocks, x, n, k)
        assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3, mult


# ---- prefill (f16 MFMA) ---------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k", [(65, 300, 1024), (128, 512, 4096), (200, 130, 768),
                                   (130, 256, 8192), (512, 1024, 4096), (300, 4096, 14336)])
def test_q5k_prefill_parity(m, n, k):
    blocks, x = _case(m, n, k, seed=m + 3 * n + k)
    ql = QuantLinear.from_blocks(Q5_K, n, k, blocks)
    assert ql.select_path(m) == PATH_PREFILL_MFMA
    print(f"q5k prefill m={m} n={n} k={k}", flush=True)
    y = ql.forward(_dev(x))
    torch.cuda.synchronize()
    ref = oracle.qmatmul_f64(Q5_K, blocks, x, n, k)
    assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3


def test_q5k_prefill_large_tiles_rows_sampled():
    m, n, k = 2048, 8192, 2048
    blocks, x = _case(m, n, k, seed=77)
    ql = QuantLinear.from_blocks(Q5_K, n, k, blocks)
    print(f"q5k prefill large m={m} n={n} k={k}", flush=True)
    y = ql.forward(_dev(x))
    torch.cuda.synchronize()
    rows = np.array([0, 1, 255, 256, 1023, m - 77, m - 1])
    ref = oracle.qmatmul_f64(Q5_K, blocks, x[rows], n, k)
    assert oracle.normwise_error(y.cpu().numpy()[rows], ref) < 1e-3
    y2 = ql.forward(_dev(x) * 2.0)
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy(), 2.0 * y.cpu().numpy())


# ---- fused epilogues on every path ---------------------------------------------------------

def _layer_norm(x, g, b, eps):
    x = x.astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * g.astype(np.float64) + b.astype(np.float64)


@pytest.mark.parametrize("m", [1, 3, 9, 40, 130])
def test_q5k_epilogues(m):
    k, half = 2048, 320
    n = 2 * half
    blocks, x = _case(m, n, k, seed=900 + m)
    ql = QuantLinear.from_blocks(Q5_K, n, k, blocks)
    rng = np.random.default_rng(m)
    g = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    b = (0.1 * rng.standard_normal(k)).astype(np.float32)
    y0 = rng.standard_normal((m, n)).astype(np.float32)
    xd, gd, bd = _dev(x), _dev(g), _dev(b)
    print(f"q5k epilogues m={m}", flush=True)
    r = oracle.qmatmul_f64(Q5_K, blocks, x, n, k)
    y = _dev(y0)
    ql.forward_add(xd, y)
    assert oracle.normwise_error(y.cpu().numpy(), y0 + r) < 1e-3
    xn = _layer_norm(x, g, b, 1e-6).astype(np.float32)
    rn = oracle.qmatmul_f64(Q5_K, blocks, xn, n, k)
    got = ql.forward_norm(xd, gd, bd, eps=1e-6).cpu().numpy()
    assert oracle.normwise_error(got, rn) < 1e-3
    act = ql.forward_swiglu(xd, norm=(gd, bd, 1e-6)).cpu().numpy()
    gg, uu = rn[:, :half], rn[:, half:]
    assert oracle.normwise_error(act, gg / (1.0 + np.exp(-gg)) * uu) < 2e-3
