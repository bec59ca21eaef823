"""GPU parity for Q4_K weights (GGML block_q4_K), through the C ABI, against the oracle.

Bars as for Q4_0: dequant bit-exact with GGML's dequantize_row_q4_K (oracle
restatement, pinned in tests/test_oracle.py); GEMV, batched decode and the f16
MFMA prefill within 1e-3 normwise of the f64 matmul of the exactly dequantized
weights.  Test weights are random valid
blocks (random codes and 6-bit scales / mins under f16 super-block scales):
GGML's Q4_K quantizer is not on the path and is not restated.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import Q4_K
from unillm_amd import PATH_DECODE_MFMA, PATH_GEMV, PATH_PREFILL_MFMA, HipError, QuantLinear

pytestmark = pytest.mark.gpu


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _dequant_check(blocks: np.ndarray, n: int, k: int):
    # bit-exact; NaNs (d or dmin inf / nan) only need to be NaN on both sides
    got = QuantLinear.from_blocks(Q4_K, n, k, blocks).dequantize().cpu().numpy()
    want = oracle.dequant(Q4_K, blocks, n, k)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(_bits(got)[~nan], _bits(want)[~nan])


def test_q4k_dequant_bit_exact_every_d():
    # one block per f16 d value (all 65536, inf / nan included), every code in
    # both nibbles of every group, random scales, mins and dmin
    rng = np.random.default_rng(1)
    blocks = oracle.random_q4_k(65536, 256, seed=2).reshape(65536, 144)
    blocks[:, 0:2] = np.arange(65536, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    blocks[:, 16:] = np.tile(np.array([j | ((15 - j) << 4) for j in range(16)], np.uint8), 8)
    blocks[:, 4:16] = rng.integers(0, 256, size=(65536, 12), dtype=np.uint8)
    _dequant_check(blocks, 65536, 256)


def test_q4k_dequant_bit_exact_every_dmin():
    blocks = oracle.random_q4_k(65536, 256, seed=3).reshape(65536, 144)
    blocks[:, 2:4] = np.arange(65536, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    _dequant_check(blocks, 65536, 256)


@pytest.mark.parametrize("n,k", [(1, 256), (37, 512), (300, 4096), (64, 11008)])
def test_q4k_dequant_bit_exact_random(n, k):
    _dequant_check(oracle.random_q4_k(n, k, seed=n + k), n, k)


def test_q4k_device_bytes_and_layout_limits():
    ql = QuantLinear.from_blocks(Q4_K, 3, 512, oracle.random_q4_k(3, 512, seed=4))
    # per row: 16 payload + 2 (sc, m) bytes per 32 weights, 4 header bytes per 256
    assert ql.device_bytes >= 3 * (16 * 16 + 2 * 16 + 4 * 2)
    with pytest.raises(HipError):  # k must be a multiple of 256
        QuantLinear.from_blocks(Q4_K, 1, 288, np.zeros(9 * 18, np.uint8))


def _gemv_case(m, n, k, seed, scale=1.0):
    blocks = oracle.random_q4_k(n, k, seed=seed)
    x = (oracle.normal(m * k, seed=seed + 1) * scale).reshape(m, k).astype(np.float32)
    return blocks, x


@pytest.mark.parametrize("m,n,k", [(1, 37, 256), (1, 300, 4096), (2, 300, 4096), (3, 129, 2048),
                                   (4, 257, 4096), (1, 4096, 11008), (1, 12288, 4096),
                                   (1, 512, 14336), (2, 512, 8192), (2, 300, 11008)])
def test_q4k_gemv_parity(m, n, k):
    blocks, x = _gemv_case(m, n, k, seed=7 * n + k)
    ql = QuantLinear.from_blocks(Q4_K, n, k, blocks)
    print(f"q4k gemv m={m} n={n} k={k}", flush=True)
    y = ql.forward(_dev(x), path=PATH_GEMV)
    torch.cuda.synchronize()
    ref = oracle.qmatmul_f64(Q4_K, blocks, x, n, k)
    assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3


def test_q4k_gemv_auto_path_and_x_range():
    # auto picks the GEMV at m <= 4; x spanning many binades (the per-block x
    # scale and the block sum must both follow it)
    m, n, k = 2, 200, 2048
    blocks, x = _gemv_case(m, n, k, seed=31)
    x[0, :256] *= 1e4
    x[1, 256:512] *= 1e-4
    ql = QuantLinear.from_blocks(Q4_K, n, k, blocks)
    assert ql.select_path(m) == PATH_GEMV
    y = ql.forward(_dev(x))
    torch.cuda.synchronize()
    assert oracle.normwise_error(y.cpu().numpy(), oracle.qmatmul_f64(Q4_K, blocks, x, n, k)) < 1e-3


def test_q4k_gemv_zero_mins():
    # dmin = 0 (the min term vanishes: w = d sc q) next to the random-min cases
    m, n, k = 1, 64, 1024
    blocks = oracle.random_q4_k(n, k, seed=41).reshape(-1, 144)
    blocks[:, 2:4] = 0
    x = oracle.normal(m * k, seed=42).reshape(m, k)
    y = QuantLinear.from_blocks(Q4_K, n, k, blocks).forward(_dev(x), path=PATH_GEMV)
    ref = oracle.qmatmul_f64(Q4_K, blocks, x, n, k)
    assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3


# ---- batched decode (f16 MFMA): per-block f16 (d sc 2^-E, dmin m 2^-E) ---------------------

@pytest.mark.parametrize("m,n,k", [(5, 257, 256), (8, 300, 4096), (16, 4096, 4096),
                                   (33, 129, 2048), (64, 512, 4096), (16, 257, 11008),
                                   (12, 1024, 14336)])
def test_q4k_decode_parity(m, n, k):
    # k = 11008: 86 chunks in slices that start on odd chunks (a 256-weight group
    # split between two workgroups); m = 33, 64: two token tiles
    blocks, x = _gemv_case(m, n, k, seed=5 * m + n + k)
    ql = QuantLinear.from_blocks(Q4_K, n, k, blocks)
    assert ql.select_path(m) == PATH_DECODE_MFMA
    print(f"q4k decode m={m} n={n} k={k}", flush=True)
    y = ql.forward(_dev(x))
    torch.cuda.synchronize()
    ref = oracle.qmatmul_f64(Q4_K, blocks, x, n, k)
    assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3


def test_q4k_decode_scale_range():
    # scales far from 1 (the weight's f16 exponent offset must keep d sc and dmin m
    # normal in f16): d, dmin around 2^-20 and around 2^6
    m, n, k = 16, 128, 2048
    x = oracle.normal(m * k, seed=61).reshape(m, k)
    for mult in (2.0 ** -14, 2.0 ** 12):
        blocks = oracle.random_q4_k(n, k, seed=62).reshape(-1, 144)
        for off in (0, 2):
            v = blocks[:, off:off + 2].copy().view(np.float16).astype(np.float32) * mult
            blocks[:, off:off + 2] = v.astype(np.float16).view(np.uint8)
        y = QuantLinear.from_blocks(Q4_K, n, k, blocks).forward(_dev(x), path=PATH_DECODE_MFMA)
        ref = oracle.qmatmul_f64(Q4_K, blocks, x, n, k)
        assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3, mult


# ---- prefill (f16 MFMA): the same kernel as Q4_0 with per-block (d sc, dmin m) -----------

@pytest.mark.parametrize("m,n,k", [(65, 300, 1024), (128, 512, 4096), (200, 130, 768),
                                   (130, 256, 8192), (512, 1024, 4096)])
def test_q4k_prefill_parity(m, n, k):
    # (130, 256, 8192): two tiles -> the k range splits over workgroups
    blocks, x = _gemv_case(m, n, k, seed=m + 3 * n + k)
    ql = QuantLinear.from_blocks(Q4_K, n, k, blocks)
    assert ql.select_path(m) == PATH_PREFILL_MFMA
    print(f"q4k prefill m={m} n={n} k={k}", flush=True)
    y = ql.forward(_dev(x))
    torch.cuda.synchronize()
    ref = oracle.qmatmul_f64(Q4_K, blocks, x, n, k)
    # f16 operands (x rows scaled by powers of two; sc and the minimum rounded to
    # f16 once each, the weight once more), the decode bar
    assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3


def test_q4k_prefill_small_m_explicit_path():
    # the prefill kernel takes any m when asked for (tiles of 128 rows, rows past m unused)
    m, n, k = 5, 300, 1024
    blocks, x = _gemv_case(m, n, k, seed=71)
    y = QuantLinear.from_blocks(Q4_K, n, k, blocks).forward(_dev(x), path=PATH_PREFILL_MFMA)
    ref = oracle.qmatmul_f64(Q4_K, blocks, x, n, k)
    assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3


def test_q4k_prefill_large_tiles_rows_sampled():
    # 256-row tiles (8 x 32 tiles fill the CUs); the oracle checks sampled rows
    m, n, k = 2048, 8192, 2048
    blocks, x = _gemv_case(m, n, k, seed=77)
    ql = QuantLinear.from_blocks(Q4_K, n, k, blocks)
    print(f"q4k prefill large m={m} n={n} k={k}", flush=True)
    y = ql.forward(_dev(x))
    torch.cuda.synchronize()
    rows = np.array([0, 1, 255, 256, 1023, m - 77, m - 1])
    ref = oracle.qmatmul_f64(Q4_K, blocks, x[rows], n, k)
    assert oracle.normwise_error(y.cpu().numpy()[rows], ref) < 1e-3
    y2 = ql.forward(_dev(x) * 2.0)
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy(), 2.0 * y.cpu().numpy())  # no k split here
