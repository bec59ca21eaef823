"""GPU parity for Q6_K weights (GGML block_q6_K), through the C ABI, against the oracle.

Q6_K is what GGUF Q4_K_M files use for output.weight (lm_head) and for some
attn_v / ffn_down tensors.  Bars: dequant bit-exact with GGML's
dequantize_row_q6_K (oracle restatement, pinned in tests/test_oracle.py);
GEMV, batched decode and the f16 prefill within 1e-3, normwise
against the f64 matmul of the exactly dequantized weights.  Test weights are
random valid blocks (random 6-bit codes, int8 scales, f16 d).
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import Q6_K
from unillm_amd import PATH_DECODE_MFMA, PATH_GEMV, PATH_PREFILL_MFMA, HipError, QuantLinear

pytestmark = pytest.mark.gpu


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _dequant_check(blocks: np.ndarray, n: int, k: int):
    got = QuantLinear.from_blocks(Q6_K, n, k, blocks).dequantize().cpu().numpy()
    want = oracle.dequant(Q6_K, blocks, n, k)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got.view(np.uint32)[~nan], want.view(np.uint32)[~nan])


def test_q6k_dequant_bit_exact_every_d():
    # one block per f16 d (all 65536), every 6-bit code in every position class,
    # every int8 scale value across the blocks
    rng = np.random.default_rng(1)
    blocks = oracle.random_q6_k(65536, 256, seed=2).reshape(65536, 210)
    blocks[:, 208:210] = np.arange(65536, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    blocks[:, 192:208] = rng.integers(0, 256, size=(65536, 16), dtype=np.uint8)
    _dequant_check(blocks, 65536, 256)


@pytest.mark.parametrize("n,k", [(1, 256), (37, 512), (300, 4096), (64, 11008)])
def test_q6k_dequant_bit_exact_random(n, k):
    _dequant_check(oracle.random_q6_k(n, k, seed=n + k), n, k)


def _case(m, n, k, seed):
    blocks = oracle.random_q6_k(n, k, seed=seed)
    x = oracle.normal(m * k, seed=seed + 1).reshape(m, k)
    return blocks, x


def _check(m, n, k, path, bar, seed):
    blocks, x = _case(m, n, k, seed)
    ql = QuantLinear.from_blocks(Q6_K, n, k, blocks)
    if path is not None:
        assert ql.select_path(m) == path
    print(f"q6k m={m} n={n} k={k} path={path}", flush=True)
    y = ql.forward(_dev(x))
    torch.cuda.synchronize()
    err = oracle.normwise_error(y.cpu().numpy(), oracle.qmatmul_f64(Q6_K, blocks, x, n, k))
    assert err < bar, err


@pytest.mark.parametrize("m,n,k", [(1, 37, 256), (1, 300, 4096), (2, 300, 4096), (3, 129, 2048),
                                   (4, 257, 4096), (1, 32000, 4096), (1, 512, 8192),
                                   (2, 300, 11008), (1, 300, 11008), (1, 2049, 12288),
                                   (1, 300, 14336), (1, 129, 16384)])
def test_q6k_gemv_parity(m, n, k):
    _check(m, n, k, PATH_GEMV, 1e-3, seed=7 * n + k + m)


@pytest.mark.parametrize("m,n,k", [(5, 257, 256), (16, 1024, 4096), (33, 129, 2048),
                                   (64, 512, 4096), (16, 257, 11008), (1, 512, 16640)])
def test_q6k_decode_parity(m, n, k):
    # (1, 512, 16640): k beyond the GEMV's reach at m = 1 -> batched decode
    _check(m, n, k, PATH_DECODE_MFMA, 1e-3, seed=5 * m + n + k)


@pytest.mark.parametrize("m,n,k", [(65, 300, 1024), (128, 512, 4096), (130, 256, 8192),
                                   (512, 1024, 4096)])
def test_q6k_prefill_parity(m, n, k):
    _check(m, n, k, PATH_PREFILL_MFMA, 1e-3, seed=m + 3 * n + k)  # f16 operands


def test_q6k_prefill_large_tiles_rows_sampled():
    m, n, k = 2048, 8192, 2048
    blocks, x = _case(m, n, k, seed=77)
    ql = QuantLinear.from_blocks(Q6_K, n, k, blocks)
    y = ql.forward(_dev(x)).cpu().numpy()
    rows = np.array([0, 1, 255, 256, 1023, m - 77, m - 1])
    assert oracle.normwise_error(y[rows], oracle.qmatmul_f64(Q6_K, blocks, x[rows], n, k)) < 1e-3


def test_q6k_layout_limits():
    with pytest.raises(HipError):  # k must be a multiple of 256
        QuantLinear.from_blocks(Q6_K, 1, 288, np.zeros(300, np.uint8))
    ql = QuantLinear.from_blocks(Q6_K, 2, 512, oracle.random_q6_k(2, 512, seed=3))
    assert ql.gguf_bytes == 2 * 2 * 210
