"""GPU parity for Q5_0 weights (GGML block_q5_0), through the C ABI, against the oracle.

A Q5_0 block is 32 five-bit codes q and an f16 d, w = (q - 16) d: int8 codes times
an f16 scale, which is Q8_0's form.  The device repacks it into Q8_0's frame and
runs the Q8_0 kernels; unillm_hip_qweight_info still reports Q5_0.  Bars as for
Q8_0: dequant bit-exact with GGML's dequantize_row_q5_0 (oracle restatement,
pinned in tests/test_oracle.py), every path within 1e-3 normwise of the f64
matmul of the exactly dequantized weights.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from oracle import Q5_0
from unillm_amd import PATH_DECODE_MFMA, PATH_GEMV, PATH_PREFILL_MFMA, QuantLinear, _capi

pytestmark = pytest.mark.gpu


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_q5_0_dequant_bit_exact_every_d_every_code():
    # one block per f16 d (inf / nan included); element e holds code e (all 32)
    blocks = np.zeros((65536, 22), np.uint8)
    blocks[:, 0:2] = np.arange(65536, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:6] = np.array([0xFFFF0000], np.uint32).view(np.uint8)
    blocks[:, 6:] = np.array([j | (j << 4) for j in range(16)], np.uint8)
    got = QuantLinear.from_blocks(Q5_0, 65536, 32, blocks).dequantize().cpu().numpy()
    want = oracle.dequant(Q5_0, blocks, 65536, 32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("n,k", [(1, 32), (37, 96), (300, 4096), (64, 11008)])
def test_q5_0_dequant_bit_exact_random(n, k):
    blocks = oracle.random_q5_0(n, k, seed=n + k)
    got = QuantLinear.from_blocks(Q5_0, n, k, blocks).dequantize().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), oracle.dequant(Q5_0, blocks, n, k).view(np.uint32))


def test_q5_0_reports_its_type_and_keeps_q8_0_bytes():
    n, k = 5, 64
    ql = QuantLinear.from_blocks(Q5_0, n, k, oracle.random_q5_0(n, k, seed=3))
    qt = ctypes.c_int()
    nb = ctypes.c_size_t()
    _capi.check(_capi.lib().unillm_hip_qweight_info(ql._h, ctypes.byref(qt), None, None,
                                                    ctypes.byref(nb)))
    assert qt.value == Q5_0
    assert nb.value >= n * (k // 32) * 34  # int8 codes + the f16 d, as Q8_0


@pytest.mark.parametrize("m,n,k,path", [(1, 300, 4096, PATH_GEMV), (3, 129, 2048, PATH_GEMV),
                                        (4, 2049, 4096, PATH_GEMV),
                                        (1, 4096, 11008, PATH_DECODE_MFMA),
                                        (1, 4096, 11008, PATH_GEMV),
                                        (16, 1000, 4096, PATH_DECODE_MFMA),
                                        (64, 512, 2048, PATH_DECODE_MFMA),
                                        (130, 512, 4096, PATH_PREFILL_MFMA),
                                        (700, 1024, 2048, PATH_PREFILL_MFMA)])
def test_q5_0_paths_parity(m, n, k, path):
    blocks = oracle.random_q5_0(n, k, seed=m + n + k)
    x = oracle.normal(m * k, seed=m + 2 * n).reshape(m, k)
    ql = QuantLinear.from_blocks(Q5_0, n, k, blocks)
    print(f"q5_0 m={m} n={n} k={k} path={path}", flush=True)
    y = ql.forward(_dev(x), path=path).cpu().numpy()
    rows = np.arange(m) if m <= 64 else np.array([0, 1, m // 2, m - 1])
    ref = oracle.qmatmul_f64(Q5_0, blocks, x[rows], n, k)
    assert oracle.normwise_error(y[rows], ref) < 1e-3
