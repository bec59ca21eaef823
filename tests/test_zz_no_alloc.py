"""unillm_hip_qmatmul_noalloc against unillm_hip_qmatmul, through the C ABI.

The no-allocation entry point runs the same kernels as unillm_hip_qmatmul, with the
MFMA paths' f16 copy of x in the library's fixed per-GPU scratch instead of the
stream's workspace.  Each case makes two calls in a row on one weight, the second
with fewer rows (the scratch keeps the first call's contents), and compares each
with unillm_hip_qmatmul on the same input: bit for bit where every output is
summed in one fixed order (GEMV, prefill), to f32 rounding where the batched
decode's split k ranges meet by atomic adds.  Both also meet the oracle's 1e-3.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from oracle import Q4_0, Q8_0
from unillm_amd import PATH_DECODE_MFMA, PATH_GEMV, PATH_PREFILL_MFMA, QuantLinear, _capi

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


def _call(fn, ql, x, n, stream):
    y = torch.empty(x.shape[0], n, device="cuda")
    rc = fn(ql._h, ctypes.c_void_p(x.data_ptr()), x.shape[0], ctypes.c_void_p(y.data_ptr()),
            ctypes.c_void_p(stream.cuda_stream))
    assert rc == _capi.OK, _capi.last_error()
    return y


# (qtype, n, k, first m, second m, path both calls take, exact).  Not exact: the
# batched decode's split k meets by atomics; a prefill whose k split does not fit
# the scratch runs unsplit there, so the two agree to f32 rounding.
CASES = [
    (Q4_0, 4096, 4096, 4, 1, PATH_GEMV, True),
    (Q8_0, 5632, 2048, 2, 1, PATH_GEMV, True),
    (Q4_0, 14336, 4096, 64, 16, PATH_DECODE_MFMA, False),
    (Q8_0, 4096, 11008, 33, 5, PATH_DECODE_MFMA, False),
    (Q4_0, 14336, 4096, 2048, 512, PATH_PREFILL_MFMA, True),
    # 128-row tiles with k split 5 ways, then 8 ways: the same plans in both calls
    (Q4_0, 4096, 14336, 300, 130, PATH_PREFILL_MFMA, True),
    # the library call splits k over 256-row tiles, whose slabs do not fit the
    # scratch beside x: the no-allocation call runs 128-row tiles unsplit
    (Q4_0, 4096, 14336, 2048, 1100, PATH_PREFILL_MFMA, False),
]


@pytest.mark.parametrize("qtype,n,k,m1,m2,path,exact", CASES)
def test_noalloc_matches_qmatmul_twice(qtype, n, k, m1, m2, path, exact):
    lib = _capi.lib()
    w = oracle.normal(n * k, seed=n + k, std=0.02).reshape(n, k)
    blocks = oracle.quantize(qtype, w)
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    s = torch.cuda.Stream()
    for call, m in enumerate((m1, m2)):
        assert ql.select_path(m) == path or (path == PATH_PREFILL_MFMA and m > 64)
        xh = oracle.normal(m * k, seed=17 * m + call).reshape(m, k)
        x = torch.from_numpy(xh).cuda()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            a = _call(lib.unillm_hip_qmatmul_noalloc, ql, x, n, s)
            b = _call(lib.unillm_hip_qmatmul, ql, x, n, s)
        s.synchronize()
        a, b = a.cpu().numpy(), b.cpu().numpy()
        if exact:
            assert np.array_equal(a, b), (call, m)
        else:
            # the same k steps grouped differently in f32: ~1e-6 at these k
            assert oracle.normwise_error(a, b) < 1e-5, (call, m)
        rows = np.arange(m) if m <= 64 else np.array([0, 1, m // 2, m - 1])
        ref = oracle.qmatmul_f64(qtype, blocks, xh[rows], n, k)
        assert oracle.normwise_error(a[rows], ref) < 1e-3, (call, m)



def _random_cases(count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        qtype = Q4_0 if rng.random() < 0.6 else Q8_0
        r = rng.random()
        m1 = int(rng.integers(1, 5) if r < 0.3 else rng.integers(5, 65) if r < 0.65
                 else rng.integers(65, 700))
        k = int(rng.integers(1, 12000 // 32 + 1)) * 32
        n = int(rng.integers(1, 6000))
        while n * k > 8e6:
            n = max(1, n // 2)
        out.append((i, qtype, n, k, m1, int(rng.integers(1, m1 + 1)), int(rng.integers(1 << 30))))
    return out


@pytest.mark.parametrize("case", _random_cases(40, seed=20261205), ids=lambda c: f"r{c[0]}")
def test_noalloc_matches_qmatmul_random_shapes(case):
    # seeded random shapes over every path, two calls in a row (the second no larger),
    # each against unillm_hip_qmatmul on the same input to f32 rounding
    i, qtype, n, k, m1, m2, seed = case
    print(f"noalloc random {case}", flush=True)
    lib = _capi.lib()
    w = oracle.normal(n * k, seed=seed, std=0.02).reshape(n, k)
    ql = QuantLinear.from_blocks(qtype, n, k, oracle.quantize(qtype, w))
    s = torch.cuda.Stream()
    for call, m in enumerate((m1, m2)):
        x = torch.from_numpy(oracle.normal(m * k, seed=seed + 1 + call).reshape(m, k)).cuda()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            a = _call(lib.unillm_hip_qmatmul_noalloc, ql, x, n, s)
            b = _call(lib.unillm_hip_qmatmul, ql, x, n, s)
        s.synchronize()
        assert oracle.normwise_error(a.cpu().numpy(), b.cpu().numpy()) < 1e-5, (call, m)

def test_noalloc_under_graph_capture_without_reserve():
    # the case it exists for: a fresh stream (no workspace) captured straight away
    lib = _capi.lib()
    n, k, m = 2048, 4096, 16
    w = oracle.normal(n * k, seed=5, std=0.02).reshape(n, k)
    blocks = oracle.quantize(Q4_0, w)
    ql = QuantLinear.from_blocks(Q4_0, n, k, blocks)
    xh = oracle.normal(m * k, seed=6).reshape(m, k)
    x = torch.from_numpy(xh).cuda()
    y = torch.empty(m, n, device="cuda")
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
        rc = lib.unillm_hip_qmatmul_noalloc(ql._h, ctypes.c_void_p(x.data_ptr()), m,
                                            ctypes.c_void_p(y.data_ptr()),
                                            ctypes.c_void_p(s.cuda_stream))
    assert rc == _capi.OK, _capi.last_error()
    ref = oracle.qmatmul_f64(Q4_0, blocks, xh, n, k)
    for i in range(3):
        y.zero_()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3, i
    del g


def test_noalloc_rejects_beyond_scratch():
    # m k 2 bytes of f16 x beyond the 64 MiB scratch: refused before any launch
    lib = _capi.lib()
    n, k, m = 64, 16384, 2049
    assert m * k * 2 > SCRATCH_BYTES
    w = oracle.normal(n * k, seed=8, std=0.02).reshape(n, k)
    ql = QuantLinear.from_blocks(Q4_0, n, k, oracle.quantize(Q4_0, w))
    x = torch.zeros(m, k, device="cuda")
    y = torch.full((m, n), 7.0, device="cuda")
    torch.cuda.synchronize()
    rc = lib.unillm_hip_qmatmul_noalloc(ql._h, ctypes.c_void_p(x.data_ptr()), m,
                                        ctypes.c_void_p(y.data_ptr()), None)
    assert rc == _capi.ERR_UNSUPPORTED
    assert "bytes of scratch" in _capi.last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())  # nothing ran
