"""Dense projection weights (GGML F32 / F16 / BF16), through the C ABI.

candle's QMatMul::from_arc keeps such a tensor as a dequantized f32 tensor and
multiplies in f32 (its Tensor variant); the reference's loader wraps every *_proj /
lm_head tensor in a QMatMul whatever its type (weight_loader_core.rs:554-571).  The
device holds the f32 rows (F16 and BF16 widen exactly) and runs an f32 GEMM.

References: numpy float64 of the same widened weights (exact), x in f64; the f32
GEMM's rounding over k terms stays near 1e-7 relative, so the bar is 1e-5 normwise.
The epilogues (residual add, SwiGLU, layer norm in front) are checked against the
same f64 formulas as the quantized paths' tests.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from unillm_amd import (BF16, F16, F32, PATH_DECODE_MFMA, PATH_DENSE, PATH_GEMV, HipError,
                        QuantLinear, _capi)

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _weight(qtype, n, k, seed):
    """GGUF bytes of a dense [n, k] tensor and its exact f64 values."""
    w32 = (np.random.default_rng(seed).standard_normal((n, k)) * 0.05).astype(np.float32)
    if qtype == F32:
        return w32.tobytes(), w32.astype(np.float64)
    if qtype == F16:
        h = w32.astype(np.float16)
        return h.tobytes(), h.astype(np.float64)
    # BF16: round to nearest even on the upper 16 bits
    u = w32.view(np.uint32).astype(np.uint64)
    b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return b.tobytes(), (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _x(m, k, seed):
    return np.random.default_rng(seed).standard_normal((m, k)).astype(np.float32)


@pytest.mark.parametrize("qtype", [F32, F16, BF16])
@pytest.mark.parametrize("m,n,k", [(1, 300, 257), (3, 64, 4096), (17, 1000, 512), (300, 513, 768)])
def test_dense_matmul_matches_f64(qtype, m, n, k):
    raw, w = _weight(qtype, n, k, seed=7 * n + k)
    ql = QuantLinear.from_blocks(qtype, n, k, raw)
    assert ql.select_path(m) == PATH_DENSE
    x = _x(m, k, seed=m + n)
    print(f"dense qtype={qtype} m={m} n={n} k={k}", flush=True)
    y = ql.forward(_dev(x))
    torch.cuda.synchronize()
    ref = x.astype(np.float64) @ w.T
    assert oracle.normwise_error(y.cpu().numpy(), ref) < TOL
    # the product is the same bits on every call (the GEMM runs without atomics)
    assert torch.equal(ql.forward(_dev(x)), y)


@pytest.mark.parametrize("qtype", [F32, F16, BF16])
def test_dense_dequant_is_the_exact_widening(qtype):
    n, k = 37, 129
    raw, w = _weight(qtype, n, k, seed=5)
    ql = QuantLinear.from_blocks(qtype, n, k, raw)
    out = torch.empty(n, k, device="cuda")
    _capi.check(_capi.lib().unillm_hip_dequant(ql._h, ctypes.c_void_p(out.data_ptr()), None))
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().astype(np.float64), w)


def test_dense_from_torch_tensor_equals_from_bytes():
    n, k, m = 96, 200, 5
    wt = torch.randn(n, k, device="cuda", dtype=torch.float16) * 0.05
    a = QuantLinear.from_dense(wt)
    b = QuantLinear.from_blocks(F16, n, k, wt.cpu().numpy().tobytes())
    assert a.qtype == F16 and a.shape == (n, k)
    x = torch.randn(m, k, device="cuda")
    assert torch.equal(a.forward(x), b.forward(x))
    # and as f32 rows: the same as an f32 weight holding the widened values
    c = QuantLinear.from_dense(wt.float())
    assert torch.equal(c.forward(x), a.forward(x))


def _layer_norm(x, gamma, beta, eps):
    x = x.astype(np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    out = (x - mu) / np.sqrt(var + eps) * gamma.astype(np.float64)
    return out + beta.astype(np.float64) if beta is not None else out


def _silu_mul(g, u):
    return g / (1.0 + np.exp(-g)) * u


@pytest.mark.parametrize("m", [1, 9, 130])
def test_dense_epilogues(m):
    k, i_rows = 384, 200
    raw, w = _weight(F16, 2 * i_rows, k, seed=m)
    ql = QuantLinear.from_blocks(F16, 2 * i_rows, k, raw)
    x = _x(m, k, seed=11 * m)
    rng = np.random.default_rng(m)
    gamma = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(k)).astype(np.float32)
    y0 = rng.standard_normal((m, 2 * i_rows)).astype(np.float32)
    xd, gd, bd = _dev(x), _dev(gamma), _dev(beta)
    print(f"dense epilogues m={m}", flush=True)
    # residual add: y += x W^T
    y = _dev(y0)
    ql.forward_add(xd, y)
    ref = x.astype(np.float64) @ w.T
    assert oracle.normwise_error(y.cpu().numpy(), y0 + ref) < TOL
    # SwiGLU on [gate; up]
    act = ql.forward_swiglu(xd)
    assert oracle.normwise_error(act.cpu().numpy(), _silu_mul(ref[:, :i_rows], ref[:, i_rows:])) < TOL
    # layer norm in front, with and without bias, and in front of SwiGLU
    xn = _layer_norm(x, gamma, beta, 1e-6)
    got = ql.forward_norm(xd, gd, bd, eps=1e-6)
    assert oracle.normwise_error(got.cpu().numpy(), xn @ w.T) < TOL
    got = ql.forward_norm(xd, gd, None, eps=1e-5)
    assert oracle.normwise_error(got.cpu().numpy(), _layer_norm(x, gamma, None, 1e-5) @ w.T) < TOL
    rn = xn @ w.T
    act = ql.forward_swiglu(xd, norm=(gd, bd, 1e-6))
    assert oracle.normwise_error(act.cpu().numpy(), _silu_mul(rn[:, :i_rows], rn[:, i_rows:])) < TOL


def test_dense_x_on_a_4_byte_boundary():
    n, k, m = 100, 300, 4
    raw, w = _weight(F32, n, k, seed=1)
    ql = QuantLinear.from_blocks(F32, n, k, raw)
    x = _x(m, k, seed=2)
    buf = torch.zeros(m * k + 1, device="cuda")
    buf[1:] = _dev(x).reshape(-1)
    y = ql.forward(buf[1:].view(m, k))
    assert oracle.normwise_error(y.cpu().numpy(), x.astype(np.float64) @ w.T) < TOL


def test_dense_refuses_the_quantized_paths_and_the_no_allocation_entry():
    n, k, m = 64, 128, 2
    raw, _ = _weight(F16, n, k, seed=3)
    ql = QuantLinear.from_blocks(F16, n, k, raw)
    x = _dev(_x(m, k, seed=4))
    for path in (PATH_GEMV, PATH_DECODE_MFMA):
        with pytest.raises(HipError, match="dense path"):
            ql.forward(x, path=path)
    y = torch.empty(m, n, device="cuda")
    rc = _capi.lib().unillm_hip_qmatmul_noalloc(ql._h, ctypes.c_void_p(x.data_ptr()), m,
                                                ctypes.c_void_p(y.data_ptr()), None)
    assert rc == _capi.ERR_UNSUPPORTED and "quantized weights only" in _capi.last_error()
    # the device quantizer does not make dense "blocks"
    w = torch.zeros(n, k, device="cuda")
    out = torch.empty(n * k * 2, dtype=torch.uint8, device="cuda")
    rc = _capi.lib().unillm_hip_quantize(F16, ctypes.c_void_p(w.data_ptr()), n, k,
                                         ctypes.c_void_p(out.data_ptr()), None)
    assert rc == _capi.ERR_UNSUPPORTED


def test_dense_reserved_stream_captures_and_replays():
    n, k, m = 512, 1024, 16
    raw, w = _weight(BF16, n, k, seed=9)
    ql = QuantLinear.from_blocks(BF16, n, k, raw)
    s = torch.cuda.Stream()
    ql.reserve(m, stream=s)
    x = _dev(_x(m, k, seed=10))
    gamma = _dev(np.ones(k, np.float32))
    with torch.cuda.stream(s):
        eager = ql.forward_norm(x, gamma, None, eps=1e-6, stream=s).clone()
    s.synchronize()
    y = torch.empty(m, n, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
        ql.forward_norm(x, gamma, None, eps=1e-6, out=y, stream=s)
    for i in range(3):
        y.zero_()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        assert torch.equal(y, eager), i
        with torch.cuda.stream(s):  # eager work between replays
            ql.forward(x, stream=s)
        s.synchronize()
    ref = _layer_norm(x.cpu().numpy(), np.ones(k, np.float32), None, 1e-6) @ w.T
    assert oracle.normwise_error(y.cpu().numpy(), ref) < TOL
    del g
