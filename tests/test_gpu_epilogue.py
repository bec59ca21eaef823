"""GPU parity of the fused epilogues (the scope table's row f3), through the C ABI.

- unillm_hip_qmatmul_add: y += x W^T, the decoder layer's residual add
  (llama.rs:668, 677) in the projection's epilogue;
- unillm_hip_qmatmul_swiglu: silu(x G^T) * (x U^T) for a [gate; up] weight
  (LlamaMLP, llama.rs:1275-1283; fused_swiglu, tensor_core.rs:1385-1396).

References: the oracle's f64 matmul, plus the residual / activation in f64;
where the kernel's own plain output is available, the fused result must equal
"plain output, then the op" (bitwise for the add where k is not split).
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import Q4_0, Q4_K, Q6_K, Q8_0
from unillm_amd import (PATH_DECODE_MFMA, PATH_GEMV, PATH_PREFILL_MFMA, HipError, QuantLinear)

pytestmark = pytest.mark.gpu

TOL = {PATH_GEMV: 1e-3, PATH_DECODE_MFMA: 1e-3, PATH_PREFILL_MFMA: 1e-3}  # Q4_0 / Q8_0: f16 operands


def _blocks(qtype, n, k, seed):
    if qtype == Q4_K:
        return oracle.random_q4_k(n, k, seed)
    if qtype == Q6_K:
        return oracle.random_q6_k(n, k, seed)
    return oracle.quantize(qtype, oracle.normal(n * k, seed=seed, std=0.02).reshape(n, k))


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("qtype,m,n,k,path", [
    (Q4_0, 1, 300, 4096, PATH_GEMV), (Q4_0, 3, 129, 2048, PATH_GEMV),
    (Q8_0, 2, 257, 2048, PATH_GEMV), (Q4_K, 1, 512, 4096, PATH_GEMV),
    (Q4_0, 16, 4096, 4096, PATH_DECODE_MFMA), (Q4_0, 64, 300, 4096, PATH_DECODE_MFMA),
    (Q6_K, 16, 257, 2048, PATH_DECODE_MFMA), (Q4_0, 256, 1024, 4096, PATH_PREFILL_MFMA),
    (Q8_0, 130, 256, 8192, PATH_PREFILL_MFMA)])
def test_residual_add(qtype, m, n, k, path):
    # (Q4_0, 64, 300, 4096) and (Q8_0, 130, 256, 8192) split k: the partials add onto y
    blocks = _blocks(qtype, n, k, seed=3 * n + k)
    x = oracle.normal(m * k, seed=n + 1).reshape(m, k)
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    assert ql.select_path(m) == path
    ref = oracle.qmatmul_f64(qtype, blocks, x, n, k)
    y0 = (oracle.normal(m * n, seed=n + 2).reshape(m, n) * float(np.abs(ref).max()))
    y0 = y0.astype(np.float32)
    print(f"add qtype={qtype} m={m} n={n} k={k}", flush=True)
    xd = _dev(x)
    y = _dev(y0)
    ql.forward_add(xd, y)
    plain = ql.forward(xd)
    torch.cuda.synchronize()
    y, plain = y.cpu().numpy(), plain.cpu().numpy()
    assert oracle.normwise_error(y, y0.astype(np.float64) + ref) < TOL[path]
    if path == PATH_GEMV:  # one rounding of y0 + the same row sum
        assert np.array_equal(y, y0 + plain)
    else:
        assert oracle.normwise_error(y, y0 + plain) < 1e-6


def _silu_mul(g, u):
    return g / (1.0 + np.exp(-g)) * u


@pytest.mark.parametrize("qtype,m,i_rows,k,path,fused", [
    (Q4_0, 1, 1376, 4096, PATH_GEMV, True), (Q4_0, 4, 300, 1024, PATH_GEMV, True),
    (Q4_K, 2, 512, 4096, PATH_GEMV, True), (Q8_0, 1, 700, 2048, PATH_GEMV, True),
    (Q6_K, 1, 257, 4096, PATH_GEMV, True), (Q4_0, 4, 300, 4096, PATH_GEMV, False),
    (Q6_K, 3, 257, 2048, PATH_GEMV, False), (Q8_0, 1, 256, 8192, PATH_GEMV, False),
    (Q4_0, 16, 1024, 4096, PATH_DECODE_MFMA, False), (Q4_K, 64, 300, 2048, PATH_DECODE_MFMA, False),
    (Q4_0, 256, 512, 4096, PATH_PREFILL_MFMA, False)])
def test_swiglu(qtype, m, i_rows, k, path, fused):
    # [gate; up] stacked as a load-time gate_up fusion would; fused = the GEMV pair
    # epilogue (tokens x 128-bit loads per row <= 4); past its reach the GEMV
    # stores into the workspace and an elementwise pass follows
    gate = _blocks(qtype, i_rows, k, seed=11 + i_rows)
    up = _blocks(qtype, i_rows, k, seed=12 + i_rows)
    gu = np.concatenate([gate.reshape(i_rows, -1), up.reshape(i_rows, -1)], axis=0)
    x = oracle.normal(m * k, seed=13).reshape(m, k)
    ql = QuantLinear.from_blocks(qtype, 2 * i_rows, k, gu)
    assert ql.select_path(m) == path
    print(f"swiglu qtype={qtype} m={m} I={i_rows} k={k}", flush=True)
    xd = _dev(x)
    act = ql.forward_swiglu(xd)
    plain = ql.forward(xd)
    torch.cuda.synchronize()
    act, plain = act.cpu().numpy(), plain.cpu().numpy()
    assert act.shape == (m, i_rows)
    g = oracle.qmatmul_f64(qtype, gate, x, i_rows, k)
    u = oracle.qmatmul_f64(qtype, up, x, i_rows, k)
    tol = 2e-3
    assert oracle.normwise_error(act, _silu_mul(g, u)) < tol
    # the same as the activation applied to the kernel's own gate / up outputs
    mine = _silu_mul(plain[:, :i_rows].astype(np.float64), plain[:, i_rows:].astype(np.float64))
    assert oracle.normwise_error(act, mine) < (1e-6 if fused or path == PATH_GEMV else 1e-5)


def test_swiglu_odd_rows_rejected():
    ql = QuantLinear.from_blocks(Q4_0, 3, 64, _blocks(Q4_0, 3, 64, seed=1))
    with pytest.raises(HipError):
        ql.forward_swiglu(torch.zeros(1, 64, device="cuda"))


def test_add_and_swiglu_m0_noop():
    ql = QuantLinear.from_blocks(Q4_0, 4, 64, _blocks(Q4_0, 4, 64, seed=2))
    y = torch.ones(0, 4, device="cuda")
    ql.forward_add(torch.zeros(0, 64, device="cuda"), y)
    assert ql.forward_swiglu(torch.zeros(0, 64, device="cuda")).shape == (0, 2)


# ---- the layer norm fused in front of the matmul (tensor_core.rs:973-1008) ------------------

def _layer_norm(x, gamma, beta, eps):
    # the reference's formula in f64: mean, mean of squared deviations, divide, scale
    x = x.astype(np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    out = (x - mu) / np.sqrt(var + eps) * gamma.astype(np.float64)
    return out + beta.astype(np.float64) if beta is not None else out


@pytest.mark.parametrize("qtype,m,n,k,path,bias,offset", [
    (Q4_0, 1, 300, 4096, PATH_GEMV, False, 0.0), (Q4_K, 3, 257, 2048, PATH_GEMV, True, 0.0),
    (Q8_0, 2, 129, 4096, PATH_GEMV, False, 100.0), (Q4_0, 16, 1024, 4096, PATH_DECODE_MFMA, True, 0.0),
    (Q4_0, 1, 256, 11008, PATH_DECODE_MFMA, False, 0.0), (Q6_K, 64, 300, 2048, PATH_DECODE_MFMA, False, 50.0),
    (Q8_0, 256, 512, 4096, PATH_PREFILL_MFMA, True, 0.0), (Q4_0, 130, 256, 8192, PATH_PREFILL_MFMA, False, 10.0),
    (Q4_0, 3, 128, 20480, PATH_DECODE_MFMA, True, 5.0), (Q8_0, 70, 128, 20480, PATH_PREFILL_MFMA, True, 5.0)])
def test_layer_norm_matmul(qtype, m, n, k, path, bias, offset):
    # offset: x = offset + N(0, 1) per row, so the mean dwarfs the deviations (a
    # one-pass variance would lose them); (Q4_0, 1, 256, 11008): past the GEMV's
    # norm reach, routed to batched decode; k = 20480: rows longer than the norm
    # kernel holds in registers (16 x 1024 elements), the rest read again
    blocks = _blocks(qtype, n, k, seed=5 * n + k)
    rng = np.random.default_rng(n + m)
    x = (oracle.normal(m * k, seed=k + m).reshape(m, k) + offset).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.normal(size=k)).astype(np.float32)
    beta = (0.1 * rng.normal(size=k)).astype(np.float32) if bias else None
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    print(f"norm qtype={qtype} m={m} n={n} k={k}", flush=True)
    y = ql.forward_norm(_dev(x), _dev(gamma), _dev(beta) if bias else None, eps=1e-6)
    torch.cuda.synchronize()
    xn = _layer_norm(x, gamma, beta, 1e-6)
    ref = oracle.qmatmul_f64(qtype, blocks, xn.astype(np.float32), n, k)
    tol = TOL[path]
    assert oracle.normwise_error(y.cpu().numpy(), ref) < tol


@pytest.mark.parametrize("qtype,m,n,k,bias,offset", [
    (Q4_0, 16, 4096, 4096, True, 0.0),
    (Q8_0, 7, 12288, 4096, False, 50.0),
    (Q4_K, 9, 40000, 1024, True, 0.0),    # more output rows than the device has CUs
    (Q6_K, 16, 640, 2048, False, 20.0),
    (Q4_0, 3, 1000, 4128, True, 0.0),     # k: 32 chunks of 128 and one block
    (Q8_0, 16, 512, 256, False, 0.0)])    # k: two chunks
def test_layer_norm_batched_decode_shapes(qtype, m, n, k, bias, offset):
    # the fused layer norm at m <= 16 on the batched decode, over k splits of 1 to 8
    # slices and ragged k.  Against the f64 reference, and against the same product
    # of x normalized first (torch, f32): the f16 operands then differ only where an
    # f32 rounding crosses an f16 one
    blocks = _blocks(qtype, n, k, seed=7 * n + k)
    rng = np.random.default_rng(m + n)
    x = (oracle.normal(m * k, seed=k + 3 * m).reshape(m, k) + offset).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.normal(size=k)).astype(np.float32)
    beta = (0.1 * rng.normal(size=k)).astype(np.float32) if bias else None
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    assert ql.select_path(m) == PATH_DECODE_MFMA
    print(f"norm in launch qtype={qtype} m={m} n={n} k={k}", flush=True)
    xd, gd = _dev(x), _dev(gamma)
    bd = _dev(beta) if bias else None
    y = ql.forward_norm(xd, gd, bd, eps=1e-5).cpu().numpy()
    xn = _layer_norm(x, gamma, beta, 1e-5)
    ref = oracle.qmatmul_f64(qtype, blocks, xn.astype(np.float32), n, k)
    assert oracle.normwise_error(y, ref) < 1e-3
    xt = torch.nn.functional.layer_norm(xd, (k,), gd, bd, eps=1e-5)
    assert oracle.normwise_error(y, ql.forward(xt).cpu().numpy()) < 1e-4
    # a second call: the same up to the order of the k slices' f32 adds
    y2 = ql.forward_norm(xd, gd, bd, eps=1e-5).cpu().numpy()
    assert oracle.normwise_error(y2, y) < 1e-5


@pytest.mark.parametrize("qtype,m,i_rows,k", [(Q4_0, 1, 1376, 4096), (Q4_K, 16, 300, 2048)])
def test_layer_norm_swiglu(qtype, m, i_rows, k):
    # post_attention_layernorm + gate + up + SwiGLU in one call (m = 1: the GEMV
    # pair epilogue on the normalized x; m = 16: batched decode + elementwise)
    gate = _blocks(qtype, i_rows, k, seed=21 + i_rows)
    up = _blocks(qtype, i_rows, k, seed=22 + i_rows)
    gu = np.concatenate([gate.reshape(i_rows, -1), up.reshape(i_rows, -1)], axis=0)
    rng = np.random.default_rng(3)
    x = (oracle.normal(m * k, seed=23).reshape(m, k) + 3.0).astype(np.float32)
    gamma = (1.0 + 0.1 * rng.normal(size=k)).astype(np.float32)
    ql = QuantLinear.from_blocks(qtype, 2 * i_rows, k, gu)
    act = ql.forward_swiglu(_dev(x), norm=(_dev(gamma), None, 1e-6)).cpu().numpy()
    xn = _layer_norm(x, gamma, None, 1e-6).astype(np.float32)
    g = oracle.qmatmul_f64(qtype, gate, xn, i_rows, k)
    u = oracle.qmatmul_f64(qtype, up, xn, i_rows, k)
    assert oracle.normwise_error(act, _silu_mul(g, u)) < 2e-3


@pytest.mark.parametrize("qtype,m,k,path", [(Q4_0, 16, 4096, PATH_DECODE_MFMA),
                                             (Q8_0, 5, 11008, PATH_DECODE_MFMA),
                                             (Q4_0, 64, 4096, PATH_DECODE_MFMA),
                                             (Q4_0, 96, 4096, PATH_PREFILL_MFMA)])
def test_layer_norm_any_gamma_magnitude(qtype, m, k, path):
    # the normalized rows times gamma ~ 1e6 (far past f16's 65504) or ~ 1e-7 (deep in
    # its subnormals): the MFMA paths scale their f16 operand by powers of two, so
    # every row stays as accurate as a unit one
    n = 256
    blocks = _blocks(qtype, n, k, seed=31 + k)
    x = oracle.normal(m * k, seed=17 + m).reshape(m, k)
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    assert ql.select_path(m) == path
    for g in (1e6, 1e-7):
        gamma = np.full(k, g, np.float32)
        y = ql.forward_norm(_dev(x), _dev(gamma), None, eps=1e-6).cpu().numpy()
        ref = oracle.qmatmul_f64(qtype, blocks, _layer_norm(x, gamma, None, 1e-6).astype(np.float32),
                                 n, k)
        for r in range(m):
            assert oracle.normwise_error(y[r:r + 1], ref[r:r + 1]) < 1e-3, (g, r)


def test_layer_norm_argument_checks():
    ql = QuantLinear.from_blocks(Q4_0, 4, 64, _blocks(Q4_0, 4, 64, seed=2))
    x = torch.zeros(1, 64, device="cuda")
    with pytest.raises(RuntimeError):  # gamma of the wrong length
        ql.forward_norm(x, torch.ones(32, device="cuda"))
    with pytest.raises(HipError):  # negative eps
        ql.forward_norm(x, torch.ones(64, device="cuda"), eps=-1.0)
