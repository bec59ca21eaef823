"""Randomized parity: seeded random shapes, paths, epilogues and KV-cache step sequences.

The other GPU tests pin chosen shapes (the BASELINE configs, tile and split
boundaries, edge sizes).  These draw (qtype of the five, m, n, k, path, epilogue, x offset,
x magnitude) and attention (heads, kv heads, head dim, RoPE theta, capacity, step
sizes, truncations) from a fixed seed, so every case is reproducible from its id,
and check each call against the f64 oracle at the same bars as the fixed tests:
1e-3 normwise for the projections (y0 + x W^T for the residual add, LN(x) W^T
for the fused norm), 1e-4 for attention.  SwiGLU is checked against the first-order
propagation of its product's own error (silu(g) u is ill-conditioned where g and u
are large but their product small), and the product itself against 1e-3.
Paths a shape does not take (the GEMV past its register budget, decode MFMA past
m = 64) must refuse with UNILLM_ERR_UNSUPPORTED rather than compute.
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import Q4_0, Q4_K, Q5_K, Q6_K, Q8_0
from unillm_amd import HipError, KvCache, QuantLinear
from unillm_amd import _capi

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _matmul_cases(count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        qt = [Q4_0, Q8_0, Q4_K, Q5_K, Q6_K][int(rng.choice(5, p=[0.35, 0.25, 0.15, 0.15, 0.1]))]
        unit = 256 if qt in (Q4_K, Q5_K, Q6_K) else 32
        r = rng.random()
        m = int(rng.integers(1, 5) if r < 0.3 else rng.integers(5, 17) if r < 0.55
                else rng.integers(17, 65) if r < 0.75 else rng.integers(65, 400))
        k = int(rng.integers(1, 12000 // unit + 1)) * unit
        n = int(rng.integers(1, 5000))
        while m * n * k > 3e8 or n * k > 8e6:
            n = max(1, n // 2)
        op = str(rng.choice(["fwd", "add", "swiglu", "norm", "normswiglu"],
                            p=[0.4, 0.2, 0.15, 0.15, 0.1]))
        if op.endswith("swiglu") and n % 2:
            n += 1
        path = int(rng.choice([0, 0, 0, 1, 2, 3]))
        out.append((i, qt, m, n, k, op, path, int(rng.random() < 0.2), int(rng.integers(1 << 30))))
    return out


def _blocks(qt, n, k, seed):
    if qt == Q4_K:
        return oracle.random_q4_k(n, k, seed)
    if qt == Q5_K:
        return oracle.random_q5_k(n, k, seed)
    if qt == Q6_K:
        return oracle.random_q6_k(n, k, seed)
    return oracle.quantize(qt, oracle.normal(n * k, seed=seed, std=0.02).reshape(n, k))


def _layer_norm(x, g, b, eps):
    x = x.astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    o = (x - mu) / np.sqrt(var + eps) * g.astype(np.float64)
    return o + b.astype(np.float64) if b is not None else o


@pytest.mark.parametrize("case", _matmul_cases(300, seed=20261202), ids=lambda c: f"c{c[0]}")
def test_random_matmul(case):
    i, qt, m, n, k, op, path, off, seed = case
    print(f"random matmul {case}", flush=True)
    crng = np.random.default_rng(seed + 7)
    blocks = _blocks(qt, n, k, seed)
    x = oracle.normal(m * k, seed=seed + 1).reshape(m, k)
    if "norm" not in op and crng.random() < 0.15:  # any finite x: a power-of-two magnitude
        x = x * np.float32(2.0 ** int(crng.integers(-60, 60)))
    ql = QuantLinear.from_blocks(qt, n, k, blocks)
    buf = torch.zeros(m * k + off, device="cuda")
    buf[off:] = torch.from_numpy(x.reshape(-1)).cuda()
    xd = buf[off:].view(m, k)
    g = (1.0 + 0.1 * crng.standard_normal(k)).astype(np.float32)
    b = (0.1 * crng.standard_normal(k)).astype(np.float32) if crng.random() < 0.5 else None
    norm = (torch.from_numpy(g).cuda(), torch.from_numpy(b).cuda() if b is not None else None, 1e-6)
    xn = _layer_norm(x, g, b, 1e-6).astype(np.float32)
    if op == "fwd":
        try:
            got = ql.forward(xd, path=path).cpu().numpy()
        except HipError as e:
            # a forced GEMV past its register budget, or decode MFMA past m = 64
            assert e.status == _capi.ERR_UNSUPPORTED, str(e)
            assert path == 1 or (path == 2 and m > 64), str(e)
            return
        ref = oracle.qmatmul_f64(qt, blocks, x, n, k, nthreads=8)
    elif op == "add":
        y0 = crng.standard_normal((m, n)).astype(np.float32)
        y = torch.from_numpy(y0).cuda()
        ql.forward_add(xd, y)
        got = y.cpu().numpy()
        ref = y0.astype(np.float64) + oracle.qmatmul_f64(qt, blocks, x, n, k, nthreads=8)
    elif op == "norm":
        got = ql.forward_norm(xd, *norm[:2], eps=norm[2]).cpu().numpy()
        ref = oracle.qmatmul_f64(qt, blocks, xn, n, k, nthreads=8)
    else:
        xin = x if op == "swiglu" else xn
        if op == "swiglu":
            got = ql.forward_swiglu(xd).cpu().numpy()
            prod = ql.forward(xd).cpu().numpy()
        else:
            got = ql.forward_swiglu(xd, norm=norm).cpu().numpy()
            prod = ql.forward_norm(xd, *norm[:2], eps=norm[2]).cpu().numpy()
        r = oracle.qmatmul_f64(qt, blocks, xin, n, k, nthreads=8)
        pe = oracle.normwise_error(prod, r)
        assert pe < TOL
        half = n // 2
        gg, uu = r[:, :half], r[:, half:]
        sg = 0.5 * (1.0 + np.tanh(0.5 * gg))  # sigmoid, without overflow
        ref = gg * sg * uu
        dg, du = pe * np.abs(gg).max(), pe * np.abs(uu).max()
        sens = (np.abs(sg * (1 + gg * (1 - sg)) * uu) * dg + np.abs(gg * sg) * du).max()
        assert np.isfinite(got).all()
        assert np.abs(got - ref).max() <= max(TOL * np.abs(ref).max(), 2 * sens)
        return
    torch.cuda.synchronize()
    assert np.isfinite(got).all()
    assert oracle.normwise_error(got, ref) < TOL


def _attention_sequences(count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        D = int(rng.choice([64, 128, 256]))
        KVH = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.choice([1, 1, 2, 4, 8]))
        while KVH * G * D > 4096 and KVH > 1:
            KVH //= 2
        max_seq = int(rng.integers(8, 1500))
        steps = []
        for _ in range(int(rng.integers(1, 6))):
            r = rng.random()
            m = int(rng.integers(1, 5) if r < 0.5 else rng.integers(5, 40) if r < 0.8
                    else rng.integers(40, 160))
            trunc = float(rng.random()) if rng.random() < 0.2 else -1.0
            steps.append((m, trunc, int(rng.integers(1 << 30))))
        out.append((i, KVH * G, KVH, D, float(rng.choice([1e4, 5e5])), max_seq, steps))
    return out


@pytest.mark.parametrize("seq", _attention_sequences(100, seed=20261203), ids=lambda s: f"s{s[0]}")
def test_random_attention_sequence(seq):
    i, H, KVH, D, theta, max_seq, steps = seq
    print(f"random attention {seq[:6]} steps={[s[:2] for s in steps]}", flush=True)
    kv = KvCache(KVH, D, max_seq, theta)
    kc = np.zeros((KVH, max_seq, D), np.float32)
    vc = np.zeros((KVH, max_seq, D), np.float32)
    length = 0
    for m, trunc, seed in steps:
        if trunc >= 0.0:
            length = int(trunc * length)
            kv.truncate(length)
        m = min(m, max_seq - length)
        if m <= 0:
            break
        qkv = oracle.normal(m * (H + 2 * KVH) * D, seed=seed).reshape(m, -1)
        out = kv.attention(torch.from_numpy(qkv).cuda(), H).cpu().numpy()
        ref = oracle.attention_decode(qkv, H, KVH, D, theta, kc, vc, length)
        length += m
        assert kv.seq_len == length
        assert np.isfinite(out).all()
        assert oracle.normwise_error(out, ref) < 1e-4
    kv.close()


def _capture_cases(count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        qt = [Q4_0, Q8_0, Q4_K, Q5_K, Q6_K][int(rng.choice(5, p=[0.35, 0.25, 0.15, 0.15, 0.1]))]
        unit = 256 if qt in (Q4_K, Q5_K, Q6_K) else 32
        r = rng.random()
        m = int(rng.integers(1, 5) if r < 0.3 else rng.integers(5, 17) if r < 0.55
                else rng.integers(17, 65) if r < 0.75 else rng.integers(65, 600))
        k = int(rng.integers(1, 12000 // unit + 1)) * unit
        n = int(rng.integers(1, 6000))
        while n * k > 8e6:
            n = max(1, n // 2)
        op = str(rng.choice(["fwd", "add", "swiglu", "norm", "normswiglu"]))
        if op.endswith("swiglu") and n % 2:
            n += 1
        out.append((i, qt, m, n, k, op, int(rng.integers(1 << 30))))
    return out


@pytest.mark.parametrize("case", _capture_cases(60, seed=20261204), ids=lambda c: f"g{c[0]}")
def test_random_capture_replays_match_eager(case):
    """reserve, then one call captured into a HIP graph on its own stream: three replays
    with eager work between them, each equal to the eager call (to f32 rounding where
    the batched decode's split k adds by atomics; bitwise elsewhere)."""
    i, qt, m, n, k, op, seed = case
    print(f"random capture {case}", flush=True)
    crng = np.random.default_rng(seed + 3)
    ql = QuantLinear.from_blocks(qt, n, k, _blocks(qt, n, k, seed))
    x = torch.from_numpy(oracle.normal(m * k, seed=seed + 1).reshape(m, k)).cuda()
    g = torch.from_numpy((1.0 + 0.1 * crng.standard_normal(k)).astype(np.float32)).cuda()
    b = torch.from_numpy((0.1 * crng.standard_normal(k)).astype(np.float32)).cuda()
    nout = n // 2 if op.endswith("swiglu") else n
    y0 = torch.from_numpy(crng.standard_normal((m, nout)).astype(np.float32)).cuda()
    s = torch.cuda.Stream()
    ql.reserve(m, swiglu=op.endswith("swiglu"), stream=s)

    def call(out):
        if op == "fwd":
            ql.forward(x, out=out, stream=s)
        elif op == "add":
            ql.forward_add(x, out, stream=s)
        elif op == "norm":
            ql.forward_norm(x, g, b, eps=1e-6, out=out, stream=s)
        elif op == "swiglu":
            ql.forward_swiglu(x, out=out, stream=s)
        else:
            ql.forward_swiglu(x, out=out, stream=s, norm=(g, b, 1e-6))

    with torch.cuda.stream(s):
        eager = y0.clone()
        call(eager)
    s.synchronize()
    out = torch.empty(m, nout, device="cuda")
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=s, capture_error_mode="thread_local"):
        call(out)
    scale = max(eager.abs().max().item(), 1e-30)
    for rep in range(3):
        out.copy_(y0)
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            gr.replay()
        s.synchronize()
        assert (out - eager).abs().max().item() <= 1e-6 * scale, rep
        with torch.cuda.stream(s):  # eager work between replays
            ql.forward(x, stream=s)
        s.synchronize()
    del gr
