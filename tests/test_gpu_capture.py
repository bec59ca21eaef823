"""HIP-graph capture of the matmul and attention calls, and their per-stream workspace.

The MFMA paths keep x in a per-stream device buffer that grows on first use.
Growing allocates, which a capture cannot record: such a call must fail with a
clear error and leave the capture usable, and a reserved stream must capture and
replay correctly, also after later eager calls have grown the buffer again.
Replays are checked against eager calls, with eager work and synchronisations
between them.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from oracle import Q4_0
from unillm_amd import (PATH_DECODE_MFMA, PATH_GEMV, PATH_PREFILL_MFMA, HipError, KvCache,
                        QuantLinear, _capi)

pytestmark = pytest.mark.gpu


def _weight(n, k, seed):
    w = oracle.normal(n * k, seed=seed, std=0.02).reshape(n, k)
    b = oracle.quantize(Q4_0, w)
    return b, QuantLinear.from_blocks(Q4_0, n, k, b)


def _x(m, k, seed):
    return torch.from_numpy(oracle.normal(m * k, seed=seed).reshape(m, k)).cuda()


def test_capture_with_cold_workspace_fails_cleanly():
    _, ql = _weight(512, 1024, seed=11)
    # a stream no call has used, so it has no workspace yet (torch's pooled streams
    # may carry one from earlier tests)
    h = ctypes.c_void_p()
    _capi.check(_capi.lib().unillm_hip_stream_create(ctypes.byref(h)))
    s = torch.cuda.ExternalStream(h.value)
    x = _x(16, 1024, seed=12)
    y = torch.empty(16, 512, device="cuda")
    g = torch.cuda.CUDAGraph()
    with pytest.raises(HipError, match="while the stream is being captured"):
        with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
            ql.forward(x, out=y, path=PATH_DECODE_MFMA, stream=s)
    del g
    torch.cuda.synchronize()
    # the stream still works eagerly afterwards
    with torch.cuda.stream(s):
        ql.forward(x, out=y, path=PATH_DECODE_MFMA, stream=s)
    s.synchronize()
    assert torch.isfinite(y).all()


@pytest.mark.parametrize("m,path", [(16, PATH_DECODE_MFMA), (300, PATH_PREFILL_MFMA)])
def test_reserved_stream_captures_and_replays(m, path):
    n, k = 1024, 2048
    blocks, ql = _weight(n, k, seed=21 + m)
    s = torch.cuda.Stream()
    ql.reserve(m, stream=s)
    x = _x(m, k, seed=22 + m)
    y = torch.empty(m, n, device="cuda")
    with torch.cuda.stream(s):
        eager = ql.forward(x, path=path, stream=s).clone()
    s.synchronize()
    ref = oracle.qmatmul_f64(Q4_0, blocks, x.cpu().numpy(), n, k)
    assert oracle.normwise_error(eager.cpu().numpy(), ref) < 1e-3
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
        ql.forward(x, out=y, path=path, stream=s)
    big = _x(2048, k, seed=23)
    for i in range(4):
        y.zero_()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        if path == PATH_PREFILL_MFMA:  # split k slabs summed in a fixed order: exact
            assert np.array_equal(y.cpu().numpy(), eager.cpu().numpy()), i
        else:  # batched decode: split k ranges meet by f32 atomics, in any order
            assert oracle.normwise_error(y.cpu().numpy(), eager.cpu().numpy()) < 1e-6, i
        # eager work between replays; the second one grows the stream's workspace
        # (the captured buffer is retired, not freed, so the graph stays valid)
        with torch.cuda.stream(s):
            ql.forward(big if i == 1 else x, path=PATH_PREFILL_MFMA, stream=s)
        s.synchronize()
    del g


@pytest.mark.parametrize("m,path", [(1, PATH_GEMV), (16, PATH_DECODE_MFMA),
                                    (300, PATH_PREFILL_MFMA)])
def test_reserved_stream_captures_x_on_a_4_byte_boundary(m, path):
    # x one float past a 16-byte boundary is first copied into an aligned workspace:
    # the reserve covers that copy too, on every path
    n, k = 1024, 2048
    blocks, ql = _weight(n, k, seed=61 + m)
    s = torch.cuda.Stream()
    ql.reserve(m, stream=s)
    buf = torch.empty(m * k + 1, device="cuda")
    x = buf[1:].view(m, k)
    x.copy_(_x(m, k, seed=62 + m))
    y = torch.empty(m, n, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
        ql.forward(x, out=y, path=path, stream=s)
    ref = oracle.qmatmul_f64(Q4_0, blocks, x.cpu().numpy(), n, k)
    for i in range(3):
        y.zero_()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3, i
        with torch.cuda.stream(s):  # eager work between replays
            ql.forward(x, path=path, stream=s)
        s.synchronize()
    del g


def test_reserved_attention_captures_and_replays():
    H, KVH, D, L = 8, 2, 128, 256
    s = torch.cuda.Stream()
    kv = KvCache(KVH, D, L)
    kv.reserve(1, H, stream=s)
    w = (H + 2 * KVH) * D
    pre = _x(40, w, seed=31)
    q1 = _x(1, w, seed=32)
    out = torch.empty(1, H * D, device="cuda")
    with torch.cuda.stream(s):
        for t in range(40):
            kv.attention(pre[t:t + 1].contiguous(), H, stream=s)
        eager = kv.attention(q1, H, stream=s).clone()
    s.synchronize()
    kv.truncate(40)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
        kv.attention(q1, H, out=out, stream=s)
    for i in range(3):
        kv.truncate(40)
        out.zero_()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        assert torch.equal(out, eager), i


def test_attention_reserve_covers_every_shorter_call():
    # Reserving for 2048 tokens covers every shorter call, though the need is not
    # monotone in m: a 512-token prompt at 32 heads splits its key range and keeps
    # partials (more workspace than the unsplit 2048-token call), and a 4-token decode
    # step keeps per-chunk partials.  Both capture without growing the workspace.
    H, KVH, D = 32, 8, 128
    s = torch.cuda.Stream()
    kv = KvCache(KVH, D, 2048)
    kv.reserve(2048, H, stream=s)
    w = (H + 2 * KVH) * D
    for m in (512, 4):
        x = _x(m, w, seed=40 + m)
        out = torch.empty(m, H * D, device="cuda")
        kv.truncate(0)
        with torch.cuda.stream(s):
            eager = kv.attention(x, H, stream=s).clone()
        s.synchronize()
        kv.truncate(0)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
            kv.attention(x, H, out=out, stream=s)
        kv.truncate(0)
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        assert torch.equal(out, eager), m
        del g


@pytest.mark.parametrize("n,k", [(4096, 14336), (14336, 4096)])
def test_qmatmul_reserve_covers_every_shorter_call(n, k):
    # Reserving for 2048 rows covers every shorter prefill, whatever its plan:
    # 128-row tiles split up to 16 ways (m65-300), 256-row tiles split up to 8 ways
    # (deep k, m500-1536), unsplit tiles of either height.  Each call is captured
    # first, so a workspace that had to grow would fail the capture; its replay then
    # matches an eager call bit for bit.
    _, ql = _weight(n, k, seed=50 + k)
    s = torch.cuda.Stream()
    ql.reserve(2048, stream=s)
    for m in (65, 100, 130, 256, 300, 500, 600, 700, 768, 1024, 1100, 1280, 1536, 2048):
        print(f"reserve covers n={n} k={k} m={m}", flush=True)
        x = _x(m, k, seed=51 + m)
        y = torch.empty(m, n, device="cuda")
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s, capture_error_mode="thread_local"):
            ql.forward(x, out=y, path=PATH_PREFILL_MFMA, stream=s)
        with torch.cuda.stream(s):
            g.replay()
            eager = ql.forward(x, path=PATH_PREFILL_MFMA, stream=s)
        s.synchronize()
        assert torch.equal(y, eager), m
        del g
