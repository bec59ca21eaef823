"""GPU parity of decode attention with a KV cache (the scope table's row f4).

Against the oracle (oracle_attention_decode: RoPE as apply_rope_with_offset,
llama.rs:827-883; LayerKVCache::append, kv_cache.rs:91-130; causal softmax
attention of forward_with_cache, llama.rs:1108-1150, in f64), whose closed
forms, RoPE known answers and invariants are pinned in tests/test_oracle.py.
Bar: 1e-4 normwise (f32 throughout; the device's sincosf / expf differ from the
CPU's by ulps).
"""
import numpy as np
import pytest
import torch

import oracle
from unillm_amd import HipError, KvCache

pytestmark = pytest.mark.gpu


def _run_steps(H, KVH, D, steps, theta=10000.0, max_seq=None, seed=0):
    # a sequence fed in steps of m tokens; each step checked against the oracle,
    # whose cache mirrors the device's
    max_seq = max_seq or sum(steps) + 3
    kv = KvCache(KVH, D, max_seq, theta)
    kc = np.zeros((KVH, max_seq, D), np.float32)
    vc = np.zeros((KVH, max_seq, D), np.float32)
    length, worst = 0, 0.0
    for i, m in enumerate(steps):
        qkv = oracle.normal(m * (H + 2 * KVH) * D, seed=seed + i).reshape(m, -1)
        out = kv.attention(torch.from_numpy(qkv).cuda(), H).cpu().numpy()
        ref = oracle.attention_decode(qkv, H, KVH, D, theta, kc, vc, length)
        length += m
        assert kv.seq_len == length
        worst = max(worst, oracle.normwise_error(out, ref))
    return worst


@pytest.mark.parametrize("H,KVH,D,steps", [
    (4, 4, 64, [1, 1, 1]), (8, 2, 128, [4, 1, 1, 3]), (32, 8, 128, [1, 2, 1]),
    (8, 8, 256, [2, 1]), (4, 1, 128, [4, 4]),
    # hd 64 with 12 and 16 queries a kv head (more queries than the 8 lanes of a position)
    (8, 2, 64, [4, 3]),
    # 16 queries a kv head at hd 256 (the largest LDS footprint), and 16 new tokens at G = 1
    (16, 1, 256, [1, 1]), (2, 2, 64, [16, 16])])
def test_attention_steps(H, KVH, D, steps):
    print(f"attention H={H} KVH={KVH} D={D} steps={steps}", flush=True)
    assert _run_steps(H, KVH, D, steps) < 1e-4


def test_attention_long_context_many_chunks():
    # a prefix of 3000 positions (many sequence chunks), then decode steps
    H, KVH, D, L = 32, 8, 128, 3000
    max_seq = 4096
    kv = KvCache(KVH, D, max_seq)
    kc = np.zeros((KVH, max_seq, D), np.float32)
    vc = np.zeros((KVH, max_seq, D), np.float32)
    length = 0
    rng_i = 0
    while length < L:  # fill with m = 2 steps (G = 4: 8 queries a kv head)
        m = 2
        qkv = oracle.normal(m * (H + 2 * KVH) * D, seed=100 + rng_i).reshape(m, -1)
        rng_i += 1
        kv.attention(torch.from_numpy(qkv).cuda(), H)
        oracle.attention_decode(qkv, H, KVH, D, 10000.0, kc, vc, length)
        length += m
    qkv = oracle.normal((H + 2 * KVH) * D, seed=7).reshape(1, -1)
    out = kv.attention(torch.from_numpy(qkv).cuda(), H).cpu().numpy()
    ref = oracle.attention_decode(qkv, H, KVH, D, 10000.0, kc, vc, length)
    assert oracle.normwise_error(out, ref) < 1e-4


def test_attention_truncate_then_append_matches_fresh_sequence():
    # a rolled-back step (speculative decoding) must leave no trace: run two steps,
    # truncate the second away, run a different second step -- equal to a cache
    # that only ever saw step 1 then that step
    H, KVH, D = 8, 2, 64
    w = (H + 2 * KVH) * D
    a = oracle.normal(2 * w, seed=31).reshape(2, w)
    b = oracle.normal(3 * w, seed=32).reshape(3, w)
    c = oracle.normal(1 * w, seed=33).reshape(1, w)
    kv1, kv2 = KvCache(KVH, D, 16), KvCache(KVH, D, 16)
    kv1.attention(torch.from_numpy(a).cuda(), H)
    kv1.attention(torch.from_numpy(b).cuda(), H)
    kv1.truncate(2)
    o1 = kv1.attention(torch.from_numpy(c).cuda(), H).cpu().numpy()
    kv2.attention(torch.from_numpy(a).cuda(), H)
    o2 = kv2.attention(torch.from_numpy(c).cuda(), H).cpu().numpy()
    assert np.array_equal(o1, o2)


def test_attention_overflow_and_limits():
    kv = KvCache(2, 64, 4)
    qkv = torch.zeros(3, (4 + 4) * 64, device="cuda")
    kv.attention(qkv, 4)
    with pytest.raises(HipError, match="KV cache overflow"):
        kv.attention(torch.zeros(2, 8 * 64, device="cuda"), 4)
    assert kv.seq_len == 3
    kv.truncate(1)  # roll back two positions
    assert kv.seq_len == 1
    with pytest.raises(HipError):
        kv.truncate(2)  # only shortens
    kv.clear()
    assert kv.seq_len == 0
    with pytest.raises(HipError):  # 17 queries a kv head: past decode's limit
        KvCache(1, 64, 64).attention(torch.zeros(17, 3 * 64, device="cuda"), 1)
    with pytest.raises(HipError):  # head_dim 96 unsupported
        KvCache(1, 96, 8)


def test_attention_graph_replays_match_eager():
    # a call is two launches (per-chunk partial results in the stream workspace, then
    # the merge) and the cache length is host state baked into the captured launch: a
    # captured call replayed several times (eager work and synchronisations between
    # the replays) must give the eager result every time, bit for bit
    H, KVH, D, L = 32, 8, 128, 700
    w = (H + 2 * KVH) * D
    kv = KvCache(KVH, D, L + 1)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        fill = torch.from_numpy(oracle.normal(4 * w, seed=51).reshape(4, w)).cuda()
        while kv.seq_len + 4 <= L - 1:
            kv.attention(fill, H, stream=stream)
        while kv.seq_len < L - 1:
            kv.attention(fill[:1].contiguous(), H, stream=stream)
        q1 = torch.from_numpy(oracle.normal(w, seed=52).reshape(1, w)).cuda()
        out = torch.empty(1, H * D, device="cuda")
        kv.attention(q1, H, out=out, stream=stream)
        eager = out.clone()
        kv.truncate(L - 1)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
            kv.attention(q1, H, out=out, stream=stream)
        kv.truncate(L - 1)
        for i in range(4):
            out.zero_()
            g.replay()
            stream.synchronize()
            assert torch.equal(out, eager), f"replay {i} differs from the eager call"
            kv.attention(q1, H, stream=stream)  # eager work between replays
            kv.truncate(L - 1)
            stream.synchronize()
