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


def test_attention_decode_past_4096_with_32_kv_heads():
    # with 32 kv heads the CUs fill with chunks of L / 16 positions, beyond the
    # 256-position maximum once L > 4096: the chunk length must cap, not fail.  The
    # decode step's output for token 4100 is checked against the prompt path's
    # output for the same token (the prompt path's own parity is pinned above; the
    # oracle's f64 loop over a 4101-token prompt would take minutes)
    H, KVH, D, L = 32, 32, 128, 4100
    w = (H + 2 * KVH) * D
    qkv = torch.from_numpy(oracle.normal((L + 2) * w, seed=41).reshape(L + 2, w)).cuda()
    a, b = KvCache(KVH, D, L + 8), KvCache(KVH, D, L + 8)
    whole = a.attention(qkv, H).cpu().numpy()
    b.attention(qkv[:L].contiguous(), H)
    for t in (L, L + 1):
        step = b.attention(qkv[t:t + 1].contiguous(), H).cpu().numpy()
        assert oracle.normwise_error(step, whole[t:t + 1].astype(np.float64)) < 1e-5
    assert b.seq_len == L + 2


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
    with pytest.raises(HipError):  # head_dim 96 unsupported
        KvCache(1, 96, 8)
    # a prompt-length call past max_seq: the same message, nothing appended
    kv = KvCache(2, 64, 40)
    with pytest.raises(HipError, match="KV cache overflow"):
        kv.attention(torch.zeros(41, 8 * 64, device="cuda"), 4)
    assert kv.seq_len == 0


def test_attention_out_offset_by_one_float():
    # out on a 4-byte boundary: a decode step stores per float and matches the
    # oracle; a prompt-length call (16-byte stores) is refused before any launch
    H, KVH, D = 8, 2, 64
    w = (H + 2 * KVH) * D
    kv = KvCache(KVH, D, 64)
    kc = np.zeros((KVH, 64, D), np.float32)
    vc = np.zeros((KVH, 64, D), np.float32)
    for pos, m in enumerate((1, 2)):
        length = kv.seq_len
        qkv = oracle.normal(m * w, seed=60 + pos).reshape(m, w)
        buf = torch.full((m * H * D + 1,), 7.0, device="cuda")
        kv.attention(torch.from_numpy(qkv).cuda(), H, out=buf[1:].view(m, H * D))
        ref = oracle.attention_decode(qkv, H, KVH, D, 10000.0, kc, vc, length)
        got = buf.cpu().numpy()
        assert got[0] == 7.0
        assert oracle.normwise_error(got[1:].reshape(m, H * D), ref) < 1e-4
    buf = torch.zeros(20 * H * D + 1, device="cuda")
    with pytest.raises(HipError, match="16-byte aligned"):
        kv.attention(torch.zeros(20, w, device="cuda"), H, out=buf[1:].view(20, H * D))
    assert kv.seq_len == 3
    assert not bool(buf.any())


# ---- prompt-length calls (the prefill of generate_with_cache, llama.rs:488-497) ---------------

@pytest.mark.parametrize("H,KVH,D,steps", [
    (4, 4, 64, [17]),            # 17 queries a kv head: just past a decode step
    (32, 8, 128, [64]),          # Llama-2-7B-like GQA, one full query block
    (32, 32, 128, [300, 1, 1]),  # MHA prompt (ragged blocks), then decode steps
    (8, 2, 64, [130, 70]),       # a second prompt-length call on a filled cache
    (16, 2, 256, [100, 2]),      # hd 256 (32-query blocks)
    (4, 1, 128, [513]),          # MQA, blocks of 64 plus one query
])
def test_attention_prompt_parity(H, KVH, D, steps):
    print(f"prompt attention H={H} KVH={KVH} D={D} steps={steps}", flush=True)
    assert _run_steps(H, KVH, D, steps, seed=7 * D + H) < 1e-4


def test_attention_prompt_long_context():
    # a 512-token prompt onto 700 cached positions, Llama-2-7B heads
    H, KVH, D = 32, 32, 128
    assert _run_steps(H, KVH, D, [350, 350, 512], max_seq=1300, seed=3) < 1e-4


@pytest.mark.parametrize("KVH", [8, 32])
def test_attention_prompt_unsplit_matches_split(KVH):
    # A 2048-token prompt at 32 heads has query waves enough for the chip and runs in
    # one kernel.  The same prompt as two 1024-token calls splits each workgroup's key
    # tiles in two and merges the partials, the path the oracle tests above pin (their
    # sizes all split).  The two outputs agree to f32 rounding.
    H, D, m = 32, 128, 2048
    w = (H + 2 * KVH) * D
    qkv = torch.from_numpy(oracle.normal(m * w, seed=91 + KVH).reshape(m, w)).cuda()
    print(f"prompt split vs unsplit H={H} KVH={KVH} m={m}", flush=True)
    whole = KvCache(KVH, D, m).attention(qkv, H).cpu().numpy()
    kv = KvCache(KVH, D, m)
    first = kv.attention(qkv[:m // 2].contiguous(), H).cpu().numpy()
    second = kv.attention(qkv[m // 2:].contiguous(), H).cpu().numpy()
    halves = np.concatenate([first, second])
    assert kv.seq_len == m
    assert oracle.normwise_error(whole, halves) < 1e-5


def test_attention_prompt_causality():
    # changing token 9's q, k and v leaves the outputs of tokens 0 .. 8 bit for bit
    H, KVH, D, m = 8, 2, 64, 40
    w = (H + 2 * KVH) * D
    a = oracle.normal(m * w, seed=61).reshape(m, w)
    b = a.copy()
    b[9] = oracle.normal(w, seed=62)
    oa = KvCache(KVH, D, 64).attention(torch.from_numpy(a).cuda(), H).cpu().numpy()
    ob = KvCache(KVH, D, 64).attention(torch.from_numpy(b).cuda(), H).cpu().numpy()
    assert np.array_equal(oa[:9], ob[:9])
    assert not np.array_equal(oa[9], ob[9])


# ---- the cache length in device memory: a captured step replays at successive positions -----

def test_captured_decode_step_advances_each_replay():
    # generate_with_cache's loop (llama.rs:488-560) as a graph: prompt once, then one
    # captured decode step replayed for every new token -- each replay appends at the
    # next position and attends over everything before it
    H, KVH, D = 8, 2, 128
    w = (H + 2 * KVH) * D
    P, N, max_seq = 37, 6, 64
    kv = KvCache(KVH, D, max_seq)
    kc = np.zeros((KVH, max_seq, D), np.float32)
    vc = np.zeros((KVH, max_seq, D), np.float32)
    stream = torch.cuda.Stream()
    kv.reserve(1, H, stream=stream)
    prompt = oracle.normal(P * w, seed=71).reshape(P, w)
    tokens = [oracle.normal(w, seed=80 + i).reshape(1, w) for i in range(N)]
    qkv = torch.empty(1, w, device="cuda")
    out = torch.empty(1, H * D, device="cuda")
    with torch.cuda.stream(stream):
        kv.attention(torch.from_numpy(prompt).cuda(), H, stream=stream)
    stream.synchronize()
    oracle.attention_decode(prompt, H, KVH, D, 10000.0, kc, vc, 0)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
        kv.attention(qkv, H, out=out, stream=stream)
    assert kv.seq_len == P  # capture runs nothing
    for i in range(N):
        qkv.copy_(torch.from_numpy(tokens[i]))
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            g.replay()
        stream.synchronize()
        ref = oracle.attention_decode(tokens[i], H, KVH, D, 10000.0, kc, vc, P + i)
        assert oracle.normwise_error(out.cpu().numpy(), ref) < 1e-4, i
    assert kv.seq_len == P + N
    # an eager call after the replays continues from the device length
    t = oracle.normal(w, seed=99).reshape(1, w)
    o = kv.attention(torch.from_numpy(t).cuda(), H).cpu().numpy()
    assert oracle.normwise_error(o, oracle.attention_decode(t, H, KVH, D, 10000.0, kc, vc,
                                                           P + N)) < 1e-4
    assert kv.seq_len == P + N + 1
    del g


def test_replay_past_max_seq_reports_overflow():
    H, KVH, D = 4, 2, 64
    w = (H + 2 * KVH) * D
    kv = KvCache(KVH, D, 3)
    stream = torch.cuda.Stream()
    kv.reserve(1, H, stream=stream)
    qkv = torch.from_numpy(oracle.normal(w, seed=5).reshape(1, w)).cuda()
    out = torch.empty(1, H * D, device="cuda")
    with torch.cuda.stream(stream):
        kv.attention(qkv, H, stream=stream)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
        kv.attention(qkv, H, out=out, stream=stream)
    for _ in range(2):  # positions 1 and 2: fine
        with torch.cuda.stream(stream):
            g.replay()
    stream.synchronize()
    assert bool(torch.isfinite(out).all())
    with torch.cuda.stream(stream):
        g.replay()  # position 3 = max_seq: overflow
    stream.synchronize()
    assert bool(torch.isnan(out).all())
    with pytest.raises(HipError, match="KV cache overflow"):
        kv.seq_len
    # the overflowing replay appended nothing: truncating keeps the intact prefix and
    # clears the flag, and an eager call continues from it
    kc = np.zeros((KVH, 3, D), np.float32)
    vc = np.zeros((KVH, 3, D), np.float32)
    q0 = qkv.cpu().numpy()
    for pos in range(2):
        oracle.attention_decode(q0, H, KVH, D, 10000.0, kc, vc, pos)
    kv.truncate(2)
    assert kv.seq_len == 2
    t = oracle.normal(w, seed=6).reshape(1, w)
    o = kv.attention(torch.from_numpy(t).cuda(), H).cpu().numpy()
    ref = oracle.attention_decode(t, H, KVH, D, 10000.0, kc, vc, 2)
    assert oracle.normwise_error(o, ref) < 1e-4
    assert kv.seq_len == 3
    kv.clear()
    assert kv.seq_len == 0
    del g


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
