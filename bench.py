"""Benchmark of the MI355X quantized linear-layer path (one GPU).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]

Headline: Q4_0 decode GEMV at m = 1 on the
Llama-2-7B projection shapes.  One step is one decode pass over the linear
layers of a 32-layer Llama-2-7B in Q4_0: per layer QKV 4096x12288,
o_proj 4096x4096, gate 4096x11008, up 4096x11008, down 11008x4096 -- 160
GEMV launches over 3.64 GB of distinct weights, so every launch streams its
weights from HBM (the working set is 14x the 256 MB Infinity Cache).  The
launches of one step are captured once in a HIP graph and replayed.

value = algorithmic bytes (weights + x + y) / wall time per step, in GB/s.
roofline.achieved uses the same bytes over the GEMV kernel's average duration,
measured with HIP events on the stream the kernels run on.

The other BASELINE configs are reported under "extra" (Q8_0 TinyLlama GEMV,
batched decode, prefill TFLOP/s, full stack with lm_head), with decode
attention and a whole decode step (linear layers + attention over a KV cache);
they are not the headline.  Synthetic data: weights N(0, 0.02) from torch's generator,
quantized on the device with the GGML quantizer; activations N(0, 1).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
# MI355X dense MFMA peak, the same for bf16 and f16 operands (the prefill kernel
# runs f16; the "frac_dense" fields price it against this)
DENSE_PEAK_TFLOPS = 2516.6
# MI355X f32 peak (the prompt attention kernel's f32 FMA work is priced against it)
F32_PEAK_TFLOPS = 157.3
Q4_0, Q8_0, Q4_K, Q5_K = 2, 8, 12, 13
# GGUF bytes per 32 weights (Q4_K: 144 per 256, Q5_K: 176 per 256)
BPB = {Q4_0: 18, Q8_0: 34, Q4_K: 18, Q5_K: 22}

LLAMA2_7B = [("qkv", 4096, 12288), ("o_proj", 4096, 4096), ("gate", 4096, 11008),
             ("up", 4096, 11008), ("down", 11008, 4096)]


def wbytes(qtype, n, k):
    return n * (k // 32) * BPB[qtype]


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--only", default="", help="comma list of extra configs to run "
                    "(q8_gemv,batched,prefill,stack,q4_k,q5_k,attention,e2e) -- for profiling")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only copy 64 MiB once (device to device) and exit: the known-size "
                    "kernel that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE counters")
    return ap.parse_args()


COPY_PROBE_BYTES = 64 << 20
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "gemv_q4_0_decode_traffic.json")


def copy_probe():
    import torch
    src = torch.full((COPY_PROBE_BYTES,), 7, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": COPY_PROBE_BYTES}), flush=True)


def measured_traffic():
    """HBM bytes per GEMV launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by what the counter reads for the
    64 MiB copy probe), or None if it is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t["bytes_per_launch"], t
    except (OSError, ValueError, KeyError):
        return None, None


class Timer:
    """HIP events on the stream the kernels run on."""

    def __init__(self, torch, stream):
        self.torch = torch
        self.stream = stream

    def run(self, fn, reps):
        t = self.torch
        a = t.cuda.Event(enable_timing=True)
        b = t.cuda.Event(enable_timing=True)
        a.record(self.stream)
        for _ in range(reps):
            fn()
        b.record(self.stream)
        b.synchronize()
        return a.elapsed_time(b) / reps  # ms


def make_weights(torch, QuantLinear, qtype, n, k, copies, gen):
    out = []
    for _ in range(copies):
        w = torch.empty(n, k, device="cuda", dtype=torch.float32)
        w.normal_(0.0, 0.02, generator=gen)
        out.append(QuantLinear.quantize(qtype, w))
        del w
    torch.cuda.synchronize()
    return out


def decode_stack(torch, QuantLinear, args, gen, stream):
    """The headline: 32 layers x 5 Q4_0 GEMVs at m = 1, graph-replayed."""
    layers = []
    for _ in range(args.layers):
        layer = []
        for name, k, n in LLAMA2_7B:
            layer.append(make_weights(torch, QuantLinear, Q4_0, n, k, 1, gen)[0])
        layers.append(layer)
    xs = {k: torch.empty(1, k, device="cuda").normal_(generator=gen) for _, k, _ in LLAMA2_7B}
    ys = {n: torch.empty(1, n, device="cuda") for _, _, n in LLAMA2_7B}
    nbytes = 0
    for layer in layers:
        for ql, (name, k, n) in zip(layer, LLAMA2_7B):
            nbytes += wbytes(Q4_0, n, k) + 4 * k + 4 * n
    launches = len(layers) * len(LLAMA2_7B)
    path = layers[0][0].select_path(1)

    def step():
        for layer in layers:
            for ql, (name, k, n) in zip(layer, LLAMA2_7B):
                ql.forward(xs[k], out=ys[n], stream=stream)

    with torch.cuda.stream(stream):
        step()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
            step()
    torch.cuda.synchronize()
    return layers, g, nbytes, launches, path


def cpu_baseline():
    """The reference CPU path (candle QMatMul semantics: Q8_0 activations,
    integer block dots, OpenMP over columns), restated in oracle/oracle.c and
    timed on this host on one layer's five GEMVs (a bounded sample)."""
    import oracle

    threads = len(os.sched_getaffinity(0))
    # same distribution and shapes as the device weights (drawn on the host)
    rng = np.random.default_rng(1234)
    host = []
    for name, k, n in LLAMA2_7B:
        w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
        host.append((oracle.quantize(Q4_0, w), np.ascontiguousarray(
            rng.standard_normal((1, k), dtype=np.float32)), n, k))
    nbytes = sum(wbytes(Q4_0, n, k) + 4 * k + 4 * n for _, _, n, k in host)

    def one_pass():
        for b, x, n, k in host:
            oracle.candle_qmatmul(Q4_0, b, x, n, k, nthreads=threads, timing=True)

    for _ in range(3):
        one_pass()
    times = []
    t_end = time.perf_counter() + 10.0
    while len(times) < 20 or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        one_pass()
        times.append(time.perf_counter() - t0)
        if len(times) >= 20 and time.perf_counter() > t_end:
            break
    med = float(np.median(times))
    return {"value": round(nbytes / med / 1e9, 2), "unit": "GB/s", "cores": threads,
            "cpu": cpu_model(), "build": oracle.timing_lib()[1], "kind": "port",
            "sample": f"one Llama-2-7B layer's 5 Q4_0 GEMVs at m=1 ({nbytes / 1e6:.1f} MB), "
                      f"median of {len(times)} passes after 3 warm-ups, "
                      "candle QMatMul semantics restated in C (oracle/oracle.c), OpenMP",
            "ms_per_pass": round(med * 1e3, 3)}


_CPU_WEIGHTS = {}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for every cpu_baseline."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_rows(qtype, n, k, rows, budget_s=1.5, seed=0):
    """Median seconds of oracle.candle_qmatmul (the reference's CPU QMatMul: Q8_0
    activations, integer block dots, a loop over rows with OpenMP over columns) on
    `rows` rows of one [n, k] weight drawn like the device's, and the threads used."""
    import oracle

    threads = len(os.sched_getaffinity(0))
    rng = np.random.default_rng(seed)
    if (qtype, n, k) not in _CPU_WEIGHTS:  # one weight per shape (the batched widths share it)
        _CPU_WEIGHTS.clear()
        _CPU_WEIGHTS[(qtype, n, k)] = oracle.quantize(
            qtype, rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    w = _CPU_WEIGHTS[(qtype, n, k)]
    x = rng.standard_normal((rows, k), dtype=np.float32)
    oracle.candle_qmatmul(qtype, w, x, n, k, nthreads=threads, timing=True)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        oracle.candle_qmatmul(qtype, w, x, n, k, nthreads=threads, timing=True)
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), threads


def extra_cpu_baselines(extra):
    """A cpu_baseline for every extra entry of BASELINE configs 0, 2, 3 and 4, on the
    same algorithmic bytes / flops as the device figure.  Bounded samples: prefill
    times 8 rows (the reference's row loop costs the same per row, so m rows take m
    times as long); the stack times one layer's four projections and the lm_head
    (32 identical layers)."""
    import oracle

    def entry(value, unit, cores, sample):
        return {"value": round(value, 3), "unit": unit, "cores": cores, "cpu": cpu_model(),
                "build": oracle.timing_lib()[1], "kind": "port",
                "sample": sample + "; candle QMatMul semantics restated in C (oracle/oracle.c), "
                                   "OpenMP over columns, median of timed calls"}

    key = "q8_0_gemv_m1_k2048_n5632"
    if key in extra:
        t, c = cpu_rows(Q8_0, 5632, 2048, 1)
        b = wbytes(Q8_0, 5632, 2048) + 4 * 2048 + 4 * 5632
        extra[key]["cpu_baseline"] = entry(b / t / 1e9, "GB/s", c, "the full call (m = 1)")
    for n in (4096, 14336):
        for m in (4, 16, 64):
            key = f"q4_0_batched_m{m}_k4096_n{n}"
            if key in extra:
                t, c = cpu_rows(Q4_0, n, 4096, m)
                b = wbytes(Q4_0, n, 4096) + 4 * m * 4096 + 4 * m * n
                extra[key]["cpu_baseline"] = entry(b / t / 1e9, "GB/s", c, f"the full call (m = {m})")
    for qtype, qn in ((Q4_0, "q4_0"), (Q8_0, "q8_0")):
        for k, n in ((4096, 14336), (14336, 4096)):
            keys = [f"{qn}_prefill_m{m}_k{k}_n{n}" for m in (512, 2048)]
            if any(kk in extra for kk in keys):
                t, c = cpu_rows(qtype, n, k, 8)
                tf = 2 * 8 * n * k / t / 1e12
                for kk in keys:
                    if kk in extra:
                        extra[kk]["cpu_baseline"] = entry(
                            tf, "TFLOP/s", c, "8 of the m rows timed, the rate scaled to m rows")
    for m in (1, 16):
        key = f"llama2_7b_stack_q4_0_m{m}"
        if key in extra:
            layer = 0.0
            for q, k, n in ((Q4_0, 4096, 12288), (Q4_0, 4096, 4096), (Q4_0, 4096, 22016),
                            (Q4_0, 11008, 4096)):
                t, c = cpu_rows(q, n, k, m, budget_s=1.0)
                layer += t
            head, c = cpu_rows(Q8_0, 32000, 4096, m, budget_s=1.0)
            step = 32 * layer + head
            extra[key]["cpu_baseline"] = entry(
                m / step, "tokens/s", c,
                f"one layer's 4 projections and the Q8_0 lm_head at m = {m} timed, "
                f"the step = 32 layers + head ({step * 1e3:.1f} ms)")
            extra[key]["cpu_baseline"]["GB/s"] = round(
                extra[key]["GB/s"] * extra[key]["ms_per_step"] / (step * 1e3), 2)


def extra_configs(torch, QuantLinear, gen, stream, only):
    """The other BASELINE configs, each timed with HIP events (median of 3
    rounds), weights rotated over >= 1 GB where the op is HBM-bound."""
    from unillm_amd import PATH_DECODE_MFMA, PATH_PREFILL_MFMA

    timer = Timer(torch, stream)
    res = {}

    def rotate(qtype, n, k, min_bytes=1 << 30, max_copies=96):
        copies = max(1, min(max_copies, -(-min_bytes // wbytes(qtype, n, k))))
        return make_weights(torch, QuantLinear, qtype, n, k, copies, gen)

    def timed(ws, x, y, reps_per_copy=2, path=0):
        def call_all():
            for ql in ws:
                ql.forward(x, out=y, path=path, stream=stream)
        with torch.cuda.stream(stream):
            call_all()
            ts = [timer.run(call_all, reps_per_copy) / len(ws) for _ in range(3)]
        return float(np.median(ts))

    want = set(only.split(",")) if only else {"q8_gemv", "batched", "prefill", "stack", "q4_k",
                                              "q5_k", "attention", "e2e"}
    if "q8_gemv" in want:
        n, k = 5632, 2048
        ws = rotate(Q8_0, n, k)
        x = torch.empty(1, k, device="cuda").normal_(generator=gen)
        y = torch.empty(1, n, device="cuda")
        ms = timed(ws, x, y)
        b = wbytes(Q8_0, n, k) + 4 * k + 4 * n
        res["q8_0_gemv_m1_k2048_n5632"] = {"GB/s": round(b / ms / 1e6, 1),
                                           "frac_hbm": round(b / ms / 1e6 / HBM_PEAK_GBS, 3),
                                           "us": round(ms * 1e3, 2), "copies": len(ws)}
        del ws
        # a Q8_0 down projection at Llama-2-7B's shape (past k 8192: the GEMV's k split)
        n, k = 4096, 11008
        ws = rotate(Q8_0, n, k)
        x = torch.empty(1, k, device="cuda").normal_(generator=gen)
        y = torch.empty(1, n, device="cuda")
        ms = timed(ws, x, y)
        b = wbytes(Q8_0, n, k) + 4 * k + 4 * n
        res["q8_0_gemv_m1_k11008_n4096"] = {"GB/s": round(b / ms / 1e6, 1),
                                            "frac_hbm": round(b / ms / 1e6 / HBM_PEAK_GBS, 3),
                                            "us": round(ms * 1e3, 2), "copies": len(ws),
                                            "path": ws[0].select_path(1)}
        del ws
    if "batched" in want:
        for n in (4096, 14336):
            ws = rotate(Q4_0, n, 4096, max_copies=64)
            for m in (4, 16, 64):
                x = torch.empty(m, 4096, device="cuda").normal_(generator=gen)
                y = torch.empty(m, n, device="cuda")
                ms = timed(ws, x, y)
                b = wbytes(Q4_0, n, 4096) + 4 * m * 4096 + 4 * m * n
                res[f"q4_0_batched_m{m}_k4096_n{n}"] = {
                    "GB/s": round(b / ms / 1e6, 1), "frac_hbm": round(b / ms / 1e6 / HBM_PEAK_GBS, 3),
                    "TFLOP/s": round(2 * m * n * 4096 / ms / 1e9, 2), "us": round(ms * 1e3, 2),
                    "path": ws[0].select_path(m)}
            del ws
    if "prefill" in want:
        for qtype in (Q4_0, Q8_0):
            for k, n in ((4096, 14336), (14336, 4096)):
                ws = make_weights(torch, QuantLinear, qtype, n, k, 2, gen)
                for m in (512, 2048):
                    x = torch.empty(m, k, device="cuda").normal_(generator=gen)
                    y = torch.empty(m, n, device="cuda")
                    ms = timed(ws, x, y, reps_per_copy=2, path=PATH_PREFILL_MFMA)
                    tf = 2 * m * n * k / ms / 1e9
                    res[f"{'q4_0' if qtype == Q4_0 else 'q8_0'}_prefill_m{m}_k{k}_n{n}"] = {
                        "TFLOP/s": round(tf, 1), "frac_dense": round(tf / DENSE_PEAK_TFLOPS, 3),
                        "us": round(ms * 1e3, 1)}
                del ws
    for kq, bb, label in ((Q4_K, 144, "q4_k"), (Q5_K, 176, "q5_k")):
        if label not in want:
            continue
        # K-quants (GGUF Q4_K_M / Q5_K_M tensors), random valid blocks drawn on the
        # device -- no K-quant quantizer is on the path
        def kq_weights(n, k, copies):
            ws = []
            nb = n * (k // 256)
            for _ in range(copies):
                blk = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, device="cuda",
                                    generator=gen)
                for off, lo, span in ((0, 1e-5, 4e-5), (2, 1e-5, 2e-4)):  # d, dmin (f16)
                    v = (torch.rand(nb, device="cuda", generator=gen) * span + lo).half()
                    blk[:, off:off + 2] = v.view(torch.uint8).view(nb, 2)
                ws.append(QuantLinear.from_device_blocks(kq, n, k, blk.view(-1)))
            return ws

        for name, k, n in LLAMA2_7B:
            ws = kq_weights(n, k, max(1, min(48, -(-(1 << 30) // wbytes(kq, n, k)))))
            x = torch.empty(1, k, device="cuda").normal_(generator=gen)
            y = torch.empty(1, n, device="cuda")
            ms = timed(ws, x, y)
            b = wbytes(kq, n, k) + 4 * k + 4 * n
            res[f"{label}_gemv_m1_{name}_k{k}_n{n}"] = {
                "GB/s": round(b / ms / 1e6, 1), "frac_hbm": round(b / ms / 1e6 / HBM_PEAK_GBS, 3),
                "us": round(ms * 1e3, 2), "path": ws[0].select_path(1)}
            del ws
        ws = kq_weights(14336, 4096, 32)
        for m in (16, 64):
            x = torch.empty(m, 4096, device="cuda").normal_(generator=gen)
            y = torch.empty(m, 14336, device="cuda")
            ms = timed(ws, x, y)
            b = wbytes(kq, 14336, 4096) + 4 * m * 4096 + 4 * m * 14336
            res[f"{label}_batched_m{m}_k4096_n14336"] = {
                "GB/s": round(b / ms / 1e6, 1), "frac_hbm": round(b / ms / 1e6 / HBM_PEAK_GBS, 3),
                "us": round(ms * 1e3, 2), "path": ws[0].select_path(m)}
        del ws
        ws = kq_weights(14336, 4096, 2)
        x = torch.empty(2048, 4096, device="cuda").normal_(generator=gen)
        y = torch.empty(2048, 14336, device="cuda")
        ms = timed(ws, x, y, path=PATH_PREFILL_MFMA)
        tf = 2 * 2048 * 14336 * 4096 / ms / 1e9
        res[f"{label}_prefill_m2048_k4096_n14336"] = {
            "TFLOP/s": round(tf, 1), "frac_dense": round(tf / DENSE_PEAK_TFLOPS, 3),
            "us": round(ms * 1e3, 1)}
        del ws
    if "attention" in want:
        # decode attention over a KV cache of about L positions (row f4): 20 calls of
        # one new token each, starting from L - 10 cached positions (the cache is
        # rewound between samples, outside the timed region); HBM-bound on the cached
        # K and V (2 KVH L hd 4 bytes), timed per call
        from unillm_amd import KvCache
        R = 20
        for (H, KVH, D, label) in ((32, 32, 128, "llama2_7b"), (32, 8, 128, "gqa_32_8")):
            for L in (1024, 4096):
                kv = KvCache(KVH, D, L + 64)
                w = (H + 2 * KVH) * D
                start = L - R // 2
                fill = torch.empty(start, w, device="cuda").normal_(generator=gen)
                q1 = torch.empty(1, w, device="cuda").normal_(generator=gen)
                out = torch.empty(1, H * D, device="cuda")

                def one():
                    kv.attention(q1, H, out=out, stream=stream)

                def sample(fn):
                    kv.truncate(start)
                    return timer.run(fn, 1)

                with torch.cuda.stream(stream):
                    kv.attention(fill, H, stream=stream)  # the prompt, one call
                    del fill
                    one()
                    eager = float(np.median([sample(lambda: [one() for _ in range(R)])
                                             for _ in range(3)])) / R
                    # the same R calls captured once and replayed, as a decode step
                    # would run them: the cache length lives on the device, so each
                    # replayed call appends at the position the previous one left
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
                        for _ in range(R):
                            one()
                    sample(g.replay)
                    ms = float(np.median([sample(g.replay) for _ in range(5)])) / R
                    del g
                b = 2 * KVH * L * D * 4
                res[f"attention_decode_{label}_L{L}"] = {
                    "GB/s": round(b / ms / 1e6, 1), "frac_hbm": round(b / ms / 1e6 / HBM_PEAK_GBS, 3),
                    "us": round(ms * 1e3, 2), "eager_us": round(eager * 1e3, 2), "kv_bytes": b}
                del kv
        # prompt attention (m tokens into an empty cache, causal): 4 H hd m (m + 1) / 2
        # flops of f32 FMA work (scores and the weighted sum), priced against the
        # f32 vector peak
        for (H, KVH, D, label) in ((32, 32, 128, "llama2_7b"), (32, 8, 128, "gqa_32_8")):
            for m in (512, 2048):
                kv = KvCache(KVH, D, m)
                x = torch.empty(m, (H + 2 * KVH) * D, device="cuda").normal_(generator=gen)
                out = torch.empty(m, H * D, device="cuda")

                def sample():
                    kv.truncate(0)
                    return timer.run(lambda: kv.attention(x, H, out=out, stream=stream), 1)

                with torch.cuda.stream(stream):
                    sample()
                    ms = float(np.median([sample() for _ in range(5)]))
                tf = 4 * H * D * m * (m + 1) / 2 / ms / 1e9
                res[f"attention_prompt_{label}_m{m}"] = {
                    "TFLOP/s": round(tf, 1), "frac_f32": round(tf / F32_PEAK_TFLOPS, 3),
                    "us": round(ms * 1e3, 1)}
                del kv, x, out
    if "e2e" in want and "stack" not in want:
        want.add("stack")  # the end-to-end step reuses the stack's weights
    if "stack" in want:
        # config 5: 32 layers (QKV, o, gate+up fused 22016, down) + Q8_0 lm_head
        shapes = [(Q4_0, 4096, 12288), (Q4_0, 4096, 4096), (Q4_0, 4096, 22016),
                  (Q4_0, 11008, 4096)]
        layers = [[make_weights(torch, QuantLinear, q, n, k, 1, gen)[0] for q, k, n in shapes]
                  for _ in range(32)]
        head = make_weights(torch, QuantLinear, Q8_0, 32000, 4096, 1, gen)[0]
        total_w = 32 * sum(wbytes(q, n, k) for q, k, n in shapes) + wbytes(Q8_0, 32000, 4096)
        for m in (1, 16):
            xs = {k: torch.empty(m, k, device="cuda").normal_(generator=gen) for k in (4096, 11008)}
            ys = {n: torch.empty(m, n, device="cuda") for n in (12288, 4096, 22016, 32000)}

            def step():
                for layer in layers:
                    for ql, (q, k, n) in zip(layer, shapes):
                        ql.forward(xs[k], out=ys[n], stream=stream)
                head.forward(xs[4096], out=ys[32000], stream=stream)

            with torch.cuda.stream(stream):
                step()
                ms = float(np.median([timer.run(step, 3) for _ in range(3)]))
            b = total_w + 4 * m * (32 * (3 * 4096 + 11008) + 4096) + 4 * m * (
                32 * (12288 + 4096 + 22016 + 4096) + 32000)
            res[f"llama2_7b_stack_q4_0_m{m}"] = {
                "GB/s": round(b / ms / 1e6, 1), "frac_hbm": round(b / ms / 1e6 / HBM_PEAK_GBS, 3),
                "ms_per_step": round(ms, 4), "tokens/s": round(m * 1e3 / ms, 1),
                "weight_bytes": total_w}

            # the same four launches per layer with the layer's elementwise work in
            # them: input_layernorm + QKV, o_proj + residual add, post_attention_layernorm
            # + gate_up + SwiGLU, down + residual add (the lm_head as before)
            gam = torch.ones(4096, device="cuda")
            h = torch.empty(m, 4096, device="cuda").normal_(generator=gen)
            act = torch.empty(m, 11008, device="cuda")

            def fused_step():
                for qkv, o, gu, down in layers:
                    qkv.forward_norm(h, gam, eps=1e-6, out=ys[12288], stream=stream)
                    o.forward_add(xs[4096], h, stream=stream)
                    gu.forward_swiglu(h, out=act, stream=stream, norm=(gam, None, 1e-6))
                    down.forward_add(act, h, stream=stream)
                head.forward(xs[4096], out=ys[32000], stream=stream)

            with torch.cuda.stream(stream):
                h.normal_(generator=gen)
                fused_step()
                h.normal_(generator=gen)  # the residual grows by design; restart it
                msf = float(np.median([timer.run(fused_step, 3) for _ in range(3)]))
            res[f"llama2_7b_stack_q4_0_fused_m{m}"] = {
                "GB/s": round(b / msf / 1e6, 1), "ms_per_step": round(msf, 4),
                "tokens/s": round(m * 1e3 / msf, 1),
                "note": "norms, residual adds and SwiGLU fused into the same 4 launches a layer"}
        if "e2e" in want:
            res.update(decode_step_e2e(torch, layers, head, gen, stream, timer))
            res.update(prompt_step_e2e(torch, layers, head, gen, stream, timer))
        del layers, head
    torch.cuda.synchronize()
    return res


def decode_step_e2e(torch, layers, head, gen, stream, timer):
    """A whole Llama-2-7B decode step (m = 1) over a KV cache of L positions:
    per layer input_layernorm + QKV, attention (RoPE, append, causal softmax over
    the cache: 32 heads, hd 128, f32), o_proj + residual, post_attention_layernorm +
    gate_up + SwiGLU, down + residual; then the final norm + lm_head.  Captured once
    as a HIP graph (6 launches a layer) and replayed: each replay appends one
    position to every cache (the length lives on the device), starting from L - 5
    cached positions after a rewind outside the timed region."""
    from unillm_amd import KvCache
    H, D = 32, 128
    res = {}
    gam = torch.ones(4096, device="cuda")
    h = torch.empty(1, 4096, device="cuda")
    qkv_out = torch.empty(1, 3 * 4096, device="cuda")
    att = torch.empty(1, 4096, device="cuda")
    act = torch.empty(1, 11008, device="cuda")
    logits = torch.empty(1, 32000, device="cuda")
    R = 5
    for L in (1024, 4096):
        caches = [KvCache(H, D, L + 64) for _ in layers]
        start = L - R
        fill = torch.empty(start, 3 * 4096, device="cuda").normal_(generator=gen)
        with torch.cuda.stream(stream):
            for kv in caches:  # the prompt: one call a layer
                kv.attention(fill, H, stream=stream)
            del fill

            def step():
                for (qkv, o, gu, down), kv in zip(layers, caches):
                    qkv.forward_norm(h, gam, eps=1e-6, out=qkv_out, stream=stream)
                    kv.attention(qkv_out, H, out=att, stream=stream)
                    o.forward_add(att, h, stream=stream)
                    gu.forward_swiglu(h, out=act, stream=stream, norm=(gam, None, 1e-6))
                    down.forward_add(act, h, stream=stream)
                head.forward_norm(h, gam, eps=1e-6, out=logits, stream=stream)

            def sample():
                for kv in caches:
                    kv.truncate(start)
                h.normal_(generator=gen)  # the residual grows by design; restart it
                return timer.run(g.replay, R)

            h.normal_(generator=gen)
            step()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
                step()
            sample()
            ms = float(np.median([sample() for _ in range(3)]))
            del g
        kv_bytes = 32 * 2 * H * L * D * 4
        w_bytes = 32 * (wbytes(Q4_0, 12288, 4096) + wbytes(Q4_0, 4096, 4096) +
                        wbytes(Q4_0, 22016, 4096) + wbytes(Q4_0, 4096, 11008)) + \
            wbytes(Q8_0, 32000, 4096)
        res[f"llama2_7b_decode_step_e2e_m1_L{L}"] = {
            "ms_per_step": round(ms, 4), "tokens/s": round(1e3 / ms, 1),
            "GB/s": round((w_bytes + kv_bytes) / ms / 1e6, 1), "kv_bytes": kv_bytes,
            "launches_per_step": 6 * 32 + 1,
            "note": "norm+QKV, attention, o+residual, norm+gate_up+SwiGLU, down+residual a layer; "
                    "final norm + Q8_0 lm_head; HIP-graph replay"}
        del caches
    return res


def prompt_step_e2e(torch, layers, head, gen, stream, timer):
    """A whole Llama-2-7B prompt step: m tokens into empty KV caches, per layer
    input_layernorm + QKV, attention (RoPE, append, causal softmax over the prompt:
    32 heads, hd 128, f32 cache), o_proj + residual, post_attention_layernorm +
    gate_up + SwiGLU, down + residual; then the final norm + lm_head over all m
    positions, as LlamaModelV2::forward_with_cache does (llama.rs:445-449; generate
    narrows to the last position afterwards).  Eager launches; the caches are
    rewound and the residual restarted outside each timed pass."""
    from unillm_amd import KvCache
    H, D = 32, 128
    res = {}
    gam = torch.ones(4096, device="cuda")
    for m in (512, 2048):
        logits = torch.empty(m, 32000, device="cuda")
        h = torch.empty(m, 4096, device="cuda")
        qkv_out = torch.empty(m, 3 * 4096, device="cuda")
        att = torch.empty(m, 4096, device="cuda")
        act = torch.empty(m, 11008, device="cuda")
        caches = [KvCache(H, D, m) for _ in layers]

        def step():
            for (qkv, o, gu, down), kv in zip(layers, caches):
                qkv.forward_norm(h, gam, eps=1e-6, out=qkv_out, stream=stream)
                kv.attention(qkv_out, H, out=att, stream=stream)
                o.forward_add(att, h, stream=stream)
                gu.forward_swiglu(h, out=act, stream=stream, norm=(gam, None, 1e-6))
                down.forward_add(act, h, stream=stream)
            head.forward_norm(h, gam, eps=1e-6, out=logits, stream=stream)

        def sample():
            for kv in caches:
                kv.truncate(0)
            h.normal_(generator=gen)
            return timer.run(step, 1)

        with torch.cuda.stream(stream):
            sample()
            ms = float(np.median([sample() for _ in range(5)]))
        # the linear layers and the lm_head
        flops = 2 * m * 4096 * (32 * (12288 + 4096 + 22016 + 11008) + 32000)
        res[f"llama2_7b_prompt_step_e2e_m{m}"] = {
            "ms_per_step": round(ms, 3), "tokens/s": round(m * 1e3 / ms, 1),
            "linear_TFLOP/s": round(flops / ms / 1e9, 1),
            "note": "norm+QKV, attention over the prompt, o+residual, norm+gate_up+SwiGLU, "
                    "down+residual a layer into empty caches; final norm + Q8_0 lm_head on "
                    "all m positions (forward_with_cache); eager launches"}
        del caches
    return res


def main():
    args = parse()
    if args.copy_probe:
        copy_probe()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(sharding is a design note, not code); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    from unillm_amd import QuantLinear
    from unillm_amd import _capi

    _capi.check(_capi.lib().unillm_hip_init(0))
    torch.cuda.set_device(0)
    stream = torch.cuda.Stream()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(20240601)
    timer = Timer(torch, stream)

    layers, graph, nbytes, launches, path = decode_stack(torch, QuantLinear, args, gen, stream)

    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    # timed region: exactly K steps, synchronised on both sides
    t0 = time.perf_counter()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    with torch.cuda.stream(stream):
        for _ in range(args.steps):
            graph.replay()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    kern_ms = ev0.elapsed_time(ev1) / (args.steps * launches)  # average GEMV launch
    value = nbytes / (wall / args.steps) / 1e9
    achieved = (nbytes / launches) / (kern_ms * 1e-3) / 1e9

    extra = {}
    if not args.no_extra:
        extra = extra_configs(torch, QuantLinear, gen, stream, args.only)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline()
        extra_cpu_baselines(extra)

    traffic, tinfo = measured_traffic()
    traffic_src = None
    if tinfo is not None:
        traffic_src = (f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE over the same decode step "
                       f"({os.path.relpath(TRAFFIC_FILE, os.path.dirname(TRAFFIC_FILE) + '/..')}), "
                       f"scale factors {tinfo.get('fetch_factor')} / {tinfo.get('write_factor')} "
                       "from the 64 MiB copy probe")
    line = {
        "metric": "Q4_0 decode GEMV GB/s (% HBM peak) at 7B shapes; prefill GEMM TFLOP/s",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights x f32 activations held per 32-block as exact 16-bit "
                 "fixed-point integers (4 base-16 digits; the reference holds them as int8 "
                 "Q8_0), int32 block dots, fp32 accumulate",
        "data": "synthetic: weights N(0,0.02) quantized on device with the GGML Q4_0 "
                "quantizer, x N(0,1); random-init Llama-2-7B projection shapes",
        "config": {"workload": "Q4_0 decode GEMV, m=1, Llama-2-7B shapes (QKV 4096x12288, "
                               "o 4096x4096, gate/up 4096x11008, down 11008x4096), "
                               f"{args.layers} distinct layers per step, HIP-graph replay",
                   "global_batch": 1, "seq_len": 1, "parallelism": "none (1 GPU)",
                   "launches_per_step": launches, "bytes_per_step": nbytes,
                   "kernel_path": {1: "gemv", 2: "decode_mfma", 3: "prefill_mfma"}[path]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "kernel": "gemv_kernel<Q4_0, M=1>",
                     "avg_launch_us": round(kern_ms * 1e3, 3),
                     "avg_launch_us_source": "HIP events around the timed graph replays on "
                                             "the launch stream / launches (launch gaps "
                                             "included), not rocprof kernel durations",
                     "bytes_per_launch": nbytes // launches,
                     "traffic_source": traffic_src},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
