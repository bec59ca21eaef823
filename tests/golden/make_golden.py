"""Write the golden fixtures for the Q4_0 / Q8_0 linear-layer path.

This is an independent numpy restatement of the GGML block formats (written
apart from oracle/oracle.c, vectorised, with numpy's own float16 rounding), so
the committed vectors cross-check the C oracle rather than echo it.

The reference (cognisoc/unillm) is Rust and its arithmetic lives in the
un-vendored candle-core 0.8; it cannot be run here (no rustc/cargo), and its
own tests hold no vectors for this path beyond the layout-neutral known
answers restated in tests/test_oracle.py.  So the inputs are synthetic:
weights N(0, 0.02), activations N(0, 1), plus hand-built edge blocks.

Run:  python tests/golden/make_golden.py     (writes tests/golden/*.npz)
"""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F32 = np.float32


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """GGML Q4_0: d = max/-8 (max = signed element of largest magnitude, first
    occurrence), q = min(15, trunc(x*(1/d) + 8.5)), low nibble j, high j+16."""
    n, k = w.shape
    blk = w.reshape(-1, 32).astype(F32)
    idx = np.argmax(np.abs(blk), axis=1)
    mx = blk[np.arange(blk.shape[0]), idx]
    d = (mx / F32(-8.0)).astype(F32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, F32(1.0) / np.where(d != 0, d, F32(1.0)), F32(0.0)).astype(F32)
    x0 = (blk[:, :16] * inv[:, None]).astype(F32) + F32(8.5)
    x1 = (blk[:, 16:] * inv[:, None]).astype(F32) + F32(8.5)
    q0 = np.minimum(15, np.trunc(x0).astype(np.int32))
    q1 = np.minimum(15, np.trunc(x1).astype(np.int32))
    qs = (q0 | (q1 << 4)).astype(np.uint8)
    d16 = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return np.concatenate([d16, qs], axis=1).reshape(n, -1)


def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """GGML Q8_0: d = amax/127, q = round-half-away-from-zero(x * (1/d))."""
    n, k = w.shape
    blk = w.reshape(-1, 32).astype(F32)
    amax = np.max(np.abs(blk), axis=1)
    d = (amax / F32(127.0)).astype(F32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, F32(1.0) / np.where(d != 0, d, F32(1.0)), F32(0.0)).astype(F32)
    v = (blk * inv[:, None]).astype(F32).astype(np.float64)
    q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int8)
    d16 = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return np.concatenate([d16, q.view(np.uint8)], axis=1).reshape(n, -1)


def dequant(qtype: int, blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    bb = 18 if qtype == 2 else 34
    b = blocks.reshape(-1, bb)
    d = b[:, :2].copy().view(np.float16).astype(F32)  # [nb, 1]
    if qtype == 2:
        qs = b[:, 2:].astype(np.int32)
        q = np.concatenate([(qs & 0xF) - 8, (qs >> 4) - 8], axis=1)
    else:
        q = b[:, 2:].view(np.int8).astype(np.int32)
    return (q.astype(F32) * d).astype(F32).reshape(n, k)


def edge_weights(k: int) -> np.ndarray:
    """Hand-built rows exercising the quantizers' special cases."""
    rows = []
    z = np.zeros(k, F32)
    rows.append(z)                                      # all-zero blocks: d = 0
    r = np.zeros(k, F32); r[::32] = 1.0; rows.append(r)   # positive max -> d < 0
    r = np.zeros(k, F32); r[5::32] = -3.0; rows.append(r)  # negative max -> d > 0
    r = np.full(k, 0.25, F32); rows.append(r)               # constant block
    r = np.linspace(-1, 1, k, dtype=F32); rows.append(r)    # ramp: many ties
    r = np.zeros(k, F32); r[::2] = 1e-6; r[1::2] = -1e-6; rows.append(r)  # tiny: f16 subnormal d
    r = np.full(k, 7.0e4, F32); r[1::3] = -7.0e4; rows.append(r)  # large magnitudes, d still finite in f16
    return np.stack(rows)


def make_case(rng: np.random.Generator, qtype: int, m: int, n: int, k: int, edges: bool):
    w = rng.normal(0.0, 0.02, size=(n, k)).astype(F32)
    if edges:
        e = edge_weights(k)
        w[: e.shape[0]] = e
    blocks = quantize_q4_0(w) if qtype == 2 else quantize_q8_0(w)
    deq = dequant(qtype, blocks, n, k)
    x = rng.normal(0.0, 1.0, size=(m, k)).astype(F32)
    y = x.astype(np.float64) @ deq.astype(np.float64).T
    case = dict(w=w, blocks=blocks, x=x, y=y,
                qtype=np.int32(qtype), m=np.int32(m), n=np.int32(n), k=np.int32(k))
    if n * k <= 8192:
        case["deq"] = deq  # kept only where small; y pins the larger cases
    return case


CASES = [
    # name, qtype, m, n, k, edges
    ("q4_0_m1_n16_k64", 2, 1, 16, 64, True),
    ("q4_0_m3_n37_k96", 2, 3, 37, 96, True),
    ("q4_0_m5_n64_k2048", 2, 5, 64, 2048, False),
    ("q4_0_m1_n33_k4128", 2, 1, 33, 4128, True),
    ("q8_0_m1_n16_k64", 8, 1, 16, 64, True),
    ("q8_0_m2_n41_k160", 8, 2, 41, 160, True),
    ("q8_0_m4_n64_k2048", 8, 4, 64, 2048, False),
]


def main() -> None:
    rng = np.random.default_rng(20240601)
    for name, qtype, m, n, k, edges in CASES:
        case = make_case(rng, qtype, m, n, k, edges)
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **case)
        print(f"wrote {name}.npz  blocks={case['blocks'].nbytes} B")


if __name__ == "__main__":
    main()
