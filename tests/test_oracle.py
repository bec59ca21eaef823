"""Pin the CPU oracle (oracle/) before it is trusted as the parity checker.

Each check is chosen so that a plausible mistake in the oracle fails it:
wrong nibble order, a dropped -8 offset, a wrong f16 rounding mode, a sign
slip in the Q4_0 scale, a transposed matmul operand.  Sources of truth:
numpy's float16 conversions and float64 matmul (library routines), exhaustive
closed forms, the reference's layout-neutral known-answer tests, and the
independent numpy restatement whose output is committed in tests/golden/.
"""
import os
import sys

import numpy as np
import pytest

import oracle
from oracle import Q4_0, Q8_0


def _block_q4(d16: int, qs) -> np.ndarray:
    b = np.zeros(18, np.uint8)
    b[0], b[1] = d16 & 0xFF, d16 >> 8
    b[2:] = np.asarray(qs, np.uint8)
    return b


def _f16(x: float) -> int:
    return int(np.array([x], np.float16).view(np.uint16)[0])


# ---- f16 <-> f32 ---------------------------------------------------------------

def test_f16_to_f32_exhaustive_matches_numpy():
    codes = np.arange(65536, dtype=np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(c)) for c in codes], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even_matches_numpy():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, 2.0**-24, 2.0**-25,
                        2.0**-25 * 1.0000001, 3 * 2.0**-26, 2.0**-14, 2.0**-14 * (1 - 2**-12),
                        1.0 + 2**-11, 1.0 + 3 * 2**-11, np.inf, -np.inf], np.float32)
    # halfway cases between neighbouring f16 values exercise ties-to-even
    h = np.arange(0x0400, 0x7BFF, 97, dtype=np.uint16).view(np.float16).astype(np.float64)
    h2 = np.arange(0x0401, 0x7C00, 97, dtype=np.uint16).view(np.float16).astype(np.float64)
    ties = ((h + h2) / 2).astype(np.float32)
    vals = np.concatenate([vals, special, -special, ties, -ties])
    vals = vals[~np.isnan(vals)]
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


# ---- dequant: closed form, exhaustive ------------------------------------------------

def test_q4_0_dequant_exhaustive_all_scales_all_codes():
    # qs[j] = j | (15 - j) << 4 puts every code in both nibble positions.
    qs = np.array([j | ((15 - j) << 4) for j in range(16)], np.uint8)
    codes = np.arange(65536, dtype=np.uint16)
    blocks = np.zeros((65536, 18), np.uint8)
    blocks[:, 0:2] = codes.view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = qs
    got = oracle.dequant(Q4_0, blocks, 65536, 32)
    d = codes.view(np.float16).astype(np.float64)[:, None]
    q = np.concatenate([np.arange(16), 15 - np.arange(16)]).astype(np.float64) - 8
    with np.errstate(invalid="ignore"):
        want = d * q[None, :]            # exact in f64; must also be exact in f32
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].astype(np.float64), want[fin])
    assert np.array_equal(np.isnan(got), np.isnan(want))


def test_q8_0_dequant_exhaustive_all_scales_all_codes():
    codes = np.arange(65536, dtype=np.uint16)
    q = np.arange(-128, 128, dtype=np.int64)
    for part in range(8):  # 8 blocks of 32 cover all 256 byte values
        blocks = np.zeros((65536, 34), np.uint8)
        blocks[:, 0:2] = codes.view(np.uint8).reshape(-1, 2)
        qp = q[part * 32:(part + 1) * 32]
        blocks[:, 2:] = qp.astype(np.int8).view(np.uint8)
        got = oracle.dequant(Q8_0, blocks, 65536, 32)
        d = codes.view(np.float16).astype(np.float64)[:, None]
        with np.errstate(invalid="ignore"):
            want = d * qp.astype(np.float64)[None, :]
        fin = np.isfinite(want)
        assert np.array_equal(got[fin].astype(np.float64), want[fin])


# ---- the reference's known-answer tests, restated in GGML block order ----------------

def test_known_answer_0x88_is_zero():
    # crates/runtime/src/simd/quant/block.rs:398-409 (layout-neutral)
    got = oracle.dequant(Q4_0, _block_q4(_f16(0.5), [0x88] * 16), 1, 32)
    assert np.all(got == 0.0)


def test_known_answer_0xF0_in_ggml_order():
    # block.rs:411-423 asserts v[0] = -8, v[1] = +7 under its interleaved layout;
    # the GGUF/GGML layout candle reads puts low nibbles at 0..15, high at 16..31.
    got = oracle.dequant(Q4_0, _block_q4(_f16(1.0), [0xF0] * 16), 1, 32)[0]
    assert np.all(got[:16] == -8.0) and np.all(got[16:] == 7.0)


def test_known_answer_block_dot_32():
    # q4_0.rs:143-157 and arch/avx2.rs:569-594: 0x99, d = 1, x = 1 -> 32
    blocks = _block_q4(_f16(1.0), [0x99] * 16)[None, :]
    y = oracle.qmatmul_f64(Q4_0, blocks, np.ones((1, 32), np.float32), 1, 32)
    assert y[0, 0] == 32.0
    y0 = oracle.qmatmul_f64(Q4_0, _block_q4(_f16(1.0), [0x88] * 16)[None, :],
                            np.ones((1, 32), np.float32), 1, 32)
    assert y0[0, 0] == 0.0  # q4_0.rs:131-141


def test_known_answer_gemv_6p4():
    # q4_0.rs:160-178 and simd/matmul/gemv.rs:91-113: 2 rows x 64, d = f16(0.1),
    # 0x99, x = 1 -> 64 * 0.0999755859375 = 6.3984375 exactly.
    blocks = np.stack([_block_q4(_f16(0.1), [0x99] * 16)] * 4).reshape(2, 36)
    y = oracle.qmatmul_f64(Q4_0, blocks, np.ones((1, 64), np.float32), 2, 64)
    assert np.all(y == 6.3984375)
    # simd/matmul/gemm.rs:377-402: 3 tokens x (2 x 64) -> 6.3984375 everywhere
    y3 = oracle.qmatmul_f64(Q4_0, blocks, np.ones((3, 64), np.float32), 2, 64)
    assert y3.shape == (3, 2) and np.all(y3 == 6.3984375)


def test_known_answer_gemm_12p8():
    # simd/matmul/gemm.rs:404-429: 8 tokens x (4 rows x 128) -> 128 * 0.0999755859375
    blocks = np.stack([_block_q4(_f16(0.1), [0x99] * 16)] * 16).reshape(4, 72)
    y = oracle.qmatmul_f64(Q4_0, blocks, np.ones((8, 128), np.float32), 4, 128)
    assert y.shape == (8, 4) and np.all(y == 12.796875)


# ---- quantizers ------------------------------------------------------------------------

def test_quantizers_match_independent_numpy_restatement(golden_cases):
    for name, c in golden_cases.items():
        got = oracle.quantize(int(c["qtype"]), c["w"])
        assert np.array_equal(got, c["blocks"]), name


def test_dequant_matches_golden(golden_cases):
    for name, c in golden_cases.items():
        if "deq" in c:
            got = oracle.dequant(int(c["qtype"]), c["blocks"], int(c["n"]), int(c["k"]))
            assert np.array_equal(got.view(np.uint32), c["deq"].view(np.uint32)), name


def test_q4_0_quantizer_invariants():
    w = oracle.normal(64 * 256, seed=7, std=0.02).reshape(64, 256)
    blocks = oracle.quantize(Q4_0, w).reshape(-1, 18)
    blk = w.reshape(-1, 32)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32)[:, 0]
    lo = blocks[:, 2:] & 0xF
    hi = blocks[:, 2:] >> 4
    codes = np.concatenate([lo, hi], axis=1)
    # the element of largest magnitude maps to code 0, and d carries the opposite sign
    idx = np.argmax(np.abs(blk), axis=1)
    assert np.all(codes[np.arange(len(idx)), idx] == 0)
    assert np.all(np.sign(d) == -np.sign(blk[np.arange(len(idx)), idx]))
    # round trip error is at most half a step (plus the f16 rounding of d),
    # except where the code clamps at 15 (values beyond +7.5 steps): one step
    deq = oracle.dequant(Q4_0, blocks.reshape(64, -1), 64, 256).reshape(-1, 32)
    dd = np.abs(blk[np.arange(len(idx)), idx].astype(np.float64) / 8.0)[:, None]
    err = np.abs(deq.astype(np.float64) - blk)
    half_step = err <= dd * (0.5 + 8 * 2.0**-11) + 1e-12
    clamped = (codes == 15) & (err <= dd * (1.0 + 8 * 2.0**-11) + 1e-12)
    assert np.all(half_step | clamped)
    assert np.mean(half_step) > 0.99


def test_q8_0_quantizer_invariants():
    w = oracle.normal(32 * 512, seed=9, std=0.02).reshape(32, 512)
    blocks = oracle.quantize(Q8_0, w)
    deq = oracle.dequant(Q8_0, blocks, 32, 512).reshape(-1, 32).astype(np.float64)
    blk = w.reshape(-1, 32).astype(np.float64)
    d = np.max(np.abs(blk), axis=1) / 127.0
    err = np.abs(deq - blk)
    assert np.all(err <= (d * (0.5 + 127 * 2.0**-11) + 1e-12)[:, None])
    q = blocks.reshape(-1, 34)[:, 2:].view(np.int8)
    assert np.all(np.max(np.abs(q.astype(np.int32)), axis=1) == 127)


def test_q4_0_all_zero_block_is_0x88():
    # max stays 0.0f, so d = 0.0f / -8 = -0.0f: the stored scale is f16 -0 (0x8000)
    blocks = oracle.quantize(Q4_0, np.zeros((1, 32), np.float32))
    assert blocks[0, 0] == 0x00 and blocks[0, 1] == 0x80 and np.all(blocks[0, 2:] == 0x88)
    assert np.all(oracle.dequant(Q4_0, blocks, 1, 32) == 0.0)


# ---- the f64 matmul oracle -------------------------------------------------------------

@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_qmatmul_f64_matches_numpy_float64(qtype):
    n, k, m = 29, 320, 3
    w = oracle.normal(n * k, seed=11, std=0.02).reshape(n, k)
    x = oracle.normal(m * k, seed=12).reshape(m, k)
    blocks = oracle.quantize(qtype, w)
    deq = oracle.dequant(qtype, blocks, n, k).astype(np.float64)
    want = x.astype(np.float64) @ deq.T
    got = oracle.qmatmul_f64(qtype, blocks, x, n, k)
    assert got.shape == (m, n)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # a transposed or mis-indexed operand would break this non-square case
    assert not np.allclose(got[:, 1:], want[:, :-1])


def test_qmatmul_f64_matches_golden(golden_cases):
    for name, c in golden_cases.items():
        got = oracle.qmatmul_f64(int(c["qtype"]), c["blocks"], c["x"], int(c["n"]), int(c["k"]))
        np.testing.assert_allclose(got, c["y"], rtol=1e-10, atol=1e-10, err_msg=name)


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_candle_semantics_path_close_to_oracle(qtype):
    n, k, m = 300, 2048, 2
    w = oracle.normal(n * k, seed=21, std=0.02).reshape(n, k)
    x = oracle.normal(m * k, seed=22).reshape(m, k)
    blocks = oracle.quantize(qtype, w)
    ref = oracle.qmatmul_f64(qtype, blocks, x, n, k)
    got = oracle.candle_qmatmul(qtype, blocks, x, n, k)
    e = oracle.normwise_error(got, ref)
    # Q8_0 activation rounding: a few 1e-3 normwise, never exact
    assert 1e-5 < e < 2e-2


def test_fill_normal_is_deterministic_and_normal():
    a = oracle.normal(200_001, seed=5)
    b = oracle.normal(200_001, seed=5)
    assert np.array_equal(a, b)
    assert abs(float(a.mean())) < 0.01 and abs(float(a.std()) - 1.0) < 0.01
    assert not np.array_equal(a[:1000], oracle.normal(1000, seed=6))


# ---- Q5_0 (GGML block_q5_0) -------------------------------------------------------------------

from oracle import Q5_0  # noqa: E402


def _q50_block(d, qh, qs) -> np.ndarray:
    b = np.zeros(22, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:6] = np.array([qh], np.uint32).view(np.uint8)
    b[6:] = np.asarray(qs, np.uint8)
    return b


def test_q5_0_code_positions_one_hot():
    # d = 1, base code 16 (weight 0): nibble byte j -> element j (low) / j + 16
    # (high); qh bit i -> element i, adding 16
    cases, want = [], []
    base_qs = np.zeros(16, np.uint8)
    for j in range(16):
        for hi in range(2):
            qs = base_qs.copy()
            qs[j] = 0x50 if hi else 0x05
            cases.append(_q50_block(1.0, 0xFFFFFFFF, qs))  # every fifth bit set: q = 16 + code
            e = np.zeros(32, np.float32)
            e[j + 16 * hi] = 5.0
            want.append(e)
    for i in range(32):
        cases.append(_q50_block(1.0, 0xFFFFFFFF & ~(1 << i), base_qs))
        e = np.zeros(32, np.float32)
        e[i] = -16.0
        want.append(e)
    got = oracle.dequant(Q5_0, np.stack(cases), len(cases), 32)
    assert np.array_equal(got, np.stack(want))


def test_q5_0_exhaustive_scales_and_codes():
    # every f16 d against all 32 codes (element e holds code e): w = (e - 16) d exactly
    qs = np.array([j | (j << 4) for j in range(16)], np.uint8)  # both nibbles of byte j: j
    qh = 0xFFFF0000  # elements 16..31 get the fifth bit: codes 16 + j
    codes = np.concatenate([np.arange(16), 16 + np.arange(16)]).astype(np.float32)
    blocks = np.tile(_q50_block(0.0, qh, qs), (65536, 1))
    blocks[:, 0:2] = np.arange(65536, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    got = oracle.dequant(Q5_0, blocks, 65536, 32)
    d = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)[:, None]
    with np.errstate(invalid="ignore"):  # inf * 0 for the code 16 of an infinite d
        want = (codes[None, :] - 16.0) * d
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], want[~nan])


def _numpy_q5_0(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 22)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    hb = np.unpackbits(b[:, 2:6], axis=1, bitorder="little").astype(np.int32)  # [nb][32]
    qs = b[:, 6:].astype(np.int32)
    lo = np.concatenate([qs & 15, qs >> 4], axis=1)
    return ((lo | (hb << 4)) - 16).astype(np.float32) * d[:, None]


def test_q5_0_random_blocks_match_numpy_decoder():
    blocks = oracle.random_q5_0(64, 1024, seed=12)
    got = oracle.dequant(Q5_0, blocks, 64, 1024)
    assert np.array_equal(got.reshape(-1, 32), _numpy_q5_0(blocks))


# ---- Q4_K / Q5_K / Q6_K (GGML block_q4_K / block_q5_K / block_q6_K) ---------------------------------------------

from oracle import Q4_K, Q5_K, Q6_K  # noqa: E402


def _q4k_block(d, dmin, sc, m, qs) -> np.ndarray:
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    b[4:16] = oracle.pack_q4_k_scales(sc, m)
    b[16:] = np.asarray(qs, np.uint8)
    return b


def test_q4_k_code_positions_one_hot():
    # d = 1, every scale 1, every min 0: weight = code.  Byte b of qs, low nibble
    # -> weight 64 (b // 32) + b % 32; high nibble -> the same + 32.
    blocks = []
    want = np.zeros((256, 256), np.float32)
    for case in range(256):
        b, hi = case // 2, case % 2
        qs = np.zeros(128, np.uint8)
        qs[b] = 0x50 if hi else 0x05
        blocks.append(_q4k_block(1.0, 0.0, [1] * 8, [0] * 8, qs))
        want[case, 64 * (b // 32) + b % 32 + 32 * hi] = 5.0
    got = oracle.dequant(Q4_K, np.stack(blocks), 256, 256)
    assert np.array_equal(got, want)


def test_q4_k_scale_and_min_per_sub_block():
    # every code 1, scale of sub-block j = j + 1: weights 32 j .. 32 j + 31 = j + 1
    got = oracle.dequant(Q4_K, _q4k_block(1.0, 0.0, range(1, 9), [0] * 8, [0x11] * 128), 1, 256)
    assert np.array_equal(got[0], np.repeat(np.arange(1, 9, dtype=np.float32), 32))
    # every code 0, dmin 1, min of sub-block j = 2 j + 1: weights = -(2 j + 1)
    got = oracle.dequant(Q4_K, _q4k_block(1.0, 1.0, [1] * 8, range(1, 17, 2), [0] * 128), 1, 256)
    assert np.array_equal(got[0], -np.repeat(np.arange(1, 17, 2, dtype=np.float32), 32))


def test_q4_k_scale_packing_inverse_of_ggml_packer():
    # all 64 x 64 (scale, min) values in every sub-block position, the other
    # positions random: the oracle's unpacking must return exactly what GGML's
    # packer stored (codes 1 and 0 read back the scale and the min separately)
    rng = np.random.default_rng(3)
    for j in range(8):
        blocks1, blocks0, want_sc, want_m = [], [], [], []
        for v in range(64 * 64):
            sc = rng.integers(0, 64, 8)
            m = rng.integers(0, 64, 8)
            sc[j], m[j] = v // 64, v % 64
            blocks1.append(_q4k_block(1.0, 0.0, sc, m, [0x11] * 128))
            blocks0.append(_q4k_block(1.0, 1.0, sc, m, [0x00] * 128))
            want_sc.append(sc[j])
            want_m.append(m[j])
        s = oracle.dequant(Q4_K, np.stack(blocks1), 4096, 256)[:, 32 * j:32 * j + 32]
        mn = oracle.dequant(Q4_K, np.stack(blocks0), 4096, 256)[:, 32 * j:32 * j + 32]
        assert np.array_equal(s, np.repeat(np.array(want_sc, np.float32)[:, None], 32, 1))
        assert np.array_equal(mn, -np.repeat(np.array(want_m, np.float32)[:, None], 32, 1))


def _numpy_q4_k(blocks: np.ndarray) -> np.ndarray:
    """Independent vectorised decoding: 6-bit fields by bit position, codes by
    reshaping qs to [4 groups][32 bytes] (low nibbles first)."""
    b = blocks.reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    bits = np.unpackbits(b[:, 4:16], axis=1, bitorder="little")  # [nb, 96], bit i of byte i // 8
    def field(byte, lo, width):
        return sum(bits[:, 8 * byte + lo + t].astype(np.int64) << t for t in range(width))
    sc = np.stack([field(j, 0, 6) if j < 4 else field(j + 4, 0, 4) | (field(j - 4, 6, 2) << 4)
                   for j in range(8)], 1)
    m = np.stack([field(j + 4, 0, 6) if j < 4 else field(j + 4, 4, 4) | (field(j, 6, 2) << 4)
                  for j in range(8)], 1)
    q = b[:, 16:].reshape(-1, 4, 32)
    codes = np.concatenate([q & 15, q >> 4], axis=2).reshape(-1, 8, 32).astype(np.float32)
    s1 = (d[:, None] * sc.astype(np.float32))[:, :, None]
    m1 = (dmin[:, None] * m.astype(np.float32))[:, :, None]
    return (s1 * codes - m1).astype(np.float32).reshape(-1, 256)


def test_q4_k_random_blocks_match_numpy_decoder():
    blocks = oracle.random_q4_k(64, 1024, seed=9)
    got = oracle.dequant(Q4_K, blocks, 64, 1024)
    assert np.array_equal(got.reshape(-1, 256), _numpy_q4_k(blocks))


def _q5k_block(d, dmin, sc, m, qh, qs) -> np.ndarray:
    b = np.zeros(176, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    b[4:16] = oracle.pack_q4_k_scales(sc, m)
    b[16:48] = np.asarray(qh, np.uint8)
    b[48:] = np.asarray(qs, np.uint8)
    return b


def test_q5_k_code_positions_one_hot():
    # d = 1, scales 1, mins 0: weight = code.  Nibbles as Q4_K (byte b of qs: low
    # -> weight 64 (b // 32) + b % 32, high -> + 32); bit j of qh[l] adds 16 to
    # weight 32 j + l.
    cases, want = [], []
    for b in range(128):
        for hi in range(2):
            qs = np.zeros(128, np.uint8)
            qs[b] = 0x50 if hi else 0x05
            cases.append(_q5k_block(1.0, 0.0, [1] * 8, [0] * 8, np.zeros(32, np.uint8), qs))
            e = np.zeros(256, np.float32)
            e[64 * (b // 32) + b % 32 + 32 * hi] = 5.0
            want.append(e)
    for l in range(32):
        for j in range(8):
            qh = np.zeros(32, np.uint8)
            qh[l] = 1 << j
            cases.append(_q5k_block(1.0, 0.0, [1] * 8, [0] * 8, qh, np.zeros(128, np.uint8)))
            e = np.zeros(256, np.float32)
            e[32 * j + l] = 16.0
            want.append(e)
    got = oracle.dequant(Q5_K, np.stack(cases), len(cases), 256)
    assert np.array_equal(got, np.stack(want))


def test_q5_k_scale_min_and_full_code_range():
    # all codes 31 (nibble 15, every qh bit set), scale of sub-block j = j + 1:
    # weights of sub-block j = 31 (j + 1); then all codes 0 with dmin 1 and min
    # 2 j + 1: -(2 j + 1).  The scale packing is Q4_K's (pinned above).
    got = oracle.dequant(Q5_K, _q5k_block(1.0, 0.0, range(1, 9), [0] * 8, [0xFF] * 32,
                                          [0xFF] * 128), 1, 256)
    assert np.array_equal(got[0], 31.0 * np.repeat(np.arange(1, 9, dtype=np.float32), 32))
    got = oracle.dequant(Q5_K, _q5k_block(1.0, 1.0, [1] * 8, range(1, 17, 2), [0] * 32,
                                          [0] * 128), 1, 256)
    assert np.array_equal(got[0], -np.repeat(np.arange(1, 17, 2, dtype=np.float32), 32))


def _numpy_q5_k(blocks: np.ndarray) -> np.ndarray:
    """Independent decoding: Q4_K's fields by bit position, the fifth bits by
    unpacking qh to [32 weights][8 sub-blocks]."""
    b = blocks.reshape(-1, 176)
    as_q4k = np.concatenate([b[:, 0:16], b[:, 48:176]], axis=1)   # d, dmin, scales, qs
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    bits = np.unpackbits(b[:, 4:16], axis=1, bitorder="little")
    def field(byte, lo, width):
        return sum(bits[:, 8 * byte + lo + t].astype(np.int64) << t for t in range(width))
    sc = np.stack([field(j, 0, 6) if j < 4 else field(j + 4, 0, 4) | (field(j - 4, 6, 2) << 4)
                   for j in range(8)], 1)
    m = np.stack([field(j + 4, 0, 6) if j < 4 else field(j + 4, 4, 4) | (field(j, 6, 2) << 4)
                  for j in range(8)], 1)
    q = as_q4k[:, 16:].reshape(-1, 4, 32)
    lo = np.concatenate([q & 15, q >> 4], axis=2).reshape(-1, 8, 32).astype(np.int32)
    hb = np.unpackbits(b[:, 16:48].reshape(-1, 32, 1), axis=2, bitorder="little")  # [nb][l][j]
    codes = (lo + 16 * hb.transpose(0, 2, 1).astype(np.int32)).astype(np.float32)
    s1 = (d[:, None] * sc.astype(np.float32))[:, :, None]
    m1 = (dmin[:, None] * m.astype(np.float32))[:, :, None]
    return (s1 * codes - m1).astype(np.float32).reshape(-1, 256)


def test_q5_k_random_blocks_match_numpy_decoder():
    blocks = oracle.random_q5_k(64, 1024, seed=11)
    got = oracle.dequant(Q5_K, blocks, 64, 1024)
    assert np.array_equal(got.reshape(-1, 256), _numpy_q5_k(blocks))


def _q6k_block(d, sc, ql, qh) -> np.ndarray:
    b = np.zeros(210, np.uint8)
    b[0:128] = np.asarray(ql, np.uint8)
    b[128:192] = np.asarray(qh, np.uint8)
    b[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    b[208:210] = np.array([d], np.float16).view(np.uint8)
    return b


def test_q6_k_code_positions_one_hot():
    # d = 1, scales 1, all codes 32 (weight 0) except one field.  ql byte
    # 64 h + c: low nibble -> weight 128 h + c, high -> + 64 (c < 32 covers
    # weights c, c + 64; c >= 32 covers c, c + 64 as well: l + 32 and l + 96);
    # qh byte 32 h + l, bit pair t -> weight 128 h + l + 32 t.
    cases, want = [], []
    base_ql, base_qh = np.zeros(128, np.uint8), np.full(64, 0xAA, np.uint8)  # q = 0 | 2 << 4 = 32
    for h in range(2):
        for c in range(64):
            for hi in range(2):
                ql = base_ql.copy()
                ql[64 * h + c] = 0x70 if hi else 0x07
                cases.append(_q6k_block(1.0, [1] * 16, ql, base_qh))
                e = np.zeros(256, np.float32)
                e[128 * h + c + 64 * hi] = 7.0
                want.append(e)
        for l in range(32):
            for t in range(4):
                qh = base_qh.copy()
                qh[32 * h + l] = (0xAA & ~(3 << (2 * t))) | (3 << (2 * t))  # that pair 3: q = 48
                cases.append(_q6k_block(1.0, [1] * 16, base_ql, qh))
                e = np.zeros(256, np.float32)
                e[128 * h + l + 32 * t] = 16.0
                want.append(e)
    got = oracle.dequant(Q6_K, np.stack(cases), len(cases), 256)
    assert np.array_equal(got, np.stack(want))


def test_q6_k_scale_per_16_weights():
    # codes all 33 (weight = scale), scale s -> weights 16 s .. 16 s + 15 in the
    # order GGML indexes them: weight l + 32 t of half h uses scales[8 h + l // 16 + 2 t]
    sc = np.arange(1, 17, dtype=np.int8) * np.array([1, -1] * 8, np.int8)
    got = oracle.dequant(Q6_K, _q6k_block(1.0, sc, [0x11] * 128, [0xAA] * 64), 1, 256)[0]
    want = np.empty(256, np.float32)
    for e in range(256):
        h, r = divmod(e, 128)
        want[e] = sc[8 * h + (r % 32) // 16 + 2 * (r // 32)]
    assert np.array_equal(got, want)


def _numpy_q6_k(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 210)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    sc = b[:, 192:208].view(np.int8).astype(np.float32).reshape(-1, 2, 4, 2)  # [h][t][l // 16]
    ql = b[:, 0:128].reshape(-1, 2, 2, 32)   # [h][which 32][l]
    qh = b[:, 128:192].reshape(-1, 2, 32)    # [h][l]
    lo = np.stack([ql[:, :, 0] & 15, ql[:, :, 1] & 15, ql[:, :, 0] >> 4, ql[:, :, 1] >> 4], 2)
    hb = np.stack([(qh >> (2 * t)) & 3 for t in range(4)], 2)
    q = (lo.astype(np.int32) | (hb.astype(np.int32) << 4)) - 32        # [nb][h][t][l]
    s = np.repeat(sc, 16, axis=3)                                        # [nb][h][t][l]
    return ((d[:, None, None, None] * s) * q.astype(np.float32)).astype(np.float32).reshape(-1, 256)


def test_q6_k_random_blocks_match_numpy_decoder():
    blocks = oracle.random_q6_k(64, 1024, seed=10)
    got = oracle.dequant(Q6_K, blocks, 64, 1024)
    assert np.array_equal(got.reshape(-1, 256), _numpy_q6_k(blocks))


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K, Q6_K, Q5_0])
def test_qmatmul_f64_k_quants_match_numpy_float64(qtype):
    n, k, m = 29, 512, 3
    gen = {Q4_K: oracle.random_q4_k, Q5_K: oracle.random_q5_k, Q6_K: oracle.random_q6_k,
           Q5_0: oracle.random_q5_0}[qtype]
    blocks = gen(n, k, seed=12)
    x = oracle.normal(m * k, seed=13).reshape(m, k)
    want = x.astype(np.float64) @ oracle.dequant(qtype, blocks, n, k).astype(np.float64).T
    np.testing.assert_allclose(oracle.qmatmul_f64(qtype, blocks, x, n, k), want,
                               rtol=1e-12, atol=1e-12)


def test_k_quants_rejected_by_q8_paths():
    w = np.zeros((1, 256), np.float32)
    with pytest.raises(ValueError):
        oracle.quantize(Q4_K, w)
    with pytest.raises(ValueError):
        oracle.candle_qmatmul(Q4_K, oracle.random_q4_k(1, 256, 0), w, 1, 256)


# ---- decode attention with a KV cache (llama.rs:827-883, 1044-1150) --------------------------

def _attn(qkv, H, KVH, D, theta=10000.0, max_seq=64, length=0, k=None, v=None):
    k = np.zeros((KVH, max_seq, D), np.float32) if k is None else k
    v = np.zeros((KVH, max_seq, D), np.float32) if v is None else v
    out = oracle.attention_decode(qkv, H, KVH, D, theta, k, v, length)
    return out, k, v


def test_attention_single_position_returns_v():
    H, KVH, D = 4, 2, 8
    qkv = oracle.normal((H + 2 * KVH) * D, seed=1).reshape(1, -1)
    out, _, _ = _attn(qkv, H, KVH, D)
    vv = qkv[0, (H + KVH) * D:].reshape(KVH, D)
    for h in range(H):  # softmax over one position is 1; head h reads kv head h // 2
        assert np.array_equal(out[0, h * D:(h + 1) * D], vv[h // 2].astype(np.float64))


def test_attention_equal_keys_average_values():
    # every cached key the same: uniform weights, out = mean of the values seen
    H, KVH, D, L = 2, 1, 8, 5
    k = np.zeros((KVH, 16, D), np.float32)
    v = np.zeros((KVH, 16, D), np.float32)
    v[0, :L] = oracle.normal(L * D, seed=2).reshape(L, D)
    qkv = oracle.normal((H + 2 * KVH) * D, seed=3).reshape(1, -1)
    qkv[0, H * D:(H + KVH) * D] = 0.0  # the new key: 0, like the cached ones
    out, k, v = _attn(qkv, H, KVH, D, max_seq=16, length=L, k=k, v=v)
    want = v[0, :L + 1].astype(np.float64).mean(axis=0)
    for h in range(H):
        np.testing.assert_allclose(out[0, h * D:(h + 1) * D], want, rtol=1e-12, atol=1e-12)


def test_rope_known_answers_and_pairing():
    # pos 0: identity.  A unit vector at dim i of a key at position p lands on dims i
    # (cos) and i + D/2 (sin) at angle p * inv_freq[i], inv_freq in f32 as the reference
    H, KVH, D, theta = 1, 1, 8, 10000.0
    m = 6
    qkv = np.zeros((m, (H + 2 * KVH) * D), np.float32)
    kk = oracle.normal(D, seed=4)
    qkv[0, H * D:(H + 1) * D] = kk
    for t in range(1, m):
        qkv[t, H * D + (t - 1) % (D // 2)] = 1.0
    _, k, _ = _attn(qkv, H, KVH, D, theta=theta)
    assert np.array_equal(k[0, 0], kk)
    for t in range(1, m):
        i = (t - 1) % (D // 2)
        ang = np.float32(t) * np.float32(1.0 / np.power(np.float32(theta), np.float32(2 * i) / np.float32(D)))
        want = np.zeros(D, np.float32)
        want[i], want[i + D // 2] = np.cos(np.float64(ang)), np.sin(np.float64(ang))
        np.testing.assert_allclose(k[0, t], want, atol=1e-7)


def test_rope_relative_position_invariant():
    # the same key content at positions 0 .. N-1: <K_j, K_j+s> depends on s only
    H, KVH, D, N = 1, 1, 16, 12
    qkv = np.zeros((N, (H + 2 * KVH) * D), np.float32)
    qkv[:, H * D:(H + 1) * D] = oracle.normal(D, seed=5)
    _, k, _ = _attn(qkv, H, KVH, D, theta=100.0)
    K = k[0, :N].astype(np.float64)
    for s in range(1, 4):
        d = [K[j] @ K[j + s] for j in range(N - s)]
        np.testing.assert_allclose(d, d[0], rtol=1e-5)
    np.testing.assert_allclose(np.linalg.norm(K, axis=1), np.linalg.norm(K[0]), rtol=1e-6)


def test_attention_causal_and_gqa_heads():
    # two new tokens: token 0 must not see token 1's key / value
    H, KVH, D = 4, 2, 8
    qkv = oracle.normal(2 * (H + 2 * KVH) * D, seed=6).reshape(2, -1)
    out_a, _, _ = _attn(qkv, H, KVH, D, length=3,
                        k=oracle.normal(2 * 64 * D, seed=7).reshape(2, 64, D).copy(),
                        v=oracle.normal(2 * 64 * D, seed=8).reshape(2, 64, D).copy())
    qkv2 = qkv.copy()
    qkv2[1, H * D:] = 1e3  # token 1's k and v only
    out_b, _, _ = _attn(qkv2, H, KVH, D, length=3,
                        k=oracle.normal(2 * 64 * D, seed=7).reshape(2, 64, D).copy(),
                        v=oracle.normal(2 * 64 * D, seed=8).reshape(2, 64, D).copy())
    assert np.array_equal(out_a[0], out_b[0]) and not np.allclose(out_a[1], out_b[1])


def test_attention_overflow_rejected():
    with pytest.raises(ValueError):
        _attn(np.zeros((3, 4 * 8), np.float32), 2, 1, 8, max_seq=4, length=2)


# ---- the attention softmax against an independent restatement --------------------------------
# tests/golden/llama_attention_np.py restates forward_with_cache's attention (llama.rs:827-883,
# 890, 1108-1148) in numpy's tensor form; random, non-uniform keys make the softmax temperature
# and base visible, which the closed-form checks above are blind to.

def _np_attention():
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    import llama_attention_np
    return llama_attention_np


def _attention_case(H, KVH, D, L, m, seed, theta=10000.0, scale=None, exp=np.exp):
    """The oracle and the restatement on the same cache prefix and new tokens."""
    ref = _np_attention()
    max_seq = L + m + 3
    pre = oracle.normal(L * (H + 2 * KVH) * D, seed=seed).reshape(L, -1) if L else None
    qkv = oracle.normal(m * (H + 2 * KVH) * D, seed=seed + 1).reshape(m, -1)
    k = np.zeros((KVH, max_seq, D), np.float32)
    v = np.zeros((KVH, max_seq, D), np.float32)
    cache = ref.KvCacheNp(H, D)
    if L:  # fill the prefix through both: one prompt call of L tokens
        oracle.attention_decode(pre, H, KVH, D, theta, k, v, 0)
        ref.forward_with_cache_attention(pre, H, KVH, D, theta, cache)
    got = oracle.attention_decode(qkv, H, KVH, D, theta, k, v, L)
    want = ref.forward_with_cache_attention(qkv, H, KVH, D, theta, cache, scale=scale, exp=exp)
    # the cache contents agree too (GQA: every query head of kv head g holds g's rows)
    for h in range(H):
        assert np.array_equal(cache.k[h], k[h // (H // KVH), :L + m])
        assert np.array_equal(cache.v[h], v[h // (H // KVH), :L + m])
    return got, want


@pytest.mark.parametrize("D", [8, 64])
@pytest.mark.parametrize("L", [1, 5, 33])
@pytest.mark.parametrize("m", [1, 3])
def test_attention_matches_numpy_restatement(D, L, m):
    got, want = _attention_case(4, 2, D, L, m, seed=1000 + 7 * D + L + m)
    # non-uniform weights: the scores spread over more than a unit
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_attention_restatement_covers_mha_and_mqa():
    for H, KVH in ((4, 4), (4, 1)):
        got, want = _attention_case(H, KVH, 64, 9, 2, seed=77)
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("mistake", ["scale 1/hd", "scale 1", "f64 scale", "exp2"])
def test_attention_comparison_catches_planted_softmax_mistakes(mistake):
    """A wrong temperature or base planted in the restatement (on the CPU) must
    fail the comparison above: the check has the power to see it.  The f64 scale
    1/sqrt(hd) is the reference's f32 scale rounded differently: at hd 8 it moves
    results by ~1e-8, which the 1e-12 comparison sees."""
    D = 8 if mistake == "f64 scale" else 64
    scale = {"scale 1/hd": 1.0 / D, "scale 1": 1.0, "f64 scale": 1.0 / np.sqrt(D)}.get(mistake)
    exp = np.exp2 if mistake == "exp2" else np.exp
    got, want = _attention_case(4, 2, D, 5, 3, seed=4242, scale=scale, exp=exp)
    assert not np.allclose(got, want, rtol=1e-12, atol=1e-12)
