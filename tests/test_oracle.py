"""Pin the CPU oracle (oracle/) before it is trusted as the parity checker.

Each check is chosen so that a plausible mistake in the oracle fails it:
wrong nibble order, a dropped -8 offset, a wrong f16 rounding mode, a sign
slip in the Q4_0 scale, a transposed matmul operand.  Sources of truth:
numpy's float16 conversions and float64 matmul (library routines), exhaustive
closed forms, the reference's layout-neutral known-answer tests, and the
independent numpy restatement whose output is committed in tests/golden/.
"""
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
