"""GPU parity: the HIP kernels, called through the C ABI, against the CPU oracle.

Bars: dequant bit-exact; every matmul path within 1e-3 of the f64 matmul of the
exactly dequantized weights, measured normwise as max|y - r| / max|r|.  (The
north star allows 2e-2 for a bf16 prefill; the prefill path here runs f16
operands, each row of x scaled by a power of two, and meets the GEMV's 1e-3.)
"""
import numpy as np
import pytest
import torch

import oracle
from oracle import Q4_0, Q8_0
from unillm_amd import (PATH_AUTO, PATH_DECODE_MFMA, PATH_GEMV, PATH_PREFILL_MFMA, HipError,
                        QuantLinear, quantize_blocks)

pytestmark = pytest.mark.gpu

# every path runs on exact integer digits of x (GEMV) or on f16 operands (MFMA)
TOL = {PATH_GEMV: 1e-3, PATH_DECODE_MFMA: 1e-3, PATH_PREFILL_MFMA: 1e-3}


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _case(qtype, m, n, k, seed):
    w = oracle.normal(n * k, seed=seed, std=0.02).reshape(n, k)
    x = oracle.normal(m * k, seed=seed + 1).reshape(m, k)
    return oracle.quantize(qtype, w), x


def _run(ql: QuantLinear, x: np.ndarray, path: int) -> np.ndarray:
    y = ql.forward(_dev(x), path=path)
    torch.cuda.synchronize()
    return y.cpu().numpy()


# ---- dequant: bit-exact ------------------------------------------------------------------

@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_dequant_bit_exact_all_scales_all_codes(qtype):
    codes = np.arange(65536, dtype=np.uint16)
    if qtype == Q4_0:  # one block holds every code in both nibble positions
        nblk = 1
        blocks = np.zeros((65536, nblk, 18), np.uint8)
        blocks[:, 0, 2:] = np.array([j | ((15 - j) << 4) for j in range(16)], np.uint8)
    else:  # eight blocks hold all 256 byte values
        nblk = 8
        blocks = np.zeros((65536, nblk, 34), np.uint8)
        blocks[:, :, 2:] = np.arange(256, dtype=np.uint8).reshape(8, 32)
    blocks[:, :, 0:2] = codes.view(np.uint8).reshape(-1, 1, 2)
    k = 32 * nblk
    ql = QuantLinear.from_blocks(qtype, 65536, k, blocks)
    got = ql.dequantize().cpu().numpy()
    want = oracle.dequant(qtype, blocks, 65536, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qtype,n,k", [(Q4_0, 37, 96), (Q4_0, 300, 4096), (Q8_0, 41, 160),
                                       (Q8_0, 128, 2048)])
def test_dequant_bit_exact_random(qtype, n, k):
    blocks, _ = _case(qtype, 1, n, k, seed=100 + n)
    got = QuantLinear.from_blocks(qtype, n, k, blocks).dequantize().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), oracle.dequant(qtype, blocks, n, k).view(np.uint32))


def test_dequant_golden(golden_cases):
    for name, c in golden_cases.items():
        ql = QuantLinear.from_blocks(int(c["qtype"]), int(c["n"]), int(c["k"]), c["blocks"])
        got = ql.dequantize().cpu().numpy()
        want = oracle.dequant(int(c["qtype"]), c["blocks"], int(c["n"]), int(c["k"]))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name


# ---- device quantizer: bit-exact with GGML ---------------------------------------------------

@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_device_quantizer_bit_exact(qtype, golden_cases):
    for name, c in golden_cases.items():
        got = quantize_blocks(qtype, _dev(c["w"])).cpu().numpy()
        assert np.array_equal(got, oracle.quantize(qtype, c["w"]).reshape(-1)), name
    w = oracle.normal(512 * 1024, seed=3, std=0.02).reshape(512, 1024)
    w[0, :64] = 0.0
    w[1, 5] = 1e-6
    got = quantize_blocks(qtype, _dev(w)).cpu().numpy()
    assert np.array_equal(got, oracle.quantize(qtype, w).reshape(-1))


# ---- the reference's known answers --------------------------------------------------------

@pytest.mark.parametrize("path,m", [(PATH_GEMV, 1), (PATH_GEMV, 2), (PATH_GEMV, 3),
                                    (PATH_GEMV, 4), (PATH_DECODE_MFMA, 3),
                                    (PATH_DECODE_MFMA, 8)])
def test_known_answer_6p3984375(path, m):
    # simd/matmul/gemv.rs:91-113, gemm.rs:377-402: d = f16(0.1), 0x99, x = 1
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.array([0.1], np.float16).view(np.uint8)
    blk[2:] = 0x99
    blocks = np.tile(blk, 4)
    y = _run(QuantLinear.from_blocks(Q4_0, 2, 64, blocks), np.ones((m, 64), np.float32), path)
    assert np.all(y == np.float32(6.3984375))


def test_known_answer_12p796875_prefill_exact():
    # gemm.rs:404-429, 8 tokens x 4 rows x 128: f16 operands hold x = 1 (times its
    # row's power of two) and (9 - 8) d exactly, and the f32 sums of equal products
    # are exact, so the prefill path meets the known answer to the bit
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.array([0.1], np.float16).view(np.uint8)
    blk[2:] = 0x99
    y = _run(QuantLinear.from_blocks(Q4_0, 4, 128, np.tile(blk, 16)),
             np.ones((8, 128), np.float32), PATH_PREFILL_MFMA)
    assert np.all(y == np.float32(12.796875))


# ---- matmul parity vs the f64 oracle -------------------------------------------------------

SHAPES = [(37, 96), (33, 4128), (64, 2048), (300, 4096), (129, 11008), (70, 14336)]


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("path,m", [(PATH_GEMV, 1), (PATH_GEMV, 2), (PATH_GEMV, 3),
                                    (PATH_GEMV, 4), (PATH_DECODE_MFMA, 2),
                                    (PATH_DECODE_MFMA, 5), (PATH_DECODE_MFMA, 16),
                                    (PATH_DECODE_MFMA, 33), (PATH_DECODE_MFMA, 64),
                                    (PATH_PREFILL_MFMA, 65), (PATH_PREFILL_MFMA, 130)])
def test_qmatmul_parity(qtype, n, k, path, m):
    blocks, x = _case(qtype, m, n, k, seed=n * 7 + k)
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    if path == PATH_GEMV and ql.select_path(m) != PATH_GEMV:
        pytest.skip("k beyond the GEMV path's register budget at this m")
    y = _run(ql, x, path)
    ref = oracle.qmatmul_f64(qtype, blocks, x, n, k)
    assert y.shape == (m, n)
    e = oracle.normwise_error(y, ref)
    assert e < TOL[path], f"normwise {e:.3g}"
    if path == PATH_GEMV:
        assert e < 1e-4  # two int8 digits of x: ~3e-5, far inside the bar


def test_golden_fixtures_auto_path(golden_cases):
    for name, c in golden_cases.items():
        qtype, m, n, k = (int(c[f]) for f in ("qtype", "m", "n", "k"))
        ql = QuantLinear.from_blocks(qtype, n, k, c["blocks"])
        path = ql.select_path(m)
        y = _run(ql, c["x"], PATH_AUTO)
        assert oracle.normwise_error(y, c["y"]) < TOL[path], name


def test_auto_path_selection():
    blocks, _ = _case(Q4_0, 1, 16, 4096, seed=1)
    ql = QuantLinear.from_blocks(Q4_0, 16, 4096, blocks)
    assert ql.select_path(1) == PATH_GEMV
    assert ql.select_path(2) == PATH_GEMV
    assert ql.select_path(4) == PATH_GEMV
    assert ql.select_path(5) == PATH_DECODE_MFMA
    assert ql.select_path(64) == PATH_DECODE_MFMA
    big = QuantLinear.from_blocks(Q4_0, 16, 11008, _case(Q4_0, 1, 16, 11008, seed=1)[0])
    # 344 blocks per row: the x digits fit the registers at m = 1, and at m = 2 with k
    # split over wave pairs; not at m = 3
    assert big.select_path(1) == PATH_GEMV and big.select_path(2) == PATH_GEMV
    assert big.select_path(3) == PATH_DECODE_MFMA
    assert ql.select_path(65) == PATH_PREFILL_MFMA


# ---- BASELINE shapes -----------------------------------------------------------------------

@pytest.mark.parametrize("qtype,k,n", [(Q8_0, 2048, 5632), (Q4_0, 4096, 12288),
                                       (Q4_0, 4096, 4096), (Q4_0, 4096, 11008),
                                       (Q4_0, 11008, 4096)])
def test_baseline_decode_shapes_m1(qtype, k, n):
    blocks, x = _case(qtype, 1, n, k, seed=k + n)
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    y = _run(ql, x, PATH_AUTO)
    assert oracle.normwise_error(y, oracle.qmatmul_f64(qtype, blocks, x, n, k)) < 1e-4
    # size-independent properties: power-of-two scaling and negation are exact
    assert np.array_equal(_run(ql, x * np.float32(4.0), PATH_AUTO), 4.0 * y)
    assert np.array_equal(_run(ql, -x, PATH_AUTO), -y)


@pytest.mark.parametrize("qtype,k,n", [(Q4_0, 4096, 5000), (Q8_0, 2048, 5632),
                                       (Q8_0, 1024, 8191), (Q4_0, 11008, 2049)])
def test_gemv_partial_second_round(qtype, k, n):
    # more rows than waves, fewer than twice as many: the waves holding a second row
    # are numbered across the workgroups (every row still computed exactly once)
    blocks, x = _case(qtype, 1, n, k, seed=3 * n + k)
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    assert ql.select_path(1) == PATH_GEMV
    ref = oracle.qmatmul_f64(qtype, blocks, x, n, k)
    xd = _dev(x)
    print(f"gemv partial round qtype={qtype} k={k} n={n}", flush=True)
    y = ql.forward(xd).cpu().numpy()
    assert oracle.normwise_error(y, ref) < 1e-4
    # every row, not only on average: no row left out or written twice
    assert np.all(np.abs(y - ref) <= 1e-4 * np.abs(ref).max())
    y0 = oracle.normal(n, seed=n).reshape(1, n).astype(np.float32)
    ya = _dev(y0)
    ql.forward_add(xd, ya)
    assert np.array_equal(ya.cpu().numpy(), y0 + y)


@pytest.mark.parametrize("k,n", [(8224, 300), (11008, 4096), (12288, 2049), (14336, 4096),
                                 (16384, 300)])
def test_gemv_q8_0_one_token_deep_k(k, n):
    # Q8_0 at one token past k 8192 (five to eight blocks a lane): the k split over wave
    # pairs, three or four blocks a lane a half; every row against the oracle, and the add
    blocks, x = _case(Q8_0, 1, n, k, seed=k + 5 * n)
    ql = QuantLinear.from_blocks(Q8_0, n, k, blocks)
    assert ql.select_path(1) == PATH_GEMV
    ref = oracle.qmatmul_f64(Q8_0, blocks, x, n, k)
    xd = _dev(x)
    print(f"gemv q8_0 deep k={k} n={n}", flush=True)
    y = ql.forward(xd).cpu().numpy()
    assert np.all(np.abs(y - ref) <= 1e-4 * np.abs(ref).max())
    y0 = oracle.normal(n, seed=n + 1).reshape(1, n).astype(np.float32)
    ya = _dev(y0)
    ql.forward_add(xd, ya)
    assert np.array_equal(ya.cpu().numpy(), y0 + y)
    dec = ql.forward(xd, path=PATH_DECODE_MFMA).cpu().numpy()
    assert oracle.normwise_error(dec, ref) < 1e-3


@pytest.mark.parametrize("n", [393216, 393217])
def test_gemv_k_split_many_rows(n):
    # four tokens at k 4096 split k over wave pairs, each pair's row sums held in LDS
    # beside the x records: 393216 rows (192 a pair over 2048 pairs) fill the 64 KiB a
    # launch takes; one row more takes more workgroups than CUs.  The weight repeats 3001
    # distinct rows (a period no pair or wave count divides), so every row is checked.
    m, k, period = 4, 4096, 3001
    blocks, x = _case(Q4_0, m, period, k, seed=n)
    rows = _dev(np.frombuffer(blocks, np.uint8).reshape(period, -1))
    tiled = rows.repeat((n + period - 1) // period, 1)[:n].contiguous()
    ql = QuantLinear.from_device_blocks(Q4_0, n, k, tiled.view(-1))
    del rows, tiled
    assert ql.select_path(m) == PATH_GEMV
    ref = np.tile(oracle.qmatmul_f64(Q4_0, blocks, x, period, k),
                  (1, (n + period - 1) // period))[:, :n]
    xd = _dev(x)
    print(f"gemv k split rows n={n}", flush=True)
    y = ql.forward(xd).cpu().numpy()
    assert np.all(np.abs(y - ref) <= 1e-4 * np.abs(ref).max())
    y0 = oracle.normal(m * n, seed=5).reshape(m, n).astype(np.float32)
    ya = _dev(y0)
    ql.forward_add(xd, ya)
    assert np.array_equal(ya.cpu().numpy(), y0 + y)
    ql.close()


@pytest.mark.parametrize("m", [4, 16, 64])
@pytest.mark.parametrize("n", [4096, 14336])
def test_baseline_batched_decode(m, n):
    k = 4096
    blocks, x = _case(Q4_0, m, n, k, seed=m + n)
    y = _run(QuantLinear.from_blocks(Q4_0, n, k, blocks), x, PATH_AUTO)
    assert oracle.normwise_error(y, oracle.qmatmul_f64(Q4_0, blocks, x, n, k)) < 1e-3


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("m,k,n", [(512, 4096, 14336), (512, 14336, 4096),
                                   (2048, 4096, 14336), (2048, 14336, 4096)])
def test_baseline_prefill_rows_sampled(qtype, m, k, n):
    # every BASELINE prefill workload at full size; the f64 oracle checks a sample of
    # rows (both ends of the first and last tiles, tile seams), plus linearity
    blocks, x = _case(qtype, m, n, k, seed=m + k)
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    y = _run(ql, x, PATH_AUTO)
    rows = np.array(sorted({0, 1, 127, 128, 255, 256, m // 2 + 3, m - 129, m - 128, m - 1}))
    ref = oracle.qmatmul_f64(qtype, blocks, x[rows], n, k)
    assert oracle.normwise_error(y[rows], ref) < 1e-3
    xd = _dev(x)
    y2 = ql.forward(xd * 2.0)
    torch.cuda.synchronize()
    # scaling x by 2 leaves the f16 operands unchanged (each row's power-of-two
    # scale absorbs it): outputs scale exactly, also where the k range is split
    # (k = 14336 at m = 512: the slices' sums are added in a fixed order)
    assert np.array_equal(y2.cpu().numpy(), 2.0 * y)


# The Llama-2-7B stack of the full-stack workload at batch 1 and 16: QKV, the
# fused gate_up (22016 = 2 x 11008 rows), down, and the Q8_0 lm_head through
# lm_head_forward (llama.rs:396-405).  Every launch shape of that workload.
@pytest.mark.parametrize("m", [1, 16])
@pytest.mark.parametrize("qtype,k,n", [(Q4_0, 4096, 12288), (Q4_0, 4096, 4096),
                                       (Q4_0, 4096, 22016), (Q4_0, 11008, 4096),
                                       (Q8_0, 4096, 32000)])
def test_baseline_stack_shapes(qtype, k, n, m):
    from unillm_amd import lm_head_forward

    blocks, x = _case(qtype, m, n, k, seed=3 * k + n + m)
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    xd = _dev(x)
    y = (lm_head_forward(ql, xd) if n == 32000 else ql.forward(xd)).cpu().numpy()
    ref = oracle.qmatmul_f64(qtype, blocks, x, n, k)
    assert oracle.normwise_error(y, ref) < (1e-4 if m == 1 else 1e-3)


@pytest.mark.parametrize("m", [1, 16])
def test_baseline_gate_up_swiglu(m):
    # the fused [gate; up] handle of the full-stack workload (4096 -> 2 x 11008) with
    # its SwiGLU epilogue: silu(g) u, candle silu(v) = v / (1 + e^-v)
    # (tensor_core.rs:1385-1396, applied at llama.rs:1283)
    k, I = 4096, 11008
    blocks, x = _case(Q4_0, m, 2 * I, k, seed=77 + m)
    ql = QuantLinear.from_blocks(Q4_0, 2 * I, k, blocks)
    act = ql.forward_swiglu(_dev(x)).cpu().numpy()
    gu = oracle.qmatmul_f64(Q4_0, blocks, x, 2 * I, k).astype(np.float64)
    g, u = gu[:, :I], gu[:, I:]
    ref = g / (1.0 + np.exp(-g)) * u
    assert act.shape == (m, I)
    assert oracle.normwise_error(act, ref) < 1e-3


def test_lm_head_error_text():
    from unillm_amd import lm_head_forward

    blocks, _ = _case(Q8_0, 1, 64, 128, seed=5)
    ql = QuantLinear.from_blocks(Q8_0, 64, 128, blocks)
    with pytest.raises(RuntimeError, match="^QMatMul lm_head forward failed: input last dim 64"):
        lm_head_forward(ql, torch.zeros(2, 64, device="cuda"))


@pytest.mark.parametrize("qtype,m,k,n", [(Q4_0, 2048, 4096, 14336), (Q8_0, 1100, 4128, 14000),
                                         (Q4_0, 1200, 4128, 14000), (Q4_0, 768, 4096, 14336),
                                         (Q8_0, 1100, 4096, 11008), (Q4_0, 300, 4096, 22016),
                                         (Q4_0, 1100, 4096, 14336)])
def test_prefill_large_tiles(qtype, m, k, n):
    # tiles unsplit: 256 rows, one a CU or more (m2048, m1200), or one round of them
    # against two of 128-row tiles (m768, m1100 at k4096 n11008, m300); 128 rows
    # where they take as many rounds as 256-row ones (m1100 at n14000 and n14336).
    # Ragged m and n, odd blocks per row.
    blocks, x = _case(qtype, m, n, k, seed=m + n + k)
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    y = _run(ql, x, PATH_AUTO)
    rows = np.unique(np.minimum([0, 1, 255, 256, 1023, m - 77, m - 1], m - 1))
    ref = oracle.qmatmul_f64(qtype, blocks, x[rows], n, k)
    assert oracle.normwise_error(y[rows], ref) < 1e-3
    y2 = ql.forward(_dev(x) * 2.0)
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy(), 2.0 * y)  # enough tiles: no k split


@pytest.mark.parametrize("qtype,m,k,n", [(Q4_0, 65, 11008, 4096), (Q8_0, 100, 14336, 4096),
                                         (Q4_0, 768, 14336, 4096), (Q8_0, 1100, 14336, 4096),
                                         (Q4_0, 500, 11008, 4096)])
def test_prefill_short_deep_split(qtype, m, k, n):
    # a short, deep product: 16 tiles of 128 rows, the k steps split over up to 16
    # workgroups a tile; or (m > 256) 256-row tiles filling at most half the CUs,
    # the k steps split over up to CUs / tiles workgroups (m768: 48 tiles in 5
    # slices, m1100: 80 in 3, m500: 32 in 8).  The slices' sums add in slice order.
    blocks, x = _case(qtype, m, n, k, seed=m + k)
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    y = _run(ql, x, PATH_PREFILL_MFMA)
    rows = np.unique([0, 1, min(255, m - 1), min(256, m - 1), m // 2, m - 1])
    ref = oracle.qmatmul_f64(qtype, blocks, x[rows], n, k)
    assert oracle.normwise_error(y[rows], ref) < 1e-3
    xd = _dev(x)
    y2 = ql.forward(xd * 2.0, path=PATH_PREFILL_MFMA)
    torch.cuda.synchronize()
    assert np.array_equal(y2.cpu().numpy(), 2.0 * y)  # scaling exact, split or not
    y3 = ql.forward(xd, path=PATH_PREFILL_MFMA)
    torch.cuda.synchronize()
    assert np.array_equal(y3.cpu().numpy(), y)  # repeatable bit for bit


@pytest.mark.parametrize("qtype,m,k,path", [(Q4_0, 96, 1024, PATH_PREFILL_MFMA),
                                             (Q8_0, 96, 1024, PATH_PREFILL_MFMA),
                                             (Q4_0, 5, 4096, PATH_DECODE_MFMA),
                                             (Q4_0, 16, 4096, PATH_DECODE_MFMA),
                                             (Q8_0, 16, 11008, PATH_DECODE_MFMA),
                                             (Q4_0, 64, 4096, PATH_DECODE_MFMA),
                                             (Q4_0, 3, 11008, PATH_DECODE_MFMA)])
def test_rows_of_any_magnitude(qtype, m, k, path):
    # f16 operands with a power-of-two scale per row of x (prefill) or per row and k
    # slice (batched decode): rows far beyond the f16 range (|x| ~ 1e6 > 65504), rows
    # deep in its subnormals (~1e-7), an all-zero row and unit rows side by side, each
    # as accurate as a unit row alone.  (Q4_0, 3, 11008): the down projection at m = 3,
    # which auto-routes here (past the GEMV's k at that m)
    n = 256
    blocks, x = _case(qtype, m, n, k, seed=91 + m)
    scale = np.ones(m, np.float32)
    scale[0::4], scale[1::4] = 1e6, 1e-7
    zero = 2 if m > 2 else None
    if zero is not None:
        scale[zero] = 0.0
    xs = (x * scale[:, None]).astype(np.float32)
    ql = QuantLinear.from_blocks(qtype, n, k, blocks)
    if path == PATH_DECODE_MFMA and m <= 4:
        assert ql.select_path(m) == PATH_DECODE_MFMA
    y = _run(ql, xs, path)
    ref = oracle.qmatmul_f64(qtype, blocks, xs, n, k)
    if zero is not None:
        assert np.all(y[zero] == 0.0)
    for r in range(m):
        if r != zero:
            assert oracle.normwise_error(y[r:r + 1], ref[r:r + 1]) < 1e-3, (r, scale[r])
    # within a row: a slice of huge values next to slices of small ones (each k slice
    # of the batched-decode split has its own scale)
    xm = x.copy()
    xm[:, : k // 4] *= 1e5
    y = _run(ql, xm, path)
    assert oracle.normwise_error(y, oracle.qmatmul_f64(qtype, blocks, xm, n, k)) < 1e-3


@pytest.mark.parametrize("m", [5, 16, 64])
def test_batched_decode_power_of_two_scaling_exact(m):
    # x and x times a power of two give the same f16 operands (per-slice scales):
    # outputs scale exactly, up to the order of the split k's atomic adds
    blocks, x = _case(Q4_0, m, 4096, 4096, seed=3 * m)
    ql = QuantLinear.from_blocks(Q4_0, 4096, 4096, blocks)
    y = _run(ql, x, PATH_DECODE_MFMA)
    y2 = _run(ql, x * np.float32(2.0 ** 40), PATH_DECODE_MFMA)
    assert oracle.normwise_error(y2, y * 2.0 ** 40) < 1e-6


# ---- edges -----------------------------------------------------------------------------------

def test_m_zero_is_noop():
    blocks, _ = _case(Q4_0, 1, 8, 64, seed=2)
    ql = QuantLinear.from_blocks(Q4_0, 8, 64, blocks)
    y = ql.forward(torch.empty(0, 64, device="cuda"))
    assert y.shape == (0, 8)


def test_3d_input_flattens_leading_dims():
    # tensor_core.rs:857-871: [B, T, K] is treated as [B*T, K]
    blocks, x = _case(Q4_0, 6, 40, 128, seed=4)
    ql = QuantLinear.from_blocks(Q4_0, 40, 128, blocks)
    y = ql.forward(_dev(x).reshape(2, 3, 128))
    torch.cuda.synchronize()
    assert y.shape == (2, 3, 40)
    ref = oracle.qmatmul_f64(Q4_0, blocks, x, 40, 128).reshape(2, 3, 40)
    assert oracle.normwise_error(y.cpu().numpy(), ref) < 1e-3


def test_forward_argument_errors():
    blocks, _ = _case(Q4_0, 1, 8, 64, seed=2)
    ql = QuantLinear.from_blocks(Q4_0, 8, 64, blocks)
    with pytest.raises(RuntimeError, match="QMatMul forward failed"):
        ql.forward(torch.zeros(1, 32, device="cuda"))
    with pytest.raises(RuntimeError, match="QMatMul forward failed"):
        ql.forward(torch.zeros(64, device="cuda"))
    with pytest.raises(RuntimeError, match="QMatMul forward failed"):
        ql.forward(torch.zeros(1, 64, device="cuda", dtype=torch.float16))
    with pytest.raises(HipError, match="m <= 4"):
        ql.forward(torch.zeros(5, 64, device="cuda"), path=PATH_GEMV)


@pytest.mark.parametrize("m,path", [(1, PATH_GEMV), (3, PATH_GEMV), (16, PATH_DECODE_MFMA),
                                    (130, PATH_PREFILL_MFMA)])
def test_x_on_4_byte_boundary(m, path):
    # candle takes any contiguous f32 tensor: x 4 bytes past a 16-byte boundary is
    # copied to an aligned buffer first, and gives the aligned call's result
    k, n = 1024, 256
    blocks, x = _case(Q4_0, m, n, k, seed=31 + m)
    ql = QuantLinear.from_blocks(Q4_0, n, k, blocks)
    buf = torch.zeros(m * k + 4, device="cuda")
    xm = buf[1:1 + m * k].view(m, k)
    assert xm.data_ptr() % 16 == 4
    xm.copy_(_dev(x))
    a = ql.forward(_dev(x), path=path).cpu().numpy()
    b = ql.forward(xm, path=path).cpu().numpy()
    if path != PATH_DECODE_MFMA:  # one fixed order of every sum
        assert np.array_equal(a, b)
    else:  # batched decode's split k: f32 atomics in any order
        assert oracle.normwise_error(b, a) < 1e-6
    assert oracle.normwise_error(b, oracle.qmatmul_f64(Q4_0, blocks, x, n, k)) < 1e-3


def test_batched_decode_back_to_back_calls_on_one_stream():
    # Batched decode at m <= 16 runs in one launch: k slice 0 of each row group zeroes
    # y's tile and raises a flag, the other slices add after it, and the last slice
    # resets the flag for the next launch.  Calls of different shapes, widths and
    # qtypes issued back to back on one stream (no synchronisation between them) must
    # each match the oracle; a stale flag would let a slice add onto y's old contents.
    cases = [(Q4_0, 9, 4096, 2048), (Q8_0, 16, 1000, 4096), (Q4_0, 5, 12288, 4096),
             (Q4_0, 16, 300, 11008), (Q8_0, 7, 4096, 1024), (Q4_0, 16, 4096, 2048)]
    runs = []
    for i, (qtype, m, n, k) in enumerate(cases):
        blocks, x = _case(qtype, m, n, k, seed=300 + i)
        ql = QuantLinear.from_blocks(qtype, n, k, blocks)
        assert ql.select_path(m) == PATH_DECODE_MFMA
        runs.append((qtype, m, n, k, blocks, x, ql, _dev(x)))
    outs = []
    for rep in range(3):
        ys = [torch.full((m, n), float("nan"), device="cuda") for _, m, n, *_ in runs]
        for (qtype, m, n, k, blocks, x, ql, xd), y in zip(runs, ys):
            ql.forward(xd, out=y)
        torch.cuda.synchronize()
        outs.append([y.cpu().numpy() for y in ys])
    for i, (qtype, m, n, k, blocks, x, ql, xd) in enumerate(runs):
        ref = oracle.qmatmul_f64(qtype, blocks, x, n, k)
        assert oracle.normwise_error(outs[0][i], ref) < 1e-3, cases[i]
        for rep in (1, 2):  # the adds' order may vary: f32 rounding, not bitwise
            assert oracle.normwise_error(outs[rep][i], outs[0][i]) < 1e-6, (cases[i], rep)


def test_batched_decode_grid_larger_than_the_device():
    # 300 row groups, k split in 2 (16 chunks of 128, at most 8 a slice): 600
    # workgroups, more than run at once (two a CU), so the call takes the two
    # launches (y zeroed by the first) instead of the one-launch kernel
    m, n, k = 16, 38400, 2048
    blocks, x = _case(Q4_0, m, n, k, seed=77)
    ql = QuantLinear.from_blocks(Q4_0, n, k, blocks)
    y = _run(ql, x, PATH_DECODE_MFMA)
    assert oracle.normwise_error(y, oracle.qmatmul_f64(Q4_0, blocks, x, n, k)) < 1e-3


def test_repeat_calls_deterministic():
    # GEMV (m <= 4) and prefill compute every output in one fixed order: bitwise
    # repeatable, also where the prefill splits k over workgroups (m = 130 here: 32
    # tiles; the slices' sums are added in slice order).  Batched decode splits k
    # over workgroups whose partial sums meet in y by f32 atomic adds, so the order
    # of those few adds (at most 8) can vary between calls: repeatable to f32
    # rounding, not bitwise.
    for m, exact in ((1, True), (2048, True), (130, True), (16, False), (64, False)):
        blocks, x = _case(Q4_0, m, 4096, 4096, seed=9)
        ql = QuantLinear.from_blocks(Q4_0, 4096, 4096, blocks)
        xd = _dev(x)
        a = ql.forward(xd).cpu().numpy()
        for _ in range(3):
            b = ql.forward(xd).cpu().numpy()
            if exact:
                assert np.array_equal(b, a), m
            else:
                assert oracle.normwise_error(b, a) < 1e-6, m
