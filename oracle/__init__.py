"""CPU oracle for the quantized linear-layer path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed
CPU baseline.  The product (``unillm_amd``) never imports it.

It wraps ``oracle/liboracle.so`` (built from ``oracle/oracle.c`` by
``oracle/Makefile``) with numpy-friendly functions.  What each function
restates, and what pins it, is documented in ``oracle/oracle.h``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

Q4_0 = 2
Q8_0 = 8
Q4_K = 12
Q5_0 = 6
Q5_K = 13
Q6_K = 14
QK = 32
BLOCK_BYTES = {Q4_0: 18, Q5_0: 22, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}
BLOCK_ELEMS = {Q4_0: 32, Q5_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        l = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        l.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        l.oracle_f16_to_f32.restype = ctypes.c_float
        l.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        l.oracle_f32_to_f16.restype = ctypes.c_uint16
        l.oracle_quantize.argtypes = [ctypes.c_int, P, I64, I64, P]
        l.oracle_dequant.argtypes = [ctypes.c_int, P, I64, I64, P]
        l.oracle_qmatmul_f64.argtypes = [ctypes.c_int, P, P, I64, I64, I64, P, ctypes.c_int]
        l.oracle_candle_qmatmul.argtypes = [ctypes.c_int, P, P, I64, I64, I64, P, ctypes.c_int]
        l.oracle_attention_decode.argtypes = [P, I64, I64, I64, I64, ctypes.c_float, P, P, I64,
                                              I64, P]
        l.oracle_fill_normal.argtypes = [P, I64, ctypes.c_uint64, ctypes.c_double, ctypes.c_double]
        l.oracle_fill_normal.restype = None
        _lib = l
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def f16_to_f32(h: int) -> float:
    return lib().oracle_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return lib().oracle_f32_to_f16(f)


def normal(count: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    lib().oracle_fill_normal(_ptr(out), count, seed, mean, std)
    return out


def quantize(qtype: int, w: np.ndarray) -> np.ndarray:
    """f32 [n, k] -> GGUF block bytes (uint8 [n, k/32 * block_bytes])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    out = np.empty((n, (k // QK) * BLOCK_BYTES[qtype]), dtype=np.uint8)
    if lib().oracle_quantize(qtype, _ptr(w), n, k, _ptr(out)) != 0:
        raise ValueError(f"oracle_quantize rejected qtype={qtype} n={n} k={k}")
    return out


def dequant(qtype: int, blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    assert blocks.size == n * (k // BLOCK_ELEMS[qtype]) * BLOCK_BYTES[qtype]
    out = np.empty((n, k), dtype=np.float32)
    if lib().oracle_dequant(qtype, _ptr(blocks), n, k, _ptr(out)) != 0:
        raise ValueError("oracle_dequant rejected its arguments")
    return out


def qmatmul_f64(qtype: int, blocks: np.ndarray, x: np.ndarray, n: int, k: int,
                nthreads: int = 0) -> np.ndarray:
    """The parity oracle: x[m, k] . dequant(W)[n, k]^T accumulated in f64."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    m = x.shape[0]
    y = np.empty((m, n), dtype=np.float64)
    if lib().oracle_qmatmul_f64(qtype, _ptr(blocks), _ptr(x), m, n, k, _ptr(y), nthreads) != 0:
        raise ValueError("oracle_qmatmul_f64 rejected its arguments")
    return y


_timing = None


def _host_has_avx512() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            flags = next((l.split(":", 1)[1].split() for l in f if l.startswith("flags")), [])
    except OSError:
        return False
    return all(x in flags for x in ("avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"))


def timing_lib() -> tuple[ctypes.CDLL, str]:
    """The timing copy of the library for this host (bench.py's CPU baseline only):
    FMA contraction on, x86-64-v4 where the CPU has AVX-512, else v3; and its flags."""
    global _timing
    if _timing is None:
        v = "v4" if _host_has_avx512() else "v3"
        path = os.path.join(_HERE, f"liboracle_timing_{v}.so")
        if not os.path.exists(path):
            build()
        l = ctypes.CDLL(path)
        l.oracle_candle_qmatmul.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                                            ctypes.c_void_p, ctypes.c_int]
        l.oracle_candle_qmatmul.restype = ctypes.c_int
        _timing = (l, f"gcc -O3 -march=x86-64-{v} -ffp-contract=fast -fopenmp")
    return _timing


def candle_qmatmul(qtype: int, blocks: np.ndarray, x: np.ndarray, n: int, k: int,
                   nthreads: int = 0, timing: bool = False) -> np.ndarray:
    """candle CPU QMatMul semantics (Q8_0 activations, integer block dots).  timing:
    run the timing build (FMA contraction, the host's widest vectors) -- bench.py's CPU
    baseline; results agree with the checker's to f32 rounding."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    m = x.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    l = timing_lib()[0] if timing else lib()
    if l.oracle_candle_qmatmul(qtype, _ptr(blocks), _ptr(x), m, n, k, _ptr(y), nthreads) != 0:
        raise ValueError("oracle_candle_qmatmul rejected its arguments")
    return y


def normwise_error(y: np.ndarray, ref: np.ndarray) -> float:
    """max|y - r| / max|r|, the tolerance measure used by every parity test."""
    ref = np.asarray(ref, dtype=np.float64)
    denom = float(np.max(np.abs(ref))) if ref.size else 0.0
    err = float(np.max(np.abs(np.asarray(y, dtype=np.float64) - ref))) if ref.size else 0.0
    return err / denom if denom > 0 else err


def elementwise_error(y: np.ndarray, ref: np.ndarray, floor: float = 1e-3) -> float:
    """max relative error over elements with |r| > floor * max|r|."""
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    big = np.abs(ref) > floor * np.max(np.abs(ref))
    if not big.any():
        return 0.0
    d = np.abs(np.asarray(y, dtype=np.float64)[big] - ref[big]) / np.abs(ref[big])
    return float(d.max())


# ---- K-quant test data ---------------------------------------------------------------------
# GGML has no simple reference quantizer for Q4_K / Q5_K / Q6_K (quantize_row_q4_K_ref
# searches scales iteratively); the parity tests need valid blocks, not GGML's
# choice of them, so blocks are drawn directly: random codes and 6- / 8-bit
# scales under f16 super-block scales sized like N(0, 0.02) weights.

def pack_q4_k_scales(sc, m) -> np.ndarray:
    """GGML's packing of eight 6-bit scales and mins into scales[12], as
    quantize_row_q4_K_ref writes it (the inverse of get_scale_min_k4)."""
    out = np.zeros(12, np.uint8)
    for j in range(8):
        ls, lm = int(sc[j]), int(m[j])
        assert 0 <= ls < 64 and 0 <= lm < 64
        if j < 4:
            out[j] = ls
            out[j + 4] = lm
        else:
            out[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            out[j - 4] |= (ls >> 4) << 6
            out[j] |= (lm >> 4) << 6
    return out


def random_q4_k(n: int, k: int, seed: int) -> np.ndarray:
    """[n, k/256 * 144] valid Q4_K blocks, weights of roughly N(0, 0.02) size."""
    assert k % 256 == 0
    rng = np.random.default_rng(seed)
    nb = n * (k // 256)
    blk = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)  # scales[12] and qs: any bytes
    d = (np.abs(rng.normal(0, 1, nb)) * 4e-5 + 1e-5).astype(np.float16)
    dmin = (np.abs(rng.normal(0, 1, nb)) * 2e-4 + 1e-5).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return blk.reshape(n, -1)


def random_q5_k(n: int, k: int, seed: int) -> np.ndarray:
    """[n, k/256 * 176] valid Q5_K blocks, weights of roughly N(0, 0.02) size."""
    assert k % 256 == 0
    rng = np.random.default_rng(seed)
    nb = n * (k // 256)
    blk = rng.integers(0, 256, size=(nb, 176), dtype=np.uint8)  # scales, qh, qs: any bytes
    d = (np.abs(rng.normal(0, 1, nb)) * 2e-5 + 5e-6).astype(np.float16)
    dmin = (np.abs(rng.normal(0, 1, nb)) * 2e-4 + 1e-5).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return blk.reshape(n, -1)


def random_q5_0(n: int, k: int, seed: int) -> np.ndarray:
    """[n, k/32 * 22] valid Q5_0 blocks (random codes and fifth bits, f16 d sized like
    N(0, 0.02) weights)."""
    assert k % 32 == 0
    rng = np.random.default_rng(seed)
    nb = n * (k // 32)
    blk = rng.integers(0, 256, size=(nb, 22), dtype=np.uint8)
    d = (np.abs(rng.normal(0, 1, nb)) * 2e-3 + 1e-4).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    return blk.reshape(n, -1)


def random_q6_k(n: int, k: int, seed: int) -> np.ndarray:
    """[n, k/256 * 210] valid Q6_K blocks (signed 8-bit sub-block scales)."""
    assert k % 256 == 0
    rng = np.random.default_rng(seed)
    nb = n * (k // 256)
    blk = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)  # ql, qh: any bytes
    blk[:, 192:208] = rng.integers(-64, 128, size=(nb, 16)).astype(np.int8).view(np.uint8)
    d = (np.abs(rng.normal(0, 1, nb)) * 2e-5 + 5e-6).astype(np.float16)
    blk[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return blk.reshape(n, -1)


def attention_decode(qkv: np.ndarray, n_heads: int, n_kv_heads: int, head_dim: int,
                     rope_theta: float, k_cache: np.ndarray, v_cache: np.ndarray,
                     length: int) -> np.ndarray:
    """Decode attention with a KV cache (oracle.h): RoPE, append (k_cache / v_cache
    [KVH, max_seq, hd] f32, updated in place), causal softmax attention in f64.
    Returns out [m, H * hd] (f64)."""
    qkv = np.ascontiguousarray(qkv, dtype=np.float32)
    m = qkv.shape[0]
    assert k_cache.flags["C_CONTIGUOUS"] and v_cache.flags["C_CONTIGUOUS"]
    assert k_cache.dtype == np.float32 and v_cache.dtype == np.float32
    out = np.empty((m, n_heads * head_dim), dtype=np.float64)
    rc = lib().oracle_attention_decode(_ptr(qkv), m, n_heads, n_kv_heads, head_dim,
                                       float(rope_theta), _ptr(k_cache), _ptr(v_cache),
                                       k_cache.shape[1], length, _ptr(out))
    if rc != 0:
        raise ValueError("oracle_attention_decode rejected its arguments")
    return out
