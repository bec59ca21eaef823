"""ctypes binding of include/unillm_hip.h (libunillm_hip.so, built in-tree).

Loading fails loudly: there is no CPU fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libunillm_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "unillm_hip.h")

Q4_0 = 2
Q8_0 = 8
Q4_K = 12
Q5_0 = 6
Q5_K = 13
Q6_K = 14
# dense projection weights (candle's dequantized f32 QMatMul): f32 rows on the device
F32 = 0
F16 = 1
BF16 = 30
DENSE = (F32, F16, BF16)
QK = 32
# GGUF block geometry: weights per block and bytes per block (a dense element is a
# block of one)
BLOCK_ELEMS = {Q4_0: 32, Q5_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256, F32: 1, F16: 1, BF16: 1}
BLOCK_BYTES = {Q4_0: 18, Q5_0: 22, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210, F32: 4, F16: 2, BF16: 2}

PATH_AUTO = 0
PATH_GEMV = 1
PATH_DECODE_MFMA = 2
PATH_PREFILL_MFMA = 3
PATH_DENSE = 4

OK = 0
ERR_INVALID_ARG = -1
ERR_UNSUPPORTED = -2
ERR_HIP = -3
ERR_OUT_OF_MEMORY = -4
ERR_NOT_INITIALIZED = -5


class HipError(RuntimeError):
    """A negative status from the C ABI, with unillm_hip_last_error()'s text."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_lib = None

P = ctypes.c_void_p
I64 = ctypes.c_int64
SIGNATURES = {
    "unillm_hip_init": ([ctypes.c_int], ctypes.c_int),
    "unillm_hip_last_error": ([], ctypes.c_char_p),
    "unillm_hip_qweight_create": (
        [ctypes.c_int, I64, I64, P, ctypes.c_size_t, ctypes.c_int, ctypes.POINTER(P)], ctypes.c_int),
    "unillm_hip_qweight_create_device": (
        [ctypes.c_int, I64, I64, P, ctypes.c_size_t, ctypes.c_int, P, ctypes.POINTER(P)],
        ctypes.c_int),
    "unillm_hip_qweight_destroy": ([P], ctypes.c_int),
    "unillm_hip_qweight_info": (
        [P, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(I64), ctypes.POINTER(I64),
         ctypes.POINTER(ctypes.c_size_t)], ctypes.c_int),
    "unillm_hip_qmatmul": ([P, P, I64, P, P], ctypes.c_int),
    "unillm_hip_qmatmul_path": ([P, P, I64, P, ctypes.c_int, P], ctypes.c_int),
    "unillm_hip_qmatmul_noalloc": ([P, P, I64, P, P], ctypes.c_int),
    "unillm_hip_qmatmul_add": ([P, P, I64, P, P], ctypes.c_int),
    "unillm_hip_qmatmul_swiglu": ([P, P, I64, P, P], ctypes.c_int),
    "unillm_hip_qmatmul_norm": ([P, P, P, P, ctypes.c_float, I64, P, P], ctypes.c_int),
    "unillm_hip_kv_cache_create": ([I64, I64, I64, ctypes.c_float, P], ctypes.c_int),
    "unillm_hip_kv_cache_destroy": ([P], ctypes.c_int),
    "unillm_hip_kv_cache_length": ([P, P], ctypes.c_int),
    "unillm_hip_kv_cache_clear": ([P], ctypes.c_int),
    "unillm_hip_kv_cache_truncate": ([P, I64], ctypes.c_int),
    "unillm_hip_attention_decode": ([P, P, I64, I64, P, P], ctypes.c_int),
    "unillm_hip_qmatmul_norm_swiglu": ([P, P, P, P, ctypes.c_float, I64, P, P], ctypes.c_int),
    "unillm_hip_select_path": ([P, I64], ctypes.c_int),
    "unillm_hip_qmatmul_reserve": ([P, I64, ctypes.c_int, P], ctypes.c_int),
    "unillm_hip_attention_reserve": ([P, I64, I64, P], ctypes.c_int),
    "unillm_hip_dequant": ([P, P, P], ctypes.c_int),
    "unillm_hip_quantize": ([ctypes.c_int, P, I64, I64, P, P], ctypes.c_int),
    "unillm_hip_malloc": ([ctypes.POINTER(P), ctypes.c_size_t], ctypes.c_int),
    "unillm_hip_free": ([P], ctypes.c_int),
    "unillm_hip_memcpy_htod": ([P, P, ctypes.c_size_t], ctypes.c_int),
    "unillm_hip_memcpy_dtoh": ([P, P, ctypes.c_size_t], ctypes.c_int),
    "unillm_hip_synchronize": ([], ctypes.c_int),
    "unillm_hip_stream_create": ([ctypes.POINTER(P)], ctypes.c_int),
    "unillm_hip_stream_destroy": ([P], ctypes.c_int),
    "unillm_hip_stream_synchronize": ([P], ctypes.c_int),
    "unillm_hip_graph_begin": ([P], ctypes.c_int),
    "unillm_hip_graph_end": ([P, ctypes.POINTER(P)], ctypes.c_int),
    "unillm_hip_graph_launch": ([P, P], ctypes.c_int),
    "unillm_hip_graph_destroy": ([P], ctypes.c_int),
}


def header_symbols() -> list[str]:
    """Every function the public header declares."""
    with open(HEADER) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(unillm_hip_\w+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m unillm_amd.build` "
                "(the HIP library is required; there is no CPU fallback)")
        l = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = res
        _lib = l
    return _lib


def last_error() -> str:
    return (lib().unillm_hip_last_error() or b"").decode()


def check(status: int) -> None:
    if status != OK:
        raise HipError(status, last_error())
