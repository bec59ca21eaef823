"""unillm_amd -- MI355X (gfx950) device for unillm's quantized linear layer.

The product is libunillm_hip.so (HIP kernels behind the C ABI declared in
include/unillm_hip.h).  This package builds it (``unillm_amd.build``), binds
it with ctypes (``unillm_amd._capi``) and mirrors the reference's call
surface for this path (``QuantLinear``, the `Arc<QMatMul>` of
crates/runtime/src/model_core.rs:134).
"""
from ._capi import (BF16, BLOCK_BYTES, BLOCK_ELEMS, ERR_HIP, ERR_INVALID_ARG, ERR_UNSUPPORTED, F16, F32,
                    OK, PATH_AUTO, PATH_DECODE_MFMA, PATH_DENSE, PATH_GEMV, PATH_PREFILL_MFMA, QK,
                    Q4_0, Q4_K, Q5_0, Q5_K, Q6_K, Q8_0, HipError)

__all__ = [
    "BF16", "BLOCK_BYTES", "BLOCK_ELEMS", "ERR_HIP", "ERR_INVALID_ARG", "ERR_UNSUPPORTED", "F16", "F32",
    "OK", "PATH_AUTO", "PATH_DECODE_MFMA", "PATH_DENSE", "PATH_GEMV", "PATH_PREFILL_MFMA", "QK",
    "Q4_0", "Q4_K", "Q5_0", "Q5_K", "Q6_K", "Q8_0",
    "HipError",
    "QuantLinear", "quantize_blocks", "lm_head_forward", "KvCache",
]


def __getattr__(name):
    # QuantLinear needs torch; import it lazily so the ABI binding loads without it.
    if name in ("QuantLinear", "quantize_blocks", "lm_head_forward"):
        from . import quant_linear
        return getattr(quant_linear, name)
    if name == "KvCache":
        from . import attention
        return attention.KvCache
    raise AttributeError(name)
