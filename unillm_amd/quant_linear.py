"""QuantLinear: a device-resident GGUF Q4_0 / Q5_0 / Q8_0 / Q4_K / Q5_K / Q6_K weight and its
forward.

It takes the slot that `Arc<QMatMul>` holds in unillm's
`ModelWeights.quantized_tensors` (crates/runtime/src/model_core.rs:134) and
mirrors the call the model makes on it:

    qmatmul.forward(&input)   -> QuantLinear.forward(x)
      (crates/runtime/src/models_v2/llama.rs:1184-1195, 1325-1336, 396-405)

with candle's argument rules (f32, contiguous, rank >= 2, last dim == k,
output [..., n]) and its error text ("QMatMul forward failed: ...").  Torch is
used only for device memory and the current stream; all arithmetic runs in
libunillm_hip.so.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _capi
from ._capi import (BF16, BLOCK_BYTES, BLOCK_ELEMS, F16, F32, QK, Q4_0, Q4_K, Q5_0, Q5_K, Q6_K,
                    Q8_0, HipError)


def _stream_ptr(stream: torch.cuda.Stream | None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


class QuantLinear:
    """One quantized projection (W is [n, k] = [out_features, in_features])."""

    def __init__(self, handle: int, qtype: int, n: int, k: int):
        self._h = ctypes.c_void_p(handle)
        self.qtype = qtype
        self.n = n
        self.k = k

    # ---- construction (WeightLoaderCore's QMatMul::from_arc, weight_loader_core.rs:569)
    @classmethod
    def from_blocks(cls, qtype: int, n: int, k: int, blocks) -> "QuantLinear":
        """From GGUF block bytes in host memory (n * k/32 blocks of 18 / 22 / 34 B, or
        n * k/256 blocks of 144 / 176 / 210 B for Q4_K / Q5_K / Q6_K; a dense F32 / F16 / BF16
        tensor's n * k elements)."""
        buf = np.ascontiguousarray(np.frombuffer(memoryview(blocks), dtype=np.uint8))
        h = ctypes.c_void_p()
        _capi.check(_capi.lib().unillm_hip_qweight_create(
            qtype, n, k, buf.ctypes.data, buf.nbytes, 0, ctypes.byref(h)))
        return cls(h.value, qtype, n, k)

    @classmethod
    def from_device_blocks(cls, qtype: int, n: int, k: int, blocks: torch.Tensor,
                           stream: torch.cuda.Stream | None = None) -> "QuantLinear":
        """From GGUF block bytes already on the device (a uint8 CUDA tensor)."""
        if blocks.dtype != torch.uint8 or not blocks.is_cuda or not blocks.is_contiguous():
            raise ValueError("blocks must be a contiguous uint8 device tensor")
        h = ctypes.c_void_p()
        _capi.check(_capi.lib().unillm_hip_qweight_create_device(
            qtype, n, k, blocks.data_ptr(), blocks.numel(), 0, _stream_ptr(stream),
            ctypes.byref(h)))
        return cls(h.value, qtype, n, k)

    @classmethod
    def from_dense(cls, w: torch.Tensor,
                   stream: torch.cuda.Stream | None = None) -> "QuantLinear":
        """A dense [n, k] device tensor (float32, float16 or bfloat16), kept as f32 rows
        and multiplied in f32, as candle's QMatMul keeps a dense GGUF tensor."""
        qtype = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}.get(w.dtype)
        if qtype is None or w.dim() != 2 or not w.is_cuda:
            raise ValueError("w must be a 2-D float32 / float16 / bfloat16 device tensor")
        w = w.contiguous()
        return cls.from_device_blocks(qtype, w.shape[0], w.shape[1],
                                      w.view(-1).view(torch.uint8), stream)

    @classmethod
    def quantize(cls, qtype: int, w: torch.Tensor,
                 stream: torch.cuda.Stream | None = None) -> "QuantLinear":
        """Quantize an f32 [n, k] device tensor with the GGML quantizer, then load it."""
        blocks = quantize_blocks(qtype, w, stream)
        return cls.from_device_blocks(qtype, w.shape[0], w.shape[1], blocks, stream)

    # ---- queries -----------------------------------------------------------------------
    @property
    def shape(self) -> tuple[int, int]:
        return (self.n, self.k)

    @property
    def device_bytes(self) -> int:
        nb = ctypes.c_size_t()
        _capi.check(_capi.lib().unillm_hip_qweight_info(self._h, None, None, None,
                                                        ctypes.byref(nb)))
        return nb.value

    @property
    def gguf_bytes(self) -> int:
        return self.n * (self.k // BLOCK_ELEMS[self.qtype]) * BLOCK_BYTES[self.qtype]

    def select_path(self, m: int) -> int:
        return _capi.lib().unillm_hip_select_path(self._h, m)

    def reserve(self, m: int, swiglu: bool = False,
                stream: torch.cuda.Stream | None = None) -> None:
        """Grow the stream's workspace for calls of up to m rows, so they can be
        captured into a HIP graph (a capture cannot allocate)."""
        _capi.check(_capi.lib().unillm_hip_qmatmul_reserve(self._h, m, int(swiglu),
                                                           _stream_ptr(stream)))

    # ---- compute -------------------------------------------------------------------------
    def _check_input(self, x: torch.Tensor) -> int:
        if x.dtype != torch.float32:
            raise RuntimeError(f"QMatMul forward failed: expected f32 input, got {x.dtype}")
        if x.dim() < 2:
            raise RuntimeError(f"QMatMul forward failed: rank {x.dim()} input, need rank >= 2")
        if x.shape[-1] != self.k:
            raise RuntimeError(
                f"QMatMul forward failed: input last dim {x.shape[-1]} != k {self.k}")
        if not x.is_cuda:
            raise RuntimeError("QMatMul forward failed: input is not on the HIP device")
        if not x.is_contiguous():
            raise RuntimeError("QMatMul forward failed: input is not contiguous")
        return x.numel() // self.k

    def _out(self, x: torch.Tensor, m: int, n: int, out: torch.Tensor | None) -> torch.Tensor:
        if out is None:
            return torch.empty(*x.shape[:-1], n, dtype=torch.float32, device=x.device)
        if out.dtype != torch.float32 or not out.is_contiguous() or out.numel() != m * n:
            raise RuntimeError("QMatMul forward failed: bad output tensor")
        return out

    def forward(self, x: torch.Tensor, path: int = _capi.PATH_AUTO,
                out: torch.Tensor | None = None,
                stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """y[..., n] = x[..., k] . dequant(W)^T (QMatMul::forward)."""
        m = self._check_input(x)
        out = self._out(x, m, self.n, out)
        rc = _capi.lib().unillm_hip_qmatmul_path(self._h, x.data_ptr(), m, out.data_ptr(), path,
                                                 _stream_ptr(stream))
        if rc != _capi.OK:
            raise HipError(rc, _capi.last_error())
        return out

    def forward_add(self, x: torch.Tensor, residual: torch.Tensor,
                    stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """residual[..., n] += x[..., k] . dequant(W)^T in place (the decoder layer's
        residual add fused into the projection, llama.rs:668, 677); returns residual."""
        m = self._check_input(x)
        self._out(x, m, self.n, residual)
        rc = _capi.lib().unillm_hip_qmatmul_add(self._h, x.data_ptr(), m, residual.data_ptr(),
                                                _stream_ptr(stream))
        if rc != _capi.OK:
            raise HipError(rc, _capi.last_error())
        return residual

    def forward_swiglu(self, x: torch.Tensor, out: torch.Tensor | None = None,
                       stream: torch.cuda.Stream | None = None,
                       norm: tuple | None = None) -> torch.Tensor:
        """silu(x G^T) * (x U^T) for a [gate; up] weight (n = 2 I): [..., I]
        (LlamaMLP's gate, up and fused_swiglu, llama.rs:1275-1283); with norm =
        (gamma, beta or None, eps), on the layer norm of x."""
        m = self._check_input(x)
        out = self._out(x, m, self.n // 2, out)
        if norm is None:
            rc = _capi.lib().unillm_hip_qmatmul_swiglu(self._h, x.data_ptr(), m, out.data_ptr(),
                                                       _stream_ptr(stream))
        else:
            g, b, eps = self._norm_args(norm)
            rc = _capi.lib().unillm_hip_qmatmul_norm_swiglu(
                self._h, x.data_ptr(), g, b, eps, m, out.data_ptr(), _stream_ptr(stream))
        if rc != _capi.OK:
            raise HipError(rc, _capi.last_error())
        return out

    def _norm_args(self, norm):
        gamma, beta, eps = norm
        for t in (gamma, beta):
            if t is not None and (t.dtype != torch.float32 or not t.is_cuda
                                  or not t.is_contiguous() or t.numel() != self.k):
                raise RuntimeError("QMatMul forward failed: norm weight / bias must be "
                                   "contiguous f32 [k] device tensors")
        return gamma.data_ptr(), (beta.data_ptr() if beta is not None else None), float(eps)

    def forward_norm(self, x: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor | None = None,
                     eps: float = 1e-6, out: torch.Tensor | None = None,
                     stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """LN(x) . dequant(W)^T with the reference's layer norm (tensor_core.rs:973-1008)
        fused into the matmul's x preparation."""
        m = self._check_input(x)
        out = self._out(x, m, self.n, out)
        g, b, e = self._norm_args((gamma, beta, eps))
        rc = _capi.lib().unillm_hip_qmatmul_norm(self._h, x.data_ptr(), g, b, e, m,
                                                 out.data_ptr(), _stream_ptr(stream))
        if rc != _capi.OK:
            raise HipError(rc, _capi.last_error())
        return out

    __call__ = forward

    def dequantize(self, stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """f32 [n, k], bit-exact with GGML's to_float (weight_loader_core.rs:579)."""
        out = torch.empty(self.n, self.k, dtype=torch.float32, device="cuda")
        _capi.check(_capi.lib().unillm_hip_dequant(self._h, out.data_ptr(), _stream_ptr(stream)))
        return out

    # ---- lifetime ------------------------------------------------------------------------
    def close(self) -> None:
        if self._h is not None and self._h.value:
            _capi.lib().unillm_hip_qweight_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __repr__(self) -> str:
        name = {Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K",
                F32: "F32", F16: "F16", BF16: "BF16"}.get(self.qtype, str(self.qtype))
        return f"QuantLinear({name}, n={self.n}, k={self.k})"


def lm_head_forward(lm_head: QuantLinear, hidden_states: torch.Tensor,
                    out: torch.Tensor | None = None,
                    stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """LlamaModelV2::lm_head_forward (crates/runtime/src/models_v2/llama.rs:396-405)
    with a quantized lm_head: logits = hidden . dequant(W)^T, errors worded as the
    reference words them ("QMatMul lm_head forward failed: ...")."""
    prefix = "QMatMul forward failed: "
    try:
        return lm_head.forward(hidden_states, out=out, stream=stream)
    except HipError as e:
        msg = str(e)
        raise HipError(e.status, "QMatMul lm_head forward failed: " +
                       (msg[len(prefix):] if msg.startswith(prefix) else msg)) from None
    except RuntimeError as e:
        msg = str(e)
        raise RuntimeError("QMatMul lm_head forward failed: " +
                           (msg[len(prefix):] if msg.startswith(prefix) else msg)) from None


def quantize_blocks(qtype: int, w: torch.Tensor,
                    stream: torch.cuda.Stream | None = None) -> torch.Tensor:
    """GGML quantizer on the device: f32 [n, k] -> uint8 GGUF block bytes."""
    if w.dtype != torch.float32 or not w.is_cuda or not w.is_contiguous() or w.dim() != 2:
        raise ValueError("w must be a contiguous f32 [n, k] device tensor")
    if qtype not in (Q4_0, Q8_0):
        raise ValueError("the device quantizer (GGML's reference quantizer) covers Q4_0 and Q8_0")
    n, k = w.shape
    if k % QK:
        raise ValueError(f"k = {k} is not a multiple of 32")
    out = torch.empty(n * (k // QK) * BLOCK_BYTES[qtype], dtype=torch.uint8, device=w.device)
    _capi.check(_capi.lib().unillm_hip_quantize(qtype, w.data_ptr(), n, k, out.data_ptr(),
                                                _stream_ptr(stream)))
    return out
