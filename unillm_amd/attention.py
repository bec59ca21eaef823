"""KvCache: one decoder layer's KV cache on the device, and its decode attention.

Mirrors LayerKVCache (crates/runtime/src/kv_cache.rs:28-80: with_capacity,
seq_len, clear, append) and the attention of LlamaAttention::forward_with_cache
after the projections (crates/runtime/src/models_v2/llama.rs:1044-1150).  Torch
supplies device memory and the current stream; the arithmetic runs in
libunillm_hip.so.
"""
from __future__ import annotations

import ctypes

import torch

from . import _capi
from ._capi import HipError


def _stream_ptr(stream: torch.cuda.Stream | None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


class KvCache:
    """K and V of n_kv_heads heads, max_seq positions of head_dim f32 each."""

    def __init__(self, n_kv_heads: int, head_dim: int, max_seq: int, rope_theta: float = 10000.0):
        h = ctypes.c_void_p()
        _capi.check(_capi.lib().unillm_hip_kv_cache_create(n_kv_heads, head_dim, max_seq,
                                                           float(rope_theta), ctypes.byref(h)))
        self._h = h
        self.n_kv_heads, self.head_dim, self.max_seq = n_kv_heads, head_dim, max_seq

    @property
    def seq_len(self) -> int:
        n = ctypes.c_int64()
        _capi.check(_capi.lib().unillm_hip_kv_cache_length(self._h, ctypes.byref(n)))
        return n.value

    def clear(self) -> None:
        _capi.check(_capi.lib().unillm_hip_kv_cache_clear(self._h))

    def reserve(self, m: int, n_heads: int, stream: torch.cuda.Stream | None = None) -> None:
        """Grow the stream's attention workspace for calls of up to m tokens, so they
        can be captured into a HIP graph."""
        _capi.check(_capi.lib().unillm_hip_attention_reserve(self._h, m, n_heads,
                                                             _stream_ptr(stream)))

    def truncate(self, length: int) -> None:
        """Keep the first `length` positions (<= seq_len): a rolled-back step."""
        _capi.check(_capi.lib().unillm_hip_kv_cache_truncate(self._h, length))

    def attention(self, qkv: torch.Tensor, n_heads: int, out: torch.Tensor | None = None,
                  stream: torch.cuda.Stream | None = None) -> torch.Tensor:
        """qkv [m, (n_heads + 2 n_kv_heads) head_dim] (the fused projections of m new
        tokens) -> out [m, n_heads head_dim]; appends k, v (seq_len grows by m)."""
        width = (n_heads + 2 * self.n_kv_heads) * self.head_dim
        if (qkv.dtype != torch.float32 or not qkv.is_cuda or not qkv.is_contiguous()
                or qkv.dim() != 2 or qkv.shape[1] != width):
            raise RuntimeError(f"attention: qkv must be a contiguous f32 [m, {width}] device tensor")
        m = qkv.shape[0]
        if out is None:
            out = torch.empty(m, n_heads * self.head_dim, dtype=torch.float32, device=qkv.device)
        rc = _capi.lib().unillm_hip_attention_decode(self._h, qkv.data_ptr(), m, n_heads,
                                                     out.data_ptr(), _stream_ptr(stream))
        if rc != _capi.OK:
            raise HipError(rc, _capi.last_error())
        return out

    def close(self) -> None:
        if self._h is not None and self._h.value:
            _capi.lib().unillm_hip_kv_cache_destroy(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
