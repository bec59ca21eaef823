"""Numpy float64 restatement of the attention in LlamaAttention::forward_with_cache.

TEST INFRASTRUCTURE ONLY: it pins ``oracle_attention_decode`` (oracle/oracle.c)
from the reference's own text, written independently of that C code and in
the reference's tensor form rather than as per-position loops.

It follows crates/runtime/src/models_v2/llama.rs step by step:

  * 2. reshape q / k / v to [heads, new_seq, hd]            (llama.rs:1054-1064)
  * 3. apply_rope_with_offset                               (llama.rs:827-883)
       inv_freq[i] = 1 / theta^((2 i) / hd), every factor in f32  (:839-841)
       angle[p, i] = f32(p + offset) * inv_freq[i], in f32         (:844-854)
       half-split rotation [x1 c - x2 s, x1 s + x2 c]              (:868-880)
  * 4. GQA expansion: kv head g serves query heads g*G .. g*G+G-1 (:1074-1088)
  * 5. cache append, then the full cached K, V                (:1091-1108)
  * 6. scores = q k^T * scale, scale = f32(1 / sqrt(f32(hd)))  (llama.rs:890, :1118)
  * 7. causal mask: -inf where key position > query position  (:1120-1137)
       softmax over the last dimension                         (:1139)
  * 8. weights @ v, 9. back to [new_seq, heads * hd]          (:1141-1148)

Precision: the reference computes in f32.  This restatement evaluates its
expressions in f64 except where the reference stores into its f32 KV cache
(rotated k and v are rounded to f32 there) and where it forms the RoPE angles
(f32, as above); cos / sin of those f32 angles are taken in f64.  The same
points are where ``oracle_attention_decode`` rounds, so the two agree to f64
rounding (~1e-15).  The reference's own f32 rounding of cos / sin and of the
products moves results by ~1e-7 relative, inside the 1e-4 bar of the device
tests.

``scale`` and ``exp`` are parameters only so that tests can plant a wrong
softmax temperature or base here, on the CPU, and show the comparison with the
oracle catches it.
"""
from __future__ import annotations

import numpy as np


def reference_scale(head_dim: int) -> float:
    """LlamaAttention::new: ``1.0 / (head_dim as f32).sqrt()`` in f32 (llama.rs:890)."""
    return float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))


def rope_with_offset(x: np.ndarray, head_dim: int, theta: float, offset: int) -> np.ndarray:
    """apply_rope_with_offset on one tensor x[heads, seq, hd] (float64 values)."""
    half = head_dim // 2
    expo = (2 * np.arange(half)).astype(np.float32) / np.float32(head_dim)
    # f32 powf as the platform libm gives it (correctly rounded at these arguments): the
    # f64 power rounded once to f32.  numpy's own float32 power is 1 ulp off at some of them.
    powf = np.power(np.float64(np.float32(theta)), expo.astype(np.float64)).astype(np.float32)
    inv_freq = np.float32(1.0) / powf
    pos = (np.arange(x.shape[1]) + offset).astype(np.float32)
    angles = pos[:, None] * inv_freq[None, :]               # [seq, half], f32 products
    c = np.cos(angles.astype(np.float64))[None]
    s = np.sin(angles.astype(np.float64))[None]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)


class KvCacheNp:
    """LayerKVCache's content for one layer, kept as the reference keeps it after
    the GQA expansion: K and V [heads, len, hd] in f32 (kv_cache.rs:91-130)."""

    def __init__(self, n_heads: int, head_dim: int):
        self.k = np.zeros((n_heads, 0, head_dim), np.float32)
        self.v = np.zeros((n_heads, 0, head_dim), np.float32)

    @property
    def length(self) -> int:
        return self.k.shape[1]

    def append(self, k: np.ndarray, v: np.ndarray) -> None:
        self.k = np.concatenate([self.k, k.astype(np.float32)], axis=1)
        self.v = np.concatenate([self.v, v.astype(np.float32)], axis=1)


def forward_with_cache_attention(qkv: np.ndarray, n_heads: int, n_kv_heads: int, head_dim: int,
                                 theta: float, cache: KvCacheNp, scale: float | None = None,
                                 exp=np.exp) -> np.ndarray:
    """Steps 2-9 of forward_with_cache for m new tokens whose projections are
    qkv[m, (H + 2 KVH) hd] = [q | k | v].  Appends to ``cache``; returns
    attn_output[m, H hd] in float64."""
    m = qkv.shape[0]
    H, KVH, D = n_heads, n_kv_heads, head_dim
    G = H // KVH
    q = qkv[:, :H * D].astype(np.float64).reshape(m, H, D).transpose(1, 0, 2)
    k = qkv[:, H * D:(H + KVH) * D].astype(np.float64).reshape(m, KVH, D).transpose(1, 0, 2)
    v = qkv[:, (H + KVH) * D:].astype(np.float64).reshape(m, KVH, D).transpose(1, 0, 2)
    offset = cache.length
    q = rope_with_offset(q, D, theta, offset)
    k = rope_with_offset(k, D, theta, offset)
    # unsqueeze(2) + broadcast_as [KVH, G, ...] + reshape [H, ...]: head h <- kv head h // G
    k = np.repeat(k, G, axis=0)
    v = np.repeat(v, G, axis=0)
    cache.append(k, v)
    full_k = cache.k.astype(np.float64)
    full_v = cache.v.astype(np.float64)
    total = cache.length
    s = reference_scale(D) if scale is None else scale
    scores = np.matmul(q, full_k.transpose(0, 2, 1)) * s          # [H, m, total]
    qpos = offset + np.arange(m)
    mask = np.where(np.arange(total)[None, :] > qpos[:, None], -np.inf, 0.0)
    scores = scores + mask[None]
    w = exp(scores - scores.max(axis=-1, keepdims=True))
    w = w / w.sum(axis=-1, keepdims=True)
    out = np.matmul(w, full_v)                                      # [H, m, D]
    return out.transpose(1, 0, 2).reshape(m, H * D)
