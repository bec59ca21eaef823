"""Write tests/golden/tiny_llama_q4_0.gguf, tiny_llama_q4_k_m.gguf, tiny_llama_q5_k_m.gguf and
their expected outputs.

A minimal GGUF v3 file in the layout llama.cpp writes for a Llama model:
2 blocks of attn_q/k/v/output + ffn_gate/up/down (Q4_0), token_embd (Q8_0),
output (lm_head, Q8_0), attn_norm/ffn_norm/output_norm (F32).  No gguf
package exists offline, so the writer follows the published GGUF v3 spec:

  header   : magic "GGUF", u32 version = 3, u64 n_tensors, u64 n_kv
  kv       : gguf string key (u64 len + bytes), u32 value type, value
  tensors  : name, u32 n_dims, u64 ne[n_dims] (ne[0] = innermost = k),
             u32 ggml type, u64 offset (from the data section, aligned)
  data     : starts at the next multiple of general.alignment (32)

Expected values (tiny_llama_q4_0.npz): for every projection, x and
y = x . dequant(W)^T in f64 (numpy), the names after the reference's
gguf_to_hf_name map (crates/runtime/src/weight_loader_core.rs:760-798), and
which tensors stay quantized (weight_loader_core.rs:554).

tiny_llama_q4_0.step: the logits of LlamaModelV2::forward_with_cache
(llama.rs:421-462) over three calls on one cache (a 12-token prompt, then two
single tokens), computed in f64: the oracle's exact dequant, the attention with a
KV cache from llama_attention_np.py (a numpy restatement of forward_with_cache's
attention, independent of the oracle's), and numpy for the layer norms, SwiGLU
and residuals.
Layout: "USTP", u32 vocab, u32 n_steps; per step u32 m, i32 ids[m],
f64 logits[m * vocab].

tiny_llama_f16.gguf is the tiny_llama_q4_0 architecture with dense projections,
the variant candle's QMatMul::from_arc keeps as a dequantized f32 tensor: F16
everywhere (token_embd and output too) except layer 0's attn_output (F32) and
layer 1's ffn_down (BF16); .expect and .step as above, from the exact widened
weights.

tiny_llama_q4_k_m.gguf has the tensor types llama.cpp's Q4_K_M mix uses:
Q4_K projections and token_embd, Q6_K for output.weight and for layer 0's
attn_v / ffn_down.  Its blocks are random valid Q4_K / Q6_K blocks (the
oracle's generators) and its expectations the oracle's f64 matmul.
tiny_llama_q5_k_m.gguf is the same mix with Q5_K in place of Q4_K (llama.cpp's
Q5_K_M: Q5_K projections and token_embd, Q6_K for output.weight and layer 0's
attn_v / ffn_down).
"""
from __future__ import annotations

import os
import struct
import sys

import numpy as np

from make_golden import dequant, quantize_q4_0, quantize_q8_0

HERE = os.path.dirname(os.path.abspath(__file__))
ALIGN = 32
T_F32, T_F16, T_Q4_0, T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K, T_BF16 = 0, 1, 2, 8, 12, 13, 14, 30
DENSE = (T_F32, T_F16, T_BF16)
V_UINT32, V_FLOAT32, V_STRING, V_ARRAY = 4, 6, 8, 9

HIDDEN, INTER, VOCAB, LAYERS = 128, 96, 128, 2
HEADS, KV_HEADS = 2, 1  # head_dim 64, two query heads a kv head
ROPE_BASE = 20000.0
NORM_EPS = 1e-5
STEPS = [[3, 17, 42, 99, 5, 64, 127, 0, 31, 77, 12, 88], [7], [100]]


def gstr(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def kv(key: str, vtype: int, value) -> bytes:
    out = gstr(key) + struct.pack("<I", vtype)
    if vtype == V_UINT32:
        out += struct.pack("<I", value)
    elif vtype == V_FLOAT32:
        out += struct.pack("<f", value)
    elif vtype == V_STRING:
        out += gstr(value)
    elif vtype == V_ARRAY:
        etype, items = value
        out += struct.pack("<IQ", etype, len(items))
        for it in items:
            out += gstr(it) if etype == V_STRING else struct.pack("<I", it)
    return out


def main() -> None:
    rng = np.random.default_rng(7)
    tensors = []  # (gguf name, ggml type, [n, k] shape, raw bytes, dequantized f32 or None)

    def add_q(name, qtype, n, k):
        w = rng.normal(0.0, 0.02, size=(n, k)).astype(np.float32)
        blocks = quantize_q4_0(w) if qtype == T_Q4_0 else quantize_q8_0(w)
        tensors.append((name, qtype, (n, k), blocks.tobytes(), dequant(qtype, blocks, n, k)))

    def add_f32(name, n):
        v = (1.0 + rng.normal(0, 0.1, size=n)).astype(np.float32)
        tensors.append((name, T_F32, (n,), v.tobytes(), v))

    add_q("token_embd.weight", T_Q8_0, VOCAB, HIDDEN)
    for i in range(LAYERS):
        p = f"blk.{i}."
        add_f32(p + "attn_norm.weight", HIDDEN)
        add_q(p + "attn_q.weight", T_Q4_0, HIDDEN, HIDDEN)
        add_q(p + "attn_k.weight", T_Q4_0, HIDDEN // 2, HIDDEN)
        add_q(p + "attn_v.weight", T_Q4_0, HIDDEN // 2, HIDDEN)
        add_q(p + "attn_output.weight", T_Q4_0, HIDDEN, HIDDEN)
        add_f32(p + "ffn_norm.weight", HIDDEN)
        add_q(p + "ffn_gate.weight", T_Q4_0, INTER, HIDDEN)
        add_q(p + "ffn_up.weight", T_Q4_0, INTER, HIDDEN)
        add_q(p + "ffn_down.weight", T_Q4_0, HIDDEN, INTER)
    add_f32("output_norm.weight", HIDDEN)
    add_q("output.weight", T_Q8_0, VOCAB, HIDDEN)

    write(tensors, "tiny_llama_q4_0", HIDDEN, INTER, LAYERS, rng, npz=True,
          heads=(HEADS, KV_HEADS), rope_base=ROPE_BASE)
    write_steps(tensors, "tiny_llama_q4_0")
    main_kq()
    main_kq(T_Q5_K)
    main_dense()


def dense_bytes(w: np.ndarray, ttype: int):
    """GGUF bytes of a dense tensor and its exact values (f32 holds F16 and BF16)."""
    if ttype == T_F32:
        return w.astype(np.float32).tobytes(), w.astype(np.float32)
    if ttype == T_F16:
        h = w.astype(np.float16)
        return h.tobytes(), h.astype(np.float32)
    u = w.astype(np.float32).view(np.uint32).astype(np.uint64)  # BF16: round to nearest even
    b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return b.tobytes(), (b.astype(np.uint32) << 16).view(np.float32)


def main_dense() -> None:
    """The tiny Llama with dense (F32 / F16 / BF16) projections."""
    rng = np.random.default_rng(13)
    tensors = []

    def add_d(name, ttype, n, k, std=0.02):
        raw, exact = dense_bytes(rng.normal(0.0, std, size=(n, k)), ttype)
        tensors.append((name, ttype, (n, k), raw, exact))

    def add_f32(name, n):
        v = (1.0 + rng.normal(0, 0.1, size=n)).astype(np.float32)
        tensors.append((name, T_F32, (n,), v.tobytes(), v))

    add_d("token_embd.weight", T_F16, VOCAB, HIDDEN, std=1.0)
    for i in range(LAYERS):
        p = f"blk.{i}."
        add_f32(p + "attn_norm.weight", HIDDEN)
        add_d(p + "attn_q.weight", T_F16, HIDDEN, HIDDEN)
        add_d(p + "attn_k.weight", T_F16, HIDDEN // 2, HIDDEN)
        add_d(p + "attn_v.weight", T_F16, HIDDEN // 2, HIDDEN)
        add_d(p + "attn_output.weight", T_F32 if i == 0 else T_F16, HIDDEN, HIDDEN)
        add_f32(p + "ffn_norm.weight", HIDDEN)
        add_d(p + "ffn_gate.weight", T_F16, INTER, HIDDEN)
        add_d(p + "ffn_up.weight", T_F16, INTER, HIDDEN)
        add_d(p + "ffn_down.weight", T_BF16 if i == 1 else T_F16, HIDDEN, INTER)
    add_f32("output_norm.weight", HIDDEN)
    add_d("output.weight", T_F16, VOCAB, HIDDEN)
    write(tensors, "tiny_llama_f16", HIDDEN, INTER, LAYERS, rng, npz=False,
          heads=(HEADS, KV_HEADS), rope_base=ROPE_BASE)
    write_steps(tensors, "tiny_llama_f16")


def layer_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """ops_fn::layer_norm with no bias (tensor_core.rs:973-1008): mean-subtracting,
    biased variance, in f64."""
    c = x - x.mean(axis=-1, keepdims=True)
    return c / np.sqrt((c * c).mean(axis=-1, keepdims=True) + eps) * w


def write_steps(tensors, stem) -> None:
    """The f64 logits of forward_with_cache (llama.rs:421-462; the decoder layer
    llama.rs:654-680) for the calls in STEPS, one cache across them."""
    sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
    import oracle  # test infrastructure: exact dequant
    from llama_attention_np import KvCacheNp, forward_with_cache_attention

    W = {}
    for name, ttype, shape, raw, deq in tensors:
        if ttype in DENSE:  # the exact values (F16 / BF16 widened)
            W[hf_name(name)] = deq.astype(np.float64)
        else:
            n, k = shape
            blocks = np.frombuffer(raw, dtype=np.uint8)
            W[hf_name(name)] = oracle.dequant(ttype, blocks, n, k).astype(np.float64)
    hd = HIDDEN // HEADS
    caches = [KvCacheNp(HEADS, hd) for _ in range(LAYERS)]
    blob = b"USTP" + struct.pack("<II", VOCAB, len(STEPS))
    for ids in STEPS:
        h = W["model.embed_tokens.weight"][ids]
        for i, cache in enumerate(caches):
            p = f"model.layers.{i}."
            xn = layer_norm(h, W[p + "input_layernorm.weight"], 1e-6)
            qkv = np.concatenate([xn @ W[p + f"self_attn.{t}_proj.weight"].T for t in "qkv"],
                                 axis=1)
            att = forward_with_cache_attention(qkv.astype(np.float32), HEADS, KV_HEADS, hd,
                                               ROPE_BASE, cache)
            h = h + att @ W[p + "self_attn.o_proj.weight"].T
            xn = layer_norm(h, W[p + "post_attention_layernorm.weight"], 1e-6)
            g = xn @ W[p + "mlp.gate_proj.weight"].T
            u = xn @ W[p + "mlp.up_proj.weight"].T
            h = h + (g / (1.0 + np.exp(-g)) * u) @ W[p + "mlp.down_proj.weight"].T
        logits = layer_norm(h, W["model.norm.weight"], NORM_EPS) @ W["lm_head.weight"].T
        blob += struct.pack("<I", len(ids)) + struct.pack(f"<{len(ids)}i", *ids)
        blob += logits.astype("<f8").tobytes()
    with open(os.path.join(HERE, stem + ".step"), "wb") as f:
        f.write(blob)


def main_kq(kt: int = T_Q4_K) -> None:
    """The Q4_K_M-style file (kt = T_Q4_K) or the Q5_K_M-style one (kt = T_Q5_K); k a
    multiple of 256."""
    sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
    import oracle  # test infrastructure: random K-quant blocks and their exact dequant

    hidden, inter, layers = 256, 512, 2
    rng = np.random.default_rng(11 if kt == T_Q4_K else 13)
    tensors = []
    seed = [100 if kt == T_Q4_K else 200]

    def add_k(name, qtype, n, k):
        seed[0] += 1
        gen = {T_Q4_K: oracle.random_q4_k, T_Q5_K: oracle.random_q5_k,
               T_Q6_K: oracle.random_q6_k}[qtype]
        blocks = gen(n, k, seed[0])
        tensors.append((name, qtype, (n, k), blocks.tobytes(), oracle.dequant(qtype, blocks, n, k)))

    def add_f32(name, n):
        v = (1.0 + rng.normal(0, 0.1, size=n)).astype(np.float32)
        tensors.append((name, T_F32, (n,), v.tobytes(), v))

    add_k("token_embd.weight", kt, 256, hidden)
    for i in range(layers):
        p = f"blk.{i}."
        add_f32(p + "attn_norm.weight", hidden)
        add_k(p + "attn_q.weight", kt, hidden, hidden)
        add_k(p + "attn_k.weight", kt, hidden // 2, hidden)
        add_k(p + "attn_v.weight", T_Q6_K if i == 0 else kt, hidden // 2, hidden)
        add_k(p + "attn_output.weight", kt, hidden, hidden)
        add_f32(p + "ffn_norm.weight", hidden)
        add_k(p + "ffn_gate.weight", kt, inter, hidden)
        add_k(p + "ffn_up.weight", kt, inter, hidden)
        add_k(p + "ffn_down.weight", T_Q6_K if i == 0 else kt, hidden, inter)
    add_f32("output_norm.weight", hidden)
    add_k("output.weight", T_Q6_K, 256, hidden)
    stem = "tiny_llama_q4_k_m" if kt == T_Q4_K else "tiny_llama_q5_k_m"
    write(tensors, stem, hidden, inter, layers, rng, npz=False)


def write(tensors, stem, hidden, inter, layers, rng, npz, heads=(4, 2), rope_base=None) -> None:
    kvs = [
        kv("general.architecture", V_STRING, "llama"),
        kv("general.name", V_STRING, "tiny-llama-test"),
        kv("general.alignment", V_UINT32, ALIGN),
        kv("llama.embedding_length", V_UINT32, hidden),
        kv("llama.feed_forward_length", V_UINT32, inter),
        kv("llama.block_count", V_UINT32, layers),
        kv("llama.attention.head_count", V_UINT32, heads[0]),
        kv("llama.attention.head_count_kv", V_UINT32, heads[1]),
        kv("llama.attention.layer_norm_rms_epsilon", V_FLOAT32, NORM_EPS),
        kv("tokenizer.ggml.tokens", V_ARRAY, (V_STRING, [f"t{i}" for i in range(8)])),
    ]
    if rope_base is not None:
        kvs.append(kv("llama.rope.freq_base", V_FLOAT32, rope_base))
    header = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kvs)) + b"".join(kvs)

    infos = b""
    data = b""
    for name, ttype, shape, raw, _ in tensors:
        pad = (-len(data)) % ALIGN
        data += b"\0" * pad
        ne = list(reversed(shape))  # ggml ne[0] is the innermost (k) dimension
        infos += gstr(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne)
        infos += struct.pack("<IQ", ttype, len(data))
        data += raw
    meta = header + infos
    meta += b"\0" * ((-len(meta)) % ALIGN)
    with open(os.path.join(HERE, stem + ".gguf"), "wb") as f:
        f.write(meta + data)

    # expected outputs for every tensor the loader keeps quantized
    out = {}
    hf = []
    names = []
    for name, ttype, shape, raw, deq in tensors:
        mapped = hf_name(name)
        names.append(name)
        hf.append(mapped)
        if "_proj.weight" in mapped or "lm_head.weight" in mapped:
            n, k = shape
            x = rng.normal(0, 1, size=(3, k)).astype(np.float32)
            key = mapped.replace(".", "_")
            out["x__" + key] = x
            out["y__" + key] = x.astype(np.float64) @ deq.astype(np.float64).T
    out["gguf_names"] = np.array(names)
    out["hf_names"] = np.array(hf)
    if npz:
        np.savez_compressed(os.path.join(HERE, stem + ".npz"), **out)
    # the same expectations in a flat binary the C++ host test reads:
    # "UXPT", u32 count; per tensor: u32 len + gguf name, u32 len + hf name,
    # u32 type, u32 quantized, u32 m, u32 n, u32 k, f32 x[m*k], f64 y[m*n]
    blob = b"UXPT" + struct.pack("<I", len(tensors))
    for name, ttype, shape, raw, deq in tensors:
        mapped = hf_name(name)
        quant = "_proj.weight" in mapped or "lm_head.weight" in mapped
        key = mapped.replace(".", "_")
        blob += struct.pack("<I", len(name)) + name.encode()
        blob += struct.pack("<I", len(mapped)) + mapped.encode()
        if quant:
            x, y = out["x__" + key], out["y__" + key]
            blob += struct.pack("<5I", ttype, 1, x.shape[0], y.shape[1], x.shape[1])
            blob += x.astype("<f4").tobytes() + y.astype("<f8").tobytes()
        else:
            blob += struct.pack("<5I", ttype, 0, 0, 0, 0)
    with open(os.path.join(HERE, stem + ".expect"), "wb") as f:
        f.write(blob)
    print(f"wrote {stem}.gguf ({len(meta) + len(data)} B), {len(tensors)} tensors")


def hf_name(name: str) -> str:
    """The reference's GGUF -> HuggingFace name map, as a table of ordered
    substring replacements (weight_loader_core.rs:760-798)."""
    for a, b in HF_MAP:
        name = name.replace(a, b)
    return name


HF_MAP = [
    ("token_embd.weight", "model.embed_tokens.weight"),
    ("blk.", "model.layers."),
    (".attn_output.weight", ".self_attn.o_proj.weight"),
    (".attn_q.weight", ".self_attn.q_proj.weight"),
    (".attn_k.weight", ".self_attn.k_proj.weight"),
    (".attn_v.weight", ".self_attn.v_proj.weight"),
    (".attn_output.bias", ".self_attn.o_proj.bias"),
    (".attn_q.bias", ".self_attn.q_proj.bias"),
    (".attn_k.bias", ".self_attn.k_proj.bias"),
    (".attn_v.bias", ".self_attn.v_proj.bias"),
    ("output_norm.weight", "model.norm.weight"),
    ("output.weight", "lm_head.weight"),
    (".ffn_gate.weight", ".mlp.gate_proj.weight"),
    (".ffn_up.weight", ".mlp.up_proj.weight"),
    (".ffn_down.weight", ".mlp.down_proj.weight"),
    (".ffn_gate.bias", ".mlp.gate_proj.bias"),
    (".ffn_up.bias", ".mlp.up_proj.bias"),
    (".ffn_down.bias", ".mlp.down_proj.bias"),
    (".attn_norm.weight", ".input_layernorm.weight"),
    (".ffn_norm.weight", ".post_attention_layernorm.weight"),
    (".attn_norm.bias", ".input_layernorm.bias"),
    (".ffn_norm.bias", ".post_attention_layernorm.bias"),
]


if __name__ == "__main__":
    main()
