/*
 * oracle.h -- CPU restatement of unillm's quantized linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (unillm_amd/, include/)
 * links, loads or calls this code.  Only tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py use it, and only as the checker / the timed
 * CPU baseline.
 *
 * The reference (cognisoc/unillm) runs this path through candle-core 0.8
 * (crates/runtime/Cargo.toml:35, un-vendored, patch version unpinned because
 * Cargo.lock is not committed, .gitignore:4).  Candle implements the GGML
 * block formats; this file restates the published GGML definitions:
 *
 *   Q4_0 block (18 B / 32 weights): { f16 d; u8 qs[16]; }
 *        w[j]    = ((qs[j] & 0xF) - 8) * d      j = 0..15
 *        w[j+16] = ((qs[j] >>  4) - 8) * d
 *   Q8_0 block (34 B / 32 weights): { f16 d; i8 qs[32]; }   w[j] = qs[j] * d
 *   Q5_0 block (22 B / 32 weights): { f16 d; u8 qh[4]; u8 qs[16]; }  (dequantize_row_q5_0)
 *        w[j]    = ((qs[j] & 0xF) | bit j of qh << 4) - 16) * d          j = 0..15
 *        w[j+16] = ((qs[j] >>  4) | bit j + 16 of qh << 4) - 16) * d
 *   Q4_K block (144 B / 256 weights, GGML block_q4_K, candle GgmlDType::Q4K,
 *        mapped at weight_loader_core.rs:481):
 *        { f16 d; f16 dmin; u8 scales[12]; u8 qs[128]; }
 *        sub-block j (32 weights) has a 6-bit scale sc_j and min m_j packed in
 *        scales[] (get_scale_min_k4); group g = 0..3 of 64 weights uses
 *        qs[32 g .. 32 g + 31]: low nibbles -> sub-block 2 g, high -> 2 g + 1;
 *        w = (d * sc_j) * q - (dmin * m_j)       (dequantize_row_q4_K)
 *   Q5_K block (176 B / 256 weights, GGML block_q5_K, candle GgmlDType::Q5K):
 *        { f16 d; f16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]; }
 *        Q4_K's scales, mins and nibbles; weight l of sub-block j takes bit j
 *        of qh[l] as its fifth bit: q = nibble | bit << 4, 0..31;
 *        w = (d * sc_j) * q - (dmin * m_j)       (dequantize_row_q5_K)
 *   Q6_K block (210 B / 256 weights, GGML block_q6_K):
 *        { u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d; }
 *        w = (d * scales[s]) * (q - 32), q 6-bit from ql (4) and qh (2)
 *                                                  (dequantize_row_q6_K)
 *
 * Call sites in the reference that this path serves:
 *   crates/runtime/src/weight_loader_core.rs:543-584  (GGUF read, QMatMul::from_arc)
 *   crates/runtime/src/models_v2/llama.rs:1184-1195, 1325-1336, 396-405 (forward)
 *   crates/runtime/src/tensor_core.rs:843-892  (the f32 fallback matmul whose
 *       semantics -- y = x . W^T in f32 with exactly dequantized W -- define parity)
 *
 * Parity pinning (all exercised by tests/test_oracle.py):
 *   f16<->f32          : numpy's float16 conversions, exhaustive over 65536 codes
 *   dequant            : closed form, exhaustive over all scales x all codes;
 *                        the reference's layout-neutral known answers
 *                        (simd/quant/block.rs:398-423, q4_0.rs:131-178).
 *                        Q4_K / Q5_K / Q6_K: one-hot blocks that expose every index
 *                        (which byte, nibble, scale and min each weight uses),
 *                        the 6-bit scale packing as the inverse of GGML's
 *                        packer over all 64 x 64 values per sub-block, and an
 *                        independent numpy decoding (tests/test_oracle.py)
 *   quantizers         : invariants (max-magnitude element -> code 0 for Q4_0,
 *                        round-trip error <= d/2 for Q8_0), hand-computed blocks,
 *                        and an independent numpy restatement (tests/golden)
 *   f64 matmul         : numpy float64 matmul (library routine), known answers
 *                        6.3984375 / 12.796875 / 32 (simd/matmul/gemv.rs:91-113,
 *                        simd/matmul/gemm.rs:404-429, simd/arch/avx2.rs:569-594)
 *   candle-semantics   : loose bound (~1e-2 normwise) against the f64 oracle;
 *   CPU path             bit-identity with candle's SIMD summation order is
 *                        not claimed (timing baseline only).
 *   attention          : closed forms (one position returns v, equal keys
 *                        average, RoPE known answers, relative-position
 *                        invariance, causality) and, for the softmax's scale and
 *                        base, an independent numpy restatement of
 *                        forward_with_cache's tensor steps
 *                        (tests/golden/llama_attention_np.py) on random keys,
 *                        to 1e-12, with planted wrong scales / bases shown to fail
 */
#ifndef UNILLM_ORACLE_H
#define UNILLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_QK 32
#define ORACLE_Q4_0 2
#define ORACLE_Q5_0 6
#define ORACLE_Q8_0 8
#define ORACLE_Q4_K 12
#define ORACLE_Q5_K 13
#define ORACLE_Q6_K 14

/* weights per block: 32 (Q4_0, Q5_0, Q8_0) or 256 (Q4_K, Q5_K, Q6_K); 0 for unknown types */
int oracle_block_elems(int qtype);
/* bytes per block: 18 (Q4_0), 22 (Q5_0), 34 (Q8_0), 144 (Q4_K), 176 (Q5_K), 210 (Q6_K); 0 for
 * unknown */
size_t oracle_block_bytes(int qtype);

/* IEEE binary16 <-> binary32 (round to nearest even, subnormals, inf, nan) */
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);

/* GGML reference quantizers (Q4_0, Q8_0), weights [n, k] row-major -> GGUF block bytes */
int oracle_quantize(int qtype, const float* w, int64_t n, int64_t k, uint8_t* blocks);

/* exact dequant, GGUF block bytes -> f32 [n, k] (k a multiple of the block size) */
int oracle_dequant(int qtype, const uint8_t* blocks, int64_t n, int64_t k, float* out);

/* the parity oracle: y[m, n] = sum_k x[m, k] * dequant(W)[n, k], accumulated in f64 */
int oracle_qmatmul_f64(int qtype, const uint8_t* blocks, const float* x,
                       int64_t m, int64_t n, int64_t k, double* y, int nthreads);

/* candle CPU semantics (timing baseline; Q4_0 and Q8_0): x rows -> Q8_0, integer
 * block dots, f32 accumulation of isum * d_w * d_x, parallel over N in column chunks */
int oracle_candle_qmatmul(int qtype, const uint8_t* blocks, const float* x,
                          int64_t m, int64_t n, int64_t k, float* y, int nthreads);

/* Decode attention with a KV cache (LlamaAttention::forward_with_cache,
 * crates/runtime/src/models_v2/llama.rs:1044-1150; LayerKVCache::append,
 * crates/runtime/src/kv_cache.rs:91-130):
 *   qkv[m, (H + 2 KVH) hd]: the fused q / k / v projections of m new tokens;
 *   RoPE (apply_rope_with_offset, llama.rs:827-883: half-split rotation,
 *   inv_freq = 1 / theta^(2i / hd) and angle = pos * inv_freq in f32) at
 *   positions len .. len + m - 1; k, v appended to k_cache / v_cache
 *   ([KVH][max_seq][hd], updated in place); head h reads kv head h / (H / KVH);
 *   out[m, H hd] = softmax(q k^T * scale + causal mask) v, in f64, with
 *   scale = 1 / sqrt(hd) formed in f32 as LlamaAttention::new does (llama.rs:890). */
int oracle_attention_decode(const float* qkv, int64_t m, int64_t n_heads, int64_t n_kv_heads,
                            int64_t head_dim, float rope_theta, float* k_cache, float* v_cache,
                            int64_t max_seq, int64_t len, double* out);

/* deterministic N(mean, std) generator: SplitMix64 -> Box-Muller (f64) -> f32 */
void oracle_fill_normal(float* out, int64_t count, uint64_t seed, double mean, double std);

#ifdef __cplusplus
}
#endif
#endif
