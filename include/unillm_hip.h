/*
 * unillm_hip.h -- C ABI of the MI355X (gfx950) quantized linear-layer device.
 *
 * This is the drop-in boundary for unillm's quantized matmul: the matmul that
 * candle's QMatMul::forward runs today on GGUF Q4_0 / Q8_0 weights loaded by
 * WeightLoaderCore.  Plain C types only (pointers, sizes, int status) so that
 * a Rust `extern "C"` block, ctypes or C++ can bind it unchanged.
 *
 * Conventions
 *   - Status: 0 = OK, negative = error; unillm_hip_last_error() returns the
 *     message of the last failing call on the calling thread.  (The reference
 *     reports errors as anyhow::Result strings, e.g. "QMatMul forward failed:
 *     ..." at crates/runtime/src/models_v2/llama.rs:1189; a binding maps a
 *     negative status plus this message onto that.)
 *   - Layout: W is [n, k] (n = out features, k = in features), row-major GGUF
 *     blocks along k, exactly as GGUF stores a tensor with ne = [k, n]
 *     (candle reverses ne into shape [n, k]).  x is [m, k] f32 row-major and
 *     y = x . dequant(W)^T is [m, n] f32 row-major.
 *   - Preconditions checked on the host before any launch: k % 32 == 0
 *     (k % 256 == 0 for Q4_K, Q5_K, Q6_K; any k >= 1 for the dense types), n >= 1,
 *     m >= 0, non-null pointers, known qtype.
 *   - Streams: a `void* stream` is a hipStream_t (NULL = the null stream).
 *     Compute calls are asynchronous on that stream and never synchronise.
 *   - Ownership: a qweight owns its device copy of the weights and is
 *     immutable after create, so it may be shared across threads.  The caller
 *     owns x, y and the stream.
 */
#ifndef UNILLM_HIP_H
#define UNILLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids as GGUF stores them (candle GgmlDType::Q4_0 / Q8_0 / Q4K / Q5K /
 * Q6K; the reference maps Q4K at crates/runtime/src/weight_loader_core.rs:481 and
 * hands every type to QMatMul::from_arc at :569-571; Q5K holds the projections of
 * GGUF Q5_K_M files, Q6K what Q4_K_M / Q5_K_M files use for output.weight and some
 * attn_v / ffn_down). */
#define UNILLM_QTYPE_Q4_0 2
#define UNILLM_QTYPE_Q8_0 8
/* GGML Q5_0 ({f16 d; u8 qh[4]; u8 qs[16]}: 5-bit codes, (q - 16) d), e.g. the fallback
 * type of K-quant mixes for tensors whose k is not a multiple of 256.  Its values
 * are exactly int8 codes times an f16 d, so the device keeps it as a Q8_0 weight
 * (unillm_hip_qweight_info still reports 6). */
#define UNILLM_QTYPE_Q5_0 6
#define UNILLM_QTYPE_Q4_K 12
#define UNILLM_QTYPE_Q5_K 13
#define UNILLM_QTYPE_Q6_K 14
/* Dense projection weights (GGML F32 / F16 / BF16).  candle's QMatMul::from_arc
 * dequantizes such a tensor to f32 and multiplies in f32 (its Tensor variant);
 * the reference's loader wraps every *_proj / lm_head tensor in a QMatMul whatever
 * its type (crates/runtime/src/weight_loader_core.rs:554-571).  Stored here as f32
 * rows (F16 and BF16 widen exactly) and multiplied by an f32 GEMM; any k >= 1. */
#define UNILLM_QTYPE_F32 0
#define UNILLM_QTYPE_F16 1
#define UNILLM_QTYPE_BF16 30

#define UNILLM_OK 0
#define UNILLM_ERR_INVALID_ARG (-1)
#define UNILLM_ERR_UNSUPPORTED (-2)
#define UNILLM_ERR_HIP (-3)
#define UNILLM_ERR_OUT_OF_MEMORY (-4)
#define UNILLM_ERR_NOT_INITIALIZED (-5)

/* Kernel path for unillm_hip_qmatmul_path (AUTO is what qmatmul uses). */
#define UNILLM_PATH_AUTO 0
/* GEMV, m <= 4, k up to: m = 1 14336 (Q4_0, Q4_K) or 16384 (Q8_0, Q5_0, Q5_K, Q6_K);
 * m = 2 12288; m = 3, 4 4096.  Past k 8192 (byte codes at m = 1, every type at
 * m = 2) and past k 2048 at m = 3, 4 (not Q6_K), k is split over the two waves of a
 * pair.  Larger k takes the batched decode under UNILLM_PATH_AUTO. */
#define UNILLM_PATH_GEMV 1         /* fused dequant + GEMV (VALU int8 dot), m <= 4 */
#define UNILLM_PATH_DECODE_MFMA 2  /* batched decode, f16 MFMA, fp32 accumulate */
#define UNILLM_PATH_PREFILL_MFMA 3 /* prefill, LDS-staged f16 MFMA (x rows scaled by powers of two), fp32 accumulate */
#define UNILLM_PATH_DENSE 4        /* dense weights: f32 GEMM (rocBLAS), the only path they take */

typedef struct unillm_qweight unillm_qweight;
typedef struct unillm_kv_cache unillm_kv_cache;
typedef struct unillm_graph unillm_graph;

/* Select and check the device (must be gfx950).  Replaces the device choice the
 * reference makes with `Device` (crates/runtime/src/tensor_core.rs:39-44), to
 * which a binding adds HIP(usize).  Calls on other entry points made before
 * init use device 0 after an implicit init. */
int unillm_hip_init(int device);

/* Message of the last error on the calling thread ("" if none). */
const char* unillm_hip_last_error(void);

/* Upload one GGUF Q4_0 / Q5_0 / Q8_0 / Q4_K / Q5_K / Q6_K tensor ([n, k]: n * k/32 blocks
 * of 18 / 22 / 34 B, or n * k/256 blocks of 144 / 176 / 210 B), or a dense F32 / F16 / BF16 one
 * (n * k elements of 4 / 2 / 2 B), to the device, repacked there into the kernels'
 * layout (dense: f32 rows).  Replaces
 * `QMatMul::from_arc(Arc::new(qtensor))` at
 * crates/runtime/src/weight_loader_core.rs:569-571 (the QTensor read at :545).
 * layout_flags must be 0 (reserved). */
int unillm_hip_qweight_create(int qtype, int64_t n, int64_t k, const void* host_blocks,
                              size_t nbytes, int layout_flags, unillm_qweight** out);

/* As unillm_hip_qweight_create, from GGUF block bytes already in device memory
 * (e.g. produced by unillm_hip_quantize).  Runs on `stream` and synchronises it
 * before returning, so the source may be freed afterwards. */
int unillm_hip_qweight_create_device(int qtype, int64_t n, int64_t k, const void* dev_blocks,
                                     size_t nbytes, int layout_flags, void* stream,
                                     unillm_qweight** out);

/* Free a weight (NULL is a no-op).  Drop of the Arc<QMatMul> in ModelWeights
 * (crates/runtime/src/model_core.rs:134). */
int unillm_hip_qweight_destroy(unillm_qweight* w);

/* Shape and footprint of a weight; any out-pointer may be NULL. */
int unillm_hip_qweight_info(const unillm_qweight* w, int* qtype, int64_t* n, int64_t* k,
                            size_t* device_bytes);

/* y[m, n] = x[m, k] . dequant(W)^T, f32 in and out.  Replaces
 * QMatMul::forward as called from LlamaAttention/LlamaMLP::quantized_matmul
 * (crates/runtime/src/models_v2/llama.rs:1184-1195, 1325-1336) and
 * LlamaModelV2::lm_head_forward (llama.rs:396-405); the m rows are the
 * flattened leading dims of the [.., k] input.  m == 0 is a no-op.
 * Operand range: every path takes any finite x, as candle's per-block Q8_0
 * activations do: the GEMV holds x as exact integer digits per 32-block, prefill
 * rounds each row of x to f16 after scaling it by its own power of two, and
 * batched decode does the same per row and k slice of its split. */
int unillm_hip_qmatmul(const unillm_qweight* w, const float* x_dev, int64_t m, float* y_dev,
                       void* stream);

/* x and y need only f32 (4-byte) alignment, as candle's contiguous f32 tensors
 * have; x not on a 16-byte boundary is first copied (stream-ordered) into an
 * aligned per-stream buffer, since the kernels load it 16 bytes at a time.
 *
 * Workspace.  The MFMA paths (and SwiGLU off the GEMV path) use per-stream
 * device buffers that grow on first use and are then kept for later calls on
 * that stream.  Growing allocates, which cannot be recorded into a HIP graph: a
 * call that would grow a buffer while its stream is being captured fails with
 * UNILLM_ERR_UNSUPPORTED and a message naming the size.  Reserve the buffers
 * before capturing (unillm_hip_qmatmul_reserve / unillm_hip_attention_reserve),
 * or make the same calls once eagerly first.  Outgrown buffers are never freed
 * (a captured graph may still use them).  A graph uses the buffers of the stream
 * it was captured on: replay it on that stream. */

/* unillm_hip_qmatmul without any allocation.  No counterpart in the reference
 * (candle allocates per call): it is for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops.  Same result as
 * unillm_hip_qmatmul (same kernels); the MFMA paths keep their f16 copy of x in
 * a 64 MiB scratch array that the library holds on each GPU from load to process
 * end, instead of the stream's workspace.  Limits: x 16-byte aligned; the scratch
 * takes m * k * 2 bytes (+ 4 m for prefill, + S * m * n * 4 when a prefill
 * splits k into S <= 16 slices; a split that would not fit gives way to the
 * 128-row plan that fits, at worst unsplit, agreeing with unillm_hip_qmatmul to
 * f32 rounding): calls beyond 64 MiB fail with
 * UNILLM_ERR_UNSUPPORTED before any launch.  All calls on one GPU share its
 * scratch: calls that overlap in time on one GPU (concurrent streams, or threads
 * without ordering) race and must not be issued. */
int unillm_hip_qmatmul_noalloc(const unillm_qweight* w, const float* x_dev, int64_t m,
                               float* y_dev, void* stream);

/* As unillm_hip_qmatmul with an explicit kernel path (UNILLM_PATH_*), for
 * tests and benchmarks; AUTO picks what unillm_hip_qmatmul picks. */
int unillm_hip_qmatmul_path(const unillm_qweight* w, const float* x_dev, int64_t m,
                            float* y_dev, int path, void* stream);

/* y[m, n] += x[m, k] . dequant(W)^T: the projection with the decoder layer's
 * residual add in its epilogue.  Replaces qmatmul.forward followed by
 * ops_fn::add(hidden_states, out) for o_proj and down_proj
 * (crates/runtime/src/models_v2/llama.rs:668, 677).  y holds the residual on
 * entry.  Equal bit for bit to qmatmul then the add, except where k is split
 * over workgroups (partials then add onto y in any order: f32 rounding). */
int unillm_hip_qmatmul_add(const unillm_qweight* w, const float* x_dev, int64_t m, float* y_dev,
                           void* stream);

/* act[m, I] = silu(x . G^T) * (x . U^T) for a weight whose n = 2 I rows are
 * gate_proj (rows 0 .. I - 1) then up_proj (I .. 2 I - 1), e.g. a gate_up
 * handle fused at load.  Replaces the two quantized_matmul calls and
 * ops_fn::fused_swiglu of LlamaMLP::forward (llama.rs:1275-1283;
 * tensor_core.rs:1385-1396: candle silu(v) = v / (1 + e^-v)).  On the GEMV path
 * (m = 1: k <= 8192 for Q4_0 / Q4_K, 4096 for Q8_0 / Q5_K / Q6_K; half that at m = 2,
 * a quarter at m = 3, 4) the gate and up rows meet in one wave and the
 * activation is its epilogue; otherwise the
 * [m, 2 I] product goes to a per-stream workspace and one elementwise pass
 * follows.  n odd is an error. */
int unillm_hip_qmatmul_swiglu(const unillm_qweight* w, const float* x_dev, int64_t m,
                              float* act_dev, void* stream);

/* y[m, n] = LN(x)[m, k] . dequant(W)^T with LN(x) = (x - mean) / sqrt(var + eps)
 * * gamma (+ beta) along k, var = mean((x - mean)^2): the layer norm the
 * reference applies before the attention and MLP projections
 * (ops_fn::layer_norm, crates/runtime/src/tensor_core.rs:973-1008, called with
 * eps = 1e-6 at crates/runtime/src/models_v2/llama.rs:662, 671) fused into the
 * matmul: on the GEMV path every workgroup normalizes x while its first
 * weights stream in; the MFMA paths normalize in their x conversion.
 * gamma[k] (and beta[k], which may be NULL) are device f32, 16-byte aligned. */
int unillm_hip_qmatmul_norm(const unillm_qweight* w, const float* x_dev, const float* gamma_dev,
                            const float* beta_dev, float eps, int64_t m, float* y_dev,
                            void* stream);

/* unillm_hip_qmatmul_swiglu on LN(x): post_attention_layernorm, gate, up and
 * SwiGLU of LlamaMLP in one call (llama.rs:671-674, 1275-1283). */
int unillm_hip_qmatmul_norm_swiglu(const unillm_qweight* w, const float* x_dev,
                                   const float* gamma_dev, const float* beta_dev, float eps,
                                   int64_t m, float* act_dev, void* stream);

/* Kernel path that unillm_hip_qmatmul selects for m rows (UNILLM_PATH_*). */
int unillm_hip_select_path(const unillm_qweight* w, int64_t m);

/* Grow `stream`'s workspace to what any qmatmul / _add / _norm call on w with up
 * to m rows needs (and, with swiglu != 0, the _swiglu / _norm_swiglu calls), x
 * on any 4-byte boundary included, so such calls can then be captured into a
 * HIP graph.  No counterpart in the
 * reference (candle allocates per call and has no graphs): it serves callers
 * that capture.  Allocates stream-ordered on `stream`; not while capturing. */
int unillm_hip_qmatmul_reserve(const unillm_qweight* w, int64_t m, int swiglu, void* stream);

/* One decoder layer's KV cache on the device for one sequence: K and V of
 * n_kv_heads heads, max_seq positions of head_dim f32 each (zeroed), and the
 * RoPE frequencies of rope_theta.  Replaces LayerKVCache::with_capacity
 * (crates/runtime/src/kv_cache.rs:46-53; its buffers are allocated on the first
 * append there).  head_dim is 64, 128 or 256. */
int unillm_hip_kv_cache_create(int64_t n_kv_heads, int64_t head_dim, int64_t max_seq,
                               float rope_theta, unillm_kv_cache** out);
int unillm_hip_kv_cache_destroy(unillm_kv_cache* c);
/* Filled positions (LayerKVCache::seq_len, kv_cache.rs:74-76).  The length lives
 * in device memory (see unillm_hip_attention_decode); after a call on the cache
 * has been captured into a HIP graph this synchronises the device to read it. */
int unillm_hip_kv_cache_length(const unillm_kv_cache* c, int64_t* len);
/* Forget the filled positions, keep the buffers (LayerKVCache::clear,
 * kv_cache.rs:61-63).  Synchronises the device (the new length is written to
 * device memory once all issued work is done); not during graph capture. */
int unillm_hip_kv_cache_clear(unillm_kv_cache* c);
/* Keep the first len positions (0 <= len <= the filled length): a rolled-back
 * step, e.g. rejected speculative tokens.  No counterpart in LayerKVCache,
 * whose only shrink is clear(); the positions past len are rewritten by the
 * next appends.  Synchronises the device, as unillm_hip_kv_cache_clear. */
int unillm_hip_kv_cache_truncate(unillm_kv_cache* c, int64_t len);

/* The attention of LlamaAttention::forward_with_cache after its projections
 * (crates/runtime/src/models_v2/llama.rs:1044-1150) for m new tokens of one
 * sequence: qkv_dev[m, (n_heads + 2 n_kv_heads) head_dim] holds the q, k and v
 * projections (a fused qkv handle's output); RoPE (apply_rope_with_offset,
 * llama.rs:827-883) at positions len .. len + m - 1, k and v appended to the
 * cache, then softmax(q k^T / sqrt(head_dim) + causal mask) v into
 * out_dev[m, n_heads head_dim], head h reading kv head h / (n_heads /
 * n_kv_heads).  The cache's length grows by m.  Any m: decode steps
 * (m * n_heads / n_kv_heads <= 16, len + m <= 131072) split the cache into
 * chunks; longer calls (the prompt, llama.rs:488-497) run a tiled causal kernel.
 * Overflow of max_seq is an error with the reference's message
 * (kv_cache.rs:114-121).  Calls on one cache must be ordered (one stream), as
 * each appends to it.
 * Graph capture: the kernels read the cache length from device memory and
 * advance it there, so a captured call appends at the next position on every
 * replay (a decode step captured once serves successive tokens).  A replayed
 * call past max_seq appends nothing, writes NaN and makes the next length query
 * or eager call fail with the overflow message; clear / truncate reset it.
 * Alignment: qkv_dev 16 bytes; out_dev 4 bytes on a decode step, 16 bytes on a
 * longer call (its kernels store 16 bytes at a time). */
int unillm_hip_attention_decode(unillm_kv_cache* c, const float* qkv_dev, int64_t m,
                                int64_t n_heads, float* out_dev, void* stream);

/* Grow `stream`'s attention workspace to what unillm_hip_attention_decode of up to
 * m tokens and n_heads heads needs at any cache length, so such calls can be
 * captured into a HIP graph (no counterpart in the reference; as
 * unillm_hip_qmatmul_reserve). */
int unillm_hip_attention_reserve(const unillm_kv_cache* c, int64_t m, int64_t n_heads,
                                 void* stream);

/* out[n, k] = dequant(W) in f32, bit-exact with GGML's to_float.  Replaces
 * `qtensor.dequantize(&device)` at crates/runtime/src/weight_loader_core.rs:579. */
int unillm_hip_dequant(const unillm_qweight* w, float* out_dev, void* stream);

/* GGML reference quantizer on the device: w[n, k] f32 -> GGUF block bytes
 * (n * k/32 blocks of 18 / 34 B), bit-exact with GGML quantize_row_q4_0/q8_0
 * (candle QTensor::quantize; used by the reference only to make GGUF files).
 * Q4_K / Q5_K / Q6_K are refused with UNILLM_ERR_UNSUPPORTED (their GGML quantizers
 * search scales iteratively and are not on this path). */
int unillm_hip_quantize(int qtype, const float* w_dev, int64_t n, int64_t k, void* blocks_dev,
                        void* stream);

/* Device memory helpers for bindings without their own allocator. */
int unillm_hip_malloc(void** ptr, size_t bytes);
int unillm_hip_free(void* ptr);
int unillm_hip_memcpy_htod(void* dst_dev, const void* src_host, size_t bytes);
int unillm_hip_memcpy_dtoh(void* dst_host, const void* src_dev, size_t bytes);
int unillm_hip_synchronize(void);

/* Streams and HIP graphs for bindings without a HIP runtime of their own.  No
 * counterpart in the reference (candle runs eagerly): they serve a decode step
 * captured once and replayed per token, the loop of generate_with_cache
 * (crates/runtime/src/models_v2/llama.rs:525-559).  Capture: reserve the
 * workspaces of every call first (unillm_hip_qmatmul_reserve,
 * unillm_hip_attention_reserve), call graph_begin on a stream from
 * stream_create, issue the calls on it (nothing runs), then graph_end.  A
 * replay (graph_launch, on any stream) runs the captured calls on the buffers
 * they were given; attention calls append at the cache's current length. */
int unillm_hip_stream_create(void** stream);
int unillm_hip_stream_destroy(void* stream);
int unillm_hip_stream_synchronize(void* stream);
int unillm_hip_graph_begin(void* stream);
int unillm_hip_graph_end(void* stream, unillm_graph** out);
int unillm_hip_graph_launch(const unillm_graph* g, void* stream);
int unillm_hip_graph_destroy(unillm_graph* g);

#ifdef __cplusplus
}
#endif
#endif /* UNILLM_HIP_H */
