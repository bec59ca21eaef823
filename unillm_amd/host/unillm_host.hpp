// unillm_host.hpp -- C++ host side of the HIP quantized linear-layer device.
//
// The reference is Rust (cognisoc/unillm); no Rust toolchain exists in this
// build environment, so the host layer above the C ABI is C++ that mirrors
// the reference's interface for this path, name for name:
//
//   reference (crates/runtime/src/...)              here
//   tensor_core.rs:39-44   enum Device {CPU, CUDA, Metal}   Device (+ HIP(id))
//   tensor_core.rs:47-70   trait TensorStorage             HipStorage
//   tensor_core.rs:13-24   struct Tensor                   Tensor (f32, host or HIP)
//   tensor_core.rs:179-296 trait TensorOps::matmul         TensorOps / HipTensorOps
//   model_core.rs:124-138  ModelWeights{tensors, quantized_tensors}   ModelWeights
//   model_core.rs:469-471  ModelWeights::get_quantized     ModelWeights::get_quantized
//   candle QMatMul (Arc)   used at llama.rs:1184-1195       QuantLinear
//   weight_loader_core.rs:504-608  GGUFWeightLoader       GgufWeightLoader
//   weight_loader_core.rs:760-798  gguf_to_hf_name        gguf_to_hf_name
//   kv_cache.rs:28-183     LayerKVCache                    LayerKVCache (HIP, f32)
//   kv_cache.rs:193-270    KVCache                         KVCache
//   llama.rs:1044-1150     forward_with_cache after the projections   LayerKVCache::attend
//
// Errors are exceptions carrying the reference's anyhow text ("QMatMul
// forward failed: ...").  All device work goes through include/unillm_hip.h.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/unillm_hip.h"
#include "gguf.hpp"

namespace unillm {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// ---- Device ------------------------------------------------------------------------------
enum class DeviceKind { CPU, CUDA, Metal, HIP };

struct Device {
    DeviceKind kind = DeviceKind::CPU;
    size_t id = 0;
    static Device cpu() { return {DeviceKind::CPU, 0}; }
    static Device hip(size_t id) { return {DeviceKind::HIP, id}; }
    bool is_hip() const { return kind == DeviceKind::HIP; }
    bool operator==(const Device& o) const { return kind == o.kind && id == o.id; }
    bool operator!=(const Device& o) const { return !(*this == o); }
    std::string to_string() const;
};

// ---- Storage -----------------------------------------------------------------------------
// Device memory owned through the C ABI's allocator (TensorStorage on HIP).
class HipStorage {
public:
    HipStorage(size_t bytes, Device device);
    ~HipStorage();
    HipStorage(const HipStorage&) = delete;
    HipStorage& operator=(const HipStorage&) = delete;
    void* data_ptr() const { return ptr_; }
    size_t size_bytes() const { return bytes_; }
    const Device& device() const { return device_; }

private:
    void* ptr_ = nullptr;
    size_t bytes_ = 0;
    Device device_;
};

// ---- Tensor (f32 only: the dtype of this path's activations and outputs) ------------------
class Tensor {
public:
    Tensor() = default;
    static Tensor from_host(const std::vector<float>& data, std::vector<int64_t> shape,
                            const Device& device);
    static Tensor empty(std::vector<int64_t> shape, const Device& device);

    const std::vector<int64_t>& shape() const { return shape_; }
    int64_t numel() const;
    int64_t dim(int i) const;  // negative i counts from the end
    const Device& device() const { return device_; }
    const float* data() const;       // host or device pointer, per device()
    float* data_mut();
    Tensor to_device(const Device& device) const;
    std::vector<float> to_host() const;
    Tensor reshape(std::vector<int64_t> shape) const;

private:
    std::vector<int64_t> shape_;
    Device device_;
    std::shared_ptr<std::vector<float>> host_;
    std::shared_ptr<HipStorage> dev_;
};

// ---- the quantized projection --------------------------------------------------------------
// Holds one GGUF Q4_0 / Q8_0 weight [n, k] resident on the HIP device; the
// slot `Arc<QMatMul>` occupies in ModelWeights.
class QuantLinear {
public:
    static std::shared_ptr<QuantLinear> from_blocks(int qtype, int64_t n, int64_t k,
                                                    const void* blocks, size_t nbytes);
    ~QuantLinear();
    QuantLinear(const QuantLinear&) = delete;
    QuantLinear& operator=(const QuantLinear&) = delete;

    // QMatMul::forward: [.., k] f32 -> [.., n] f32 (rank >= 2, last dim k).
    Tensor forward(const Tensor& x, void* stream = nullptr) const;
    // residual += forward(x) in the projection's epilogue: the decoder layer's
    // residual add after o_proj / down_proj (llama.rs:668, 677).
    void forward_add(const Tensor& x, Tensor& residual, void* stream = nullptr) const;
    // For a [gate; up] handle (LoadOptions::fuse_gate_up): silu(gate) * up, [.., n / 2]
    // (LlamaMLP::forward's two projections and fused_swiglu, llama.rs:1275-1283).
    Tensor forward_swiglu(const Tensor& x, void* stream = nullptr) const;
    // forward on the layer norm of x along k, (x - mean) / sqrt(var + eps) *
    // gamma (+ beta) (ops_fn::layer_norm, tensor_core.rs:973-1008), fused into the
    // matmul; gamma / beta are HIP tensors of k elements (beta may be empty).
    Tensor forward_norm(const Tensor& x, const Tensor& gamma, const Tensor* beta, float eps,
                        void* stream = nullptr) const;
    // forward_swiglu on the layer norm of x: post_attention_layernorm, gate, up and
    // SwiGLU in one call (llama.rs:671-674, 1275-1283).
    Tensor forward_norm_swiglu(const Tensor& x, const Tensor& gamma, const Tensor* beta,
                               float eps, void* stream = nullptr) const;
    // qtensor.dequantize: f32 [n, k] on the device, bit-exact with GGML.
    Tensor dequantize(void* stream = nullptr) const;

    int qtype() const { return qtype_; }
    int64_t n() const { return n_; }
    int64_t k() const { return k_; }
    const unillm_qweight* handle() const { return w_; }

private:
    QuantLinear() = default;
    void check_input(const Tensor& x) const;
    unillm_qweight* w_ = nullptr;
    int qtype_ = 0;
    int64_t n_ = 0, k_ = 0;
};

// LlamaModelV2::lm_head_forward (llama.rs:396-405) with a quantized lm_head: the
// projection of the final hidden states to logits, errors reported as the reference
// reports them ("QMatMul lm_head forward failed: ...").
Tensor lm_head_forward(const QuantLinear& lm_head, const Tensor& hidden_states,
                       void* stream = nullptr);

// ---- KV cache and decode attention ------------------------------------------------------------
// One decoder layer's cache for one sequence on the HIP device: K and V of n_kv_heads
// heads, max_seq_len positions of head_dim f32 (kv_cache.rs:28-183; the reference's
// buffers are [1, heads, seq, hd] candle tensors on the CPU).  Non-copyable, movable.
class LayerKVCache {
public:
    // LayerKVCache::with_capacity(max_seq_len) (kv_cache.rs:46-53), with the shapes and
    // the RoPE base that the reference takes from the model config at append time.
    static LayerKVCache with_capacity(int64_t n_kv_heads, int64_t head_dim, int64_t max_seq_len,
                                      float rope_theta = 10000.0f);
    ~LayerKVCache();
    LayerKVCache(LayerKVCache&& o) noexcept;
    LayerKVCache& operator=(LayerKVCache&& o) noexcept;
    LayerKVCache(const LayerKVCache&) = delete;
    LayerKVCache& operator=(const LayerKVCache&) = delete;

    bool is_empty() const { return seq_len() == 0; }  // kv_cache.rs:56-58
    int64_t seq_len() const;                           // kv_cache.rs:74-76
    int64_t max_seq_len() const { return max_seq_; }   // kv_cache.rs:79-81
    void clear();                                      // kv_cache.rs:61-64
    // Keep the first len positions (a rolled-back step); no reference counterpart.
    void truncate(int64_t len);
    // The part of LlamaAttention::forward_with_cache after the q / k / v projections
    // (llama.rs:1044-1150): qkv [m, (n_heads + 2 n_kv_heads) head_dim] on the HIP device
    // (a fused qkv handle's output) -> RoPE at positions seq_len() .., k and v appended
    // (LayerKVCache::append, kv_cache.rs:91-130, including its overflow error), causal
    // softmax attention -> [m, n_heads head_dim], freshly allocated.
    Tensor attend(const Tensor& qkv, int64_t n_heads, void* stream = nullptr);
    // attend into a caller's HIP buffer of m * n_heads * head_dim floats (no allocation).
    void attend_into(const Tensor& qkv, int64_t n_heads, Tensor& out, void* stream = nullptr);

    int64_t n_kv_heads() const { return n_kv_heads_; }
    int64_t head_dim() const { return head_dim_; }
    unillm_kv_cache* handle() const { return c_; }

private:
    LayerKVCache() = default;
    unillm_kv_cache* c_ = nullptr;
    int64_t n_kv_heads_ = 0, head_dim_ = 0, max_seq_ = 0;
};

// The model's caches, one LayerKVCache per decoder layer (kv_cache.rs:193-270).
class KVCache {
public:
    static KVCache with_capacity(size_t num_layers, int64_t n_kv_heads, int64_t head_dim,
                                 int64_t max_seq_len, float rope_theta = 10000.0f);
    size_t num_layers() const { return layers_.size(); }
    LayerKVCache& layer_mut(size_t i);
    const LayerKVCache& layer(size_t i) const;
    int64_t seq_len() const;  // layer 0's, as the reference reports it
    int64_t max_seq_len() const;
    bool is_empty() const { return seq_len() == 0; }
    void clear();

private:
    std::vector<LayerKVCache> layers_;
};

// ---- ops dispatch ----------------------------------------------------------------------------
class TensorOps {
public:
    virtual ~TensorOps() = default;
    // out = a . b^T where b is a quantized [n, k] weight (the call
    // quantized_matmul makes); f32 x f32 matmul is not part of this device.
    virtual Tensor matmul(const Tensor& a, const QuantLinear& b) = 0;
};

class HipTensorOps : public TensorOps {
public:
    explicit HipTensorOps(void* stream = nullptr) : stream_(stream) {}
    Tensor matmul(const Tensor& a, const QuantLinear& b) override;

private:
    void* stream_;
};

// ---- weights and loading --------------------------------------------------------------------
struct GgufModelConfig {
    std::string architecture;
    uint64_t hidden_size = 0, intermediate_size = 0, num_hidden_layers = 0;
    uint64_t num_attention_heads = 0, num_key_value_heads = 0, vocab_size = 0;
    uint64_t head_dim = 0;                  // hidden_size / num_attention_heads
    float rms_norm_eps = 1e-5f;             // {arch}.attention.layer_norm_rms_epsilon
    float rope_theta = 10000.0f;            // {arch}.rope.freq_base
    uint64_t max_position_embeddings = 2048;  // {arch}.context_length
};

struct ModelWeights {
    std::map<std::string, Tensor> tensors;                                  // f32, host
    std::map<std::string, std::shared_ptr<QuantLinear>> quantized_tensors;  // HIP
    GgufModelConfig config;
    // fused handle -> its parts in row order: {part hf name, rows}; a part's
    // outputs are columns [sum of the earlier rows, + rows) of the fused output
    std::map<std::string, std::vector<std::pair<std::string, int64_t>>> fused_parts;
    std::shared_ptr<QuantLinear> get_quantized(const std::string& name) const;
};

// Load-time fusion of projections that read the same input.  With fuse_qkv,
// model.layers.N.self_attn.{q,k,v}_proj become one self_attn.qkv_proj handle,
// with fuse_gate_up mlp.{gate,up}_proj one mlp.gate_up_proj handle -- one launch
// instead of three / two per token -- when the parts share a GGUF type and k
// (a Q4_K_M layer whose attn_v is Q6_K keeps its parts apart).  Off by default:
// the reference model calls the parts by name.
struct LoadOptions {
    bool fuse_qkv = false;
    bool fuse_gate_up = false;
};

// weight_loader_core.rs:760-798: ordered substring replacements.
std::string gguf_to_hf_name(const std::string& gguf_name);
// weight_loader_core.rs:554: which tensors stay quantized.
bool is_quantized_weight_name(const std::string& hf_name);

class GgufWeightLoader {
public:
    bool supports(const std::string& path) const;
    // Parses the file, uploads every *_proj / lm_head tensor to the device as
    // a QuantLinear (Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, or the dense F32 / F16 / BF16) and
    // dequantizes the rest to host f32.
    ModelWeights load_weights(const std::string& path, const LoadOptions& opt = {}) const;
    // What load_weights would do, without any device work: hf name, shape,
    // type and whether it would be quantized, per tensor.
    struct Plan {
        std::string gguf_name, hf_name;
        std::vector<uint64_t> shape;
        uint32_t type;
        bool quantized;
    };
    std::vector<Plan> plan(const GgufFile& file) const;
    static GgufModelConfig config_from(const GgufFile& file);
};

// ---- the model ---------------------------------------------------------------------------
// LlamaModelV2::forward_with_cache (llama.rs:421-462) over device-resident GGUF weights.
// Per call of m new tokens:
//   1. embedding: rows of model.embed_tokens.weight (f32 on the host, as the loader
//      keeps it) gathered and copied to the device;
//   2. per decoder layer (llama.rs:654-680): input_layernorm (eps 1e-6) fused into the
//      q/k/v projection, attention with the layer's cache (LayerKVCache::attend),
//      o_proj with the residual add in its epilogue, post_attention_layernorm
//      (eps 1e-6) fused into gate_up with SwiGLU, down_proj with the residual add;
//   3. model.norm (eps = rms_norm_eps of the GGUF) fused into lm_head.
// "layer_norm" is the reference's ops_fn::layer_norm: mean-subtracting, no bias
// (tensor_core.rs:973-1008).  Six launches a layer and one for the head.
// The weights must hold the fused gate_up handle of every layer (load with
// LoadOptions::fuse_gate_up); q/k/v use the fused qkv handle where the loader made
// one, else the three projections run a token at a time into the qkv rows.
class CapturedDecodeStep;

class LlamaModel {
public:
    explicit LlamaModel(ModelWeights weights);  // throws if a tensor is missing
    // GgufWeightLoader::load_weights with q/k/v and gate/up fused, then the model.
    static LlamaModel load(const std::string& gguf_path);

    const GgufModelConfig& config() const { return w_.config; }
    int64_t vocab_size() const { return lm_head_->n(); }
    // A cache for this model: one LayerKVCache per layer, the model's kv heads, head
    // dim and rope_theta.
    KVCache new_cache(int64_t max_seq_len) const;
    // input_ids: the m new tokens -> logits [m, vocab] (HIP), freshly allocated; the
    // cache grows by m (forward_with_cache's position offset is the cache's length).
    Tensor forward_with_cache(const std::vector<int32_t>& input_ids, KVCache& cache,
                              void* stream = nullptr) const;

private:
    friend class CapturedDecodeStep;
    struct Layer {
        Tensor in_norm, post_norm;  // HIP, hidden_size each
        std::shared_ptr<QuantLinear> qkv, q, k, v, o, gate_up, down;
    };
    // The device buffers of one call of m tokens: h holds the embedded rows and is the
    // residual stream the layers add into; qkv, att and act are the per-layer
    // intermediates (reused by every layer); logits [m, vocab].
    struct StepBuffers {
        int64_t m = 0;
        Tensor h, qkv, att, act, logits;
    };
    StepBuffers step_buffers(int64_t m) const;
    // The embedding rows of input_ids (ops_fn::embedding), on the host.
    std::vector<float> embed_rows(const std::vector<int32_t>& input_ids) const;
    // Steps 2 and 3 of forward_with_cache on b.h: launches only, into b's buffers (no
    // allocation), so a step can be captured into a HIP graph.
    void forward_layers(StepBuffers& b, KVCache& cache, void* stream) const;
    ModelWeights w_;
    int64_t hidden_ = 0, heads_ = 0, kv_heads_ = 0, head_dim_ = 0;
    Tensor embed_;  // host [vocab, hidden] (shares w_'s storage)
    std::vector<Layer> layers_;
    Tensor norm_;  // HIP
    std::shared_ptr<QuantLinear> lm_head_;
};

// The loop of LlamaModelV2::generate_with_cache (llama.rs:525-559) a token at a time,
// as a HIP graph: one m = 1 call of forward_with_cache (every layer's norm + q/k/v,
// attention with the layer's cache, o_proj + residual, norm + gate_up + SwiGLU,
// down + residual, then the final norm + lm_head) captured once over device buffers of
// its own, and replayed per token.  The attention kernels read and advance each
// layer's cache length on the device, so replay i appends at the position the cache
// holds then.  The model and the cache must outlive the step; other calls on the cache
// (an eager prompt first, a truncate between tokens) keep working.
class CapturedDecodeStep {
public:
    // Reserves the workspaces and captures on a stream of its own (nothing runs).
    CapturedDecodeStep(const LlamaModel& model, KVCache& cache);
    ~CapturedDecodeStep();
    CapturedDecodeStep(const CapturedDecodeStep&) = delete;
    CapturedDecodeStep& operator=(const CapturedDecodeStep&) = delete;
    // Copies token's embedding row into the step's input and replays the graph:
    // logits [1, vocab] on the device (the step's own buffer, rewritten by the next
    // run); the cache grows by one.  Waits for the previous replay first.
    const Tensor& run(int32_t token);

private:
    const LlamaModel& model_;
    void* stream_ = nullptr;
    unillm_graph* graph_ = nullptr;
    LlamaModel::StepBuffers b_;
};

}  // namespace unillm
