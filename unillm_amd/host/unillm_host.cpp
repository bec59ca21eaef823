// unillm_host.cpp -- implementation of the C++ host layer (see unillm_host.hpp).
#include "unillm_host.hpp"

#include <algorithm>
#include <cstring>

namespace unillm {

namespace {

void check(int rc, const char* what) {
    if (rc != UNILLM_OK)
        throw Error(std::string(what) + ": " + unillm_hip_last_error());
}

// A failed matmul call: `ctx` (the caller's anyhow context, llama.rs:399, 1189) and
// the C ABI's detail, without the ABI's own "QMatMul forward failed: " prefix.
void check_qmatmul(int rc, const char* ctx) {
    if (rc == UNILLM_OK) return;
    std::string m = unillm_hip_last_error();
    const std::string p = "QMatMul forward failed: ";
    if (m.compare(0, p.size(), p) == 0) m = m.substr(p.size());
    throw Error(std::string(ctx) + ": " + m);
}

int64_t product(const std::vector<int64_t>& shape) {
    int64_t p = 1;
    for (int64_t d : shape) {
        if (d < 0) throw Error("negative dimension");
        p *= d;
    }
    return p;
}

// IEEE binary16 / bfloat16 -> binary32 (exact) for F16 / BF16 GGUF tensors.
float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            float v = (float)man * (1.0f / 16777216.0f);  // man * 2^-24, exact
            std::memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

float bf16_to_float(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

}  // namespace

std::string Device::to_string() const {
    switch (kind) {
        case DeviceKind::CPU: return "CPU";
        case DeviceKind::CUDA: return "CUDA(" + std::to_string(id) + ")";
        case DeviceKind::Metal: return "Metal(" + std::to_string(id) + ")";
        case DeviceKind::HIP: return "HIP(" + std::to_string(id) + ")";
    }
    return "?";
}

// ---- HipStorage ----------------------------------------------------------------------------
HipStorage::HipStorage(size_t bytes, Device device) : bytes_(bytes), device_(device) {
    if (!device.is_hip()) throw Error("HipStorage on " + device.to_string());
    check(unillm_hip_init((int)device.id), "unillm_hip_init");
    if (bytes) check(unillm_hip_malloc(&ptr_, bytes), "unillm_hip_malloc");
}

HipStorage::~HipStorage() {
    if (ptr_) unillm_hip_free(ptr_);
}

// ---- Tensor --------------------------------------------------------------------------------
Tensor Tensor::empty(std::vector<int64_t> shape, const Device& device) {
    Tensor t;
    const int64_t n = product(shape);
    t.shape_ = std::move(shape);
    t.device_ = device;
    if (device.is_hip())
        t.dev_ = std::make_shared<HipStorage>((size_t)n * sizeof(float), device);
    else if (device.kind == DeviceKind::CPU)
        t.host_ = std::make_shared<std::vector<float>>((size_t)n);
    else
        throw Error("tensors on " + device.to_string() + " are not supported by this build");
    return t;
}

Tensor Tensor::from_host(const std::vector<float>& data, std::vector<int64_t> shape,
                         const Device& device) {
    if ((int64_t)data.size() != product(shape)) throw Error("data size does not match shape");
    Tensor t = empty(std::move(shape), device);
    if (device.is_hip()) {
        if (!data.empty())
            check(unillm_hip_memcpy_htod(t.dev_->data_ptr(), data.data(),
                                         data.size() * sizeof(float)),
                  "copy to device");
    } else {
        *t.host_ = data;
    }
    return t;
}

int64_t Tensor::numel() const { return product(shape_); }

int64_t Tensor::dim(int i) const {
    const int r = (int)shape_.size();
    if (i < 0) i += r;
    if (i < 0 || i >= r) throw Error("dimension index out of range");
    return shape_[(size_t)i];
}

const float* Tensor::data() const {
    if (dev_) return static_cast<const float*>(dev_->data_ptr());
    return host_ ? host_->data() : nullptr;
}

float* Tensor::data_mut() {
    if (dev_) return static_cast<float*>(dev_->data_ptr());
    return host_ ? host_->data() : nullptr;
}

std::vector<float> Tensor::to_host() const {
    if (host_) return *host_;
    std::vector<float> out((size_t)numel());
    if (!out.empty())
        check(unillm_hip_memcpy_dtoh(out.data(), dev_->data_ptr(), out.size() * sizeof(float)),
              "copy to host");
    return out;
}

Tensor Tensor::to_device(const Device& device) const {
    if (device == device_) return *this;
    return from_host(to_host(), shape_, device);
}

Tensor Tensor::reshape(std::vector<int64_t> shape) const {
    if (product(shape) != numel()) throw Error("reshape changes the element count");
    Tensor t = *this;
    t.shape_ = std::move(shape);
    return t;
}

// ---- QuantLinear ---------------------------------------------------------------------------
std::shared_ptr<QuantLinear> QuantLinear::from_blocks(int qtype, int64_t n, int64_t k,
                                                      const void* blocks, size_t nbytes) {
    std::shared_ptr<QuantLinear> q(new QuantLinear());
    check(unillm_hip_qweight_create(qtype, n, k, blocks, nbytes, 0, &q->w_),
          "Failed to create QMatMul");
    q->qtype_ = qtype;
    q->n_ = n;
    q->k_ = k;
    return q;
}

QuantLinear::~QuantLinear() { unillm_hip_qweight_destroy(w_); }

void QuantLinear::check_input(const Tensor& x) const {
    // candle QMatMul::forward rules (called at llama.rs:1188): f32, rank >= 2,
    // last dim == k
    if (x.shape().size() < 2)
        throw Error("QMatMul forward failed: rank " + std::to_string(x.shape().size()) +
                    " input, need rank >= 2");
    if (x.dim(-1) != k_)
        throw Error("QMatMul forward failed: input last dim " + std::to_string(x.dim(-1)) +
                    " != k " + std::to_string(k_));
    if (!x.device().is_hip())
        throw Error("QMatMul forward failed: input is on " + x.device().to_string() +
                    ", weight is on HIP");
}

Tensor QuantLinear::forward(const Tensor& x, void* stream) const {
    check_input(x);  // output [.., n], freshly allocated
    std::vector<int64_t> oshape = x.shape();
    oshape.back() = n_;
    Tensor y = Tensor::empty(oshape, x.device());
    const int64_t m = x.numel() / k_;
    check_qmatmul(unillm_hip_qmatmul(w_, x.data(), m, y.data_mut(), stream), "QMatMul forward failed");
    return y;
}

void QuantLinear::forward_add(const Tensor& x, Tensor& residual, void* stream) const {
    check_input(x);
    std::vector<int64_t> oshape = x.shape();
    oshape.back() = n_;
    if (residual.shape() != oshape || !residual.device().is_hip())
        throw Error("QMatMul forward failed: residual must be a HIP tensor of the output shape");
    check_qmatmul(
        unillm_hip_qmatmul_add(w_, x.data(), x.numel() / k_, residual.data_mut(), stream),
        "QMatMul forward failed");
}

Tensor QuantLinear::forward_swiglu(const Tensor& x, void* stream) const {
    check_input(x);
    std::vector<int64_t> oshape = x.shape();
    oshape.back() = n_ / 2;
    Tensor act = Tensor::empty(oshape, x.device());
    check_qmatmul(
        unillm_hip_qmatmul_swiglu(w_, x.data(), x.numel() / k_, act.data_mut(), stream),
        "QMatMul forward failed");
    return act;
}

Tensor QuantLinear::forward_norm(const Tensor& x, const Tensor& gamma, const Tensor* beta,
                                 float eps, void* stream) const {
    check_input(x);
    auto vec_k = [&](const Tensor& t) {
        return t.device().is_hip() && t.numel() == k_;
    };
    if (!vec_k(gamma) || (beta && !vec_k(*beta)))
        throw Error("QMatMul forward failed: norm weight / bias must be HIP tensors of k elements");
    std::vector<int64_t> oshape = x.shape();
    oshape.back() = n_;
    Tensor y = Tensor::empty(oshape, x.device());
    check_qmatmul(unillm_hip_qmatmul_norm(w_, x.data(), gamma.data(),
                                          beta ? beta->data() : nullptr, eps, x.numel() / k_,
                                          y.data_mut(), stream),
                  "QMatMul forward failed");
    return y;
}

Tensor QuantLinear::forward_norm_swiglu(const Tensor& x, const Tensor& gamma, const Tensor* beta,
                                        float eps, void* stream) const {
    check_input(x);
    auto vec_k = [&](const Tensor& t) {
        return t.device().is_hip() && t.numel() == k_;
    };
    if (!vec_k(gamma) || (beta && !vec_k(*beta)))
        throw Error("QMatMul forward failed: norm weight / bias must be HIP tensors of k elements");
    std::vector<int64_t> oshape = x.shape();
    oshape.back() = n_ / 2;
    Tensor act = Tensor::empty(oshape, x.device());
    check_qmatmul(unillm_hip_qmatmul_norm_swiglu(w_, x.data(), gamma.data(),
                                                 beta ? beta->data() : nullptr, eps,
                                                 x.numel() / k_, act.data_mut(), stream),
                  "QMatMul forward failed");
    return act;
}

Tensor lm_head_forward(const QuantLinear& lm_head, const Tensor& hidden_states, void* stream) {
    // LlamaModelV2::lm_head_forward (llama.rs:396-405) maps the QMatMul error to
    // "QMatMul lm_head forward failed: {e}"
    try {
        return lm_head.forward(hidden_states, stream);
    } catch (const Error& e) {
        std::string m = e.what();
        const std::string p = "QMatMul forward failed: ";
        if (m.compare(0, p.size(), p) == 0) m = m.substr(p.size());
        throw Error("QMatMul lm_head forward failed: " + m);
    }
}

Tensor QuantLinear::dequantize(void* stream) const {
    Tensor out = Tensor::empty({n_, k_}, Device::hip(0));
    check(unillm_hip_dequant(w_, out.data_mut(), stream), "Failed to dequantize");
    check(unillm_hip_synchronize(), "Failed to dequantize");
    return out;
}

Tensor HipTensorOps::matmul(const Tensor& a, const QuantLinear& b) {
    return b.forward(a, stream_);
}

// ---- ModelWeights / loader -----------------------------------------------------------------
std::shared_ptr<QuantLinear> ModelWeights::get_quantized(const std::string& name) const {
    auto it = quantized_tensors.find(name);
    return it == quantized_tensors.end() ? nullptr : it->second;
}

std::string gguf_to_hf_name(const std::string& gguf_name) {
    // The reference's ordered replacement table (weight_loader_core.rs:764-795):
    // the order matters (".attn_output.weight" before "output.weight").
    static const char* const kMap[][2] = {
        {"token_embd.weight", "model.embed_tokens.weight"},
        {"blk.", "model.layers."},
        {".attn_output.weight", ".self_attn.o_proj.weight"},
        {".attn_q.weight", ".self_attn.q_proj.weight"},
        {".attn_k.weight", ".self_attn.k_proj.weight"},
        {".attn_v.weight", ".self_attn.v_proj.weight"},
        {".attn_output.bias", ".self_attn.o_proj.bias"},
        {".attn_q.bias", ".self_attn.q_proj.bias"},
        {".attn_k.bias", ".self_attn.k_proj.bias"},
        {".attn_v.bias", ".self_attn.v_proj.bias"},
        {"output_norm.weight", "model.norm.weight"},
        {"output.weight", "lm_head.weight"},
        {".ffn_gate.weight", ".mlp.gate_proj.weight"},
        {".ffn_up.weight", ".mlp.up_proj.weight"},
        {".ffn_down.weight", ".mlp.down_proj.weight"},
        {".ffn_gate.bias", ".mlp.gate_proj.bias"},
        {".ffn_up.bias", ".mlp.up_proj.bias"},
        {".ffn_down.bias", ".mlp.down_proj.bias"},
        {".attn_norm.weight", ".input_layernorm.weight"},
        {".ffn_norm.weight", ".post_attention_layernorm.weight"},
        {".attn_norm.bias", ".input_layernorm.bias"},
        {".ffn_norm.bias", ".post_attention_layernorm.bias"},
    };
    std::string s = gguf_name;
    for (const auto& m : kMap) {
        const std::string from = m[0], to = m[1];
        std::string out;
        size_t pos = 0, hit;
        while ((hit = s.find(from, pos)) != std::string::npos) {  // Rust str::replace: all, left to right
            out.append(s, pos, hit - pos);
            out += to;
            pos = hit + from.size();
        }
        out.append(s, pos, std::string::npos);
        s = std::move(out);
    }
    return s;
}

bool is_quantized_weight_name(const std::string& hf_name) {
    return hf_name.find("_proj.weight") != std::string::npos ||
           hf_name.find("lm_head.weight") != std::string::npos;
}

bool GgufWeightLoader::supports(const std::string& path) const {
    return path.size() >= 5 && path.compare(path.size() - 5, 5, ".gguf") == 0;
}

GgufModelConfig GgufWeightLoader::config_from(const GgufFile& f) {
    // GGUFModelConfig::from_gguf_metadata (weight_loader_core.rs:35-98):
    // "{arch}.key" first, then the llama key.
    GgufModelConfig c;
    c.architecture = f.get_string("general.architecture", "llama");
    auto get = [&](const std::string& key) {
        return f.get_uint(c.architecture + "." + key, f.get_uint("llama." + key, 0));
    };
    c.hidden_size = get("embedding_length");
    c.intermediate_size = get("feed_forward_length");
    c.num_hidden_layers = get("block_count");
    c.num_attention_heads = get("attention.head_count");
    c.num_key_value_heads = f.get_uint(c.architecture + ".attention.head_count_kv",
                                       f.get_uint("llama.attention.head_count_kv",
                                                  c.num_attention_heads));
    c.vocab_size = get("vocab_size");
    if (c.vocab_size == 0)
        if (const GgufValue* t = f.find("tokenizer.ggml.tokens"))
            if (t->kind == GgufValue::ARRAY) c.vocab_size = t->items.size();
    c.head_dim = c.num_attention_heads ? c.hidden_size / c.num_attention_heads : 128;
    auto getf = [&](const std::string& key, double dflt) {
        return (float)f.get_float(c.architecture + "." + key, f.get_float("llama." + key, dflt));
    };
    c.rms_norm_eps = getf("attention.layer_norm_rms_epsilon", 1e-5);
    c.rope_theta = getf("rope.freq_base", 10000.0);
    c.max_position_embeddings = f.get_uint(c.architecture + ".context_length",
                                           f.get_uint("llama.context_length", 2048));
    return c;
}

std::vector<GgufWeightLoader::Plan> GgufWeightLoader::plan(const GgufFile& f) const {
    std::vector<Plan> out;
    for (const GgufTensorInfo& t : f.tensors()) {
        Plan p;
        p.gguf_name = t.name;
        p.hf_name = gguf_to_hf_name(t.name);
        p.shape = t.shape();
        p.type = t.type;
        p.quantized = is_quantized_weight_name(p.hf_name);
        out.push_back(std::move(p));
    }
    return out;
}

namespace {

// the types a projection keeps on the device: the block types, and the dense F32 / F16 /
// BF16 that candle's QMatMul::from_arc keeps as a dequantized f32 tensor
bool device_qtype(uint32_t t) {
    return t == GGML_Q4_0 || t == GGML_Q5_0 || t == GGML_Q8_0 || t == GGML_Q4_K ||
           t == GGML_Q5_K || t == GGML_Q6_K || t == GGML_F32 || t == GGML_F16 || t == GGML_BF16;
}

// The fusable groups of one layer: {fused hf name, part hf names}.
std::vector<std::pair<std::string, std::vector<std::string>>> fusion_groups(
    const std::string& layer, const LoadOptions& opt) {
    std::vector<std::pair<std::string, std::vector<std::string>>> g;
    if (opt.fuse_qkv)
        g.push_back({layer + "self_attn.qkv_proj.weight",
                     {layer + "self_attn.q_proj.weight", layer + "self_attn.k_proj.weight",
                      layer + "self_attn.v_proj.weight"}});
    if (opt.fuse_gate_up)
        g.push_back({layer + "mlp.gate_up_proj.weight",
                     {layer + "mlp.gate_proj.weight", layer + "mlp.up_proj.weight"}});
    return g;
}

}  // namespace

ModelWeights GgufWeightLoader::load_weights(const std::string& path,
                                            const LoadOptions& opt) const {
    const GgufFile f = GgufFile::open(path);
    ModelWeights w;
    w.config = config_from(f);
    std::map<std::string, const GgufTensorInfo*> by_hf;
    for (const GgufTensorInfo& t : f.tensors()) by_hf[gguf_to_hf_name(t.name)] = &t;

    // Fused projections: parts that share a type and k are concatenated row-wise
    // (GGUF rows are whole blocks, so the block bytes simply follow each other)
    // into one handle; the parts are then not loaded on their own.
    std::map<std::string, bool> fused_part;
    for (uint64_t L = 0; L < w.config.num_hidden_layers; ++L) {
        const std::string layer = "model.layers." + std::to_string(L) + ".";
        for (const auto& [fname, parts] : fusion_groups(layer, opt)) {
            std::vector<const GgufTensorInfo*> ts;
            for (const std::string& pn : parts) {
                auto it = by_hf.find(pn);
                if (it == by_hf.end()) break;
                ts.push_back(it->second);
            }
            if (ts.size() != parts.size()) continue;
            bool same = true;
            for (const GgufTensorInfo* t : ts)
                same = same && t->ne.size() == 2 && t->type == ts[0]->type &&
                       t->ne[0] == ts[0]->ne[0] && device_qtype(t->type);
            if (!same) continue;  // mixed types (a Q4_K_M layer): keep the parts apart
            std::vector<uint8_t> bytes;
            int64_t rows = 0;
            std::vector<std::pair<std::string, int64_t>> split;
            for (size_t i = 0; i < ts.size(); ++i) {
                const std::vector<uint8_t> b = f.read(*ts[i]);
                bytes.insert(bytes.end(), b.begin(), b.end());
                split.push_back({parts[i], (int64_t)ts[i]->ne[1]});
                rows += (int64_t)ts[i]->ne[1];
                fused_part[parts[i]] = true;
            }
            w.quantized_tensors[fname] = QuantLinear::from_blocks(
                (int)ts[0]->type, rows, (int64_t)ts[0]->ne[0], bytes.data(), bytes.size());
            w.fused_parts[fname] = std::move(split);
        }
    }

    for (const GgufTensorInfo& t : f.tensors()) {
        const std::string hf = gguf_to_hf_name(t.name);
        if (fused_part.count(hf)) continue;
        const std::vector<uint8_t> bytes = f.read(t);
        const std::vector<uint64_t> shp = t.shape();
        if (is_quantized_weight_name(hf)) {
            if (t.ne.size() != 2 || !device_qtype(t.type))
                throw Error("Failed to create QMatMul for '" + t.name + "': " +
                            ggml_type_name(t.type) + " " + std::to_string(t.ne.size()) +
                            "-D weights are not supported on the HIP device "
                            "(Q4_0 / Q5_0 / Q8_0 / Q4_K / Q5_K / Q6_K / F32 / F16 / BF16 "
                            "only)");
            w.quantized_tensors[hf] = QuantLinear::from_blocks(
                (int)t.type, (int64_t)t.ne[1], (int64_t)t.ne[0], bytes.data(), bytes.size());
            continue;
        }
        // embeddings, norms: dequantize to f32 on the host (weight_loader_core.rs:579)
        std::vector<int64_t> shape(shp.begin(), shp.end());
        int64_t elems = 1;
        for (int64_t d : shape) elems *= d;
        std::vector<float> v((size_t)elems);
        if (t.type == GGML_F32) {
            std::memcpy(v.data(), bytes.data(), v.size() * 4);
        } else if (t.type == GGML_F16 || t.type == GGML_BF16) {
            for (size_t i = 0; i < v.size(); ++i) {
                uint16_t h;
                std::memcpy(&h, bytes.data() + 2 * i, 2);
                v[i] = t.type == GGML_F16 ? half_to_float(h) : bf16_to_float(h);
            }
        } else if (device_qtype(t.type)) {
            const int64_t k = (int64_t)t.ne[0];
            const int64_t n = elems / k;
            auto q = QuantLinear::from_blocks((int)t.type, n, k, bytes.data(), bytes.size());
            v = q->dequantize().to_host();
        } else {
            throw Error("Failed to dequantize tensor '" + t.name + "': " +
                        ggml_type_name(t.type) + " is not supported by this build");
        }
        w.tensors[hf] = Tensor::from_host(v, shape, Device::cpu());
    }
    return w;
}

// ---- KV cache and decode attention --------------------------------------------------------------

namespace {
// the C ABI's message as is: it carries the reference's text ("KV cache append failed: ...")
void check_msg(int rc) {
    if (rc != UNILLM_OK) throw Error(unillm_hip_last_error());
}
}  // namespace

LayerKVCache LayerKVCache::with_capacity(int64_t n_kv_heads, int64_t head_dim,
                                         int64_t max_seq_len, float rope_theta) {
    LayerKVCache c;
    check_msg(unillm_hip_kv_cache_create(n_kv_heads, head_dim, max_seq_len, rope_theta, &c.c_));
    c.n_kv_heads_ = n_kv_heads;
    c.head_dim_ = head_dim;
    c.max_seq_ = max_seq_len;
    return c;
}

LayerKVCache::~LayerKVCache() {
    if (c_) unillm_hip_kv_cache_destroy(c_);
}

LayerKVCache::LayerKVCache(LayerKVCache&& o) noexcept
    : c_(o.c_), n_kv_heads_(o.n_kv_heads_), head_dim_(o.head_dim_), max_seq_(o.max_seq_) {
    o.c_ = nullptr;
}

LayerKVCache& LayerKVCache::operator=(LayerKVCache&& o) noexcept {
    if (this != &o) {
        if (c_) unillm_hip_kv_cache_destroy(c_);
        c_ = o.c_;
        n_kv_heads_ = o.n_kv_heads_;
        head_dim_ = o.head_dim_;
        max_seq_ = o.max_seq_;
        o.c_ = nullptr;
    }
    return *this;
}

int64_t LayerKVCache::seq_len() const {
    int64_t n = 0;
    check_msg(unillm_hip_kv_cache_length(c_, &n));
    return n;
}

void LayerKVCache::clear() { check_msg(unillm_hip_kv_cache_clear(c_)); }

void LayerKVCache::truncate(int64_t len) { check_msg(unillm_hip_kv_cache_truncate(c_, len)); }

Tensor LayerKVCache::attend(const Tensor& qkv, int64_t n_heads, void* stream) {
    if (!qkv.device().is_hip() || qkv.shape().size() != 2)
        throw Error("attention: qkv must be a [m, (n_heads + 2 n_kv_heads) head_dim] HIP tensor");
    Tensor out = Tensor::empty({qkv.dim(0), n_heads * head_dim_}, qkv.device());
    attend_into(qkv, n_heads, out, stream);
    return out;
}

void LayerKVCache::attend_into(const Tensor& qkv, int64_t n_heads, Tensor& out, void* stream) {
    if (!qkv.device().is_hip() || qkv.shape().size() != 2)
        throw Error("attention: qkv must be a [m, (n_heads + 2 n_kv_heads) head_dim] HIP tensor");
    if (n_heads < 1 || qkv.dim(-1) != (n_heads + 2 * n_kv_heads_) * head_dim_)
        throw Error("attention: qkv width " + std::to_string(qkv.dim(-1)) + " is not (" +
                    std::to_string(n_heads) + " + 2 x " + std::to_string(n_kv_heads_) + ") x " +
                    std::to_string(head_dim_));
    const int64_t m = qkv.dim(0);
    if (!out.device().is_hip() || out.numel() != m * n_heads * head_dim_)
        throw Error("attention: out must be a HIP tensor of [m, n_heads head_dim]");
    check_msg(unillm_hip_attention_decode(c_, qkv.data(), m, n_heads, out.data_mut(), stream));
}

KVCache KVCache::with_capacity(size_t num_layers, int64_t n_kv_heads, int64_t head_dim,
                               int64_t max_seq_len, float rope_theta) {
    KVCache c;
    c.layers_.reserve(num_layers);
    for (size_t i = 0; i < num_layers; ++i)
        c.layers_.push_back(LayerKVCache::with_capacity(n_kv_heads, head_dim, max_seq_len, rope_theta));
    return c;
}

LayerKVCache& KVCache::layer_mut(size_t i) {
    if (i >= layers_.size()) throw Error("layer index out of range");
    return layers_[i];
}

const LayerKVCache& KVCache::layer(size_t i) const {
    if (i >= layers_.size()) throw Error("layer index out of range");
    return layers_[i];
}

int64_t KVCache::seq_len() const { return layers_.empty() ? 0 : layers_[0].seq_len(); }

int64_t KVCache::max_seq_len() const { return layers_.empty() ? 0 : layers_[0].max_seq_len(); }

void KVCache::clear() {
    for (auto& l : layers_) l.clear();
}

// ---- LlamaModel ----------------------------------------------------------------------------
LlamaModel::LlamaModel(ModelWeights weights) : w_(std::move(weights)) {
    const GgufModelConfig& c = w_.config;
    if (c.num_attention_heads == 0 || c.num_key_value_heads == 0 ||
        c.hidden_size % c.num_attention_heads != 0 ||
        c.num_attention_heads % c.num_key_value_heads != 0)
        throw Error("LlamaModel: hidden_size, head_count and head_count_kv do not make heads");
    hidden_ = (int64_t)c.hidden_size;
    heads_ = (int64_t)c.num_attention_heads;
    kv_heads_ = (int64_t)c.num_key_value_heads;
    head_dim_ = hidden_ / heads_;
    auto host = [&](const std::string& name) -> const Tensor& {
        auto it = w_.tensors.find(name);
        if (it == w_.tensors.end()) throw Error("LlamaModel: missing weight " + name);
        return it->second;
    };
    auto vec = [&](const std::string& name) {
        const Tensor& t = host(name);
        if (t.numel() != hidden_)
            throw Error("LlamaModel: " + name + " has " + std::to_string(t.numel()) +
                        " elements, not hidden_size " + std::to_string(hidden_));
        return t.to_device(Device::hip(0));
    };
    auto proj = [&](const std::string& name, int64_t n, int64_t k) {
        std::shared_ptr<QuantLinear> q = w_.get_quantized(name);
        if (!q) throw Error("LlamaModel: missing quantized weight " + name);
        if (q->n() != n || q->k() != k)
            throw Error("LlamaModel: " + name + " is [" + std::to_string(q->n()) + ", " +
                        std::to_string(q->k()) + "], not [" + std::to_string(n) + ", " +
                        std::to_string(k) + "]");
        return q;
    };
    embed_ = host("model.embed_tokens.weight");
    if (embed_.shape().size() != 2 || embed_.dim(1) != hidden_)
        throw Error("LlamaModel: model.embed_tokens.weight is not [vocab, hidden_size]");
    const int64_t kvw = kv_heads_ * head_dim_, inter = (int64_t)c.intermediate_size;
    for (uint64_t L = 0; L < c.num_hidden_layers; ++L) {
        const std::string p = "model.layers." + std::to_string(L) + ".";
        Layer l;
        l.in_norm = vec(p + "input_layernorm.weight");
        l.post_norm = vec(p + "post_attention_layernorm.weight");
        if (w_.get_quantized(p + "self_attn.qkv_proj.weight")) {
            l.qkv = proj(p + "self_attn.qkv_proj.weight", hidden_ + 2 * kvw, hidden_);
        } else {
            l.q = proj(p + "self_attn.q_proj.weight", hidden_, hidden_);
            l.k = proj(p + "self_attn.k_proj.weight", kvw, hidden_);
            l.v = proj(p + "self_attn.v_proj.weight", kvw, hidden_);
        }
        l.o = proj(p + "self_attn.o_proj.weight", hidden_, hidden_);
        if (!w_.get_quantized(p + "mlp.gate_up_proj.weight"))
            throw Error("LlamaModel: layer " + std::to_string(L) +
                        " has no fused gate_up handle (load with LoadOptions::fuse_gate_up)");
        l.gate_up = proj(p + "mlp.gate_up_proj.weight", 2 * inter, hidden_);
        l.down = proj(p + "mlp.down_proj.weight", hidden_, inter);
        layers_.push_back(std::move(l));
    }
    norm_ = vec("model.norm.weight");
    lm_head_ = w_.get_quantized("lm_head.weight");
    if (!lm_head_ || lm_head_->k() != hidden_)
        throw Error("LlamaModel: missing quantized lm_head.weight [vocab, hidden_size]");
}

LlamaModel LlamaModel::load(const std::string& gguf_path) {
    LoadOptions opt;
    opt.fuse_qkv = opt.fuse_gate_up = true;
    return LlamaModel(GgufWeightLoader().load_weights(gguf_path, opt));
}

KVCache LlamaModel::new_cache(int64_t max_seq_len) const {
    return KVCache::with_capacity(layers_.size(), kv_heads_, head_dim_, max_seq_len,
                                  w_.config.rope_theta);
}

std::vector<float> LlamaModel::embed_rows(const std::vector<int32_t>& input_ids) const {
    const int64_t m = (int64_t)input_ids.size(), vocab = embed_.dim(0);
    std::vector<float> rows((size_t)(m * hidden_));
    const float* table = embed_.data();
    for (int64_t t = 0; t < m; ++t) {
        const int32_t id = input_ids[(size_t)t];
        if (id < 0 || id >= vocab)
            throw Error("forward_with_cache: token id " + std::to_string(id) + " outside [0, " +
                        std::to_string(vocab) + ")");
        std::copy(table + (int64_t)id * hidden_, table + ((int64_t)id + 1) * hidden_,
                  rows.begin() + t * hidden_);
    }
    return rows;
}

LlamaModel::StepBuffers LlamaModel::step_buffers(int64_t m) const {
    const Device d = Device::hip(0);
    StepBuffers b;
    b.m = m;
    b.h = Tensor::empty({m, hidden_}, d);
    b.qkv = Tensor::empty({m, hidden_ + 2 * kv_heads_ * head_dim_}, d);
    b.att = Tensor::empty({m, hidden_}, d);
    b.act = Tensor::empty({m, (int64_t)w_.config.intermediate_size}, d);
    b.logits = Tensor::empty({m, lm_head_->n()}, d);
    return b;
}

void LlamaModel::forward_layers(StepBuffers& b, KVCache& cache, void* stream) const {
    const int64_t m = b.m;
    if (cache.num_layers() != layers_.size())
        throw Error("forward_with_cache: the cache has " + std::to_string(cache.num_layers()) +
                    " layers, the model " + std::to_string(layers_.size()));
    // 2. the decoder layers (llama.rs:654-680)
    const int64_t kvw = kv_heads_ * head_dim_, width = hidden_ + 2 * kvw;
    float* h = b.h.data_mut();
    for (size_t L = 0; L < layers_.size(); ++L) {
        const Layer& l = layers_[L];
        if (l.qkv) {  // input_layernorm fused into the q/k/v projection
            check_qmatmul(unillm_hip_qmatmul_norm(l.qkv->handle(), h, l.in_norm.data(), nullptr,
                                                  1e-6f, m, b.qkv.data_mut(), stream),
                          "QMatMul forward failed");
        } else {  // parts of different GGUF types: each part into its columns, a row at a time
            const std::pair<const QuantLinear*, int64_t> parts[3] = {
                {l.q.get(), 0}, {l.k.get(), hidden_}, {l.v.get(), hidden_ + kvw}};
            for (int64_t t = 0; t < m; ++t)
                for (const auto& [q, off] : parts)
                    check_qmatmul(unillm_hip_qmatmul_norm(q->handle(), h + t * hidden_,
                                                          l.in_norm.data(), nullptr, 1e-6f, 1,
                                                          b.qkv.data_mut() + t * width + off,
                                                          stream),
                                  "QMatMul forward failed");
        }
        cache.layer_mut(L).attend_into(b.qkv, heads_, b.att, stream);
        check_qmatmul(unillm_hip_qmatmul_add(l.o->handle(), b.att.data(), m, h, stream),
                      "QMatMul forward failed");
        check_qmatmul(unillm_hip_qmatmul_norm_swiglu(l.gate_up->handle(), h, l.post_norm.data(),
                                                     nullptr, 1e-6f, m, b.act.data_mut(), stream),
                      "QMatMul forward failed");
        check_qmatmul(unillm_hip_qmatmul_add(l.down->handle(), b.act.data(), m, h, stream),
                      "QMatMul forward failed");
    }
    // 3. final norm fused into the head (lm_head_forward's error context, llama.rs:399)
    check_qmatmul(unillm_hip_qmatmul_norm(lm_head_->handle(), h, norm_.data(), nullptr,
                                          w_.config.rms_norm_eps, m, b.logits.data_mut(), stream),
                  "QMatMul lm_head forward failed");
}

Tensor LlamaModel::forward_with_cache(const std::vector<int32_t>& input_ids, KVCache& cache,
                                      void* stream) const {
    const int64_t m = (int64_t)input_ids.size();
    if (m == 0) throw Error("forward_with_cache: no input tokens");
    if (cache.num_layers() != layers_.size())
        throw Error("forward_with_cache: the cache has " + std::to_string(cache.num_layers()) +
                    " layers, the model " + std::to_string(layers_.size()));
    // 1. token embedding (ops_fn::embedding: rows of the table); the outputs are
    // freshly allocated per call, as the reference's are
    const std::vector<float> rows = embed_rows(input_ids);
    StepBuffers b = step_buffers(m);
    b.h = Tensor::from_host(rows, {m, hidden_}, Device::hip(0));
    forward_layers(b, cache, stream);
    return b.logits;
}

// ---- CapturedDecodeStep --------------------------------------------------------------------
CapturedDecodeStep::CapturedDecodeStep(const LlamaModel& model, KVCache& cache)
    : model_(model), b_(model.step_buffers(1)) {
    if (cache.num_layers() != model.layers_.size())
        throw Error("CapturedDecodeStep: the cache has " + std::to_string(cache.num_layers()) +
                    " layers, the model " + std::to_string(model.layers_.size()));
    check_msg(unillm_hip_stream_create(&stream_));
    try {
        // a capture cannot allocate: every call's workspace is grown first, on this stream
        for (size_t L = 0; L < model.layers_.size(); ++L) {
            const LlamaModel::Layer& l = model.layers_[L];
            for (const auto* q : {l.qkv.get(), l.q.get(), l.k.get(), l.v.get(), l.o.get(),
                                  l.down.get()})
                if (q) check_msg(unillm_hip_qmatmul_reserve(q->handle(), 1, 0, stream_));
            check_msg(unillm_hip_qmatmul_reserve(l.gate_up->handle(), 1, 1, stream_));
            check_msg(unillm_hip_attention_reserve(cache.layer(L).handle(), 1, model.heads_,
                                                   stream_));
        }
        check_msg(unillm_hip_qmatmul_reserve(model.lm_head_->handle(), 1, 0, stream_));
        check_msg(unillm_hip_stream_synchronize(stream_));
        check_msg(unillm_hip_graph_begin(stream_));
        try {
            model.forward_layers(b_, cache, stream_);
        } catch (...) {
            unillm_graph* g = nullptr;  // end the failed capture; its graph is discarded
            if (unillm_hip_graph_end(stream_, &g) == UNILLM_OK) unillm_hip_graph_destroy(g);
            throw;
        }
        check_msg(unillm_hip_graph_end(stream_, &graph_));
    } catch (...) {
        unillm_hip_stream_destroy(stream_);
        throw;
    }
}

CapturedDecodeStep::~CapturedDecodeStep() {
    if (stream_) unillm_hip_stream_synchronize(stream_);
    unillm_hip_graph_destroy(graph_);
    unillm_hip_stream_destroy(stream_);
}

const Tensor& CapturedDecodeStep::run(int32_t token) {
    const std::vector<float> row = model_.embed_rows({token});
    // the previous replay reads and rewrites h: it must be done before the new row lands
    check_msg(unillm_hip_stream_synchronize(stream_));
    check_msg(unillm_hip_memcpy_htod(b_.h.data_mut(), row.data(), row.size() * sizeof(float)));
    check_msg(unillm_hip_graph_launch(graph_, stream_));
    check_msg(unillm_hip_stream_synchronize(stream_));
    return b_.logits;
}

}  // namespace unillm
