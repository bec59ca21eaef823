// test_host.cpp -- tests of the C++ host layer (unillm_amd/host), run by
// tests/test_host_cpp.py.
//
//   test_host cpu <file.gguf> <file.expect>      parsing, name map, plan, errors
//   test_host gpu <file.gguf> <file.expect>      load to the device + forward parity
//   test_host cpu-kq / gpu-kq <q4_k_m.gguf> <.expect>   the Q4_K / Q6_K file (or the
//                                                 Q5_K / Q6_K one): plan, parity, QKV
//                                                 and gate+up fusion
//   test_host gpu-step <file.gguf> <file.step>   LlamaModel::forward_with_cache logits,
//                                                 eager and as a captured decode step
//
// The .gguf / .expect pairs are written by tests/golden/make_gguf.py.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <map>
#include <string>
#include <vector>

#include "../../unillm_amd/host/unillm_host.hpp"

using namespace unillm;

static int g_fail = 0, g_pass = 0;

#define CHECK(cond)                                                                     \
    do {                                                                                \
        if (cond) {                                                                     \
            ++g_pass;                                                                   \
        } else {                                                                        \
            ++g_fail;                                                                   \
            std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);        \
        }                                                                               \
    } while (0)

template <typename F>
static bool throws_with(F&& f, const std::string& needle) {
    try {
        f();
    } catch (const std::exception& e) {
        if (std::string(e.what()).find(needle) != std::string::npos) return true;
        std::fprintf(stderr, "  unexpected message: %s\n", e.what());
        return false;
    }
    return false;
}

struct Expect {
    std::string gguf_name, hf_name;
    uint32_t type, quantized, m, n, k;
    std::vector<float> x;
    std::vector<double> y;
};

static std::vector<Expect> read_expect(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    auto u32 = [&]() {
        uint32_t v;
        f.read(reinterpret_cast<char*>(&v), 4);
        return v;
    };
    auto str = [&]() {
        std::string s(u32(), '\0');
        f.read(s.data(), (std::streamsize)s.size());
        return s;
    };
    char magic[4];
    f.read(magic, 4);
    if (std::memcmp(magic, "UXPT", 4) != 0) throw std::runtime_error("bad expect file");
    std::vector<Expect> out(u32());
    for (Expect& e : out) {
        e.gguf_name = str();
        e.hf_name = str();
        e.type = u32();
        e.quantized = u32();
        e.m = u32();
        e.n = u32();
        e.k = u32();
        e.x.resize((size_t)e.m * e.k);
        e.y.resize((size_t)e.m * e.n);
        f.read(reinterpret_cast<char*>(e.x.data()), (std::streamsize)(e.x.size() * 4));
        f.read(reinterpret_cast<char*>(e.y.data()), (std::streamsize)(e.y.size() * 8));
    }
    if (!f) throw std::runtime_error("truncated expect file");
    return out;
}

static std::string write_tmp(const std::string& name, const std::vector<char>& bytes) {
    const std::string path = "/tmp/unillm_host_test_" + name;
    std::ofstream o(path, std::ios::binary);
    o.write(bytes.data(), (std::streamsize)bytes.size());
    return path;
}

static std::vector<char> slurp(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    return std::vector<char>(std::istreambuf_iterator<char>(f), {});
}

static void test_cpu(const std::string& gguf, const std::vector<Expect>& ex) {
    // name map: the reference's own examples and its ordering hazards
    CHECK(gguf_to_hf_name("blk.3.attn_output.weight") == "model.layers.3.self_attn.o_proj.weight");
    CHECK(gguf_to_hf_name("output.weight") == "lm_head.weight");
    CHECK(gguf_to_hf_name("output_norm.weight") == "model.norm.weight");
    CHECK(gguf_to_hf_name("token_embd.weight") == "model.embed_tokens.weight");
    CHECK(gguf_to_hf_name("blk.0.ffn_down.weight") == "model.layers.0.mlp.down_proj.weight");
    CHECK(gguf_to_hf_name("blk.12.attn_norm.weight") ==
          "model.layers.12.input_layernorm.weight");
    CHECK(is_quantized_weight_name("model.layers.0.mlp.up_proj.weight"));
    CHECK(is_quantized_weight_name("lm_head.weight"));
    CHECK(!is_quantized_weight_name("model.embed_tokens.weight"));
    CHECK(!is_quantized_weight_name("model.layers.0.input_layernorm.weight"));

    const GgufFile f = GgufFile::open(gguf);
    CHECK(f.version() == 3);
    CHECK(f.alignment() == 32);
    CHECK(f.data_offset() % 32 == 0);
    CHECK(f.tensors().size() == ex.size());
    const GgufModelConfig c = GgufWeightLoader::config_from(f);
    CHECK(c.architecture == "llama");
    CHECK(c.hidden_size == 128 && c.intermediate_size == 96 && c.num_hidden_layers == 2);
    CHECK(c.num_attention_heads == 2 && c.num_key_value_heads == 1 && c.head_dim == 64);
    CHECK(c.vocab_size == 8);  // from tokenizer.ggml.tokens
    // GGUFModelConfig::from_gguf_metadata's float keys (weight_loader_core.rs:72-82)
    CHECK(c.rms_norm_eps == 1e-5f && c.rope_theta == 20000.0f);
    CHECK(c.max_position_embeddings == 2048);  // no context_length key: the default

    GgufWeightLoader loader;
    CHECK(loader.supports("model.gguf") && !loader.supports("model.safetensors"));
    const auto plan = loader.plan(f);
    size_t nq = 0;
    for (size_t i = 0; i < plan.size() && i < ex.size(); ++i) {
        CHECK(plan[i].gguf_name == ex[i].gguf_name);
        CHECK(plan[i].hf_name == ex[i].hf_name);
        CHECK(plan[i].type == ex[i].type);
        CHECK(plan[i].quantized == (ex[i].quantized != 0));
        if (plan[i].quantized) {
            ++nq;
            CHECK(plan[i].shape.size() == 2 && plan[i].shape[0] == ex[i].n &&
                  plan[i].shape[1] == ex[i].k);  // ne reversed: [n, k]
        }
    }
    CHECK(nq == 2 * 7 + 1);  // 7 projections per layer + lm_head

    // raw bytes of a Q4_0 tensor: 18 B per block
    const GgufTensorInfo* q = nullptr;
    for (const auto& t : f.tensors())
        if (t.name == "blk.0.attn_q.weight") q = &t;
    CHECK(q && q->type == GGML_Q4_0 && q->nbytes == 128 * 4 * 18);
    if (q) CHECK(f.read(*q).size() == q->nbytes);

    // malformed files
    std::vector<char> bytes = slurp(gguf);
    std::vector<char> bad = bytes;
    bad[0] = 'X';
    CHECK(throws_with([&] { GgufFile::open(write_tmp("magic.gguf", bad)); }, "bad magic"));
    bad = bytes;
    bad[4] = 7;  // version 7
    CHECK(throws_with([&] { GgufFile::open(write_tmp("ver.gguf", bad)); }, "version"));
    std::vector<char> cut(bytes.begin(), bytes.begin() + (long)bytes.size() / 2);
    CHECK(throws_with([&] { GgufFile::open(write_tmp("cut.gguf", cut)); }, "past the end"));
    std::vector<char> hdr(bytes.begin(), bytes.begin() + 40);
    CHECK(throws_with([&] { GgufFile::open(write_tmp("hdr.gguf", hdr)); }, "end of file"));
    CHECK(throws_with([&] { GgufFile::open("/nonexistent/x.gguf"); }, "cannot open"));
    // a header declaring one metadata array of 2^31 one-byte items over a few MB of
    // file: each parsed item costs far more memory than its byte, so the reader
    // must run out of file (GgufError), not out of memory (bad_alloc)
    {
        std::vector<char> h;
        auto put = [&](const void* p, size_t n) {
            const char* c = static_cast<const char*>(p);
            h.insert(h.end(), c, c + n);
        };
        const uint32_t ver = 3, t_arr = 9, t_u8 = 0;
        const uint64_t n_tensors = 0, n_kv = 1, klen = 3, count = 1ull << 31;
        put("GGUF", 4);
        put(&ver, 4);
        put(&n_tensors, 8);
        put(&n_kv, 8);
        put(&klen, 8);
        put("arr", 3);
        put(&t_arr, 4);
        put(&t_u8, 4);
        put(&count, 8);
        h.resize(h.size() + (4u << 20), 1);  // 4 MiB of items, far short of the count
        CHECK(throws_with([&] { GgufFile::open(write_tmp("huge_array.gguf", h)); },
                          "array length"));
        // 2^22 two-byte items: a count the remaining bytes pass, twice the bytes they
        // hold: parsed item by item (the reserve stays bounded) until the file ends
        const uint32_t t_u16 = 2;
        const uint64_t fits = 4u << 20;
        std::memcpy(h.data() + 4 + 4 + 8 + 8 + 8 + 3 + 4, &t_u16, 4);
        std::memcpy(h.data() + 4 + 4 + 8 + 8 + 8 + 3 + 4 + 4, &fits, 8);
        CHECK(throws_with([&] { GgufFile::open(write_tmp("short_array.gguf", h)); },
                          "end of file"));
    }

    // shape rules of QMatMul::forward are checked before any device work
    Device d = Device::hip(0);
    CHECK(d.to_string() == "HIP(0)" && d != Device::cpu());
}

static double normwise(const std::vector<float>& y, const std::vector<double>& r) {
    double num = 0, den = 0;
    for (size_t i = 0; i < r.size(); ++i) {
        num = std::max(num, std::fabs((double)y[i] - r[i]));
        den = std::max(den, std::fabs(r[i]));
    }
    return den > 0 ? num / den : num;
}

static void test_gpu_kv();

static void test_gpu(const std::string& gguf, const std::vector<Expect>& ex) {
    GgufWeightLoader loader;
    const ModelWeights w = loader.load_weights(gguf);
    CHECK(w.quantized_tensors.size() == 15);
    CHECK(w.get_quantized("model.layers.1.mlp.down_proj.weight") != nullptr);
    CHECK(w.get_quantized("model.embed_tokens.weight") == nullptr);
    CHECK(w.tensors.count("model.embed_tokens.weight") == 1);
    CHECK(w.tensors.at("model.embed_tokens.weight").shape() == std::vector<int64_t>({128, 128}));
    HipTensorOps ops;
    for (const Expect& e : ex) {
        if (!e.quantized) continue;
        auto q = w.get_quantized(e.hf_name);
        CHECK(q != nullptr);
        if (!q) continue;
        CHECK(q->n() == (int64_t)e.n && q->k() == (int64_t)e.k);
        const Tensor x = Tensor::from_host(e.x, {(int64_t)e.m, (int64_t)e.k}, Device::hip(0));
        const std::vector<float> y = q->forward(x).to_host();
        const double err = normwise(y, e.y);
        if (err >= 1e-3) std::fprintf(stderr, "  %s: normwise %.3g\n", e.hf_name.c_str(), err);
        CHECK(err < 1e-3);
        // TensorOps dispatch gives the same answer; a 3-D input keeps its leading dims
        const std::vector<float> y2 = ops.matmul(x, *q).to_host();
        CHECK(y2 == y);
        const Tensor x3 = x.reshape({1, (int64_t)e.m, (int64_t)e.k});
        const Tensor y3 = q->forward(x3);
        CHECK(y3.shape() == std::vector<int64_t>({1, (int64_t)e.m, (int64_t)e.n}));
    }
    auto q = w.get_quantized("lm_head.weight");
    CHECK(throws_with([&] { q->forward(Tensor::empty({3, 32}, Device::hip(0))); },
                      "QMatMul forward failed: input last dim 32"));
    CHECK(throws_with([&] { q->forward(Tensor::empty({64}, Device::hip(0))); },
                      "QMatMul forward failed: rank 1"));
    CHECK(throws_with([&] { q->forward(Tensor::empty({2, 128}, Device::cpu())); },
                      "QMatMul forward failed: input is on CPU"));
    // lm_head_forward (llama.rs:396-405): the same result, the reference's lm_head context
    {
        const Tensor h = Tensor::from_host(std::vector<float>(2 * 128, 0.25f), {2, 128},
                                           Device::hip(0));
        CHECK(lm_head_forward(*q, h).to_host() == q->forward(h).to_host());
        CHECK(throws_with([&] { lm_head_forward(*q, Tensor::empty({3, 32}, Device::hip(0))); },
                          "QMatMul lm_head forward failed: input last dim 32"));
    }
    test_gpu_kv();
}

// LlamaModel::forward_with_cache (llama.rs:421-462) on the tiny Q4_0 model: three calls
// on one cache (a 12-token prompt -- the prompt-length attention kernels -- then two
// single tokens -- the decode kernels), logits against the f64 chain of the .step
// file at 1e-3 normwise per call.  Both the fused-qkv load and the unfused one (q, k, v
// a token at a time) are run; they must agree with each other as well.
static void test_gpu_step(const std::string& gguf, const std::string& step_path) {
    std::ifstream f(step_path, std::ios::binary);
    char magic[4];
    f.read(magic, 4);
    CHECK(f && std::memcmp(magic, "USTP", 4) == 0);
    uint32_t vocab = 0, nsteps = 0;
    f.read(reinterpret_cast<char*>(&vocab), 4);
    f.read(reinterpret_cast<char*>(&nsteps), 4);
    std::vector<std::vector<int32_t>> ids(nsteps);
    std::vector<std::vector<double>> ref(nsteps);
    for (uint32_t s = 0; s < nsteps; ++s) {
        uint32_t m = 0;
        f.read(reinterpret_cast<char*>(&m), 4);
        ids[s].resize(m);
        ref[s].resize((size_t)m * vocab);
        f.read(reinterpret_cast<char*>(ids[s].data()), (std::streamsize)(m * 4));
        f.read(reinterpret_cast<char*>(ref[s].data()), (std::streamsize)(ref[s].size() * 8));
    }
    CHECK((bool)f);
    if (!f) return;

    const LlamaModel fused = LlamaModel::load(gguf);
    LoadOptions only_gate_up;
    only_gate_up.fuse_gate_up = true;
    const LlamaModel split(GgufWeightLoader().load_weights(gguf, only_gate_up));
    CHECK(fused.vocab_size() == (int64_t)vocab && fused.config().rope_theta == 20000.0f);
    KVCache c1 = fused.new_cache(64), c2 = split.new_cache(64);
    int64_t len = 0;
    for (uint32_t s = 0; s < nsteps; ++s) {
        const std::vector<float> a = fused.forward_with_cache(ids[s], c1).to_host();
        const std::vector<float> b = split.forward_with_cache(ids[s], c2).to_host();
        len += (int64_t)ids[s].size();
        const double ea = normwise(a, ref[s]), eb = normwise(b, ref[s]);
        std::printf("  step %u (m = %zu): normwise %.3g fused, %.3g unfused\n", s, ids[s].size(),
                    ea, eb);
        CHECK(ea < 1e-3 && eb < 1e-3);
        CHECK(c1.seq_len() == len && c2.seq_len() == len);
    }
    // The single tokens again through a captured decode step (the loop of
    // generate_with_cache, llama.rs:525-559): the prompt eagerly, then one HIP graph
    // captured once and replayed per token, each replay appending at the next position
    // of every layer's cache.  Then the last token rolled back and run eagerly: the
    // same logits.
    for (const LlamaModel* model : {&fused, &split}) {
        KVCache c = model->new_cache(64);
        model->forward_with_cache(ids[0], c);
        int64_t n = (int64_t)ids[0].size();
        CapturedDecodeStep step(*model, c);
        CHECK(c.seq_len() == n);  // capturing runs nothing
        std::vector<float> last;
        for (uint32_t s = 1; s < nsteps; ++s) {
            CHECK(ids[s].size() == 1);
            last = step.run(ids[s][0]).to_host();
            ++n;
            const double e = normwise(last, ref[s]);
            std::printf("  captured step %u: normwise %.3g (%s)\n", s, e,
                        model == &fused ? "fused" : "unfused");
            CHECK(e < 1e-3);
            CHECK(c.seq_len() == n);
            for (size_t L = 0; L < c.num_layers(); ++L) CHECK(c.layer(L).seq_len() == n);
        }
        for (size_t L = 0; L < c.num_layers(); ++L) c.layer_mut(L).truncate(n - 1);
        const std::vector<float> eager =
            model->forward_with_cache({ids[nsteps - 1][0]}, c).to_host();
        const std::vector<double> last64(last.begin(), last.end());
        CHECK(normwise(eager, last64) < 1e-5);
        CHECK(c.seq_len() == n);
    }
    // argument errors
    CHECK(throws_with([&] { fused.forward_with_cache({}, c1); }, "no input tokens"));
    CHECK(throws_with([&] { fused.forward_with_cache({128}, c1); }, "token id 128 outside"));
    KVCache one = KVCache::with_capacity(1, 1, 64, 8);
    CHECK(throws_with([&] { fused.forward_with_cache({1}, one); }, "the cache has 1 layers"));
    KVCache small = fused.new_cache(4);
    CHECK(throws_with([&] { fused.forward_with_cache({1, 2, 3, 4, 5}, small); },
                      "KV cache overflow"));
    LoadOptions none;
    CHECK(throws_with([&] { LlamaModel(GgufWeightLoader().load_weights(gguf, none)); },
                      "no fused gate_up handle"));
}

// LayerKVCache / KVCache (kv_cache.rs) and LayerKVCache::attend (forward_with_cache
// after the projections) through the C ABI: closed forms (one position returns its
// v exactly; zero keys average the visible values), the length bookkeeping, and the
// reference's overflow message.  The kernel's parity with the oracle over random
// inputs is tested from Python (tests/test_gpu_attention.py).
static void test_gpu_kv() {
    const int64_t H = 4, KVH = 2, D = 64, W = (H + 2 * KVH) * D;
    auto row = [&](std::vector<float>& q, int64_t t, int64_t part, int64_t head, int64_t d) -> float& {
        // part 0 = q heads, 1 = k heads, 2 = v heads
        const int64_t off = part == 0 ? head * D : part == 1 ? (H + head) * D : (H + KVH + head) * D;
        return q[(size_t)(t * W + off + d)];
    };
    {
        LayerKVCache c = LayerKVCache::with_capacity(KVH, D, 8);
        CHECK(c.is_empty() && c.seq_len() == 0 && c.max_seq_len() == 8);
        std::vector<float> qkv((size_t)W);
        for (size_t i = 0; i < qkv.size(); ++i) qkv[i] = (float)((i * 37 % 101) - 50) / 16.0f;
        const std::vector<float> out =
            c.attend(Tensor::from_host(qkv, {1, W}, Device::hip(0)), H).to_host();
        CHECK(c.seq_len() == 1);
        bool exact = out.size() == (size_t)(H * D);
        for (int64_t h = 0; h < H && exact; ++h)  // head h reads kv head h / (H / KVH)
            for (int64_t d = 0; d < D; ++d)
                exact = exact && out[(size_t)(h * D + d)] == row(qkv, 0, 2, h / (H / KVH), d);
        CHECK(exact);
        c.truncate(0);
        CHECK(c.is_empty());
    }
    {
        // three tokens with zero keys: token t sees positions 0 .. t, all scores 0
        LayerKVCache c = LayerKVCache::with_capacity(KVH, D, 3);
        std::vector<float> qkv((size_t)(3 * W), 0.0f);
        for (int64_t t = 0; t < 3; ++t)
            for (int64_t g = 0; g < KVH; ++g)
                for (int64_t d = 0; d < D; ++d) {
                    row(qkv, t, 0, 2 * g, d) = 1.0f + (float)d;  // queries: anything
                    row(qkv, t, 2, g, d) = (float)(t * 100 + g * 10) + (float)d / 8.0f;
                }
        const std::vector<float> out =
            c.attend(Tensor::from_host(qkv, {3, W}, Device::hip(0)), H).to_host();
        double worst = 0;
        for (int64_t t = 0; t < 3; ++t)
            for (int64_t h = 0; h < H; ++h)
                for (int64_t d = 0; d < D; ++d) {
                    double mean = 0;
                    for (int64_t j = 0; j <= t; ++j) mean += row(qkv, j, 2, h / 2, d);
                    mean /= (double)(t + 1);
                    worst = std::max(worst, std::fabs(out[(size_t)((t * H + h) * D + d)] - mean) /
                                                std::max(1.0, std::fabs(mean)));
                }
        CHECK(worst < 1e-6);
        CHECK(c.seq_len() == 3);
        // full: one more position is the reference's overflow error, and nothing changes
        CHECK(throws_with([&] { c.attend(Tensor::from_host(qkv, {3, W}, Device::hip(0)).reshape({3, W}), H); },
                          "KV cache append failed: KV cache overflow"));
        CHECK(c.seq_len() == 3);
        CHECK(throws_with([&] { c.attend(Tensor::empty({1, W - D}, Device::hip(0)), H); },
                          "attention: qkv width"));
        c.clear();
        CHECK(c.is_empty() && c.max_seq_len() == 3);
    }
    {
        KVCache kv = KVCache::with_capacity(3, KVH, D, 16);
        CHECK(kv.num_layers() == 3 && kv.max_seq_len() == 16 && kv.is_empty());
        std::vector<float> qkv((size_t)(2 * W), 0.5f);
        kv.layer_mut(0).attend(Tensor::from_host(qkv, {2, W}, Device::hip(0)), H);
        kv.layer_mut(2).attend(Tensor::from_host(qkv, {2, W}, Device::hip(0)), H);
        CHECK(kv.seq_len() == 2 && kv.layer(1).seq_len() == 0 && kv.layer(2).seq_len() == 2);
        kv.clear();
        CHECK(kv.is_empty() && kv.layer(2).seq_len() == 0);
        CHECK(throws_with([&] { kv.layer_mut(3); }, "layer index out of range"));
    }
}

// Dense projections (tiny_llama_f16: F16, layer 0's o_proj F32, layer 1's down_proj
// BF16), the variant candle's QMatMul::from_arc keeps as a dequantized f32 tensor:
// every projection and lm_head against the f64 expectations at 1e-5 (an f32 GEMM of
// the exactly widened weights), the types kept, and same-typed groups fused at load.
static void test_gpu_dense(const std::string& gguf, const std::vector<Expect>& ex) {
    GgufWeightLoader loader;
    const ModelWeights w = loader.load_weights(gguf);
    CHECK(w.quantized_tensors.size() == 15);
    CHECK(w.get_quantized("model.layers.0.self_attn.o_proj.weight")->qtype() == GGML_F32);
    CHECK(w.get_quantized("model.layers.1.mlp.down_proj.weight")->qtype() == GGML_BF16);
    CHECK(w.get_quantized("lm_head.weight")->qtype() == GGML_F16);
    CHECK(w.tensors.at("model.embed_tokens.weight").shape() == std::vector<int64_t>({128, 128}));
    std::map<std::string, std::vector<float>> ys;
    for (const Expect& e : ex) {
        if (!e.quantized) continue;
        auto q = w.get_quantized(e.hf_name);
        CHECK(q != nullptr);
        if (!q) continue;
        const Tensor x = Tensor::from_host(e.x, {(int64_t)e.m, (int64_t)e.k}, Device::hip(0));
        ys[e.hf_name] = q->forward(x).to_host();
        const double err = normwise(ys[e.hf_name], e.y);
        if (err >= 1e-5) std::fprintf(stderr, "  %s: normwise %.3g\n", e.hf_name.c_str(), err);
        CHECK(err < 1e-5);
    }
    // q / k / v and gate / up share their type in both layers: all four groups fuse, and a
    // fused handle's column slices equal its parts' products (the same f32 GEMM per row)
    LoadOptions opt;
    opt.fuse_qkv = opt.fuse_gate_up = true;
    const ModelWeights fw = loader.load_weights(gguf, opt);
    CHECK(fw.fused_parts.size() == 4);
    auto qkv = fw.get_quantized("model.layers.1.self_attn.qkv_proj.weight");
    CHECK(qkv != nullptr && qkv->qtype() == GGML_F16 && qkv->n() == 256);
    if (qkv) {
        const Expect* eq = nullptr;
        for (const Expect& e : ex)
            if (e.hf_name == "model.layers.1.self_attn.q_proj.weight") eq = &e;
        CHECK(eq != nullptr);
        if (eq) {
            const Tensor x = Tensor::from_host(eq->x, {(int64_t)eq->m, 128}, Device::hip(0));
            const std::vector<float> y = qkv->forward(x).to_host();
            std::vector<float> q_cols;
            for (uint32_t r = 0; r < eq->m; ++r)
                q_cols.insert(q_cols.end(), y.begin() + r * 256, y.begin() + r * 256 + 128);
            CHECK(normwise(q_cols, eq->y) < 1e-5);
        }
    }
}

// The file's main K-quant type (Q4_K in the Q4_K_M mix, Q5_K in the Q5_K_M one): that
// of blk.1.attn_q.weight.
static uint32_t main_ktype(const GgufFile& f) {
    for (const auto& t : f.tensors())
        if (t.name == "blk.1.attn_q.weight") return t.type;
    return 0;
}

static void test_cpu_kq(const std::string& gguf, const std::vector<Expect>& ex) {
    const GgufFile f = GgufFile::open(gguf);
    const GgufModelConfig c = GgufWeightLoader::config_from(f);
    CHECK(c.hidden_size == 256 && c.intermediate_size == 512 && c.num_hidden_layers == 2);
    const uint32_t kt = main_ktype(f);
    CHECK(kt == GGML_Q4_K || kt == GGML_Q5_K);
    GgufWeightLoader loader;
    const auto plan = loader.plan(f);
    size_t nk = 0, n6 = 0;
    for (size_t i = 0; i < plan.size() && i < ex.size(); ++i) {
        CHECK(plan[i].type == ex[i].type);
        CHECK(plan[i].quantized == (ex[i].quantized != 0));
        nk += plan[i].type == kt;
        n6 += plan[i].type == GGML_Q6_K;
    }
    CHECK(nk == 12 + 1 && n6 == 3);  // token_embd kt; attn_v.0, ffn_down.0, output Q6_K
    const GgufTensorInfo* q = nullptr;
    for (const auto& t : f.tensors())
        if (t.name == "output.weight") q = &t;
    CHECK(q && q->type == GGML_Q6_K && q->nbytes == 256 * 1 * 210);  // 256 rows x 1 block
}

static void test_gpu_kq(const std::string& gguf, const std::vector<Expect>& ex) {
    GgufWeightLoader loader;
    const ModelWeights w = loader.load_weights(gguf);
    CHECK(w.quantized_tensors.size() == 15 && w.fused_parts.empty());
    CHECK(w.get_quantized("lm_head.weight")->qtype() == GGML_Q6_K);
    CHECK(w.get_quantized("model.layers.1.mlp.down_proj.weight")->qtype() ==
          (int)main_ktype(GgufFile::open(gguf)));
    CHECK(w.tensors.at("model.embed_tokens.weight").shape() == std::vector<int64_t>({256, 256}));
    std::map<std::string, std::vector<float>> ys;
    for (const Expect& e : ex) {
        if (!e.quantized) continue;
        auto q = w.get_quantized(e.hf_name);
        CHECK(q != nullptr);
        if (!q) continue;
        const Tensor x = Tensor::from_host(e.x, {(int64_t)e.m, (int64_t)e.k}, Device::hip(0));
        ys[e.hf_name] = q->forward(x).to_host();
        const double err = normwise(ys[e.hf_name], e.y);
        if (err >= 1e-3) std::fprintf(stderr, "  %s: normwise %.3g\n", e.hf_name.c_str(), err);
        CHECK(err < 1e-3);
    }
    // fusion: layer 1 (all one type) fuses q/k/v and gate/up; layer 0 keeps q/k/v apart
    // (its attn_v is Q6_K) but fuses gate/up
    LoadOptions opt;
    opt.fuse_qkv = opt.fuse_gate_up = true;
    const ModelWeights fw = loader.load_weights(gguf, opt);
    CHECK(fw.get_quantized("model.layers.1.self_attn.qkv_proj.weight") != nullptr);
    CHECK(fw.get_quantized("model.layers.1.self_attn.q_proj.weight") == nullptr);
    CHECK(fw.get_quantized("model.layers.0.self_attn.qkv_proj.weight") == nullptr);
    CHECK(fw.get_quantized("model.layers.0.self_attn.v_proj.weight") != nullptr);
    CHECK(fw.get_quantized("model.layers.0.mlp.gate_up_proj.weight") != nullptr);
    CHECK(fw.fused_parts.size() == 3);  // qkv.1, gate_up.0, gate_up.1
    for (const auto& [fname, parts] : fw.fused_parts) {
        auto q = fw.get_quantized(fname);
        CHECK(q != nullptr);
        if (!q) continue;
        const Expect* first = nullptr;
        for (const Expect& e : ex)
            if (e.hf_name == parts[0].first) first = &e;
        CHECK(first != nullptr);
        if (!first) continue;
        // the parts' own expectations share x (same input, same k) only through
        // the first part's x: run the fused handle on it and compare each column
        // slice with the part loaded on its own, run on the same x
        const Tensor x =
            Tensor::from_host(first->x, {(int64_t)first->m, (int64_t)first->k}, Device::hip(0));
        const std::vector<float> y = q->forward(x).to_host();
        int64_t off = 0;
        for (const auto& [pname, rows] : parts) {
            const std::vector<float> yp = w.get_quantized(pname)->forward(x).to_host();
            bool same = true;
            for (int64_t r = 0; r < (int64_t)first->m; ++r)
                for (int64_t c = 0; c < rows; ++c)
                    same = same && y[r * q->n() + off + c] == yp[r * rows + c];
            if (!same) std::fprintf(stderr, "  %s: slice of %s differs\n", pname.c_str(), fname.c_str());
            CHECK(same);
            off += rows;
        }
        CHECK(off == q->n());
        // the fused gate_up handle's SwiGLU: silu(gate) * up of the parts' own outputs
        if (fname.find("gate_up_proj") != std::string::npos) {
            const Tensor act = q->forward_swiglu(x);
            CHECK(act.shape() == std::vector<int64_t>({(int64_t)first->m, q->n() / 2}));
            const std::vector<float> a = act.to_host();
            const int64_t I = q->n() / 2;
            double worst = 0.0;
            for (int64_t r = 0; r < (int64_t)first->m; ++r)
                for (int64_t c = 0; c < I; ++c) {
                    const double g = y[r * q->n() + c], u = y[r * q->n() + I + c];
                    const double want = g / (1.0 + std::exp(-g)) * u;
                    worst = std::max(worst, std::fabs(a[r * I + c] - want) / (1e-6 + std::fabs(want)));
                }
            CHECK(worst < 1e-5);
        }
    }
    // the residual add: r + forward(x) in the projection's epilogue
    {
        auto q = w.get_quantized("model.layers.1.self_attn.o_proj.weight");
        const Expect* e = nullptr;
        for (const Expect& ee : ex)
            if (ee.hf_name == "model.layers.1.self_attn.o_proj.weight") e = &ee;
        CHECK(q && e);
        if (q && e) {
            const Tensor x = Tensor::from_host(e->x, {(int64_t)e->m, (int64_t)e->k}, Device::hip(0));
            std::vector<float> r0((size_t)e->m * e->n);
            for (size_t i = 0; i < r0.size(); ++i) r0[i] = 0.25f * (float)(i % 13) - 1.0f;
            Tensor r = Tensor::from_host(r0, {(int64_t)e->m, (int64_t)e->n}, Device::hip(0));
            q->forward_add(x, r);
            const std::vector<float> got = r.to_host(), plain = q->forward(x).to_host();
            bool same = true;
            for (size_t i = 0; i < got.size(); ++i) same = same && got[i] == r0[i] + plain[i];
            CHECK(same);  // GEMV: one rounding of r + the same row sum
            // the layer norm in front: gamma = 1, no bias -> the same as normalizing on
            // the host (two-pass mean and variance, eps 1e-6) and a plain forward
            std::vector<float> xn(e->x.size());
            for (uint32_t row = 0; row < e->m; ++row) {
                const float* xr = e->x.data() + (size_t)row * e->k;
                double mu = 0, var = 0;
                for (uint32_t c = 0; c < e->k; ++c) mu += xr[c];
                mu /= e->k;
                for (uint32_t c = 0; c < e->k; ++c) var += (xr[c] - mu) * (xr[c] - mu);
                const double sd = std::sqrt(var / e->k + 1e-6);
                for (uint32_t c = 0; c < e->k; ++c) xn[(size_t)row * e->k + c] = (float)((xr[c] - mu) / sd);
            }
            const Tensor gamma = Tensor::from_host(std::vector<float>(e->k, 1.0f), {(int64_t)e->k},
                                                   Device::hip(0));
            const std::vector<float> yn = q->forward_norm(x, gamma, nullptr, 1e-6f).to_host();
            const std::vector<float> yh =
                q->forward(Tensor::from_host(xn, {(int64_t)e->m, (int64_t)e->k}, Device::hip(0)))
                    .to_host();
            double num = 0, den = 0;
            for (size_t i = 0; i < yn.size(); ++i) {
                num = std::max(num, (double)std::fabs(yn[i] - yh[i]));
                den = std::max(den, (double)std::fabs(yh[i]));
            }
            CHECK(num <= 1e-3 * den);
        }
    }
}

int main(int argc, char** argv) {
    if (argc != 4) {
        std::fprintf(stderr, "usage: %s cpu|gpu file.gguf file.expect\n", argv[0]);
        return 2;
    }
    const std::string mode = argv[1];
    try {
        const std::vector<Expect> ex = mode == "gpu-step" ? std::vector<Expect>{}
                                                           : read_expect(argv[3]);
        if (mode == "cpu") test_cpu(argv[2], ex);
        else if (mode == "gpu") test_gpu(argv[2], ex);
        else if (mode == "cpu-kq") test_cpu_kq(argv[2], ex);
        else if (mode == "gpu-kq") test_gpu_kq(argv[2], ex);
        else if (mode == "gpu-dense") test_gpu_dense(argv[2], ex);
        else if (mode == "gpu-step") test_gpu_step(argv[2], argv[3]);
        else return 2;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "FAIL: uncaught exception: %s\n", e.what());
        return 1;
    }
    std::printf("%s: %d passed, %d failed\n", mode.c_str(), g_pass, g_fail);
    return g_fail ? 1 : 0;
}
