// gguf.hpp -- GGUF (v2 / v3) reader for the quantized linear-layer path.
//
// Replaces the external candle calls the reference makes at load time:
//   gguf_file::Content::read      (crates/runtime/src/weight_loader_core.rs:509-511)
//   TensorInfo::read               (weight_loader_core.rs:545)
// File layout (GGUF spec): magic "GGUF", u32 version, u64 tensor count,
// u64 metadata count, metadata key/values, tensor infos (name, u32 n_dims,
// u64 ne[n_dims] with ne[0] innermost, u32 ggml type, u64 offset), padding to
// general.alignment (default 32), then tensor data.  A 2-D tensor with
// ne = [k, n] is the [n, k] row-major matrix candle builds (dims reversed).
#pragma once

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

namespace unillm {

struct GgufError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// GGML tensor type ids (the subset with a fixed block layout).
enum GgmlType : uint32_t {
    GGML_F32 = 0, GGML_F16 = 1, GGML_Q4_0 = 2, GGML_Q4_1 = 3, GGML_Q5_0 = 6, GGML_Q5_1 = 7,
    GGML_Q8_0 = 8, GGML_Q8_1 = 9, GGML_Q2_K = 10, GGML_Q3_K = 11, GGML_Q4_K = 12,
    GGML_Q5_K = 13, GGML_Q6_K = 14, GGML_Q8_K = 15, GGML_BF16 = 30,
};

// {elements per block, bytes per block}; {0, 0} for ids this reader cannot size.
struct GgmlTypeSize {
    uint32_t block_elems;
    uint32_t block_bytes;
};
GgmlTypeSize ggml_type_size(uint32_t type);
const char* ggml_type_name(uint32_t type);

struct GgufValue {
    enum Kind { UINT, INT, FLOAT, BOOL, STRING, ARRAY } kind = UINT;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    bool b = false;
    std::string s;
    uint32_t array_type = 0;
    std::vector<GgufValue> items;  // ARRAY
};

struct GgufTensorInfo {
    std::string name;
    std::vector<uint64_t> ne;  // ne[0] innermost
    uint32_t type = 0;
    uint64_t offset = 0;       // from the start of the data section
    uint64_t nbytes = 0;
    // candle shape: ne reversed, e.g. [n, k] for a 2-D weight
    std::vector<uint64_t> shape() const { return {ne.rbegin(), ne.rend()}; }
};

class GgufFile {
public:
    // Parses the header, metadata and tensor infos; validates every tensor's
    // byte range against the file size.  Throws GgufError on malformed input.
    static GgufFile open(const std::string& path);

    uint32_t version() const { return version_; }
    uint64_t alignment() const { return alignment_; }
    uint64_t data_offset() const { return data_offset_; }
    const std::vector<GgufTensorInfo>& tensors() const { return tensors_; }
    const std::map<std::string, GgufValue>& metadata() const { return metadata_; }
    const GgufValue* find(const std::string& key) const;
    uint64_t get_uint(const std::string& key, uint64_t dflt) const;
    double get_float(const std::string& key, double dflt) const;  // FLOAT (or integer) values
    std::string get_string(const std::string& key, const std::string& dflt) const;

    // Raw bytes of one tensor (block bytes for quantized types).
    std::vector<uint8_t> read(const GgufTensorInfo& t) const;

private:
    std::string path_;
    uint32_t version_ = 0;
    uint64_t alignment_ = 32;
    uint64_t data_offset_ = 0;
    uint64_t file_size_ = 0;
    std::map<std::string, GgufValue> metadata_;
    std::vector<GgufTensorInfo> tensors_;
};

}  // namespace unillm
