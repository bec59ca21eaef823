// gguf.cpp -- GGUF reader (see gguf.hpp).  Every read is bounds-checked
// against the file size, so truncated or hostile files raise GgufError.
#include "gguf.hpp"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>

namespace unillm {

namespace {

// GGUF metadata value types (spec).
enum : uint32_t {
    V_UINT8 = 0, V_INT8 = 1, V_UINT16 = 2, V_INT16 = 3, V_UINT32 = 4, V_INT32 = 5,
    V_FLOAT32 = 6, V_BOOL = 7, V_STRING = 8, V_ARRAY = 9, V_UINT64 = 10, V_INT64 = 11,
    V_FLOAT64 = 12,
};

constexpr uint64_t kMaxString = 1ull << 30;
constexpr uint64_t kMaxCount = 1ull << 32;

struct FileCloser {
    void operator()(FILE* f) const { if (f) std::fclose(f); }
};

class Reader {
public:
    Reader(FILE* f, uint64_t size) : f_(f), size_(size) {}
    uint64_t pos() const { return pos_; }

    void bytes(void* dst, uint64_t n) {
        if (n > size_ - pos_) throw GgufError("gguf: unexpected end of file at byte " +
                                              std::to_string(pos_));
        if (n && std::fread(dst, 1, n, f_) != n) throw GgufError("gguf: read error");
        pos_ += n;
    }
    template <typename T>
    T pod() {
        T v;
        bytes(&v, sizeof(T));  // GGUF is little-endian, as is every host we target
        return v;
    }
    std::string str() {
        const uint64_t n = pod<uint64_t>();
        if (n > kMaxString) throw GgufError("gguf: string length " + std::to_string(n));
        std::string s(n, '\0');
        bytes(s.data(), n);
        return s;
    }
    GgufValue value(uint32_t type, int depth) {
        if (depth > 4) throw GgufError("gguf: arrays nested too deeply");
        GgufValue v;
        switch (type) {
            case V_UINT8: v.kind = GgufValue::UINT; v.u = pod<uint8_t>(); break;
            case V_UINT16: v.kind = GgufValue::UINT; v.u = pod<uint16_t>(); break;
            case V_UINT32: v.kind = GgufValue::UINT; v.u = pod<uint32_t>(); break;
            case V_UINT64: v.kind = GgufValue::UINT; v.u = pod<uint64_t>(); break;
            case V_INT8: v.kind = GgufValue::INT; v.i = pod<int8_t>(); break;
            case V_INT16: v.kind = GgufValue::INT; v.i = pod<int16_t>(); break;
            case V_INT32: v.kind = GgufValue::INT; v.i = pod<int32_t>(); break;
            case V_INT64: v.kind = GgufValue::INT; v.i = pod<int64_t>(); break;
            case V_FLOAT32: v.kind = GgufValue::FLOAT; v.f = pod<float>(); break;
            case V_FLOAT64: v.kind = GgufValue::FLOAT; v.f = pod<double>(); break;
            case V_BOOL: v.kind = GgufValue::BOOL; v.b = pod<uint8_t>() != 0; break;
            case V_STRING: v.kind = GgufValue::STRING; v.s = str(); break;
            case V_ARRAY: {
                v.kind = GgufValue::ARRAY;
                v.array_type = pod<uint32_t>();
                const uint64_t n = pod<uint64_t>();
                if (n > kMaxCount || n > size_ - pos_)
                    throw GgufError("gguf: array length " + std::to_string(n));
                // a parsed item is ~100 bytes against >= 1 byte of file: reserve a
                // bounded count and let the vector grow with the items actually read
                v.items.reserve((size_t)std::min<uint64_t>(n, 4096));
                for (uint64_t i = 0; i < n; ++i) v.items.push_back(value(v.array_type, depth + 1));
                break;
            }
            default:
                throw GgufError("gguf: unknown metadata value type " + std::to_string(type));
        }
        return v;
    }

private:
    FILE* f_;
    uint64_t size_;
    uint64_t pos_ = 0;
};

}  // namespace

GgmlTypeSize ggml_type_size(uint32_t type) {
    // GGML's block geometry per type id (the on-disk format, fixed by GGML).
    switch (type) {
        case GGML_F32: return {1, 4};
        case GGML_F16: return {1, 2};
        case GGML_BF16: return {1, 2};
        case GGML_Q4_0: return {32, 18};
        case GGML_Q4_1: return {32, 20};
        case GGML_Q5_0: return {32, 22};
        case GGML_Q5_1: return {32, 24};
        case GGML_Q8_0: return {32, 34};
        case GGML_Q8_1: return {32, 36};
        case GGML_Q2_K: return {256, 84};
        case GGML_Q3_K: return {256, 110};
        case GGML_Q4_K: return {256, 144};
        case GGML_Q5_K: return {256, 176};
        case GGML_Q6_K: return {256, 210};
        case GGML_Q8_K: return {256, 292};
        default: return {0, 0};
    }
}

const char* ggml_type_name(uint32_t type) {
    switch (type) {
        case GGML_F32: return "F32";
        case GGML_F16: return "F16";
        case GGML_BF16: return "BF16";
        case GGML_Q4_0: return "Q4_0";
        case GGML_Q4_1: return "Q4_1";
        case GGML_Q5_0: return "Q5_0";
        case GGML_Q5_1: return "Q5_1";
        case GGML_Q8_0: return "Q8_0";
        case GGML_Q8_1: return "Q8_1";
        case GGML_Q2_K: return "Q2_K";
        case GGML_Q3_K: return "Q3_K";
        case GGML_Q4_K: return "Q4_K";
        case GGML_Q5_K: return "Q5_K";
        case GGML_Q6_K: return "Q6_K";
        case GGML_Q8_K: return "Q8_K";
        default: return "unknown";
    }
}

GgufFile GgufFile::open(const std::string& path) {
    std::unique_ptr<FILE, FileCloser> f(std::fopen(path.c_str(), "rb"));
    if (!f) throw GgufError("gguf: cannot open " + path);
    if (std::fseek(f.get(), 0, SEEK_END) != 0) throw GgufError("gguf: cannot seek " + path);
    const long end = std::ftell(f.get());
    if (end < 0) throw GgufError("gguf: cannot size " + path);
    std::rewind(f.get());

    GgufFile g;
    g.path_ = path;
    g.file_size_ = (uint64_t)end;
    Reader r(f.get(), g.file_size_);
    char magic[4];
    r.bytes(magic, 4);
    if (std::memcmp(magic, "GGUF", 4) != 0) throw GgufError("gguf: bad magic in " + path);
    g.version_ = r.pod<uint32_t>();
    if (g.version_ != 2 && g.version_ != 3)
        throw GgufError("gguf: unsupported version " + std::to_string(g.version_));
    const uint64_t n_tensors = r.pod<uint64_t>();
    const uint64_t n_kv = r.pod<uint64_t>();
    if (n_tensors > kMaxCount || n_kv > kMaxCount) throw GgufError("gguf: implausible counts");

    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = r.str();
        const uint32_t type = r.pod<uint32_t>();
        g.metadata_[key] = r.value(type, 0);
    }
    if (const GgufValue* a = g.find("general.alignment")) {
        if (a->kind != GgufValue::UINT || a->u == 0 || (a->u & (a->u - 1)) != 0)
            throw GgufError("gguf: general.alignment must be a power of two");
        g.alignment_ = a->u;
    }
    g.tensors_.reserve((size_t)std::min<uint64_t>(n_tensors, 4096));  // grows as read
    for (uint64_t i = 0; i < n_tensors; ++i) {
        GgufTensorInfo t;
        t.name = r.str();
        const uint32_t nd = r.pod<uint32_t>();
        if (nd == 0 || nd > 4) throw GgufError("gguf: tensor '" + t.name + "' has " +
                                               std::to_string(nd) + " dims");
        uint64_t elems = 1;
        for (uint32_t d = 0; d < nd; ++d) {
            const uint64_t e = r.pod<uint64_t>();
            if (e == 0 || e > (1ull << 40) || elems > (1ull << 50) / e)
                throw GgufError("gguf: tensor '" + t.name + "' has a bad dimension");
            t.ne.push_back(e);
            elems *= e;
        }
        t.type = r.pod<uint32_t>();
        t.offset = r.pod<uint64_t>();
        const GgmlTypeSize ts = ggml_type_size(t.type);
        if (ts.block_elems == 0)
            throw GgufError("gguf: tensor '" + t.name + "' has unsupported ggml type " +
                            std::to_string(t.type));
        if (t.ne[0] % ts.block_elems != 0)
            throw GgufError("gguf: tensor '" + t.name + "' row of " + std::to_string(t.ne[0]) +
                            " is not a whole number of " + ggml_type_name(t.type) + " blocks");
        t.nbytes = elems / ts.block_elems * ts.block_bytes;
        if (t.offset % g.alignment_ != 0)
            throw GgufError("gguf: tensor '" + t.name + "' offset is not aligned");
        g.tensors_.push_back(std::move(t));
    }
    g.data_offset_ = (r.pos() + g.alignment_ - 1) / g.alignment_ * g.alignment_;
    for (const GgufTensorInfo& t : g.tensors_)
        if (g.data_offset_ > g.file_size_ || t.offset > g.file_size_ - g.data_offset_ ||
            t.nbytes > g.file_size_ - g.data_offset_ - t.offset)
            throw GgufError("gguf: tensor '" + t.name + "' extends past the end of the file");
    return g;
}

const GgufValue* GgufFile::find(const std::string& key) const {
    auto it = metadata_.find(key);
    return it == metadata_.end() ? nullptr : &it->second;
}

uint64_t GgufFile::get_uint(const std::string& key, uint64_t dflt) const {
    const GgufValue* v = find(key);
    if (!v) return dflt;
    if (v->kind == GgufValue::UINT) return v->u;
    if (v->kind == GgufValue::INT && v->i >= 0) return (uint64_t)v->i;
    return dflt;
}

double GgufFile::get_float(const std::string& key, double dflt) const {
    const GgufValue* v = find(key);
    if (!v) return dflt;
    if (v->kind == GgufValue::FLOAT) return v->f;
    if (v->kind == GgufValue::UINT) return (double)v->u;
    if (v->kind == GgufValue::INT) return (double)v->i;
    return dflt;
}

std::string GgufFile::get_string(const std::string& key, const std::string& dflt) const {
    const GgufValue* v = find(key);
    return v && v->kind == GgufValue::STRING ? v->s : dflt;
}

std::vector<uint8_t> GgufFile::read(const GgufTensorInfo& t) const {
    std::unique_ptr<FILE, FileCloser> f(std::fopen(path_.c_str(), "rb"));
    if (!f) throw GgufError("gguf: cannot reopen " + path_);
    std::vector<uint8_t> out(t.nbytes);
    if (std::fseek(f.get(), (long)(data_offset_ + t.offset), SEEK_SET) != 0 ||
        std::fread(out.data(), 1, t.nbytes, f.get()) != t.nbytes)
        throw GgufError("gguf: failed to read tensor '" + t.name + "'");
    return out;
}

}  // namespace unillm
