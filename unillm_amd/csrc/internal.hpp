// internal.hpp -- shared definitions of the gfx950 quantized-matmul library.
//
// Device layout of a weight (written once by the repack kernel at upload).
// Row n occupies `row_bytes` = align16(kb * (QB + 2)) bytes at n * row_bytes:
//   [kb x QB payload bytes][kb x f16 scales][pad to 16 B]
// QB = 16 (Q4_0 nibbles) or 32 (Q8_0 int8).  Q4_0 nibbles are stored as the
// signed 4-bit value q - 8 (the GGUF byte XOR 0x88), the operand form of
// v_dot8_i32_i4; the GGUF nibble order is kept (low nibble of byte j = element
// j, high nibble = element j + 16).  The payloads of a row are back
// to back, so a 128-bit load is exactly one Q4_0 block payload (or half a
// Q8_0 one), and the row's scales sit in the same DRAM pages right after
// them (measured: cheaper to stream than a separate scale plane).  The byte
// count is GGUF's (18 or 34 B per 32 weights) plus at most 15 B of row
// padding; dequant of this layout is bit-exact with the GGUF bytes.
//
// Q5_0 (GGML block_q5_0: f16 d, 32 fifth bits, 16 nibble bytes) holds int8 codes
// q - 16 times d: it is repacked into Q8_0's frame and runs as Q8_0.
//
// Q4_K (GGML block_q4_K: 256 weights = 8 sub-blocks of 32 under one f16 d and
// one f16 dmin, 6-bit scale sc_j and min m_j per sub-block) is repacked into the
// same frame, one 32-weight sub-block per block:
//   [kb x 16 B payload][kb x u16 (sc | m << 8)][kb / 8 x u32 (d | dmin << 16)][pad]
// The payload is the sub-block's 32 codes q in Q4_0's order and form (signed
// q - 8; element j low nibble of byte j, element j + 16 high nibble), so
// w = (d sc) q - dmin m = (d sc)(q - 8) + (8 d sc - dmin m).  18.5 B per 32
// weights against GGUF's 18; d sc and dmin m are exact in f32.
//
// Q6_K (GGML block_q6_K: 256 weights, 6-bit codes q, int8 scale per 16
// weights, one f16 d) is repacked into Q8_0's frame:
//   [kb x 32 B int8 codes q - 32][kb x u16 (sc_lo | sc_hi << 8)][kb / 8 x u32 d][pad]
// sc_lo scales weights 0 .. 15 of the block, sc_hi 16 .. 31 (GGML's scales[j]
// covers weights 16 j .. 16 j + 15); w = (d sc) (q - 32), d sc exact in f32.
// 34.5 B per 32 weights against GGUF's 26.25: the 6-bit codes take a byte each.
//
// Q5_K (GGML block_q5_K: Q4_K's d, dmin, scales and nibbles, plus a fifth bit
// per weight) is repacked into Q8_0's frame with Q4_K's scale words and header:
//   [kb x 32 B int8 codes q - 16][kb x u16 (sc | m << 8)][kb / 8 x u32 (d | dmin << 16)][pad]
// in element order, so w = (d sc) q - dmin m = (d sc)(q - 16) + (16 d sc - dmin m).
// 34.5 B per 32 weights against GGUF's 22: the 5-bit codes take a byte each.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/unillm_hip.h"

// The opaque handle of the C ABI is the weight descriptor itself.
struct unillm_qweight {
    int qtype;             // the layout and kernels' type (Q5_0 is held as Q8_0)
    int src_qtype;         // the GGUF type the caller created it from
    int device;
    int64_t n, k, kb;      // kb = k / 32
    int64_t row_bytes;     // bytes per row: payloads, scales, padding
    uint8_t* base;         // n * row_bytes, then a 256-byte scratch slot
    size_t bytes;
    int f16_exp;           // smallest E with max|q d| 2^-E <= 65504 (f16 range)
};

// The opaque KV-cache handle (one decoder layer, one sequence): K and V of
// n_kv_heads heads, [n_kv_heads][max_seq][head_dim] f32 each, the first len
// positions filled; inv_freq[head_dim / 2] the RoPE frequencies in f32.
// The filled length lives in device memory, state[0], read and advanced by the
// attention kernels themselves (so a captured call replays at successive
// positions); state[1] is set to 1 by a kernel that found len + m > max_seq (the
// call then appends nothing and writes NaN); state[2] is scratch between a call's
// kernels.  `len` is the host's copy, exact while only eager calls ran; once a call
// on the cache has been captured (captured), replays can move the device length at
// any time, so the host reads state[0] back before each later use (len_stale).
struct unillm_kv_cache {
    int device;
    int64_t n_kv_heads, head_dim, max_seq, len;
    float rope_theta;
    float* k;
    float* v;
    float* inv_freq;
    int* state;
    bool len_stale;
    bool captured;
};

namespace unillm {

constexpr int QK = 32;  // weights per block
using QWeight = ::unillm_qweight;

int64_t gemv_max_kb(int64_t m, int qtype);
bool gemv_supports(const unillm_qweight& w, int64_t m);
bool gemv_supports_swiglu(const unillm_qweight& w, int64_t m);
bool gemv_supports_norm(const unillm_qweight& w, int64_t m);

// Epilogues of the matmul launches: y = x W^T (store), y += x W^T (the decoder
// layer's residual add, llama.rs:668, 677), or for a [gate; up] weight of 2 I
// rows y[m, I] = silu(x G^T) * (x U^T) (fused_swiglu, tensor_core.rs:1385-1396).
constexpr int kEpiStore = 0, kEpiAdd = 1, kEpiSwiglu = 2;

// The layer norm applied to x before the matmul (gamma == nullptr: none):
// (x - mean) / sqrt(var + eps) * gamma (+ beta) along k, var = mean((x - mean)^2)
// (ops_fn::layer_norm, tensor_core.rs:973-1008; eps 1e-6 at llama.rs:662, 671).
struct NormArgs {
    const float* gamma;
    const float* beta;  // may be nullptr
    float eps;
};

inline bool is_kquant(int qtype) {
    return qtype == UNILLM_QTYPE_Q4_K || qtype == UNILLM_QTYPE_Q5_K || qtype == UNILLM_QTYPE_Q6_K;
}
// byte codes (one int8 a weight): Q8_0, and Q5_K / Q6_K as repacked
inline bool byte_codes(int qtype) {
    return qtype == UNILLM_QTYPE_Q8_0 || qtype == UNILLM_QTYPE_Q5_K || qtype == UNILLM_QTYPE_Q6_K;
}
inline int qbytes(int qtype) { return byte_codes(qtype) ? 32 : 16; }
inline int64_t row_bytes_for(int qtype, int64_t kb) {
    const int64_t hdr = is_kquant(qtype) ? kb / 8 * 4 : 0;
    return (kb * (qbytes(qtype) + 2) + hdr + 15) / 16 * 16;
}

// Addresses inside a row (QB = payload bytes per block).
template <int QB>
__host__ __device__ __forceinline__ const uint8_t* blk_payload(const uint8_t* base, int64_t rb,
                                                                int64_t row, int64_t b) {
    return base + row * rb + b * QB;
}
template <int QB>
__host__ __device__ __forceinline__ const uint16_t* blk_scale(const uint8_t* base, int64_t rb,
                                                               int64_t kb, int64_t row, int64_t b) {
    return reinterpret_cast<const uint16_t*>(base + row * rb + kb * QB) + b;
}
// K-quants: the u32 header of the 256-weight group holding block b (Q4_K, Q5_K:
// d | dmin << 16; Q6_K: d), after the payload (QB bytes a block) and u16 planes.
template <int QB>
__host__ __device__ __forceinline__ const uint32_t* kq_header(const uint8_t* base, int64_t rb,
                                                              int64_t kb, int64_t row, int64_t b) {
    return reinterpret_cast<const uint32_t*>(base + row * rb + kb * (QB + 2)) + (b >> 3);
}
__host__ __device__ __forceinline__ const uint32_t* q4k_header(const uint8_t* base, int64_t rb,
                                                               int64_t kb, int64_t row, int64_t b) {
    return kq_header<16>(base, rb, kb, row, b);
}
// GGUF bytes per block and weights per block
inline int gguf_block_elems(int qtype) { return is_kquant(qtype) ? 256 : QK; }
inline int gguf_block_bytes(int qtype) {
    switch (qtype) {
        case UNILLM_QTYPE_Q8_0: return 34;
        case UNILLM_QTYPE_Q5_0: return 22;
        case UNILLM_QTYPE_Q4_K: return 144;
        case UNILLM_QTYPE_Q5_K: return 176;
        case UNILLM_QTYPE_Q6_K: return 210;
        default: return 18;
    }
}

// Per-device properties cached at init.
struct DeviceInfo {
    int cu_count;
    int max_lds;     // per workgroup
    int max_lds_cu;  // per CU
};
const DeviceInfo& device_info();
// A device buffer of at least `bytes` for work on stream s, kept and reused by
// later calls on the same stream (stream order makes the reuse safe: a call's
// kernels finish before the next call's start).  Grows stream-ordered; the
// memory is held until the process ends.  Calls on one stream from several
// host threads are ordered by the stream, the map by a mutex.
// Slot 0 holds x in the MFMA paths' operand type; slot 1 the [gate | up] outputs
// of a SwiGLU call off the GEMV path (both live during that call); slot 2 the
// rotated queries and the per-chunk partials of decode attention; slot 3 an
// aligned copy of x; slot kSyncSlot the batched decode's arrival tickets, zeroed
// when allocated (every launch leaves them zero again).
constexpr int kSyncSlot = 4;
hipError_t stream_workspace(hipStream_t s, size_t bytes, void** out, int slot = 0);
// UNILLM_DEBUG_LAUNCH=1 prints each kernel's launch shape to stderr.
bool debug_launch();

// ---- launchers (each in the translation unit that holds its kernel) ----------
// All return a hipError_t from the launch; shapes are validated by the caller.
hipError_t launch_repack(const QWeight& w, const uint8_t* gguf, hipStream_t s);
hipError_t launch_dequant(const QWeight& w, float* out, hipStream_t s);
// max over the scale plane of (f16 bits & 0x7FFF), atomically max-ed into out[0]
// (Q4_K, Q5_K: max |d| into out[0], max |dmin| into out[1]; Q6_K: max |d| into out[0])
hipError_t launch_scale_absmax(const QWeight& w, uint32_t* out, hipStream_t s);
hipError_t launch_quantize(int qtype, const float* w, int64_t n, int64_t k, uint8_t* out,
                           hipStream_t s);
// epi: kEpiStore or kEpiAdd on every path; kEpiSwiglu on the GEMV only
// (gemv_supports_swiglu), the other paths run it as store + swiglu_kernel.
hipError_t launch_gemv(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t s,
                       int epi = kEpiStore, const NormArgs& norm = NormArgs{nullptr, nullptr, 0.f});
// The MFMA paths take their x operand buffer from `ws` when it is given (at least
// decode_workspace_bytes / prefill_call_bytes for this w and m), else from the
// stream's workspace (slot 0).
// sync_ws: the arrival tickets of the one-launch batched decode (m <= 16 without a
// norm; at least decode_sync_bytes, zero), else the stream's slot kSyncSlot.
hipError_t launch_decode_mfma(const QWeight& w, const float* x, int64_t m, float* y,
                              hipStream_t s, int epi = kEpiStore,
                              const NormArgs& norm = NormArgs{nullptr, nullptr, 0.f},
                              void* ws = nullptr, void* sync_ws = nullptr);
hipError_t launch_prefill_mfma(const QWeight& w, const float* x, int64_t m, float* y,
                               hipStream_t s, int epi = kEpiStore,
                               const NormArgs& norm = NormArgs{nullptr, nullptr, 0.f},
                               void* ws = nullptr, size_t ws_bytes = 0);
// The batched decode's x operand workspace (0 where the kernel converts x itself),
// and its arrival tickets.
// (no default for norm: the size depends on it)
size_t decode_workspace_bytes(const QWeight& w, int64_t m, const NormArgs& norm);
size_t decode_sync_bytes(const QWeight& w);
// The prefill's workspace: this call's own need (cap > 0: in a fixed workspace of
// cap bytes, which may pick a plan without a k split), and a bound for every call
// of up to m rows (the size a reserve takes).
size_t prefill_call_bytes(const QWeight& w, int64_t m, size_t cap = 0);
size_t prefill_workspace_bytes(const QWeight& w, int64_t m);
// Both MFMA paths address weight bytes with 32-bit offsets: weights under 4 GiB.
inline bool mfma_supports(const QWeight& w) {
    return (uint64_t)w.n * (uint64_t)w.row_bytes < (1ull << 32);
}
// x[m, k] -> its layer norm as f16 in the MFMA paths' element order, one workgroup
// per row, scaled by powers of two: per row (rs[row] <- the undoing factor) for the
// prefill path, or per k slice of the batched-decode split (S slices, rf[s * 64 +
// row]); zeroes y rows [0, m) of width ny when ny > 0 (a split k adds into it).
hipError_t launch_norm_convert(const float* x, int64_t m, int64_t k, const NormArgs& norm,
                               void* out, float* y, int64_t ny, hipStream_t s,
                               float* rs = nullptr, int S = 0, float* rf = nullptr);
// x[m, k] (k % 32 == 0) -> f16 rows (round to nearest even) in the decode kernel's
// element order (each aligned 8 as 0 2 1 3 4 6 5 7), each row scaled by a power
// of two that puts its largest magnitude in [2^14, 2^15); rs[row] <- the factor
// that undoes it.  launch_norm_convert with rs != nullptr (f16) scales its rows the
// same way.
hipError_t launch_x_to_f16_rows(const float* x, int64_t m, int64_t k, void* out, float* rs,
                                hipStream_t s);
// act[m, I] = silu(g[m, i]) * u[m, i] with g, u the two halves of each row of
// gu[m, 2 I] (the SwiGLU of the MFMA paths, after their store)
hipError_t launch_swiglu(const float* gu, int64_t m, int64_t I, float* act, hipStream_t s);

// Dense (F32 / F16 / BF16) weights: f32 rows [n][k] at base (row_bytes = 4 k).
bool is_dense(int qtype);
int dense_elem_bytes(int qtype);
// the weight's f32 rows from its GGUF elements at src (device memory), on s
hipError_t launch_dense_upload(const QWeight& w, const void* src, hipStream_t s);
// y = x W^T (add: y += x W^T) in f32; the GEMM's handle is created on first use
// (dense_prepare creates it ahead, outside any capture)
hipError_t launch_dense(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t s,
                        int add);
hipError_t dense_prepare(hipStream_t s);
// the layer norm of each row of x into out (f32), ops_fn::layer_norm's two passes
hipError_t launch_norm_rows(const float* x, int64_t m, int64_t k, const NormArgs& norm,
                            float* out, hipStream_t s);
// the message of the last failing dense call on this thread
std::string dense_error();

// Attention (attention.hip): RoPE at positions len .. len + m - 1 on the fused QKV
// rows qkv[m, (H + 2 KVH) hd], k / v appended to the cache, causal softmax
// attention into out[m, H hd]; the kernels read len from kv.state[0] and advance
// it by m.  Decode steps (m H / KVH <= attention_max_queries()) split the cache
// into chunks merged by log-sum-exp; longer calls (a prompt) run a tiled kernel
// per (query block, head).  `len_hint` is the host's length, used only to size the
// decode grid; a negative hint sizes it for max_seq (graph capture).
using KvCache = ::unillm_kv_cache;
hipError_t launch_attention(const KvCache& kv, const float* qkv, int64_t m, int64_t H,
                            float* out, int64_t len_hint, hipStream_t s);
// Workspace (slot 2) a call of m tokens and H heads needs at any cache length.
size_t attention_workspace_bytes(const KvCache& kv, int64_t m, int64_t H);
int attention_max_queries();  // m * H / KVH per decode call
int64_t attention_max_positions();  // len + m per call

constexpr int64_t kGemvMaxM = 4;
constexpr int64_t kDecodeMaxM = 64;

}  // namespace unillm
