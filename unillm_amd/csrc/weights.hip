// weights.hip -- load-time kernels: GGUF repack, exact dequant, GGML quantizer.
//
// None of these is on the per-token path; they run once per weight (repack)
// or in tests and tooling (dequant, quantize).  All are HBM-bound byte work.
#include <hip/hip_fp16.h>

#include <algorithm>

#include "internal.hpp"

namespace unillm {
namespace {

__device__ __forceinline__ uint16_t ld_u16(const uint8_t* p) {
    return (uint16_t)(p[0] | ((uint16_t)p[1] << 8));
}

// One thread per block: GGUF {f16 d; qs[QB]} (18 / 34 B, only 2-byte aligned)
// -> the row layout [kb payloads][kb scales] (payloads 16-byte aligned).
template <int QB>
__global__ __launch_bounds__(256) void repack_kernel(const uint8_t* __restrict__ src,
                                                     uint8_t* __restrict__ base, int64_t rb,
                                                     int64_t kb, int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const int64_t row = i / kb, blk = i - row * kb;
    const uint8_t* b = src + i * (QB + 2);
    *const_cast<uint16_t*>(blk_scale<QB>(base, rb, kb, row, blk)) = ld_u16(b);
    // Q4_0 codes are stored as signed nibbles q - 8 (two's complement: q ^ 8)
    constexpr uint32_t kFlip = QB == 16 ? 0x88888888u : 0u;
    uint32_t words[QB / 4];
#pragma unroll
    for (int w = 0; w < QB / 4; ++w) {
        const uint8_t* p = b + 2 + 4 * w;
        words[w] = ((uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
                    ((uint32_t)p[3] << 24)) ^ kFlip;
    }
    uint4* dst = reinterpret_cast<uint4*>(const_cast<uint8_t*>(blk_payload<QB>(base, rb, row, blk)));
#pragma unroll
    for (int v = 0; v < QB / 16; ++v)
        dst[v] = make_uint4(words[4 * v], words[4 * v + 1], words[4 * v + 2], words[4 * v + 3]);
}

// One thread per GGUF Q5_0 block ({f16 d; u8 qh[4]; u8 qs[16]}, 22 B, 2-byte aligned):
// element e's code is its nibble (low of qs[e] for e < 16, high of qs[e - 16] above)
// plus bit e of the little-endian u32 qh as the fifth bit (GGML dequantize_row_q5_0)
// -> Q8_0's frame: the int8 codes q - 16 in element order and d as the block's scale.
__global__ __launch_bounds__(256) void repack_q5_0_kernel(const uint8_t* __restrict__ src,
                                                          uint8_t* __restrict__ base, int64_t rb,
                                                          int64_t kb, int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const int64_t row = i / kb, blk = i - row * kb;
    const uint8_t* b = src + i * 22;
    *const_cast<uint16_t*>(blk_scale<32>(base, rb, kb, row, blk)) = ld_u16(b);
    const uint32_t qh = (uint32_t)ld_u16(b + 2) | ((uint32_t)ld_u16(b + 4) << 16);
    const uint8_t* qs = b + 6;
    uint32_t words[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        uint32_t v = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = 4 * w + u;
            const uint32_t nib = e < 16 ? qs[e] & 15u : (uint32_t)qs[e - 16] >> 4;
            const uint32_t q = nib | (((qh >> e) & 1u) << 4);
            v |= ((q - 16u) & 0xFFu) << (8 * u);
        }
        words[w] = v;
    }
    uint4* dst = reinterpret_cast<uint4*>(const_cast<uint8_t*>(blk_payload<32>(base, rb, row, blk)));
    dst[0] = make_uint4(words[0], words[1], words[2], words[3]);
    dst[1] = make_uint4(words[4], words[5], words[6], words[7]);
}

// GGML get_scale_min_k4: 6-bit scale and min of sub-block j from scales[12].
__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t* q, uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = q[j] & 63u;
        m = q[j + 4] & 63u;
    } else {
        sc = (q[j + 4] & 0x0Fu) | ((uint32_t)(q[j - 4] >> 6) << 4);
        m = (uint32_t)(q[j + 4] >> 4) | ((uint32_t)(q[j] >> 6) << 4);
    }
}

// One thread per 32-weight sub-block of GGUF Q4_K (144-byte blocks {f16 d;
// f16 dmin; u8 scales[12]; u8 qs[128]}; 64-weight group g = j / 2 of a block
// takes qs[32 g .. 32 g + 31], low nibbles for sub-block 2 g, high for 2 g + 1)
// -> payload in Q4_0 order (signed q - 8), u16 (sc | m << 8), and for j = 0 the
// group header u32 (d | dmin << 16).
__global__ __launch_bounds__(256) void repack_q4k_kernel(const uint8_t* __restrict__ src,
                                                         uint8_t* __restrict__ base, int64_t rb,
                                                         int64_t kb, int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const int64_t row = i / kb, blk = i - row * kb;
    const int j = (int)(blk & 7);
    const uint8_t* b = src + (i >> 3) * 144;  // kb % 8 == 0: a row's groups are whole blocks
    uint32_t sc, m;
    q4k_scale_min(j, b + 4, sc, m);
    *const_cast<uint16_t*>(blk_scale<16>(base, rb, kb, row, blk)) = (uint16_t)(sc | (m << 8));
    if (j == 0)
        *const_cast<uint32_t*>(q4k_header(base, rb, kb, row, blk)) =
            (uint32_t)ld_u16(b) | ((uint32_t)ld_u16(b + 2) << 16);
    const uint8_t* qs = b + 16 + 32 * (j >> 1);
    const int sh = 4 * (j & 1);
    uint32_t words[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t v = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int e = 4 * w + t;  // byte e: element e (low), element e + 16 (high)
            const uint32_t lo = ((uint32_t)qs[e] >> sh) & 15u, hi = ((uint32_t)qs[e + 16] >> sh) & 15u;
            v |= ((lo ^ 8u) | ((hi ^ 8u) << 4)) << (8 * t);
        }
        words[w] = v;
    }
    *reinterpret_cast<uint4*>(const_cast<uint8_t*>(blk_payload<16>(base, rb, row, blk))) =
        make_uint4(words[0], words[1], words[2], words[3]);
}

// One thread per 32-weight sub-block j of GGUF Q5_K (176-byte blocks {f16 d; f16 dmin;
// u8 scales[12]; u8 qh[32]; u8 qs[128]}: sub-block j = 2 g + h takes nibble h of
// qs[32 g + l] and bit j of qh[l] for its weight l, GGML dequantize_row_q5_K) -> int8
// codes q - 16 in element order, u16 (sc | m << 8) and for j = 0 the group header
// u32 (d | dmin << 16), as Q4_K's.
__global__ __launch_bounds__(256) void repack_q5k_kernel(const uint8_t* __restrict__ src,
                                                         uint8_t* __restrict__ base, int64_t rb,
                                                         int64_t kb, int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const int64_t row = i / kb, blk = i - row * kb;
    const int j = (int)(blk & 7);
    const uint8_t* b = src + (i >> 3) * 176;
    uint32_t sc, m;
    q4k_scale_min(j, b + 4, sc, m);
    *const_cast<uint16_t*>(blk_scale<32>(base, rb, kb, row, blk)) = (uint16_t)(sc | (m << 8));
    if (j == 0)
        *const_cast<uint32_t*>(kq_header<32>(base, rb, kb, row, blk)) =
            (uint32_t)ld_u16(b) | ((uint32_t)ld_u16(b + 2) << 16);
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + 48 + 32 * (j >> 1);
    const int sh = 4 * (j & 1);
    uint32_t words[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        uint32_t v = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int l = 4 * w + u;
            const uint32_t q = (((uint32_t)qs[l] >> sh) & 15u) | ((((uint32_t)qh[l] >> j) & 1u) << 4);
            v |= ((q - 16u) & 0xFFu) << (8 * u);
        }
        words[w] = v;
    }
    uint4* dst = reinterpret_cast<uint4*>(const_cast<uint8_t*>(blk_payload<32>(base, rb, row, blk)));
    dst[0] = make_uint4(words[0], words[1], words[2], words[3]);
    dst[1] = make_uint4(words[4], words[5], words[6], words[7]);
}

// One thread per 32-weight block of GGUF Q6_K (210-byte blocks {u8 ql[128];
// u8 qh[64]; i8 scales[16]; f16 d}).  Weight e of a block (half h = e / 128,
// r = e % 128, t = r / 32, l = r % 32): q = (nibble t / 2 of ql[64 h + 32 (t % 2)
// + l]) | (bits 2 t .. 2 t + 1 of qh[32 h + l]) << 4, scale scales[e / 16]
// (GGML dequantize_row_q6_K) -> int8 codes q - 32, the two scales, and for the
// first block of a group the header d.
__global__ __launch_bounds__(256) void repack_q6k_kernel(const uint8_t* __restrict__ src,
                                                         uint8_t* __restrict__ base, int64_t rb,
                                                         int64_t kb, int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const int64_t row = i / kb, blk = i - row * kb;
    const int j = (int)(blk & 7);
    const uint8_t* b = src + (i >> 3) * 210;
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    *const_cast<uint16_t*>(blk_scale<32>(base, rb, kb, row, blk)) =
        (uint16_t)(b[192 + 2 * j] | (b[192 + 2 * j + 1] << 8));
    if (j == 0) *const_cast<uint32_t*>(kq_header<32>(base, rb, kb, row, blk)) = ld_u16(b + 208);
    uint32_t words[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        uint32_t v = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = 32 * j + 4 * w + u;
            const int h = e >> 7, r = e & 127, t = r >> 5, l = r & 31;
            const uint32_t lo = ((uint32_t)ql[64 * h + 32 * (t & 1) + l] >> (4 * (t >> 1))) & 15u;
            const uint32_t hi = ((uint32_t)qh[32 * h + l] >> (2 * t)) & 3u;
            v |= (((lo | (hi << 4)) - 32u) & 0xFFu) << (8 * u);
        }
        words[w] = v;
    }
    uint4* dst = reinterpret_cast<uint4*>(const_cast<uint8_t*>(blk_payload<32>(base, rb, row, blk)));
    dst[0] = make_uint4(words[0], words[1], words[2], words[3]);
    dst[1] = make_uint4(words[4], words[5], words[6], words[7]);
}

// Exact dequant (GGML to_float): Q4_0 w[j] = (lo(qs[j]) - 8) * d,
// w[j + 16] = (hi(qs[j]) - 8) * d (stored here as the signed nibbles q - 8);
// Q8_0 w[j] = qs[j] * d.  One thread per
// block.  Every product is exact in f32, so any evaluation order is bit-exact.
// Q4_K (dequantize_row_q4_K): w = (d sc) q - dmin m with q = nibble + 8; d sc
// and (d sc) q are exact in f32, so the subtraction is the one rounding, fused
// into a multiply-add or not.  Q5_K (dequantize_row_q5_K) the same with q = code + 16.
template <int QT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ base,
                                                      int64_t rb, int64_t kb,
                                                      float* __restrict__ out,
                                                      int64_t nblocks) {
    constexpr int QB =
        QT == UNILLM_QTYPE_Q8_0 || QT == UNILLM_QTYPE_Q5_K || QT == UNILLM_QTYPE_Q6_K ? 32 : 16;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const int64_t row = i / kb, blk = i - row * kb;
    const uint16_t sw = *blk_scale<QB>(base, rb, kb, row, blk);
    if constexpr (QT == UNILLM_QTYPE_Q5_K) {
        // (d sc) q - dmin m with q = code + 16, as Q4_K: (d sc) q exact, one rounding
        const uint32_t h = *kq_header<32>(base, rb, kb, row, blk);
        const float s = __half2float(__ushort_as_half((uint16_t)h)) * (float)(sw & 0xFFu);
        const float mn = __half2float(__ushort_as_half((uint16_t)(h >> 16))) * (float)(sw >> 8);
        const uint4* q = reinterpret_cast<const uint4*>(blk_payload<QB>(base, rb, row, blk));
        float4* o = reinterpret_cast<float4*>(out + i * QK);
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const uint4 qq = q[v];
            const uint32_t w[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float f[4];
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    f[b] = s * (float)((int)(int8_t)(w[t] >> (8 * b)) + 16) - mn;
                o[4 * v + t] = make_float4(f[0], f[1], f[2], f[3]);
            }
        }
        return;
    }
    if constexpr (QT == UNILLM_QTYPE_Q6_K) {
        // (d sc) (q - 32), as GGML evaluates it: d sc exact, the second product rounds once
        const float d = __half2float(__ushort_as_half((uint16_t)*kq_header<32>(base, rb, kb, row, blk)));
        const float s0 = d * (float)(int8_t)(sw & 0xFFu), s1 = d * (float)(int8_t)(sw >> 8);
        const uint4* q = reinterpret_cast<const uint4*>(blk_payload<QB>(base, rb, row, blk));
        float4* o = reinterpret_cast<float4*>(out + i * QK);
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const uint4 qq = q[v];
            const uint32_t w[4] = {qq.x, qq.y, qq.z, qq.w};
            const float sv = v ? s1 : s0;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float f[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) f[b] = __fmul_rn(sv, (float)(int8_t)(w[t] >> (8 * b)));
                o[4 * v + t] = make_float4(f[0], f[1], f[2], f[3]);
            }
        }
        return;
    }
    const uint8_t* qs = blk_payload<QB>(base, rb, row, blk);
    float4* o = reinterpret_cast<float4*>(out + i * QK);
    if constexpr (QT == UNILLM_QTYPE_Q4_K) {
        const uint32_t h = *q4k_header(base, rb, kb, row, blk);
        const float s = __half2float(__ushort_as_half((uint16_t)h)) * (float)(sw & 0xFFu);
        const float mn = __half2float(__ushort_as_half((uint16_t)(h >> 16))) * (float)(sw >> 8);
        const uint4 q = *reinterpret_cast<const uint4*>(qs);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float lo[4], hi[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t byte = (w[t] >> (8 * b)) & 0xFFu;
                lo[b] = s * (float)((byte & 15u) ^ 8u) - mn;  // code q = (q - 8) ^ 8
                hi[b] = s * (float)((byte >> 4) ^ 8u) - mn;
            }
            o[t] = make_float4(lo[0], lo[1], lo[2], lo[3]);
            o[4 + t] = make_float4(hi[0], hi[1], hi[2], hi[3]);
        }
        return;
    }
    const float d = __half2float(__ushort_as_half(sw));
    if constexpr (QT == UNILLM_QTYPE_Q4_0) {
        const uint4 q = *reinterpret_cast<const uint4*>(qs);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float lo[4], hi[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const uint32_t byte = (w[t] >> (8 * b)) & 0xFFu;
                lo[b] = (float)(((int)(byte << 28)) >> 28) * d;  // signed nibble q - 8
                hi[b] = (float)(((int)(byte << 24)) >> 28) * d;
            }
            o[t] = make_float4(lo[0], lo[1], lo[2], lo[3]);
            o[4 + t] = make_float4(hi[0], hi[1], hi[2], hi[3]);
        }
    } else {
        const uint4* q = reinterpret_cast<const uint4*>(qs);
#pragma unroll
        for (int v = 0; v < 2; ++v) {
            const uint4 qq = q[v];
            const uint32_t w[4] = {qq.x, qq.y, qq.z, qq.w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                float f[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) f[b] = (float)(int8_t)(w[t] >> (8 * b)) * d;
                o[4 * v + t] = make_float4(f[0], f[1], f[2], f[3]);
            }
        }
    }
}

// GGML reference quantizers (quantize_row_q4_0_ref / q8_0_ref, which candle's
// BlockQ4_0/BlockQ8_0::from_float restate).  Explicit _rn intrinsics keep the
// multiply and the add separately rounded, as the reference does: a fused
// multiply-add here would change which side of x.5 some values fall on.
template <int QT>
__global__ __launch_bounds__(256) void quantize_kernel(const float* __restrict__ w,
                                                       uint8_t* __restrict__ out,
                                                       int64_t nblocks) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float4* src = reinterpret_cast<const float4*>(w + i * QK);
    float x[QK];
#pragma unroll
    for (int v = 0; v < 8; ++v) {
        const float4 f = src[v];
        x[4 * v] = f.x; x[4 * v + 1] = f.y; x[4 * v + 2] = f.z; x[4 * v + 3] = f.w;
    }
    constexpr int BB = QT == UNILLM_QTYPE_Q4_0 ? 18 : 34;
    uint8_t* o = out + i * BB;
    if constexpr (QT == UNILLM_QTYPE_Q4_0) {
        float amax = 0.0f, mx = 0.0f;
#pragma unroll
        for (int j = 0; j < QK; ++j) {  // first element of largest magnitude, signed
            const float a = fabsf(x[j]);
            if (amax < a) { amax = a; mx = x[j]; }
        }
        // d = mx / -8 is exact in f32.  An all-zero block keeps mx = +0, so GGML
        // stores d = -0.0 (f16 0x8000); that case is written explicitly because
        // the compiler folds the product into the f16 conversion as
        // fma(mx, -0.125, +0), whose zero result is +0.
        const float d = __fmul_rn(mx, -0.125f);
        const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
        const uint16_t dh = amax == 0.0f ? (uint16_t)0x8000u
                                         : __half_as_ushort(__float2half_rn(d));
        o[0] = (uint8_t)dh;
        o[1] = (uint8_t)(dh >> 8);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            int q0 = (int)(int8_t)(int)__fadd_rn(__fmul_rn(x[j], id), 8.5f);
            int q1 = (int)(int8_t)(int)__fadd_rn(__fmul_rn(x[j + 16], id), 8.5f);
            q0 = q0 > 15 ? 15 : q0;
            q1 = q1 > 15 ? 15 : q1;
            o[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    } else {
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < QK; ++j) amax = fmaxf(amax, fabsf(x[j]));
        const float d = __fdiv_rn(amax, 127.0f);
        const float id = d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f;
        const uint16_t dh = __half_as_ushort(__float2half_rn(d));
        o[0] = (uint8_t)dh;
        o[1] = (uint8_t)(dh >> 8);
#pragma unroll
        for (int j = 0; j < QK; ++j) o[2 + j] = (uint8_t)(int8_t)roundf(__fmul_rn(x[j], id));
    }
}

// max |d| over the scale plane, as f16 magnitude bits (monotone in |d| for
// finite values).  Used once per weight to pick the f16 exponent offset.
template <int QB>
__global__ __launch_bounds__(256) void scale_absmax_kernel(const uint8_t* __restrict__ base,
                                                           int64_t rb, int64_t kb, int64_t count,
                                                           uint32_t* __restrict__ out) {
    __shared__ uint32_t part[256];
    uint32_t m = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / kb;
        m = max(m, (uint32_t)(*blk_scale<QB>(base, rb, kb, row, i - row * kb) & 0x7FFFu));
    }
    part[threadIdx.x] = m;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) part[threadIdx.x] = max(part[threadIdx.x], part[threadIdx.x + s]);
        __syncthreads();
    }
    if (threadIdx.x == 0) atomicMax(out, part[0]);
}

// Q4_K (QB 16), Q5_K (QB 32): max |d| and max |dmin| over the group headers, as f16
// magnitude bits.
template <int QB>
__global__ __launch_bounds__(256) void q4k_header_absmax_kernel(const uint8_t* __restrict__ base,
                                                                int64_t rb, int64_t kb,
                                                                int64_t count,
                                                                uint32_t* __restrict__ out) {
    __shared__ uint32_t part[2][256];
    uint32_t md = 0, mm = 0;
    const int64_t groups = kb / 8;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / groups;
        const uint32_t h = *kq_header<QB>(base, rb, kb, row, 8 * (i - row * groups));
        md = max(md, h & 0x7FFFu);
        mm = max(mm, (h >> 16) & 0x7FFFu);
    }
    part[0][threadIdx.x] = md;
    part[1][threadIdx.x] = mm;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            part[0][threadIdx.x] = max(part[0][threadIdx.x], part[0][threadIdx.x + s]);
            part[1][threadIdx.x] = max(part[1][threadIdx.x], part[1][threadIdx.x + s]);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        atomicMax(out, part[0][0]);
        atomicMax(out + 1, part[1][0]);
    }
}

// Q6_K: max |d| over the group headers.
__global__ __launch_bounds__(256) void q6k_header_absmax_kernel(const uint8_t* __restrict__ base,
                                                                int64_t rb, int64_t kb,
                                                                int64_t count,
                                                                uint32_t* __restrict__ out) {
    __shared__ uint32_t part[256];
    uint32_t md = 0;
    const int64_t groups = kb / 8;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / groups;
        md = max(md, *kq_header<32>(base, rb, kb, row, 8 * (i - row * groups)) & 0x7FFFu);
    }
    part[threadIdx.x] = md;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) part[threadIdx.x] = max(part[threadIdx.x], part[threadIdx.x + s]);
        __syncthreads();
    }
    if (threadIdx.x == 0) atomicMax(out, part[0]);
}

inline unsigned grid_for(int64_t items, int block) {
    return (unsigned)((items + block - 1) / block);
}

}  // namespace

hipError_t launch_repack(const QWeight& w, const uint8_t* gguf, hipStream_t s) {
    const int64_t nb = w.n * w.kb;
    if (w.src_qtype == UNILLM_QTYPE_Q5_0)
        repack_q5_0_kernel<<<grid_for(nb, 256), 256, 0, s>>>(gguf, w.base, w.row_bytes, w.kb, nb);
    else if (w.qtype == UNILLM_QTYPE_Q4_K)
        repack_q4k_kernel<<<grid_for(nb, 256), 256, 0, s>>>(gguf, w.base, w.row_bytes, w.kb, nb);
    else if (w.qtype == UNILLM_QTYPE_Q5_K)
        repack_q5k_kernel<<<grid_for(nb, 256), 256, 0, s>>>(gguf, w.base, w.row_bytes, w.kb, nb);
    else if (w.qtype == UNILLM_QTYPE_Q6_K)
        repack_q6k_kernel<<<grid_for(nb, 256), 256, 0, s>>>(gguf, w.base, w.row_bytes, w.kb, nb);
    else if (w.qtype == UNILLM_QTYPE_Q4_0)
        repack_kernel<16><<<grid_for(nb, 256), 256, 0, s>>>(gguf, w.base, w.row_bytes, w.kb, nb);
    else
        repack_kernel<32><<<grid_for(nb, 256), 256, 0, s>>>(gguf, w.base, w.row_bytes, w.kb, nb);
    return hipGetLastError();
}

hipError_t launch_scale_absmax(const QWeight& w, uint32_t* out, hipStream_t s) {
    const int64_t nb = w.n * w.kb;
    const unsigned grid = (unsigned)std::min<int64_t>(1024, (nb + 255) / 256);
    if (w.qtype == UNILLM_QTYPE_Q4_K)
        q4k_header_absmax_kernel<16><<<grid, 256, 0, s>>>(w.base, w.row_bytes, w.kb, nb / 8, out);
    else if (w.qtype == UNILLM_QTYPE_Q5_K)
        q4k_header_absmax_kernel<32><<<grid, 256, 0, s>>>(w.base, w.row_bytes, w.kb, nb / 8, out);
    else if (w.qtype == UNILLM_QTYPE_Q6_K)
        q6k_header_absmax_kernel<<<grid, 256, 0, s>>>(w.base, w.row_bytes, w.kb, nb / 8, out);
    else if (w.qtype == UNILLM_QTYPE_Q4_0)
        scale_absmax_kernel<16><<<grid, 256, 0, s>>>(w.base, w.row_bytes, w.kb, nb, out);
    else
        scale_absmax_kernel<32><<<grid, 256, 0, s>>>(w.base, w.row_bytes, w.kb, nb, out);
    return hipGetLastError();
}

hipError_t launch_dequant(const QWeight& w, float* out, hipStream_t s) {
    const int64_t nb = w.n * w.kb;
    if (w.qtype == UNILLM_QTYPE_Q4_K)
        dequant_kernel<UNILLM_QTYPE_Q4_K><<<grid_for(nb, 256), 256, 0, s>>>(w.base, w.row_bytes,
                                                                            w.kb, out, nb);
    else if (w.qtype == UNILLM_QTYPE_Q5_K)
        dequant_kernel<UNILLM_QTYPE_Q5_K><<<grid_for(nb, 256), 256, 0, s>>>(w.base, w.row_bytes,
                                                                            w.kb, out, nb);
    else if (w.qtype == UNILLM_QTYPE_Q6_K)
        dequant_kernel<UNILLM_QTYPE_Q6_K><<<grid_for(nb, 256), 256, 0, s>>>(w.base, w.row_bytes,
                                                                            w.kb, out, nb);
    else if (w.qtype == UNILLM_QTYPE_Q4_0)
        dequant_kernel<UNILLM_QTYPE_Q4_0><<<grid_for(nb, 256), 256, 0, s>>>(w.base, w.row_bytes,
                                                                            w.kb, out, nb);
    else
        dequant_kernel<UNILLM_QTYPE_Q8_0><<<grid_for(nb, 256), 256, 0, s>>>(w.base, w.row_bytes,
                                                                            w.kb, out, nb);
    return hipGetLastError();
}

hipError_t launch_quantize(int qtype, const float* w, int64_t n, int64_t k, uint8_t* out,
                           hipStream_t s) {
    if (qtype != UNILLM_QTYPE_Q4_0 && qtype != UNILLM_QTYPE_Q8_0) return hipErrorInvalidValue;
    const int64_t nb = n * (k / QK);
    if (qtype == UNILLM_QTYPE_Q4_0)
        quantize_kernel<UNILLM_QTYPE_Q4_0><<<grid_for(nb, 256), 256, 0, s>>>(w, out, nb);
    else
        quantize_kernel<UNILLM_QTYPE_Q8_0><<<grid_for(nb, 256), 256, 0, s>>>(w, out, nb);
    return hipGetLastError();
}

}  // namespace unillm
