// decode.hip -- batched decode (5 <= m <= 64): fused dequant + f16 MFMA.
//
// y[m, n] = x[m, k] . dequant(W)[n, k]^T for continuous-batching widths, the
// QMatMul::forward call of llama.rs:1188 / 1329 with a few tokens per step.
// Bound: HBM for the weights (each byte read once) with the dequant VALU
// close behind; the tokens are few, so the matrix cores have slack.
//
// Orientation: the weights are the MFMA A operand (16 weight rows x 32 k, one
// Q4_0 / Q8_0 block per row and fragment) and the tokens the B operand, so
// C = W . x^T is [16 rows][16 tokens] per tile (v_mfma_f32_16x16x32_f16).
//   - A workgroup of 4 waves owns 64 weight rows; wave w owns rows 16 w ..
//     16 w + 15 over all of k.  Each lane loads exactly the 8 payload bytes
//     behind its A fragment (row l % 16, elements 8 (l / 16) .. +7 of the
//     block) and the row's scales, three 256-k chunks ahead, and dequantizes them
//     in registers to f16 with packed f16 arithmetic:
//       (code | 0x6400) is the f16 1024 + code (exact), minus 1024 + offset
//       gives the signed code exactly, times d 2^-E rounds once
//     -- the same single rounding as (q - 8) d 2^-E computed in fp32 and
//     rounded to f16.  Codes are taken two at a time from bytes (0, 2) and
//     (1, 3) of a dword, so a fragment holds its 8 elements in the order
//     0 2 1 3 4 6 5 7; x is staged in that same order, which leaves every dot
//     product unchanged.
//   - x (f32) is rounded to f16 and staged per 256-k chunk in LDS, shared by
//     the workgroup's 4 waves (double-buffered, loaded one chunk ahead).
//   - E is the weight's f16 exponent offset (8 max|d| 2^-E <= 65504), undone
//     on the output: both scalings are exact.
// Normwise error vs the f64 oracle ~3e-4 (f16 operands; bound 1e-3).
#include <hip/hip_fp16.h>

#include <algorithm>

#include "internal.hpp"
#include "lds.hpp"

namespace unillm {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int DROWS = 64;       // weight rows per workgroup (4 waves x 16)

__device__ __forceinline__ uint32_t pk_f16(float a, float b) {
    uint32_t r;  // round to nearest even, a in the low half
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// Two codes (bytes 0 and 2 of `sel`, already masked to the code bits) -> f16 pair
// (code - bias) * dh: 0x6400 | code is 1024 + code exactly.
__device__ __forceinline__ uint32_t codes2(uint32_t sel, f16x2 bias, f16x2 dh) {
    const f16x2 v = __builtin_bit_cast(f16x2, sel | 0x64006400u);
    return __builtin_bit_cast(uint32_t, (v - bias) * dh);
}

// One lane's A fragment of one block: 8 bytes of payload -> 8 f16 in the order
// 0 2 1 3 4 6 5 7.  Q4_0: nibbles at bit offset `shift` of each byte (signed
// codes stored as q - 8, flipped back to q); Q8_0: whole bytes (flipped to q + 128).
template <int QT>
__device__ __forceinline__ f16x8 dequant_frag(u32x2 raw, int shift, f16x2 dh) {
    constexpr uint32_t kFlip = QT == UNILLM_QTYPE_Q4_0 ? 0x88888888u : 0x80808080u;
    constexpr uint32_t kMask = QT == UNILLM_QTYPE_Q4_0 ? 0x000F000Fu : 0x00FF00FFu;
    const _Float16 b = QT == UNILLM_QTYPE_Q4_0 ? (_Float16)1032.0f : (_Float16)1152.0f;
    const f16x2 bias = {b, b};
    u32x4 out;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t w = (raw[h] ^ kFlip) >> shift;
        out[2 * h] = codes2(w & kMask, bias, dh);               // bytes 0, 2
        out[2 * h + 1] = codes2((w >> 8) & kMask, bias, dh);    // bytes 1, 3
    }
    return __builtin_bit_cast(f16x8, out);
}

// x ring: S stages of one 128-k chunk of TOK token rows in f32 (512 B per row),
// filled by direct global -> LDS loads (a 1 KiB load covers two rows).  The
// 16-byte chunk c of row r sits in slot c ^ (r % 16), so the 16 rows a
// fragment read touches fall on distinct banks.
constexpr int DKC = 128;  // k per chunk (4 blocks)
constexpr int DS = 3;     // stages: chunks ch + 1, ch + 2 in flight while ch is used

template <int MT>
struct XRing {
    static constexpr int TOK = MT * 16;
    static constexpr int STAGE = TOK * DKC * 4;
    static constexpr int BYTES = DS * STAGE;
    static constexpr int DMA = TOK * DKC * 4 / 1024 / 4;  // direct loads per wave per chunk
};

template <int QT, int MT>
__global__ __launch_bounds__(256) void decode_kernel(const uint8_t* __restrict__ base, int64_t rb,
                                                     const float* __restrict__ x,
                                                     float* __restrict__ y, int M, int N, int KB,
                                                     float wscale, float oscale) {
    constexpr int QB = QT == UNILLM_QTYPE_Q4_0 ? 16 : 32;  // payload bytes per block
    using XR = XRing<MT>;
    constexpr int LPC = XR::DMA + 5;  // a wave's loads per chunk: x + 4 payloads + scales
    extern __shared__ __attribute__((aligned(16))) uint8_t xring[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane / 16, fr = lane % 16;
    const uint32_t K = (uint32_t)KB * QK;
    const int chunks = (KB + 3) / 4;

    // ---- weights: row 64 blockIdx + 16 wv + fr; bytes 8 (g & 1) .. +7 of each block
    // (Q4_0, nibble shift 4 (g >> 1)) or 8 g .. +7 (Q8_0).  32-bit byte offsets.
    const int row = blockIdx.x * DROWS + wv * 16 + fr;
    const bool rval = row < N;
    const uint32_t roff = (uint32_t)min(row, N - 1) * (uint32_t)rb;
    const uint32_t boff = QT == UNILLM_QTYPE_Q4_0 ? 8 * (g & 1) : 8 * g;
    const int bshift = QT == UNILLM_QTYPE_Q4_0 ? 4 * (g >> 1) : 0;
    const uint32_t sbase = (uint32_t)KB * QB;

    // ---- x: this wave's direct loads q = XR::DMA wv .. : rows 2 q + lane / 32, slot
    // lane % 32 <- global chunk (lane % 32) ^ (row % 16).  Rows past m read row m - 1
    // and k past K the row's last chunk (finite values against zero weights).
    uint32_t xrow[XR::DMA], xchunk[XR::DMA];
#pragma unroll
    for (int q = 0; q < XR::DMA; ++q) {
        const int r = 2 * (XR::DMA * wv + q) + lane / 32;
        xrow[q] = (uint32_t)min(r, M - 1) * K;
        xchunk[q] = (uint32_t)(((lane % 32) ^ (r % 16)) * 4);
    }

    struct WChunk {
        u32x2 p[4];  // the 4 blocks' fragment bytes
        u32x2 s;     // the 4 blocks' f16 scales
    };
    auto issue = [&](WChunk& c, int ch) {  // this wave's LPC loads of chunk ch
        uint8_t* st = xring + (ch % DS) * XR::STAGE;
#pragma unroll
        for (int q = 0; q < XR::DMA; ++q)
            dma16(x + xrow[q] + min((uint32_t)ch * DKC + xchunk[q], K - 4),
                  st + (XR::DMA * wv + q) * 1024);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t kb = (uint32_t)min(4 * ch + b, KB - 1);
            c.p[b] = *reinterpret_cast<const u32x2*>(base + roff + kb * QB + boff);
        }
        // scales of blocks 4 ch .. 4 ch + 3 (8-byte aligned); a partial last chunk
        // reads past the row's scales only inside the row padding, the next row or
        // the weight's tail slot, and those blocks get d = 0
        c.s = *reinterpret_cast<const u32x2*>(base + roff + sbase + 8u * ch);
    };

    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // LDS byte offset of this lane's x fragment (token 16 t + fr, k 32 b + 8 g, i.e.
    // chunks 8 b + 2 g and 8 b + 2 g + 1 of the row): row and the pair of slots
    const uint32_t ring0 = (uint32_t)(uintptr_t)xring;
    auto compute = [&](const WChunk& c, int ch) {
        const uint32_t st = ring0 + (uint32_t)((ch % DS) * XR::STAGE);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const bool bok = rval && 4 * ch + b < KB;
            const uint16_t sb = (uint16_t)(c.s[b / 2] >> (16 * (b % 2)));
            const _Float16 d = bok ? (_Float16)(__half2float(__ushort_as_half(sb)) * wscale)
                                   : (_Float16)0.0f;
            const f16x2 dh = {d, d};
            const f16x8 a = dequant_frag<QT>(c.p[b], bshift, dh);
            const uint32_t c0 = (uint32_t)(((8 * b + 2 * g) ^ fr) * 16);
            const uint32_t c1 = (uint32_t)(((8 * b + 2 * g + 1) ^ fr) * 16);
            lds_u32x4 lo[MT], hi[MT];
            constexpr_for<MT>([&](auto T) {
                constexpr int t = T.value;
                lo[t] = lds_read128<t * 16 * 512>(st + fr * 512 + c0);
                hi[t] = lds_read128<t * 16 * 512>(st + fr * 512 + c1);
            });
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                asm volatile("" : "+v"(lo[t]), "+v"(hi[t]));
                const float* f0 = reinterpret_cast<const float*>(&lo[t]);
                const float* f1 = reinterpret_cast<const float*>(&hi[t]);
                const u32x4 h = {pk_f16(f0[0], f0[2]), pk_f16(f0[1], f0[3]),
                                 pk_f16(f1[0], f1[2]), pk_f16(f1[1], f1[3])};
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(f16x8, h),
                                                                acc[t], 0, 0, 0);
            }
        }
    };

    // chunks 0 .. DS - 2 in flight; step ch waits for its own loads (the later chunk
    // may stay in flight), meets the other waves (its x chunk is then complete),
    // issues chunk ch + DS - 1 and computes.  Steady state unconditionally; the
    // last chunks in a separate tail.
    WChunk wc[DS];
#pragma unroll
    for (int d = 0; d < DS - 1; ++d) issue(wc[d], min(d, chunks - 1));
    auto step = [&](WChunk& cur, WChunk& next, int ch, bool last) {
        if (last) wait_vmcnt<0>();
        else wait_vmcnt<LPC * (DS - 2)>();
        __builtin_amdgcn_s_barrier();
        if (ch + DS - 1 < chunks) issue(next, ch + DS - 1);
        compute(cur, ch);
    };
    int c0 = 0;
    for (; c0 + 2 * DS <= chunks; c0 += DS) {
#pragma unroll
        for (int d = 0; d < DS; ++d) step(wc[d], wc[(d + DS - 1) % DS], c0 + d, false);
    }
#pragma unroll
    for (int d = 0; d < 2 * DS; ++d)
        if (c0 + d < chunks)
            step(wc[d % DS], wc[(d + DS - 1) % DS], c0 + d, c0 + d + 1 >= chunks);

    // ---- epilogue: lane holds C[4 g + e][fr] = y[token 16 t + fr][row 4 g + e] ----
    const int rbase = blockIdx.x * DROWS + wv * 16 + 4 * g;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int m = 16 * t + fr;
        if (m >= M) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (rbase + e < N) y[(int64_t)m * N + rbase + e] = acc[t][e] * oscale;
    }
}

template <int QT, int MT>
hipError_t launch_mt(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t s) {
    static const bool attr = hipFuncSetAttribute((const void*)decode_kernel<QT, MT>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 XRing<MT>::BYTES) == hipSuccess;
    if (!attr) return hipErrorInvalidValue;
    const float wscale = ldexpf(1.0f, -w.f16_exp), oscale = ldexpf(1.0f, w.f16_exp);
    const int grid = (int)((w.n + DROWS - 1) / DROWS);
    decode_kernel<QT, MT><<<grid, 256, XRing<MT>::BYTES, s>>>(w.base, w.row_bytes, x, y, (int)m,
                                                              (int)w.n, (int)w.kb, wscale, oscale);
    return hipGetLastError();
}

template <int QT>
hipError_t launch_qt(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t s) {
    if (m <= 16) return launch_mt<QT, 1>(w, x, m, y, s);
    if (m <= 32) return launch_mt<QT, 2>(w, x, m, y, s);
    if (m <= 48) return launch_mt<QT, 3>(w, x, m, y, s);
    return launch_mt<QT, 4>(w, x, m, y, s);
}

}  // namespace

// m in [1, 64]; x is addressed with 32-bit offsets (m k < 2^30 always holds here).
hipError_t launch_decode_mfma(const QWeight& w, const float* x, int64_t m, float* y,
                              hipStream_t s) {
    if (w.qtype == UNILLM_QTYPE_Q4_0) return launch_qt<UNILLM_QTYPE_Q4_0>(w, x, m, y, s);
    return launch_qt<UNILLM_QTYPE_Q8_0>(w, x, m, y, s);
}

}  // namespace unillm
