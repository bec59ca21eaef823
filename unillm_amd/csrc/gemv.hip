// gemv.hip -- fused dequant + GEMV for decode (m <= 4).
//
// What it computes: y[m, n] = sum_k x[m, k] * dequant(W)[n, k], the decode
// step of QMatMul::forward (crates/runtime/src/models_v2/llama.rs:1188) for
// one to four tokens.  Bound: HBM -- each weight byte is read once; the
// arithmetic intensity is ~3.6 flop/B per token (Q4_0).
//
// Arithmetic.  The weight codes are exact small integers, so each block's dot
// product with x is computed as an exact int32 sum and scaled once.  x is
// turned, per 32-element block, into integers T_j over a power-of-two scale:
//   Q4_0: x_j ~= sx * T_j, T_j = rint(x_j / s * 2^12), max|x| / 7 < s <= 2 max|x| / 7,
//         sx = s * 2^-12 (|T_j| <= 7 * 2^12; error <= s * 2^-13 <= max|x| / 28672).
//         T_j is written as four balanced base-16 digits in [-8, 7], so with the
//         weight nibbles stored as the signed values q - 8 one v_dot8_i32_i4
//         takes eight weights against one digit of eight x values, with no
//         unpacking: A = sum_j (q_j - 8) T_j = sum_k 16^k sum_j (q_j - 8) d_kj
//         (16 dot8 per block, |A| < 2^24).
//   Q8_0: x_j ~= sx * (254 d0_j + d1_j), d0 = rint(x / s), d1 = rint((x / s - d0) * 254),
//         max|x| / 127 < s <= 2 max|x| / 127, sx = s / 254; v_dot4_i32_i8 against each
//         int8 digit, A = 254 sum q d0 + sum q d1 (error <= s / 508 <= max|x| / 32258).
// x / s is exact (a power-of-two scale), so scaling x by a power of two scales
// y exactly.  Block results are scaled by d_w * sx and summed in fp32;
// normwise error vs the f64 oracle is ~3e-5 (bound 1e-3).
//
// Why integers: a wave64 VALU instruction occupies a gfx950 SIMD for about
// four cycles (fp32 FMA and the dot instructions alike, measured), so the
// decode GEMV is VALU-heavy unless each instruction covers many weights.
// dot8 covers 8 Q4_0 weights per digit; the inner loop is ~22 instructions per
// 32-weight block (vs ~64 for an fp32 dequant-FMA).
//
// Mapping (MI355X, wave64).  One workgroup per CU (1024 threads, or 512 where
// a lane needs more than 128 VGPRs); wave w owns rows w, w + W, w + 2W, ...
// (so the rows requested at one moment form one contiguous stretch of the
// matrix), R rows per chunk, and lane l owns blocks l, l + 64, ... of every
// row (a wave-wide 128-bit load reads 1 KiB of contiguous Q4_0 payload).
//   1. every wave requests x (the waves that hold x quarters) and its first
//      chunk of weights;
//   2. the workgroup turns x into digit records in LDS, four threads per
//      32-block, once per CU, while that chunk streams in;
//   3. each lane reads its records into registers, requests its second chunk
//      (when it has more rows), then computes chunk by chunk.
// Instructions issue in order, and once loads back up in the memory pipeline
// everything behind them waits until they are accepted -- so a wave requests
// only one chunk before the digit work, and x before its weights.  Every
// load is branch-free (indices are clamped, validity is applied through the
// x scale), so a memory wait never covers more loads than it needs.  Row
// partials are reduced with DPP rotations and two cross-row shuffles.
#include <hip/hip_fp16.h>

#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "internal.hpp"

namespace unillm {
namespace {

// LDS dwords per x block: 16 digit dwords + sx (17 used; 20 keeps the
// 128-bit reads of the 64 lanes of a wave spread over the banks)
constexpr int kXWords = 20;
constexpr float kRound = 12582912.0f;   // 1.5 * 2^23: t + kRound rounds t to an integer
// kRound + 0x8888: the low 16 bits of (t + kRound4) are rint(t) + 0x8888
constexpr float kRound4 = 12582912.0f + 34952.0f;

template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, dpp_i32<CTRL>(__builtin_bit_cast(int, v)));
}

// Sum over the 64 lanes; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x124>(v);  // row_ror:4
    v += dpp_f32<0x128>(v);  // row_ror:8 -> every lane holds its 16-lane row sum
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

__device__ __forceinline__ int sdot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}
__device__ __forceinline__ int sdot8(int a, int b, int c) {
    return __builtin_amdgcn_sdot8(a, b, c, false);
}

// Low bytes of four registers -> one dword (v_perm_b32 selects bytes; 0x0C = zero).
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t a0, uint32_t a1, uint32_t a2,
                                                   uint32_t a3) {
    return __builtin_amdgcn_perm(a1, a0, 0x0C0C0400u) | __builtin_amdgcn_perm(a3, a2, 0x04000C0Cu);
}

// Bits of a where m is set, of b elsewhere (v_bfi_b32).
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) {
    return (m & a) | (~m & b);
}

// Max of |v| over the 8 values of this thread and its DPP quad.
__device__ __forceinline__ float quad_absmax(const float (&v)[8]) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, dpp_f32<0xB1>(amax));
    return fmaxf(amax, dpp_f32<0x4E>(amax));
}

// ---- x digit records -------------------------------------------------------------------------
// One record per 32-element x block (kXWords dwords in LDS), built by the four
// threads of a DPP quad (one per weight-payload dword t = 0..3), in the
// operand order of the weight payload so that payload dword t meets digit
// dword t:
//   Q4_0: dwords 4L + t (L = 0..3) hold digit 3 - L of the eight elements of
//         payload dword t, in its nibble order 4t, 4t+16, 4t+1, 4t+17, ...;
//         dword 16 = sx.
//   Q8_0: dwords 0-7 digit d0 of elements 4t..4t+3 (t = 0..7), 8-15 digit d1,
//         dword 16 = sx.
//
// The math runs on every thread and only the stores are conditional, so the
// compiler keeps the x loads where they are issued.

// Q4_0: v[2i] = x[4t + i], v[2i + 1] = x[16 + 4t + i] (i = 0..3).  SUM (Q4_K):
// dword 17 = the block's sum of x, for the term (8 d sc - dmin m) sum x.
template <bool SUM = false>
__device__ __forceinline__ void prep_q4(const float (&v)[8], int t, bool store,
                                        uint32_t* __restrict__ dst) {
    const float amax = quad_absmax(v);
    float xsum = 0.0f;
    if constexpr (SUM) {
#pragma unroll
        for (int j = 0; j < 8; ++j) xsum += v[j];
        xsum += dpp_f32<0xB1>(xsum);
        xsum += dpp_f32<0x4E>(xsum);
    }
    // s = 2^e with max|x| / 7 < s: frexp gives max|x| / 7 = f * 2^e, f in [0.5, 1);
    // e >= -100 keeps 2^(12 - e) finite (blocks below 2^-100 round to zero)
    int e = 0;
    (void)frexpf(amax * (1.0f / 7.0f), &e);
    e = max(e, -100);
    const float inv = amax > 0.0f ? ldexpf(1.0f, 12 - e) : 0.0f;
    // low 16 bits of a[j]: U_j = T_j + 0x8888, T_j = rint(x_j * 2^12 / s) (one rounding:
    // the product is exact).  For balanced digits, U = sum_k (d_k + 8) 16^k, so
    // nibble k of U is digit k XOR 8 (its 4-bit two's complement pattern, XOR 8).
    uint32_t a[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = __float_as_uint(fmaf(v[j], inv, kRound4));
    // nibble transpose: P[i] byte 0 = nibble 0 of a[2i] | nibble 0 of a[2i+1] << 4,
    // byte 1 = the same for nibble 2; Q[i] the same for nibbles 1 and 3
    uint32_t P[4], Q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        P[i] = bfi(0x0F0Fu, a[2 * i], a[2 * i + 1] << 4);
        Q[i] = bfi(0x0F0Fu, a[2 * i] >> 4, a[2 * i + 1]);
    }
    const uint32_t P01 = __builtin_amdgcn_perm(P[1], P[0], 0x05010400u);
    const uint32_t P23 = __builtin_amdgcn_perm(P[3], P[2], 0x05010400u);
    const uint32_t Q01 = __builtin_amdgcn_perm(Q[1], Q[0], 0x05010400u);
    const uint32_t Q23 = __builtin_amdgcn_perm(Q[3], Q[2], 0x05010400u);
    const uint32_t d0 = __builtin_amdgcn_perm(P23, P01, 0x05040100u) ^ 0x88888888u;
    const uint32_t d2 = __builtin_amdgcn_perm(P23, P01, 0x07060302u) ^ 0x88888888u;
    const uint32_t d1 = __builtin_amdgcn_perm(Q23, Q01, 0x05040100u) ^ 0x88888888u;
    const uint32_t d3 = __builtin_amdgcn_perm(Q23, Q01, 0x07060302u) ^ 0x88888888u;
    if (!store) return;
    dst[t] = d3;
    dst[4 + t] = d2;
    dst[8 + t] = d1;
    dst[12 + t] = d0;
    if (t == 0) dst[16] = __float_as_uint(amax > 0.0f ? ldexpf(1.0f, e - 12) : 0.0f);
    if (SUM && t == 0) dst[17] = __float_as_uint(xsum);
}

// Q8_0: v[j] = x[8u + j], u = quarter 0..3.  SUM (Q5_K): dword 17 = the block's sum
// of x, for the term (16 d sc - dmin m) sum x.
template <bool SUM = false>
__device__ __forceinline__ void prep_q8(const float (&v)[8], int u, bool store,
                                        uint32_t* __restrict__ dst) {
    const float amax = quad_absmax(v);
    float xsum = 0.0f;
    if constexpr (SUM) {
#pragma unroll
        for (int j = 0; j < 8; ++j) xsum += v[j];
        xsum += dpp_f32<0xB1>(xsum);
        xsum += dpp_f32<0x4E>(xsum);
    }
    // s = 2^e with max|x| / 127 < s
    int e = 0;
    (void)frexpf(amax * (1.0f / 127.0f), &e);
    e = max(e, -100);
    const float inv = amax > 0.0f ? ldexpf(1.0f, -e) : 0.0f;
    uint32_t b0[8], b1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float t = v[j] * inv;                     // exact, |t| < 127
        const float a = t + kRound;                     // low byte: rint(t) as int8
        const float r = t - (a - kRound);               // exact, |r| <= 1/2
        b0[j] = __float_as_uint(a);
        b1[j] = __float_as_uint(fmaf(r, 254.0f, kRound));  // low byte: rint(254 r)
    }
    if (!store) return;
    dst[2 * u] = pack_low_bytes(b0[0], b0[1], b0[2], b0[3]);
    dst[2 * u + 1] = pack_low_bytes(b0[4], b0[5], b0[6], b0[7]);
    dst[8 + 2 * u] = pack_low_bytes(b1[0], b1[1], b1[2], b1[3]);
    dst[8 + 2 * u + 1] = pack_low_bytes(b1[4], b1[5], b1[6], b1[7]);
    if (u == 0) dst[16] = __float_as_uint(amax > 0.0f ? ldexpf(1.0f, e) * (1.0f / 254.0f) : 0.0f);
    if (SUM && u == 0) dst[17] = __float_as_uint(xsum);
}

// The x elements a prep thread handles (q = 4 * block + quarter), as two float4 offsets.
// Byte codes (Q8_0, and Q5_K / Q6_K repacked to int8) or nibbles (Q4_0, Q4_K).
template <int QT>
constexpr bool kByteCodes =
    QT == UNILLM_QTYPE_Q8_0 || QT == UNILLM_QTYPE_Q5_K || QT == UNILLM_QTYPE_Q6_K;
// K-quants with a per-block minimum (a sum-of-x term): Q4_K, Q5_K
template <int QT>
constexpr bool kHasMin = QT == UNILLM_QTYPE_Q4_K || QT == UNILLM_QTYPE_Q5_K;

template <int QT>
__device__ __forceinline__ void quarter_offsets(int quarter, int& o0, int& o1) {
    if constexpr (!kByteCodes<QT>) {
        o0 = 4 * quarter;       // x[4t .. 4t+3]
        o1 = 16 + 4 * quarter;  // x[16+4t .. 16+4t+3]
    } else {
        o0 = 8 * quarter;       // x[8u .. 8u+7]
        o1 = 8 * quarter + 4;
    }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct XBlock {
    u32x4 dg[4];  // 16 digit dwords, in record order
    float sx;     // 0 for a lane's clamped (duplicate) block
    float xsum;   // Q4_K, Q5_K: sum of the block's x (0 for a clamped block)
};

template <int QT>
__device__ __forceinline__ void load_xblock(const uint32_t* __restrict__ src, bool valid,
                                            XBlock& o) {
    const u32x4* p = reinterpret_cast<const u32x4*>(src);
#pragma unroll
    for (int i = 0; i < 4; ++i) o.dg[i] = p[i];
    o.sx = valid ? __uint_as_float(src[16]) : 0.0f;
    o.xsum = kHasMin<QT> && valid ? __uint_as_float(src[17]) : 0.0f;
}

// A wave's x records: read once from LDS into registers (M * NB records,
// 17 VGPRs each) and reused for every row of the wave.
template <int QT, int M, int NB>
struct XRegs {
    XBlock xb[M][NB];
    __device__ __forceinline__ XRegs(const uint32_t* xlds, int KB, const int (&bidx)[NB],
                                     const bool (&bval)[NB]) {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int i = 0; i < NB; ++i)
                load_xblock<QT>(xlds + ((size_t)m * KB + bidx[i]) * kXWords, bval[i], xb[m][i]);
    }
};

// ---- weights --------------------------------------------------------------------------------
template <int QT>
struct Payload {
    static constexpr int V = kByteCodes<QT> ? 2 : 1;  // 128-bit loads per block
};

template <int QT, int NB, int R>
struct Chunk {
    u32x4 q[R][NB][Payload<QT>::V];
    uint16_t d[R][NB];  // f16 d; Q4_K, Q5_K: sc | m << 8; Q6_K: int8 scales of the two halves
    uint32_t h[R][NB];  // Q4_K, Q5_K: d | dmin << 16 of the block's 256-weight group; Q6_K: d
};

// Weight addresses: base + row * rb + a lane offset, with the row offset
// row * rb (wave-uniform, 32-bit: weights under 4 GiB) and each lane's byte
// offsets inside a row (its payloads at 16 * V * b, its scales after the
// row's payloads) fixed for the whole kernel.  Payload loads are
// non-temporal: the weights are streamed once and should not evict x from
// the caches.  (Measured against raw buffer loads with the same offsets:
// these are 1-4 % faster here.)
// Branch-free: indices are clamped into the matrix and validity is applied
// later through the x scale (sx = 0), so no divergent branch sits around a
// load.  (A load under a divergent branch whose other side writes the same
// register makes the compiler wait for the load at the join, serialising
// the loads.)  Rows of a wave: w, w + W, w + 2W, ... (W = waves), so the rows
// the whole grid requests at one moment form one contiguous stretch of the
// matrix.  Chunk j0 holds the wave's rows j0 .. j0 + R - 1; rows past the
// wave's last are clamped to that last row (an address the wave reads anyway).
// PAIR (the SwiGLU epilogue, R = 2): chunk j0 is the wave's logical row
// L = w + j0 W of a [gate; up] weight with I rows each: physical rows L and I + L.
template <int QT, int NB, int R, bool PAIR = false>
__device__ __forceinline__ void load_chunk(Chunk<QT, NB, R>& c, const uint8_t* __restrict__ base,
                                           uint32_t rb, int w, int W, int j0, int jlast,
                                           const uint32_t (&poff)[NB], const uint32_t (&soff)[NB],
                                           const uint32_t (&hoff)[NB], int I = 0) {
    constexpr int V = Payload<QT>::V;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = PAIR ? w + min(j0, jlast) * W + r * I : w + min(j0 + r, jlast) * W;
        const uint32_t ro = __builtin_amdgcn_readfirstlane((uint32_t)row * rb);
#pragma unroll
        for (int i = 0; i < NB; ++i) {
#pragma unroll
            for (int v = 0; v < V; ++v)
                c.q[r][i][v] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4*>(base + ro + poff[i]) + v);
            c.d[r][i] = *reinterpret_cast<const uint16_t*>(base + ro + soff[i]);
            if constexpr (kHasMin<QT> || QT == UNILLM_QTYPE_Q6_K)
                c.h[r][i] = *reinterpret_cast<const uint32_t*>(base + ro + hoff[i]);
        }
    }
}

// Epilogue: y = sum (store), y += sum (the residual add, `add`), or with PAIR
// y[m, L] = silu(gate) * up over the I logical rows (candle silu: v / (1 + e^-v)).
// KS (k split over a wave pair): the wave's half of each sum is added into the pair's
// LDS slots ksum[j][m] instead, and the workgroup stores them after its last chunk.
template <int QT, int M, int NB, int R, bool PAIR = false, bool KS = false>
__device__ __forceinline__ void compute_chunk(const Chunk<QT, NB, R>& c, const XRegs<QT, M, NB>& xs,
                                              float* __restrict__ y, int w, int W, int j0,
                                              int jcount, int N, int lane, int m_real, int add,
                                              float* ksum = nullptr) {
    float part[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) part[m][r] = 0.0f;
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const XBlock& xb = xs.xb[m][i];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                int acc;
                if constexpr (QT == UNILLM_QTYPE_Q6_K) {
                    // per 16-weight half v: A_v = 254 sum q d0 + sum q d1, scaled by d sc_v
                    int ah[2];
#pragma unroll
                    for (int v = 0; v < 2; ++v) {
                        const u32x4 w4 = c.q[r][i][v];
                        int a0 = 0, a1 = 0;
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            a0 = sdot4((int)w4[t], (int)xb.dg[v][t], a0);
                            a1 = sdot4((int)w4[t], (int)xb.dg[2 + v][t], a1);
                        }
                        ah[v] = a0 * 254 + a1;
                    }
                    const uint32_t sm = c.d[r][i];
                    const float dd = __half2float(__ushort_as_half((uint16_t)c.h[r][i]));
                    const float sv = fmaf((float)(int8_t)(sm & 0xFFu), (float)ah[0],
                                          (float)(int8_t)(sm >> 8) * (float)ah[1]);
                    part[m][r] = fmaf(dd, sv * xb.sx, part[m][r]);
                    continue;
                } else if constexpr (!kByteCodes<QT>) {
                    // digit levels 3..0: A = ((a3 * 16 + a2) * 16 + a1) * 16 + a0
                    const u32x4 w4 = c.q[r][i][0];
                    int lv[4] = {0, 0, 0, 0};
#pragma unroll
                    for (int t = 0; t < 4; ++t)
#pragma unroll
                        for (int L = 0; L < 4; ++L) lv[L] = sdot8((int)w4[t], (int)xb.dg[L][t], lv[L]);
                    acc = ((lv[0] * 16 + lv[1]) * 16 + lv[2]) * 16 + lv[3];
                } else {
                    int a0 = 0, a1 = 0;
#pragma unroll
                    for (int v = 0; v < 2; ++v) {
                        const u32x4 w4 = c.q[r][i][v];
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            a0 = sdot4((int)w4[t], (int)xb.dg[v][t], a0);
                            a1 = sdot4((int)w4[t], (int)xb.dg[2 + v][t], a1);
                        }
                    }
                    acc = a0 * 254 + a1;
                }
                if constexpr (kHasMin<QT>) {
                    // (d sc) (acc sx + c0 sum x) - (dmin m) sum x: acc is sum (q - c0) x,
                    // c0 = 8 (Q4_K nibbles) or 16 (Q5_K bytes)
                    constexpr float c0 = QT == UNILLM_QTYPE_Q5_K ? 16.0f : 8.0f;
                    const uint32_t h = c.h[r][i], sm = c.d[r][i];
                    const float s = __half2float(__ushort_as_half((uint16_t)h)) * (float)(sm & 0xFFu);
                    const float o = __half2float(__ushort_as_half((uint16_t)(h >> 16))) * (float)(sm >> 8);
                    const float t = fmaf((float)acc, xb.sx, c0 * xb.xsum);
                    part[m][r] = fmaf(-o, xb.xsum, fmaf(s, t, part[m][r]));
                } else {
                    const float dw = __half2float(__ushort_as_half(c.d[r][i]));
                    part[m][r] = fmaf(dw, (float)acc * xb.sx, part[m][r]);
                }
            }
        }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) part[m][r] = wave_sum(part[m][r]);
    if (lane == 0) {
        if constexpr (KS) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (j0 + r < jcount)
#pragma unroll
                    for (int m = 0; m < M; ++m) atomicAdd(ksum + (j0 + r) * M + m, part[m][r]);
        } else if constexpr (PAIR) {
            if (j0 < jcount)
#pragma unroll
                for (int m = 0; m < M; ++m)
                    if (m < m_real) {
                        const float g = part[m][0], u = part[m][1];
                        y[(int64_t)m * N + w + j0 * W] = g / (1.0f + expf(-g)) * u;
                    }
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (j0 + r < jcount)
#pragma unroll
                    for (int m = 0; m < M; ++m)
                        if (m < m_real) {
                            float* dst = y + (int64_t)m * N + w + (j0 + r) * W;
                            *dst = add ? *dst + part[m][r] : part[m][r];
                        }
        }
    }
}

// Workgroup size: 1024 threads (128 VGPRs per lane) when the records and a
// chunk fit that budget, else 512 (256 VGPRs).  Either way the launch puts
// one workgroup on each CU, so the x digits are built once per CU.  One block a
// lane (k <= 2048) fits the budget up to four 128-bit records (M V <= 4): the
// doubled waves hide more latency (Q4_0 m = 3, 4 at k2048 n14336: 9.26 -> 8.49 us a
// call; Q8_0 m = 2 at k2048 n5632: 5.52 -> 5.38).  Two blocks at m = 2 (k4096)
// measured mixed (n14336 -3 %, n4096 +3 %) and keep 512.
template <int QT, int M, int NB>
constexpr int gemv_threads() {
    return M * NB * Payload<QT>::V <= 2 || (NB == 1 && M * Payload<QT>::V <= 4) ? 1024 : 512;
}

// m_real <= M rows of x are used; rows m >= m_real repeat row m_real - 1 and
// are not written.  Dynamic LDS: M * KB * kXWords dwords of x digits.
// KB <= NB * 64, so a thread builds at most PASSES = ceil(M * NB * 256 / THREADS) quarter-blocks.
// PAIR: the weight is [gate; up] (2 I rows); the waves cover the I logical rows
// and y is [m, I] = silu(gate) * up.  Otherwise `add` selects y += x W^T.
//
// norm.gamma != nullptr: x is first replaced by its layer norm along k,
// (x - mean) / sqrt(var + eps) * gamma (+ beta), var the mean of the squared
// deviations (the reference's ops_fn::layer_norm before the projections,
// tensor_core.rs:973-1008).  Every workgroup reads all of x anyway, so each
// computes the row statistics itself (one barrier, gamma and beta requested with x),
// no extra launch.
// XW: waves numbered across the workgroups (wave w of workgroup b is b + w grid), so
// that the waves holding one row more than the others (a partial last round) spread
// over every CU instead of filling the first CUs.
// KS: the k range split over the two waves of a pair (waves 2 p and 2 p + 1 of a
// workgroup): each takes NB blocks a lane of its half and the rows of "wave" p, so a
// lane holds half the records and twice the waves fit a CU; the halves' sums meet in
// LDS (after the x records: the workgroup's pairs x jmax rows x M floats) and are
// stored after a workgroup barrier that follows every wave's last chunk.
template <int QT, int M, int NB, int R, int THREADS, bool PAIR = false, bool NORM = false,
          bool XW = false, bool KS = false>
__global__ __launch_bounds__(THREADS) void gemv_kernel(const uint8_t* __restrict__ base,
                                                       int64_t rb,
                                                       const float* __restrict__ x,
                                                       float* __restrict__ y, int N_rows, int KB,
                                                       int m_real, int add, NormArgs norm) {
    static_assert(!PAIR || R == 2, "the SwiGLU pair is one gate and one up row per chunk");
    static_assert(!KS || (!PAIR && !NORM && !XW), "the k split takes the plain and add epilogues");
    constexpr int LR = PAIR ? 1 : R;  // logical rows per chunk
    constexpr int KSF = KS ? 2 : 1;   // waves a row's k range is split over
    const int I = PAIR ? N_rows / 2 : 0;
    const int N = PAIR ? I : N_rows;  // logical rows (output columns)
    constexpr int WAVES = THREADS / 64;
    constexpr int RW = WAVES / KSF;  // row-owning waves (pairs with KS) per workgroup
    constexpr int PASSES = (M * KSF * NB * 256 + THREADS - 1) / THREADS;  // quarter-blocks a thread
    extern __shared__ uint32_t xlds[];
    const int lane = threadIdx.x & 63;
    const int half = KS ? (int)((threadIdx.x >> 6) & 1) : 0;  // KS: which half of k
    const int wave = __builtin_amdgcn_readfirstlane(
        XW   ? (int)(threadIdx.x >> 6) * (int)gridDim.x + (int)blockIdx.x
        : KS ? (int)blockIdx.x * RW + (int)(threadIdx.x >> 7)
             : (int)(blockIdx.x * WAVES + (threadIdx.x >> 6)));
    const int waves = gridDim.x * RW;
    const int64_t K = (int64_t)KB * QK;
    // this wave's rows: wave, wave + waves, ... (counts differ by at most one);
    // wave-uniform, so every branch on them is a scalar branch
    const int jcount = wave < N ? (N - 1 - wave) / waves + 1 : 0;
    const int jlast = max(jcount - 1, 0);
    const int wrow = min(wave, N - 1);  // a wave without rows reads row N - 1

    int bidx[NB];
    bool bval[NB];
    uint32_t poff[NB], soff[NB], hoff[NB];  // this lane's byte offsets inside a row
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int b = half * NB * 64 + i * 64 + lane;
        bval[i] = b < KB;
        bidx[i] = min(b, KB - 1);
        poff[i] = (uint32_t)bidx[i] * (16 * Payload<QT>::V);
        soff[i] = (uint32_t)KB * (16 * Payload<QT>::V) + 2u * (uint32_t)bidx[i];
        // K-quant group header, after the payload and scale planes
        hoff[i] = (uint32_t)KB * (16u * Payload<QT>::V + 2u) + 4u * (uint32_t)(bidx[i] >> 3);
    }

    // 1. x for the digits.  A wave whose quarters of a pass all lie past nq
    //    neither loads nor builds anything in that pass (a wave-uniform, scalar
    //    branch); inside a wave, indices are clamped into x.
    const int nq = M * KB * 4;
    const int wave0 = __builtin_amdgcn_readfirstlane((int)threadIdx.x & ~63);
    float v[PASSES][8];
    auto order = [](float (&d)[8], float4 f0, float4 f1) {
        if constexpr (!kByteCodes<QT>) {  // payload nibble order
            d[0] = f0.x; d[1] = f1.x; d[2] = f0.y; d[3] = f1.y;
            d[4] = f0.z; d[5] = f1.z; d[6] = f0.w; d[7] = f1.w;
        } else {
            d[0] = f0.x; d[1] = f0.y; d[2] = f0.z; d[3] = f0.w;
            d[4] = f1.x; d[5] = f1.y; d[6] = f1.z; d[7] = f1.w;
        }
    };
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        if (wave0 + p * THREADS >= nq) continue;
        const int q = min((int)threadIdx.x + p * THREADS, nq - 1);
        const int blk = q >> 2;
        const int m = blk / KB;
        const int64_t e = (int64_t)(blk - m * KB) * QK;
        const float* xb = x + (int64_t)min(m, m_real - 1) * K + e;
        int o0, o1;
        quarter_offsets<QT>(q & 3, o0, o1);
        order(v[p], *reinterpret_cast<const float4*>(xb + o0),
              *reinterpret_cast<const float4*>(xb + o1));
    }

    // KS: the pairs' sum slots, zeroed before the records' barrier
    const int jmax = (N + waves - 1) / waves;
    float* const ksum_wg = reinterpret_cast<float*>(xlds + (size_t)M * KB * kXWords);
    if constexpr (KS)
        for (int i = threadIdx.x; i < RW * jmax * M; i += THREADS) ksum_wg[i] = 0.0f;
    float* const ksum = ksum_wg + (KS ? (int)(threadIdx.x >> 7) : 0) * jmax * M;

    // gamma and beta of this thread's quarters (the norm), requested with x
    float gmv[NORM ? PASSES : 1][8], btv[NORM ? PASSES : 1][8];
    if constexpr (NORM) {
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            if (wave0 + p * THREADS >= nq) continue;
            const int q = min((int)threadIdx.x + p * THREADS, nq - 1);
            const int blk = q >> 2;
            const int m = blk / KB;
            const int64_t e = (int64_t)(blk - m * KB) * QK;
            int o0, o1;
            quarter_offsets<QT>(q & 3, o0, o1);
            const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
            order(gmv[p], *reinterpret_cast<const float4*>(norm.gamma + e + o0),
                  *reinterpret_cast<const float4*>(norm.gamma + e + o1));
            order(btv[p], norm.beta ? *reinterpret_cast<const float4*>(norm.beta + e + o0) : z,
                  norm.beta ? *reinterpret_cast<const float4*>(norm.beta + e + o1) : z);
        }
    }

    // 2. the first chunk of weights: one chunk per wave keeps the memory
    //    pipeline busy while x arrives and is turned into digits, without
    //    filling it -- instructions issue in order, and once weight loads back
    //    up, everything behind them (here: the digit work every row needs)
    //    waits until they are accepted.
    Chunk<QT, NB, R> a, b;
    load_chunk<QT, NB, R, PAIR>(a, base, (uint32_t)rb, wrow, waves, 0, jlast, poff, soff, hoff, I);

    // 2b. the layer norm of x.  Each wave takes its elements' count, mean and sum
    //     of squared deviations from that mean (two DPP sums, no barrier); the
    //     waves' triples meet in LDS behind one barrier and combine exactly
    //     (Chan et al.: M2 = sum M2_w + sum n_w (mean_w - mean)^2).  Two passes
    //     over the data within a wave, as the reference's two passes.
    if constexpr (NORM) {
        __shared__ float red[3][M * WAVES];
        const int wv = threadIdx.x >> 6;
        float s[M], c[M];
#pragma unroll
        for (int mm = 0; mm < M; ++mm) s[mm] = c[mm] = 0.0f;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            if (wave0 + p * THREADS >= nq) continue;
            const int q = (int)threadIdx.x + p * THREADS;
            const int m = min(q, nq - 1) / (4 * KB);
            float t = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) t += v[p][j];
#pragma unroll
            for (int mm = 0; mm < M; ++mm) {
                s[mm] += q < nq && m == mm ? t : 0.0f;
                c[mm] += q < nq && m == mm ? 8.0f : 0.0f;
            }
        }
        float mw[M], nw[M];
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
            nw[mm] = wave_sum(c[mm]);
            const float sw = wave_sum(s[mm]);
            mw[mm] = nw[mm] > 0.0f ? sw / nw[mm] : 0.0f;
            s[mm] = 0.0f;
        }
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            if (wave0 + p * THREADS >= nq) continue;
            const int q = (int)threadIdx.x + p * THREADS;
            const int m = min(q, nq - 1) / (4 * KB);
            float mu = mw[0];
#pragma unroll
            for (int mm = 1; mm < M; ++mm) mu = m == mm ? mw[mm] : mu;
            float t = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) t += (v[p][j] - mu) * (v[p][j] - mu);
#pragma unroll
            for (int mm = 0; mm < M; ++mm) s[mm] += q < nq && m == mm ? t : 0.0f;
        }
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
            const float m2 = wave_sum(s[mm]);
            if (lane == 0) {
                red[0][mm * WAVES + wv] = nw[mm];
                red[1][mm * WAVES + wv] = mw[mm];
                red[2][mm * WAVES + wv] = m2;
            }
        }
        __syncthreads();
        // lane w2 < WAVES takes wave w2's triple; a wave sum combines them
        float mean[M], rsd[M];
#pragma unroll
        for (int mm = 0; mm < M; ++mm) {
            const bool mine = lane < WAVES;
            const int li = mm * WAVES + (mine ? lane : 0);
            const float n_l = mine ? red[0][li] : 0.0f, mu_l = mine ? red[1][li] : 0.0f,
                        q_l = mine ? red[2][li] : 0.0f;
            mean[mm] = wave_sum(n_l * mu_l) / (float)K;
            const float d = mu_l - mean[mm];
            // one reciprocal a row, a product an element (within an f32 rounding of
            // the quotient, far below what the x digits keep)
            rsd[mm] = 1.0f / sqrtf(wave_sum(q_l + n_l * d * d) / (float)K + norm.eps);
        }
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            if (wave0 + p * THREADS >= nq) continue;
            const int q = min((int)threadIdx.x + p * THREADS, nq - 1);
            const int m = (q >> 2) / KB;
            float mu = mean[0], rs = rsd[0];
#pragma unroll
            for (int mm = 1; mm < M; ++mm) {
                mu = m == mm ? mean[mm] : mu;
                rs = m == mm ? rsd[mm] : rs;
            }
            const float (&g)[8] = gmv[p];
            const float (&bb)[8] = btv[p];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[p][j] = (v[p][j] - mu) * rs * g[j] + bb[j];
        }
    }

    // 3. x digit records for all M * KB blocks, four threads per block (threads
    //    past nq compute on a clamped copy and store nothing; nq is a multiple
    //    of 4, so a DPP quad is either all real or all clamped).
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        if (wave0 + p * THREADS >= nq) continue;
        const int q = threadIdx.x + p * THREADS;
        uint32_t* dst = xlds + (size_t)(min(q, nq - 1) >> 2) * kXWords;
        if constexpr (kByteCodes<QT>) prep_q8<QT == UNILLM_QTYPE_Q5_K>(v[p], q & 3, q < nq, dst);
        else prep_q4<QT == UNILLM_QTYPE_Q4_K>(v[p], q & 3, q < nq, dst);
        __builtin_amdgcn_sched_barrier(0);  // one pass's temporaries live at a time
    }
    __syncthreads();


    // 4. this lane's records, read once from LDS into registers for all rows
    const XRegs<QT, M, NB> xs(xlds, KB, bidx, bval);
    __builtin_amdgcn_sched_barrier(0);

    // 5. with more rows than one chunk: request the second chunk, then compute
    //    both, then two chunks per step; with one chunk, just compute it.  The
    //    branch is wave-uniform and each side has its own memory waits (a
    //    shared join would make the wait for chunk a cover chunk b as well).
    if (jcount > LR) {
        load_chunk<QT, NB, R, PAIR>(b, base, (uint32_t)rb, wrow, waves, LR, jlast, poff, soff, hoff, I);
        compute_chunk<QT, M, NB, R, PAIR, KS>(a, xs, y, wrow, waves, 0, jcount, N, lane, m_real,
                                              add, ksum);
        compute_chunk<QT, M, NB, R, PAIR, KS>(b, xs, y, wrow, waves, LR, jcount, N, lane, m_real,
                                              add, ksum);
        for (int j = 2 * LR; j < jcount; j += 2 * LR) {
            load_chunk<QT, NB, R, PAIR>(a, base, (uint32_t)rb, wrow, waves, j, jlast, poff, soff,
                                        hoff, I);
            load_chunk<QT, NB, R, PAIR>(b, base, (uint32_t)rb, wrow, waves, j + LR, jlast, poff,
                                        soff, hoff, I);
            compute_chunk<QT, M, NB, R, PAIR, KS>(a, xs, y, wrow, waves, j, jcount, N, lane,
                                                  m_real, add, ksum);
            compute_chunk<QT, M, NB, R, PAIR, KS>(b, xs, y, wrow, waves, j + LR, jcount, N, lane,
                                                  m_real, add, ksum);
        }
    } else {
        compute_chunk<QT, M, NB, R, PAIR, KS>(a, xs, y, wrow, waves, 0, jcount, N, lane, m_real,
                                              add, ksum);
    }
    if constexpr (KS) {
        // both halves of every pair are done: slot (pair p, row j, token m) -> y
        __syncthreads();
        for (int i = threadIdx.x; i < RW * jmax * M; i += THREADS) {
            const int pl = i / (jmax * M), j = i / M % jmax, m = i % M;
            const int pw = (int)blockIdx.x * RW + pl;
            const int jc = pw < N ? (N - 1 - pw) / waves + 1 : 0;
            if (j < jc && m < m_real) {
                float* dst = y + (int64_t)m * N + pw + j * waves;
                *dst = add ? *dst + ksum_wg[i] : ksum_wg[i];
            }
        }
    }
}

// The norm variants exist for k <= 8192 (NB <= 4): the layer-normed inputs
// feed QKV and gate/up, whose k is the hidden size; larger k with a norm runs
// on the batched-decode path (gemv_supports_norm).
template <int QT, int M, int NB, int R, bool PAIR = false, bool XW = false>
hipError_t launch_r(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t st,
                    int waves, int add, const NormArgs& norm) {
    constexpr int THREADS = gemv_threads<QT, M, NB>();
    constexpr int WAVES = THREADS / 64;
    const size_t lds = (size_t)M * w.kb * kXWords * sizeof(uint32_t);
    const int grid = (waves + WAVES - 1) / WAVES;
    if (norm.gamma) {
        if constexpr (NB <= 4)
            gemv_kernel<QT, M, NB, R, THREADS, PAIR, true><<<grid, THREADS, lds, st>>>(
                w.base, w.row_bytes, x, y, (int)w.n, (int)w.kb, (int)m, add, norm);
        else
            return hipErrorInvalidValue;
    } else {
        gemv_kernel<QT, M, NB, R, THREADS, PAIR, false, XW><<<grid, THREADS, lds, st>>>(
            w.base, w.row_bytes, x, y, (int)w.n, (int)w.kb, (int)m, add, norm);
    }
    return hipGetLastError();
}

// Launch shape.  Every workgroup is resident at once; there is a workgroup
// for every CU, and each wave gets at least two rows where the matrix has
// enough (a second row keeps a wave's loads in flight while its x digits are
// built).  The chunk size R (rows per request) is capped by the registers a
// chunk may take (at most 4 payload loads per lane).
template <int QT, int M, int NB>
hipError_t launch_nb(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t st,
                     int epi, const NormArgs& norm) {
    constexpr int V = Payload<QT>::V;
    constexpr int THREADS = gemv_threads<QT, M, NB>();
    // four rows a chunk at four tokens would spill in the 1024-thread budget
    constexpr int RMAX = NB * V >= 4 ? 1 : M >= 4 && THREADS == 1024 ? 2 : 4 / (NB * V);
    constexpr int WAVES = THREADS / 64;
    int per_cu = 0;
    const size_t lds = (size_t)M * w.kb * kXWords * sizeof(uint32_t);
    const int64_t cus = device_info().cu_count;
    if (epi == kEpiSwiglu) {  // one gate and one up row per chunk, over the I = n / 2 outputs
        if constexpr (M * NB * V <= 4) {
            hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_cu, gemv_kernel<QT, M, NB, 2, THREADS, true>, THREADS, lds);
            if (e != hipSuccess) return e;
            const int64_t I = w.n / 2;
            const int64_t resident = cus * std::max(per_cu, 1) * WAVES;
            const int64_t waves = std::max<int64_t>(
                1, std::min({resident, std::max<int64_t>(I / 2, cus * WAVES), I}));
            return launch_r<QT, M, NB, 2, true>(w, x, m, y, st, (int)waves, 0, norm);
        }
        return hipErrorInvalidValue;
    }
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &per_cu, gemv_kernel<QT, M, NB, RMAX, THREADS>, THREADS, lds);
    if (e != hipSuccess) return e;
    const int64_t resident = cus * std::max(per_cu, 1) * WAVES;
    const int64_t want = std::max<int64_t>(w.n / 2, cus * WAVES);
    const int64_t waves = std::max<int64_t>(1, std::min({resident, want, w.n}));
    const int64_t rows = (w.n + waves - 1) / waves;  // per wave, at most
    if (debug_launch())
        fprintf(stderr, "unillm gemv: n=%lld kb=%lld m=%lld threads=%d waves=%lld rows=%lld\n",
                (long long)w.n, (long long)w.kb, (long long)m, THREADS, (long long)waves,
                (long long)rows);
    const int add = epi == kEpiAdd;
    if (RMAX >= 4 && rows > 4)
        return launch_r<QT, M, NB, RMAX>(w, x, m, y, st, (int)waves, add, norm);
    if (RMAX >= 2 && rows > 2)
        return launch_r<QT, M, NB, (RMAX >= 2 ? 2 : 1)>(w, x, m, y, st, (int)waves, add, norm);
    if constexpr (M == 1) {
        // at most two rows a wave with a partial second round (the Q8_0 k 2048 n 5632
        // GEMV: 1536 of 4096 waves hold two rows): the two-row waves across all CUs
        const int64_t all = (waves + WAVES - 1) / WAVES * WAVES;
        if (!norm.gamma && rows == 2 && w.n % all != 0)
            return launch_r<QT, M, NB, 1, false, true>(w, x, m, y, st, (int)waves, add, norm);
    }
    return launch_r<QT, M, NB, 1>(w, x, m, y, st, (int)waves, add, norm);
}

// Four tokens at two blocks a lane (k 2049 .. 4096): the k range split over wave pairs
// (KS), so each lane holds one block's records and a workgroup of 1024 threads fits a
// CU, as at k <= 2048 (Q6_K's header words would spill there: it keeps launch_nb).
// One workgroup a CU, pairs as launch_nb sizes waves.
template <int QT, int M, int NBH = 1, int THREADS = 1024>
hipError_t launch_ks(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t st,
                     int epi, const NormArgs& norm) {
    const int add = epi == kEpiAdd;
    constexpr int RW = THREADS / 128;  // row-owning pairs a workgroup
    constexpr int V = Payload<QT>::V;
    constexpr int RMAX = NBH * V >= 4 ? 1 : M >= 4 ? 2 : 4 / (NBH * V);
    const int64_t cus = device_info().cu_count;
    const int64_t want = std::max<int64_t>(w.n / 2, cus * RW);
    const int64_t pairs = std::max<int64_t>(1, std::min<int64_t>({cus * RW, want, w.n}));
    // the x records and the pairs' sum slots stay within the 64 KiB a launch takes
    // without a raised dynamic-LDS limit: past jcap rows a pair (393216 rows at four
    // tokens and k 4096), more workgroups than CUs
    const size_t xbytes = (size_t)M * w.kb * kXWords * sizeof(uint32_t);
    if (xbytes + (size_t)RW * M * sizeof(float) > 65536) return hipErrorInvalidValue;
    const int64_t jcap = (int64_t)((65536 - xbytes) / ((size_t)RW * M * sizeof(float)));
    const int64_t grid64 = std::max((pairs + RW - 1) / RW, (w.n + RW * jcap - 1) / (RW * jcap));
    if (grid64 > INT32_MAX) return hipErrorInvalidValue;
    const int grid = (int)grid64;
    const int64_t jmax = (w.n + (int64_t)grid * RW - 1) / ((int64_t)grid * RW);
    const size_t lds = xbytes + (size_t)RW * jmax * M * sizeof(float);
    if (debug_launch())
        fprintf(stderr, "unillm gemv (k split): n=%lld kb=%lld m=%lld pairs=%lld rows=%lld\n",
                (long long)w.n, (long long)w.kb, (long long)m, (long long)grid * RW,
                (long long)jmax);
    const NormArgs none{nullptr, nullptr, 0.f};
    if (RMAX >= 4 && jmax > 4)
        gemv_kernel<QT, M, NBH, RMAX, THREADS, false, false, false, true>
            <<<grid, THREADS, lds, st>>>(w.base, w.row_bytes, x, y, (int)w.n, (int)w.kb, (int)m,
                                         add, none);
    else if (RMAX >= 2 && jmax > 2)
        gemv_kernel<QT, M, NBH, (RMAX >= 2 ? 2 : 1), THREADS, false, false, false, true>
            <<<grid, THREADS, lds, st>>>(w.base, w.row_bytes, x, y, (int)w.n, (int)w.kb, (int)m,
                                         add, none);
    else
        gemv_kernel<QT, M, NBH, 1, THREADS, false, false, false, true>
            <<<grid, THREADS, lds, st>>>(w.base, w.row_bytes, x, y, (int)w.n, (int)w.kb, (int)m,
                                         add, none);
    return hipGetLastError();
}

template <int QT, int M>
hipError_t launch_m(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t st,
                    int epi, const NormArgs& norm) {
    switch ((int)((w.kb + 63) / 64)) {
        case 1: return launch_nb<QT, M, 1>(w, x, m, y, st, epi, norm);
        case 2:
            if constexpr (M == 4 && QT != UNILLM_QTYPE_Q6_K)
                if (epi != kEpiSwiglu && !norm.gamma)
                    return launch_ks<QT, M>(w, x, m, y, st, epi, norm);
            return launch_nb<QT, M, 2>(w, x, m, y, st, epi, norm);
        case 3: if constexpr (M <= 2) return launch_nb<QT, M, 3>(w, x, m, y, st, epi, norm); break;
        case 4: if constexpr (M <= 2) return launch_nb<QT, M, 4>(w, x, m, y, st, epi, norm); break;
        // k 8193 .. 12288 at one token for the byte codes (1024 threads for Q8_0's frame,
        // Q8_0 and Q5_0; 512 for Q5_K and Q6_K, whose header words would spill at 1024)
        // and at two tokens for every type (512 threads): the k split over wave pairs,
        // three blocks a lane a half
        case 5:
            if constexpr (M == 1 && !kByteCodes<QT>) return launch_nb<QT, M, 5>(w, x, m, y, st, epi, norm);
            if constexpr (M == 1 && QT == UNILLM_QTYPE_Q8_0)
                if (epi != kEpiSwiglu && !norm.gamma) return launch_ks<QT, M, 3>(w, x, m, y, st, epi, norm);
            if constexpr (M == 1 && kByteCodes<QT> && QT != UNILLM_QTYPE_Q8_0)
                if (epi != kEpiSwiglu && !norm.gamma) return launch_ks<QT, M, 3, 512>(w, x, m, y, st, epi, norm);
            if constexpr (M == 2)
                if (epi != kEpiSwiglu && !norm.gamma) return launch_ks<QT, M, 3, 512>(w, x, m, y, st, epi, norm);
            break;
        case 6:
            if constexpr (M == 1 && !kByteCodes<QT>) return launch_nb<QT, M, 6>(w, x, m, y, st, epi, norm);
            if constexpr (M == 1 && QT == UNILLM_QTYPE_Q8_0)
                if (epi != kEpiSwiglu && !norm.gamma) return launch_ks<QT, M, 3>(w, x, m, y, st, epi, norm);
            if constexpr (M == 1 && kByteCodes<QT> && QT != UNILLM_QTYPE_Q8_0)
                if (epi != kEpiSwiglu && !norm.gamma) return launch_ks<QT, M, 3, 512>(w, x, m, y, st, epi, norm);
            if constexpr (M == 2)
                if (epi != kEpiSwiglu && !norm.gamma) return launch_ks<QT, M, 3, 512>(w, x, m, y, st, epi, norm);
            break;
        case 7:
            if constexpr (M == 1 && !kByteCodes<QT>) return launch_nb<QT, M, 7>(w, x, m, y, st, epi, norm);
            [[fallthrough]];
        case 8:
            // the byte codes at one token, k 12289 .. 16384: four blocks a lane a half
            if constexpr (M == 1 && kByteCodes<QT>)
                if (epi != kEpiSwiglu && !norm.gamma) return launch_ks<QT, M, 4, 512>(w, x, m, y, st, epi, norm);
            break;
        default: break;
    }
    return hipErrorInvalidValue;
}

}  // namespace

// Largest K (in blocks) the GEMV path takes at m rows, set by the registers
// two chunks of NB blocks per lane need (NB = ceil(KB / 64)): Q4_0 up to
// NB = 7 at one row (K = 14336), 4 at two, 2 at four; byte-code payloads are twice
// as wide, so one wave a row stops at NB = 4 at one row.  The k split over wave
// pairs takes the byte codes at one row up to NB = 8 (K = 16384; three or four
// blocks a lane a half) and every type at two rows up to NB = 6 (K = 12288).  M * KB <= 768 also bounds the x records in LDS
// (60 KiB).
int64_t gemv_max_kb(int64_t m, int qtype) {
    if (m <= 1) return byte_codes(qtype) ? 512 : 448;
    if (m <= 2) return 384;
    return 128;
}

// The SwiGLU pair epilogue holds two chunks of one gate and one up row: the
// tokens times the 128-bit payload loads of a row at most 4, past which it spills
// (m = 1: Q4_0 / Q4_K k <= 8192, Q8_0 / Q5_K / Q6_K k <= 4096; halved per doubling of m).
bool gemv_supports_swiglu(const QWeight& w, int64_t m) {
    const int64_t nbv = (w.kb + 63) / 64 * (qbytes(w.qtype) / 16);
    const int64_t mb = m <= 1 ? 1 : m <= 2 ? 2 : 4;  // the kernel's token count M
    return gemv_supports(w, m) && w.n % 2 == 0 && mb * nbv <= 4;
}

bool gemv_supports_norm(const QWeight& w, int64_t m) {
    return gemv_supports(w, m) && (w.kb + 63) / 64 <= 4;
}

// The GEMV addresses a weight with 32-bit row offsets.
bool gemv_supports(const QWeight& w, int64_t m) {
    return m >= 1 && m <= kGemvMaxM && w.kb <= gemv_max_kb(m, w.qtype) &&
           (uint64_t)w.n * (uint64_t)w.row_bytes <= 0xFFFFFFFFull;
}

hipError_t launch_gemv(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t s,
                       int epi, const NormArgs& norm) {
    if (w.qtype == UNILLM_QTYPE_Q4_K) {
        if (m == 1) return launch_m<UNILLM_QTYPE_Q4_K, 1>(w, x, m, y, s, epi, norm);
        if (m == 2) return launch_m<UNILLM_QTYPE_Q4_K, 2>(w, x, m, y, s, epi, norm);
        return launch_m<UNILLM_QTYPE_Q4_K, 4>(w, x, m, y, s, epi, norm);
    }
    if (w.qtype == UNILLM_QTYPE_Q5_K) {
        if (m == 1) return launch_m<UNILLM_QTYPE_Q5_K, 1>(w, x, m, y, s, epi, norm);
        if (m == 2) return launch_m<UNILLM_QTYPE_Q5_K, 2>(w, x, m, y, s, epi, norm);
        return launch_m<UNILLM_QTYPE_Q5_K, 4>(w, x, m, y, s, epi, norm);
    }
    if (w.qtype == UNILLM_QTYPE_Q6_K) {
        if (m == 1) return launch_m<UNILLM_QTYPE_Q6_K, 1>(w, x, m, y, s, epi, norm);
        if (m == 2) return launch_m<UNILLM_QTYPE_Q6_K, 2>(w, x, m, y, s, epi, norm);
        return launch_m<UNILLM_QTYPE_Q6_K, 4>(w, x, m, y, s, epi, norm);
    }
    if (w.qtype == UNILLM_QTYPE_Q4_0) {
        if (m == 1) return launch_m<UNILLM_QTYPE_Q4_0, 1>(w, x, m, y, s, epi, norm);
        if (m == 2) return launch_m<UNILLM_QTYPE_Q4_0, 2>(w, x, m, y, s, epi, norm);
        return launch_m<UNILLM_QTYPE_Q4_0, 4>(w, x, m, y, s, epi, norm);
    }
    if (m == 1) return launch_m<UNILLM_QTYPE_Q8_0, 1>(w, x, m, y, s, epi, norm);
    if (m == 2) return launch_m<UNILLM_QTYPE_Q8_0, 2>(w, x, m, y, s, epi, norm);
    return launch_m<UNILLM_QTYPE_Q8_0, 4>(w, x, m, y, s, epi, norm);
}

}  // namespace unillm
