// decode.hip -- batched decode (m <= 64 off the GEMV path): fused dequant + f16 MFMA.
//
// y[m, n] = x[m, k] . dequant(W)[n, k]^T for continuous-batching widths, the
// QMatMul::forward call of llama.rs:1188 / 1329 with a few tokens per step.
// Bound: HBM for the weights (each byte read once).  The dequant VALU and the
// matrix cores share the rest of the time; x is re-read from L2 by every row
// group, so a workgroup owns enough rows to keep that below the weight bytes.
//
// Two kernels on the caller's stream:
//   1. xprep_kernel rounds x to f16 (round to nearest even) into a stream-ordered
//      workspace, each aligned group of 8 k stored in the order 0 2 1 3 4 6 5 7
//      (the order the dequant below produces), and zeroes y when k is split.
//      Each (token, k slice of the split below) is first scaled by the power of two
//      that puts its largest magnitude in [2^14, 2^15); the decode kernel multiplies
//      each token's partial sum by the factor that undoes it.  So any finite x works
//      (no f16 overflow, no loss to f16 subnormals), and x and x times a power of
//      two give the same operands.
//   2. decode_kernel: v_mfma_f32_32x32x16_f16 with the tokens as the A operand
//      (32 tokens x 16 k) and the weights as B (16 k x 32 weight rows), so a
//      lane's accumulator column is one weight row and the output stores and
//      atomics are 128-byte rows.
//        - A workgroup (4 waves) owns 128 weight rows and a contiguous slice of
//          the k chunks (64 k = 2 blocks each); the k range is split over S
//          workgroups when the row groups alone cannot fill the chip, and the S
//          partial sums meet in y by f32 atomic adds.
//        - Every operand comes through a D-stage LDS ring filled by direct
//          global -> LDS loads (no VGPRs): the chunk's x rows (f16), its weight
//          payloads (2 blocks per row) and its f16 scales.  Step j waits for
//          its own chunk (exact vmcnt: younger chunks stay in flight), meets
//          the other waves, issues chunk j + D - 1 and computes chunk j.
//        - Dequant, per lane (h = lane / 32): Q4_0 -- a lane takes one whole
//          block (16 payload bytes, 32 signed nibbles flipped back to q), the
//          two blocks of a pair on the two lane halves, and makes four B
//          fragments of 8 elements; MFMA q then runs over elements 8q .. 8q + 7
//          of both blocks, each lane with its own block's scale.  Q8_0 -- a lane
//          takes 16 bytes of a block (elements 16h .. 16h + 15): two fragments.
//          (code | 0x6400) is the f16 1024 + code exactly; minus 1024 + offset
//          gives the signed code exactly, times d 2^-E rounds once -- the same
//          single rounding as (q - 8) d 2^-E computed in f32 and rounded to f16.
//          Codes go two at a time from bytes (0, 2) and (1, 3) of a dword, hence
//          the element order 0 2 1 3 within each 8, matched by x's layout.
//   E is the weight's f16 exponent offset (8 max|d| 2^-E <= 65504), undone on
//   the output: both scalings are exact.
// Normwise error vs the f64 oracle ~3e-4 (f16 operands, f32 accumulation;
// bound 1e-3).
#include <hip/hip_fp16.h>

#include <algorithm>

#include "internal.hpp"
#include "lds.hpp"

namespace unillm {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int DROWS = 128;  // weight rows per workgroup (4 waves x 32)
constexpr int DCK = 128;    // k per chunk (4 blocks)

__device__ __forceinline__ uint32_t pk_f16(float a, float b) {
    uint32_t r;  // round to nearest even, a in the low half
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// v combined by op over the 64 lanes of a (whole, converged) wave, the same value in
// every lane: four DPP steps give each lane its 16-lane row's result (quad_perm
// [1,0,3,2], [2,3,0,1], row_ror 4, row_ror 8), and the four rows are read with
// v_readlane -- no LDS round trips, as a shuffle across rows would take.
template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
    v = op(v, dpp_mov<0xB1>(v));
    v = op(v, dpp_mov<0x4E>(v));
    v = op(v, dpp_mov<0x124>(v));
    v = op(v, dpp_mov<0x128>(v));
    auto lane = [&](int l) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
    };
    return op(op(lane(0), lane(16)), op(lane(32), lane(48)));
}
__device__ __forceinline__ float wave_max(float v) {
    return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ float wave_sum(float v) {
    return wave_reduce(v, [](float a, float b) { return a + b; });
}

// A signed nibble pair of w (mask 0x000F000F: bits 0 .. 3 and 16 .. 19; 0x00F000F0:
// bits 4 .. 7 and 20 .. 23) flipped to q = s + 8 under the f16 exponent 0x6400:
// ((w ^ 0x88888888) & mask) | 0x64006400 as one v_bitop3 ((w & mask) ^ k, k the
// masked flip bits and the exponent bits, which the mask leaves clear).
constexpr uint32_t kNibLo = 0x000F000Fu, kNibHi = 0x00F000F0u;
__device__ __forceinline__ uint32_t nib_f16(uint32_t w, uint32_t mask) {
    return (w & mask) ^ ((0x88888888u & mask) | 0x64006400u);
}

// f16 pair (v - bias) * dh, v holding two f16 1024 + code: exact but the last step.
__device__ __forceinline__ uint32_t scale2(uint32_t v, f16x2 bias, f16x2 dh) {
    return __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, v) - bias) * dh);
}

// Q4_0: one block's 16 payload bytes (signed nibbles: low = elements 0 .. 15,
// high = 16 .. 31) -> four fragments, elements 8q .. 8q + 7 for q = 0 .. 3, each
// in the order 0 2 1 3 4 6 5 7.  A low nibble u lands in an f16 as 1024 + u
// (minus 1032, times d); a high nibble in place, bits 4 .. 7, as 1024 + 16 u
// (minus 1152, times d / 16): one shift per dword instead of three.  dh16 = d / 16
// is exact (the weight's exponent offset keeps the scales normal in f16).
__device__ __forceinline__ void dequant_q4(u32x4 raw, f16x2 dh, f16x2 dh16, f16x8 (&f)[4]) {
    const f16x2 blo = {(_Float16)1032.0f, (_Float16)1032.0f};
    const f16x2 bhi = {(_Float16)1152.0f, (_Float16)1152.0f};
    u32x4 o[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {  // bytes 4d .. 4d + 3: elements 4d .. (low), 16 + 4d .. (high)
        const uint32_t w = raw[d], w8 = w >> 8;
        const int lo = d / 2, e = 2 * (d % 2);
        o[lo][e] = scale2(nib_f16(w, kNibLo), blo, dh);             // bytes 0, 2 low
        o[lo][e + 1] = scale2(nib_f16(w8, kNibLo), blo, dh);        // bytes 1, 3 low
        o[2 + lo][e] = scale2(nib_f16(w, kNibHi), bhi, dh16);       // bytes 0, 2 high
        o[2 + lo][e + 1] = scale2(nib_f16(w8, kNibHi), bhi, dh16);  // bytes 1, 3 high
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) f[q] = __builtin_bit_cast(f16x8, o[q]);
}

// Q4_K: as dequant_q4 with the block's f16 scale s = d sc 2^-E and min o =
// dmin m 2^-E: (1024 + q - 1024) s - o (high nibbles: (1024 + 16 q - 1024) s / 16 - o).
// s and o are rounded to f16 once each, the weight once more.
__device__ __forceinline__ void dequant_q4k(u32x4 raw, f16x2 sh, f16x2 sh16, f16x2 oh,
                                            f16x8 (&f)[4]) {
    const f16x2 b = {(_Float16)1024.0f, (_Float16)1024.0f};
    auto fma2 = [&](uint32_t v, f16x2 sc) {
        return __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, v) - b) * sc - oh);
    };
    u32x4 o[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t w = raw[d], w8 = w >> 8;
        const int lo = d / 2, e = 2 * (d % 2);
        o[lo][e] = fma2(nib_f16(w, kNibLo), sh);
        o[lo][e + 1] = fma2(nib_f16(w8, kNibLo), sh);
        o[2 + lo][e] = fma2(nib_f16(w, kNibHi), sh16);
        o[2 + lo][e + 1] = fma2(nib_f16(w8, kNibHi), sh16);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) f[q] = __builtin_bit_cast(f16x8, o[q]);
}

// Q8_0: 16 payload bytes (elements 16h .. 16h + 15) -> two fragments (elements
// 16h .. +7 and 16h + 8 .. +7), each in the order 0 2 1 3 4 6 5 7.
__device__ __forceinline__ void dequant_q8(u32x4 raw, f16x2 dh, f16x8& f0, f16x8& f1) {
    const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t magic = 0x64646464u;
    u32x4 a, b;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t w = raw[d] ^ 0x80808080u;  // int8 -> q + 128
        // bytes (0, 2) and (1, 3) each under a 0x64 byte: f16 1024 + byte
        const uint32_t p02 = __builtin_amdgcn_perm(magic, w, 0x04020400u);
        const uint32_t p13 = __builtin_amdgcn_perm(magic, w, 0x04030401u);
        u32x4& o = d < 2 ? a : b;
        o[2 * (d & 1)] = scale2(p02, bias, dh);
        o[2 * (d & 1) + 1] = scale2(p13, bias, dh);
    }
    f0 = __builtin_bit_cast(f16x8, a);
    f1 = __builtin_bit_cast(f16x8, b);
}

// Q5_K: as dequant_q8 for the int8 codes c = q - 16, with the block's f16 scale s =
// d sc 2^-E and min o = dmin m 2^-E: (1024 + c + 128 - 1136) s - o = q s - o (s and o
// rounded to f16 once each, as Q4_K's).
__device__ __forceinline__ void dequant_q8m(u32x4 raw, f16x2 sh, f16x2 oh, f16x8& f0, f16x8& f1) {
    const f16x2 bias = {(_Float16)1136.0f, (_Float16)1136.0f};
    const uint32_t magic = 0x64646464u;
    auto fma2 = [&](uint32_t v) {
        return __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, v) - bias) * sh - oh);
    };
    u32x4 a, b;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint32_t w = raw[d] ^ 0x80808080u;  // int8 -> c + 128
        const uint32_t p02 = __builtin_amdgcn_perm(magic, w, 0x04020400u);
        const uint32_t p13 = __builtin_amdgcn_perm(magic, w, 0x04030401u);
        u32x4& o = d < 2 ? a : b;
        o[2 * (d & 1)] = fma2(p02);
        o[2 * (d & 1) + 1] = fma2(p13);
    }
    f0 = __builtin_bit_cast(f16x8, a);
    f1 = __builtin_bit_cast(f16x8, b);
}

}  // namespace

// The power-of-two scale of an f16 operand row (or slice) whose largest magnitude is
// mx: the values are multiplied by 2^(15 - e) (mx < 2^e), so the largest lands in
// [2^14, 2^15) whatever the range; thread 0 stores the inverse, the output factor
// 2^(e - 15), at *rs.  Zero or non-finite inputs keep the factor 1.  Both scalings are
// exact, so x and x times a power of two give the same f16 operand.
__device__ __forceinline__ float f16_row_scale(float mx, float* rs) {
    int e = 0;
    const bool ok = mx > 0.0f && mx <= 3.402823466e38f;
    if (ok) (void)frexpf(mx, &e);
    e = e < -111 ? -111 : e;  // keep 2^(15 - e) and 2^(e - 15) in range
    if (threadIdx.x == 0) *rs = ok ? ldexpf(1.0f, e - 15) : 1.0f;
    return ok ? ldexpf(1.0f, 15 - e) : 1.0f;
}

namespace {

// Slice s of S of a row of k elements: the decode kernel's k split, 128-k chunks
// [s C / S, (s + 1) C / S) with C = ceil(k / 128) (elements [e0, e1)).
__device__ __forceinline__ void slice_range(int64_t k, int S, int s, int64_t& e0, int64_t& e1) {
    const int64_t C = (k + 127) / 128;
    e0 = (int64_t)s * C / S * 128;
    e1 = min((int64_t)(s + 1) * C / S * 128, k);
}

// One workgroup (128 threads, one aligned group of 8 elements each) per (row r, k slice
// s) of x[m, k]: the slice's largest magnitude, then the slice scaled by the power of two
// that puts it in [2^14, 2^15) and rounded to f16 (round to nearest even) in the fragment
// order 0 2 1 3 4 6 5 7 of each 8; rf[s * 64 + r] <- the factor that undoes the scaling
// (f16_row_scale).  Each slice is at most kMaxSliceChunks * 128 = 1024 elements.  Any
// finite x works: no overflow past 65504, no loss to f16 subnormals, and x and x times
// a power of two give the same operand.  y row r is zeroed over columns
// [s ny / S, (s + 1) ny / S) when ny > 0 (a split k range adds into it).
__global__ __launch_bounds__(128) void xprep_kernel(const float* __restrict__ x, int64_t k,
                                                    int S, uint4* __restrict__ xh,
                                                    float* __restrict__ rf,
                                                    float* __restrict__ y, int64_t ny) {
    __shared__ float red[2];
    const int r = blockIdx.x / S, s = blockIdx.x % S;
    const int t = threadIdx.x;
    int64_t e0, e1;
    slice_range(k, S, s, e0, e1);
    const int64_t g = e0 / 8 + t;
    const bool live = 8 * (int64_t)t < e1 - e0;
    const float4* xr = reinterpret_cast<const float4*>(x + (int64_t)r * k);
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    if (live) {
        a = xr[2 * g];
        b = xr[2 * g + 1];
    }
    auto amax4 = [](float4 v) {
        return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    };
    float mx = fmaxf(amax4(a), amax4(b));
    mx = wave_max(mx);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    const float sc = f16_row_scale(fmaxf(red[0], red[1]), rf + (int64_t)s * 64 + r);
    if (live)
        xh[(int64_t)r * (k / 8) + g] =
            make_uint4(pk_f16(a.x * sc, a.z * sc), pk_f16(a.y * sc, a.w * sc),
                       pk_f16(b.x * sc, b.z * sc), pk_f16(b.y * sc, b.w * sc));
    if (ny > 0) {
        const int64_t c0 = (int64_t)s * ny / S, c1 = (int64_t)(s + 1) * ny / S;
        for (int64_t c = c0 + t; c < c1; c += 128) y[(int64_t)r * ny + c] = 0.0f;
    }
}

// LDS: a D-stage ring, each stage one 128-k chunk of
//   x   [TOK rows][256 B] f16; the 16-byte group g of row r sits in slot g ^ (r % 16);
//   W   [128 rows][4 QB] payloads of the chunk's 4 blocks; the 16-byte piece c
//       of row r sits in slot c ^ swz(r),
// then the workgroup's k-slice scales, per wave [32 rows][8 x 8 B] (at most
// kMaxSliceChunks = 8 chunks: 2 KiB a wave), chunk j of row r at position
// (j + r) % 8, loaded once before the ring starts.  The swizzles and the
// rotation put the rows (tokens) that one LDS read pass serves -- 8 or 16
// consecutive lanes -- on distinct banks.
constexpr int kMaxSliceChunks = 8;
// most k slices of one row (a row of up to 256 * 8 * 128 = 262144 elements)
constexpr int kMaxSplitSlices = 256;
// At most this many k slices add into one output when the row groups alone leave
// CUs idle: 8 for one 32-token tile (m16 n4096: 9.9 us a call against 11.1 with 4),
// 4 for two (more slices contend on the same y lines with their atomics; m64 n4096:
// 16.0 us with 4 against 16.4 with 8).
constexpr int kMaxSplit1 = 8, kMaxSplit2 = 4;

template <int QT, int MT2>
struct Stage {
    static constexpr int QB =
        QT == UNILLM_QTYPE_Q8_0 || QT == UNILLM_QTYPE_Q5_K || QT == UNILLM_QTYPE_Q6_K ? 32 : 16;
    static constexpr int TOK = 32 * MT2;
    static constexpr int X = TOK * 256;
    static constexpr int P = DROWS * 4 * QB;
    static constexpr int BYTES = X + P;
    static constexpr int XD = TOK * 256 / 1024 / 4;  // x direct loads per wave per chunk
    static constexpr int PD = 32 * 4 * QB / 1024;    // payload direct loads per wave (2 / 4)
    static constexpr int LPC = XD + PD;
    static constexpr int LPR = 4 * QB / 16;          // payload lanes per row (4 / 8)
    static constexpr int RPI = 64 / LPR;             // payload rows per direct load
    static constexpr int SCALES = 4 * 32 * 8 * kMaxSliceChunks;
    // K-quants: the slice's group headers, per wave [32 rows][8 x 4 B] (a slice of
    // at most 8 chunks touches at most 5 groups of 2 chunks)
    static constexpr int HDR =
        QT == UNILLM_QTYPE_Q4_K || QT == UNILLM_QTYPE_Q5_K || QT == UNILLM_QTYPE_Q6_K ? 4 * 32 * 32
                                                                                     : 0;
    // depth: as deep as keeps two workgroups per CU, where the stage allows
    static constexpr int D = BYTES <= 16384 ? 4 : 3;
    static constexpr int LDS = D * BYTES + SCALES + HDR;
};

// s_waitcnt vmcnt(rem * LPC) for a wave-uniform rem in [0, R].
template <int LPC, int R>
__device__ __forceinline__ void wait_chunks(int rem) {
    if constexpr (R == 0) {
        wait_vmcnt<0>();
    } else {
        if (rem >= R) wait_vmcnt<R * LPC>();
        else wait_chunks<LPC, R - 1>(rem);
    }
}

// The LDS reads for half a chunk (two blocks) and the wait for them in ONE asm
// statement: the outputs are early-clobber and defined only once the statement
// ends, so the compiler cannot copy a destination register before its data has
// landed (with separate asm reads it may, and the copy reads a stale register).
//   x: four fragment groups (a0 .. a3), tile 1 at +8192; payload: Q4_0 one
//   block (16 bytes at p0), Q8_0 half of each of two blocks (16 bytes at p0, p1);
//   the chunk's four f16 scales (8 bytes at sa).
#define UNILLM_DS128(o, a, off) "ds_read_b128 %" #o ", %" #a " offset:" #off "\n"
#define UNILLM_DS64(o, a, off) "ds_read_b64 %" #o ", %" #a " offset:" #off "\n"
template <bool Q4, int MT2>
__device__ __forceinline__ void read_half(lds_u32x4 (&xa)[MT2][4], u32x4 (&pw)[2],
                                          lds_u32x2& scp, uint32_t a0, uint32_t a1, uint32_t a2,
                                          uint32_t a3, uint32_t p0, uint32_t p1, uint32_t sa) {
    lds_u32x4 w0, w1;
    if constexpr (Q4 && MT2 == 1) {
        asm volatile(UNILLM_DS128(0, 6, 0) UNILLM_DS128(1, 7, 0) UNILLM_DS128(2, 8, 0)
                         UNILLM_DS128(3, 9, 0) UNILLM_DS128(4, 10, 0) UNILLM_DS64(5, 11, 0)
                             "s_waitcnt lgkmcnt(0)"
                     : "=&v"(xa[0][0]), "=&v"(xa[0][1]), "=&v"(xa[0][2]), "=&v"(xa[0][3]),
                       "=&v"(w0), "=&v"(scp)
                     : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "v"(p0), "v"(sa));
        w1 = w0;
    } else if constexpr (Q4) {
        asm volatile(UNILLM_DS128(0, 10, 0) UNILLM_DS128(1, 11, 0) UNILLM_DS128(2, 12, 0)
                         UNILLM_DS128(3, 13, 0) UNILLM_DS128(4, 10, 8192) UNILLM_DS128(5, 11, 8192)
                             UNILLM_DS128(6, 12, 8192) UNILLM_DS128(7, 13, 8192)
                                 UNILLM_DS128(8, 14, 0) UNILLM_DS64(9, 15, 0)
                                     "s_waitcnt lgkmcnt(0)"
                     : "=&v"(xa[0][0]), "=&v"(xa[0][1]), "=&v"(xa[0][2]), "=&v"(xa[0][3]),
                       "=&v"(xa[MT2 - 1][0]), "=&v"(xa[MT2 - 1][1]), "=&v"(xa[MT2 - 1][2]),
                       "=&v"(xa[MT2 - 1][3]), "=&v"(w0), "=&v"(scp)
                     : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "v"(p0), "v"(sa));
        w1 = w0;
    } else if constexpr (MT2 == 1) {
        asm volatile(UNILLM_DS128(0, 7, 0) UNILLM_DS128(1, 8, 0) UNILLM_DS128(2, 9, 0)
                         UNILLM_DS128(3, 10, 0) UNILLM_DS128(4, 11, 0) UNILLM_DS128(5, 12, 0)
                             UNILLM_DS64(6, 13, 0) "s_waitcnt lgkmcnt(0)"
                     : "=&v"(xa[0][0]), "=&v"(xa[0][1]), "=&v"(xa[0][2]), "=&v"(xa[0][3]),
                       "=&v"(w0), "=&v"(w1), "=&v"(scp)
                     : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "v"(p0), "v"(p1), "v"(sa));
    } else {
        asm volatile(UNILLM_DS128(0, 11, 0) UNILLM_DS128(1, 12, 0) UNILLM_DS128(2, 13, 0)
                         UNILLM_DS128(3, 14, 0) UNILLM_DS128(4, 11, 8192) UNILLM_DS128(5, 12, 8192)
                             UNILLM_DS128(6, 13, 8192) UNILLM_DS128(7, 14, 8192)
                                 UNILLM_DS128(8, 15, 0) UNILLM_DS128(9, 16, 0)
                                     UNILLM_DS64(10, 17, 0) "s_waitcnt lgkmcnt(0)"
                     : "=&v"(xa[0][0]), "=&v"(xa[0][1]), "=&v"(xa[0][2]), "=&v"(xa[0][3]),
                       "=&v"(xa[MT2 - 1][0]), "=&v"(xa[MT2 - 1][1]), "=&v"(xa[MT2 - 1][2]),
                       "=&v"(xa[MT2 - 1][3]), "=&v"(w0), "=&v"(w1), "=&v"(scp)
                     : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "v"(p0), "v"(p1), "v"(sa));
    }
    pw[0] = __builtin_bit_cast(u32x4, w0);
    pw[1] = __builtin_bit_cast(u32x4, w1);
}
#undef UNILLM_DS128
#undef UNILLM_DS64

template <int QT, int MT2>
__global__ __launch_bounds__(256) void decode_kernel(const uint8_t* __restrict__ base, int64_t rb,
                                                     const _Float16* __restrict__ xh,
                                                     const float* __restrict__ rf,
                                                     float* __restrict__ y, int M, int N, int KB,
                                                     int S, float wscale, float oscale, int add) {
    using ST = Stage<QT, MT2>;
    constexpr int QB = ST::QB, D = ST::D, LPC = ST::LPC;
    // 4-bit codes: Q4_0 and Q4_K; byte codes: Q8_0, Q5_K and Q6_K (repacked to int8)
    constexpr bool Q4 = QT == UNILLM_QTYPE_Q4_0 || QT == UNILLM_QTYPE_Q4_K;
    constexpr bool K4 = QT == UNILLM_QTYPE_Q4_K, K6 = QT == UNILLM_QTYPE_Q6_K;
    constexpr bool K5 = QT == UNILLM_QTYPE_Q5_K;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t* const ring = lds;
    uint8_t* const scl = lds + D * ST::BYTES;
    uint8_t* const hdr = scl + ST::SCALES;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, col = lane & 31;
    const uint32_t K = (uint32_t)KB * QK;

    // workgroup -> (row group, k slice); the slice is chunks [c0, c1), at most
    // kMaxSliceChunks of them (the host picks S so)
    const int rg = blockIdx.x / S, sp = blockIdx.x % S;
    const int chunks = (KB + 3) / 4;
    const int c0 = (int)((int64_t)sp * chunks / S), c1 = (int)((int64_t)(sp + 1) * chunks / S);
    const int nch = c1 - c0;
    const int row0 = rg * DROWS + 32 * wv;  // this wave's 32 weight rows
    const uint32_t sbase = (uint32_t)KB * QB;  // the scales follow the payloads in a row

    // ---- the output factors of this k slice's token rows (the power-of-two scale x's
    // slice took in xprep_kernel): token 32 t + 8 q + 4 h + e in fac[t][q] component e.
    // Loaded first, so every later wait covers them; tokens past m read unused values.
    float4 fac[MT2][4];
#pragma unroll
    for (int t = 0; t < MT2; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            fac[t][q] = *reinterpret_cast<const float4*>(rf + sp * 64 + 32 * t + 8 * q + 4 * h);

    // ---- the slice's scales: 8 positions of 8 bytes a row (kMaxSliceChunks), 8
    // dword loads per wave; lane -> flat dword f = 64 i + lane = row f / 16,
    // position f % 16 / 2, which holds chunk (position - row) % 8 (positions past
    // the slice repeat its last chunk; past the last block: the row's padding, the
    // next row or the tail slot, zeroed below) ----
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int f = 64 * i + lane;
        const int r = f >> 4, dw = f & 15;
        const int jj = min(((dw >> 1) - r) & 7, nch - 1);
        const uint32_t g = (uint32_t)min(row0 + r, N - 1) * (uint32_t)rb + sbase +
                           8u * (uint32_t)(c0 + jj) + 4u * (uint32_t)(dw & 1);
        dma4(base + g, scl + wv * 2048 + i * 256);
    }
    // ---- K-quants: the slice's group headers (Q4_K, Q5_K d | dmin << 16, Q6_K d), 8
    // positions of 4 bytes a row; lane -> flat dword f = 64 i + lane = row f / 8,
    // position f % 8 = group c0 / 2 + position (clamped to the slice's last group) ----
    if constexpr (K4 || K5 || K6) {
        const int g0 = c0 >> 1, glast = (c1 - 1) >> 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int f = 64 * i + lane;
            const int r = f >> 3, grp = min(g0 + (f & 7), glast);
            const uint32_t g = (uint32_t)min(row0 + r, N - 1) * (uint32_t)rb +
                               (uint32_t)KB * (QB + 2u) + 4u * (uint32_t)grp;
            dma4(base + g, hdr + wv * 1024 + i * 256);
        }
    }

    // ---- per-chunk direct-load sources (32-bit offsets; the host checks sizes) ----
    // x: load q = XD wv + i covers token rows 4q .. 4q + 3; lane -> row 4q + lane / 16,
    // slot lane % 16 <- group (lane % 16) ^ (row % 16).  Rows past m read row m - 1
    // and k past K the row's last group (finite values against zero weights).
    uint32_t xoff[ST::XD], xgrp[ST::XD];
#pragma unroll
    for (int i = 0; i < ST::XD; ++i) {
        const int r = 4 * (ST::XD * wv + i) + (lane >> 4);
        xoff[i] = (uint32_t)min(r, M - 1) * K;
        xgrp[i] = (uint32_t)(((lane & 15) ^ (r & 15)) * 8);
    }
    // payload: load i covers wave rows RPI i ..; lane -> row RPI i + lane / LPR,
    // slot lane % LPR <- piece (lane % LPR) ^ swz(row)
    //   Q4_0 ((r / 2) % 4) ^ (r / 8 % 2), Q8_0 (r % 8) ^ (r / 8 % 2): distinct (row
    //   parity, slot) pairs over any 8 and any aligned 16 consecutive rows
    auto swz = [](int r) { return (Q4 ? (r >> 1) & 3 : r & 7) ^ ((r >> 3) & 1); };
    uint32_t poff[ST::PD];
#pragma unroll
    for (int i = 0; i < ST::PD; ++i) {
        const int r = ST::RPI * i + lane / ST::LPR;
        const int piece = (lane % ST::LPR) ^ swz(r);
        poff[i] = (uint32_t)min(row0 + r, N - 1) * (uint32_t)rb + (uint32_t)(16 * piece);
    }
    // A wave whose x rows all lie past m loads none: padded token rows only feed
    // the outputs of padded tokens (never stored), so their LDS rows may hold
    // anything.  Its loads per chunk are then PD, not LPC.
    const bool xw = 4 * ST::XD * wv < M;
    auto issue = [&](int j) {  // this wave's loads of chunk c0 + j into stage j % D
        const uint32_t c = (uint32_t)(c0 + j);
        uint8_t* st = ring + (j % D) * ST::BYTES;
        if (xw) {
#pragma unroll
            for (int i = 0; i < ST::XD; ++i)
                dma16(xh + xoff[i] + min(c * DCK + xgrp[i], K - 8),
                      st + (ST::XD * wv + i) * 1024);
        }
#pragma unroll
        for (int i = 0; i < ST::PD; ++i)
            dma16(base + poff[i] + c * (4 * QB), st + ST::X + (ST::PD * wv + i) * 1024);
    };

    f32x16 acc[MT2];
#pragma unroll
    for (int t = 0; t < MT2; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[t][e] = 0.0f;

    // ---- LDS offsets within a stage (chunk-independent) ----
    // Q4_0: half p of the chunk is blocks 2p (h = 0) and 2p + 1 (h = 1); a lane
    // reads its block (piece 2p + h) and feeds four MFMAs, the q-th with elements
    // 8q .. 8q + 7 of that block (x group 4 (2p + h) + q).  Q8_0: half p is blocks
    // 2p, 2p + 1; a lane reads half h of each (piece 2i + h), elements 16h .. +15
    // (x groups 4i + 2h, 4i + 2h + 1).
    uint32_t xo[8];
#pragma unroll
    for (int hp = 0; hp < 2; ++hp)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = 2 * hp + q / 2;  // Q8_0 block
            const int g = Q4 ? 8 * hp + 4 * h + q : 4 * i + 2 * h + (q & 1);
            xo[4 * hp + q] = (uint32_t)(col * 256 + 16 * (g ^ (col & 15)));
        }
    uint32_t po[4];
    const int prow = 32 * wv + col;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int piece = Q4 ? (2 * (i & 1) + h) : 2 * i + h;  // Q4_0 uses po[0], po[1]
        po[i] = (uint32_t)(ST::X + prow * 4 * QB + 16 * (piece ^ swz(col)));
    }
    const uint32_t ring0 = (uint32_t)(uintptr_t)ring;
    const uint32_t srow = (uint32_t)(uintptr_t)scl + (uint32_t)(wv * 2048 + col * 64);
    const uint32_t hrow = (uint32_t)(uintptr_t)hdr + (uint32_t)(wv * 1024 + col * 32);

    auto compute = [&](int j) {
        const uint32_t st = ring0 + (uint32_t)((j % D) * ST::BYTES);
        const int kb0 = 4 * (c0 + j);
        const uint32_t sa = srow + 8 * ((j + col) & 7);
        // Q4_K: the chunk's group header (the 4 blocks of a chunk share one group)
        float gd = 0.0f, gm = 0.0f;
        if constexpr (K4 || K5 || K6) {
            uint32_t hd;
            asm volatile("ds_read_b32 %0, %1\n s_waitcnt lgkmcnt(0)"
                         : "=&v"(hd)
                         : "v"(hrow + 4u * (uint32_t)(((c0 + j) >> 1) - (c0 >> 1))));
            gd = __half2float(__ushort_as_half((uint16_t)hd)) * wscale;
            gm = __half2float(__ushort_as_half((uint16_t)(hd >> 16))) * wscale;
        }
#pragma unroll
        for (int hp = 0; hp < 2; ++hp) {
            lds_u32x4 xa[MT2][4];
            u32x4 pw[2];
            lds_u32x2 scp;
            read_half<Q4, MT2>(xa, pw, scp, st + xo[4 * hp], st + xo[4 * hp + 1],
                               st + xo[4 * hp + 2], st + xo[4 * hp + 3],
                               st + po[Q4 ? hp : 2 * hp], st + po[Q4 ? hp : 2 * hp + 1], sa);
            if constexpr (Q4) {
                // this lane's block 2 hp + h and its scale
                const uint16_t sb = (uint16_t)(scp[hp] >> (16 * h));
                const bool ok = kb0 + 2 * hp + h < KB;
                f16x8 b[4];
                if constexpr (K4) {
                    // sb = sc | m << 8: s = d sc 2^-E and o = dmin m 2^-E, each once to f16
                    const float sv = ok ? gd * (float)(sb & 0xFFu) : 0.0f;
                    const float ov = ok ? gm * (float)(sb >> 8) : 0.0f;
                    const _Float16 s1 = (_Float16)sv, s16 = (_Float16)(sv * 0.0625f),
                                   o1 = (_Float16)ov;
                    const f16x2 sh = {s1, s1}, sh16 = {s16, s16}, oh = {o1, o1};
                    dequant_q4k(pw[0], sh, sh16, oh, b);
                } else {
                    const float dv = ok ? __half2float(__ushort_as_half(sb)) * wscale : 0.0f;
                    const _Float16 d = (_Float16)dv, d16 = (_Float16)(dv * 0.0625f);
                    const f16x2 dh = {d, d}, dh16 = {d16, d16};
                    dequant_q4(pw[0], dh, dh16, b);
                }
#pragma unroll
                for (int t = 0; t < MT2; ++t)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(f16x8, xa[t][q]), b[q], acc[t], 0, 0, 0);
            } else {
#pragma unroll
                for (int bi = 0; bi < 2; ++bi) {
                    const uint16_t sb = (uint16_t)(scp[hp] >> (16 * bi));
                    const bool ok = kb0 + 2 * hp + bi < KB;
                    // Q6_K: sb = the two int8 scales; this lane's 16 weights take half h's
                    f16x8 b0, b1;
                    if constexpr (K5) {
                        // sb = sc | m << 8: s = d sc 2^-E, o = dmin m 2^-E, each once to f16
                        const _Float16 s1 = (_Float16)(ok ? gd * (float)(sb & 0xFFu) : 0.0f);
                        const _Float16 o1 = (_Float16)(ok ? gm * (float)(sb >> 8) : 0.0f);
                        const f16x2 sh = {s1, s1}, oh = {o1, o1};
                        dequant_q8m(pw[bi], sh, oh, b0, b1);
                    } else {
                        const float dv = !ok ? 0.0f
                                         : K6 ? gd * (float)(int8_t)(sb >> (8 * h))
                                              : __half2float(__ushort_as_half(sb)) * wscale;
                        const _Float16 d = (_Float16)dv;
                        const f16x2 dh = {d, d};
                        dequant_q8(pw[bi], dh, b0, b1);
                    }
#pragma unroll
                    for (int t = 0; t < MT2; ++t) {
                        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(f16x8, xa[t][2 * bi]), b0, acc[t], 0, 0, 0);
                        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(f16x8, xa[t][2 * bi + 1]), b1, acc[t], 0, 0, 0);
                    }
                }
            }
        }
    };

    // chunks 0 .. D - 2 in flight before the first step; step j waits for its own
    // chunk (the min(D - 2, nch - 1 - j) younger ones may stay in flight; the
    // scale loads are older than all), meets the other waves (its x rows are then
    // complete and stage (j - 1) % D is free), issues chunk j + D - 1 and computes
    // chunk j.  The last step waits for everything: no direct load outlives the loop.
    for (int j = 0; j < D - 1 && j < nch; ++j) issue(j);
    for (int j = 0; j < nch; ++j) {
        if (xw) wait_chunks<LPC, D - 2>(min(D - 2, nch - 1 - j));
        else wait_chunks<ST::PD, D - 2>(min(D - 2, nch - 1 - j));
        __builtin_amdgcn_s_barrier();
        if (j + D - 1 < nch) issue(j + D - 1);
        compute(j);
    }

    // ---- epilogue: acc[t][r] = C[token 32 t + 8 (r / 4) + 4 h + r % 4][row row0 + col] ----
    // Each token's sum is scaled back by its slice factor and the weight's 2^E.  A
    // split k range (S > 1) meets in y by f32 atomic adds onto zeros.  With m % 8 == 0
    // a token block (t, r / 4) is valid for all lanes or none.
    const int n = row0 + col;
    if (n < N) {
        float* yb = y + (int64_t)(4 * h) * N + n;
        // y += (the residual add) or y =; a split k range always adds (onto zeros
        // written by xprep_kernel, or onto y itself with add)
        auto put = [&](float* dst, float v, float f) {
            const float o = v * (f * oscale);
            if (S == 1) *dst = add ? *dst + o : o;
            else unsafeAtomicAdd(dst, o);
        };
        auto fct = [&](int t, int r) {
            const float4 f = fac[t][r / 4];
            return r % 4 == 0 ? f.x : r % 4 == 1 ? f.y : r % 4 == 2 ? f.z : f.w;
        };
        if (M % 8 == 0) {
#pragma unroll
            for (int t = 0; t < MT2; ++t)
#pragma unroll
                for (int rb4 = 0; rb4 < 4; ++rb4) {
                    if (32 * t + 8 * rb4 >= M) break;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        put(yb + (int64_t)(32 * t + 8 * rb4 + e) * N, acc[t][4 * rb4 + e],
                            fct(t, 4 * rb4 + e));
                }
        } else {
#pragma unroll
            for (int t = 0; t < MT2; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m0 = 32 * t + 8 * (r / 4) + (r % 4);
                    if (m0 + 4 * h < M) put(yb + (int64_t)m0 * N, acc[t][r], fct(t, r));
                }
        }
    }
}

// ---- one launch for up to 16 tokens (decode_x_kernel) ---------------------------------------
// The same product as decode_kernel at m <= 16, with x read as f32 by the kernel itself:
// each workgroup turns its k slice of the m rows of x into f16 in LDS (the slice's
// power-of-two scale per row, as xprep_kernel computes it) while its first weight
// chunks stream in, so no conversion launch runs before it.  The ring then carries
// weights only.  A k range split over S workgroups meets in y as decode_kernel's
// does, by f32 atomic adds; y is zeroed by the row group's k slice 0 at its start,
// which then raises the group's flag (after its prologue, long before any slice
// finishes).  Each slice checks the flag before it adds; the last to pass resets the
// flag for the next launch (the words live in the stream's workspace, zeroed when it
// is allocated).  The host takes this kernel only where every workgroup of the grid
// fits on the device at once, so each wait is on a workgroup that runs; it is
// bounded all the same.
constexpr int kXinMaxM = 16;
constexpr int kXinRowBytes = 256;  // one 128-k chunk of one row, f16
constexpr int kXinLdsBudget = 80 * 1024;  // two workgroups a CU (160 KiB)
constexpr int kSyncStride = 32;    // u32 words between counters (128-byte lines)
constexpr int kSyncPoll = 1 << 20;

// XC: the chunks of x the LDS holds (a slice's length at most: 4 or kMaxSliceChunks);
// the ring takes as many weight stages as the rest of the budget holds, so a short
// slice is requested whole in the prologue.
template <int QT, int XC>
struct XinStage {
    static constexpr int QB = Stage<QT, 1>::QB;
    static constexpr int P = DROWS * 4 * QB;         // the chunk's weight payloads
    static constexpr int PD = 32 * 4 * QB / 1024;    // direct loads per wave (2 / 4)
    static constexpr int LPR = 4 * QB / 16;
    static constexpr int RPI = 64 / LPR;
    static constexpr int SCALES = Stage<QT, 1>::SCALES;
    static constexpr int HDR = Stage<QT, 1>::HDR;
    static constexpr int XAREA = XC * kXinMaxM * kXinRowBytes;
    static constexpr int D = (kXinLdsBudget - XAREA - SCALES - HDR - 64 * 4) / P;
    static constexpr int LDS = XAREA + D * P + SCALES + HDR + 64 * 4;
    static_assert(D >= 2 && XC <= kMaxSliceChunks, "ring of at least two stages");
};

// Sync words per row group (128-byte lines apart): [0] y's tile is zero, [32] slices
// past the flag, [64] unused.
size_t xin_sync_bytes(int64_t groups) { return (size_t)(groups + 1) * 3 * kSyncStride * 4; }

template <int QT, int XC>
__global__ __launch_bounds__(256) void decode_x_kernel(const uint8_t* __restrict__ base, int64_t rb,
                                                       const float* __restrict__ x,
                                                       float* __restrict__ y, int M, int N, int KB,
                                                       int S, float wscale, float oscale, int add,
                                                       unsigned* __restrict__ sync) {
    // every argument in registers behind one wait (left to itself the compiler fetches
    // them one branch at a time, a round trip each)
    asm volatile("" ::"s"(base), "s"(rb), "s"(x), "s"(y), "s"(M), "s"(N), "s"(KB), "s"(S),
                 "s"(wscale), "s"(oscale), "s"(add), "s"(sync));
    using ST = XinStage<QT, XC>;
    constexpr int QB = ST::QB, D = ST::D;
    constexpr bool Q4 = QT == UNILLM_QTYPE_Q4_0 || QT == UNILLM_QTYPE_Q4_K;
    constexpr bool K4 = QT == UNILLM_QTYPE_Q4_K, K6 = QT == UNILLM_QTYPE_Q6_K;
    constexpr bool K5 = QT == UNILLM_QTYPE_Q5_K;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t* const xarea = lds;
    uint8_t* const ring = lds + ST::XAREA;
    uint8_t* const scl = ring + D * ST::P;
    uint8_t* const hdr = scl + ST::SCALES;
    // [16] the rows' factors; [32] NaN when the epilogue's wait gave up (64 floats held)
    float* const facs = reinterpret_cast<float*>(hdr + ST::HDR);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, col = lane & 31;
    const int K = KB * QK;
    const int rg = blockIdx.x / S, sp = blockIdx.x % S;
    const int chunks = (KB + 3) / 4;
    const int c0 = (int)((int64_t)sp * chunks / S), c1 = (int)((int64_t)(sp + 1) * chunks / S);
    const int nch = c1 - c0;
    const int row0 = rg * DROWS + 32 * wv;
    const uint32_t sbase = (uint32_t)KB * QB;

    // ---- k slice 0 of a split that stores: y's tile of this row group to zero first
    // (device-coherent stores; the flag follows once they are complete) ----
    const bool zero_tile = S > 1 && !add && sp == 0;
    if (zero_tile) {
        for (int i = tid; i < M * DROWS; i += 256) {
            const int t = i / DROWS, n = rg * DROWS + i % DROWS;
            if (n < N)
                __hip_atomic_store(reinterpret_cast<unsigned*>(y + (int64_t)t * N + n), 0u,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    // ---- x: row r = tid / 16 of the slice, groups of 8 elements g = tid % 16 + 16 i
    // (chunk i, group g % 16 of its 16); requested first.  Rows past m, chunks past the
    // slice and elements past k are not read: zero. ----
    const int xr = tid >> 4, xg = tid & 15;
    float4 xv[XC][2];
#pragma unroll
    for (int i = 0; i < XC; ++i) {
        const int e = (c0 + i) * 128 + 8 * xg;
        xv[i][0] = xv[i][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (xr < M && i < nch && e < K) {
            const float4* src = reinterpret_cast<const float4*>(x + (int64_t)xr * K + e);
            xv[i][0] = src[0];
            xv[i][1] = src[1];
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // x requested before every direct load


    // ---- the slice's weight scales and K-quant headers (as decode_kernel) ----
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int f = 64 * i + lane;
        const int r = f >> 4, dw = f & 15;
        const int jj = min(((dw >> 1) - r) & 7, nch - 1);
        const uint32_t g = (uint32_t)min(row0 + r, N - 1) * (uint32_t)rb + sbase +
                           8u * (uint32_t)(c0 + jj) + 4u * (uint32_t)(dw & 1);
        dma4(base + g, scl + wv * 2048 + i * 256);
    }
    if constexpr (K4 || K5 || K6) {
        const int g0 = c0 >> 1, glast = (c1 - 1) >> 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int f = 64 * i + lane;
            const int r = f >> 3, grp = min(g0 + (f & 7), glast);
            const uint32_t g = (uint32_t)min(row0 + r, N - 1) * (uint32_t)rb +
                               (uint32_t)KB * (QB + 2u) + 4u * (uint32_t)grp;
            dma4(base + g, hdr + wv * 1024 + i * 256);
        }
    }

    // ---- weight payloads: the ring's direct loads (decode_kernel's layout) ----
    auto swz = [](int r) { return (Q4 ? (r >> 1) & 3 : r & 7) ^ ((r >> 3) & 1); };
    uint32_t poff[ST::PD];
#pragma unroll
    for (int i = 0; i < ST::PD; ++i) {
        const int r = ST::RPI * i + lane / ST::LPR;
        const int piece = (lane % ST::LPR) ^ swz(r);
        poff[i] = (uint32_t)min(row0 + r, N - 1) * (uint32_t)rb + (uint32_t)(16 * piece);
    }
    auto issue = [&](int j) {
        const uint32_t c = (uint32_t)(c0 + min(j, nch - 1));
        uint8_t* st = ring + (j % D) * ST::P;
#pragma unroll
        for (int i = 0; i < ST::PD; ++i)
            dma16(base + poff[i] + c * (4 * QB), st + (ST::PD * wv + i) * 1024);
    };
    // the first D - 1 chunks of the slice (each later one is requested D - 1 chunks
    // ahead of its use, so the chunk waits below count exactly what is in flight)
#pragma unroll
    for (int j = 0; j < D - 1; ++j)
        if (j < nch) issue(j);
    __builtin_amdgcn_sched_barrier(0);

    // ---- x to f16 in LDS: the row's largest magnitude over the 16 lanes of its
    // DPP row, the power of two that puts it in [2^14, 2^15), the factor that undoes
    // it into facs[r]; groups in the fragment order 0 2 1 3 4 6 5 7, 16-byte group g
    // of row r at slot g ^ r of the chunk's row (the reads below are conflict-free).
    // Asm stores: the compiler would otherwise wait for the direct loads first. ----
    {
        auto amax4 = [](float4 v) {
            return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        };
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < XC; ++i) mx = fmaxf(mx, fmaxf(amax4(xv[i][0]), amax4(xv[i][1])));
        mx = fmaxf(mx, dpp_mov<0xB1>(mx));   // quad_perm [1,0,3,2]
        mx = fmaxf(mx, dpp_mov<0x4E>(mx));   // quad_perm [2,3,0,1]
        mx = fmaxf(mx, dpp_mov<0x141>(mx));  // row_half_mirror
        mx = fmaxf(mx, dpp_mov<0x140>(mx));  // row_mirror: the 16-lane row's max
        int e = 0;
        const bool ok = mx > 0.0f && mx <= 3.402823466e38f;
        if (ok) (void)frexpf(mx, &e);
        e = e < -111 ? -111 : e;
        const float sc = ok ? ldexpf(1.0f, 15 - e) : 1.0f;
        if (xg == 0) {
            const float f = ok ? ldexpf(1.0f, e - 15) : 1.0f;
            asm volatile("ds_write_b32 %0, %1" ::"v"((uint32_t)(uintptr_t)(facs + xr)), "v"(f));
        }
        // every chunk position is written (zeros past the slice): no divergent loop
#pragma unroll
        for (int i = 0; i < XC; ++i) {
            const float4 a = xv[i][0], b = xv[i][1];
            const lds_u32x4 v = {pk_f16(a.x * sc, a.z * sc), pk_f16(a.y * sc, a.w * sc),
                                 pk_f16(b.x * sc, b.z * sc), pk_f16(b.y * sc, b.w * sc)};
            const uint32_t addr = (uint32_t)(uintptr_t)xarea +
                                  (uint32_t)(i * kXinMaxM * kXinRowBytes + xr * kXinRowBytes +
                                             16 * (xg ^ xr));
            asm volatile("ds_write_b128 %0, %1" ::"v"(addr), "v"(v));
        }
    }
    if (zero_tile) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the zeros have landed
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    unsigned* const flag = sync + (size_t)rg * 3 * kSyncStride;
    if (zero_tile && tid == 0)
        __hip_atomic_store(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;

    // LDS offsets: x of token row min(col, 15) (tokens 16 .. 31 of the MFMA tile are
    // padding whose outputs are never stored), payloads as decode_kernel
    const int xrow = min(col, kXinMaxM - 1);
    uint32_t xo[8];
#pragma unroll
    for (int hp = 0; hp < 2; ++hp)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = 2 * hp + q / 2;
            const int g = Q4 ? 8 * hp + 4 * h + q : 4 * i + 2 * h + (q & 1);
            xo[4 * hp + q] = (uint32_t)(xrow * kXinRowBytes + 16 * (g ^ xrow));
        }
    uint32_t po[4];
    const int prow = 32 * wv + col;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int piece = Q4 ? (2 * (i & 1) + h) : 2 * i + h;
        po[i] = (uint32_t)(prow * 4 * QB + 16 * (piece ^ swz(col)));
    }
    const uint32_t ring0 = (uint32_t)(uintptr_t)ring;
    const uint32_t x0 = (uint32_t)(uintptr_t)xarea;
    const uint32_t srow = (uint32_t)(uintptr_t)scl + (uint32_t)(wv * 2048 + col * 64);
    const uint32_t hrow = (uint32_t)(uintptr_t)hdr + (uint32_t)(wv * 1024 + col * 32);

    auto compute = [&](int j) {
        const uint32_t st = ring0 + (uint32_t)((j % D) * ST::P);
        const uint32_t xs = x0 + (uint32_t)(j * kXinMaxM * kXinRowBytes);
        const int kb0 = 4 * (c0 + j);
        const uint32_t sa = srow + 8 * ((j + col) & 7);
        float gd = 0.0f, gm = 0.0f;
        if constexpr (K4 || K5 || K6) {
            uint32_t hd;
            asm volatile("ds_read_b32 %0, %1\n s_waitcnt lgkmcnt(0)"
                         : "=&v"(hd)
                         : "v"(hrow + 4u * (uint32_t)(((c0 + j) >> 1) - (c0 >> 1))));
            gd = __half2float(__ushort_as_half((uint16_t)hd)) * wscale;
            gm = __half2float(__ushort_as_half((uint16_t)(hd >> 16))) * wscale;
        }
#pragma unroll
        for (int hp = 0; hp < 2; ++hp) {
            lds_u32x4 xa[1][4];
            u32x4 pw[2];
            lds_u32x2 scp;
            read_half<Q4, 1>(xa, pw, scp, xs + xo[4 * hp], xs + xo[4 * hp + 1], xs + xo[4 * hp + 2],
                             xs + xo[4 * hp + 3], st + po[Q4 ? hp : 2 * hp],
                             st + po[Q4 ? hp : 2 * hp + 1], sa);
            if constexpr (Q4) {
                const uint16_t sb = (uint16_t)(scp[hp] >> (16 * h));
                const bool ok = kb0 + 2 * hp + h < KB;
                f16x8 b[4];
                if constexpr (K4) {
                    const float sv = ok ? gd * (float)(sb & 0xFFu) : 0.0f;
                    const float ov = ok ? gm * (float)(sb >> 8) : 0.0f;
                    const _Float16 s1 = (_Float16)sv, s16 = (_Float16)(sv * 0.0625f),
                                   o1 = (_Float16)ov;
                    const f16x2 sh = {s1, s1}, sh16 = {s16, s16}, oh = {o1, o1};
                    dequant_q4k(pw[0], sh, sh16, oh, b);
                } else {
                    const float dv = ok ? __half2float(__ushort_as_half(sb)) * wscale : 0.0f;
                    const _Float16 d = (_Float16)dv, d16 = (_Float16)(dv * 0.0625f);
                    const f16x2 dh = {d, d}, dh16 = {d16, d16};
                    dequant_q4(pw[0], dh, dh16, b);
                }
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, xa[0][q]),
                                                                 b[q], acc, 0, 0, 0);
            } else {
#pragma unroll
                for (int bi = 0; bi < 2; ++bi) {
                    const uint16_t sb = (uint16_t)(scp[hp] >> (16 * bi));
                    const bool ok = kb0 + 2 * hp + bi < KB;
                    f16x8 b0, b1;
                    if constexpr (K5) {
                        // sb = sc | m << 8: s = d sc 2^-E, o = dmin m 2^-E, each once to f16
                        const _Float16 s1 = (_Float16)(ok ? gd * (float)(sb & 0xFFu) : 0.0f);
                        const _Float16 o1 = (_Float16)(ok ? gm * (float)(sb >> 8) : 0.0f);
                        const f16x2 sh = {s1, s1}, oh = {o1, o1};
                        dequant_q8m(pw[bi], sh, oh, b0, b1);
                    } else {
                        const float dv = !ok ? 0.0f
                                         : K6 ? gd * (float)(int8_t)(sb >> (8 * h))
                                              : __half2float(__ushort_as_half(sb)) * wscale;
                        const _Float16 d = (_Float16)dv;
                        const f16x2 dh = {d, d};
                        dequant_q8(pw[bi], dh, b0, b1);
                    }
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                        __builtin_bit_cast(f16x8, xa[0][2 * bi]), b0, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                        __builtin_bit_cast(f16x8, xa[0][2 * bi + 1]), b1, acc, 0, 0, 0);
                }
            }
        }
    };

    // Each wave reads only what its own direct loads wrote (its rows' payloads, scales
    // and headers; x is in LDS already), so its own load count is the only wait: no
    // barrier, and the waves do not wait for each other chunk by chunk.  The slot a
    // chunk's loads overwrite was last read by this wave's previous chunk, whose reads
    // completed before its MFMAs.
    for (int j = 0; j < nch; ++j) {
        wait_chunks<ST::PD, D - 2>(min(D - 2, nch - 1 - j));
        if (j + D - 1 < nch) issue(j + D - 1);
        compute(j);
    }

    // ---- epilogue: acc[r] = C[token 8 (r / 4) + 4 h + r % 4][row row0 + col] ----
    // Tokens past m (and the tile's padding rows 16 .. 31) are not stored.
    const int n = row0 + col;
    float fv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int t = 8 * (r / 4) + 4 * h + (r % 4);
        fv[r] = facs[min(t, kXinMaxM - 1)] * oscale;  // plain read: no direct load is in flight
    }
    auto each = [&](auto&& f) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int t = 8 * (r / 4) + 4 * h + (r % 4);
            if (t < M && n < N) f(y + (int64_t)t * N + n, acc[r] * fv[r]);
        }
    };
    if (S == 1) {
        each([&](float* dst, float v) { *dst = add ? *dst + v : v; });
    } else if (add) {
        each([&](float* dst, float v) { unsafeAtomicAdd(dst, v); });
    } else {
        // slice 0 zeroed the tile and raised the flag after its prologue: the wait is
        // normally over at the first look.  A wait that gives up (which needs slice 0
        // not to run, and the host launches only grids that are resident at once) adds
        // NaN, so that the result is visibly wrong rather than silently so.
        if (tid == 0) {
            unsigned seen = 0;
            for (int it = 0; it < kSyncPoll && !seen; ++it) {
                seen = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (!seen) __builtin_amdgcn_s_sleep(2);
            }
            facs[32] = seen ? 0.0f : __builtin_nanf("");
        }
        __syncthreads();
        const float give_up = facs[32];
        each([&](float* dst, float v) { unsafeAtomicAdd(dst, v + give_up); });
        if (tid == 0 && __hip_atomic_fetch_add(flag + kSyncStride, 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT) == (unsigned)S - 1) {
            // every slice of this row group is past the flag: reset for the next launch
            __hip_atomic_store(flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(flag + kSyncStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int QT, int XC>
hipError_t launch_x(const QWeight& w, const float* x, int64_t m, float* y, int S, hipStream_t s,
                    int add, unsigned* sync) {
    using ST = XinStage<QT, XC>;
    static const bool attr = hipFuncSetAttribute((const void*)decode_x_kernel<QT, XC>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 ST::LDS) == hipSuccess;
    if (!attr) return hipErrorInvalidValue;
    const float wscale = ldexpf(1.0f, -w.f16_exp), oscale = ldexpf(1.0f, w.f16_exp);
    const int groups = (int)((w.n + DROWS - 1) / DROWS);
    decode_x_kernel<QT, XC><<<groups * S, 256, ST::LDS, s>>>(w.base, w.row_bytes, x, y, (int)m,
                                                         (int)w.n, (int)w.kb, S, wscale, oscale,
                                                         add, sync);
    return hipGetLastError();
}

template <int QT, int MT2>
hipError_t launch_mt(const QWeight& w, const _Float16* xh, const float* rf, int64_t m, float* y,
                     int S, hipStream_t s, int add) {
    using ST = Stage<QT, MT2>;
    static const bool attr = hipFuncSetAttribute((const void*)decode_kernel<QT, MT2>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 ST::LDS) == hipSuccess;
    if (!attr) return hipErrorInvalidValue;
    const float wscale = ldexpf(1.0f, -w.f16_exp), oscale = ldexpf(1.0f, w.f16_exp);
    const int groups = (int)((w.n + DROWS - 1) / DROWS);
    decode_kernel<QT, MT2><<<groups * S, 256, ST::LDS, s>>>(
        w.base, w.row_bytes, xh, rf, y, (int)m, (int)w.n, (int)w.kb, S, wscale, oscale, add);
    return hipGetLastError();
}

// k split S: the fewest slices of at most kMaxSliceChunks chunks, then more
// while the workgroups still fit the CUs at once (lds_bytes each).
int choose_split(const QWeight& w, int lds_bytes, bool wide) {
    const int64_t groups = (w.n + DROWS - 1) / DROWS;
    const int64_t chunks = (w.kb + 3) / 4;
    const int64_t per_cu = std::max(1, device_info().max_lds_cu / lds_bytes);
    const int64_t slots = (int64_t)device_info().cu_count * per_cu;
    int64_t S = (chunks + kMaxSliceChunks - 1) / kMaxSliceChunks;
    const int64_t cap = std::min<int64_t>(chunks, wide ? kMaxSplit2 : kMaxSplit1);
    while (S < cap && groups * (S + 1) <= slots) ++S;
    return (int)S;
}

// act[m, I] = silu(g) * u from gu[m, 2 I] (g = columns 0 .. I - 1, u = I .. 2 I - 1);
// candle's silu, v / (1 + e^-v).
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ gu, int64_t m,
                                                     int64_t I, float* __restrict__ act) {
    const int64_t total = m * I;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / I, c = i - r * I;
        const float g = gu[r * 2 * I + c], u = gu[r * 2 * I + I + c];
        act[i] = g / (1.0f + expf(-g)) * u;
    }
}

}  // namespace

// x[m, k] -> f16 rows in the fragment order (each aligned 8 as 0 2 1 3 4 6 5 7),
// each row scaled by its power of two (f16_row_scale; the factor to undo it in
// rs[row]).  One workgroup per row (64 .. 1024 threads, two groups of 8 a thread where the row
// allows), one HBM read: a thread keeps its first two groups in registers (rows up
// to 16384 elements); a longer row's further groups are read again for the
// conversion.
__global__ __launch_bounds__(1024) void xrows_kernel(const float* __restrict__ x, int64_t k,
                                                     uint4* __restrict__ xh,
                                                     float* __restrict__ rs) {
    __shared__ float red[16];
    const int64_t r = blockIdx.x, g8 = k / 8;
    const int t = threadIdx.x, nt = blockDim.x;
    const float4* xr = reinterpret_cast<const float4*>(x + r * k);
    auto amax = [](float4 v) {
        return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    };
    float4 a[2], b[2];
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int64_t i = t + nt * j;
        a[j] = b[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (i < g8) {
            a[j] = xr[2 * i];
            b[j] = xr[2 * i + 1];
        }
        mx = fmaxf(mx, fmaxf(amax(a[j]), amax(b[j])));
    }
    for (int64_t i = t + 2 * nt; i < g8; i += nt)
        mx = fmaxf(mx, fmaxf(amax(xr[2 * i]), amax(xr[2 * i + 1])));
    mx = wave_max(mx);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = 0.0f;
    for (int w = 0; w < nt / 64; ++w) mx = fmaxf(mx, red[w]);
    const float sc = f16_row_scale(mx, rs + r);
    uint4* xo = xh + r * g8;
    auto put = [&](int64_t i, float4 p, float4 q) {
        xo[i] = make_uint4(pk_f16(p.x * sc, p.z * sc), pk_f16(p.y * sc, p.w * sc),
                           pk_f16(q.x * sc, q.z * sc), pk_f16(q.y * sc, q.w * sc));
    };
#pragma unroll
    for (int j = 0; j < 2; ++j)
        if (t + nt * j < g8) put(t + nt * j, a[j], b[j]);
    for (int64_t i = t + 2 * nt; i < g8; i += nt) put(i, xr[2 * i], xr[2 * i + 1]);
}

// One workgroup per row r of x: the row's layer norm (two passes for the mean and
// the mean squared deviation, as ops_fn::layer_norm computes them), then each group
// of 8 normalized values rounded to f16 in the fragment order 0 2 1 3 4 6 5 7, and
// y's row r zeroed over ny columns.  The f16 values are scaled by powers of two as x
// is on the path without the norm: per row (rs != nullptr: the prefill operand, as
// xrows_kernel) or per k slice of the row (rf != nullptr: the S slices of the
// batched-decode split, factors at rf[s * 64 + r], as xprep_kernel).
// One HBM read: a thread holds groups t and t + nt of x, gamma and beta in registers
// across the passes (rows up to 16 nt elements); a longer row's further groups are
// read again in each pass.  Grid (m, 1 + Z): blockIdx.y == 0 normalizes row r, the
// Z others zero parts of y's row r.
__global__ __launch_bounds__(1024) void norm_convert_kernel(const float* __restrict__ x, int64_t k,
                                                           NormArgs norm, uint4* __restrict__ out,
                                                           float* __restrict__ y, int64_t ny,
                                                           float* __restrict__ rs, int S,
                                                           float* __restrict__ rf) {
    __shared__ float red[16];
    __shared__ unsigned smax[kMaxSplitSlices];  // per-slice max |v| as f32 bits (>= 0)
    __shared__ float ssc[kMaxSplitSlices];
    const int64_t r = blockIdx.x, g8 = k / 8;
    const int t = threadIdx.x, nt = blockDim.x, lane = t & 63, wv = t >> 6;
    if (blockIdx.y > 0) {  // (uniform) zero y's row r over column range blockIdx.y - 1 of Z
        const int64_t Z = gridDim.y - 1, z = blockIdx.y - 1;
        const int64_t c0 = ny * z / Z, c1 = ny * (z + 1) / Z;
        float* yr = y + r * ny;
        for (int64_t i = c0 + t; i < c1; i += nt) yr[i] = 0.0f;
        return;
    }
    const float4* xr = reinterpret_cast<const float4*>(x + r * k);
    const float4* g4 = reinterpret_cast<const float4*>(norm.gamma);
    const float4* b4 = reinterpret_cast<const float4*>(norm.beta);
    auto ld8 = [](const float4* p, int64_t i) {
        const float4 a = p[2 * i], b = p[2 * i + 1];
        return f32x8{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    };
    auto hsum = [](f32x8 v) {
        return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    };
    auto amax = [](f32x8 v) {
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[e]));
        return m;
    };
    auto block_sum = [&](float v) {
        v = wave_sum(v);
        if (lane == 0) red[wv] = v;
        __syncthreads();
        float sum = 0.0f;
        for (int w = 0; w < nt / 64; ++w) sum += red[w];
        __syncthreads();
        return sum;
    };
    const bool l0 = t < g8, l1 = t + nt < g8;
    const f32x8 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    f32x8 x0 = zero, x1 = zero, ga0 = zero, ga1 = zero, be0 = zero, be1 = zero;
    if (l0) {
        x0 = ld8(xr, t);
        ga0 = ld8(g4, t);
        if (b4) be0 = ld8(b4, t);
    }
    if (l1) {
        x1 = ld8(xr, t + nt);
        ga1 = ld8(g4, t + nt);
        if (b4) be1 = ld8(b4, t + nt);
    }
    float acc = hsum(x0) + hsum(x1);
    for (int64_t i = t + 2 * nt; i < g8; i += nt) acc += hsum(ld8(xr, i));
    const float mean = block_sum(acc) / (float)k;
    auto dev2 = [&](f32x8 v) {
        const f32x8 d = v - mean;
        return hsum(d * d);
    };
    acc = (l0 ? dev2(x0) : 0.0f) + (l1 ? dev2(x1) : 0.0f);
    for (int64_t i = t + 2 * nt; i < g8; i += nt) acc += dev2(ld8(xr, i));
    const float sd = sqrtf(block_sum(acc) / (float)k + norm.eps);
    // the normalized elements of a group from its x, gamma and beta
    auto normed = [&](f32x8 v, f32x8 g, f32x8 b) { return (v - mean) / sd * g + b; };
    auto values = [&](int64_t i) {  // a group past the registers, read again
        return normed(ld8(xr, i), ld8(g4, i), b4 ? ld8(b4, i) : zero);
    };
    const f32x8 v0 = normed(x0, ga0, be0), v1 = normed(x1, ga1, be1);
    // the scale of group i: per row (sc) or per slice (ssc[slice of i])
    float sc = 1.0f;
    // 128-k chunks; slice s = chunks [s C / S, (s + 1) C / S), its first group sb[s]
    // (16 groups a chunk; sb[S] = 16 C).  The slice of group i: a float estimate of
    // floor(c S / C), then the largest s with sb[s] <= i (no 64-bit division per group)
    __shared__ int sb[kMaxSplitSlices + 1];
    const int64_t C = (k + 127) / 128;
    const float sfac = (float)S / (float)C;
    auto slice_of = [&](int64_t i) {
        int s = min(S - 1, (int)((float)(i >> 4) * sfac));
        while (s + 1 < S && sb[s + 1] <= i) ++s;
        while (s > 0 && sb[s] > i) --s;
        return s;
    };
    int s0 = 0, s1 = 0;  // the slices of groups t and t + nt
    if (rs || rf) {  // kernel arguments: every branch on them is uniform, barriers included
        if (rf) {
            for (int s = t; s < S; s += nt) smax[s] = 0u;
            for (int s = t; s <= S; s += nt) sb[s] = (int)((int64_t)s * C / S) * 16;
            __syncthreads();
            s0 = l0 ? slice_of(t) : 0;
            s1 = l1 ? slice_of(t + nt) : 0;
            if (l0) atomicMax(&smax[s0], __float_as_uint(amax(v0)));
            if (l1) atomicMax(&smax[s1], __float_as_uint(amax(v1)));
            for (int64_t i = t + 2 * nt; i < g8; i += nt)
                atomicMax(&smax[slice_of(i)], __float_as_uint(amax(values(i))));
            __syncthreads();
            for (int s = t; s < S; s += nt) {
                // the scale of f16_row_scale, one thread per slice (f16_row_scale
                // stores from thread 0 only)
                const float m = __uint_as_float(smax[s]);
                int e = 0;
                const bool ok = m > 0.0f && m <= 3.402823466e38f;
                if (ok) (void)frexpf(m, &e);
                e = e < -111 ? -111 : e;
                rf[(int64_t)s * 64 + r] = ok ? ldexpf(1.0f, e - 15) : 1.0f;
                ssc[s] = ok ? ldexpf(1.0f, 15 - e) : 1.0f;
            }
            __syncthreads();
        } else {
            float mx = fmaxf(l0 ? amax(v0) : 0.0f, l1 ? amax(v1) : 0.0f);
            for (int64_t i = t + 2 * nt; i < g8; i += nt) mx = fmaxf(mx, amax(values(i)));
            mx = wave_max(mx);
            if (lane == 0) red[wv] = mx;
            __syncthreads();
            mx = 0.0f;
            for (int w = 0; w < nt / 64; ++w) mx = fmaxf(mx, red[w]);
            sc = f16_row_scale(mx, rs + r);
        }
    }
    uint4* xo = out + r * g8;
    auto put = [&](int64_t i, f32x8 v, float f) {
        v *= f;
        xo[i] = make_uint4(pk_f16(v[0], v[2]), pk_f16(v[1], v[3]), pk_f16(v[4], v[6]),
                           pk_f16(v[5], v[7]));
    };
    if (l0) put(t, v0, rf ? ssc[s0] : sc);
    if (l1) put(t + nt, v1, rf ? ssc[s1] : sc);
    for (int64_t i = t + 2 * nt; i < g8; i += nt) put(i, values(i), rf ? ssc[slice_of(i)] : sc);
}

hipError_t launch_swiglu(const float* gu, int64_t m, int64_t I, float* act, hipStream_t s) {
    const int64_t total = m * I;
    const int grid = (int)std::min<int64_t>((total + 255) / 256, (int64_t)device_info().cu_count * 8);
    swiglu_kernel<<<std::max(grid, 1), 256, 0, s>>>(gu, m, I, act);
    return hipGetLastError();
}

hipError_t launch_norm_convert(const float* x, int64_t m, int64_t k, const NormArgs& norm,
                               void* out, float* y, int64_t ny, hipStream_t s, float* rs, int S,
                               float* rf) {
    if (m <= 0) return hipSuccess;
    if (rf && (S < 1 || S > kMaxSplitSlices)) return hipErrorInvalidValue;
    // two groups of 8 a thread, whole waves, 64 .. 1024 threads; y zeroed by further
    // workgroups, 2048 columns (8 KiB) each, at most 16 a row
    const int nt = (int)std::min<int64_t>(1024, std::max<int64_t>(64, (k / 16 + 63) / 64 * 64));
    const unsigned Z = ny > 0 ? (unsigned)std::min<int64_t>(16, (ny + 2047) / 2048) : 0;
    norm_convert_kernel<<<dim3((unsigned)m, 1 + Z), nt, 0, s>>>(
        x, k, norm, static_cast<uint4*>(out), y, ny, rs, S, rf);
    return hipGetLastError();
}

hipError_t launch_x_to_f16_rows(const float* x, int64_t m, int64_t k, void* out, float* rs,
                                hipStream_t s) {
    if (m <= 0) return hipSuccess;
    // two groups of 8 a thread, whole waves, 64 .. 1024 threads
    const int nt = (int)std::min<int64_t>(1024, std::max<int64_t>(64, (k / 16 + 63) / 64 * 64));
    xrows_kernel<<<(unsigned)m, nt, 0, s>>>(x, k, static_cast<uint4*>(out), rs);
    return hipGetLastError();
}

namespace {
// The k split of a batched-decode call of m rows on w (as the launch picks it).
int decode_split(const QWeight& w, int64_t m) {
    const bool q4 = w.qtype == UNILLM_QTYPE_Q4_0, k4 = w.qtype == UNILLM_QTYPE_Q4_K,
               k5 = w.qtype == UNILLM_QTYPE_Q5_K, k6 = w.qtype == UNILLM_QTYPE_Q6_K, wide = m > 32;
    const int lds = k4   ? (wide ? Stage<UNILLM_QTYPE_Q4_K, 2>::LDS : Stage<UNILLM_QTYPE_Q4_K, 1>::LDS)
                    : k5 ? (wide ? Stage<UNILLM_QTYPE_Q5_K, 2>::LDS : Stage<UNILLM_QTYPE_Q5_K, 1>::LDS)
                    : k6 ? (wide ? Stage<UNILLM_QTYPE_Q6_K, 2>::LDS : Stage<UNILLM_QTYPE_Q6_K, 1>::LDS)
                    : q4 ? (wide ? Stage<UNILLM_QTYPE_Q4_0, 2>::LDS : Stage<UNILLM_QTYPE_Q4_0, 1>::LDS)
                         : (wide ? Stage<UNILLM_QTYPE_Q8_0, 2>::LDS : Stage<UNILLM_QTYPE_Q8_0, 1>::LDS);
    return choose_split(w, lds, wide);
}
// The larger of the two LDS layouts (XC = 8); both fit two workgroups a CU.
int xin_lds(const QWeight& w) {
    switch (w.qtype) {
        case UNILLM_QTYPE_Q4_0: return XinStage<UNILLM_QTYPE_Q4_0, kMaxSliceChunks>::LDS;
        case UNILLM_QTYPE_Q8_0: return XinStage<UNILLM_QTYPE_Q8_0, kMaxSliceChunks>::LDS;
        case UNILLM_QTYPE_Q4_K: return XinStage<UNILLM_QTYPE_Q4_K, kMaxSliceChunks>::LDS;
        case UNILLM_QTYPE_Q5_K: return XinStage<UNILLM_QTYPE_Q5_K, kMaxSliceChunks>::LDS;
        default: return XinStage<UNILLM_QTYPE_Q6_K, kMaxSliceChunks>::LDS;
    }
}
// k split S of the one-launch kernel: the fewest slices of at most kMaxSliceChunks
// chunks, then more while slices keep at least 4 chunks and the grid still fits the
// device at once (a round count of workgroups a CU evens the tail), at most 16 (more
// partial sums of one output contend in the adds).
int xin_split(const QWeight& w) {
    const int64_t groups = (w.n + DROWS - 1) / DROWS, chunks = (w.kb + 3) / 4;
    const int64_t slots =
        (int64_t)device_info().cu_count * std::max(1, device_info().max_lds_cu / xin_lds(w));
    int64_t S = (chunks + kMaxSliceChunks - 1) / kMaxSliceChunks;
    while (S < 16 && chunks >= 4 * (S + 1) && groups * (S + 1) <= slots) ++S;
    return (int)S;
}
// The one-launch kernel takes m <= 16 without a fused layer norm (the norm needs
// the whole row's statistics: its conversion stays a launch of its own), and only
// where its whole grid fits on the device at once (a slice may wait for slice 0 of
// its row group), else the two launches (y zeroed by the first).
bool decode_one_launch(const QWeight& w, int64_t m, const NormArgs& norm) {
    if (m > kXinMaxM || norm.gamma) return false;
    const int64_t groups = (w.n + DROWS - 1) / DROWS;
    const int64_t per_cu = std::max(1, device_info().max_lds_cu / xin_lds(w));
    return groups * xin_split(w) <= (int64_t)device_info().cu_count * per_cu;
}
// x as f16 (m k 2 bytes, padded to 256), then the slice factors rf[S][64]
size_t decode_x_bytes(const QWeight& w, int64_t m) {
    return ((size_t)m * (size_t)w.k * 2 + 255) / 256 * 256;
}
}  // namespace

size_t decode_workspace_bytes(const QWeight& w, int64_t m, const NormArgs& norm) {
    if (decode_one_launch(w, m, norm)) return 0;
    return decode_x_bytes(w, m) + (size_t)decode_split(w, m) * 64 * sizeof(float);
}

size_t decode_sync_bytes(const QWeight& w) { return xin_sync_bytes((w.n + DROWS - 1) / DROWS); }

hipError_t launch_decode_mfma(const QWeight& w, const float* x, int64_t m, float* y,
                              hipStream_t s, int epi, const NormArgs& norm, void* ws,
                              void* sync_ws) {
    // 32-bit offsets: x in f16 elements, weight bytes
    if ((uint64_t)m * (uint64_t)w.k >= (1ull << 31) || !mfma_supports(w) || m > 64)
        return hipErrorInvalidValue;
    const bool q4 = w.qtype == UNILLM_QTYPE_Q4_0, k4 = w.qtype == UNILLM_QTYPE_Q4_K,
               k5 = w.qtype == UNILLM_QTYPE_Q5_K, k6 = w.qtype == UNILLM_QTYPE_Q6_K, wide = m > 32;
    hipError_t e = hipSuccess;
    if (decode_one_launch(w, m, norm)) {
        // x converted by the kernel itself; the stream's workspace holds the row groups'
        // arrival tickets (zeroed when allocated, reset by each launch)
        const int S = xin_split(w);
        const int add = epi == kEpiAdd;
        void* sy = sync_ws;
        if (!sy && (e = stream_workspace(s, decode_sync_bytes(w), &sy, kSyncSlot)) != hipSuccess)
            return e;
        unsigned* sync = static_cast<unsigned*>(sy);
        // slices of at most 4 chunks: the short x area and the deeper ring
        const bool short_slices = ((w.kb + 3) / 4 + S - 1) / S <= 4;
        if (k4)
            return short_slices ? launch_x<UNILLM_QTYPE_Q4_K, 4>(w, x, m, y, S, s, add, sync)
                                : launch_x<UNILLM_QTYPE_Q4_K, 8>(w, x, m, y, S, s, add, sync);
        if (k5)
            return short_slices ? launch_x<UNILLM_QTYPE_Q5_K, 4>(w, x, m, y, S, s, add, sync)
                                : launch_x<UNILLM_QTYPE_Q5_K, 8>(w, x, m, y, S, s, add, sync);
        if (k6)
            return short_slices ? launch_x<UNILLM_QTYPE_Q6_K, 4>(w, x, m, y, S, s, add, sync)
                                : launch_x<UNILLM_QTYPE_Q6_K, 8>(w, x, m, y, S, s, add, sync);
        if (q4)
            return short_slices ? launch_x<UNILLM_QTYPE_Q4_0, 4>(w, x, m, y, S, s, add, sync)
                                : launch_x<UNILLM_QTYPE_Q4_0, 8>(w, x, m, y, S, s, add, sync);
        return short_slices ? launch_x<UNILLM_QTYPE_Q8_0, 4>(w, x, m, y, S, s, add, sync)
                            : launch_x<UNILLM_QTYPE_Q8_0, 8>(w, x, m, y, S, s, add, sync);
    }
    const int S = decode_split(w, m);
    if (!ws && (e = stream_workspace(s, decode_workspace_bytes(w, m, norm), &ws)) != hipSuccess)
        return e;
    float* rf = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + decode_x_bytes(w, m));
    const int add = epi == kEpiAdd;
    const int64_t ny = S > 1 && !add ? w.n : 0;  // y columns to zero per row
    if (norm.gamma) {
        if ((e = launch_norm_convert(x, m, w.k, norm, ws, y, ny, s, nullptr, S, rf)) !=
            hipSuccess)
            return e;
    } else {
        xprep_kernel<<<(unsigned)(m * S), 128, 0, s>>>(x, w.k, S, static_cast<uint4*>(ws), rf, y,
                                                        ny);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    const _Float16* xh = static_cast<const _Float16*>(ws);
    if (k4)
        return wide ? launch_mt<UNILLM_QTYPE_Q4_K, 2>(w, xh, rf, m, y, S, s, add)
                    : launch_mt<UNILLM_QTYPE_Q4_K, 1>(w, xh, rf, m, y, S, s, add);
    if (k5)
        return wide ? launch_mt<UNILLM_QTYPE_Q5_K, 2>(w, xh, rf, m, y, S, s, add)
                    : launch_mt<UNILLM_QTYPE_Q5_K, 1>(w, xh, rf, m, y, S, s, add);
    if (k6)
        return wide ? launch_mt<UNILLM_QTYPE_Q6_K, 2>(w, xh, rf, m, y, S, s, add)
                    : launch_mt<UNILLM_QTYPE_Q6_K, 1>(w, xh, rf, m, y, S, s, add);
    if (!wide)
        return q4 ? launch_mt<UNILLM_QTYPE_Q4_0, 1>(w, xh, rf, m, y, S, s, add)
                  : launch_mt<UNILLM_QTYPE_Q8_0, 1>(w, xh, rf, m, y, S, s, add);
    return q4 ? launch_mt<UNILLM_QTYPE_Q4_0, 2>(w, xh, rf, m, y, S, s, add)
              : launch_mt<UNILLM_QTYPE_Q8_0, 2>(w, xh, rf, m, y, S, s, add);
}

}  // namespace unillm
