// mfma.hip -- dequant -> MFMA matmul for batched decode and prefill.
//
// y[m, n] = x[m, k] . dequant(W)[n, k]^T with fp32 accumulation on the gfx950
// matrix cores (v_mfma_f32_16x16x32_{f16,bf16}).  Per K tile of BK = 64:
//   - A: the x tile (BM x 64 f32) is read once per workgroup, rounded to the
//     element type and staged in LDS;
//   - B: the W tile (BN columns x 2 blocks) is read as packed blocks, each
//     weight dequantized to (q - 8) * d (Q4_0) or q * d (Q8_0) in fp32 --
//     exactly -- then rounded once to the element type and staged in LDS;
//   - each wave runs its (BM / WM) x (BN / WN) sub-tile as 16x16x32 MFMAs.
// Element type: f16 for decode (m <= 64; x and w rounded to 11 significant
// bits, ~3e-4 normwise vs the f64 oracle, inside the 1e-3 GEMV bound) and
// bf16 for prefill (as the prefill contract states; ~2e-3, bound 2e-2).
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <math.h>

#include <type_traits>

#include "internal.hpp"

namespace unillm {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma;
template <>
struct Mfma<_Float16> {
    typedef f16x8 vec;
    static __device__ __forceinline__ f32x4 run(vec a, vec b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Mfma<__bf16> {
    typedef bf16x8 vec;
    static __device__ __forceinline__ f32x4 run(vec a, vec b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

constexpr int BK = 64;        // k per tile (two blocks)
constexpr int LDK = BK + 8;   // padded LDS row (elements): breaks power-of-two strides

template <typename T, int QT, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(256) void mfma_kernel(const uint8_t* __restrict__ base, int64_t rb,
                                                   const float* __restrict__ x,
                                                   float* __restrict__ y, int M, int N,
                                                   int KB, float wscale, float oscale) {
    static_assert(WM * WN == 4, "4 waves");
    constexpr int TM = BM / WM / 16;  // 16x16 sub-tiles per wave along m
    constexpr int TN = BN / WN / 16;
    typedef typename Mfma<T>::vec vec;

    __shared__ __attribute__((aligned(16))) T As[BM * LDK];
    __shared__ __attribute__((aligned(16))) T Bs[BN * LDK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    const int wm = wv / WN;
    const int wn = wv % WN;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int64_t K = (int64_t)KB * QK;
    const int ktiles = (KB + 1) / 2;

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int kt = 0; kt < ktiles; ++kt) {
        // ---- A: BM x 64 f32 -> T (float4 units: BM * 16 per tile) ----
#pragma unroll
        for (int u = tid; u < BM * 16; u += 256) {
            const int r = u / 16;
            const int c4 = u % 16;
            const int kblk = kt * 2 + c4 / 8;
            float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m0 + r < M && kblk < KB)
                f = *reinterpret_cast<const float4*>(x + (int64_t)(m0 + r) * K +
                                                     (int64_t)kt * BK + c4 * 4);
            T* dst = As + r * LDK + c4 * 4;
            dst[0] = (T)f.x;
            dst[1] = (T)f.y;
            dst[2] = (T)f.z;
            dst[3] = (T)f.w;
        }
        // ---- B: BN columns x 2 blocks, dequantized, 8-byte payload units ----
        if constexpr (QT == UNILLM_QTYPE_Q4_0) {
            // unit = (column, block, half): 8 bytes = elements 8h..8h+7 and 16+8h..
#pragma unroll
            for (int u = tid; u < BN * 4; u += 256) {
                const int col = u / 4;
                const int b = (u % 4) / 2;
                const int h = u % 2;
                const int kblk = kt * 2 + b;
                T lo[8], hi[8];
                if (n0 + col < N && kblk < KB) {
                    const uint2 p = *reinterpret_cast<const uint2*>(
                        blk_payload<16>(base, rb, n0 + col, kblk) + 8 * h);
                    const float d =
                        __half2float(__ushort_as_half(*blk_scale<16>(base, rb, KB, n0 + col, kblk)));
                    const uint32_t w2[2] = {p.x, p.y};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const uint32_t byte = (w2[j / 4] >> (8 * (j % 4))) & 0xFFu;
                        // signed nibbles q - 8
                        lo[j] = (T)((float)(((int)(byte << 28)) >> 28) * d * wscale);
                        hi[j] = (T)((float)(((int)(byte << 24)) >> 28) * d * wscale);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 8; ++j) lo[j] = hi[j] = (T)0.0f;
                }
                T* dst = Bs + col * LDK + b * 32;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    dst[8 * h + j] = lo[j];
                    dst[16 + 8 * h + j] = hi[j];
                }
            }
        } else {
            // unit = (column, block, eighth-of-32... 8 bytes = 8 elements)
#pragma unroll
            for (int u = tid; u < BN * 8; u += 256) {
                const int col = u / 8;
                const int b = (u % 8) / 4;
                const int e = u % 4;
                const int kblk = kt * 2 + b;
                T v8[8];
                if (n0 + col < N && kblk < KB) {
                    const uint2 p = *reinterpret_cast<const uint2*>(
                        blk_payload<32>(base, rb, n0 + col, kblk) + 8 * e);
                    const float d =
                        __half2float(__ushort_as_half(*blk_scale<32>(base, rb, KB, n0 + col, kblk)));
                    const uint32_t w2[2] = {p.x, p.y};
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        v8[j] = (T)((float)(int8_t)(w2[j / 4] >> (8 * (j % 4))) * d * wscale);
                } else {
#pragma unroll
                    for (int j = 0; j < 8; ++j) v8[j] = (T)0.0f;
                }
                T* dst = Bs + col * LDK + b * 32 + 8 * e;
#pragma unroll
                for (int j = 0; j < 8; ++j) dst[j] = v8[j];
            }
        }
        __syncthreads();

        // ---- MFMA: lane (l % 16) picks the row / column, (l / 16) the 8-wide k group
        const int fr = lane % 16;
        const int fk = (lane / 16) * 8;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            vec a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                a[i] = *reinterpret_cast<const vec*>(As + (wm * TM * 16 + i * 16 + fr) * LDK + kk +
                                                     fk);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                b[j] = *reinterpret_cast<const vec*>(Bs + (wn * TN * 16 + j * 16 + fr) * LDK + kk +
                                                     fk);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = Mfma<T>::run(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }

    // ---- epilogue: lane holds C[4 * (l / 16) + e][l % 16] of each sub-tile
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * TN * 16 + j * 16 + lane % 16;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = m0 + wm * TM * 16 + i * 16 + 4 * (lane / 16) + e;
                if (row < M && col < N) y[(int64_t)row * N + col] = acc[i][j][e] * oscale;
            }
        }
}

// f16 has 5 exponent bits: the weight's exponent offset E (chosen at create)
// keeps every (q - 8) * d * 2^-E finite; the output is scaled back by 2^E.
// Both scalings are exact.  bf16 has f32's range and needs none.
template <typename T, int BM, int BN, int WM, int WN>
hipError_t launch_cfg(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t s) {
    dim3 grid((unsigned)((w.n + BN - 1) / BN), (unsigned)((m + BM - 1) / BM));
    const int E = std::is_same<T, _Float16>::value ? w.f16_exp : 0;
    const float wscale = ldexpf(1.0f, -E), oscale = ldexpf(1.0f, E);
    if (w.qtype == UNILLM_QTYPE_Q4_0)
        mfma_kernel<T, UNILLM_QTYPE_Q4_0, BM, BN, WM, WN><<<grid, 256, 0, s>>>(
            w.base, w.row_bytes, x, y, (int)m, (int)w.n, (int)w.kb, wscale, oscale);
    else
        mfma_kernel<T, UNILLM_QTYPE_Q8_0, BM, BN, WM, WN><<<grid, 256, 0, s>>>(
            w.base, w.row_bytes, x, y, (int)m, (int)w.n, (int)w.kb, wscale, oscale);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_mfma(const QWeight& w, const float* x, int64_t m, float* y,
                              hipStream_t s) {
    if (m <= 16) return launch_cfg<_Float16, 16, 64, 1, 4>(w, x, m, y, s);
    return launch_cfg<_Float16, 64, 64, 2, 2>(w, x, m, y, s);
}


}  // namespace unillm
