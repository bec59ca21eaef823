// gemv.hip -- fused dequant + GEMV for decode (m = 1, 2), fp32 VALU.
//
// What it computes: y[m, n] = sum_k x[m, k] * dequant(W)[n, k], the decode
// step of QMatMul::forward (crates/runtime/src/models_v2/llama.rs:1188) on one
// token (m = 1) or two.  Bound: HBM -- every weight byte is read exactly once
// and the arithmetic intensity is ~3.6 flop/B (Q4_0), far below the ridge.
//
// Mapping (MI355X, wave64):
//   - a wave owns a K-slice of at most 64 * NB blocks; lane l takes blocks
//     l, l + 64, ... of the slice, so one wave-wide 128-bit load reads 1 KiB of
//     contiguous Q4_0 payload (or half of that many Q8_0 blocks);
//   - the lane keeps its slice of x in registers for all rows it visits
//     (x[j] for the low nibbles, x[j + 16] / 16 for the high nibbles, so the
//     masked byte 16*q converts with one v_cvt_f32_ubyte), and -8 * sum(x) of
//     each block seeds the block accumulator, which folds the Q4_0 offset
//     (Q8_0: bytes are biased by 128 and -128 * sum(x) seeds it);
//   - R rows are loaded before any is used, so each wave has R * NB 128-bit
//     loads in flight; the per-row partials are reduced with DPP row
//     rotations plus two cross-row swizzles;
//   - when K needs S > 1 slices, the S waves of a workgroup share the rows
//     and combine their partials through LDS.
// Numerics: every product (q - 8) * x is formed exactly in an fp32 FMA; block
// sums are scaled by d in fp32.  Error vs the f64 oracle is ~1e-6 normwise.
#include <hip/hip_fp16.h>

#include "internal.hpp"

namespace unillm {
namespace {

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
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

template <int QT>
struct Payload;
template <>
struct Payload<UNILLM_QTYPE_Q4_0> {
    static constexpr int V = 1;  // uint4 loads per block
};
template <>
struct Payload<UNILLM_QTYPE_Q8_0> {
    static constexpr int V = 2;
};

template <int QT, int M, int NB, int R>
__global__ __launch_bounds__(512) void gemv_kernel(const uint8_t* __restrict__ qs,
                                                   const uint16_t* __restrict__ dsc,
                                                   const float* __restrict__ x,
                                                   float* __restrict__ y, int N, int KB, int S,
                                                   int SB, int G) {
    constexpr int V = Payload<QT>::V;
    constexpr int QB = 16 * V;
    __shared__ float red[8 * R * M];

    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int s = wv % S;
    const int g = wv / S;
    const int row0 = (blockIdx.x * G + g) * R;
    const int64_t K = (int64_t)KB * QK;

    int bidx[NB];
    bool bval[NB];
    const int slice_len = min(SB, KB - s * SB);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int lb = i * 64 + lane;
        bval[i] = lb < slice_len;
        bidx[i] = bval[i] ? s * SB + lb : 0;
    }

    // x slice in registers: xa[m][i][0..31], seed c[m][i]
    float xa[M][NB][QK];
    float c[M][NB];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            float sum = 0.0f;
            if (bval[i]) {
                const float4* xp = reinterpret_cast<const float4*>(x + m * K + (int64_t)bidx[i] * QK);
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    const float4 f = xp[v];
                    xa[m][i][4 * v + 0] = f.x;
                    xa[m][i][4 * v + 1] = f.y;
                    xa[m][i][4 * v + 2] = f.z;
                    xa[m][i][4 * v + 3] = f.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < QK; ++j) xa[m][i][j] = 0.0f;
            }
#pragma unroll
            for (int j = 0; j < QK; ++j) sum += xa[m][i][j];
            if constexpr (QT == UNILLM_QTYPE_Q4_0) {
                c[m][i] = -8.0f * sum;
#pragma unroll
                for (int j = 16; j < QK; ++j) xa[m][i][j] *= 0.0625f;  // exact
            } else {
                c[m][i] = -128.0f * sum;
            }
        }

    // issue every load of the R rows first
    uint4 q[R][NB][V];
    float dd[R][NB];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            if (row < N && bval[i]) {
                const int64_t blk = (int64_t)row * KB + bidx[i];
                const uint4* p = reinterpret_cast<const uint4*>(qs + blk * QB);
#pragma unroll
                for (int v = 0; v < V; ++v) q[r][i][v] = p[v];
                dd[r][i] = __half2float(__ushort_as_half(dsc[blk]));
            } else {
#pragma unroll
                for (int v = 0; v < V; ++v) q[r][i][v] = make_uint4(0, 0, 0, 0);
                dd[r][i] = 0.0f;
            }
        }
    }

    float part[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) part[m][r] = 0.0f;

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            float acc[M];
#pragma unroll
            for (int m = 0; m < M; ++m) acc[m] = c[m][i];
            if constexpr (QT == UNILLM_QTYPE_Q4_0) {
                const uint32_t w4[4] = {q[r][i][0].x, q[r][i][0].y, q[r][i][0].z, q[r][i][0].w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t lo = w4[t] & 0x0F0F0F0Fu;
                    const uint32_t hi = w4[t] & 0xF0F0F0F0u;
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const float fl = (float)((lo >> (8 * b)) & 0xFFu);
                        const float fh = (float)((hi >> (8 * b)) & 0xFFu);
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            acc[m] = fmaf(fl, xa[m][i][4 * t + b], acc[m]);
                            acc[m] = fmaf(fh, xa[m][i][16 + 4 * t + b], acc[m]);
                        }
                    }
                }
            } else {
#pragma unroll
                for (int v = 0; v < 2; ++v) {
                    const uint32_t w4[4] = {q[r][i][v].x, q[r][i][v].y, q[r][i][v].z,
                                            q[r][i][v].w};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const uint32_t u = w4[t] ^ 0x80808080u;  // q + 128 per byte
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const float f = (float)((u >> (8 * b)) & 0xFFu);
#pragma unroll
                            for (int m = 0; m < M; ++m)
                                acc[m] = fmaf(f, xa[m][i][16 * v + 4 * t + b], acc[m]);
                        }
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < M; ++m) part[m][r] = fmaf(dd[r][i], acc[m], part[m][r]);
        }

#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) part[m][r] = wave_sum(part[m][r]);

    if (S == 1) {
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < N)
#pragma unroll
                    for (int m = 0; m < M; ++m) y[(int64_t)m * N + row0 + r] = part[m][r];
        }
        return;
    }
    // S slices of one row group combine through LDS (uniform control flow:
    // every wave of the workgroup reaches the barrier exactly once).
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) red[(wv * R + r) * M + m] = part[m][r];
    }
    __syncthreads();
    if (s == 0 && lane < R * M) {
        const int r = lane / M;
        const int m = lane % M;
        float tot = 0.0f;
        for (int t = 0; t < S; ++t) tot += red[((g * S + t) * R + r) * M + m];
        if (row0 + r < N) y[(int64_t)m * N + row0 + r] = tot;
    }
}

constexpr int kRows = 4;  // rows in flight per wave

template <int QT, int M, int NB>
hipError_t launch_t(const QWeight& w, const float* x, float* y, hipStream_t st) {
    const int KB = (int)w.kb;
    const int S = (KB + 64 * NB - 1) / (64 * NB);
    const int SB = (KB + S - 1) / S;
    const int G = S >= 4 ? 1 : 4 / S;
    const int64_t rows_per_wg = (int64_t)G * kRows;
    const unsigned grid = (unsigned)((w.n + rows_per_wg - 1) / rows_per_wg);
    gemv_kernel<QT, M, NB, kRows><<<grid, 64 * S * G, 0, st>>>(w.qs, w.d, x, y, (int)w.n, KB, S,
                                                               SB, G);
    return hipGetLastError();
}

}  // namespace

// Largest K (in blocks) the GEMV path takes: 8 waves x 64 lanes x NB blocks.
int64_t gemv_max_kb(int64_t m) { return m == 1 ? 8 * 64 * 2 : 8 * 64; }

hipError_t launch_gemv(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t s) {
    if (w.qtype == UNILLM_QTYPE_Q4_0)
        return m == 1 ? launch_t<UNILLM_QTYPE_Q4_0, 1, 2>(w, x, y, s)
                      : launch_t<UNILLM_QTYPE_Q4_0, 2, 1>(w, x, y, s);
    return m == 1 ? launch_t<UNILLM_QTYPE_Q8_0, 1, 2>(w, x, y, s)
                  : launch_t<UNILLM_QTYPE_Q8_0, 2, 1>(w, x, y, s);
}

}  // namespace unillm
