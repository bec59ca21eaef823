// gemv.hip -- fused dequant + GEMV for decode (m <= 4).
//
// What it computes: y[m, n] = sum_k x[m, k] * dequant(W)[n, k], the decode
// step of QMatMul::forward (crates/runtime/src/models_v2/llama.rs:1188) for
// one to four tokens.  Bound: HBM -- each weight byte is read once; the
// arithmetic intensity is ~3.6 flop/B per token (Q4_0).
//
// Arithmetic.  Each 32-element block of x is written as two signed int8
// digits over a per-block power-of-two scale s, max|x| / 127 < s <= 2 max|x| / 127:
//     x[j] ~= s * (d0[j] + d1[j] / 254),  d0 = rint(x/s), d1 = rint((x/s - d0) * 254)
// (|error| <= s / 508 <= max|x| / 32258 per element; x / s is exact, so
// scaling x by a power of two scales y exactly).  The weight codes are exact
// small integers, so each block's dot products are exact int32 sums computed
// with v_dot4_i32_i8 (four products per instruction, ~1 VALU op per weight):
//     Q4_0: sum_j (q_j - 8) x_j = s * ((D0 - 8 S0) + (D1 - 8 S1) / 254),
//     D_i = sum_j q_j d_i[j], S_i = sum_j d_i[j]  (the -8 S_i seeds the sum);
//     Q8_0: the same with signed codes and no offset.
// Block results are scaled by d_w * s and summed in fp32.  Normwise error vs
// the f64 oracle is ~3e-5 (bound 1e-3).
//
// Mapping (MI355X, wave64).  One 1024-thread workgroup per CU (two of 512
// where a lane needs more than 128 VGPRs):
//   1. the workgroup turns x into digits in LDS, four threads per 32-block,
//      so each CU does this once -- before any weight load, because
//      instructions issue in order and weight loads that fill the memory
//      pipeline would hold back everything behind them;
//   2. every wave then requests its first two chunks of weights at once;
//   3. wave w owns rows w, w + W, w + 2W, ... (so the rows requested at one
//      moment form one contiguous stretch of the matrix) and walks them in
//      chunks of R rows (lane l owns blocks l, l + 64, ... of every row),
//      two chunks at a time; a wave-wide 128-bit load reads 1 KiB of
//      contiguous Q4_0 payload.  Every load is branch-free (indices are
//      clamped, validity is applied through the scale), so the in-order
//      memory counter lets the x digits be built while the weights stream.  Row partials are reduced with DPP rotations and two
//      cross-row shuffles.
#include <hip/hip_fp16.h>

#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

#include "internal.hpp"

namespace unillm {
namespace {

constexpr int kXWords = 20;             // LDS dwords per x block (19 used; conflict-free)
constexpr float kRound = 12582912.0f;   // 1.5 * 2^23: t + kRound rounds t to an integer

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

// Low bytes of four registers -> one dword (v_perm_b32 selects bytes; 0x0C = zero).
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t a0, uint32_t a1, uint32_t a2,
                                                   uint32_t a3) {
    return __builtin_amdgcn_perm(a1, a0, 0x0C0C0400u) | __builtin_amdgcn_perm(a3, a2, 0x04000C0Cu);
}

// ---- x digits -----------------------------------------------------------------------------
// LDS record of one 32-element x block, in the byte order of the weight payload:
// dwords 0-7 digit 0 of elements 4t..4t+3, 8-15 digit 1, 16 / 17 the seeds
// c0 / c1 (-8 S_i for Q4_0, 0 for Q8_0), 18 the scale s.  (For Q4_0, payload
// dword t meets digit dwords t (low nibbles) and 4 + t (high nibbles).)
//
// One thread builds one quarter (8 elements) of a block; the four threads of a
// block are one DPP quad, so the block max and digit sums are quad reductions.
// The math runs on every thread and only the stores are conditional, so the
// compiler keeps the x loads where they are issued (ahead of the weights).
template <int QT>
__device__ __forceinline__ void prep_quarter(const float (&v)[8], int u, bool store,
                                             uint32_t* __restrict__ dst) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, dpp_f32<0xB1>(amax));
    amax = fmaxf(amax, dpp_f32<0x4E>(amax));
    // s = 2^e with amax / 127 < s: frexp gives amax / 127 = f * 2^e, f in [0.5, 1)
    int e = 0;
    (void)frexpf(amax * (1.0f / 127.0f), &e);
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
    const uint32_t p00 = pack_low_bytes(b0[0], b0[1], b0[2], b0[3]);
    const uint32_t p01 = pack_low_bytes(b0[4], b0[5], b0[6], b0[7]);
    const uint32_t p10 = pack_low_bytes(b1[0], b1[1], b1[2], b1[3]);
    const uint32_t p11 = pack_low_bytes(b1[4], b1[5], b1[6], b1[7]);
    int s0 = sdot4((int)p00, 0x01010101, sdot4((int)p01, 0x01010101, 0));
    int s1 = sdot4((int)p10, 0x01010101, sdot4((int)p11, 0x01010101, 0));
    s0 += dpp_i32<0xB1>(s0);
    s0 += dpp_i32<0x4E>(s0);
    s1 += dpp_i32<0xB1>(s1);
    s1 += dpp_i32<0x4E>(s1);
    if (!store) return;
    dst[2 * u] = p00;
    dst[2 * u + 1] = p01;
    dst[8 + 2 * u] = p10;
    dst[8 + 2 * u + 1] = p11;
    if (u == 0) {
        dst[16] = (uint32_t)(QT == UNILLM_QTYPE_Q4_0 ? -8 * s0 : 0);
        dst[17] = (uint32_t)(QT == UNILLM_QTYPE_Q4_0 ? -8 * s1 : 0);
        dst[18] = __float_as_uint(amax > 0.0f ? ldexpf(1.0f, e) : 0.0f);
    }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct XBlock {
    u32x4 d0[2], d1[2];  // 8 dwords each
    int c0, c1;
    float s;
};

__device__ __forceinline__ void load_xblock(const uint32_t* __restrict__ src, XBlock& o) {
    const u32x4* p = reinterpret_cast<const u32x4*>(src);
    o.d0[0] = p[0];
    o.d0[1] = p[1];
    o.d1[0] = p[2];
    o.d1[1] = p[3];
    const u32x4 e = p[4];
    o.c0 = (int)e.x;
    o.c1 = (int)e.y;
    o.s = __uint_as_float(e.z);
}

// ---- weights --------------------------------------------------------------------------------
template <int QT>
struct Payload {
    static constexpr int V = QT == UNILLM_QTYPE_Q4_0 ? 1 : 2;  // 128-bit loads per block
};

template <int QT, int NB, int R>
struct Chunk {
    u32x4 q[R][NB][Payload<QT>::V];
    uint16_t d[R][NB];
};

// Branch-free: indices are clamped into the matrix and validity is applied
// later through the scale (d = 0), so no divergent branch sits around a load.
// (A load under a divergent branch whose other side writes the same register
// makes the compiler wait for the load at the join, serialising the loads.)
// Rows of a wave: w, w + W, w + 2W, ... (W = waves), so the rows the whole
// grid requests at one moment form one contiguous stretch of the matrix.
// Chunk j0 holds the wave's rows j0 .. j0 + R - 1; rows past the wave's last
// are clamped to that last row (an address the wave reads anyway).
template <int QT, int NB, int R>
__device__ __forceinline__ void load_chunk(Chunk<QT, NB, R>& c, const uint8_t* __restrict__ base,
                                           int64_t rb, int w, int W, int j0, int jlast, int KB,
                                           const int* bidx) {
    constexpr int V = Payload<QT>::V;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = w + min(j0 + r, jlast) * W;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            // streamed once: non-temporal, so it does not evict x from the caches
            const u32x4* p =
                reinterpret_cast<const u32x4*>(blk_payload<16 * V>(base, rb, row, bidx[i]));
#pragma unroll
            for (int v = 0; v < V; ++v) c.q[r][i][v] = __builtin_nontemporal_load(p + v);
            c.d[r][i] = *blk_scale<16 * V>(base, rb, KB, row, bidx[i]);
        }
    }
}

template <int QT, int M, int NB, int R>
__device__ __forceinline__ void compute_chunk(const Chunk<QT, NB, R>& c, const XBlock (&xbs)[M][NB],
                                              const bool* bval, float* __restrict__ y, int w,
                                              int W, int j0, int jcount, int N, int lane,
                                              int m_real) {
    float part[M][R];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) part[m][r] = 0.0f;
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const XBlock& xb = xbs[m][i];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                int a0 = xb.c0, a1 = xb.c1;
                if constexpr (QT == UNILLM_QTYPE_Q4_0) {
                    const u32x4 w4 = c.q[r][i][0];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int lo = (int)(w4[t] & 0x0F0F0F0Fu);
                        const int hi = (int)((w4[t] >> 4) & 0x0F0F0F0Fu);
                        a0 = sdot4(lo, (int)xb.d0[0][t], a0);
                        a0 = sdot4(hi, (int)xb.d0[1][t], a0);
                        a1 = sdot4(lo, (int)xb.d1[0][t], a1);
                        a1 = sdot4(hi, (int)xb.d1[1][t], a1);
                    }
                } else {
#pragma unroll
                    for (int v = 0; v < 2; ++v) {
                        const u32x4 w4 = c.q[r][i][v];
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            a0 = sdot4((int)w4[t], (int)xb.d0[v][t], a0);
                            a1 = sdot4((int)w4[t], (int)xb.d1[v][t], a1);
                        }
                    }
                }
                // lanes past the row end (clamped duplicates) contribute nothing
                const float dw = bval[i] ? __half2float(__ushort_as_half(c.d[r][i])) : 0.0f;
                const float blk = fmaf((float)a1, 1.0f / 254.0f, (float)a0);
                part[m][r] = fmaf(dw * xb.s, blk, part[m][r]);
            }
        }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) part[m][r] = wave_sum(part[m][r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (j0 + r < jcount)
#pragma unroll
                for (int m = 0; m < M; ++m)
                    if (m < m_real) y[(int64_t)m * N + w + (j0 + r) * W] = part[m][r];
    }
}

// Workgroup size: 1024 threads (one workgroup per CU, 128 VGPRs per lane)
// when a chunk and one x block fit that budget, else 512 (two per CU, 256).
template <int QT, int M, int NB>
constexpr int gemv_threads() {
    return M * NB * Payload<QT>::V <= 2 ? 1024 : 512;
}

// m_real <= M rows of x are used; rows m >= m_real repeat row m_real - 1 and
// are not written.  Dynamic LDS: M * KB * kXWords dwords of x digits.
// M * KB * 4 <= 2048, so a thread builds at most 2048 / THREADS quarter-blocks.
template <int QT, int M, int NB, int R, int THREADS>
__global__ __launch_bounds__(THREADS) void gemv_kernel(const uint8_t* __restrict__ base,
                                                       int64_t rb,
                                                       const float* __restrict__ x,
                                                       float* __restrict__ y, int N, int KB,
                                                       int m_real) {
    constexpr int WAVES = THREADS / 64;
    constexpr int PASSES = 2048 / THREADS;
    extern __shared__ uint32_t xlds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * WAVES + (threadIdx.x >> 6));
    const int waves = gridDim.x * WAVES;
    const int64_t K = (int64_t)KB * QK;
    // this wave's rows: wave, wave + waves, ... (counts differ by at most one);
    // wave-uniform, so every branch on them is a scalar branch
    const int jcount = wave < N ? (N - 1 - wave) / waves + 1 : 0;
    const int jlast = max(jcount - 1, 0);
    const int wrow = min(wave, N - 1);  // a wave without rows reads row N - 1

    int bidx[NB];
    bool bval[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int b = i * 64 + lane;
        bval[i] = b < KB;
        bidx[i] = min(b, KB - 1);
    }

    // 1. x for the digits
    const int nq = M * KB * 4;
    float v[PASSES][8];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int q = threadIdx.x + p * THREADS;
        const int blk = min(q, nq - 1) >> 2;
        const int m = blk / KB;
        const float4* src = reinterpret_cast<const float4*>(
            x + (int64_t)min(m, m_real - 1) * K + (int64_t)(blk - m * KB) * QK) + 2 * (q & 3);
        float4 f0 = make_float4(0.f, 0.f, 0.f, 0.f), f1 = f0;
        if (q < nq) {  // only the quarters that exist are fetched
            f0 = src[0];
            f1 = src[1];
        }
        v[p][0] = f0.x; v[p][1] = f0.y; v[p][2] = f0.z; v[p][3] = f0.w;
        v[p][4] = f1.x; v[p][5] = f1.y; v[p][6] = f1.z; v[p][7] = f1.w;
    }
    // Unconditional (indices clamped into the matrix): a load under a branch
    // would make the waits that follow it conservative.
    // 2. x digits for all M * KB blocks, four threads per block (threads past
    //    nq compute on a clamped copy and store nothing; nq is a multiple of 4,
    //    so a DPP quad is either all real or all clamped).  This comes before
    //    the weight loads: instructions issue in order, and once the weight
    //    loads fill the memory pipeline, anything behind them waits until they
    //    are accepted -- the digits would then be late for every row.
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int q = threadIdx.x + p * THREADS;
        prep_quarter<QT>(v[p], q & 3, q < nq, xlds + (size_t)(min(q, nq - 1) >> 2) * kXWords);
    }
    __syncthreads();

    // 3. this lane's x digits, read once from LDS into registers for all rows
    //    (also ahead of the weight loads, for the same in-order reason)
    XBlock xb[M][NB];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < NB; ++i) load_xblock(xlds + ((size_t)m * KB + bidx[i]) * kXWords, xb[m][i]);
    __builtin_amdgcn_sched_barrier(0);  // keep the reads above the weight loads

    // 4. the weights: the first two chunks at once (unconditional, indices
    //    clamped: a load under a branch would make the waits that follow it
    //    conservative)
    Chunk<QT, NB, R> a, b;
    load_chunk<QT, NB, R>(a, base, rb, wrow, waves, 0, jlast, KB, bidx);
    load_chunk<QT, NB, R>(b, base, rb, wrow, waves, R, jlast, KB, bidx);

    // 5. the first two chunks, then (for ranges longer than 2R rows) two
    //    chunks per step
    compute_chunk<QT, M, NB, R>(a, xb, bval, y, wrow, waves, 0, jcount, N, lane, m_real);
    compute_chunk<QT, M, NB, R>(b, xb, bval, y, wrow, waves, R, jcount, N, lane, m_real);
    for (int j = 2 * R; j < jcount; j += 2 * R) {
        load_chunk<QT, NB, R>(a, base, rb, wrow, waves, j, jlast, KB, bidx);
        load_chunk<QT, NB, R>(b, base, rb, wrow, waves, j + R, jlast, KB, bidx);
        compute_chunk<QT, M, NB, R>(a, xb, bval, y, wrow, waves, j, jcount, N, lane, m_real);
        compute_chunk<QT, M, NB, R>(b, xb, bval, y, wrow, waves, j + R, jcount, N, lane, m_real);
    }
}

template <int QT, int M, int NB, int R>
hipError_t launch_r(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t st,
                    int waves) {
    constexpr int THREADS = gemv_threads<QT, M, NB>();
    constexpr int WAVES = THREADS / 64;
    const size_t lds = (size_t)M * w.kb * kXWords * sizeof(uint32_t);
    const int grid = (waves + WAVES - 1) / WAVES;
    gemv_kernel<QT, M, NB, R, THREADS><<<grid, THREADS, lds, st>>>(w.base, w.row_bytes, x, y,
                                                                  (int)w.n, (int)w.kb, (int)m);
    return hipGetLastError();
}

// Launch shape.  Every workgroup is resident at once (the occupancy the
// registers and LDS allow), each wave gets at least two rows, and the chunk
// size R (rows) is the smallest that lets the two chunks a wave requests up
// front cover its rows -- so no wave loads rows it does not own -- capped by
// the registers a chunk may take (at most 4 payload loads per lane).
template <int QT, int M, int NB>
hipError_t launch_nb(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t st) {
    constexpr int V = Payload<QT>::V;
    constexpr int RMAX = NB * V >= 4 ? 1 : 4 / (NB * V);
    constexpr int THREADS = gemv_threads<QT, M, NB>();
    constexpr int WAVES = THREADS / 64;
    int per_cu = 0;
    const size_t lds = (size_t)M * w.kb * kXWords * sizeof(uint32_t);
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &per_cu, gemv_kernel<QT, M, NB, RMAX, THREADS>, THREADS, lds);
    if (e != hipSuccess) return e;
    const int64_t resident = (int64_t)device_info().cu_count * std::max(per_cu, 1) * WAVES;
    const int64_t waves = std::max<int64_t>(1, std::min(resident, w.n / 2));
    const int64_t rows = (w.n + waves - 1) / waves;  // per wave, at most
    if (debug_launch())
        fprintf(stderr, "unillm gemv: n=%lld kb=%lld m=%lld threads=%d per_cu=%d waves=%lld rows=%lld\n",
                (long long)w.n, (long long)w.kb, (long long)m, THREADS, per_cu, (long long)waves,
                (long long)rows);
    if (RMAX >= 4 && rows > 4) return launch_r<QT, M, NB, RMAX>(w, x, m, y, st, (int)waves);
    if (RMAX >= 2 && rows > 2) return launch_r<QT, M, NB, (RMAX >= 2 ? 2 : 1)>(w, x, m, y, st, (int)waves);
    return launch_r<QT, M, NB, 1>(w, x, m, y, st, (int)waves);
}

template <int QT, int M>
hipError_t launch_m(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t st) {
    switch ((int)((w.kb + 63) / 64)) {
        case 1: return launch_nb<QT, M, 1>(w, x, m, y, st);
        case 2: return launch_nb<QT, M, 2>(w, x, m, y, st);
        case 3: if constexpr (M <= 2) return launch_nb<QT, M, 3>(w, x, m, y, st); break;
        case 4: if constexpr (M <= 2) return launch_nb<QT, M, 4>(w, x, m, y, st); break;
        case 5: if constexpr (M == 1 && QT == UNILLM_QTYPE_Q4_0) return launch_nb<QT, M, 5>(w, x, m, y, st); break;
        case 6: if constexpr (M == 1 && QT == UNILLM_QTYPE_Q4_0) return launch_nb<QT, M, 6>(w, x, m, y, st); break;
        case 7: if constexpr (M == 1 && QT == UNILLM_QTYPE_Q4_0) return launch_nb<QT, M, 7>(w, x, m, y, st); break;
        default: break;
    }
    return hipErrorInvalidValue;
}

}  // namespace

// Largest K (in blocks) the GEMV path takes at m rows, set by the registers
// two chunks of NB blocks per lane need (NB = ceil(KB / 64)): Q4_0 up to
// NB = 7 at one row (K = 14336), 4 at two, 2 at four; Q8_0 payloads are twice
// as wide, so it stops at NB = 4.  M * KB <= 512 also bounds the LDS (40 KiB).
int64_t gemv_max_kb(int64_t m, int qtype) {
    if (m <= 1) return qtype == UNILLM_QTYPE_Q8_0 ? 256 : 448;
    if (m <= 2) return 256;
    return 128;
}

hipError_t launch_gemv(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t s) {
    if (w.qtype == UNILLM_QTYPE_Q4_0) {
        if (m == 1) return launch_m<UNILLM_QTYPE_Q4_0, 1>(w, x, m, y, s);
        if (m == 2) return launch_m<UNILLM_QTYPE_Q4_0, 2>(w, x, m, y, s);
        return launch_m<UNILLM_QTYPE_Q4_0, 4>(w, x, m, y, s);
    }
    if (m == 1) return launch_m<UNILLM_QTYPE_Q8_0, 1>(w, x, m, y, s);
    if (m == 2) return launch_m<UNILLM_QTYPE_Q8_0, 2>(w, x, m, y, s);
    return launch_m<UNILLM_QTYPE_Q8_0, 4>(w, x, m, y, s);
}

}  // namespace unillm
