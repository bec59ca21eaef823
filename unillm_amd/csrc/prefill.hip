// prefill.hip -- fused dequant + bf16 MFMA GEMM for prefill (m >= 65).
//
// y[m, n] = x[m, k] . dequant(W)[n, k]^T, the prefill call of QMatMul::forward
// (crates/runtime/src/models_v2/llama.rs:1188, 1329) with x f32 rounded to
// bf16 on the device, weights dequantized exactly ((q - 8) * d, or q * d for
// Q8_0, in fp32) and rounded once to bf16, fp32 accumulation on the gfx950
// matrix cores (v_mfma_f32_16x16x32_bf16).  Bound: MFMA (2 m n k flops over
// ~n k / 32 * 18 + 4 m k + 4 m n bytes).
//
// Tile per workgroup: BM rows of x (BM = 256 or 128) x 256 weight rows
// (output columns), k in steps of 64 (two blocks).  Four waves; wave w owns
// output columns [64 w, 64 w + 64) for all BM rows: BM / 16 x 4 MFMA tiles,
// 4 fp32 accumulators each (256 per lane at BM = 256; one wave per SIMD).
//   A (x): BM x 64 f32 per step, loaded into registers one step ahead,
//     rounded to bf16 and written to a double-buffered LDS tile; every wave
//     reads all BM rows of it.
//   B (weights): no LDS.  Each wave's 64 columns are its own, so each lane
//     loads exactly the 8 payload bytes behind its MFMA B fragment (column
//     l % 16 of a 16-column tile, elements 8 (l / 16) .. +7 of a 32-block)
//     plus the block scale, one step ahead, and dequantizes them in
//     registers; nothing is dequantized twice within a workgroup.
// LDS traffic per CU per 32-wide k slice: reads 4 x BM x 32 x 2 B, writes
// BM x 32 x 2 B -- 80 B/clk at BM = 256 against ~128 B/clk available, with the
// MFMAs of the slice taking BM x 256 x 32 x 2 / 4096 flop/clk cycles.
//
// Workgroup -> tile: workgroups are dealt round-robin over the 8 XCDs, so
// workgroup b takes tile (b % 8) * (T / 8) + b / 8 (T tiles, padded to a
// multiple of 8): each XCD gets a contiguous run of tiles in row-major
// (m-tile, n-tile) order, i.e. mostly one m-tile, whose A rows then stay in
// that XCD's L2 while its CUs sweep the n-tiles.
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <algorithm>

#include "internal.hpp"

namespace unillm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int PBN = 256;         // output columns per workgroup
constexpr int PBK = 64;          // k per step (two blocks)
constexpr int PLD = PBK + 8;     // LDS row stride in bf16 (144 B): spreads rows over banks
#ifndef PREFILL_WAVES
#define PREFILL_WAVES 8
#endif
constexpr int kWaves = PREFILL_WAVES;  // waves per workgroup (8: two per SIMD)
#ifndef PREFILL_DEPTH
#define PREFILL_DEPTH 1
#endif
constexpr int kDepth = PREFILL_DEPTH;  // k steps of weight loads in flight

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    // round to nearest even; the pair in one dword, lo in the low half
    const __bf16 a = (__bf16)lo, b = (__bf16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// One lane's B fragment of one 32-block: 8 codes (4 per dword of `raw`, in
// element order) -> 8 bf16 of code * d + off (off = -8 d for Q4_0, -128 d for
// Q8_0, the codes being unsigned here).  Exact in fp32, one rounding to bf16.
template <int QT>
__device__ __forceinline__ bf16x8 dequant8(u32x2 raw, int shift, float d) {
    constexpr uint32_t kFlip = QT == UNILLM_QTYPE_Q4_0 ? 0x88888888u : 0x80808080u;
    const float off = d * (QT == UNILLM_QTYPE_Q4_0 ? -8.0f : -128.0f);
    uint32_t u[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t w = raw[h] ^ kFlip;  // signed codes -> unsigned (q, or q + 128)
        u[h] = QT == UNILLM_QTYPE_Q4_0 ? (w >> shift) & 0x0F0F0F0Fu : w;
    }
    float f[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int e = 0; e < 4; ++e)  // v_cvt_f32_ubyte{e}
            f[4 * h + e] = fmaf((float)((u[h] >> (8 * e)) & 0xFFu), d, off);
    }
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 p = {pack_bf16(f[0], f[1]), pack_bf16(f[2], f[3]), pack_bf16(f[4], f[5]),
                     pack_bf16(f[6], f[7])};
    return __builtin_bit_cast(bf16x8, p);
}

// x (f32) -> bf16, round to nearest even; 8 elements per thread per pass.
__global__ __launch_bounds__(256) void x_to_bf16_kernel(const float* __restrict__ x,
                                                        uint4* __restrict__ xb, int64_t n8) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float4 a = reinterpret_cast<const float4*>(x)[2 * i];
        const float4 b = reinterpret_cast<const float4*>(x)[2 * i + 1];
        xb[i] = make_uint4(pack_bf16(a.x, a.y), pack_bf16(a.z, a.w), pack_bf16(b.x, b.y),
                           pack_bf16(b.z, b.w));
    }
}

// Register-staged operands of one k step (64 k): the bf16 A slice this thread
// copies into LDS (A comes from L2 -- the XCD's CUs share it -- and is loaded
// one step ahead), and this lane's raw B fragments with their scales (B comes
// from HBM and is loaded D steps ahead).
template <int BM, int NW>
struct AStage {
    static constexpr int APASS = BM * 8 / (64 * NW);  // 16-byte A chunks per thread
    uint4 a[APASS];
};
template <int TJ>
struct BStage {
    u32x2 b[TJ][2];    // [16-column tile j][block of the step]
    uint32_t sc[TJ];   // the two f16 scales of the step's blocks, per j
};

template <int QT, int BM, int NW, int D>
__global__ __launch_bounds__(NW * 64, 1) void prefill_kernel(const uint8_t* __restrict__ base,
                                                              int64_t rb,
                                                              const __bf16* __restrict__ xb,
                                                              float* __restrict__ y, int M, int N,
                                                              int KB, int tiles_n, int tiles,
                                                              int tiles_pad) {
    constexpr int QB = QT == UNILLM_QTYPE_Q4_0 ? 16 : 32;  // payload bytes per block
    constexpr int TI = BM / 16;                            // MFMA tiles along m per wave
    constexpr int WC = PBN / NW;                           // output columns per wave
    constexpr int TJ = WC / 16;                            // MFMA tiles along n per wave
    constexpr int NT = NW * 64;                            // threads
    constexpr int AROWS = NT / 8;                          // rows one pass of A chunks covers
    constexpr int APASS = AStage<BM, NW>::APASS;
    __shared__ __attribute__((aligned(16))) __bf16 As[2][BM * PLD];

    // ---- tile (XCD-aware) ----
    const int per_xcd = tiles_pad / 8;
    const int t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (t >= tiles) return;  // padding workgroups (uniform: the whole workgroup leaves)
    const int mt = t / tiles_n, nt = t % tiles_n;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int m0 = mt * BM;
    const uint32_t K = (uint32_t)KB * QK;
    const int ksteps = (KB + 1) / 2;

    // ---- A: thread -> 16-byte chunk (tid % 8) of rows tid / 8 + AROWS p (bf16, 32-bit
    // element offsets: the launcher keeps m * k below 2^30); rows past m read row m - 1
    // and are never stored
    const int arow = tid / 8, ach = tid % 8;

    // ---- B: lane -> column (l % 16) of each 16-column tile, elements 8 g .. +7 of a
    // block (g = l / 16): Q4_0 payload bytes 8 (g & 1) .. +7, low nibbles for g < 2,
    // high for g >= 2; Q8_0 bytes 8 g .. +7.  32-bit byte offsets (weights < 4 GiB).
    const int g = lane / 16;
    const uint32_t boff = QT == UNILLM_QTYPE_Q4_0 ? 8 * (g & 1) : 8 * g;
    const int bshift = QT == UNILLM_QTYPE_Q4_0 ? 4 * (g >> 1) : 0;
    uint32_t bcol[TJ];
    bool bval[TJ];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int c = nt * PBN + wv * WC + j * 16 + (lane % 16);
        bval[j] = c < N;
        bcol[j] = (uint32_t)min(c, N - 1) * (uint32_t)rb;
    }
    const uint32_t sbase = (uint32_t)KB * QB;  // scales follow the row's payloads

    auto load_a = [&](AStage<BM, NW>& st, int ks) {
        // k chunks past the end (an odd KB's last step) re-read the row's last chunk
        const uint32_t kk = min((uint32_t)ks * PBK + ach * 8, K - 8);
#pragma unroll
        for (int p = 0; p < APASS; ++p) {
            const uint32_t row = (uint32_t)min(m0 + arow + AROWS * p, M - 1);
            st.a[p] = *reinterpret_cast<const uint4*>(xb + row * K + kk);
        }
    };
    auto load_b = [&](BStage<TJ>& st, int ks) {
        const int kb0 = 2 * ks, kb1 = min(2 * ks + 1, KB - 1);
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            st.b[j][0] = *reinterpret_cast<const u32x2*>(base + bcol[j] + (uint32_t)kb0 * QB + boff);
            st.b[j][1] = *reinterpret_cast<const u32x2*>(base + bcol[j] + (uint32_t)kb1 * QB + boff);
            // scales kb0, kb0 + 1 in one dword (kb0 is even; an odd KB's last step reads
            // two bytes past the scales, inside the row padding or the weight's tail slot)
            st.sc[j] = *reinterpret_cast<const uint32_t*>(base + bcol[j] + sbase + 2u * kb0);
        }
    };
    auto store_a = [&](const AStage<BM, NW>& st, int ks, int buf) {
        const uint32_t keep = 0u - (uint32_t)((uint32_t)ks * PBK + ach * 8 < K);
#pragma unroll
        for (int p = 0; p < APASS; ++p) {
            const uint4 v = make_uint4(st.a[p].x & keep, st.a[p].y & keep, st.a[p].z & keep,
                                       st.a[p].w & keep);
            *reinterpret_cast<uint4*>(&As[buf][(arow + AROWS * p) * PLD + ach * 8]) = v;
        }
    };
    bf16x8 bfrag[TJ][2];
    auto dequant_b = [&](const BStage<TJ>& st, int ks) {
        const bool b1ok = 2 * ks + 1 < KB;
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const float d0 = bval[j] ? __half2float(__ushort_as_half((uint16_t)st.sc[j])) : 0.0f;
            const float d1 = bval[j] && b1ok
                                 ? __half2float(__ushort_as_half((uint16_t)(st.sc[j] >> 16)))
                                 : 0.0f;
            bfrag[j][0] = dequant8<QT>(st.b[j][0], bshift, d0);
            bfrag[j][1] = dequant8<QT>(st.b[j][1], bshift, d1);
        }
    };

    f32x4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int fr = lane % 16, fk = (lane / 16) * 8;
    auto mfma_step = [&](int buf) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const bf16x8 a = *reinterpret_cast<const bf16x8*>(
                    &As[buf][(16 * i + fr) * PLD + 32 * kk + fk]);
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bfrag[j][kk],
                                                                        acc[i][j], 0, 0, 0);
            }
        // schedule: one A fragment read, then its TJ MFMAs (a fragment is live for
        // one group only; the SIMD's other wave covers the LDS latency)
#pragma unroll
        for (int g2 = 0; g2 < 2 * TI; ++g2) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
            __builtin_amdgcn_sched_group_barrier(0x008, TJ, 0);  // MFMA
        }
    };

    // A one step ahead, B D steps ahead.  Steady state: every step loads (no
    // conditions); the last steps run in a separate tail.
    AStage<BM, NW> sa;
    BStage<TJ> sb[D];
    load_a(sa, 0);
#pragma unroll
    for (int d = 0; d < D; ++d) load_b(sb[d], min(d, ksteps - 1));
    auto step = [&](BStage<TJ>& b_, int ks, bool more_a, bool more_b) {
        store_a(sa, ks, ks & 1);
        dequant_b(b_, ks);
        if (more_a) load_a(sa, ks + 1);
        // A's loads stay older than B's: the wait for A next step then leaves
        // B's D-step-ahead loads in flight (vmcnt counts in issue order)
        __builtin_amdgcn_sched_barrier(0);
        if (more_b) load_b(b_, ks + D);
        __syncthreads();
        mfma_step(ks & 1);
    };
    int k0 = 0;
    for (; k0 + 2 * D <= ksteps; k0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) step(sb[d], k0 + d, true, true);
    }
    // tail: fewer than 2 D steps left
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (k0 + d < ksteps) step(sb[d], k0 + d, k0 + d + 1 < ksteps, k0 + d + D < ksteps);
#pragma unroll
    for (int d = 0; d < D; ++d)
        if (k0 + D + d < ksteps) step(sb[d], k0 + D + d, k0 + D + d + 1 < ksteps, false);

    // ---- epilogue: lane holds C[4 (l / 16) + e][l % 16] of each 16 x 16 tile ----
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
        const int col = nt * PBN + wv * WC + j * 16 + fr;
        if (col >= N) continue;
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = m0 + 16 * i + 4 * (lane / 16) + e;
                if (row < M) y[(int64_t)row * N + col] = acc[i][j][e];
            }
    }
}

template <int QT, int BM>
hipError_t launch_bm(const QWeight& w, const __bf16* xb, int64_t m, float* y, hipStream_t s) {
    // x is addressed with 32-bit element offsets: launch in row chunks below 2^30 elements
    const int64_t chunk = std::max<int64_t>(BM, ((int64_t)1 << 30) / w.k / BM * BM);
    if (m > chunk) {
        for (int64_t r = 0; r < m; r += chunk) {
            hipError_t e = launch_bm<QT, BM>(w, xb + r * w.k, std::min(chunk, m - r), y + r * w.n, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const int tiles_m = (int)((m + BM - 1) / BM);
    const int tiles_n = (int)((w.n + PBN - 1) / PBN);
    const int tiles = tiles_m * tiles_n;
    const int tiles_pad = (tiles + 7) / 8 * 8;
    prefill_kernel<QT, BM, kWaves, kDepth><<<tiles_pad, kWaves * 64, 0, s>>>(
        w.base, w.row_bytes, xb, y, (int)m, (int)w.n, (int)w.kb, tiles_n, tiles, tiles_pad);
    return hipGetLastError();
}

template <int QT>
hipError_t launch_qt(const QWeight& w, const __bf16* xb, int64_t m, float* y, hipStream_t s) {
    // 256-row tiles when they give at least one tile per CU, else 128-row tiles
    const int64_t tiles_n = (w.n + PBN - 1) / PBN;
    const int64_t tiles256 = (m + 255) / 256 * tiles_n;
    if (tiles256 >= device_info().cu_count) return launch_bm<QT, 256>(w, xb, m, y, s);
    return launch_bm<QT, 128>(w, xb, m, y, s);
}

}  // namespace

hipError_t launch_prefill_mfma(const QWeight& w, const float* x, int64_t m, float* y,
                               hipStream_t s) {
    // x in bf16 (the operand precision) in a stream-ordered workspace: the GEMM
    // re-reads x once per 256-column tile, so it reads half the bytes, and no
    // conversion sits in its inner loop.  The pool keeps the memory between calls.
    const int64_t n = m * w.k;  // k % 32 == 0, so n % 8 == 0
    void* ws = nullptr;
    hipError_t e = hipMallocAsync(&ws, (size_t)n * sizeof(__bf16), s);
    if (e != hipSuccess) return e;
    const int64_t n8 = n / 8;
    const int grid = (int)std::min<int64_t>((n8 + 255) / 256, (int64_t)device_info().cu_count * 16);
    x_to_bf16_kernel<<<grid, 256, 0, s>>>(x, static_cast<uint4*>(ws), n8);
    e = hipGetLastError();
    if (e == hipSuccess) {
        const __bf16* xb = static_cast<const __bf16*>(ws);
        e = w.qtype == UNILLM_QTYPE_Q4_0 ? launch_qt<UNILLM_QTYPE_Q4_0>(w, xb, m, y, s)
                                         : launch_qt<UNILLM_QTYPE_Q8_0>(w, xb, m, y, s);
    }
    hipError_t f = hipFreeAsync(ws, s);
    return e != hipSuccess ? e : f;
}

}  // namespace unillm
