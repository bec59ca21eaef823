// prefill_probe.hip -- the prefill kernel's loop skeleton on synthetic LDS operands:
// what its matrix-core loop reaches alone, and what the operand ring costs on top.
// Measurement infrastructure for the prefill roofline, not part of libunillm_hip.so.
//
//   ./unillm_amd/probe/prefill_probe            (built by python -m unillm_amd.build)
//
// Every mode runs 8 waves a workgroup (two a SIMD), one workgroup a CU, 1024
// workgroups, 512 steps of 64 k each: per step a wave multiplies 256 rows x 32
// columns (16 x 2 tiles of v_mfma_f32_16x16x32_f16, 64 MFMAs), reading its A and B
// fragments from LDS (the A region XOR-swizzled as the kernel's), then all waves meet
// at a barrier.  No dequant; the results are discarded.
//   compiler      fragment reads the compiler schedules (a k half, then its MFMAs)
//   asm 2 ahead   the kernel's reads: inline-asm ds_read_b128 two fragments ahead of
//                 their MFMAs with exact lgkmcnt waits, B once a step
//   asm 4 ahead   the same, four ahead
//   + ring        asm 2 ahead, plus the kernel's operand ring: per step each wave
//                 issues its 6 direct global -> LDS loads (4 x 1 KiB of A, 1 KiB of B
//                 payload, 256 B of scales: 42 KiB a step per workgroup, from an
//                 L2-resident 1 MiB buffer) into a 3-stage ring, waits for its own
//                 loads of the current stage (vmcnt 6) and meets the others
//   ring, no wait the ring's loads without the per-step vmcnt wait (one full wait after
//                 the loop; the loads' LDS writes land while the loop reads)
//   ring waits    the ring's waits and barriers, no loads
//   via VGPRs     the same bytes through registers: global_load_dwordx4 one step
//                 ahead, ds_write_b128 into the ring after the barrier
// Time: best of 5 launches.  TFLOP/s counts the MFMAs; the percentage is of the
// 2516.6 TFLOP/s dense f16 peak.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>

#include "../csrc/lds.hpp"

using namespace unillm;

#define CK(x)                                                                     \
    do {                                                                          \
        hipError_t e_ = (x);                                                      \
        if (e_ != hipSuccess) {                                                   \
            printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            exit(1);                                                              \
        }                                                                         \
    } while (0)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x24 __attribute__((ext_vector_type(24)));

enum Mode { COMPILER, ASM2, ASM4, RING, RING_NOWAIT, RING_WAITS, RING_VGPR };

constexpr int kStageBytes = 43008;          // 42 KiB: the kernel's stage at 256-row tiles
constexpr int kLds = 32768 + 3 * kStageBytes;  // A region + a 3-stage ring over the B region

template <int MODE>
__global__ __launch_bounds__(512, 1) void probe(float* out, int steps, const uint8_t* gsrc) {
    constexpr int TI = 16, TJ = 2;
    constexpr bool ring_mode = MODE >= RING;
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    f32x4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int i = threadIdx.x; i < 65536 / 16; i += 512)  // f16 1.0-ish operands
        reinterpret_cast<uint4*>(lds)[i] = make_uint4(0x3c003c00u ^ i, 0x3c003c00u, 0x3c003c00u,
                                                      0x3c003c00u);
    __syncthreads();
    const int fr = lane % 16, g = lane / 16;
    const uint32_t base = (uint32_t)(uintptr_t)lds;
    uint32_t aoff[2], boff[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
        aoff[kk] = base + (uint32_t)(fr * 128 + (((4 * kk + g) ^ (fr % 8)) * 16));
        boff[kk] = base + 32768 + (uint32_t)(wv * 2 * 16 * 128 + fr * 128 + (((4 * kk + g) ^ (fr % 8)) * 16));
    }
    // the ring: stage st at 32 KiB + (st % 3) * 42 KiB (over the B region: the
    // values change, the bounds hold); wave wv's 6 loads a step
    auto issue = [&](int st) {
        uint8_t* ring = lds + 32768 + (st % 3) * kStageBytes;
        const uint8_t* src = gsrc + ((st * 8 + wv) % 128) * 8192;
#pragma unroll
        for (int q = 0; q < 4; ++q) dma16(src + q * 1024 + lane * 16, ring + (wv * 4 + q) * 1024);
        dma16(src + 4096 + lane * 16, ring + 32768 + wv * 1024);
        dma4(src + 5120 + lane * 4, ring + 40960 + wv * 256);
    };
    u32x24 stg;  // RING_VGPR's staged bytes (one vector: stays in registers)
    auto gload = [&](int st) {
        const uint8_t* src = gsrc + ((st * 8 + wv) % 128) * 8192;
#pragma unroll
        for (int q = 0; q < 5; ++q) {
            const uint4 v = *reinterpret_cast<const uint4*>(src + (q < 4 ? q * 1024 : 4096) + lane * 16);
            stg[4 * q] = v.x;
            stg[4 * q + 1] = v.y;
            stg[4 * q + 2] = v.z;
            stg[4 * q + 3] = v.w;
        }
        stg[20] = *reinterpret_cast<const uint32_t*>(src + 5120 + lane * 4);
    };
    auto lwrite = [&](int st) {
        uint8_t* ring = lds + 32768 + (st % 3) * kStageBytes;
#pragma unroll
        for (int q = 0; q < 5; ++q)
            *reinterpret_cast<uint4*>(ring + (q < 4 ? (wv * 4 + q) * 1024 : 32768 + wv * 1024) + lane * 16) =
                make_uint4(stg[4 * q], stg[4 * q + 1], stg[4 * q + 2], stg[4 * q + 3]);
        *reinterpret_cast<uint32_t*>(ring + 40960 + wv * 256 + lane * 4) = stg[20];
    };
    if constexpr (MODE == RING_VGPR) gload(0);
    if constexpr (MODE == RING || MODE == RING_NOWAIT) {
        issue(0);
        issue(1);
    }
    for (int s = 0; s < steps; ++s) {
        if constexpr (MODE == RING_VGPR) {
            __builtin_amdgcn_s_barrier();
            lwrite(s);
            if (s + 1 < steps) gload(s + 1);
        } else if constexpr (ring_mode) {
            if constexpr (MODE != RING_NOWAIT) {
                if (s + 1 < steps) wait_vmcnt<6>();
                else wait_vmcnt<0>();
            }
            __builtin_amdgcn_s_barrier();
            if constexpr (MODE != RING_WAITS)
                if (s + 2 < steps) issue(s + 2);
        }
        if constexpr (MODE == COMPILER) {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                f16x8 a[TI], b[TJ];
#pragma unroll
                for (int i = 0; i < TI; ++i)
                    a[i] = *reinterpret_cast<const f16x8*>(lds + (16 * i + fr) * 128 + ((4 * kk + g) ^ (fr % 8)) * 16);
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    b[j] = *reinterpret_cast<const f16x8*>(lds + 32768 + (wv * 2 * 16 + 16 * j + fr) * 128 +
                                                           ((4 * kk + g) ^ (fr % 8)) * 16);
#pragma unroll
                for (int i = 0; i < TI; ++i)
#pragma unroll
                    for (int j = 0; j < TJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
            }
        } else {
            f16x8 bf[TJ][2];
            {
                lds_u32x4 b00 = lds_read128<0>(boff[0]), b01 = lds_read128<0>(boff[1]);
                lds_u32x4 b10 = lds_read128<2048>(boff[0]), b11 = lds_read128<2048>(boff[1]);
                asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(b00), "+v"(b01), "+v"(b10), "+v"(b11));
                bf[0][0] = __builtin_bit_cast(f16x8, b00);
                bf[0][1] = __builtin_bit_cast(f16x8, b01);
                bf[1][0] = __builtin_bit_cast(f16x8, b10);
                bf[1][1] = __builtin_bit_cast(f16x8, b11);
            }
            constexpr int PF = MODE == ASM4 ? 4 : 2;
            f16x8 afr[2 * TI];
            constexpr_for<PF>([&](auto F) {
                afr[F.value] = __builtin_bit_cast(f16x8, lds_read128<(F.value % TI) * 2048>(aoff[F.value / TI]));
            });
#pragma unroll
            for (int f = 0; f < 2 * TI; ++f) {
                if (f + PF < 2 * TI) {
                    constexpr_for<2 * TI>([&](auto F) {
                        if (F.value == f + PF)
                            afr[F.value] =
                                __builtin_bit_cast(f16x8, lds_read128<(F.value % TI) * 2048>(aoff[F.value / TI]));
                    });
                    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(afr[f]) : "n"(PF));
                } else {
                    const int left = 2 * TI - 1 - f;  // reads issued after fragment f
                    if (left >= 3) asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(afr[f]));
                    else if (left == 2) asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(afr[f]));
                    else if (left == 1) asm volatile("s_waitcnt lgkmcnt(1)" : "+v"(afr[f]));
                    else asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(afr[f]));
                }
                const int kk = f / TI, i = f % TI;
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afr[f], bf[j][kk], acc[i][j], 0, 0, 0);
            }
        }
        if constexpr (!ring_mode) __builtin_amdgcn_s_barrier();
    }
    if constexpr (ring_mode) wait_vmcnt<0>();  // every direct load done before the waves end
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) t += acc[i][j][0] + acc[i][j][3];
    if (t == 12345.678f) out[threadIdx.x] = t;  // never true: keeps the MFMAs
}

template <int MODE>
void run(float* out, const uint8_t* gsrc, const char* name) {
    const int steps = 512, grid = 256 * 4;
    const int lds = MODE >= RING ? kLds : 65536;
    CK(hipFuncSetAttribute((const void*)probe<MODE>, hipFuncAttributeMaxDynamicSharedMemorySize, lds));
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    probe<MODE><<<grid, 512, lds>>>(out, steps, gsrc);
    CK(hipDeviceSynchronize());
    float best = 1e30f;
    for (int r = 0; r < 5; ++r) {
        CK(hipEventRecord(a));
        probe<MODE><<<grid, 512, lds>>>(out, steps, gsrc);
        CK(hipEventRecord(b));
        CK(hipEventSynchronize(b));
        float ms;
        CK(hipEventElapsedTime(&ms, a, b));
        best = ms < best ? ms : best;
    }
    const double flops = 2.0 * 16 * 16 * 32 * 64 * (double)steps * 8 * grid;
    printf("%-14s %.3f ms  %6.0f TFLOP/s  %5.1f %% of 2516.6\n", name, best, flops / best / 1e9,
           flops / best / 1e9 / 2516.6 * 100);
    fflush(stdout);
    CK(hipEventDestroy(a));
    CK(hipEventDestroy(b));
}

int main() {
    static_assert(kLds <= 160 * 1024, "the ring fits the CU's LDS");
    float* out;
    uint8_t* g;
    CK(hipMalloc(&out, 4096 * sizeof(float)));
    CK(hipMalloc(&g, 2 << 20));
    CK(hipMemset(g, 0x3c, 2 << 20));
    for (int rep = 0; rep < 2; ++rep) {
        run<COMPILER>(out, g, "compiler");
        run<ASM2>(out, g, "asm 2 ahead");
        run<ASM4>(out, g, "asm 4 ahead");
        run<RING>(out, g, "+ ring");
        run<RING_NOWAIT>(out, g, "ring, no wait");
        run<RING_WAITS>(out, g, "ring waits");
        run<RING_VGPR>(out, g, "via VGPRs");
    }
    CK(hipFree(out));
    CK(hipFree(g));
    return 0;
}
