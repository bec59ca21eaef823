// step_probe.hip -- the headline decode step (32 layers x {QKV 4096x12288, o 4096x4096,
// gate 4096x11008, up 4096x11008, down 11008x4096} Q4_0 GEMVs at m = 1, 160 distinct
// weights, 3.64 GB) as one HIP graph, timed three ways.  Measurement infrastructure
// for the decode GEMV's ceiling, not part of libunillm_hip.so.
//
//   ./unillm_amd/probe/step_probe            (built by python -m unillm_amd.build)
//
//   distinct      the step as bench.py times it: every weight read from HBM.
//   cached        the same 160 launches, every layer calling layer 0's five weights
//                 (114 MB, inside the 256 MB Infinity Cache): the chain with its
//                 weights already on chip.
//   prefetch G    distinct weights, plus a chain on a second stream that reads weight
//                 i + 1 with G workgroups while GEMV i runs (prefetch i + 1 waits
//                 for GEMV i - 1; the GEMV chain does not wait for the prefetches
//                 until the end of the step).
//   empty G x B   160 launches of an empty kernel, G workgroups of B threads (the
//                 GEMV's 256 x 1024, and two others): the graph's own cost per
//                 dependent launch, with no work.
// Each figure is the best of 8 rounds of 5 graph replays, per replay.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <vector>

#include "../../include/unillm_hip.h"
#include "../csrc/internal.hpp"

#define CK(x)                                                                        \
    do {                                                                             \
        hipError_t e_ = (x);                                                         \
        if (e_ != hipSuccess) {                                                      \
            printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);    \
            exit(1);                                                                 \
        }                                                                            \
    } while (0)
#define CU(x)                                                                        \
    do {                                                                             \
        int e_ = (x);                                                                \
        if (e_ != 0) {                                                               \
            printf("unillm error %d (%s) at line %d\n", e_, unillm_hip_last_error(), \
                   __LINE__);                                                        \
            exit(1);                                                                 \
        }                                                                            \
    } while (0)

// Reads n16 16-byte pieces with plain (cache-allocating) loads, 8 in flight per
// thread; the XOR keeps the loads alive (sink is never written for real data).
__global__ __launch_bounds__(256) void prefetch(const uint4* __restrict__ p, size_t n16, int* sink) {
    uint32_t acc = 0;
    const size_t stride = (size_t)gridDim.x * 2048;
    for (size_t i0 = (size_t)blockIdx.x * 2048 + threadIdx.x; i0 < n16; i0 += stride) {
        uint4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const size_t i = i0 + 256 * j;
            v[j] = i < n16 ? p[i] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) acc ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
    }
    if (acc == 0x9E3779B9u && sink) *sink = (int)acc;
}

// Does nothing; the pointer test keeps the launch from being optimized out.
__global__ __launch_bounds__(1024) void empty(int* sink) {
    if (sink && threadIdx.x == 1023 && blockIdx.x == 0) sink[0] = 0;
}

int main() {
    CU(unillm_hip_init(0));
    const int L = 32;
    const int64_t shapes[5][2] = {{12288, 4096}, {4096, 4096}, {11008, 4096}, {11008, 4096},
                                  {4096, 11008}};
    std::vector<unillm_qweight*> w;  // shape s, layer l at s L + l
    for (int s = 0; s < 5; ++s) {
        const int64_t n = shapes[s][0], k = shapes[s][1];
        const size_t nb = (size_t)n * (k / 32);
        std::vector<uint8_t> host(nb * 18);
        uint32_t r = 12345u + (uint32_t)s;
        for (size_t b = 0; b < nb; ++b) {
            uint8_t* blk = host.data() + b * 18;
            blk[0] = 0x00;
            blk[1] = 0x20;  // d = f16 0x2000 (2^-7)
            for (int j = 2; j < 18; ++j) {
                r = r * 1664525u + 1013904223u;
                blk[j] = (uint8_t)(r >> 24);
            }
        }
        for (int l = 0; l < L; ++l) {
            unillm_qweight* q = nullptr;
            CU(unillm_hip_qweight_create(UNILLM_QTYPE_Q4_0, n, k, host.data(), host.size(), 0, &q));
            w.push_back(q);
        }
    }
    std::vector<unillm_qweight*> distinct, cached;  // call order: layer by layer, 5 each
    for (int l = 0; l < L; ++l)
        for (int s = 0; s < 5; ++s) {
            distinct.push_back(w[s * L + l]);
            cached.push_back(w[s * L]);
        }
    size_t total = 0;
    for (auto* q : distinct) total += (size_t)(q->n * q->row_bytes);
    const int NW = (int)distinct.size();

    float *x, *y;
    CK(hipMalloc(&x, 11008 * 4));
    CK(hipMalloc(&y, 5 * 12288 * 4));
    std::vector<float> hx(11008);
    for (int i = 0; i < 11008; ++i) hx[i] = (float)((i * 37) % 101) / 50.0f - 1.0f;
    CK(hipMemcpy(x, hx.data(), hx.size() * 4, hipMemcpyHostToDevice));
    hipStream_t s, s2;
    CK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    CK(hipStreamCreateWithFlags(&s2, hipStreamNonBlocking));
    std::vector<hipEvent_t> ev(NW + 2);
    for (auto& e : ev) CK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    for (int i = 0; i < NW; ++i) CU(unillm_hip_qmatmul(distinct[i], x, 1, y + (i % 5) * 12288, s));
    CK(hipStreamSynchronize(s));

    auto build = [&](const std::vector<unillm_qweight*>& order, int G) {
        hipGraph_t g;
        hipGraphExec_t ge;
        auto pf = [&](int j) {
            prefetch<<<G, 256, 0, s2>>>(reinterpret_cast<const uint4*>(order[j]->base),
                                       (size_t)(order[j]->n * order[j]->row_bytes) / 16, nullptr);
        };
        CK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        if (G > 0) {  // fork s2 off s; prefetch 1 starts with GEMV 0
            CK(hipEventRecord(ev[NW], s));
            CK(hipStreamWaitEvent(s2, ev[NW], 0));
            pf(1);
        }
        for (int i = 0; i < NW; ++i) {
            if (G > 0 && i >= 1 && i + 1 < NW) {
                CK(hipStreamWaitEvent(s2, ev[i - 1], 0));
                pf(i + 1);
            }
            CU(unillm_hip_qmatmul(order[i], x, 1, y + (i % 5) * 12288, s));
            if (G > 0) CK(hipEventRecord(ev[i], s));
        }
        if (G > 0) {  // join
            CK(hipEventRecord(ev[NW + 1], s2));
            CK(hipStreamWaitEvent(s, ev[NW + 1], 0));
        }
        CK(hipStreamEndCapture(s, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        CK(hipGraphDestroy(g));
        return ge;
    };
    hipEvent_t t0, t1;
    CK(hipEventCreate(&t0));
    CK(hipEventCreate(&t1));
    auto timeit = [&](hipGraphExec_t ge) {
        CK(hipGraphLaunch(ge, s));
        CK(hipGraphLaunch(ge, s));
        CK(hipStreamSynchronize(s));
        float best = 1e30f;
        for (int r = 0; r < 8; ++r) {
            CK(hipEventRecord(t0, s));
            for (int j = 0; j < 5; ++j) CK(hipGraphLaunch(ge, s));
            CK(hipEventRecord(t1, s));
            CK(hipEventSynchronize(t1));
            float ms;
            CK(hipEventElapsedTime(&ms, t0, t1));
            best = std::min(best, ms / 5);
        }
        return best;
    };
    auto run = [&](const char* name, const std::vector<unillm_qweight*>& order, int G) {
        hipGraphExec_t ge = build(order, G);
        const float ms = timeit(ge);
        printf("%-14s %.4f ms/step  %.3f us/launch  %.1f GB/s (%.3f GB of distinct weights)\n",
               name, ms, ms * 1e3 / NW, total / ms / 1e6, total / 1e9);
        fflush(stdout);
        CK(hipGraphExecDestroy(ge));
    };
    run("distinct", distinct, 0);
    run("cached", cached, 0);
    run("prefetch 64", distinct, 64);
    run("prefetch 128", distinct, 128);
    run("distinct", distinct, 0);
    const int grids[3][2] = {{256, 1024}, {256, 64}, {2048, 256}};
    for (const auto& gb : grids) {
        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        for (int i = 0; i < NW; ++i) empty<<<gb[0], gb[1], 0, s>>>(nullptr);
        CK(hipStreamEndCapture(s, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        CK(hipGraphDestroy(g));
        const float ms = timeit(ge);
        printf("empty %4dx%-4d %.4f ms/step  %.3f us/launch\n", gb[0], gb[1], ms, ms * 1e3 / NW);
        fflush(stdout);
        CK(hipGraphExecDestroy(ge));
    }
    for (auto* q : w) CU(unillm_hip_qweight_destroy(q));
    return 0;
}
