// decode_probe.hip -- the weight stream of the batched-decode kernel without its
// arithmetic: which request pattern and which workgroup arrangement stream a Q4_0
// matrix (k = 4096: rows of 2304 bytes, 2048 of payload) fastest through a D-stage LDS
// ring filled by direct global -> LDS loads (16 bytes a lane).  Measurement
// infrastructure for the batched-decode roofline, not part of libunillm_hip.so.
//
//   ./unillm_amd/probe/decode_probe            (built by python -m unillm_amd.build)
//
// Each launch streams the payload of one matrix copy (96 or 64 distinct copies, so the
// data comes from HBM); time = best of 5 rounds of back-to-back launches / launches.
// Chunk = 8 KiB per workgroup step, laid out as
//   MODE 0  128 rows x 64 B (the batched-decode kernel's chunk), workgroup = (128-row
//           group, k slice)
//   MODE 3  64 rows x 128 B,  MODE 1  32 rows x 256 B
//   MODE 2  8 KiB contiguous (what a tile-major weight layout would give)
// and "persist": MODE 0 chunks, G workgroups walking all (row group, slice) items
// through one continuous ring.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <vector>
#include <algorithm>
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1);} } while (0)
typedef __attribute__((address_space(1))) const void* gbl_ptr;
typedef __attribute__((address_space(3))) void* lds_ptr;
__device__ __forceinline__ void dma16(const void* g, uint8_t* l) {
    __builtin_amdgcn_global_load_lds((gbl_ptr)g, (lds_ptr)l, 16, 0, 0);
}
template <int N> __device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N)); }

template <int MODE, int D>
__global__ __launch_bounds__(256) void probe(const uint8_t* __restrict__ base, int rb, int N,
                                             int chunks_row, int S, float* out) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int rg = blockIdx.x / S, sp = blockIdx.x % S;
    // chunks: MODE 0/2: 128 k (64 B) x 128 rows; MODE 1: 512 k (256 B) x 32 rows; MODE 3: 256 k x 64 rows
    const int cpr = MODE == 1 ? chunks_row / 4 : MODE == 3 ? chunks_row / 2 : chunks_row;
    const int c0 = sp * cpr / S, c1 = (sp + 1) * cpr / S, nch = c1 - c0;
    auto issue = [&](int j) {
        const int c = c0 + j;
        uint8_t* st = lds + (j % D) * 8192 + wv * 2048;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint8_t* src;
            if constexpr (MODE == 0) {  // wave: 32 rows; load i: rows 16 i + lane / 4, piece lane % 4
                const int r = rg * 128 + 32 * wv + 16 * i + lane / 4;
                src = base + (size_t)min(r, N - 1) * rb + c * 64 + 16 * (lane % 4);
            } else if constexpr (MODE == 1) {  // wave: 8 rows; load i: rows 4 i + lane / 16, piece lane % 16
                const int r = rg * 32 + 8 * wv + 4 * i + lane / 16;
                src = base + (size_t)min(r, N - 1) * rb + c * 256 + 16 * (lane % 16);
            } else if constexpr (MODE == 3) {  // wave: 16 rows; load i: rows 8 i + lane / 8
                const int r = rg * 64 + 16 * wv + 8 * i + lane / 8;
                src = base + (size_t)min(r, N - 1) * rb + c * 128 + 16 * (lane % 8);
            } else {  // contiguous 8 KB per (row group, chunk)
                const size_t t = (size_t)rg * chunks_row + c;
                src = base + t * 8192 + wv * 2048 + i * 1024 + 16 * lane;
            }
            dma16(src, st + i * 1024);
        }
    };
    for (int j = 0; j < D - 1 && j < nch; ++j) issue(j);
    float acc = 0.f;
    for (int j = 0; j < nch; ++j) {
        if (j + D - 1 < nch) { wait_vm<2 * (D - 2)>(); } else { wait_vm<0>(); }
        __builtin_amdgcn_s_barrier();
        if (j + D - 1 < nch) issue(j + D - 1);
        acc += *reinterpret_cast<const float*>(lds + (j % D) * 8192 + tid * 4);
    }
    if (acc == 12345.f) out[blockIdx.x] = acc;
}

__global__ void fillr(uint32_t* p, size_t n, uint32_t seed) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        uint32_t h = (uint32_t)i * 2654435761u ^ seed; h ^= h >> 15; h *= 2246822519u; h ^= h >> 13; p[i] = h;
    }
}

template <int MODE, int D>
void run(const char* name, int N, int rb, int S, int lds_bytes, std::vector<uint8_t*>& ptrs, float* out) {
    const int chunks_row = 32;  // k = 4096: 32 chunks of 128 k (64 B payload each)
    const int groups = MODE == 1 ? (N + 31) / 32 : MODE == 3 ? (N + 63) / 64 : (N + 127) / 128;
    CK(hipFuncSetAttribute((const void*)probe<MODE, D>, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes));
    hipEvent_t a, b;
    CK(hipEventCreate(&a)); CK(hipEventCreate(&b));
    const int copies = (int)ptrs.size();
    for (int w = 0; w < 2; ++w)
        for (int c = 0; c < copies; ++c)
            probe<MODE, D><<<groups * S, 256, lds_bytes>>>(ptrs[c], rb, N, chunks_row, S, out);
    CK(hipDeviceSynchronize());
    float best = 1e9;
    for (int rep = 0; rep < 5; ++rep) {
        CK(hipEventRecord(a));
        for (int c = 0; c < copies; ++c)
            probe<MODE, D><<<groups * S, 256, lds_bytes>>>(ptrs[c], rb, N, chunks_row, S, out);
        CK(hipEventRecord(b));
        CK(hipEventSynchronize(b));
        float ms; CK(hipEventElapsedTime(&ms, a, b));
        best = std::min(best, ms / copies);
    }
    const double bytes = (double)N * 2048;  // payload bytes streamed
    printf("%-34s N=%5d S=%d wgs=%5d lds=%6d: %7.2f us  %6.0f GB/s\n", name, N, S, groups * S, lds_bytes,
           best * 1e3, bytes / (best * 1e-3) / 1e9);
    fflush(stdout);
}

template <int D>
__global__ __launch_bounds__(256) void probe_persist(const uint8_t* __restrict__ base, int rb, int N,
                                                     int chunks_row, int S, int items, float* out) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int G = gridDim.x;
    const int per = chunks_row / S;  // chunks per item (S divides)
    const int my_items = (items - (int)blockIdx.x + G - 1) / G;
    const int total = my_items * per;
    auto issue = [&](int j) {
        const int it = blockIdx.x + (j / per) * G;
        const int rg = it / S, sp = it % S;
        const int c = sp * per + j % per;
        uint8_t* st = lds + (j % D) * 8192 + wv * 2048;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = rg * 128 + 32 * wv + 16 * i + lane / 4;
            dma16(base + (size_t)min(r, N - 1) * rb + c * 64 + 16 * (lane % 4), st + i * 1024);
        }
    };
    for (int j = 0; j < D - 1 && j < total; ++j) issue(j);
    float acc = 0.f;
    for (int j = 0; j < total; ++j) {
        if (j + D - 1 < total) { wait_vm<2 * (D - 2)>(); } else { wait_vm<0>(); }
        __builtin_amdgcn_s_barrier();
        if (j + D - 1 < total) issue(j + D - 1);
        acc += *reinterpret_cast<const float*>(lds + (j % D) * 8192 + tid * 4);
    }
    if (acc == 12345.f) out[blockIdx.x] = acc;
}

template <int D>
void run_p(const char* name, int N, int rb, int S, int G, int lds_bytes, std::vector<uint8_t*>& ptrs, float* out) {
    const int chunks_row = 32;
    const int items = (N + 127) / 128 * S;
    CK(hipFuncSetAttribute((const void*)probe_persist<D>, hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes));
    hipEvent_t a, b;
    CK(hipEventCreate(&a)); CK(hipEventCreate(&b));
    const int copies = (int)ptrs.size();
    for (int w = 0; w < 2; ++w)
        for (int c = 0; c < copies; ++c)
            probe_persist<D><<<G, 256, lds_bytes>>>(ptrs[c], rb, N, chunks_row, S, items, out);
    CK(hipDeviceSynchronize());
    float best = 1e9;
    for (int rep = 0; rep < 5; ++rep) {
        CK(hipEventRecord(a));
        for (int c = 0; c < copies; ++c)
            probe_persist<D><<<G, 256, lds_bytes>>>(ptrs[c], rb, N, chunks_row, S, items, out);
        CK(hipEventRecord(b));
        CK(hipEventSynchronize(b));
        float ms; CK(hipEventElapsedTime(&ms, a, b));
        best = std::min(best, ms / copies);
    }
    const double bytes = (double)N * 2048;
    printf("%-34s N=%5d S=%d G=%4d items=%4d lds=%6d: %7.2f us  %6.0f GB/s\n", name, N, S, G, items, lds_bytes,
           best * 1e3, bytes / (best * 1e-3) / 1e9);
    fflush(stdout);
}

int main() {
    const int rb = 2304;
    const int maxN = 14336;
    const size_t bytes = (size_t)maxN * rb;
    std::vector<uint8_t*> ptrs(96);
    for (auto& p : ptrs) {
        CK(hipMalloc(&p, bytes + 65536));
        fillr<<<1024, 256>>>((uint32_t*)p, (bytes + 65536) / 4, 7);
    }
    float* out; CK(hipMalloc(&out, 1 << 20));
    CK(hipDeviceSynchronize());
    for (int N : {4096, 14336}) {
        std::vector<uint8_t*> use(ptrs.begin(), ptrs.begin() + (N == 4096 ? 96 : 64));
        for (int S : {4, 8}) {
            run<0, 4>("rows128x64B D4 (the kernel's chunk)", N, rb, S, 73728, use, out);
            run<3, 4>("rows64x128B D4", N, rb, S, 73728, use, out);
            run<1, 4>("rows32x256B D4", N, rb, S, 73728, use, out);
            run<2, 4>("contig8KB D4", N, rb, S, 73728, use, out);
        }
        run<1, 4>("rows32x256B D4, 4 wg/CU", N, rb, 4, 32768, use, out);
        for (int S : {4, 8, 16})
            for (int G : {256, 512}) run_p<4>("persist rows128x64B D4", N, rb, S, G, 40960, use, out);
    }
    return 0;
}
