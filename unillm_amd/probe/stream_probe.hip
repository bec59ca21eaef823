// stream_probe.hip -- the HBM streaming ceiling of one decode-GEMV-sized launch, and
// where the Q4_0 GEMV sits against it.  Measurement infrastructure for the decode
// GEMV's roofline, not part of libunillm_hip.so.
//
//   ./unillm_amd/probe/stream_probe            (built by python -m unillm_amd.build)
//
// One harness, one timing method for every row: a HIP graph of back-to-back launches
// over distinct copies of the data (at least 1 GiB in total, so nothing is served from
// the 256 MB Infinity Cache), replayed 6 times, the best replay divided by the launch
// count.  Data is random.  Rows:
//   per-launch   one launch per segment (256 x 1024 threads): each wave reads 1 KiB
//                pieces c = j W + w of a flat segment, 16 bytes a lane, all NL pieces
//                requested at once, their XOR consumed -- the plain read of one
//                GEMV's bytes;
//   one-launch   ONE launch reads all segments back to back (the next segment's
//                pieces requested before the current one is consumed): the same
//                bytes per segment without a launch boundary between segments;
//   rows         the GEMV's own request order without its arithmetic: wave w owns
//                rows w, w + W, ..., lane l the 16-byte pieces l, l + 64, ... of each
//                row's payload, rows of 2304 bytes (a repacked Q4_0 row of k = 4096);
//   gemv         unillm_hip_qmatmul on Q4_0 weights of the same shape (m = 1).
// The difference per-launch - one-launch is the cost of a launch boundary (dispatch,
// the first requests' latency, the drain); gemv - per-launch is what the GEMV's own
// dependencies and arithmetic add to a plain read of its bytes.
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <vector>

#include "../../include/unillm_hip.h"

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

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
        if ((x) != UNILLM_OK) {                                                      \
            printf("unillm error %s at line %d\n", unillm_hip_last_error(), __LINE__); \
            exit(1);                                                                 \
        }                                                                            \
    } while (0)

constexpr int kThreads = 1024, kWavesPerBlock = kThreads / 64, kBlocks = 256;

template <int NL>
__device__ __forceinline__ unsigned read_segment(const uint8_t* seg, int nch, int wave, int waves,
                                                 int lane) {
    u32x4 r[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int c = min(j * waves + wave, nch - 1);
        r[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(seg + (size_t)c * 1024) + lane);
    }
    unsigned a = 0;
#pragma unroll
    for (int j = 0; j < NL; ++j) a += r[j][0] ^ r[j][1] ^ r[j][2] ^ r[j][3];
    return a;
}

// per-launch: one segment
template <int NL>
__global__ __launch_bounds__(kThreads) void per_launch(const uint8_t* seg, int nch, unsigned* out) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const unsigned a = read_segment<NL>(seg, nch, wave, gridDim.x * kWavesPerBlock, lane);
    if (a == 0x12345678u) out[wave] = a;  // consumed, practically never stored
}

// one-launch: nseg segments, the next one's pieces requested before the current is consumed
template <int NL>
__global__ __launch_bounds__(kThreads) void one_launch(const uint8_t* base, size_t seg_bytes,
                                                       int nseg, int nch, unsigned* out) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const int waves = gridDim.x * kWavesPerBlock;
    u32x4 A[NL], B[NL];
    auto load = [&](u32x4 (&r)[NL], const uint8_t* seg) {
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const int c = min(j * waves + wave, nch - 1);
            r[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(seg + (size_t)c * 1024) + lane);
        }
    };
    auto use = [&](const u32x4 (&r)[NL]) {
        unsigned a = 0;
#pragma unroll
        for (int j = 0; j < NL; ++j) a += r[j][0] ^ r[j][1] ^ r[j][2] ^ r[j][3];
        return a;
    };
    unsigned acc = 0;
    load(A, base);
    for (int s = 0; s < nseg; s += 2) {
        if (s + 1 < nseg) load(B, base + (size_t)(s + 1) * seg_bytes);
        acc += use(A);
        if (s + 2 < nseg) load(A, base + (size_t)(s + 2) * seg_bytes);
        if (s + 1 < nseg) acc += use(B);
    }
    if (acc == 0x12345678u) out[wave] = acc;
}

// rows: the GEMV's request order (rows of rb bytes, payload pb bytes each), no arithmetic
template <int RPW>
__global__ __launch_bounds__(kThreads) void rows(const uint8_t* base, int nrows, int rb, int pb,
                                                 unsigned* out) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const int waves = gridDim.x * kWavesPerBlock;
    constexpr int P = 2;  // 1 KiB pieces per row (pb = 2048)
    u32x4 r[RPW * P];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int row = min(wave + i * waves, nrows - 1);
#pragma unroll
        for (int p = 0; p < P; ++p)
            r[i * P + p] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(base + (size_t)row * rb + p * 1024) + lane);
    }
    unsigned a = 0;
#pragma unroll
    for (int j = 0; j < RPW * P; ++j) a += r[j][0] ^ r[j][1] ^ r[j][2] ^ r[j][3];
    if (pb < 0) a += rb;  // keep pb live
    if (a == 0x12345678u) out[wave] = a;
}

__global__ void fill_random(uint32_t* p, size_t n, uint32_t seed) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        uint32_t h = (uint32_t)i * 2654435761u ^ seed;
        h ^= h >> 15;
        h *= 2246822519u;
        h ^= h >> 13;
        p[i] = h;
    }
}

// N(0, 0.02)-like weights: uniform in [-0.035, 0.035] (same variance), enough for timing
__global__ void fill_weights(float* w, size_t n, uint32_t seed) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        uint32_t h = (uint32_t)i * 2654435761u ^ seed;
        h ^= h >> 15;
        h *= 2246822519u;
        h ^= h >> 13;
        w[i] = ((float)(h >> 8) * (1.0f / 16777216.0f) - 0.5f) * 0.0693f;
    }
}

// Best per-launch time (us) of `launches` back-to-back launches captured into a graph.
template <typename F>
double time_graph(hipStream_t s, int launches, F&& launch_all) {
    hipGraph_t g;
    hipGraphExec_t ge;
    CK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    launch_all();
    CK(hipStreamEndCapture(s, &g));
    CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    double best = 1e30;
    for (int rep = 0; rep < 7; ++rep) {
        CK(hipEventRecord(e0, s));
        CK(hipGraphLaunch(ge, s));
        CK(hipEventRecord(e1, s));
        CK(hipEventSynchronize(e1));
        float ms;
        CK(hipEventElapsedTime(&ms, e0, e1));
        if (rep) best = std::min(best, (double)ms * 1e3 / launches);
    }
    CK(hipGraphExecDestroy(ge));
    CK(hipGraphDestroy(g));
    CK(hipEventDestroy(e0));
    CK(hipEventDestroy(e1));
    return best;
}

void report(const char* what, double bytes, double us) {
    printf("| %-44s | %10.0f | %7.2f | %7.0f | %5.1f %% |\n", what, bytes, us, bytes / us / 1e3,
           bytes / us / 1e3 / 80.0);
    fflush(stdout);
}

int main() {
    CU(unillm_hip_init(0));
    hipStream_t s;
    CK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    unsigned* out;
    CK(hipMalloc(&out, 1 << 20));
    printf("| read | bytes / launch | us / launch | GB/s | of 8 TB/s |\n|---|---|---|---|---|\n");

    // the decode shapes: QKV (12288 rows) and o (4096 rows) of k = 4096, Q4_0
    for (int n : {12288, 4096}) {
        const int k = 4096, rb = 2304, pb = 2048;
        const size_t wbytes = (size_t)n * rb;           // repacked Q4_0 bytes
        const int nch = (int)(wbytes / 1024);
        const int copies = (int)std::max<size_t>(8, ((size_t)1 << 30) / wbytes + 1);
        uint8_t* data;
        CK(hipMalloc(&data, (size_t)nch * 1024 * copies + 65536));
        fill_random<<<4096, 256, 0, s>>>(reinterpret_cast<uint32_t*>(data),
                                         ((size_t)nch * 1024 * copies + 65536) / 4, 7u + n);
        CK(hipStreamSynchronize(s));
        const double bytes = (double)nch * 1024;
        // pieces a lane requests per segment: nch / (256 blocks x 16 waves), rounded up
        // (7 at n = 12288, 3 at n = 4096; a lane past the last piece re-requests it)
        const int nl = (nch + kBlocks * kWavesPerBlock - 1) / (kBlocks * kWavesPerBlock);
        char label[96];
        auto per = [&]() {
            for (int c = 0; c < copies; ++c) {
                const uint8_t* seg = data + (size_t)nch * 1024 * c;
                if (nl <= 3) per_launch<3><<<kBlocks, kThreads, 0, s>>>(seg, nch, out);
                else if (nl <= 7) per_launch<7><<<kBlocks, kThreads, 0, s>>>(seg, nch, out);
                else per_launch<8><<<kBlocks, kThreads, 0, s>>>(seg, nch, out);
            }
        };
        snprintf(label, sizeof label, "per-launch, n = %d", n);
        report(label, bytes, time_graph(s, copies, per));
        auto one = [&]() {
            if (nl <= 3) one_launch<3><<<kBlocks, kThreads, 0, s>>>(data, (size_t)nch * 1024, copies, nch, out);
            else if (nl <= 7) one_launch<7><<<kBlocks, kThreads, 0, s>>>(data, (size_t)nch * 1024, copies, nch, out);
            else one_launch<8><<<kBlocks, kThreads, 0, s>>>(data, (size_t)nch * 1024, copies, nch, out);
        };
        snprintf(label, sizeof label, "one-launch (per segment), n = %d", n);
        report(label, bytes, time_graph(s, copies, one));
        auto rw = [&]() {
            for (int c = 0; c < copies; ++c) {
                const uint8_t* seg = data + (size_t)nch * 1024 * c;
                if (n > 8192) rows<3><<<kBlocks, kThreads, 0, s>>>(seg, n, rb, pb, out);
                else rows<1><<<kBlocks, kThreads, 0, s>>>(seg, n, rb, pb, out);
            }
        };
        snprintf(label, sizeof label, "rows (GEMV request order), n = %d", n);
        report(label, (double)n * pb, time_graph(s, copies, rw));
        CK(hipFree(data));

        // the library's GEMV on Q4_0 weights of the same shape
        const size_t gb = (size_t)n * (k / 32) * 18;
        const int wc = (int)std::max<size_t>(8, ((size_t)1 << 30) / gb + 1);
        float* wf;
        void* blocks;
        CK(hipMalloc(&wf, (size_t)n * k * 4));
        CK(hipMalloc(&blocks, gb));
        std::vector<unillm_qweight*> ws(wc);
        for (int c = 0; c < wc; ++c) {
            fill_weights<<<4096, 256, 0, s>>>(wf, (size_t)n * k, 11u + c);
            CU(unillm_hip_quantize(UNILLM_QTYPE_Q4_0, wf, n, k, blocks, s));
            CU(unillm_hip_qweight_create_device(UNILLM_QTYPE_Q4_0, n, k, blocks, gb, 0, s, &ws[c]));
        }
        CK(hipStreamSynchronize(s));
        float *x, *y;
        CK(hipMalloc(&x, k * 4));
        CK(hipMalloc(&y, n * 4));
        fill_weights<<<16, 256, 0, s>>>(x, k, 5u);
        for (int c = 0; c < wc; ++c) CU(unillm_hip_qmatmul(ws[c], x, 1, y, s));  // warm workspaces
        CK(hipStreamSynchronize(s));
        auto gemv = [&]() {
            for (int c = 0; c < wc; ++c) CU(unillm_hip_qmatmul(ws[c], x, 1, y, s));
        };
        snprintf(label, sizeof label, "gemv (unillm_hip_qmatmul, m = 1), n = %d", n);
        report(label, (double)gb + 4.0 * k + 4.0 * n, time_graph(s, wc, gemv));
        for (auto w : ws) CU(unillm_hip_qweight_destroy(w));
        CK(hipFree(wf));
        CK(hipFree(blocks));
        CK(hipFree(x));
        CK(hipFree(y));
    }
    CK(hipFree(out));
    CK(hipStreamDestroy(s));
    return 0;
}
