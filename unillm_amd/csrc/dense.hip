// dense.hip -- dense (GGML F32 / F16 / BF16) projection weights.
//
// candle's QMatMul::from_arc dequantizes an F32 / F16 / BF16 tensor to an f32
// tensor, and its forward multiplies in f32 (the Tensor variant: x.matmul(w.t())).
// The reference's loader wraps every *_proj.weight / lm_head.weight tensor in a
// QMatMul whatever its GGML type (crates/runtime/src/weight_loader_core.rs:554-571),
// so a GGUF with F16 projections takes this variant.  Here such a weight is held as
// f32 rows [n][k] (F16 and BF16 widen exactly, as candle's dequantize does) and the
// product is one f32 GEMM through rocBLAS: there is no dequant to fuse, so a plain
// library GEMM is the kernel.  The epilogues keep their meaning: the residual add is
// the GEMM's beta = 1, the layer norm a row pass into the stream's workspace first,
// SwiGLU the elementwise pass after the product.
#include <hip/hip_fp16.h>
#include <rocblas/rocblas.h>

#include <mutex>
#include <string>

#include "internal.hpp"

namespace unillm {
namespace {

// dst[i] = src[i] widened to f32 (F16: the half value; BF16: the upper 16 bits of an f32)
__global__ __launch_bounds__(256) void widen_kernel(const uint16_t* __restrict__ src,
                                                    float* __restrict__ dst, int64_t count,
                                                    int bf16) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (int64_t)gridDim.x * blockDim.x) {
        const uint16_t v = src[i];
        dst[i] = bf16 ? __uint_as_float((uint32_t)v << 16) : __half2float(__ushort_as_half(v));
    }
}

// out[r] = (x[r] - mean) / sqrt(var + eps) * gamma (+ beta), one workgroup a row: the
// mean, then the mean of the squared deviations (ops_fn::layer_norm's two passes,
// tensor_core.rs:973-1008), in f32
__global__ __launch_bounds__(256) void norm_rows_kernel(const float* __restrict__ x, int64_t k,
                                                        NormArgs norm, float* __restrict__ out) {
    __shared__ float red[4];
    const float* xr = x + (int64_t)blockIdx.x * k;
    float* orow = out + (int64_t)blockIdx.x * k;
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    auto block_sum = [&](float v) {
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
        if (lane == 0) red[wv] = v;
        __syncthreads();
        const float s = (red[0] + red[1]) + (red[2] + red[3]);
        __syncthreads();
        return s;
    };
    float acc = 0.0f;
    for (int64_t i = t; i < k; i += 256) acc += xr[i];
    const float mean = block_sum(acc) / (float)k;
    acc = 0.0f;
    for (int64_t i = t; i < k; i += 256) {
        const float d = xr[i] - mean;
        acc += d * d;
    }
    const float sd = sqrtf(block_sum(acc) / (float)k + norm.eps);
    for (int64_t i = t; i < k; i += 256)
        orow[i] = (xr[i] - mean) / sd * norm.gamma[i] + (norm.beta ? norm.beta[i] : 0.0f);
}

// One rocBLAS handle per process (the library uses one device), with a workspace
// of its own so that no call allocates (HIP-graph capture records no allocation);
// atomics off, so a product is the same bits every call.
constexpr size_t kBlasWorkspace = (size_t)64 << 20;
std::mutex g_blas_mutex;
rocblas_handle g_blas = nullptr;
void* g_blas_ws = nullptr;
thread_local std::string g_dense_error;

const char* blas_status(rocblas_status st) { return rocblas_status_to_string(st); }

// The handle, created on first use (never while `s` is being captured).
hipError_t blas_handle(hipStream_t s, rocblas_handle* out) {
    if (!g_blas) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        hipError_t e = hipStreamIsCapturing(s, &cs);
        if (e != hipSuccess) return e;
        if (cs != hipStreamCaptureStatusNone) {
            g_dense_error = "the f32 GEMM's handle is created on first use, which cannot happen "
                            "while the stream is being captured; reserve before capture";
            return hipErrorStreamCaptureUnsupported;
        }
        rocblas_handle h = nullptr;
        rocblas_status st = rocblas_create_handle(&h);
        if (st != rocblas_status_success) {
            g_dense_error = std::string("rocblas_create_handle: ") + blas_status(st);
            return hipErrorUnknown;
        }
        void* ws = nullptr;
        if ((e = hipMalloc(&ws, kBlasWorkspace)) != hipSuccess) {
            (void)rocblas_destroy_handle(h);
            return e;
        }
        if ((st = rocblas_set_workspace(h, ws, kBlasWorkspace)) != rocblas_status_success ||
            (st = rocblas_set_atomics_mode(h, rocblas_atomics_not_allowed)) !=
                rocblas_status_success) {
            g_dense_error = std::string("rocBLAS handle set-up: ") + blas_status(st);
            (void)rocblas_destroy_handle(h);
            (void)hipFree(ws);
            return hipErrorUnknown;
        }
        g_blas = h;
        g_blas_ws = ws;
    }
    *out = g_blas;
    return hipSuccess;
}

}  // namespace

bool is_dense(int qtype) {
    return qtype == UNILLM_QTYPE_F32 || qtype == UNILLM_QTYPE_F16 || qtype == UNILLM_QTYPE_BF16;
}

int dense_elem_bytes(int qtype) { return qtype == UNILLM_QTYPE_F32 ? 4 : 2; }

std::string dense_error() { return g_dense_error; }

hipError_t launch_dense_upload(const QWeight& w, const void* src, hipStream_t s) {
    const int64_t count = w.n * w.k;
    if (w.qtype == UNILLM_QTYPE_F32)
        return hipMemcpyAsync(w.base, src, (size_t)count * 4, hipMemcpyDeviceToDevice, s);
    const int blocks = (int)std::min<int64_t>((count + 255) / 256, 8 * device_info().cu_count);
    widen_kernel<<<blocks, 256, 0, s>>>(static_cast<const uint16_t*>(src),
                                        reinterpret_cast<float*>(w.base), count,
                                        w.qtype == UNILLM_QTYPE_BF16);
    return hipGetLastError();
}

hipError_t launch_norm_rows(const float* x, int64_t m, int64_t k, const NormArgs& norm,
                            float* out, hipStream_t s) {
    norm_rows_kernel<<<(unsigned)m, 256, 0, s>>>(x, k, norm, out);
    return hipGetLastError();
}

hipError_t dense_prepare(hipStream_t s) {
    std::lock_guard<std::mutex> lock(g_blas_mutex);
    rocblas_handle h = nullptr;
    return blas_handle(s, &h);
}

// y[m, n] = x[m, k] W^T (+ y when add): row-major y is the column-major n x m
// matrix W x^T, i.e. sgemm(op(A) = A^T with A = W as a column-major k x n matrix,
// B = x as a column-major k x m matrix).
hipError_t launch_dense(const QWeight& w, const float* x, int64_t m, float* y, hipStream_t s,
                        int add) {
    std::lock_guard<std::mutex> lock(g_blas_mutex);
    rocblas_handle h = nullptr;
    hipError_t e = blas_handle(s, &h);
    if (e != hipSuccess) return e;
    rocblas_status st = rocblas_set_stream(h, s);
    const float alpha = 1.0f, beta = add ? 1.0f : 0.0f;
    if (st == rocblas_status_success)
        st = rocblas_sgemm(h, rocblas_operation_transpose, rocblas_operation_none, (rocblas_int)w.n,
                           (rocblas_int)m, (rocblas_int)w.k, &alpha,
                           reinterpret_cast<const float*>(w.base), (rocblas_int)w.k, x,
                           (rocblas_int)w.k, &beta, y, (rocblas_int)w.n);
    if (st != rocblas_status_success) {
        g_dense_error = std::string("rocblas_sgemm: ") + blas_status(st);
        return hipErrorUnknown;
    }
    return hipSuccess;
}

}  // namespace unillm
