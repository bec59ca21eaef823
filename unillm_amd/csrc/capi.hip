// capi.hip -- the extern "C" boundary (include/unillm_hip.h): argument checks,
// error reporting, weight lifetime and kernel-path dispatch.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include <hip/hip_fp16.h>
#include <math.h>

#include "internal.hpp"

namespace unillm {
namespace {

// The scratch of the no-allocation entry point (unillm_hip_qmatmul_noalloc): the x
// operand of the MFMA paths, in device memory that exists from module load to
// process end, one copy per GPU.  In host code the array's name denotes a host-side
// stand-in, not device memory: host code uses only the device address that
// hipGetSymbolAddress returns at init, kept per device in g_scratch_ptr.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
// Its last kNoAllocSyncBytes hold the batched decode's arrival tickets (cleared at
// init, and every launch leaves them zero); the x operand uses the rest.
constexpr size_t kNoAllocSyncBytes = (size_t)256 << 10;
std::vector<void*> g_scratch_ptr;  // by device index; nullptr before that device's init

thread_local std::string g_last_error;
std::once_flag g_init_once;
int g_init_status = UNILLM_ERR_NOT_INITIALIZED;
int g_device = -1;
DeviceInfo g_info{};

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int fail_hip(hipError_t e, const char* what) {
    return fail(UNILLM_ERR_HIP, std::string(what) + ": " + hipGetErrorName(e) + " (" +
                                    hipGetErrorString(e) + ")");
}

int do_init(int device) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return fail_hip(e, "hipGetDeviceCount");
    if (device < 0 || device >= count)
        return fail(UNILLM_ERR_INVALID_ARG, "device " + std::to_string(device) +
                                                " out of range (have " + std::to_string(count) +
                                                ")");
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess)
        return fail_hip(e, "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(UNILLM_ERR_UNSUPPORTED,
                    std::string("unillm_hip requires gfx950 (MI355X); device reports ") +
                        prop.gcnArchName);
    if ((e = hipSetDevice(device)) != hipSuccess) return fail_hip(e, "hipSetDevice");
    g_info.cu_count = prop.multiProcessorCount;
    g_info.max_lds = (int)prop.sharedMemPerBlock;
    g_info.max_lds_cu = (int)prop.maxSharedMemoryPerMultiProcessor;
    if (g_info.max_lds_cu <= 0) g_info.max_lds_cu = 160 * 1024;
    // workspaces come from the stream-ordered pool: keep freed memory in the
    // pool instead of returning it
    hipMemPool_t pool;
    if (hipDeviceGetDefaultMemPool(&pool, device) == hipSuccess) {
        uint64_t keep = UINT64_MAX;
        (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
    }
    // this GPU's copy of the no-allocation scratch: its device address, once
    void* sp = nullptr;
    if ((e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch))) != hipSuccess)
        return fail_hip(e, "hipGetSymbolAddress (no-allocation scratch)");
    if (!sp) return fail(UNILLM_ERR_HIP, "hipGetSymbolAddress returned no address for scratch");
    // the tickets at its tail start at zero (a device global is zero at load as well)
    if ((e = hipMemset(static_cast<uint8_t*>(sp) + kNoAllocScratchBytes - kNoAllocSyncBytes, 0,
                       kNoAllocSyncBytes)) != hipSuccess ||
        (e = hipDeviceSynchronize()) != hipSuccess)
        return fail_hip(e, "clearing the no-allocation tickets");
    g_scratch_ptr.assign((size_t)count, nullptr);
    g_scratch_ptr[(size_t)device] = sp;
    g_device = device;
    return UNILLM_OK;
}

int ensure_init() {
    if (g_device >= 0) {
        hipError_t e = hipSetDevice(g_device);
        return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipSetDevice");
    }
    std::call_once(g_init_once, [] { g_init_status = do_init(0); });
    return g_init_status;
}

bool valid_qtype(int q) {
    return q == UNILLM_QTYPE_Q4_0 || q == UNILLM_QTYPE_Q5_0 || q == UNILLM_QTYPE_Q8_0 ||
           q == UNILLM_QTYPE_Q4_K || q == UNILLM_QTYPE_Q5_K || q == UNILLM_QTYPE_Q6_K ||
           is_dense(q);
}

int check_shape(int qtype, int64_t n, int64_t k) {
    if (!valid_qtype(qtype))
        return fail(UNILLM_ERR_UNSUPPORTED,
                    "unsupported qtype " + std::to_string(qtype) +
                        " (want 2 = Q4_0, 6 = Q5_0, 8 = Q8_0, 12 = Q4_K, 13 = Q5_K, 14 = Q6_K, or dense 0 = F32, "
                        "1 = F16, 30 = BF16)");
    if (is_dense(qtype)) {
        if (n < 1 || k < 1)
            return fail(UNILLM_ERR_INVALID_ARG, "bad weight shape [" + std::to_string(n) + ", " +
                                                    std::to_string(k) + "]: need n, k >= 1");
        if (n > (int64_t)INT32_MAX || k > (int64_t)INT32_MAX)
            return fail(UNILLM_ERR_INVALID_ARG, "weight shape too large");
        return UNILLM_OK;
    }
    const int64_t blk = gguf_block_elems(qtype);
    if (n < 1 || k < blk || k % blk != 0)
        return fail(UNILLM_ERR_INVALID_ARG, "bad weight shape [" + std::to_string(n) + ", " +
                                                std::to_string(k) +
                                                "]: need n >= 1 and k a positive multiple of " +
                                                std::to_string(blk));
    if (n > (int64_t)INT32_MAX || k / QK > (int64_t)INT32_MAX / 4)
        return fail(UNILLM_ERR_INVALID_ARG, "weight shape too large");
    return UNILLM_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// GGUF bytes of an [n, k] tensor of this type
size_t gguf_bytes(int qtype, int64_t n, int64_t k) {
    if (is_dense(qtype)) return (size_t)n * (size_t)k * (size_t)dense_elem_bytes(qtype);
    return (size_t)(n * (k / gguf_block_elems(qtype))) * gguf_block_bytes(qtype);
}

int alloc_weight(int qtype, int64_t n, int64_t k, QWeight** out) {
    QWeight* w = new (std::nothrow) QWeight{};
    if (!w) return fail(UNILLM_ERR_OUT_OF_MEMORY, "host allocation failed");
    // Q5_0 runs as Q8_0 (its int8 codes q - 16 times d): repacked into that frame
    w->qtype = qtype == UNILLM_QTYPE_Q5_0 ? UNILLM_QTYPE_Q8_0 : qtype;
    w->src_qtype = qtype;
    w->device = g_device;
    w->n = n;
    w->k = k;
    w->kb = is_dense(qtype) ? 0 : k / QK;
    w->row_bytes = is_dense(qtype) ? 4 * k : row_bytes_for(w->qtype, w->kb);
    // + a 256-byte tail slot for the scale reduction run at create
    w->bytes = (((size_t)n * (size_t)w->row_bytes + 255) & ~(size_t)255) + 256;
    void* mem = nullptr;
    hipError_t e = hipMalloc(&mem, w->bytes);
    if (e != hipSuccess) {
        delete w;
        return e == hipErrorOutOfMemory ? fail(UNILLM_ERR_OUT_OF_MEMORY, "hipMalloc of weight")
                                        : fail_hip(e, "hipMalloc");
    }
    w->base = static_cast<uint8_t*>(mem);
    // row padding is never read as data; zero it anyway so device memory
    // holds only defined bytes
    if ((e = hipMemset(mem, 0, w->bytes)) != hipSuccess) {
        (void)hipFree(mem);
        delete w;
        return fail_hip(e, "hipMemset");
    }
    *out = w;
    return UNILLM_OK;
}

// After repack: find max|d| and the f16 exponent offset E the decode MFMA path
// applies, so that every (q - 8) * d * 2^-E (or q * d * 2^-E) fits f16.
// Synchronises `s`.
int finish_weight(QWeight* w, hipStream_t s) {
    uint32_t* slot = reinterpret_cast<uint32_t*>(w->base + w->bytes - 256);
    uint32_t bits[2] = {0, 0};
    hipError_t e;
    if (is_dense(w->qtype)) {  // f32 rows: no scales to range
        w->f16_exp = 0;
        if ((e = hipStreamSynchronize(s)) != hipSuccess) return fail_hip(e, "weight upload");
        return UNILLM_OK;
    }
    if ((e = hipMemsetAsync(slot, 0, sizeof(bits), s)) != hipSuccess)
        return fail_hip(e, "hipMemsetAsync");
    if ((e = launch_scale_absmax(*w, slot, s)) != hipSuccess) return fail_hip(e, "scale scan");
    if ((e = hipMemcpyAsync(bits, slot, sizeof(bits), hipMemcpyDeviceToHost, s)) != hipSuccess)
        return fail_hip(e, "hipMemcpyAsync");
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return fail_hip(e, "weight upload");
    auto f16max = [](uint32_t b) {  // finite f16 magnitude bits -> float (inf/nan clamp to max)
        return __half2float(__ushort_as_half((unsigned short)(b > 0x7BFFu ? 0x7BFFu : b)));
    };
    // |code| <= 8 (Q4_0) or 128 (Q8_0); Q4_K: |(d sc) q - dmin m| <= 63 (15 |d| + |dmin|);
    // Q5_K: 63 (31 |d| + |dmin|); Q6_K: |(d sc)(q - 32)| <= 128 * 32 |d|; f16 holds
    // magnitudes up to 65504
    const float wmax = w->qtype == UNILLM_QTYPE_Q4_K   ? 63.0f * (15.0f * f16max(bits[0]) + f16max(bits[1]))
                       : w->qtype == UNILLM_QTYPE_Q5_K ? 63.0f * (31.0f * f16max(bits[0]) + f16max(bits[1]))
                       : w->qtype == UNILLM_QTYPE_Q6_K ? 4096.0f * f16max(bits[0])
                       : f16max(bits[0]) * (w->qtype == UNILLM_QTYPE_Q4_0        ? 8.0f
                                            : w->src_qtype == UNILLM_QTYPE_Q5_0 ? 16.0f
                                                                                : 128.0f);
    // the largest power-of-two scaling that keeps every dequantized weight in
    // f16 range: small scales stay normal in f16 (also divided by 16)
    int E = 0;
    while (E < 30 && wmax * ldexpf(1.0f, -E) > 65504.0f) ++E;
    while (wmax > 0.0f && E > -30 && wmax * ldexpf(1.0f, -(E - 1)) <= 65504.0f) --E;
    w->f16_exp = E;
    return UNILLM_OK;
}

// stream -> workspace: see stream_workspace
struct StreamWs {
    void* buf = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::map<std::pair<hipStream_t, int>, StreamWs> g_ws;
// Buffers a workspace has outgrown.  A graph captured while one of them was
// current still reads and writes it at every replay, so none is ever freed;
// growth at least doubles a slot, so they add up to less than the slot itself.
std::vector<void*> g_ws_retired;
thread_local size_t g_ws_capture_need = 0;  // size a capture-time growth asked for

}  // namespace

const DeviceInfo& device_info() { return g_info; }

hipError_t stream_workspace(hipStream_t s, size_t bytes, void** out, int slot) {
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    StreamWs& w = g_ws[{s, slot}];
    if (w.bytes < bytes) {
        // Growing allocates: refused while s is being captured (the allocation and
        // the buffer it replaces would belong to the graph, not to later eager calls)
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        hipError_t e = hipStreamIsCapturing(s, &cs);
        if (e != hipSuccess) return e;
        if (cs != hipStreamCaptureStatusNone) {
            g_ws_capture_need = bytes;
            return hipErrorStreamCaptureUnsupported;
        }
        // Grow in stream order: work on s already issued keeps the old buffer, later
        // work uses the new one.  The old buffer is retired, never freed.
        const size_t want = std::max({bytes, (size_t)1 << 20, 2 * w.bytes});
        void* nb = nullptr;
        if ((e = hipMallocAsync(&nb, want, s)) != hipSuccess) return e;
        // the tickets start at zero (never under capture: growth is refused there)
        if (slot == kSyncSlot && (e = hipMemsetAsync(nb, 0, want, s)) != hipSuccess) return e;
        if (w.buf) g_ws_retired.push_back(w.buf);
        w.buf = nb;
        w.bytes = want;
    }
    *out = w.buf;
    return hipSuccess;
}


bool debug_launch() {
    static const bool on = [] {
        const char* e = getenv("UNILLM_DEBUG_LAUNCH");
        return e && e[0] == '1';
    }();
    return on;
}

}  // namespace unillm

using namespace unillm;

extern "C" {

int unillm_hip_init(int device) {
    int rc = UNILLM_OK;
    std::call_once(g_init_once, [&] { g_init_status = do_init(device); });
    rc = g_init_status;
    if (rc == UNILLM_OK && device != g_device)
        return fail(UNILLM_ERR_INVALID_ARG, "already initialised on device " +
                                                std::to_string(g_device));
    return rc;
}

const char* unillm_hip_last_error(void) { return g_last_error.c_str(); }

int unillm_hip_qweight_create(int qtype, int64_t n, int64_t k, const void* host_blocks,
                              size_t nbytes, int layout_flags, unillm_qweight** out) {
    if (!out) return fail(UNILLM_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (int rc = check_shape(qtype, n, k)) return rc;
    if (!host_blocks) return fail(UNILLM_ERR_INVALID_ARG, "host_blocks is NULL");
    if (layout_flags != 0) return fail(UNILLM_ERR_INVALID_ARG, "layout_flags must be 0");
    const size_t want = gguf_bytes(qtype, n, k);
    if (nbytes != want)
        return fail(UNILLM_ERR_INVALID_ARG, "nbytes " + std::to_string(nbytes) + " != " +
                                                std::to_string(want) + " for this shape");
    if (int rc = ensure_init()) return rc;
    void* staging = nullptr;
    hipError_t e = hipMalloc(&staging, want);
    if (e != hipSuccess) return fail_hip(e, "hipMalloc (staging)");
    QWeight* w = nullptr;
    int rc = alloc_weight(qtype, n, k, &w);
    if (rc == UNILLM_OK) {
        if ((e = hipMemcpy(staging, host_blocks, want, hipMemcpyHostToDevice)) != hipSuccess)
            rc = fail_hip(e, "hipMemcpy (upload)");
        else if ((e = is_dense(qtype) ? launch_dense_upload(*w, staging, nullptr)
                                      : launch_repack(*w, static_cast<const uint8_t*>(staging),
                                                      nullptr)) != hipSuccess)
            rc = fail_hip(e, "repack launch");
        else
            rc = finish_weight(w, nullptr);
    }
    (void)hipFree(staging);
    if (rc != UNILLM_OK) {
        if (w) {
            (void)hipFree(w->base);
            delete w;
        }
        return rc;
    }
    *out = w;
    return UNILLM_OK;
}

int unillm_hip_qweight_create_device(int qtype, int64_t n, int64_t k, const void* dev_blocks,
                                     size_t nbytes, int layout_flags, void* stream,
                                     unillm_qweight** out) {
    if (!out) return fail(UNILLM_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (int rc = check_shape(qtype, n, k)) return rc;
    if (!dev_blocks) return fail(UNILLM_ERR_INVALID_ARG, "dev_blocks is NULL");
    if (layout_flags != 0) return fail(UNILLM_ERR_INVALID_ARG, "layout_flags must be 0");
    const size_t want = gguf_bytes(qtype, n, k);
    if (nbytes != want)
        return fail(UNILLM_ERR_INVALID_ARG, "nbytes " + std::to_string(nbytes) + " != " +
                                                std::to_string(want) + " for this shape");
    if (((uintptr_t)dev_blocks & (qtype == UNILLM_QTYPE_F32 ? 3u : 1u)) != 0)
        return fail(UNILLM_ERR_INVALID_ARG, qtype == UNILLM_QTYPE_F32
                                                ? "dev_blocks must be 4-byte aligned"
                                                : "dev_blocks must be 2-byte aligned");
    if (int rc = ensure_init()) return rc;
    QWeight* w = nullptr;
    if (int rc = alloc_weight(qtype, n, k, &w)) return rc;
    hipError_t e = is_dense(qtype) ? launch_dense_upload(*w, dev_blocks, static_cast<hipStream_t>(stream))
                                   : launch_repack(*w, static_cast<const uint8_t*>(dev_blocks),
                                                   static_cast<hipStream_t>(stream));
    int rc = e == hipSuccess ? finish_weight(w, static_cast<hipStream_t>(stream))
                             : fail_hip(e, "repack launch");
    if (rc != UNILLM_OK) {
        (void)hipFree(w->base);
        delete w;
        return rc;
    }
    *out = w;
    return UNILLM_OK;
}

int unillm_hip_qweight_destroy(unillm_qweight* w) {
    if (!w) return UNILLM_OK;
    hipError_t e = hipFree(w->base);
    delete w;
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipFree (weight)");
}

int unillm_hip_qweight_info(const unillm_qweight* w, int* qtype, int64_t* n, int64_t* k,
                            size_t* device_bytes) {
    if (!w) return fail(UNILLM_ERR_INVALID_ARG, "weight is NULL");
    if (qtype) *qtype = w->src_qtype;
    if (n) *n = w->n;
    if (k) *k = w->k;
    if (device_bytes) *device_bytes = w->bytes;
    return UNILLM_OK;
}

int unillm_hip_select_path(const unillm_qweight* w, int64_t m) {
    if (!w || m < 0) return fail(UNILLM_ERR_INVALID_ARG, "bad arguments to select_path");
    if (is_dense(w->qtype)) return UNILLM_PATH_DENSE;
    if (gemv_supports(*w, m)) return UNILLM_PATH_GEMV;
    if (m <= kDecodeMaxM) return UNILLM_PATH_DECODE_MFMA;
    return UNILLM_PATH_PREFILL_MFMA;
}

namespace {

// A failed launch or workspace request as a status: a workspace that would have
// to grow while its stream is being captured gets its own message.
int fail_launch(hipError_t e, const std::string& what) {
    if (e == hipErrorStreamCaptureUnsupported)
        return fail(UNILLM_ERR_UNSUPPORTED,
                    what + ": the stream's workspace must grow to " +
                        std::to_string(g_ws_capture_need) +
                        " bytes, which cannot happen while the stream is being captured; "
                        "reserve it before capture (unillm_hip_qmatmul_reserve / "
                        "unillm_hip_attention_reserve) or make the same call once eagerly");
    return fail_hip(e, what.c_str());
}

// A dense weight's call: the layer norm (if any) into the stream's workspace (slot 0),
// the f32 GEMM, and for SwiGLU the product into slot 1 and the elementwise pass.
int dense_impl(const unillm_qweight* w, const float* x, int64_t m, float* y, int path,
               hipStream_t s, int epi, const NormArgs& norm, const std::string& what,
               void* fixed_ws) {
    if (path != UNILLM_PATH_AUTO && path != UNILLM_PATH_DENSE)
        return fail(UNILLM_ERR_UNSUPPORTED,
                    what + ": a dense (F32 / F16 / BF16) weight takes the dense path only");
    if (fixed_ws)
        return fail(UNILLM_ERR_UNSUPPORTED,
                    what + ": the no-allocation entry point takes quantized weights only "
                           "(the dense path's GEMM library)");
    if (m > (int64_t)INT32_MAX)
        return fail(UNILLM_ERR_INVALID_ARG, what + ": m too large for the f32 GEMM");
    hipError_t e = hipSuccess;
    auto failed = [&](const std::string& where) {
        const std::string d = dense_error();
        if (e == hipErrorUnknown && !d.empty()) return fail(UNILLM_ERR_HIP, what + ": " + d);
        return fail_launch(e, what + ": " + where);
    };
    if (norm.gamma) {
        void* xn = nullptr;
        if ((e = stream_workspace(s, (size_t)m * (size_t)w->k * sizeof(float), &xn, 0)) != hipSuccess)
            return failed("workspace");
        if ((e = launch_norm_rows(x, m, w->k, norm, static_cast<float*>(xn), s)) != hipSuccess)
            return failed("layer norm launch");
        x = static_cast<const float*>(xn);
    }
    float* out = y;
    if (epi == kEpiSwiglu) {
        void* ws = nullptr;
        if ((e = stream_workspace(s, (size_t)m * (size_t)w->n * sizeof(float), &ws, 1)) != hipSuccess)
            return failed("workspace");
        out = static_cast<float*>(ws);
    }
    if ((e = launch_dense(*w, x, m, out, s, epi == kEpiAdd)) != hipSuccess) return failed("f32 GEMM");
    if (out != y && (e = launch_swiglu(out, m, w->n / 2, y, s)) != hipSuccess)
        return failed("SwiGLU launch");
    return UNILLM_OK;
}

// The matmul on `path` with epilogue `epi` (kEpiStore / kEpiAdd; kEpiSwiglu runs
// fused on the GEMV, else as store into the stream's second workspace + swiglu).
// `what` prefixes every error message (the caller's anyhow context).
// fixed_ws != nullptr (the no-allocation entry point, store epilogue only): the MFMA
// paths take their x operand from fixed_ws (fixed_bytes long), and nothing allocates.
int qmatmul_impl(const unillm_qweight* w, const float* x_dev, int64_t m, float* y_dev, int path,
                 void* stream, int epi, const NormArgs& norm = NormArgs{nullptr, nullptr, 0.f},
                 const std::string& what = "QMatMul forward failed", void* fixed_ws = nullptr,
                 size_t fixed_bytes = 0) {
    if (!w) return fail(UNILLM_ERR_INVALID_ARG, what + ": weight is NULL");
    if (m < 0) return fail(UNILLM_ERR_INVALID_ARG, what + ": m < 0");
    if (epi == kEpiSwiglu && w->n % 2 != 0)
        return fail(UNILLM_ERR_INVALID_ARG,
                    what + ": a SwiGLU weight stacks gate and up rows (even n)");
    if (m == 0) return UNILLM_OK;
    if (!x_dev || !y_dev) return fail(UNILLM_ERR_INVALID_ARG, what + ": x or y is NULL");
    if (((uintptr_t)x_dev & 3u) != 0 || ((uintptr_t)y_dev & 3u) != 0)
        return fail(UNILLM_ERR_INVALID_ARG, what + ": x and y must be 4-byte aligned (f32)");
    if (m > (int64_t)INT32_MAX / 2) return fail(UNILLM_ERR_INVALID_ARG, what + ": m too large");
    if (norm.gamma && (!aligned16(norm.gamma) || (norm.beta && !aligned16(norm.beta)) ||
                       !(norm.eps >= 0.0f)))
        return fail(UNILLM_ERR_INVALID_ARG,
                    what + ": norm weight / bias must be 16-byte aligned, eps >= 0");
    if (path == UNILLM_PATH_AUTO && !is_dense(w->qtype)) {
        path = unillm_hip_select_path(w, m);
        // a fused layer norm on the GEMV takes k <= 8192; past it, batched decode
        if (norm.gamma && path == UNILLM_PATH_GEMV && !gemv_supports_norm(*w, m))
            path = UNILLM_PATH_DECODE_MFMA;
    }
    if (norm.gamma && path == UNILLM_PATH_GEMV && !gemv_supports_norm(*w, m))
        return fail(UNILLM_ERR_UNSUPPORTED,
                    what + ": a fused layer norm on the GEMV path takes k <= 8192");
    if ((path == UNILLM_PATH_DECODE_MFMA || path == UNILLM_PATH_PREFILL_MFMA) &&
        !mfma_supports(*w))
        return fail(UNILLM_ERR_UNSUPPORTED,
                    what + ": the MFMA paths take weights under 4 GiB (32-bit byte offsets)");
    if (int rc = ensure_init()) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    if (is_dense(w->qtype)) return dense_impl(w, x_dev, m, y_dev, path, s, epi, norm, what, fixed_ws);
    // x not on a 16-byte boundary (candle takes any contiguous f32): the kernels
    // load x 16 bytes at a time, so it is first copied, stream-ordered, into an
    // aligned workspace (slot 3)
    void* fixed_sync = nullptr;
    if (fixed_ws) {
        if (!aligned16(x_dev))
            return fail(UNILLM_ERR_INVALID_ARG,
                        what + ": the no-allocation entry point takes x 16-byte aligned");
        // the tickets at the scratch's tail, the x operand in the rest
        fixed_bytes -= kNoAllocSyncBytes;
        fixed_sync = static_cast<uint8_t*>(fixed_ws) + fixed_bytes;
        const size_t need = path == UNILLM_PATH_DECODE_MFMA ? decode_workspace_bytes(*w, m, norm)
                            : path == UNILLM_PATH_PREFILL_MFMA ? prefill_call_bytes(*w, m, fixed_bytes)
                                                               : 0;
        if (need > fixed_bytes ||
            (path == UNILLM_PATH_DECODE_MFMA && decode_sync_bytes(*w) > kNoAllocSyncBytes))
            return fail(UNILLM_ERR_UNSUPPORTED,
                        what + ": this call needs " + std::to_string(need) +
                            " bytes of scratch; the no-allocation entry point holds " +
                            std::to_string(fixed_bytes) + " (m * k or n too large)");
    }
    if (!aligned16(x_dev)) {
        void* xa = nullptr;
        const size_t xb = (size_t)m * (size_t)w->k * sizeof(float);
        if ((e = stream_workspace(s, xb, &xa, 3)) != hipSuccess)
            return fail_launch(e, what + ": workspace");
        if ((e = hipMemcpyAsync(xa, x_dev, xb, hipMemcpyDeviceToDevice, s)) != hipSuccess)
            return fail_hip(e, (what + ": staging x").c_str());
        x_dev = static_cast<const float*>(xa);
    }
    float* out = y_dev;
    int run_epi = epi;
    if (epi == kEpiSwiglu && !(path == UNILLM_PATH_GEMV && gemv_supports_swiglu(*w, m))) {
        void* ws = nullptr;
        e = stream_workspace(s, (size_t)m * (size_t)w->n * sizeof(float), &ws, 1);
        if (e != hipSuccess) return fail_launch(e, what + ": workspace");
        out = static_cast<float*>(ws);
        run_epi = kEpiStore;
    }
    switch (path) {
        case UNILLM_PATH_GEMV:
            if (!gemv_supports(*w, m))
                return fail(UNILLM_ERR_UNSUPPORTED,
                            what + ": GEMV path takes m <= 4, k <= " +
                                std::to_string(gemv_max_kb(m, w->qtype) * QK) +
                                " at this m and weights under 4 GiB");
            e = launch_gemv(*w, x_dev, m, out, s, run_epi, norm);
            break;
        case UNILLM_PATH_DECODE_MFMA:
            if (m > kDecodeMaxM)
                return fail(UNILLM_ERR_UNSUPPORTED, what + ": decode MFMA path takes m <= 64");
            e = launch_decode_mfma(*w, x_dev, m, out, s, run_epi, norm, fixed_ws, fixed_sync);
            break;
        case UNILLM_PATH_PREFILL_MFMA:
            e = launch_prefill_mfma(*w, x_dev, m, out, s, run_epi, norm, fixed_ws, fixed_bytes);
            break;
        default:
            return fail(UNILLM_ERR_INVALID_ARG, what + ": unknown path " + std::to_string(path));
    }
    if (e == hipSuccess && out != y_dev) e = launch_swiglu(out, m, w->n / 2, y_dev, s);
    return e == hipSuccess ? UNILLM_OK : fail_launch(e, what + ": kernel launch");
}

}  // namespace

int unillm_hip_qmatmul_path(const unillm_qweight* w, const float* x_dev, int64_t m,
                            float* y_dev, int path, void* stream) {
    return qmatmul_impl(w, x_dev, m, y_dev, path, stream, kEpiStore);
}

int unillm_hip_qmatmul_add(const unillm_qweight* w, const float* x_dev, int64_t m, float* y_dev,
                           void* stream) {
    return qmatmul_impl(w, x_dev, m, y_dev, UNILLM_PATH_AUTO, stream, kEpiAdd);
}

int unillm_hip_qmatmul_swiglu(const unillm_qweight* w, const float* x_dev, int64_t m,
                              float* act_dev, void* stream) {
    return qmatmul_impl(w, x_dev, m, act_dev, UNILLM_PATH_AUTO, stream, kEpiSwiglu);
}

int unillm_hip_qmatmul_norm(const unillm_qweight* w, const float* x_dev, const float* gamma_dev,
                            const float* beta_dev, float eps, int64_t m, float* y_dev,
                            void* stream) {
    if (!gamma_dev) return fail(UNILLM_ERR_INVALID_ARG, "QMatMul forward failed: gamma is NULL");
    return qmatmul_impl(w, x_dev, m, y_dev, UNILLM_PATH_AUTO, stream, kEpiStore,
                        NormArgs{gamma_dev, beta_dev, eps});
}

int unillm_hip_qmatmul_norm_swiglu(const unillm_qweight* w, const float* x_dev,
                                   const float* gamma_dev, const float* beta_dev, float eps,
                                   int64_t m, float* act_dev, void* stream) {
    if (!gamma_dev) return fail(UNILLM_ERR_INVALID_ARG, "QMatMul forward failed: gamma is NULL");
    return qmatmul_impl(w, x_dev, m, act_dev, UNILLM_PATH_AUTO, stream, kEpiSwiglu,
                        NormArgs{gamma_dev, beta_dev, eps});
}

int unillm_hip_qmatmul(const unillm_qweight* w, const float* x_dev, int64_t m, float* y_dev,
                       void* stream) {
    return unillm_hip_qmatmul_path(w, x_dev, m, y_dev, UNILLM_PATH_AUTO, stream);
}

int unillm_hip_qmatmul_noalloc(const unillm_qweight* w, const float* x_dev, int64_t m,
                               float* y_dev, void* stream) {
    if (int rc = ensure_init()) return rc;
    void* sp = (size_t)g_device < g_scratch_ptr.size() ? g_scratch_ptr[(size_t)g_device] : nullptr;
    if (!sp) return fail(UNILLM_ERR_NOT_INITIALIZED, "no-allocation scratch has no device address");
    return qmatmul_impl(w, x_dev, m, y_dev, UNILLM_PATH_AUTO, stream, kEpiStore,
                        NormArgs{nullptr, nullptr, 0.f}, "QMatMul forward failed", sp,
                        kNoAllocScratchBytes);
}

int unillm_hip_qmatmul_reserve(const unillm_qweight* w, int64_t m, int swiglu, void* stream) {
    if (!w || m < 0) return fail(UNILLM_ERR_INVALID_ARG, "reserve: weight is NULL or m < 0");
    if (m == 0) return UNILLM_OK;
    if (m > (int64_t)INT32_MAX / 2) return fail(UNILLM_ERR_INVALID_ARG, "reserve: m too large");
    if (int rc = ensure_init()) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (is_dense(w->qtype)) {
        // the f32 GEMM's handle, slot 0 (a fused norm's rows), slot 1 (SwiGLU's product)
        void* p = nullptr;
        hipError_t e = dense_prepare(s);
        if (e == hipSuccess)
            e = stream_workspace(s, (size_t)m * (size_t)w->k * sizeof(float), &p, 0);
        if (e == hipSuccess && swiglu)
            e = stream_workspace(s, (size_t)m * (size_t)w->n * sizeof(float), &p, 1);
        return e == hipSuccess ? UNILLM_OK : fail_launch(e, "reserve");
    }
    // slot 0: the x operand of either MFMA path at any m' <= m (both sizes grow with m;
    // the batched decode's with a fused norm bounds the one without)
    const float unused_gamma = 0.0f;
    const NormArgs any_norm{&unused_gamma, nullptr, 0.0f};
    const size_t x0 =
        std::max(decode_workspace_bytes(*w, std::min<int64_t>(m, kDecodeMaxM), any_norm),
                 prefill_workspace_bytes(*w, m));
    void* p = nullptr;
    hipError_t e = stream_workspace(s, x0, &p, 0);
    // the batched decode's arrival tickets
    if (e == hipSuccess) e = stream_workspace(s, decode_sync_bytes(*w), &p, kSyncSlot);
    // slot 1: the [gate | up] product of a SwiGLU call off the GEMV path
    if (e == hipSuccess && swiglu)
        e = stream_workspace(s, (size_t)m * (size_t)w->n * sizeof(float), &p, 1);
    // slot 3: the aligned copy of an x that sits only on a 4-byte boundary (any path)
    if (e == hipSuccess) e = stream_workspace(s, (size_t)m * (size_t)w->k * sizeof(float), &p, 3);
    return e == hipSuccess ? UNILLM_OK : fail_launch(e, "reserve");
}

int unillm_hip_attention_reserve(const unillm_kv_cache* c, int64_t m, int64_t n_heads,
                                 void* stream) {
    if (!c || m < 1 || n_heads < c->n_kv_heads || n_heads % c->n_kv_heads != 0)
        return fail(UNILLM_ERR_INVALID_ARG,
                    "attention reserve: need a cache, m >= 1 and n_heads a multiple of n_kv_heads");
    if (int rc = ensure_init()) return rc;
    void* p = nullptr;
    hipError_t e = stream_workspace(static_cast<hipStream_t>(stream),
                                    attention_workspace_bytes(*c, m, n_heads), &p, 2);
    return e == hipSuccess ? UNILLM_OK : fail_launch(e, "attention reserve");
}

int unillm_hip_dequant(const unillm_qweight* w, float* out_dev, void* stream) {
    if (!w || !out_dev) return fail(UNILLM_ERR_INVALID_ARG, "weight or out is NULL");
    if (!aligned16(out_dev)) return fail(UNILLM_ERR_INVALID_ARG, "out must be 16-byte aligned");
    if (int rc = ensure_init()) return rc;
    hipError_t e = is_dense(w->qtype)
                       ? hipMemcpyAsync(out_dev, w->base, (size_t)w->n * (size_t)w->k * sizeof(float),
                                        hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream))
                       : launch_dequant(*w, out_dev, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "dequant launch");
}

int unillm_hip_quantize(int qtype, const float* w_dev, int64_t n, int64_t k, void* blocks_dev,
                        void* stream) {
    if (int rc = check_shape(qtype, n, k)) return rc;
    if (is_kquant(qtype) || is_dense(qtype))
        return fail(UNILLM_ERR_UNSUPPORTED, "the device quantizer covers Q4_0 and Q8_0 only");
    if (!w_dev || !blocks_dev) return fail(UNILLM_ERR_INVALID_ARG, "w or blocks is NULL");
    if (!aligned16(w_dev)) return fail(UNILLM_ERR_INVALID_ARG, "w must be 16-byte aligned");
    if (int rc = ensure_init()) return rc;
    hipError_t e = launch_quantize(qtype, w_dev, n, k, static_cast<uint8_t*>(blocks_dev),
                                   static_cast<hipStream_t>(stream));
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "quantize launch");
}

int unillm_hip_kv_cache_create(int64_t n_kv_heads, int64_t head_dim, int64_t max_seq,
                               float rope_theta, unillm_kv_cache** out) {
    if (!out) return fail(UNILLM_ERR_INVALID_ARG, "out is NULL");
    *out = nullptr;
    if (n_kv_heads < 1 || max_seq < 1 || !(head_dim == 64 || head_dim == 128 || head_dim == 256) ||
        !(rope_theta > 0.0f) || n_kv_heads * max_seq * head_dim > ((int64_t)1 << 31))
        return fail(UNILLM_ERR_INVALID_ARG,
                    "KV cache: need n_kv_heads >= 1, head_dim 64 / 128 / 256, max_seq >= 1, "
                    "rope_theta > 0 and under 2^31 elements per buffer");
    if (int rc = ensure_init()) return rc;
    unillm_kv_cache* c = new (std::nothrow) unillm_kv_cache{};
    if (!c) return fail(UNILLM_ERR_OUT_OF_MEMORY, "host allocation failed");
    c->device = g_device;
    c->n_kv_heads = n_kv_heads;
    c->head_dim = head_dim;
    c->max_seq = max_seq;
    c->rope_theta = rope_theta;
    const size_t buf = (size_t)(n_kv_heads * max_seq * head_dim) * sizeof(float);
    // inv_freq[i] = 1 / theta^(2 i / hd) in f32, as apply_rope_with_offset computes it
    // (crates/runtime/src/models_v2/llama.rs:839-841)
    std::vector<float> inv((size_t)head_dim / 2);
    for (size_t i = 0; i < inv.size(); ++i)
        inv[i] = 1.0f / powf(rope_theta, (float)(2 * i) / (float)head_dim);
    hipError_t e;
    void *k = nullptr, *v = nullptr, *f = nullptr, *st = nullptr;
    if ((e = hipMalloc(&k, buf)) != hipSuccess || (e = hipMalloc(&v, buf)) != hipSuccess ||
        (e = hipMalloc(&f, inv.size() * sizeof(float))) != hipSuccess ||
        (e = hipMalloc(&st, 4 * sizeof(int))) != hipSuccess ||
        (e = hipMemset(k, 0, buf)) != hipSuccess || (e = hipMemset(v, 0, buf)) != hipSuccess ||
        (e = hipMemset(st, 0, 4 * sizeof(int))) != hipSuccess ||
        (e = hipMemcpy(f, inv.data(), inv.size() * sizeof(float), hipMemcpyHostToDevice)) !=
            hipSuccess) {
        (void)hipFree(k);
        (void)hipFree(v);
        (void)hipFree(f);
        (void)hipFree(st);
        delete c;
        return e == hipErrorOutOfMemory ? fail(UNILLM_ERR_OUT_OF_MEMORY, "KV cache allocation")
                                        : fail_hip(e, "KV cache allocation");
    }
    c->k = static_cast<float*>(k);
    c->v = static_cast<float*>(v);
    c->inv_freq = static_cast<float*>(f);
    c->state = static_cast<int*>(st);
    *out = c;
    return UNILLM_OK;
}

int unillm_hip_kv_cache_destroy(unillm_kv_cache* c) {
    if (!c) return UNILLM_OK;
    hipError_t e = hipFree(c->k), e2 = hipFree(c->v), e3 = hipFree(c->inv_freq),
               e4 = hipFree(c->state);
    delete c;
    if (e == hipSuccess) e = e2;
    if (e == hipSuccess) e = e3;
    if (e == hipSuccess) e = e4;
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipFree (KV cache)");
}

namespace {
// The cache's device state after all work issued so far on `s` (s == nullptr and
// device_wide: after all work on the device): refreshes the host's copy of the length.
// A replayed call that overflowed is reported with the reference's message, unless
// report_overflow is false (a truncate, which clears the flag, reads the length only).
int refresh_length(unillm_kv_cache* c, hipStream_t s, bool device_wide,
                   bool report_overflow = true) {
    int st[2] = {0, 0};
    hipError_t e = device_wide ? hipDeviceSynchronize() : hipSuccess;
    if (e == hipSuccess) e = hipMemcpyAsync(st, c->state, sizeof(st), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail_hip(e, "KV cache: reading the device length");
    c->len = st[0];
    // once a call on this cache has been captured, replays may run at any time
    // between calls: the host copy is read back before every later use
    c->len_stale = c->captured;
    if (st[1] && report_overflow)
        return fail(UNILLM_ERR_INVALID_ARG,
                    "KV cache append failed: KV cache overflow in a replayed call: current_len=" +
                        std::to_string(st[0]) + ", max_seq_len=" + std::to_string(c->max_seq));
    return UNILLM_OK;
}

// Sets the device length (and clears the overflow flag) once all device work is done.
int set_length(unillm_kv_cache* c, int64_t len) {
    const int st[3] = {(int)len, 0, (int)len};
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(c->state, st, sizeof(st), hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail_hip(e, "KV cache: setting the device length");
    c->len = len;
    c->len_stale = c->captured;
    return UNILLM_OK;
}
}  // namespace

int unillm_hip_kv_cache_length(const unillm_kv_cache* c, int64_t* len) {
    if (!c || !len) return fail(UNILLM_ERR_INVALID_ARG, "cache or len is NULL");
    if (c->len_stale) {
        if (int rc = refresh_length(const_cast<unillm_kv_cache*>(c), nullptr, true)) return rc;
    }
    *len = c->len;
    return UNILLM_OK;
}

int unillm_hip_kv_cache_clear(unillm_kv_cache* c) {
    if (!c) return fail(UNILLM_ERR_INVALID_ARG, "cache is NULL");
    return set_length(c, 0);
}

int unillm_hip_kv_cache_truncate(unillm_kv_cache* c, int64_t len) {
    if (!c) return fail(UNILLM_ERR_INVALID_ARG, "cache is NULL");
    // a replay that overflowed appended nothing: the length it left is intact, and
    // set_length below clears the flag, so truncating recovers the prefix
    if (c->len_stale) {
        if (int rc = refresh_length(c, nullptr, true, false)) return rc;
    }
    if (len < 0 || len > c->len)
        return fail(UNILLM_ERR_INVALID_ARG, "KV cache truncate: length " + std::to_string(len) +
                                                " outside [0, " + std::to_string(c->len) + "]");
    return set_length(c, len);
}

int unillm_hip_attention_decode(unillm_kv_cache* c, const float* qkv_dev, int64_t m,
                                int64_t n_heads, float* out_dev, void* stream) {
    if (!c || !qkv_dev || !out_dev)
        return fail(UNILLM_ERR_INVALID_ARG, "attention: cache, qkv or out is NULL");
    if (m < 1 || n_heads < c->n_kv_heads || n_heads % c->n_kv_heads != 0)
        return fail(UNILLM_ERR_INVALID_ARG,
                    "attention: need m >= 1 and n_heads a multiple of n_kv_heads");
    if (((uintptr_t)qkv_dev & 15u) != 0 || ((uintptr_t)out_dev & 3u) != 0)
        return fail(UNILLM_ERR_INVALID_ARG, "attention: qkv must be 16-byte aligned, out 4-byte");
    if (int rc = ensure_init()) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s, &cs);
    if (e != hipSuccess) return fail_hip(e, "attention: hipStreamIsCapturing");
    const bool capturing = cs != hipStreamCaptureStatusNone;
    const bool decode = m * (n_heads / c->n_kv_heads) <= attention_max_queries();
    // the prompt kernels store out 16 bytes at a time
    if (!decode && !aligned16(out_dev))
        return fail(UNILLM_ERR_INVALID_ARG,
                    "attention: a prompt-length call (more than " +
                        std::to_string(attention_max_queries()) +
                        " queries a kv head) takes out 16-byte aligned");
    if (capturing) {
        // the kernels read the length from the device at each replay: the grid covers
        // the longest the cache holds, and the host's copy is unknown afterwards
        if (decode && c->max_seq > attention_max_positions())
            return fail(UNILLM_ERR_UNSUPPORTED,
                        "attention: a captured decode step covers at most " +
                            std::to_string(attention_max_positions()) + " cache positions");
        e = launch_attention(*c, qkv_dev, m, n_heads, out_dev, -1, s);
        if (e != hipSuccess) return fail_launch(e, "attention launch");
        c->captured = true;
        c->len_stale = true;
        return UNILLM_OK;
    }
    if (c->len_stale) {
        if (int rc = refresh_length(c, s, false)) return rc;
    }
    if (c->len + m > c->max_seq)  // LayerKVCache::append's check (kv_cache.rs:114-121)
        return fail(UNILLM_ERR_INVALID_ARG,
                    "KV cache append failed: KV cache overflow: current_len=" +
                        std::to_string(c->len) + ", new_len=" + std::to_string(m) +
                        ", max_seq_len=" + std::to_string(c->max_seq));
    if (decode && c->len + m > attention_max_positions())
        return fail(UNILLM_ERR_UNSUPPORTED, "attention: len + m must be <= " +
                                                std::to_string(attention_max_positions()) +
                                                " on a decode step");
    e = launch_attention(*c, qkv_dev, m, n_heads, out_dev, c->len, s);
    if (e != hipSuccess) return fail_launch(e, "attention launch");
    c->len += m;  // the kernels advance the device copy in stream order
    return UNILLM_OK;
}

int unillm_hip_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail(UNILLM_ERR_INVALID_ARG, "ptr is NULL");
    if (int rc = ensure_init()) return rc;
    hipError_t e = hipMalloc(ptr, bytes);
    if (e == hipErrorOutOfMemory) return fail(UNILLM_ERR_OUT_OF_MEMORY, "hipMalloc");
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipMalloc");
}

int unillm_hip_free(void* ptr) {
    hipError_t e = hipFree(ptr);
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipFree");
}

int unillm_hip_memcpy_htod(void* dst_dev, const void* src_host, size_t bytes) {
    if (int rc = ensure_init()) return rc;
    hipError_t e = hipMemcpy(dst_dev, src_host, bytes, hipMemcpyHostToDevice);
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipMemcpy H2D");
}

int unillm_hip_memcpy_dtoh(void* dst_host, const void* src_dev, size_t bytes) {
    if (int rc = ensure_init()) return rc;
    hipError_t e = hipMemcpy(dst_host, src_dev, bytes, hipMemcpyDeviceToHost);
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipMemcpy D2H");
}

int unillm_hip_synchronize(void) {
    if (int rc = ensure_init()) return rc;
    hipError_t e = hipDeviceSynchronize();
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipDeviceSynchronize");
}

int unillm_hip_stream_create(void** stream) {
    if (!stream) return fail(UNILLM_ERR_INVALID_ARG, "stream is NULL");
    *stream = nullptr;
    if (int rc = ensure_init()) return rc;
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);  // default priority
    if (e != hipSuccess) return fail_hip(e, "hipStreamCreate");
    *stream = s;
    return UNILLM_OK;
}

int unillm_hip_stream_destroy(void* stream) {
    if (!stream) return UNILLM_OK;
    hipError_t e = hipStreamDestroy(static_cast<hipStream_t>(stream));
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipStreamDestroy");
}

int unillm_hip_stream_synchronize(void* stream) {
    if (int rc = ensure_init()) return rc;
    hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipStreamSynchronize");
}

int unillm_hip_graph_begin(void* stream) {
    if (!stream)
        return fail(UNILLM_ERR_INVALID_ARG, "graph capture needs a stream (not the null stream)");
    if (int rc = ensure_init()) return rc;
    // thread-local mode: other threads' HIP calls do not invalidate the capture
    hipError_t e = hipStreamBeginCapture(static_cast<hipStream_t>(stream),
                                         hipStreamCaptureModeThreadLocal);
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipStreamBeginCapture");
}

int unillm_hip_graph_end(void* stream, unillm_graph** out) {
    if (!stream || !out) return fail(UNILLM_ERR_INVALID_ARG, "stream or out is NULL");
    *out = nullptr;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(static_cast<hipStream_t>(stream), &g);
    if (e != hipSuccess) return fail_hip(e, "hipStreamEndCapture");
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return fail_hip(e, "hipGraphInstantiate");
    *out = reinterpret_cast<unillm_graph*>(x);
    return UNILLM_OK;
}

int unillm_hip_graph_launch(const unillm_graph* g, void* stream) {
    if (!g) return fail(UNILLM_ERR_INVALID_ARG, "graph is NULL");
    hipError_t e = hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(const_cast<unillm_graph*>(g)),
                                  static_cast<hipStream_t>(stream));
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipGraphLaunch");
}

int unillm_hip_graph_destroy(unillm_graph* g) {
    if (!g) return UNILLM_OK;
    hipError_t e = hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(g));
    return e == hipSuccess ? UNILLM_OK : fail_hip(e, "hipGraphExecDestroy");
}

}  // extern "C"
