//! Rust bindings to `libunillm_hip.so`: GGUF quantized matmuls (Q4_0, Q5_0, Q8_0, Q4_K,
//! Q5_K, Q6_K) and KV-cache attention on an MI355X (gfx950).
//!
//! * [`sys`] is the C ABI of `include/unillm_hip.h`, one declaration per function.
//! * [`QuantLinear`] takes the slot of candle's `QMatMul` in the reference's
//!   `ModelWeights.quantized_tensors` (crates/runtime/src/model_core.rs:134), built by
//!   `GGUFWeightLoader` (crates/runtime/src/weight_loader_core.rs:569-571) and called
//!   by `quantized_matmul` / `lm_head_forward` (crates/runtime/src/models_v2/llama.rs:
//!   1184-1195, 396-405).
//! * [`KvCache`] takes the slot of `LayerKVCache` (crates/runtime/src/kv_cache.rs:28-150)
//!   together with the attention of `LlamaAttention::forward_with_cache` after the
//!   projections (llama.rs:1044-1150).
//!
//! No dependencies: errors are [`HipError`], which implements `std::error::Error`, so
//! `?` turns it into the reference's `anyhow::Error`.  Its message is the library's
//! (`"QMatMul forward failed: ..."` for matmul calls, the reference's own context).
//!
//! Device pointers are plain `*const f32` / `*mut f32` into HIP memory: the `_raw`
//! methods are `unsafe` and take them as they are; the safe methods take
//! [`DeviceBuffer`]s and check sizes first.  Streams are `hipStream_t` as
//! `*mut c_void` (null: the default stream); every compute call is asynchronous on it.

use std::ffi::{c_int, c_void, CStr};
use std::fmt;
use std::ptr;

/// The C ABI (`include/unillm_hip.h`).
#[allow(non_camel_case_types)]
pub mod sys {
    use std::ffi::{c_char, c_int, c_void};

    /// Opaque quantized weight handle.
    #[repr(C)]
    pub struct unillm_qweight {
        _private: [u8; 0],
    }
    /// Opaque per-layer KV cache handle.
    #[repr(C)]
    pub struct unillm_kv_cache {
        _private: [u8; 0],
    }
    /// Opaque instantiated HIP graph.
    #[repr(C)]
    pub struct unillm_graph {
        _private: [u8; 0],
    }

    pub const UNILLM_QTYPE_Q4_0: c_int = 2;
    pub const UNILLM_QTYPE_Q8_0: c_int = 8;
    pub const UNILLM_QTYPE_Q5_0: c_int = 6;
    pub const UNILLM_QTYPE_Q4_K: c_int = 12;
    pub const UNILLM_QTYPE_Q5_K: c_int = 13;
    pub const UNILLM_QTYPE_Q6_K: c_int = 14;
    pub const UNILLM_QTYPE_F32: c_int = 0;
    pub const UNILLM_QTYPE_F16: c_int = 1;
    pub const UNILLM_QTYPE_BF16: c_int = 30;

    pub const UNILLM_OK: c_int = 0;
    pub const UNILLM_ERR_INVALID_ARG: c_int = -1;
    pub const UNILLM_ERR_UNSUPPORTED: c_int = -2;
    pub const UNILLM_ERR_HIP: c_int = -3;
    pub const UNILLM_ERR_OUT_OF_MEMORY: c_int = -4;
    pub const UNILLM_ERR_NOT_INITIALIZED: c_int = -5;

    pub const UNILLM_PATH_AUTO: c_int = 0;
    pub const UNILLM_PATH_GEMV: c_int = 1;
    pub const UNILLM_PATH_DECODE_MFMA: c_int = 2;
    pub const UNILLM_PATH_PREFILL_MFMA: c_int = 3;
    pub const UNILLM_PATH_DENSE: c_int = 4;

    extern "C" {
        pub fn unillm_hip_init(device: c_int) -> c_int;
        pub fn unillm_hip_last_error() -> *const c_char;
        pub fn unillm_hip_qweight_create(qtype: c_int, n: i64, k: i64, host_blocks: *const c_void,
                                         nbytes: usize, layout_flags: c_int,
                                         out: *mut *mut unillm_qweight) -> c_int;
        pub fn unillm_hip_qweight_create_device(qtype: c_int, n: i64, k: i64,
                                                dev_blocks: *const c_void, nbytes: usize,
                                                layout_flags: c_int, stream: *mut c_void,
                                                out: *mut *mut unillm_qweight) -> c_int;
        pub fn unillm_hip_qweight_destroy(w: *mut unillm_qweight) -> c_int;
        pub fn unillm_hip_qweight_info(w: *const unillm_qweight, qtype: *mut c_int, n: *mut i64,
                                       k: *mut i64, device_bytes: *mut usize) -> c_int;
        pub fn unillm_hip_qmatmul(w: *const unillm_qweight, x_dev: *const f32, m: i64,
                                  y_dev: *mut f32, stream: *mut c_void) -> c_int;
        pub fn unillm_hip_qmatmul_noalloc(w: *const unillm_qweight, x_dev: *const f32, m: i64,
                                          y_dev: *mut f32, stream: *mut c_void) -> c_int;
        pub fn unillm_hip_qmatmul_path(w: *const unillm_qweight, x_dev: *const f32, m: i64,
                                       y_dev: *mut f32, path: c_int, stream: *mut c_void) -> c_int;
        pub fn unillm_hip_qmatmul_add(w: *const unillm_qweight, x_dev: *const f32, m: i64,
                                      y_dev: *mut f32, stream: *mut c_void) -> c_int;
        pub fn unillm_hip_qmatmul_swiglu(w: *const unillm_qweight, x_dev: *const f32, m: i64,
                                         act_dev: *mut f32, stream: *mut c_void) -> c_int;
        pub fn unillm_hip_qmatmul_norm(w: *const unillm_qweight, x_dev: *const f32,
                                       gamma_dev: *const f32, beta_dev: *const f32, eps: f32,
                                       m: i64, y_dev: *mut f32, stream: *mut c_void) -> c_int;
        pub fn unillm_hip_qmatmul_norm_swiglu(w: *const unillm_qweight, x_dev: *const f32,
                                              gamma_dev: *const f32, beta_dev: *const f32,
                                              eps: f32, m: i64, act_dev: *mut f32,
                                              stream: *mut c_void) -> c_int;
        pub fn unillm_hip_select_path(w: *const unillm_qweight, m: i64) -> c_int;
        pub fn unillm_hip_qmatmul_reserve(w: *const unillm_qweight, m: i64, swiglu: c_int,
                                          stream: *mut c_void) -> c_int;
        pub fn unillm_hip_kv_cache_create(n_kv_heads: i64, head_dim: i64, max_seq: i64,
                                          rope_theta: f32, out: *mut *mut unillm_kv_cache) -> c_int;
        pub fn unillm_hip_kv_cache_destroy(c: *mut unillm_kv_cache) -> c_int;
        pub fn unillm_hip_kv_cache_length(c: *const unillm_kv_cache, len: *mut i64) -> c_int;
        pub fn unillm_hip_kv_cache_clear(c: *mut unillm_kv_cache) -> c_int;
        pub fn unillm_hip_kv_cache_truncate(c: *mut unillm_kv_cache, len: i64) -> c_int;
        pub fn unillm_hip_attention_decode(c: *mut unillm_kv_cache, qkv_dev: *const f32, m: i64,
                                           n_heads: i64, out_dev: *mut f32,
                                           stream: *mut c_void) -> c_int;
        pub fn unillm_hip_attention_reserve(c: *const unillm_kv_cache, m: i64, n_heads: i64,
                                            stream: *mut c_void) -> c_int;
        pub fn unillm_hip_dequant(w: *const unillm_qweight, out_dev: *mut f32,
                                  stream: *mut c_void) -> c_int;
        pub fn unillm_hip_quantize(qtype: c_int, w_dev: *const f32, n: i64, k: i64,
                                   blocks_dev: *mut c_void, stream: *mut c_void) -> c_int;
        pub fn unillm_hip_malloc(ptr: *mut *mut c_void, bytes: usize) -> c_int;
        pub fn unillm_hip_free(ptr: *mut c_void) -> c_int;
        pub fn unillm_hip_memcpy_htod(dst_dev: *mut c_void, src_host: *const c_void,
                                      bytes: usize) -> c_int;
        pub fn unillm_hip_memcpy_dtoh(dst_host: *mut c_void, src_dev: *const c_void,
                                      bytes: usize) -> c_int;
        pub fn unillm_hip_synchronize() -> c_int;
        pub fn unillm_hip_stream_create(stream: *mut *mut c_void) -> c_int;
        pub fn unillm_hip_stream_destroy(stream: *mut c_void) -> c_int;
        pub fn unillm_hip_stream_synchronize(stream: *mut c_void) -> c_int;
        pub fn unillm_hip_graph_begin(stream: *mut c_void) -> c_int;
        pub fn unillm_hip_graph_end(stream: *mut c_void, out: *mut *mut unillm_graph) -> c_int;
        pub fn unillm_hip_graph_launch(g: *const unillm_graph, stream: *mut c_void) -> c_int;
        pub fn unillm_hip_graph_destroy(g: *mut unillm_graph) -> c_int;
    }
}

// ---- errors ------------------------------------------------------------------------------

/// A failed call: the status code (`sys::UNILLM_ERR_*`) and the library's message.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct HipError {
    pub code: i32,
    pub message: String,
}

impl fmt::Display for HipError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.write_str(&self.message)
    }
}

impl std::error::Error for HipError {}

pub type Result<T> = std::result::Result<T, HipError>;

fn check(rc: c_int) -> Result<()> {
    if rc == sys::UNILLM_OK {
        return Ok(());
    }
    // SAFETY: the library returns a NUL-terminated string owned by the calling thread,
    // valid until its next call on that thread.
    let p = unsafe { sys::unillm_hip_last_error() };
    let message = if p.is_null() {
        format!("unillm_hip error {rc}")
    } else {
        unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
    };
    Err(HipError { code: rc, message })
}

fn invalid(message: String) -> HipError {
    HipError { code: sys::UNILLM_ERR_INVALID_ARG, message }
}

fn to_i64(v: usize, what: &str) -> Result<i64> {
    i64::try_from(v).map_err(|_| invalid(format!("{what} {v} does not fit in i64")))
}

/// Selects and initialises the device (once per process; later calls must name the same one).
pub fn init(device: i32) -> Result<()> {
    check(unsafe { sys::unillm_hip_init(device) })
}

/// Waits for all work on the device.
pub fn synchronize() -> Result<()> {
    check(unsafe { sys::unillm_hip_synchronize() })
}

// ---- device memory -------------------------------------------------------------------------

/// HIP device memory owned through the library's allocator: the storage a `HipStorage`
/// (the reference's `TensorStorage`, crates/runtime/src/tensor_core.rs:47-70) would hold.
#[derive(Debug)]
pub struct DeviceBuffer {
    ptr: *mut c_void,
    bytes: usize,
}

// SAFETY: the buffer is plain device memory; moving the owner between threads is fine.
unsafe impl Send for DeviceBuffer {}

impl DeviceBuffer {
    pub fn new(bytes: usize) -> Result<Self> {
        let mut ptr = ptr::null_mut();
        if bytes > 0 {
            check(unsafe { sys::unillm_hip_malloc(&mut ptr, bytes) })?;
        }
        Ok(Self { ptr, bytes })
    }

    /// A buffer holding `data` (a synchronous copy).
    pub fn from_f32(data: &[f32]) -> Result<Self> {
        let b = Self::new(std::mem::size_of_val(data))?;
        if b.bytes > 0 {
            check(unsafe {
                sys::unillm_hip_memcpy_htod(b.ptr, data.as_ptr() as *const c_void, b.bytes)
            })?;
        }
        Ok(b)
    }

    /// The buffer's contents as f32 (waits for the device).
    pub fn to_f32(&self) -> Result<Vec<f32>> {
        let mut out = vec![0.0f32; self.bytes / 4];
        if !out.is_empty() {
            check(unsafe {
                sys::unillm_hip_memcpy_dtoh(out.as_mut_ptr() as *mut c_void, self.ptr, out.len() * 4)
            })?;
        }
        Ok(out)
    }

    pub fn len_bytes(&self) -> usize {
        self.bytes
    }
    pub fn len_f32(&self) -> usize {
        self.bytes / 4
    }
    pub fn as_ptr(&self) -> *const f32 {
        self.ptr as *const f32
    }
    pub fn as_mut_ptr(&mut self) -> *mut f32 {
        self.ptr as *mut f32
    }
}

impl Drop for DeviceBuffer {
    fn drop(&mut self) {
        if !self.ptr.is_null() {
            unsafe {
                sys::unillm_hip_free(self.ptr);
            }
        }
    }
}

// ---- the quantized projection --------------------------------------------------------------

/// GGUF tensor types the device takes (ggml type ids): the block types, and the dense
/// F32 / F16 / BF16 that candle keeps as a dequantized f32 QMatMul.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
#[allow(non_camel_case_types)]
pub enum QType {
    Q4_0 = 2,
    Q5_0 = 6,
    Q8_0 = 8,
    Q4_K = 12,
    Q5_K = 13,
    Q6_K = 14,
    F32 = 0,
    F16 = 1,
    BF16 = 30,
}

impl QType {
    /// From a ggml type id (candle's `GgmlDType` as matched at weight_loader_core.rs:479-483).
    pub fn from_ggml(id: u32) -> Option<Self> {
        match id {
            2 => Some(Self::Q4_0),
            6 => Some(Self::Q5_0),
            8 => Some(Self::Q8_0),
            12 => Some(Self::Q4_K),
            13 => Some(Self::Q5_K),
            14 => Some(Self::Q6_K),
            0 => Some(Self::F32),
            1 => Some(Self::F16),
            30 => Some(Self::BF16),
            _ => None,
        }
    }
}

/// Which kernel a call runs (`sys::UNILLM_PATH_*`); `Auto` lets the library choose by m.
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Path {
    Auto = 0,
    Gemv = 1,
    DecodeMfma = 2,
    PrefillMfma = 3,
    Dense = 4,
}

/// One GGUF weight [n, k] resident on the device; immutable after creation, so shared
/// across threads like the reference's `Arc<QMatMul>`.
#[derive(Debug)]
pub struct QuantLinear {
    w: *mut sys::unillm_qweight,
    qtype: QType,
    n: usize,
    k: usize,
}

// SAFETY: the handle is immutable after create (the C ABI's contract); concurrent
// calls on different streams only read it.
unsafe impl Send for QuantLinear {}
unsafe impl Sync for QuantLinear {}

impl QuantLinear {
    /// Uploads GGUF block bytes (`QTensor::data()` of a tensor of shape [n, k]).
    pub fn from_gguf_blocks(qtype: QType, n: usize, k: usize, raw: &[u8]) -> Result<Self> {
        let mut w = ptr::null_mut();
        check(unsafe {
            sys::unillm_hip_qweight_create(qtype as c_int, to_i64(n, "n")?, to_i64(k, "k")?,
                                           raw.as_ptr() as *const c_void, raw.len(), 0, &mut w)
        })?;
        Ok(Self { w, qtype, n, k })
    }

    pub fn n(&self) -> usize {
        self.n
    }
    pub fn k(&self) -> usize {
        self.k
    }
    pub fn qtype(&self) -> QType {
        self.qtype
    }
    pub fn handle(&self) -> *const sys::unillm_qweight {
        self.w
    }

    /// Device bytes the handle holds (its repacked blocks).
    pub fn device_bytes(&self) -> Result<usize> {
        let (mut q, mut n, mut k, mut bytes) = (0 as c_int, 0i64, 0i64, 0usize);
        check(unsafe { sys::unillm_hip_qweight_info(self.w, &mut q, &mut n, &mut k, &mut bytes) })?;
        Ok(bytes)
    }

    /// The kernel path a call of m rows runs.
    pub fn select_path(&self, m: usize) -> Result<Path> {
        let p = unsafe { sys::unillm_hip_select_path(self.w, to_i64(m, "m")?) };
        match p {
            1 => Ok(Path::Gemv),
            2 => Ok(Path::DecodeMfma),
            3 => Ok(Path::PrefillMfma),
            4 => Ok(Path::Dense),
            _ => check(p).map(|_| Path::Auto),
        }
    }

    /// Grows `stream`'s workspace for calls of up to m rows, so they can be captured.
    pub fn reserve(&self, m: usize, swiglu: bool, stream: *mut c_void) -> Result<()> {
        check(unsafe {
            sys::unillm_hip_qmatmul_reserve(self.w, to_i64(m, "m")?, swiglu as c_int, stream)
        })
    }

    /// QMatMul::forward: y[m, n] = x[m, k] . dequant(W)^T.
    ///
    /// # Safety
    /// `x` and `y` point to device memory of m k and m n f32; `stream` is a HIP stream
    /// of the library's device, or null.
    pub unsafe fn forward_raw(&self, x: *const f32, m: usize, y: *mut f32,
                              stream: *mut c_void) -> Result<()> {
        check(sys::unillm_hip_qmatmul(self.w, x, to_i64(m, "m")?, y, stream))
    }

    /// forward_raw on a chosen kernel path.
    ///
    /// # Safety
    /// As [`QuantLinear::forward_raw`].
    pub unsafe fn forward_path_raw(&self, x: *const f32, m: usize, y: *mut f32, path: Path,
                                   stream: *mut c_void) -> Result<()> {
        check(sys::unillm_hip_qmatmul_path(self.w, x, to_i64(m, "m")?, y, path as c_int, stream))
    }

    /// forward_raw with no device allocation (a fixed per-device scratch; calls that
    /// overlap on one device race).
    ///
    /// # Safety
    /// As [`QuantLinear::forward_raw`].
    pub unsafe fn forward_noalloc_raw(&self, x: *const f32, m: usize, y: *mut f32,
                                      stream: *mut c_void) -> Result<()> {
        check(sys::unillm_hip_qmatmul_noalloc(self.w, x, to_i64(m, "m")?, y, stream))
    }

    /// y += x . dequant(W)^T: the residual add after o_proj / down_proj (llama.rs:668, 677).
    ///
    /// # Safety
    /// As [`QuantLinear::forward_raw`]; y holds the residual on entry.
    pub unsafe fn forward_add_raw(&self, x: *const f32, m: usize, y: *mut f32,
                                  stream: *mut c_void) -> Result<()> {
        check(sys::unillm_hip_qmatmul_add(self.w, x, to_i64(m, "m")?, y, stream))
    }

    /// On a [gate; up] handle: act[m, n / 2] = silu(gate) * up (llama.rs:1275-1283).
    ///
    /// # Safety
    /// `x` holds m k f32 and `act` m n / 2 f32 of device memory; `stream` as above.
    pub unsafe fn forward_swiglu_raw(&self, x: *const f32, m: usize, act: *mut f32,
                                     stream: *mut c_void) -> Result<()> {
        check(sys::unillm_hip_qmatmul_swiglu(self.w, x, to_i64(m, "m")?, act, stream))
    }

    /// forward on the layer norm of x along k (ops_fn::layer_norm, tensor_core.rs:973-1008).
    ///
    /// # Safety
    /// As [`QuantLinear::forward_raw`]; `gamma` (and `beta` unless null) hold k device f32.
    pub unsafe fn forward_norm_raw(&self, x: *const f32, gamma: *const f32, beta: *const f32,
                                   eps: f32, m: usize, y: *mut f32,
                                   stream: *mut c_void) -> Result<()> {
        check(sys::unillm_hip_qmatmul_norm(self.w, x, gamma, beta, eps, to_i64(m, "m")?, y, stream))
    }

    /// forward_swiglu on the layer norm of x: post_attention_layernorm + gate_up + SwiGLU.
    ///
    /// # Safety
    /// As [`QuantLinear::forward_swiglu_raw`] and [`QuantLinear::forward_norm_raw`].
    pub unsafe fn forward_norm_swiglu_raw(&self, x: *const f32, gamma: *const f32,
                                          beta: *const f32, eps: f32, m: usize, act: *mut f32,
                                          stream: *mut c_void) -> Result<()> {
        check(sys::unillm_hip_qmatmul_norm_swiglu(self.w, x, gamma, beta, eps, to_i64(m, "m")?,
                                                  act, stream))
    }

    /// `qtensor.dequantize` (weight_loader_core.rs:579): f32 [n, k], bit-exact with GGML.
    ///
    /// # Safety
    /// `out` holds n k device f32.
    pub unsafe fn dequantize_raw(&self, out: *mut f32, stream: *mut c_void) -> Result<()> {
        check(sys::unillm_hip_dequant(self.w, out, stream))
    }

    /// QMatMul::forward on device buffers, sizes checked (the default stream).
    pub fn forward(&self, x: &DeviceBuffer, m: usize, y: &mut DeviceBuffer) -> Result<()> {
        if x.len_f32() < m * self.k || y.len_f32() < m * self.n {
            return Err(invalid(format!(
                "QMatMul forward failed: buffers of {} and {} f32 for m = {m}, k = {}, n = {}",
                x.len_f32(), y.len_f32(), self.k, self.n)));
        }
        unsafe { self.forward_raw(x.as_ptr(), m, y.as_mut_ptr(), ptr::null_mut()) }
    }
}

impl Drop for QuantLinear {
    fn drop(&mut self) {
        unsafe {
            sys::unillm_hip_qweight_destroy(self.w);
        }
    }
}

/// `LlamaModelV2::lm_head_forward` (llama.rs:396-405) with a quantized lm_head: the
/// error reads "QMatMul lm_head forward failed: ..." as the reference's does.
pub fn lm_head_forward(lm_head: &QuantLinear, hidden: &DeviceBuffer, m: usize,
                       logits: &mut DeviceBuffer) -> Result<()> {
    lm_head.forward(hidden, m, logits).map_err(|e| {
        let detail = e.message.strip_prefix("QMatMul forward failed: ").unwrap_or(&e.message);
        HipError { code: e.code, message: format!("QMatMul lm_head forward failed: {detail}") }
    })
}

// ---- KV cache and attention ----------------------------------------------------------------

/// One decoder layer's cache for one sequence: K and V of n_kv_heads heads,
/// max_seq_len positions of head_dim f32, the filled length held on the device.
/// Calls must be ordered (one stream): each appends to the cache.
#[derive(Debug)]
pub struct KvCache {
    c: *mut sys::unillm_kv_cache,
    n_kv_heads: usize,
    head_dim: usize,
    max_seq_len: usize,
}

// SAFETY: the owner may move between threads; &mut self orders the appending calls.
unsafe impl Send for KvCache {}

impl KvCache {
    /// `LayerKVCache::with_capacity` (kv_cache.rs:46-53) with the shapes and RoPE base the
    /// reference takes from the model config.
    pub fn with_capacity(n_kv_heads: usize, head_dim: usize, max_seq_len: usize,
                         rope_theta: f32) -> Result<Self> {
        let mut c = ptr::null_mut();
        check(unsafe {
            sys::unillm_hip_kv_cache_create(to_i64(n_kv_heads, "n_kv_heads")?,
                                            to_i64(head_dim, "head_dim")?,
                                            to_i64(max_seq_len, "max_seq_len")?, rope_theta,
                                            &mut c)
        })?;
        Ok(Self { c, n_kv_heads, head_dim, max_seq_len })
    }

    /// `seq_len` (kv_cache.rs:74-76).
    pub fn seq_len(&self) -> Result<usize> {
        let mut n = 0i64;
        check(unsafe { sys::unillm_hip_kv_cache_length(self.c, &mut n) })?;
        Ok(n as usize)
    }
    pub fn max_seq_len(&self) -> usize {
        self.max_seq_len
    }
    pub fn n_kv_heads(&self) -> usize {
        self.n_kv_heads
    }
    pub fn head_dim(&self) -> usize {
        self.head_dim
    }

    /// `clear` (kv_cache.rs:61-64).
    pub fn clear(&mut self) -> Result<()> {
        check(unsafe { sys::unillm_hip_kv_cache_clear(self.c) })
    }

    /// Keeps the first `len` positions (a rolled-back step).
    pub fn truncate(&mut self, len: usize) -> Result<()> {
        check(unsafe { sys::unillm_hip_kv_cache_truncate(self.c, to_i64(len, "len")?) })
    }

    /// Grows `stream`'s attention workspace for calls of up to m tokens.
    pub fn reserve(&self, m: usize, n_heads: usize, stream: *mut c_void) -> Result<()> {
        check(unsafe {
            sys::unillm_hip_attention_reserve(self.c, to_i64(m, "m")?, to_i64(n_heads, "n_heads")?,
                                              stream)
        })
    }

    /// RoPE at positions seq_len() .., append k and v, causal softmax attention:
    /// qkv [m, (n_heads + 2 n_kv_heads) head_dim] -> out [m, n_heads head_dim].
    ///
    /// # Safety
    /// `qkv` and `out` point to device memory of those sizes (qkv 16-byte aligned);
    /// `stream` is a HIP stream of the library's device, or null.
    pub unsafe fn attention_raw(&mut self, qkv: *const f32, m: usize, n_heads: usize,
                                out: *mut f32, stream: *mut c_void) -> Result<()> {
        check(sys::unillm_hip_attention_decode(self.c, qkv, to_i64(m, "m")?,
                                               to_i64(n_heads, "n_heads")?, out, stream))
    }

    /// attention_raw on device buffers, sizes checked (the default stream).
    pub fn attention(&mut self, qkv: &DeviceBuffer, m: usize, n_heads: usize,
                     out: &mut DeviceBuffer) -> Result<()> {
        let width = (n_heads + 2 * self.n_kv_heads) * self.head_dim;
        if qkv.len_f32() < m * width || out.len_f32() < m * n_heads * self.head_dim {
            return Err(invalid(format!(
                "attention: buffers of {} and {} f32 for m = {m}, qkv width {width}",
                qkv.len_f32(), out.len_f32())));
        }
        unsafe { self.attention_raw(qkv.as_ptr(), m, n_heads, out.as_mut_ptr(), ptr::null_mut()) }
    }
}

impl Drop for KvCache {
    fn drop(&mut self) {
        unsafe {
            sys::unillm_hip_kv_cache_destroy(self.c);
        }
    }
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn qtype_ids_are_ggml_ids() {
        assert_eq!(QType::from_ggml(2), Some(QType::Q4_0));
        assert_eq!(QType::from_ggml(6), Some(QType::Q5_0));
        assert_eq!(QType::from_ggml(8), Some(QType::Q8_0));
        assert_eq!(QType::from_ggml(12), Some(QType::Q4_K));
        assert_eq!(QType::from_ggml(13), Some(QType::Q5_K));
        assert_eq!(QType::from_ggml(14), Some(QType::Q6_K));
        assert_eq!(QType::from_ggml(3), None);
        assert_eq!(QType::Q4_0 as c_int, sys::UNILLM_QTYPE_Q4_0);
    }

    // Needs the device: UNILLM_HIP_TEST_GPU=1 cargo test
    #[test]
    fn q4_0_known_answer_on_device() {
        if std::env::var("UNILLM_HIP_TEST_GPU").is_err() {
            return;
        }
        // one row of two Q4_0 blocks, d = 1.0 (f16 0x3C00), every nibble 9 -> weight 1
        let mut raw = Vec::new();
        for _ in 0..2 {
            raw.extend_from_slice(&[0x00, 0x3C]);
            raw.extend_from_slice(&[0x99; 16]);
        }
        let w = QuantLinear::from_gguf_blocks(QType::Q4_0, 1, 64, &raw).unwrap();
        let x = DeviceBuffer::from_f32(&[0.5f32; 64]).unwrap();
        let mut y = DeviceBuffer::new(4).unwrap();
        w.forward(&x, 1, &mut y).unwrap();
        assert_eq!(y.to_f32().unwrap(), vec![32.0]);
        let err = lm_head_forward(&w, &x, 2, &mut y).unwrap_err();
        assert!(err.message.starts_with("QMatMul lm_head forward failed: "), "{}", err.message);
    }
}
