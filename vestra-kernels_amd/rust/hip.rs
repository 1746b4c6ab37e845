//! HIP device backend for vestra-kernels (feature `hip`), the drop-in
//! replacement of the `cuda` module (src/cuda.rs) on AMD Instinct MI355X.
//!
//! Every method calls one function of the C ABI in `include/vestra_hip.h`
//! (library `libvestra_hip.so`, hand-written gfx950 HIP kernels).  The public
//! types keep the shape of src/cuda.rs: a cloneable runtime bound to one
//! device and one ordered stream (`HipRuntime` for `CudaRuntime`,
//! src/cuda.rs:357-1279), opaque device tensors (`HipTensorF32` for
//! `CudaTensorF32`, src/cuda.rs:1283-1286, 1347-1357), prepared projections
//! (`HipLinearF32` for `CudaLinearF32`, src/cuda.rs:1291-1345) and one error
//! variant per `CudaError` variant (src/cuda.rs:337-354).  The `Cuda*` type
//! aliases at the end let engine code written against src/cuda.rs compile
//! against this module unchanged apart from the module path.
//!
//! Threading: the C runtime wants external synchronisation when shared
//! between host threads, so every call holds the runtime's lock; clones of a
//! runtime (and the tensors, projections and blocks made from it) share that
//! lock, which makes the handles `Send + Sync` soundly.
//!
//! This file is written against the C ABI of this repository; it is compiled
//! by the crate's build (see build.rs next to it) and is not built here.

#![allow(clippy::too_many_arguments)]

use std::ffi::{c_char, c_int, c_void, CStr};
use std::ptr;
use std::sync::{Arc, Mutex, MutexGuard};

use crate::BlockQ8_0;

#[cfg(all(feature = "cuda", feature = "hip"))]
compile_error!("features `cuda` and `hip` are exclusive: `hip` replaces the CUDA driver/cuBLAS path");

// ---- FFI: include/vestra_hip.h --------------------------------------------

#[repr(C)]
pub struct VhRuntime {
    _p: [u8; 0],
}
#[repr(C)]
pub struct VhTensor {
    _p: [u8; 0],
}
#[repr(C)]
pub struct VhLinear {
    _p: [u8; 0],
}
#[repr(C)]
pub struct VhQ8Tensor {
    _p: [u8; 0],
}
#[repr(C)]
pub struct VhBlock {
    _p: [u8; 0],
}
#[repr(C)]
pub struct VhLinearQ8 {
    _p: [u8; 0],
}
#[repr(C)]
pub struct VhConv2d {
    _p: [u8; 0],
}
#[repr(C)]
pub struct VhConvTranspose2d {
    _p: [u8; 0],
}

type Status = c_int;

/// `vh_block_params`: host pointers to one block's parameters, row-major
/// [in, out] weights; the four Q/K LayerNorm vectors are null for a plain
/// block (DA3 late blocks set all four).
#[repr(C)]
struct VhBlockParams {
    ln1_gamma: *const f32,
    ln1_beta: *const f32,
    w_qkv: *const f32,
    b_qkv: *const f32,
    w_proj: *const f32,
    b_proj: *const f32,
    ls1: *const f32,
    ln2_gamma: *const f32,
    ln2_beta: *const f32,
    w_fc1: *const f32,
    b_fc1: *const f32,
    w_fc2: *const f32,
    b_fc2: *const f32,
    ls2: *const f32,
    q_norm_gamma: *const f32,
    q_norm_beta: *const f32,
    k_norm_gamma: *const f32,
    k_norm_beta: *const f32,
}

// Linked by build.rs (cargo:rustc-link-lib=dylib=vestra_hip).
unsafe extern "C" {
    fn vh_last_error() -> *const c_char;
    fn vh_last_length_mismatch(destination: *mut usize, source_len: *mut usize);

    fn vh_runtime_new(device: usize, out: *mut *mut VhRuntime) -> Status;
    fn vh_runtime_free(rt: *mut VhRuntime);
    fn vh_runtime_device(rt: *const VhRuntime) -> usize;
    fn vh_runtime_stream(rt: *const VhRuntime) -> *mut c_void;
    fn vh_runtime_synchronize(rt: *const VhRuntime) -> Status;

    fn vh_upload_f32(rt: *const VhRuntime, values: *const f32, len: usize, out: *mut *mut VhTensor) -> Status;
    fn vh_download_f32(rt: *const VhRuntime, t: *const VhTensor, out: *mut f32, out_len: usize) -> Status;
    fn vh_tensor_alloc(rt: *const VhRuntime, len: usize, out: *mut *mut VhTensor) -> Status;
    fn vh_tensor_free(t: *mut VhTensor);
    fn vh_tensor_len(t: *const VhTensor) -> usize;
    fn vh_tensor_device_ptr(t: *const VhTensor) -> *mut f32;

    fn vh_copy_f32(rt: *const VhRuntime, source: *const VhTensor, out: *mut *mut VhTensor) -> Status;
    fn vh_copy_segment_f32(rt: *const VhRuntime, source: *const VhTensor, source_offset: usize, len: usize,
                           out: *mut *mut VhTensor) -> Status;
    fn vh_copy_segment_into_f32(rt: *const VhRuntime, destination: *mut VhTensor, destination_offset: usize,
                                source: *const VhTensor, source_offset: usize, len: usize) -> Status;
    fn vh_overwrite_prefix_f32(rt: *const VhRuntime, destination: *mut VhTensor, source: *const VhTensor,
                               len: usize) -> Status;
    fn vh_add_f32_in_place(rt: *const VhRuntime, destination: *mut VhTensor, source: *const VhTensor) -> Status;

    fn vh_gemm_row_major_f32(rt: *const VhRuntime, a: *const VhTensor, b: *const VhTensor, m: usize, k: usize,
                             n: usize, out: *mut *mut VhTensor) -> Status;
    fn vh_bias_scale_f32_in_place(rt: *const VhRuntime, values: *mut VhTensor, bias: *const VhTensor,
                                  gamma: *const VhTensor, rows: usize, columns: usize) -> Status;
    fn vh_gelu_f32_in_place(rt: *const VhRuntime, values: *mut VhTensor) -> Status;

    fn vh_layernorm_f32(rt: *const VhRuntime, input: *const VhTensor, gamma: *const VhTensor,
                        beta: *const VhTensor, rows: usize, columns: usize, epsilon: f32,
                        out: *mut *mut VhTensor) -> Status;
    fn vh_layernorm_f32_cpu_order(rt: *const VhRuntime, input: *const VhTensor, gamma: *const VhTensor,
                                  beta: *const VhTensor, rows: usize, columns: usize, epsilon: f32,
                                  out: *mut *mut VhTensor) -> Status;

    fn vh_attention_online_f32(rt: *const VhRuntime, q: *const VhTensor, k: *const VhTensor, v: *const VhTensor,
                               heads: usize, tokens: usize, head_dim: usize, out: *mut *mut VhTensor) -> Status;
    fn vh_flash_attention_f32_da3_base(rt: *const VhRuntime, q: *const VhTensor, k: *const VhTensor,
                                       v: *const VhTensor, heads: usize, tokens: usize, token_major: c_int,
                                       out: *mut *mut VhTensor) -> Status;
    fn vh_flash_attention_f32_da3_base_into(rt: *const VhRuntime, q: *const VhTensor, k: *const VhTensor,
                                            v: *const VhTensor, heads: usize, tokens: usize,
                                            token_major: c_int, out: *mut VhTensor) -> Status;

    fn vh_split_qkv_hnd_f32(rt: *const VhRuntime, qkv: *const VhTensor, tokens: usize, heads: usize,
                            head_dim: usize, q: *mut *mut VhTensor, k: *mut *mut VhTensor,
                            v: *mut *mut VhTensor) -> Status;
    fn vh_hnd_to_token_f32(rt: *const VhRuntime, hnd: *const VhTensor, tokens: usize, heads: usize,
                           head_dim: usize, out: *mut *mut VhTensor) -> Status;
    fn vh_token_to_chw_f32(rt: *const VhRuntime, token_major: *const VhTensor, tokens: usize, channels: usize,
                           out: *mut *mut VhTensor) -> Status;
    fn vh_patchify_nchw_f32(rt: *const VhRuntime, image: *const VhTensor, height: usize, width: usize,
                            patch: usize, channels: usize, out: *mut *mut VhTensor) -> Status;
    fn vh_prepend_cls_add_pos_f32(rt: *const VhRuntime, patches: *const VhTensor, cls: *const VhTensor,
                                  position: *const VhTensor, patch_count: usize, embed: usize,
                                  out: *mut *mut VhTensor) -> Status;

    fn vh_rope2d_f32_in_place(rt: *const VhRuntime, x: *mut VhTensor, heads: usize, n: usize, head_dim: usize,
                              pos_yx: *const i64, frequency: f32) -> Status;
    fn vh_qk_norm_rope_f32_da3_base(rt: *const VhRuntime, q: *mut VhTensor, k: *mut VhTensor,
                                    q_gamma: *const VhTensor, q_beta: *const VhTensor, k_gamma: *const VhTensor,
                                    k_beta: *const VhTensor, positions_yx: *const VhTensor, heads: usize,
                                    tokens: usize, frequency: f32, epsilon: f32) -> Status;

    fn vh_prepare_linear_f32(rt: *const VhRuntime, input_features: usize, output_features: usize,
                             weight: *const f32, bias: *const f32, gamma: *const f32,
                             out: *mut *mut VhLinear) -> Status;
    fn vh_linear_free(l: *mut VhLinear);
    fn vh_linear_input_features(l: *const VhLinear) -> usize;
    fn vh_linear_output_features(l: *const VhLinear) -> usize;
    fn vh_linear_run(l: *const VhLinear, input: *const VhTensor, rows: usize, out: *mut *mut VhTensor) -> Status;
    fn vh_linear_run_chw(l: *const VhLinear, input: *const VhTensor, rows: usize, out: *mut *mut VhTensor) -> Status;
    fn vh_linear_run_gelu(l: *const VhLinear, input: *const VhTensor, rows: usize, out: *mut *mut VhTensor) -> Status;
    fn vh_linear_run_residual(l: *const VhLinear, input: *const VhTensor, rows: usize,
                              residual: *mut VhTensor) -> Status;
    fn vh_linear_run_qkv_hnd(l: *const VhLinear, input: *const VhTensor, images: usize, tokens: usize,
                             heads: usize, pos_yx: *const i64, frequency: f32, q: *mut *mut VhTensor,
                             k: *mut *mut VhTensor, v: *mut *mut VhTensor) -> Status;

    fn vh_q8_0_upload(rt: *const VhRuntime, blocks: *const c_void, rows: usize, k: usize,
                      out: *mut *mut VhQ8Tensor) -> Status;
    fn vh_q8_0_download(rt: *const VhRuntime, t: *const VhQ8Tensor, blocks: *mut c_void, nblocks: usize) -> Status;
    fn vh_q8_tensor_free(t: *mut VhQ8Tensor);
    fn vh_q8_tensor_rows(t: *const VhQ8Tensor) -> usize;
    fn vh_q8_tensor_k(t: *const VhQ8Tensor) -> usize;
    fn vh_quantize_q8_0(rt: *const VhRuntime, x: *const VhTensor, rows: usize, k: usize,
                        out: *mut *mut VhQ8Tensor) -> Status;
    fn vh_quantize_q8_0_into(rt: *const VhRuntime, x: *const VhTensor, rows: usize, k: usize,
                             out: *mut VhQ8Tensor) -> Status;
    fn vh_gemm_q8_0(rt: *const VhRuntime, a_q: *const VhQ8Tensor, b_q: *const VhQ8Tensor, m: usize, n: usize,
                    k: usize, out: *mut *mut VhTensor) -> Status;
    fn vh_gemm_q8_0_into(rt: *const VhRuntime, a_q: *const VhQ8Tensor, b_q: *const VhQ8Tensor, m: usize,
                         n: usize, k: usize, c: *mut VhTensor) -> Status;

    fn vh_prepare_linear_q8_0(rt: *const VhRuntime, input_features: usize, output_features: usize,
                              weight_blocks: *const c_void, bias: *const f32, gamma: *const f32,
                              out: *mut *mut VhLinearQ8) -> Status;
    fn vh_linear_q8_0_free(l: *mut VhLinearQ8);
    fn vh_linear_q8_0_input_features(l: *const VhLinearQ8) -> usize;
    fn vh_linear_q8_0_output_features(l: *const VhLinearQ8) -> usize;
    fn vh_linear_q8_0_run(l: *const VhLinearQ8, input: *const VhTensor, rows: usize, out: *mut *mut VhTensor) -> Status;
    fn vh_linear_q8_0_run_gelu(l: *const VhLinearQ8, input: *const VhTensor, rows: usize,
                               out: *mut *mut VhTensor) -> Status;
    fn vh_linear_q8_0_run_residual(l: *const VhLinearQ8, input: *const VhTensor, rows: usize,
                                   residual: *mut VhTensor) -> Status;

    fn vh_block_prepare(rt: *const VhRuntime, params: *const VhBlockParams, out: *mut *mut VhBlock) -> Status;
    fn vh_block_prepare_q8_0(rt: *const VhRuntime, params: *const VhBlockParams, out: *mut *mut VhBlock) -> Status;
    fn vh_block_is_q8_0(b: *const VhBlock) -> c_int;
    fn vh_block_free(b: *mut VhBlock);
    fn vh_vit_block_run(rt: *const VhRuntime, b: *const VhBlock, x: *mut VhTensor, images: usize, tokens: usize,
                        pos_yx: *const i64, rope_frequency: f32, epsilon: f32) -> Status;
    fn vh_encoder_run(rt: *const VhRuntime, blocks: *const *const VhBlock, layers: usize, x: *mut VhTensor,
                      images: usize, tokens: usize, pos_yx: *const i64, rope_frequency: f32,
                      epsilon: f32) -> Status;

    fn vh_prepare_conv2d_f32(rt: *const VhRuntime, in_c: usize, out_c: usize, kh: usize, kw: usize,
                             stride: usize, pad: usize, weight: *const f32, bias: *const f32,
                             out: *mut *mut VhConv2d) -> Status;
    fn vh_conv2d_free(c: *mut VhConv2d);
    fn vh_conv2d_output_height(c: *const VhConv2d, ih: usize) -> usize;
    fn vh_conv2d_output_width(c: *const VhConv2d, iw: usize) -> usize;
    fn vh_conv2d_run(c: *const VhConv2d, input: *const VhTensor, ih: usize, iw: usize,
                     out: *mut *mut VhTensor) -> Status;
    fn vh_conv2d_run_relu_input(c: *const VhConv2d, input: *const VhTensor, ih: usize, iw: usize,
                                out: *mut *mut VhTensor) -> Status;
    fn vh_conv2d_run_resize_align_corners(c: *const VhConv2d, input: *const VhTensor, ih: usize, iw: usize,
                                          oh: usize, ow: usize, add: *const VhTensor,
                                          out: *mut *mut VhTensor) -> Status;
    fn vh_conv2d_f32(rt: *const VhRuntime, input: *const VhTensor, in_c: usize, ih: usize, iw: usize,
                     weight: *const f32, out_c: usize, kh: usize, kw: usize, stride: usize, pad: usize,
                     bias: *const f32, out: *mut *mut VhTensor) -> Status;
    fn vh_prepare_conv_transpose2d_f32(rt: *const VhRuntime, in_c: usize, out_c: usize, kh: usize, kw: usize,
                                       stride: usize, weight: *const f32, bias: *const f32,
                                       out: *mut *mut VhConvTranspose2d) -> Status;
    fn vh_conv_transpose2d_free(c: *mut VhConvTranspose2d);
    fn vh_conv_transpose2d_run(c: *const VhConvTranspose2d, input: *const VhTensor, ih: usize, iw: usize,
                               out: *mut *mut VhTensor) -> Status;
    fn vh_conv_transpose2d_f32(rt: *const VhRuntime, input: *const VhTensor, in_c: usize, ih: usize, iw: usize,
                               weight: *const f32, out_c: usize, kh: usize, kw: usize, stride: usize,
                               bias: *const f32, out: *mut *mut VhTensor) -> Status;
    fn vh_bilinear_resize_f32(rt: *const VhRuntime, input: *const VhTensor, c: usize, ih: usize, iw: usize,
                              oh: usize, ow: usize, out: *mut *mut VhTensor) -> Status;
    fn vh_bilinear_resize_align_corners_f32(rt: *const VhRuntime, input: *const VhTensor, c: usize, ih: usize,
                                            iw: usize, oh: usize, ow: usize, add: *const VhTensor,
                                            out: *mut *mut VhTensor) -> Status;

    fn vh_profile_enable(rt: *mut VhRuntime, enabled: c_int) -> Status;
    fn vh_profile_reset(rt: *mut VhRuntime) -> Status;
    fn vh_profile_report(rt: *mut VhRuntime, buf: *mut c_char, buflen: usize) -> Status;
    fn vh_timer_start(rt: *mut VhRuntime) -> Status;
    fn vh_timer_stop(rt: *mut VhRuntime, elapsed_ms: *mut f32) -> Status;
}

// ---- errors: CudaError (src/cuda.rs:337-354) ------------------------------

/// One variant per `CudaError` variant; the status codes of the C ABI map
/// onto them (`VH_ERR_INVALID_ARGUMENT`, a null handle, cannot arise from
/// these safe wrappers and is reported as `Kernel`).
#[derive(Debug, thiserror::Error)]
pub enum HipError {
    #[error("failed to initialize HIP device {device}: {detail}")]
    Initialize { device: usize, detail: String },
    #[error("HIP host-to-device transfer failed: {0}")]
    Upload(String),
    #[error("HIP device-to-host transfer failed: {0}")]
    Download(String),
    #[error("HIP residual add requires equally sized tensors, got {destination} and {source_len}")]
    LengthMismatch { destination: usize, source_len: usize },
    #[error("HIP kernel launch failed: {0}")]
    Kernel(String),
    #[error("HIP GEMM operation failed: {0}")]
    Blas(String),
}

fn check(status: Status, device: usize) -> Result<(), HipError> {
    if status == 0 {
        return Ok(());
    }
    // SAFETY: vh_last_error returns the calling thread's NUL-terminated message.
    let msg = unsafe { CStr::from_ptr(vh_last_error()) }.to_string_lossy().into_owned();
    Err(match status {
        1 => HipError::Initialize { device, detail: msg },
        2 => HipError::Upload(msg),
        3 => HipError::Download(msg),
        4 => {
            let (mut destination, mut source_len) = (0usize, 0usize);
            // SAFETY: both pointers are valid for one write.
            unsafe { vh_last_length_mismatch(&mut destination, &mut source_len) };
            HipError::LengthMismatch { destination, source_len }
        }
        6 => HipError::Blas(msg),
        _ => HipError::Kernel(msg),
    })
}

fn opt_ptr(v: Option<&[f32]>) -> *const f32 {
    v.map_or(ptr::null(), <[f32]>::as_ptr)
}

// ---- runtime ---------------------------------------------------------------

struct RuntimeInner {
    raw: *mut VhRuntime,
    device: usize,
    lock: Mutex<()>,
}

// SAFETY: the C runtime may be used from any thread; concurrent use is
// serialised by `lock`, which every call through a clone holds.
unsafe impl Send for RuntimeInner {}
unsafe impl Sync for RuntimeInner {}

impl Drop for RuntimeInner {
    fn drop(&mut self) {
        // SAFETY: raw came from vh_runtime_new and is freed once, last.
        unsafe { vh_runtime_free(self.raw) }
    }
}

/// `CudaRuntime` (src/cuda.rs:357-1279): one device and one ordered stream.
/// All operations are asynchronous on that stream; `download_f32`,
/// `synchronize` and the Q8_0 download synchronise.
#[derive(Clone)]
pub struct HipRuntime {
    inner: Arc<RuntimeInner>,
}

/// `CudaTensorF32` (src/cuda.rs:1283-1286): an opaque device f32 buffer.
pub struct HipTensorF32 {
    raw: *mut VhTensor,
    runtime: HipRuntime,
}

// SAFETY: the tensor is a device allocation owned by this handle; every use
// goes through its runtime's lock.
unsafe impl Send for HipTensorF32 {}
unsafe impl Sync for HipTensorF32 {}

impl Drop for HipTensorF32 {
    fn drop(&mut self) {
        let _g = self.runtime.guard();
        // SAFETY: raw came from the library and is freed once.
        unsafe { vh_tensor_free(self.raw) }
    }
}

impl HipTensorF32 {
    /// src/cuda.rs:1349-1351
    #[must_use]
    pub fn len(&self) -> usize {
        // SAFETY: raw is a live tensor handle.
        unsafe { vh_tensor_len(self.raw) }
    }

    /// src/cuda.rs:1353-1356
    #[must_use]
    pub fn is_empty(&self) -> bool {
        self.len() == 0
    }

    /// Raw device address, for interop with other device libraries.
    #[must_use]
    pub fn device_ptr(&self) -> *mut f32 {
        // SAFETY: raw is a live tensor handle.
        unsafe { vh_tensor_device_ptr(self.raw) }
    }
}

impl HipRuntime {
    fn guard(&self) -> MutexGuard<'_, ()> {
        self.inner.lock.lock().unwrap_or_else(std::sync::PoisonError::into_inner)
    }

    fn ok(&self, status: Status) -> Result<(), HipError> {
        check(status, self.inner.device)
    }

    fn tensor(&self, raw: *mut VhTensor) -> HipTensorF32 {
        HipTensorF32 { raw, runtime: self.clone() }
    }

    /// Runs `f` with the lock held and wraps the tensor it creates.
    fn make(&self, f: impl FnOnce(*mut *mut VhTensor) -> Status) -> Result<HipTensorF32, HipError> {
        let mut out = ptr::null_mut();
        let status = {
            let _g = self.guard();
            f(&mut out)
        };
        self.ok(status)?;
        Ok(self.tensor(out))
    }

    fn call(&self, f: impl FnOnce() -> Status) -> Result<(), HipError> {
        let status = {
            let _g = self.guard();
            f()
        };
        self.ok(status)
    }

    /// src/cuda.rs:383-465
    pub fn new(device: usize) -> Result<Self, HipError> {
        let mut raw = ptr::null_mut();
        // SAFETY: out-pointer valid for one write.
        check(unsafe { vh_runtime_new(device, &mut raw) }, device)?;
        Ok(Self { inner: Arc::new(RuntimeInner { raw, device, lock: Mutex::new(()) }) })
    }

    /// src/cuda.rs:467-470
    #[must_use]
    pub fn device(&self) -> usize {
        // SAFETY: raw is a live runtime.
        unsafe { vh_runtime_device(self.inner.raw) }
    }

    /// src/cuda.rs:1271-1279 (`context()` / `stream()`): the hipStream_t of
    /// every operation, for interop (a device context has no HIP analogue).
    #[must_use]
    pub fn stream(&self) -> *mut c_void {
        // SAFETY: raw is a live runtime.
        unsafe { vh_runtime_stream(self.inner.raw) }
    }

    /// Blocks until the stream's work has finished.
    pub fn synchronize(&self) -> Result<(), HipError> {
        let raw = self.inner.raw;
        // SAFETY: raw is a live runtime.
        self.call(|| unsafe { vh_runtime_synchronize(raw) })
    }

    /// src/cuda.rs:474-483
    pub fn upload_f32(&self, values: &[f32]) -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: values is valid for values.len() reads.
        self.make(|out| unsafe { vh_upload_f32(raw, values.as_ptr(), values.len(), out) })
    }

    /// src/cuda.rs:487-491
    pub fn download_f32(&self, tensor: &HipTensorF32) -> Result<Vec<f32>, HipError> {
        let mut host = vec![0.0f32; tensor.len()];
        let raw = self.inner.raw;
        // SAFETY: host is valid for its length of writes.
        self.call(|| unsafe { vh_download_f32(raw, tensor.raw, host.as_mut_ptr(), host.len()) })?;
        Ok(host)
    }

    /// An uninitialised device tensor of `len` floats (an output buffer for
    /// `flash_attention_f32_da3_base_into`).
    pub fn alloc_f32(&self, len: usize) -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: out-pointer valid for one write.
        self.make(|out| unsafe { vh_tensor_alloc(raw, len, out) })
    }

    /// src/cuda.rs:496-515
    pub fn copy_f32(&self, source: &HipTensorF32) -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe { vh_copy_f32(raw, source.raw, out) })
    }

    /// src/cuda.rs:519-539
    pub fn copy_segment_f32(&self, source: &HipTensorF32, source_offset: usize, len: usize)
        -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles; bounds are checked by the library.
        self.make(|out| unsafe { vh_copy_segment_f32(raw, source.raw, source_offset, len, out) })
    }

    /// src/cuda.rs:543-595
    pub fn copy_segment_into_f32(&self, destination: &mut HipTensorF32, destination_offset: usize,
                                 source: &HipTensorF32, source_offset: usize, len: usize)
        -> Result<(), HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles; bounds are checked by the library.
        self.call(|| unsafe {
            vh_copy_segment_into_f32(raw, destination.raw, destination_offset, source.raw, source_offset, len)
        })
    }

    /// src/cuda.rs:599-626
    pub fn overwrite_prefix_f32(&self, destination: &mut HipTensorF32, source: &HipTensorF32, len: usize)
        -> Result<(), HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.call(|| unsafe { vh_overwrite_prefix_f32(raw, destination.raw, source.raw, len) })
    }

    /// src/cuda.rs:630-654
    pub fn add_f32_in_place(&self, destination: &mut HipTensorF32, source: &HipTensorF32)
        -> Result<(), HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.call(|| unsafe { vh_add_f32_in_place(raw, destination.raw, source.raw) })
    }

    /// src/cuda.rs:661-704 (fp32-MFMA GEMM in place of cublasSgemm)
    pub fn gemm_row_major_f32(&self, a: &HipTensorF32, b: &HipTensorF32, m: usize, k: usize, n: usize)
        -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe { vh_gemm_row_major_f32(raw, a.raw, b.raw, m, k, n, out) })
    }

    /// src/cuda.rs:708-742
    pub fn bias_scale_f32_in_place(&self, values: &mut HipTensorF32, bias: &HipTensorF32,
                                   gamma: &HipTensorF32, rows: usize, columns: usize)
        -> Result<(), HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.call(|| unsafe { vh_bias_scale_f32_in_place(raw, values.raw, bias.raw, gamma.raw, rows, columns) })
    }

    /// src/cuda.rs:747-759
    pub fn gelu_f32_in_place(&self, values: &mut HipTensorF32) -> Result<(), HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.call(|| unsafe { vh_gelu_f32_in_place(raw, values.raw) })
    }

    /// src/cuda.rs:764-810
    pub fn layernorm_f32(&self, input: &HipTensorF32, gamma: &HipTensorF32, beta: &HipTensorF32,
                         rows: usize, columns: usize, epsilon: f32) -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe { vh_layernorm_f32(raw, input.raw, gamma.raw, beta.raw, rows, columns, epsilon, out) })
    }

    /// src/cuda.rs:815-863
    pub fn layernorm_f32_cpu_order(&self, input: &HipTensorF32, gamma: &HipTensorF32, beta: &HipTensorF32,
                                   rows: usize, columns: usize, epsilon: f32)
        -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe {
            vh_layernorm_f32_cpu_order(raw, input.raw, gamma.raw, beta.raw, rows, columns, epsilon, out)
        })
    }

    /// src/cuda.rs:868-922
    pub fn attention_online_f32(&self, q: &HipTensorF32, k: &HipTensorF32, v: &HipTensorF32, heads: usize,
                                tokens: usize, head_dim: usize) -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe { vh_attention_online_f32(raw, q.raw, k.raw, v.raw, heads, tokens, head_dim, out) })
    }

    /// flash_attention_f32_da3_base (src/lib.rs:82-91) on the device; head-major
    /// or token-major output.
    pub fn flash_attention_f32_da3_base(&self, q: &HipTensorF32, k: &HipTensorF32, v: &HipTensorF32,
                                        heads: usize, tokens: usize, token_major: bool)
        -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe {
            vh_flash_attention_f32_da3_base(raw, q.raw, k.raw, v.raw, heads, tokens, c_int::from(token_major), out)
        })
    }

    /// The same attention into `out`, allocating nothing (no counterpart in
    /// src/cuda.rs: for callers that cannot allocate device memory).
    pub fn flash_attention_f32_da3_base_into(&self, q: &HipTensorF32, k: &HipTensorF32, v: &HipTensorF32,
                                             heads: usize, tokens: usize, token_major: bool,
                                             out: &mut HipTensorF32) -> Result<(), HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.call(|| unsafe {
            vh_flash_attention_f32_da3_base_into(raw, q.raw, k.raw, v.raw, heads, tokens,
                                                 c_int::from(token_major), out.raw)
        })
    }

    /// src/cuda.rs:927-980
    pub fn split_qkv_hnd_f32(&self, qkv: &HipTensorF32, tokens: usize, heads: usize, head_dim: usize)
        -> Result<(HipTensorF32, HipTensorF32, HipTensorF32), HipError> {
        let (mut q, mut k, mut v) = (ptr::null_mut(), ptr::null_mut(), ptr::null_mut());
        let raw = self.inner.raw;
        // SAFETY: live handles; out-pointers valid for one write each.
        self.call(|| unsafe { vh_split_qkv_hnd_f32(raw, qkv.raw, tokens, heads, head_dim, &mut q, &mut k, &mut v) })?;
        Ok((self.tensor(q), self.tensor(k), self.tensor(v)))
    }

    /// src/cuda.rs:984-1028
    pub fn hnd_to_token_f32(&self, hnd: &HipTensorF32, tokens: usize, heads: usize, head_dim: usize)
        -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe { vh_hnd_to_token_f32(raw, hnd.raw, tokens, heads, head_dim, out) })
    }

    /// src/cuda.rs:1032-1069
    pub fn token_to_chw_f32(&self, token_major: &HipTensorF32, tokens: usize, channels: usize)
        -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe { vh_token_to_chw_f32(raw, token_major.raw, tokens, channels, out) })
    }

    /// src/cuda.rs:1073-1126
    pub fn patchify_nchw_f32(&self, image: &HipTensorF32, height: usize, width: usize, patch: usize,
                             channels: usize) -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe { vh_patchify_nchw_f32(raw, image.raw, height, width, patch, channels, out) })
    }

    /// src/cuda.rs:1130-1174
    pub fn prepend_cls_add_pos_f32(&self, patches: &HipTensorF32, cls: &HipTensorF32, position: &HipTensorF32,
                                   patch_count: usize, embed: usize) -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe {
            vh_prepend_cls_add_pos_f32(raw, patches.raw, cls.raw, position.raw, patch_count, embed, out)
        })
    }

    /// rope::rope2d (src/rope.rs:30-80) on a device [heads, n, head_dim]
    /// tensor; pos_yx holds (y, x) per token.
    pub fn rope2d_f32_in_place(&self, x: &mut HipTensorF32, heads: usize, n: usize, head_dim: usize,
                               pos_yx: &[i64], frequency: f32) -> Result<(), HipError> {
        if pos_yx.len() != n.saturating_mul(2) {
            return Err(HipError::LengthMismatch { destination: n.saturating_mul(2), source_len: pos_yx.len() });
        }
        let raw = self.inner.raw;
        // SAFETY: live handles; pos_yx holds n * 2 values.
        self.call(|| unsafe { vh_rope2d_f32_in_place(raw, x.raw, heads, n, head_dim, pos_yx.as_ptr(), frequency) })
    }

    /// src/cuda.rs:1178-1228
    pub fn qk_norm_rope_f32_da3_base(&self, q: &mut HipTensorF32, k: &mut HipTensorF32, q_gamma: &HipTensorF32,
                                     q_beta: &HipTensorF32, k_gamma: &HipTensorF32, k_beta: &HipTensorF32,
                                     positions_yx: &HipTensorF32, heads: usize, tokens: usize, frequency: f32,
                                     epsilon: f32) -> Result<(), HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.call(|| unsafe {
            vh_qk_norm_rope_f32_da3_base(raw, q.raw, k.raw, q_gamma.raw, q_beta.raw, k_gamma.raw, k_beta.raw,
                                         positions_yx.raw, heads, tokens, frequency, epsilon)
        })
    }

    /// src/cuda.rs:1233-1268
    pub fn prepare_linear_f32(&self, input_features: usize, output_features: usize, weight: &[f32], bias: &[f32],
                              gamma: Option<&[f32]>) -> Result<HipLinearF32, HipError> {
        let want = input_features.saturating_mul(output_features);
        if weight.len() != want {
            return Err(HipError::Blas(format!(
                "linear weight K={input_features}, N={output_features} does not match length {}", weight.len())));
        }
        if bias.len() != output_features || gamma.is_some_and(|g| g.len() != output_features) {
            return Err(HipError::Blas(format!("linear bias/gamma must hold N={output_features} values")));
        }
        let mut out = ptr::null_mut();
        let raw = self.inner.raw;
        // SAFETY: weight / bias / gamma hold the lengths checked above.
        self.call(|| unsafe {
            vh_prepare_linear_f32(raw, input_features, output_features, weight.as_ptr(), bias.as_ptr(),
                                  opt_ptr(gamma), &mut out)
        })?;
        Ok(HipLinearF32 { raw: out, runtime: self.clone() })
    }

    // -- Q8_0 ------------------------------------------------------------------

    /// Rows of BlockQ8_0 (src/lib.rs:33-38) moved to the device.
    pub fn q8_0_upload(&self, blocks: &[BlockQ8_0], rows: usize, k: usize) -> Result<HipQ8Tensor, HipError> {
        if k % 32 != 0 || blocks.len() != rows.saturating_mul(k / 32) {
            return Err(HipError::LengthMismatch { destination: rows.saturating_mul(k / 32), source_len: blocks.len() });
        }
        let mut out = ptr::null_mut();
        let raw = self.inner.raw;
        // SAFETY: blocks holds rows * k / 32 repr(C) 34-byte blocks.
        self.call(|| unsafe { vh_q8_0_upload(raw, blocks.as_ptr().cast(), rows, k, &mut out) })?;
        Ok(HipQ8Tensor { raw: out, runtime: self.clone() })
    }

    /// The blocks of a device Q8_0 tensor (synchronising).
    pub fn q8_0_download(&self, tensor: &HipQ8Tensor) -> Result<Vec<BlockQ8_0>, HipError> {
        let n = tensor.rows() * (tensor.k() / 32);
        let mut host: Vec<BlockQ8_0> = Vec::with_capacity(n);
        let raw = self.inner.raw;
        // SAFETY: the library writes exactly n blocks into the capacity.
        self.call(|| unsafe { vh_q8_0_download(raw, tensor.raw, host.as_mut_ptr().cast(), n) })?;
        // SAFETY: n blocks were initialised above.
        unsafe { host.set_len(n) };
        Ok(host)
    }

    /// quantize_row_q8_0 (src/q8_0_dot.rs:27-46) of each row of x [rows, k].
    pub fn quantize_q8_0(&self, x: &HipTensorF32, rows: usize, k: usize) -> Result<HipQ8Tensor, HipError> {
        let mut out = ptr::null_mut();
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.call(|| unsafe { vh_quantize_q8_0(raw, x.raw, rows, k, &mut out) })?;
        Ok(HipQ8Tensor { raw: out, runtime: self.clone() })
    }

    /// quantize_row_q8_0(x, out) (src/q8_0_dot.rs:27-46) into an existing
    /// [rows, k] Q8_0 tensor of this runtime.
    pub fn quantize_q8_0_into(&self, x: &HipTensorF32, rows: usize, k: usize, out: &mut HipQ8Tensor)
        -> Result<(), HipError> {
        let raw = self.inner.raw;
        let dst = out.raw;
        // SAFETY: live handles; `out` is borrowed mutably for the call.
        self.call(|| unsafe { vh_quantize_q8_0_into(raw, x.raw, rows, k, dst) })
    }

    /// Kernels::gemm_q8_0 (src/dispatch.rs:91-105) with b pre-transposed [n, k].
    pub fn gemm_q8_0(&self, a_q: &HipQ8Tensor, b_q: &HipQ8Tensor, m: usize, n: usize, k: usize)
        -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe { vh_gemm_q8_0(raw, a_q.raw, b_q.raw, m, n, k, out) })
    }

    /// Kernels::gemm_q8_0(m, n, k, a_q, b_q, c) into an existing [m, n]
    /// tensor of this runtime, as the reference writes `c`.
    pub fn gemm_q8_0_into(&self, a_q: &HipQ8Tensor, b_q: &HipQ8Tensor, m: usize, n: usize, k: usize,
                          c: &mut HipTensorF32) -> Result<(), HipError> {
        let raw = self.inner.raw;
        let dst = c.raw;
        // SAFETY: live handles; `c` is borrowed mutably for the call.
        self.call(|| unsafe { vh_gemm_q8_0_into(raw, a_q.raw, b_q.raw, m, n, k, dst) })
    }

    /// A projection with BlockQ8_0 weights (rows of W^T), bias and gamma [N].
    pub fn prepare_linear_q8_0(&self, input_features: usize, output_features: usize, weight_blocks: &[BlockQ8_0],
                               bias: Option<&[f32]>, gamma: Option<&[f32]>) -> Result<HipLinearQ8, HipError> {
        if input_features % 32 != 0 || weight_blocks.len() != output_features.saturating_mul(input_features / 32) {
            return Err(HipError::Blas(format!(
                "Q8_0 weight N={output_features}, K={input_features} does not match {} blocks", weight_blocks.len())));
        }
        if bias.is_some_and(|b| b.len() != output_features) || gamma.is_some_and(|g| g.len() != output_features) {
            return Err(HipError::Blas(format!("Q8_0 bias/gamma must hold N={output_features} values")));
        }
        let mut out = ptr::null_mut();
        let raw = self.inner.raw;
        // SAFETY: lengths checked above.
        self.call(|| unsafe {
            vh_prepare_linear_q8_0(raw, input_features, output_features, weight_blocks.as_ptr().cast(),
                                   opt_ptr(bias), opt_ptr(gamma), &mut out)
        })?;
        Ok(HipLinearQ8 { raw: out, runtime: self.clone() })
    }

    // -- DA3-BASE block and encoder -------------------------------------------------

    fn block(&self, p: &BlockParams<'_>, q8_0: bool) -> Result<HipBlock, HipError> {
        p.validate()?;
        let c = p.raw();
        let mut out = ptr::null_mut();
        let raw = self.inner.raw;
        // SAFETY: every pointer in c refers to a slice of the length validated above.
        self.call(|| unsafe {
            if q8_0 { vh_block_prepare_q8_0(raw, &c, &mut out) } else { vh_block_prepare(raw, &c, &mut out) }
        })?;
        Ok(HipBlock { raw: out, runtime: self.clone() })
    }

    /// Uploads and repacks one block's parameters (model-load time).
    pub fn prepare_block(&self, params: &BlockParams<'_>) -> Result<HipBlock, HipError> {
        self.block(params, false)
    }

    /// The same block with its four projections in Q8_0.
    pub fn prepare_block_q8_0(&self, params: &BlockParams<'_>) -> Result<HipBlock, HipError> {
        self.block(params, true)
    }

    /// One pre-LN DA3-BASE block in place on x [images * tokens * 768].
    pub fn vit_block_run(&self, block: &HipBlock, x: &mut HipTensorF32, images: usize, tokens: usize,
                         pos_yx: Option<&[i64]>, rope_frequency: f32, epsilon: f32) -> Result<(), HipError> {
        let pos = positions(pos_yx, tokens)?;
        let raw = self.inner.raw;
        // SAFETY: live handles; pos is null or holds tokens * 2 values.
        self.call(|| unsafe { vh_vit_block_run(raw, block.raw, x.raw, images, tokens, pos, rope_frequency, epsilon) })
    }

    /// `blocks.len()` blocks in sequence (the 12-layer encoder).
    pub fn encoder_run(&self, blocks: &[&HipBlock], x: &mut HipTensorF32, images: usize, tokens: usize,
                       pos_yx: Option<&[i64]>, rope_frequency: f32, epsilon: f32) -> Result<(), HipError> {
        let pos = positions(pos_yx, tokens)?;
        let raws: Vec<*const VhBlock> = blocks.iter().map(|b| b.raw.cast_const()).collect();
        let raw = self.inner.raw;
        // SAFETY: live handles; raws holds blocks.len() block handles.
        self.call(|| unsafe {
            vh_encoder_run(raw, raws.as_ptr(), raws.len(), x.raw, images, tokens, pos, rope_frequency, epsilon)
        })
    }

    // -- DPT head ----------------------------------------------------------------------

    /// conv2d weights OIHW prepared once (src/conv.rs:174-177 on the CPU side).
    pub fn prepare_conv2d_f32(&self, in_c: usize, out_c: usize, kh: usize, kw: usize, stride: usize, pad: usize,
                              weight: &[f32], bias: Option<&[f32]>) -> Result<HipConv2d, HipError> {
        if weight.len() != out_c * in_c * kh * kw || bias.is_some_and(|b| b.len() != out_c) {
            return Err(HipError::LengthMismatch { destination: out_c * in_c * kh * kw, source_len: weight.len() });
        }
        let mut out = ptr::null_mut();
        let raw = self.inner.raw;
        // SAFETY: lengths checked above.
        self.call(|| unsafe {
            vh_prepare_conv2d_f32(raw, in_c, out_c, kh, kw, stride, pad, weight.as_ptr(), opt_ptr(bias), &mut out)
        })?;
        Ok(HipConv2d { raw: out, runtime: self.clone() })
    }

    /// conv2d (src/conv.rs:877-945) in one call.
    pub fn conv2d_f32(&self, input: &HipTensorF32, in_c: usize, ih: usize, iw: usize, weight: &[f32], out_c: usize,
                      kh: usize, kw: usize, stride: usize, pad: usize, bias: Option<&[f32]>)
        -> Result<HipTensorF32, HipError> {
        if weight.len() != out_c * in_c * kh * kw || bias.is_some_and(|b| b.len() != out_c) {
            return Err(HipError::LengthMismatch { destination: out_c * in_c * kh * kw, source_len: weight.len() });
        }
        let raw = self.inner.raw;
        // SAFETY: lengths checked above.
        self.make(|out| unsafe {
            vh_conv2d_f32(raw, input.raw, in_c, ih, iw, weight.as_ptr(), out_c, kh, kw, stride, pad,
                          opt_ptr(bias), out)
        })
    }

    /// Transposed convolution weights IOHW prepared once (src/conv.rs:83-93).
    pub fn prepare_conv_transpose2d_f32(&self, in_c: usize, out_c: usize, kh: usize, kw: usize, stride: usize,
                                        weight: &[f32], bias: Option<&[f32]>)
        -> Result<HipConvTranspose2d, HipError> {
        if weight.len() != in_c * out_c * kh * kw || bias.is_some_and(|b| b.len() != out_c) {
            return Err(HipError::LengthMismatch { destination: in_c * out_c * kh * kw, source_len: weight.len() });
        }
        let mut out = ptr::null_mut();
        let raw = self.inner.raw;
        // SAFETY: lengths checked above.
        self.call(|| unsafe {
            vh_prepare_conv_transpose2d_f32(raw, in_c, out_c, kh, kw, stride, weight.as_ptr(), opt_ptr(bias), &mut out)
        })?;
        Ok(HipConvTranspose2d { raw: out, runtime: self.clone() })
    }

    /// conv_transpose2d (src/conv.rs:1009-1098) in one call.
    pub fn conv_transpose2d_f32(&self, input: &HipTensorF32, in_c: usize, ih: usize, iw: usize, weight: &[f32],
                                out_c: usize, kh: usize, kw: usize, stride: usize, bias: Option<&[f32]>)
        -> Result<HipTensorF32, HipError> {
        if weight.len() != in_c * out_c * kh * kw || bias.is_some_and(|b| b.len() != out_c) {
            return Err(HipError::LengthMismatch { destination: in_c * out_c * kh * kw, source_len: weight.len() });
        }
        let raw = self.inner.raw;
        // SAFETY: lengths checked above.
        self.make(|out| unsafe {
            vh_conv_transpose2d_f32(raw, input.raw, in_c, ih, iw, weight.as_ptr(), out_c, kh, kw, stride,
                                    opt_ptr(bias), out)
        })
    }

    /// bilinear_resize (src/resample.rs:10-77).
    pub fn bilinear_resize_f32(&self, input: &HipTensorF32, c: usize, ih: usize, iw: usize, oh: usize, ow: usize)
        -> Result<HipTensorF32, HipError> {
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe { vh_bilinear_resize_f32(raw, input.raw, c, ih, iw, oh, ow, out) })
    }

    /// bilinear_resize_align_corners (src/resample.rs:184-245), then + add.
    pub fn bilinear_resize_align_corners_f32(&self, input: &HipTensorF32, c: usize, ih: usize, iw: usize,
                                             oh: usize, ow: usize, add: Option<&HipTensorF32>)
        -> Result<HipTensorF32, HipError> {
        let add = add.map_or(ptr::null(), |t| t.raw.cast_const());
        let raw = self.inner.raw;
        // SAFETY: live handles.
        self.make(|out| unsafe { vh_bilinear_resize_align_corners_f32(raw, input.raw, c, ih, iw, oh, ow, add, out) })
    }

    // -- profiling (device twin of DA3_FLASH_PROFILE, src/specialized.rs:1324) ----

    pub fn profile_enable(&self, enabled: bool) -> Result<(), HipError> {
        let raw = self.inner.raw;
        // SAFETY: live runtime; the lock serialises the mutation.
        self.call(|| unsafe { vh_profile_enable(raw, c_int::from(enabled)) })
    }

    pub fn profile_reset(&self) -> Result<(), HipError> {
        let raw = self.inner.raw;
        // SAFETY: live runtime.
        self.call(|| unsafe { vh_profile_reset(raw) })
    }

    /// "name count total_ms" lines, one per kernel name (synchronising).
    pub fn profile_report(&self) -> Result<String, HipError> {
        let mut buf = vec![0u8; 1 << 16];
        let raw = self.inner.raw;
        // SAFETY: buf is writable for its length; the library NUL-terminates.
        self.call(|| unsafe { vh_profile_report(raw, buf.as_mut_ptr().cast(), buf.len()) })?;
        let end = buf.iter().position(|&b| b == 0).unwrap_or(buf.len());
        Ok(String::from_utf8_lossy(&buf[..end]).into_owned())
    }

    pub fn timer_start(&self) -> Result<(), HipError> {
        let raw = self.inner.raw;
        // SAFETY: live runtime.
        self.call(|| unsafe { vh_timer_start(raw) })
    }

    /// Milliseconds since `timer_start` on the stream (synchronising).
    pub fn timer_stop(&self) -> Result<f32, HipError> {
        let mut ms = 0.0f32;
        let raw = self.inner.raw;
        // SAFETY: live runtime; ms valid for one write.
        self.call(|| unsafe { vh_timer_stop(raw, &mut ms) })?;
        Ok(ms)
    }
}

fn positions(pos_yx: Option<&[i64]>, tokens: usize) -> Result<*const i64, HipError> {
    match pos_yx {
        None => Ok(ptr::null()),
        Some(p) if p.len() == tokens.saturating_mul(2) => Ok(p.as_ptr()),
        Some(p) => Err(HipError::LengthMismatch { destination: tokens.saturating_mul(2), source_len: p.len() }),
    }
}

// ---- prepared projections: CudaLinearF32 (src/cuda.rs:1291-1345) -----------

/// Immutable device-resident parameters of one row-major f32 projection,
/// repacked once for the MFMA kernel.
pub struct HipLinearF32 {
    raw: *mut VhLinear,
    runtime: HipRuntime,
}

// SAFETY: owned device state; every use goes through the runtime's lock.
unsafe impl Send for HipLinearF32 {}
unsafe impl Sync for HipLinearF32 {}

impl Drop for HipLinearF32 {
    fn drop(&mut self) {
        let _g = self.runtime.guard();
        // SAFETY: raw came from vh_prepare_linear_f32 and is freed once.
        unsafe { vh_linear_free(self.raw) }
    }
}

impl HipLinearF32 {
    /// src/cuda.rs:1301-1304
    #[must_use]
    pub fn input_features(&self) -> usize {
        // SAFETY: live handle.
        unsafe { vh_linear_input_features(self.raw) }
    }

    /// src/cuda.rs:1306-1309
    #[must_use]
    pub fn output_features(&self) -> usize {
        // SAFETY: live handle.
        unsafe { vh_linear_output_features(self.raw) }
    }

    /// src/cuda.rs:1312-1334: (input x weight + bias) x gamma, one launch.
    pub fn run(&self, input: &HipTensorF32, rows: usize) -> Result<HipTensorF32, HipError> {
        let raw = self.raw;
        // SAFETY: live handles.
        self.runtime.make(|out| unsafe { vh_linear_run(raw, input.raw, rows, out) })
    }

    /// src/cuda.rs:1340-1344: run, then token-major -> CHW.
    pub fn run_chw(&self, input: &HipTensorF32, rows: usize) -> Result<HipTensorF32, HipError> {
        let raw = self.raw;
        // SAFETY: live handles.
        self.runtime.make(|out| unsafe { vh_linear_run_chw(raw, input.raw, rows, out) })
    }

    /// run + gelu_f32_in_place fused (the fc1 step; gamma must be unit).
    pub fn run_gelu(&self, input: &HipTensorF32, rows: usize) -> Result<HipTensorF32, HipError> {
        let raw = self.raw;
        // SAFETY: live handles.
        self.runtime.make(|out| unsafe { vh_linear_run_gelu(raw, input.raw, rows, out) })
    }

    /// residual += (input x weight + bias) x gamma (out-projection / fc2).
    pub fn run_residual(&self, input: &HipTensorF32, rows: usize, residual: &mut HipTensorF32)
        -> Result<(), HipError> {
        let raw = self.raw;
        // SAFETY: live handles.
        self.runtime.call(|| unsafe { vh_linear_run_residual(raw, input.raw, rows, residual.raw) })
    }

    /// qkv_f32_da3_base (src/specialized.rs:996-1167) on the device: head-major
    /// Q/K/V with bias, and the 2-D RoPE when positions are given.
    pub fn run_qkv_hnd(&self, input: &HipTensorF32, images: usize, tokens: usize, heads: usize,
                       pos_yx: Option<&[i64]>, frequency: f32)
        -> Result<(HipTensorF32, HipTensorF32, HipTensorF32), HipError> {
        let pos = positions(pos_yx, tokens)?;
        let (mut q, mut k, mut v) = (ptr::null_mut(), ptr::null_mut(), ptr::null_mut());
        let raw = self.raw;
        // SAFETY: live handles; pos null or tokens * 2 values.
        self.runtime.call(|| unsafe {
            vh_linear_run_qkv_hnd(raw, input.raw, images, tokens, heads, pos, frequency, &mut q, &mut k, &mut v)
        })?;
        Ok((self.runtime.tensor(q), self.runtime.tensor(k), self.runtime.tensor(v)))
    }
}

// ---- Q8_0 -------------------------------------------------------------------

/// Rows of BlockQ8_0 held on the device (values and scales as two arrays).
pub struct HipQ8Tensor {
    raw: *mut VhQ8Tensor,
    runtime: HipRuntime,
}

// SAFETY: owned device state; every use goes through the runtime's lock.
unsafe impl Send for HipQ8Tensor {}
unsafe impl Sync for HipQ8Tensor {}

impl Drop for HipQ8Tensor {
    fn drop(&mut self) {
        let _g = self.runtime.guard();
        // SAFETY: raw came from the library and is freed once.
        unsafe { vh_q8_tensor_free(self.raw) }
    }
}

impl HipQ8Tensor {
    #[must_use]
    pub fn rows(&self) -> usize {
        // SAFETY: live handle.
        unsafe { vh_q8_tensor_rows(self.raw) }
    }

    #[must_use]
    pub fn k(&self) -> usize {
        // SAFETY: live handle.
        unsafe { vh_q8_tensor_k(self.raw) }
    }
}

/// A projection whose weights are GGUF-style BlockQ8_0 rows of W^T.
pub struct HipLinearQ8 {
    raw: *mut VhLinearQ8,
    runtime: HipRuntime,
}

// SAFETY: owned device state; every use goes through the runtime's lock.
unsafe impl Send for HipLinearQ8 {}
unsafe impl Sync for HipLinearQ8 {}

impl Drop for HipLinearQ8 {
    fn drop(&mut self) {
        let _g = self.runtime.guard();
        // SAFETY: raw came from vh_prepare_linear_q8_0 and is freed once.
        unsafe { vh_linear_q8_0_free(self.raw) }
    }
}

impl HipLinearQ8 {
    #[must_use]
    pub fn input_features(&self) -> usize {
        // SAFETY: live handle.
        unsafe { vh_linear_q8_0_input_features(self.raw) }
    }

    #[must_use]
    pub fn output_features(&self) -> usize {
        // SAFETY: live handle.
        unsafe { vh_linear_q8_0_output_features(self.raw) }
    }

    /// (gemm_q8_0(quantize(input), W) + bias) * gamma
    pub fn run(&self, input: &HipTensorF32, rows: usize) -> Result<HipTensorF32, HipError> {
        let raw = self.raw;
        // SAFETY: live handles.
        self.runtime.make(|out| unsafe { vh_linear_q8_0_run(raw, input.raw, rows, out) })
    }

    /// gelu(gemm_q8_0(quantize(input), W) + bias)
    pub fn run_gelu(&self, input: &HipTensorF32, rows: usize) -> Result<HipTensorF32, HipError> {
        let raw = self.raw;
        // SAFETY: live handles.
        self.runtime.make(|out| unsafe { vh_linear_q8_0_run_gelu(raw, input.raw, rows, out) })
    }

    /// residual += (gemm_q8_0(quantize(input), W) + bias) * gamma
    pub fn run_residual(&self, input: &HipTensorF32, rows: usize, residual: &mut HipTensorF32)
        -> Result<(), HipError> {
        let raw = self.raw;
        // SAFETY: live handles.
        self.runtime.call(|| unsafe { vh_linear_q8_0_run_residual(raw, input.raw, rows, residual.raw) })
    }
}

// ---- DA3-BASE block ------------------------------------------------------------

/// One block's parameters, row-major [in, out] weights; the four Q/K
/// LayerNorm vectors ([64] each) are set together for DA3's late blocks.
pub struct BlockParams<'a> {
    pub ln1_gamma: &'a [f32],
    pub ln1_beta: &'a [f32],
    pub w_qkv: &'a [f32],
    pub b_qkv: &'a [f32],
    pub w_proj: &'a [f32],
    pub b_proj: &'a [f32],
    pub ls1: &'a [f32],
    pub ln2_gamma: &'a [f32],
    pub ln2_beta: &'a [f32],
    pub w_fc1: &'a [f32],
    pub b_fc1: &'a [f32],
    pub w_fc2: &'a [f32],
    pub b_fc2: &'a [f32],
    pub ls2: &'a [f32],
    pub qk_norm: Option<[&'a [f32]; 4]>,
}

impl BlockParams<'_> {
    fn validate(&self) -> Result<(), HipError> {
        const D: usize = 768;
        const F: usize = 3072;
        let expect: [(&[f32], usize); 14] = [
            (self.ln1_gamma, D), (self.ln1_beta, D), (self.w_qkv, D * 3 * D), (self.b_qkv, 3 * D),
            (self.w_proj, D * D), (self.b_proj, D), (self.ls1, D), (self.ln2_gamma, D), (self.ln2_beta, D),
            (self.w_fc1, D * F), (self.b_fc1, F), (self.w_fc2, F * D), (self.b_fc2, D), (self.ls2, D),
        ];
        for (v, n) in expect {
            if v.len() != n {
                return Err(HipError::LengthMismatch { destination: n, source_len: v.len() });
            }
        }
        if let Some(qk) = &self.qk_norm {
            for v in qk {
                if v.len() != 64 {
                    return Err(HipError::LengthMismatch { destination: 64, source_len: v.len() });
                }
            }
        }
        Ok(())
    }

    fn raw(&self) -> VhBlockParams {
        let qk = self.qk_norm.map_or([ptr::null(); 4], |q| [q[0].as_ptr(), q[1].as_ptr(), q[2].as_ptr(), q[3].as_ptr()]);
        VhBlockParams {
            ln1_gamma: self.ln1_gamma.as_ptr(),
            ln1_beta: self.ln1_beta.as_ptr(),
            w_qkv: self.w_qkv.as_ptr(),
            b_qkv: self.b_qkv.as_ptr(),
            w_proj: self.w_proj.as_ptr(),
            b_proj: self.b_proj.as_ptr(),
            ls1: self.ls1.as_ptr(),
            ln2_gamma: self.ln2_gamma.as_ptr(),
            ln2_beta: self.ln2_beta.as_ptr(),
            w_fc1: self.w_fc1.as_ptr(),
            b_fc1: self.b_fc1.as_ptr(),
            w_fc2: self.w_fc2.as_ptr(),
            b_fc2: self.b_fc2.as_ptr(),
            ls2: self.ls2.as_ptr(),
            q_norm_gamma: qk[0],
            q_norm_beta: qk[1],
            k_norm_gamma: qk[2],
            k_norm_beta: qk[3],
        }
    }
}

/// A prepared DA3-BASE encoder block (f32 or Q8_0 projections).
pub struct HipBlock {
    raw: *mut VhBlock,
    runtime: HipRuntime,
}

// SAFETY: owned device state; every use goes through the runtime's lock.
unsafe impl Send for HipBlock {}
unsafe impl Sync for HipBlock {}

impl Drop for HipBlock {
    fn drop(&mut self) {
        let _g = self.runtime.guard();
        // SAFETY: raw came from vh_block_prepare* and is freed once.
        unsafe { vh_block_free(self.raw) }
    }
}

impl HipBlock {
    #[must_use]
    pub fn is_q8_0(&self) -> bool {
        // SAFETY: live handle.
        unsafe { vh_block_is_q8_0(self.raw) != 0 }
    }
}

// ---- DPT head ---------------------------------------------------------------------

/// A prepared 2-D convolution (CHW tensors, batch 1, as src/conv.rs).
pub struct HipConv2d {
    raw: *mut VhConv2d,
    runtime: HipRuntime,
}

// SAFETY: owned device state; every use goes through the runtime's lock.
unsafe impl Send for HipConv2d {}
unsafe impl Sync for HipConv2d {}

impl Drop for HipConv2d {
    fn drop(&mut self) {
        let _g = self.runtime.guard();
        // SAFETY: raw came from vh_prepare_conv2d_f32 and is freed once.
        unsafe { vh_conv2d_free(self.raw) }
    }
}

impl HipConv2d {
    #[must_use]
    pub fn output_height(&self, ih: usize) -> usize {
        // SAFETY: live handle.
        unsafe { vh_conv2d_output_height(self.raw, ih) }
    }

    #[must_use]
    pub fn output_width(&self, iw: usize) -> usize {
        // SAFETY: live handle.
        unsafe { vh_conv2d_output_width(self.raw, iw) }
    }

    /// conv3x3_winograd_f2_prepared (src/conv.rs:282-293) for any kernel.
    pub fn run(&self, input: &HipTensorF32, ih: usize, iw: usize) -> Result<HipTensorF32, HipError> {
        let raw = self.raw;
        // SAFETY: live handles.
        self.runtime.make(|out| unsafe { vh_conv2d_run(raw, input.raw, ih, iw, out) })
    }

    /// conv3x3_winograd_f2_prepared_relu_input (src/conv.rs:651-679).
    pub fn run_relu_input(&self, input: &HipTensorF32, ih: usize, iw: usize) -> Result<HipTensorF32, HipError> {
        let raw = self.raw;
        // SAFETY: live handles.
        self.runtime.make(|out| unsafe { vh_conv2d_run_relu_input(raw, input.raw, ih, iw, out) })
    }

    /// conv3x3_winograd_f2_prepared_resize_align_corners (src/conv.rs:304-320).
    pub fn run_resize_align_corners(&self, input: &HipTensorF32, ih: usize, iw: usize, oh: usize, ow: usize,
                                    add: Option<&HipTensorF32>) -> Result<HipTensorF32, HipError> {
        let add = add.map_or(ptr::null(), |t| t.raw.cast_const());
        let raw = self.raw;
        // SAFETY: live handles.
        self.runtime.make(|out| unsafe { vh_conv2d_run_resize_align_corners(raw, input.raw, ih, iw, oh, ow, add, out) })
    }
}

/// A prepared transposed convolution (src/conv.rs:83-105).
pub struct HipConvTranspose2d {
    raw: *mut VhConvTranspose2d,
    runtime: HipRuntime,
}

// SAFETY: owned device state; every use goes through the runtime's lock.
unsafe impl Send for HipConvTranspose2d {}
unsafe impl Sync for HipConvTranspose2d {}

impl Drop for HipConvTranspose2d {
    fn drop(&mut self) {
        let _g = self.runtime.guard();
        // SAFETY: raw came from vh_prepare_conv_transpose2d_f32 and is freed once.
        unsafe { vh_conv_transpose2d_free(self.raw) }
    }
}

impl HipConvTranspose2d {
    /// conv_transpose2d_prepared (src/conv.rs:95-105).
    pub fn run(&self, input: &HipTensorF32, ih: usize, iw: usize) -> Result<HipTensorF32, HipError> {
        let raw = self.raw;
        // SAFETY: live handles.
        self.runtime.make(|out| unsafe { vh_conv_transpose2d_run(raw, input.raw, ih, iw, out) })
    }
}

// ---- names of src/cuda.rs, for engine code written against it -------------------

pub type CudaRuntime = HipRuntime;
pub type CudaTensorF32 = HipTensorF32;
pub type CudaLinearF32 = HipLinearF32;
pub type CudaError = HipError;
