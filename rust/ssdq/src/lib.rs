//! `GpuCompute`: the methods of ssd-llm's `MetalCompute` that the quantized path uses
//! (`src/metal/compute.rs:47-71`, `157-191`, `217-264`), plus the loader's and the swap
//! file's host helpers (`src/ssd/streamer.rs:93-125`, `src/ssd/block_swap.rs:36-74`), on
//! libssdq.  dtype arguments are `GgmlType` ids (`src/model/gguf.rs:17-48`): a caller passes
//! `dtype as i32`.  Resident weights (`ResidentWeights`) keep a layer's raw GGUF bytes in HBM
//! for the device entry points (`ssdq_sys::ssdq_decode_layer_dev` and the `_dev` family).
pub use ssdq_sys as ffi;

use std::ffi::{CStr, CString};
use std::fmt;
use std::os::raw::{c_int, c_void};
use std::sync::OnceLock;

/// A negative libssdq status with the library's message for it.
#[derive(Debug, Clone)]
pub struct SsdqError {
    pub code: i32,
    pub message: String,
}

impl fmt::Display for SsdqError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        write!(f, "libssdq error {}: {}", self.code, self.message)
    }
}

impl std::error::Error for SsdqError {}

/// The calling thread's last libssdq error message.
pub fn last_error() -> String {
    let p = unsafe { ffi::ssdq_last_error() };
    if p.is_null() {
        return String::new();
    }
    unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
}

/// Status -> Result: negative codes are errors; 0 and SSDQ_WARN_UNSUPPORTED_ZEROED (the
/// output was zero-filled, as the reference's matvec does for unsupported types) pass.
pub fn check(rc: c_int) -> Result<c_int, SsdqError> {
    if rc < 0 {
        Err(SsdqError { code: rc, message: last_error() })
    } else {
        Ok(rc)
    }
}

pub struct GpuCompute {
    ctx: *mut ffi::ssdq_ctx,
}

// The library serializes calls on one context.
unsafe impl Send for GpuCompute {}
unsafe impl Sync for GpuCompute {}

impl GpuCompute {
    /// `MetalCompute::new() -> Option<Self>` (compute.rs:47-71): None when no GPU is usable,
    /// and the caller keeps its CPU path.
    pub fn new() -> Option<Self> {
        let mut ctx = std::ptr::null_mut();
        let rc = unsafe { ffi::ssdq_ctx_create(-1, &mut ctx) };
        (rc == ffi::SSDQ_OK && !ctx.is_null()).then_some(Self { ctx })
    }

    /// One context per process.  The reference builds a `MetalCompute` per forward pass
    /// (transformer.rs:301-302) and per token for the output head (:704); with device
    /// buffers and streams behind it, one shared context is the cheaper equivalent.
    pub fn global() -> Option<&'static GpuCompute> {
        static G: OnceLock<Option<GpuCompute>> = OnceLock::new();
        G.get_or_init(GpuCompute::new).as_ref()
    }

    /// `MetalCompute::has_gpu` (compute.rs:261-263).
    pub fn has_gpu(&self) -> bool {
        true
    }

    /// The HIP device ordinal this context runs on.
    pub fn device(&self) -> i32 {
        unsafe { ffi::ssdq_ctx_device(self.ctx) }
    }

    /// `MetalCompute::matvec_quantized` (compute.rs:157-191): y[out_dim] = W x for raw GGUF
    /// bytes `w_raw` of type `dtype`.  Unsupported types give zeros (compute.rs:672-675).
    /// Panics where the reference would index out of bounds (a short `w_raw` or `x`).
    pub fn matvec_quantized(&self, w_raw: &[u8], x: &[f32], out_dim: usize, in_dim: usize, dtype: i32) -> Vec<f32> {
        let mut y = vec![0.0f32; out_dim];
        let rc = unsafe {
            ffi::ssdq_matvec_quantized(self.ctx, w_raw.as_ptr(), w_raw.len(), x.as_ptr(), x.len(), out_dim, in_dim,
                                       dtype, y.as_mut_ptr())
        };
        if let Err(e) = check(rc) {
            panic!("matvec_quantized: {e}");
        }
        y
    }

    /// `MetalCompute::flash_attention_f32` (compute.rs:217-258): one query position over
    /// positions [window_start, min(window_end, seq_len)) of f32 K/V caches laid out
    /// [seq_len, n_head_kv, head_dim].  None below seq_len 4 (compute.rs:232: the caller's
    /// CPU path), as the reference.
    #[allow(clippy::too_many_arguments)]
    pub fn flash_attention_f32(&self, q_heads: &[f32], k_cache: &[f32], v_cache: &[f32], n_head: usize,
                               n_head_kv: usize, head_dim: usize, seq_len: usize, window_start: usize,
                               window_end: usize) -> Option<Vec<f32>> {
        if seq_len < 4 {
            return None;
        }
        let mut out = vec![0.0f32; n_head * head_dim];
        let rc = unsafe {
            ffi::ssdq_flash_attention_f32(self.ctx, q_heads.as_ptr(), k_cache.as_ptr(), v_cache.as_ptr(), n_head,
                                          n_head_kv, head_dim, seq_len, window_start, window_end,
                                          out.as_mut_ptr())
        };
        check(rc).ok().map(|_| out)
    }

    /// `dequantize_to_f32` (streamer.rs:93-125): the f32 elements of `n_elements` of a tensor.
    pub fn dequantize_to_f32(&self, data: &[u8], dtype: i32, n_elements: usize) -> Result<Vec<f32>, SsdqError> {
        let mut out = vec![0.0f32; n_elements];
        let rc = unsafe {
            ffi::ssdq_dequantize_to_f32(self.ctx, dtype, data.as_ptr(), data.len(), n_elements, out.as_mut_ptr())
        };
        check(rc).map(|_| out)
    }

    /// `quantize_vectors_int8` (block_swap.rs:36-60): per-row absmax INT8 codes and scales
    /// of `data.len() / dim` rows, bit-identical to the reference's.
    pub fn quantize_vectors_int8(&self, data: &[f32], dim: usize) -> (Vec<i8>, Vec<f32>) {
        let n_rows = if dim == 0 { 0 } else { data.len() / dim };
        let mut codes = vec![0i8; n_rows * dim];
        let mut scales = vec![0.0f32; n_rows];
        let rc = unsafe {
            ffi::ssdq_quantize_vectors_int8(self.ctx, data.as_ptr(), n_rows, dim, codes.as_mut_ptr(),
                                            scales.as_mut_ptr())
        };
        if let Err(e) = check(rc) {
            panic!("quantize_vectors_int8: {e}");
        }
        (codes, scales)
    }

    /// `dequantize_vectors_int8` (block_swap.rs:63-74).
    pub fn dequantize_vectors_int8(&self, quantized: &[i8], scales: &[f32], dim: usize) -> Vec<f32> {
        let n_rows = scales.len();
        let mut out = vec![0.0f32; quantized.len()];
        let rc = unsafe {
            ffi::ssdq_dequantize_vectors_int8(self.ctx, quantized.as_ptr(), scales.as_ptr(), n_rows, dim,
                                              out.as_mut_ptr())
        };
        if let Err(e) = check(rc) {
            panic!("dequantize_vectors_int8: {e}");
        }
        out
    }
}

impl Drop for GpuCompute {
    fn drop(&mut self) {
        unsafe { ffi::ssdq_ctx_destroy(self.ctx) }
    }
}

/// A resident tensor: device pointer to its raw GGUF bytes, type and shape.
#[derive(Debug, Clone, Copy)]
pub struct ResidentTensor {
    pub data: *const c_void,
    pub dtype: i32,
    pub dims: [u64; 4],
    pub n_dims: usize,
    pub n_bytes: usize,
}

/// Raw GGUF tensors kept in HBM by name: replaces `SsdStreamer::load_layer` /
/// `load_tensor_f32` (streamer.rs:33-66), which dequantize every tensor on each load, and
/// `find_tensor_in_layer` (transformer.rs:552-559).
pub struct ResidentWeights {
    w: *mut ffi::ssdq_weights,
}

unsafe impl Send for ResidentWeights {}
unsafe impl Sync for ResidentWeights {}

impl ResidentWeights {
    pub fn new(device: i32) -> Result<Self, SsdqError> {
        let mut w = std::ptr::null_mut();
        check(unsafe { ffi::ssdq_weights_create(device, &mut w) })?;
        Ok(Self { w })
    }

    /// Uploads one tensor's mapped bytes (`get_tensor_data(offset, size_bytes)`) once.
    pub fn put(&self, name: &str, dtype: i32, dims: &[u64], data: &[u8]) -> Result<(), SsdqError> {
        let name = CString::new(name).map_err(|_| SsdqError { code: ffi::SSDQ_ERR_INVALID_ARG,
                                                              message: "tensor name holds a NUL".into() })?;
        check(unsafe {
            ffi::ssdq_weights_put(self.w, name.as_ptr(), dtype, dims.as_ptr(), dims.len(),
                                  data.as_ptr() as *const c_void, data.len())
        })
        .map(|_| ())
    }

    /// `find_tensor_in_layer`: `blk.{layer}.{suffix}`, None when absent.
    pub fn find_tensor_in_layer(&self, layer_idx: u32, suffix: &str) -> Option<ResidentTensor> {
        self.find(&format!("blk.{layer_idx}.{suffix}"))
    }

    pub fn find(&self, name: &str) -> Option<ResidentTensor> {
        let name = CString::new(name).ok()?;
        let mut t = ResidentTensor { data: std::ptr::null(), dtype: 0, dims: [0; 4], n_dims: 0, n_bytes: 0 };
        let p = unsafe {
            ffi::ssdq_weights_find(self.w, name.as_ptr(), &mut t.dtype, t.dims.as_mut_ptr(), &mut t.n_dims,
                                   &mut t.n_bytes)
        };
        (!p.is_null()).then(|| ResidentTensor { data: p, ..t })
    }

    pub fn count(&self) -> usize {
        unsafe { ffi::ssdq_weights_count(self.w) }
    }

    pub fn bytes(&self) -> usize {
        unsafe { ffi::ssdq_weights_bytes(self.w) }
    }

    /// The handle for `ffi::ssdq_decode_layer_dev`.
    pub fn as_ptr(&self) -> *const ffi::ssdq_weights {
        self.w
    }
}

impl Drop for ResidentWeights {
    fn drop(&mut self) {
        unsafe { ffi::ssdq_weights_destroy(self.w) }
    }
}
