//! Raw `extern "C"` bindings to libssdq, one declaration per function of `include/ssdq.h`,
//! in the header's order and with the header's argument names.  C types map as:
//! `int` -> `c_int`, `size_t` -> `usize`, `float` -> `f32`, `T*` -> `*mut T`,
//! `const T*` -> `*const T`, `void*` -> `c_void` pointers, `ssdq_stream_t` (a
//! `hipStream_t`) -> `ssdq_stream_t`.  `tests/test_rust_binding.py` in the
//! repository checks this file against the header.
#![allow(non_camel_case_types)]
use std::os::raw::{c_char, c_int, c_void};

pub const SSDQ_ABI_VERSION: c_int = 1;

pub const SSDQ_OK: c_int = 0;
pub const SSDQ_WARN_UNSUPPORTED_ZEROED: c_int = 1;
pub const SSDQ_ERR_INVALID_ARG: c_int = -1;
pub const SSDQ_ERR_UNSUPPORTED: c_int = -2;
pub const SSDQ_ERR_HIP: c_int = -3;
pub const SSDQ_ERR_NO_DEVICE: c_int = -4;
pub const SSDQ_ERR_OUT_OF_MEMORY: c_int = -5;

// GgmlType ids (src/model/gguf.rs:17-48)
pub const SSDQ_TYPE_F32: c_int = 0;
pub const SSDQ_TYPE_F16: c_int = 1;
pub const SSDQ_TYPE_Q4_0: c_int = 2;
pub const SSDQ_TYPE_Q8_0: c_int = 8;
pub const SSDQ_TYPE_Q2_K: c_int = 10;
pub const SSDQ_TYPE_Q3_K: c_int = 11;
pub const SSDQ_TYPE_Q4_K: c_int = 12;
pub const SSDQ_TYPE_Q5_K: c_int = 13;
pub const SSDQ_TYPE_Q6_K: c_int = 14;
pub const SSDQ_TYPE_Q8_K: c_int = 15;
pub const SSDQ_TYPE_IQ2_XXS: c_int = 16;
pub const SSDQ_TYPE_IQ2_XS: c_int = 17;
pub const SSDQ_TYPE_IQ3_XXS: c_int = 18;
pub const SSDQ_TYPE_IQ4_NL: c_int = 20;
pub const SSDQ_TYPE_IQ3_S: c_int = 21;
pub const SSDQ_TYPE_IQ4_XS: c_int = 23;
pub const SSDQ_TYPE_BF16: c_int = 30;

/// A `hipStream_t`; null is the default stream.
pub type ssdq_stream_t = *mut c_void;

#[repr(C)]
pub struct ssdq_ctx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct ssdq_weights {
    _p: [u8; 0],
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct ssdq_layer_config {
    pub n_embd: usize,
    pub n_head: usize,
    pub n_head_kv: usize,
    pub head_dim: usize,
    pub n_ff: usize,
    pub rope_theta: f32,
    pub norm_eps: f32,
}

// Regions of the decode layer's scratch (ssdq_decode_layer_scratch_bytes offsets)
pub const SSDQ_LAYER_ATTN_IN: usize = 0;
pub const SSDQ_LAYER_Q: usize = 1;
pub const SSDQ_LAYER_K: usize = 2;
pub const SSDQ_LAYER_V: usize = 3;
pub const SSDQ_LAYER_ATTN: usize = 4;
pub const SSDQ_LAYER_ATTN_OUT: usize = 5;
pub const SSDQ_LAYER_FFN_IN: usize = 6;
pub const SSDQ_LAYER_FFN_H: usize = 7;
pub const SSDQ_LAYER_FFN_GATE: usize = 8;
pub const SSDQ_LAYER_FFN_UP: usize = 9;
pub const SSDQ_LAYER_FFN_OUT: usize = 10;
pub const SSDQ_LAYER_NORM_W: usize = 11;
pub const SSDQ_LAYER_HIDDEN_MID: usize = 12;
pub const SSDQ_LAYER_N_STAGES: usize = 13;

extern "C" {
    pub fn ssdq_abi_version() -> c_int;
    pub fn ssdq_last_error() -> *const c_char;
    pub fn ssdq_block_size(dtype: c_int) -> usize;
    pub fn ssdq_type_size(dtype: c_int) -> usize;
    pub fn ssdq_row_bytes(dtype: c_int, in_dim: usize) -> usize;

    pub fn ssdq_ctx_create(device: c_int, out: *mut *mut ssdq_ctx) -> c_int;
    pub fn ssdq_ctx_destroy(ctx: *mut ssdq_ctx);
    pub fn ssdq_ctx_device(ctx: *const ssdq_ctx) -> c_int;

    // per-stream workspace: grow before a HIP graph capture; free what growth retired
    pub fn ssdq_reserve_workspace(bytes: usize, stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_release_workspaces() -> c_int;

    // GGUF dequantization (streamer.rs:93-125)
    pub fn ssdq_dequant_dev(dtype: c_int, w: *const c_void, n_elements: usize, out: *mut f32,
                            stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_dequantize_to_f32(ctx: *mut ssdq_ctx, dtype: c_int, data: *const u8, data_len: usize,
                                  n_elements: usize, out: *mut f32) -> c_int;

    // quantized matvec (MetalCompute::matvec_quantized, compute.rs:157-191; batches:
    // batch_scheduler.rs:242-276)
    pub fn ssdq_matvec_dev(dtype: c_int, w: *const c_void, x: *const f32, y: *mut f32, out_dim: usize,
                           in_dim: usize, batch: usize, stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_matvec_quantized(ctx: *mut ssdq_ctx, w_raw: *const u8, w_len: usize, x: *const f32,
                                 x_len: usize, out_dim: usize, in_dim: usize, dtype: c_int,
                                 y: *mut f32) -> c_int;

    // INT8 KV swap slots (SwapQuantMode::Int8, block_swap.rs:148-370)
    pub fn ssdq_kv_slot_bytes(block_size: usize, kv_dim: usize) -> usize;
    pub fn ssdq_kv_swap_out_dev(k_codes: *const i8, k_scales: *const f32, v_codes: *const i8,
                                v_scales: *const f32, block_ids: *const i32, num_filled: *const u32,
                                n_blocks: usize, block_size: usize, kv_dim: usize, n_pool_blocks: usize,
                                slots: *mut c_void, stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_kv_swap_in_dev(slots: *const c_void, block_ids: *const i32, n_blocks: usize,
                               block_size: usize, kv_dim: usize, n_pool_blocks: usize, k_codes: *mut i8,
                               k_scales: *mut f32, v_codes: *mut i8, v_scales: *mut f32,
                               num_filled: *mut u32, stream: ssdq_stream_t) -> c_int;

    // decode-layer ops on quantized weights (batch 1)
    pub fn ssdq_qkv_rope_dev(dtype_q: c_int, wq: *const c_void, dtype_k: c_int, wk: *const c_void,
                             dtype_v: c_int, wv: *const c_void, x: *const f32, q: *mut f32, k: *mut f32,
                             v: *mut f32, q_dim: usize, kv_dim: usize, n_embd: usize, head_dim: usize,
                             position: usize, theta_base: f32, stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_swiglu_dev(dtype: c_int, w_gate: *const c_void, w_up: *const c_void, x: *const f32,
                           h: *mut f32, n_ff: usize, n_embd: usize, stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_rmsnorm_matvec_dev(dtype: c_int, w: *const c_void, x: *const f32, norm_weight: *const f32,
                                   eps: f32, y: *mut f32, out_dim: usize, n_embd: usize,
                                   stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_rmsnorm_dev(x: *const f32, residual: *const f32, weight: *const f32, eps: f32,
                            hidden_out: *mut f32, out: *mut f32, n: usize, stream: ssdq_stream_t) -> c_int;

    // prefill GEMM (transformer.rs:166-196 runs it as one matvec per token)
    pub fn ssdq_gemm_q4k_bf16_dev(w: *const c_void, x_bf16: *const u16, y: *mut f32, M: usize, N: usize,
                                  K: usize, stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_gemm_q4k_bf16_multi_dev(w: *const *const c_void, n: *const usize, count: usize,
                                        x_bf16: *const u16, y: *const *mut f32, M: usize, K: usize,
                                        stream: ssdq_stream_t) -> c_int;

    // INT8 per-row KV quantization (block_swap.rs:36-74 = quantized_kv_cache.rs:23-53)
    pub fn ssdq_kv_quantize_rows_dev(r#in: *const f32, codes: *mut i8, scales: *mut f32, n_rows: usize,
                                     row_len: usize, stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_kv_dequantize_rows_dev(codes: *const i8, scales: *const f32, out: *mut f32, n_rows: usize,
                                       row_len: usize, stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_quantize_vectors_int8(ctx: *mut ssdq_ctx, data: *const f32, n_rows: usize, dim: usize,
                                      codes: *mut i8, scales: *mut f32) -> c_int;
    pub fn ssdq_dequantize_vectors_int8(ctx: *mut ssdq_ctx, codes: *const i8, scales: *const f32,
                                        n_rows: usize, dim: usize, out: *mut f32) -> c_int;

    // paged INT8 KV cache and decode attention (paged_attention.rs, flash_attention.rs)
    pub fn ssdq_paged_kv_append_dev(k: *const f32, v: *const f32, slot_mapping: *const i32,
                                    k_codes: *mut i8, k_scales: *mut f32, v_codes: *mut i8,
                                    v_scales: *mut f32, n_tokens: usize, kv_dim: usize,
                                    stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_paged_attention_int8_dev(q: *const f32, k_codes: *const i8, k_scales: *const f32,
                                         v_codes: *const i8, v_scales: *const f32, block_tables: *const i32,
                                         ctx_lens: *const i32, out: *mut f32, n_seq: usize, n_head: usize,
                                         n_head_kv: usize, head_dim: usize, block_size: usize,
                                         max_blocks_per_seq: usize, max_ctx: usize,
                                         stream: ssdq_stream_t) -> c_int;
    // positions [window_starts[s], min(window_ends[s], ctx_lens[s])) per sequence
    // (flash_attention_windowed, flash_attention.rs:146-227); null arrays = [0, ctx_len)
    pub fn ssdq_paged_attention_int8_window_dev(q: *const f32, k_codes: *const i8, k_scales: *const f32,
                                                v_codes: *const i8, v_scales: *const f32,
                                                block_tables: *const i32, ctx_lens: *const i32,
                                                window_starts: *const i32, window_ends: *const i32,
                                                out: *mut f32, n_seq: usize, n_head: usize, n_head_kv: usize,
                                                head_dim: usize, block_size: usize, max_blocks_per_seq: usize,
                                                max_ctx: usize, stream: ssdq_stream_t) -> c_int;
    // allocation-free twin of ssdq_paged_attention_int8_dev for callers that cannot allocate
    // (graph capture, serving loops): partials in a 16 MiB static device scratch per GPU,
    // larger calls rejected, overlapping calls on one GPU race (serialize them)
    pub fn ssdq_paged_attention_int8_noalloc_dev(q: *const f32, k_codes: *const i8, k_scales: *const f32,
                                                 v_codes: *const i8, v_scales: *const f32,
                                                 block_tables: *const i32, ctx_lens: *const i32,
                                                 out: *mut f32, n_seq: usize, n_head: usize,
                                                 n_head_kv: usize, head_dim: usize, block_size: usize,
                                                 max_blocks_per_seq: usize, max_ctx: usize,
                                                 stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_flash_attention_f32_dev(q: *const f32, k: *const f32, v: *const f32, out: *mut f32,
                                        n_head: usize, n_head_kv: usize, head_dim: usize, seq_len: usize,
                                        window_start: usize, window_end: usize,
                                        stream: ssdq_stream_t) -> c_int;
    pub fn ssdq_flash_attention_f32(ctx: *mut ssdq_ctx, q: *const f32, k: *const f32, v: *const f32,
                                    n_head: usize, n_head_kv: usize, head_dim: usize, seq_len: usize,
                                    window_start: usize, window_end: usize, out: *mut f32) -> c_int;

    // resident GGUF tensors (raw bytes in HBM, found by name)
    pub fn ssdq_weights_create(device: c_int, out: *mut *mut ssdq_weights) -> c_int;
    pub fn ssdq_weights_destroy(w: *mut ssdq_weights);
    pub fn ssdq_weights_put(w: *mut ssdq_weights, name: *const c_char, dtype: c_int, dims: *const u64,
                            n_dims: usize, data: *const c_void, data_len: usize) -> c_int;
    pub fn ssdq_weights_find(w: *const ssdq_weights, name: *const c_char, dtype: *mut c_int, dims: *mut u64,
                             n_dims: *mut usize, n_bytes: *mut usize) -> *const c_void;
    pub fn ssdq_weights_count(w: *const ssdq_weights) -> usize;
    pub fn ssdq_weights_bytes(w: *const ssdq_weights) -> usize;
    pub fn ssdq_weights_device(w: *const ssdq_weights) -> c_int;

    // one decoder layer for one token from resident tensors, KV in the paged INT8 pool
    pub fn ssdq_decode_layer_scratch_bytes(cfg: *const ssdq_layer_config, offsets: *mut usize) -> usize;
    pub fn ssdq_decode_layer_dev(w: *const ssdq_weights, layer: u32, cfg: *const ssdq_layer_config,
                                 hidden: *mut f32, position: usize, k_codes: *mut i8, k_scales: *mut f32,
                                 v_codes: *mut i8, v_scales: *mut f32, block_size: usize,
                                 block_table: *const i32, max_blocks_per_seq: usize, slot_mapping: *const i32,
                                 ctx_len: *const i32, max_ctx: usize, scratch: *mut c_void,
                                 scratch_bytes: usize, stream: ssdq_stream_t) -> c_int;

    // testing: the byte-addressed matvec kernel that unaligned weights take
    pub fn ssdq_matvec_generic_dev(dtype: c_int, w: *const c_void, x: *const f32, y: *mut f32,
                                   out_dim: usize, in_dim: usize, batch: usize,
                                   stream: ssdq_stream_t) -> c_int;
}
