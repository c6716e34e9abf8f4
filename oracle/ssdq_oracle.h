/*
 * ssdq_oracle.h — CPU oracle for the ssd-llm quantized compute path.
 *
 * TEST INFRASTRUCTURE ONLY. This is not part of the product: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker or as the timed CPU baseline. The product library
 * (libssdq.so) never links or calls it.
 *
 * It restates the reference's Rust CPU path op for op (every a*b+c is two
 * IEEE roundings: the file is built with -ffp-contract=off). Each function
 * cites the reference file:line it follows (paths relative to the
 * ssd-llm source tree). The reference is Rust and cannot be compiled in this
 * image (no cargo/rustc), so there is no oracle/_ref build.
 */
#ifndef SSDQ_ORACLE_H
#define SSDQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GgmlType ids, src/model/gguf.rs:17-48 */
enum {
    SSDO_F32 = 0, SSDO_F16 = 1, SSDO_Q4_0 = 2, SSDO_Q8_0 = 8,
    SSDO_Q2_K = 10, SSDO_Q3_K = 11, SSDO_Q4_K = 12, SSDO_Q5_K = 13, SSDO_Q6_K = 14,
    SSDO_Q8_K = 15, SSDO_IQ2_XXS = 16, SSDO_IQ2_XS = 17, SSDO_IQ3_XXS = 18, SSDO_IQ4_NL = 20,
    SSDO_IQ3_S = 21, SSDO_IQ4_XS = 23, SSDO_BF16 = 30
};

/* block_size / type_size, src/model/gguf.rs:87-135 (0 for unknown ids) */
size_t ssdo_block_size(int dtype);
size_t ssdo_type_size(int dtype);

/* half::f16::to_f32 as called by f16_to_f32, src/metal/compute.rs:2243-2246 */
float ssdo_f16_to_f32(uint16_t h);
void ssdo_f16_to_f32_array(const uint16_t* h, size_t n, float* out);
/* bf16 widening, src/ssd/streamer.rs:108-114 */
float ssdo_bf16_to_f32(uint16_t h);

/* Load-time dequantization, src/ssd/streamer.rs:93-220.  Q4_K has no
 * standalone reference dequantizer (streamer.rs:119-123 returns zeros); its
 * element values are the ones matvec_q4_k_cpu forms, src/metal/compute.rs:718-744.
 * `data_len` is the byte length of `data`; blocks that do not fit are left as
 * zeros like the reference's `break` + `resize`. */
void ssdo_dequant_q4_0(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
void ssdo_dequant_q8_0(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
void ssdo_dequant_q6_k(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
void ssdo_dequant_q4_k(const uint8_t* data, size_t data_len, size_t n_elements, float* out);
/* dequantize_to_f32 dispatch, streamer.rs:93-125: returns 0, or 1 when the type
 * is unsupported there and the output was zero-filled (the reference's warning path). */
int ssdo_dequantize_to_f32(int dtype, const uint8_t* data, size_t data_len, size_t n_elements,
                           float* out);

/* Quantized matvec, src/metal/compute.rs:648-925 (serial fp32 chain per row).
 * Returns 0, or 1 when dtype is outside {Q4_0,Q8_0,Q4_K,Q6_K} and y was
 * zero-filled (compute.rs:672-675). */
int ssdo_matvec_quantized(const uint8_t* w, const float* x, size_t out_dim, size_t in_dim,
                          int dtype, float* y);
/* Same, rows sharded over `nthreads` std::thread-style workers
 * (src/inference/tensor_parallel.rs:45-96); bit-identical to the serial version. */
int ssdo_matvec_quantized_mt(const uint8_t* w, const float* x, size_t out_dim, size_t in_dim,
                             int dtype, float* y, int nthreads);
/* Exact value of the same dot products: sum over elements of
 * (double)elem * (double)x in double precision, where elem is the reference's
 * bit-exact fp32 element value.  Used only to tell apart the reference's own
 * fp32 rounding error from a device error. */
/* The element values each matvec multiplies by x, [out_dim][whole blocks of in_dim]
 * (1 and nothing written for types the matvec does not support). */
int ssdo_matvec_elements(const uint8_t* w, size_t out_dim, size_t in_dim, int dtype, float* e);
int ssdo_matvec_exact(const uint8_t* w, const float* x, size_t out_dim, size_t in_dim, int dtype,
                      double* y);

/* INT8 per-row quantizer, src/ssd/block_swap.rs:36-60
 * == QuantizedVec::quantize, src/inference/quantized_kv_cache.rs:23-41. */
void ssdo_quantize_rows_int8(const float* data, size_t n_rows, size_t dim, int8_t* codes,
                             float* scales);
/* src/ssd/block_swap.rs:63-74 == quantized_kv_cache.rs:44-53 */
void ssdo_dequantize_rows_int8(const int8_t* codes, const float* scales, size_t n_rows,
                               size_t dim, float* out);

/* Single-query GQA online-softmax attention over flattened f32 KV
 * [seq, n_head_kv, head_dim], src/inference/flash_attention.rs:70-139 (the
 * MetalCompute::flash_attention_f32 contract, compute.rs:217-258), positions
 * [window_start, min(window_end, seq_len)). */
void ssdo_flash_attention_f32(const float* q, const float* k, const float* v, size_t n_head,
                              size_t n_head_kv, size_t head_dim, size_t seq_len,
                              size_t window_start, size_t window_end, float* out);

/* Decode attention over the paged INT8 cache: the composition of
 * QuantizedVec::dequantize_into (quantized_kv_cache.rs:49-53), the block-table
 * mapping (paged_attention.rs:113-123, block layout 34-35, 72-76) and the
 * online softmax of flash_attention.rs:70-139.
 *   q            [n_seq, n_head, head_dim] f32
 *   k/v codes    [n_blocks, block_size, n_head_kv*head_dim] i8
 *   k/v scales   [n_blocks, block_size] f32 (one per token row)
 *   block_tables [n_seq, max_blocks_per_seq] i32
 *   ctx_lens     [n_seq] i32
 *   out          [n_seq, n_head, head_dim] f32 */
void ssdo_paged_attention_int8(const float* q, const int8_t* k_codes, const float* k_scales,
                               const int8_t* v_codes, const float* v_scales,
                               const int32_t* block_tables, const int32_t* ctx_lens,
                               size_t n_seq, size_t n_head, size_t n_head_kv, size_t head_dim,
                               size_t block_size, size_t max_blocks_per_seq, float* out);
/* Same over (n_seq*n_head) units sharded on `nthreads` workers. */
/* The same over a per-sequence window (flash_attention_windowed,
 * flash_attention.rs:146-227): positions [window_starts[s],
 * min(window_ends[s], ctx_lens[s])), zeros when empty; either array may be
 * NULL (start 0, no end bound). */
void ssdo_paged_attention_int8_window_mt(const float* q, const int8_t* k_codes, const float* k_scales,
                                         const int8_t* v_codes, const float* v_scales,
                                         const int32_t* block_tables, const int32_t* ctx_lens,
                                         const int32_t* window_starts, const int32_t* window_ends,
                                         size_t n_seq, size_t n_head, size_t n_head_kv, size_t head_dim,
                                         size_t block_size, size_t max_blocks_per_seq, float* out,
                                         int nthreads);
void ssdo_paged_attention_int8_mt(const float* q, const int8_t* k_codes, const float* k_scales,
                                  const int8_t* v_codes, const float* v_scales,
                                  const int32_t* block_tables, const int32_t* ctx_lens,
                                  size_t n_seq, size_t n_head, size_t n_head_kv, size_t head_dim,
                                  size_t block_size, size_t max_blocks_per_seq, float* out,
                                  int nthreads);

/* Prefill GEMM oracle: Y[t,:] = matvec_q4_k_cpu(W, widen_bf16(X[t,:]))
 * (per-token matvec, src/inference/transformer.rs:166-196; compute.rs:707-750).
 * X bf16 [M,K], W Q4_K [N, K/256 blocks], Y f32 [M,N]. */
void ssdo_gemm_q4k_bf16(const uint8_t* w, const uint16_t* x, size_t M, size_t N, size_t K,
                        float* y, int nthreads);
/* Exact (double) counterpart of ssdo_gemm_q4k_bf16, for rounding attribution. */
void ssdo_gemm_q4k_bf16_exact(const uint8_t* w, const uint16_t* x, size_t M, size_t N, size_t K,
                              double* y, int nthreads);

/* Decode-layer f32 ops: rope_f32_multi_head (compute.rs:482-507), silu_f32
 * (641-645), rmsnorm_f32_fast_scalar (580-589), fused_post_attn_norm_f32_cpu
 * (536-555) and fused_rmsnorm_linear_f32_cpu (557-578, projection through
 * matvec_quantized_cpu). */
void ssdo_rope_multi_head(float* x, size_t len, size_t head_dim, size_t n_heads, size_t position,
                          float theta_base);
void ssdo_silu(float* x, size_t n);
void ssdo_rmsnorm(float* x, const float* w, size_t n, float eps);
void ssdo_fused_post_attn_norm(float* hidden, const float* attn, const float* w, size_t n,
                               float eps, float* out);
int ssdo_fused_rmsnorm_linear(int dtype, const uint8_t* w, const float* x, const float* norm_w,
                              size_t vocab, size_t n_embd, float* y);

/* INT8 swap-file slots of the paged KV cache: slot size, write_block and
 * read_block of SwapFile in SwapQuantMode::Int8 (src/ssd/block_swap.rs:148-370). */
size_t ssdo_kv_slot_bytes(size_t block_size, size_t kv_dim);
void ssdo_kv_swap_write(const float* keys, const float* values, size_t block_size, size_t kv_dim,
                        uint32_t num_filled, uint8_t* slot);
void ssdo_kv_swap_read(const uint8_t* slot, size_t block_size, size_t kv_dim, float* keys, float* values,
                       uint32_t* num_filled);

#ifdef __cplusplus
}
#endif
#endif
