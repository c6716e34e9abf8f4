/*
 * ssdq.h — C ABI of libssdq.so, the MI355X (gfx950) quantized compute path
 * for the ssd-llm inference engine.
 *
 * Replaces the kernel-dispatch surface that src/inference calls in place of
 * src/metal (MetalCompute, src/metal/compute.rs:29-373; MetalGpu,
 * src/metal/gpu.rs:71-1258) for:
 *   - GGUF block dequantization (Q4_0, Q8_0, Q4_K, Q6_K) fused into matvec /
 *     small-batch matmul and the batched prefill GEMM,
 *   - INT8 per-row KV-cache quantize / dequantize and the paged append,
 *   - single-query GQA decode attention over f32 or paged INT8 KV.
 *
 * Conventions
 *   - Every function returns an int status: SSDQ_OK (0), a negative
 *     SSDQ_ERR_* code, or SSDQ_WARN_UNSUPPORTED_ZEROED (1) when the reference
 *     would have returned zeros for an unsupported dtype (the output is then
 *     zero-filled, compute.rs:672-675). ssdq_last_error() describes the last
 *     failure on the calling thread. No C++ exception crosses this boundary.
 *   - "dev" functions take device pointers and a stream (a hipStream_t, NULL
 *     for the default stream); they only enqueue work and return at once.
 *   - "host" functions take host pointers, copy in, compute, copy out and
 *     return when the result is in place: the synchronous, allocate-per-call
 *     contract of MetalCompute (gpu.rs:492-535), on a context that is created
 *     once (not per forward pass, unlike transformer.rs:301-302). Calls on one
 *     context are serialized by the context; contexts are independent.
 *   - dtype uses the GgmlType numeric ids of src/model/gguf.rs:17-48.
 *   - Sizes are element counts unless named *_bytes.
 */
#ifndef SSDQ_H
#define SSDQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SSDQ_ABI_VERSION 1

/* status codes */
#define SSDQ_OK 0
#define SSDQ_WARN_UNSUPPORTED_ZEROED 1
#define SSDQ_ERR_INVALID_ARG (-1)
#define SSDQ_ERR_UNSUPPORTED (-2)
#define SSDQ_ERR_HIP (-3)
#define SSDQ_ERR_NO_DEVICE (-4)
#define SSDQ_ERR_OUT_OF_MEMORY (-5)

/* GgmlType ids, src/model/gguf.rs:17-48 */
#define SSDQ_TYPE_F32 0
#define SSDQ_TYPE_F16 1
#define SSDQ_TYPE_Q4_0 2
#define SSDQ_TYPE_Q8_0 8
#define SSDQ_TYPE_Q2_K 10
#define SSDQ_TYPE_Q3_K 11
#define SSDQ_TYPE_Q4_K 12
#define SSDQ_TYPE_Q5_K 13
#define SSDQ_TYPE_Q6_K 14
#define SSDQ_TYPE_Q8_K 15
#define SSDQ_TYPE_IQ2_XXS 16
#define SSDQ_TYPE_IQ2_XS 17
#define SSDQ_TYPE_IQ3_XXS 18
#define SSDQ_TYPE_IQ4_NL 20
#define SSDQ_TYPE_IQ3_S 21
#define SSDQ_TYPE_IQ4_XS 23
#define SSDQ_TYPE_BF16 30

typedef void* ssdq_stream_t; /* a hipStream_t; NULL = default stream */
typedef struct ssdq_ctx ssdq_ctx;

/* ---------------------------------------------------------------- library */
int ssdq_abi_version(void);
/* Message of the last failing call on this thread ("" if none). */
const char* ssdq_last_error(void);
/* GgmlType::block_size / type_size, src/model/gguf.rs:87-135 (0 if unknown),
 * except Q3_K: 110 bytes, the block matvec_q3_k_cpu reads (compute.rs:798),
 * where gguf.rs:127 computes 174. */
size_t ssdq_block_size(int dtype);
size_t ssdq_type_size(int dtype);
/* Bytes of one weight row of in_dim elements: (in_dim / block) * type_size,
 * the row stride matvec_*_cpu uses (compute.rs:683-688). */
size_t ssdq_row_bytes(int dtype, size_t in_dim);

/* ---------------------------------------------------------------- context */
/* Replaces MetalCompute::new() -> Option<Self> (compute.rs:47-71): fails with
 * SSDQ_ERR_NO_DEVICE when no GPU is usable, where the caller keeps its CPU
 * path. `device` is a HIP device ordinal (-1: the current device). */
int ssdq_ctx_create(int device, ssdq_ctx** out);
void ssdq_ctx_destroy(ssdq_ctx* ctx);
/* MetalCompute::has_gpu (compute.rs:262-264) */
int ssdq_ctx_device(const ssdq_ctx* ctx);

/* ------------------------------------------------------------- workspace */
/* The "dev" functions that need scratch memory (K-sliced matvec partials,
 * split-K GEMM partials and its prepared X, attention split partials) take it
 * from a grow-only buffer the library keeps per (device, stream). Growth is
 * geometric (at least double, in 2 MiB steps). A replaced buffer that was
 * handed out while its stream was being captured into a HIP graph is retired,
 * not freed, so the graph keeps a valid address; any other replaced buffer is
 * freed once the stream has drained the work queued with it (one stream
 * synchronize per growth). Growth is refused while the stream is being
 * captured (SSDQ_ERR_HIP): run the call once on the stream before capture, or
 * reserve. No reference counterpart (the reference allocates Metal buffers per
 * call, gpu.rs:492-535). */
/* Grows the stream's scratch buffer of the current device to at least
 * `bytes` now, so later calls up to that need do not allocate. */
int ssdq_reserve_workspace(size_t bytes, ssdq_stream_t stream);
/* Frees the retired buffers (after a device synchronize). A graph captured
 * while one of them was current must not be replayed after this call. */
int ssdq_release_workspaces(void);

/* --------------------------------------------------- dequant (bit-exact) */
/* Device dequantization of n_elements into f32, element values bit-identical
 * to the reference: dequantize_q4_0 / q8_0 / q6_k (src/ssd/streamer.rs:128-220)
 * and the Q4_K values of matvec_q4_k_cpu (compute.rs:716-744; the reference's
 * loader has no Q4_K path and returns zeros, streamer.rs:119-123). Elements past
 * the last whole block are zero (streamer.rs `output.resize`). F32 / F16 /
 * BF16 tensors are copied / widened (streamer.rs:95-115; w element-aligned).
 * Replaces dequantize_to_f32 (streamer.rs:93-125) on the device. */
int ssdq_dequant_dev(int dtype, const void* w, size_t n_elements, float* out,
                     ssdq_stream_t stream);
/* Host twin of dequantize_to_f32 (streamer.rs:93-125): data_len bytes in,
 * n_elements floats out. Quantized types decode the whole blocks present in
 * data_len and zero the rest (the dequantizers' early `break` + `resize`);
 * float types need n_elements values; unsupported dtypes give zeros and
 * SSDQ_WARN_UNSUPPORTED_ZEROED (streamer.rs:117-123). Q4_K, zeros in the
 * reference's loader, is decoded. Synchronous. */
int ssdq_dequantize_to_f32(ssdq_ctx* ctx, int dtype, const uint8_t* data, size_t data_len,
                           size_t n_elements, float* out);

/* ---------------------------------------------------------------- matvec */
/* y[b, r] = sum_k dequant(W)[r, k] * x[b, k] for b < batch, r < out_dim, over
 * the (in_dim / block) whole blocks of each row.  W is out_dim rows of
 * ssdq_row_bytes(dtype, in_dim) bytes in the reference's GGUF block layout;
 * x is [batch, in_dim] f32, y is [batch, out_dim] f32.
 * Replaces MetalCompute::matvec_quantized (compute.rs:157-191), MetalGpu::
 * matvec_q4_0/q4_k/q6_k/q8_0 (gpu.rs:396-428) and matvec_quantized_cpu
 * (compute.rs:648-677); batch > 1 replaces the per-row loop of
 * batch_scheduler.rs:242-276. Types: Q4_0, Q8_0, Q4_K, Q6_K and the other
 * matvec_quantized types Q2_K, Q3_K, Q5_K, Q8_K, IQ2_XXS, IQ2_XS, IQ3_XXS,
 * IQ3_S, IQ4_NL, IQ4_XS, F16, BF16 (matvec_*_cpu, compute.rs:796-2238,
 * 2249-2285). Other dtypes (F32 included,
 * as in compute.rs:672-675) zero-fill y and return SSDQ_WARN_UNSUPPORTED_ZEROED. */
int ssdq_matvec_dev(int dtype, const void* w, const float* x, float* y, size_t out_dim,
                    size_t in_dim, size_t batch, ssdq_stream_t stream);
/* Host twin with the MetalCompute::matvec_quantized contract
 * (compute.rs:157-191): w_len bytes of raw blocks, x_len floats, y gets out_dim
 * floats. Synchronous. */
int ssdq_matvec_quantized(ssdq_ctx* ctx, const uint8_t* w_raw, size_t w_len, const float* x,
                          size_t x_len, size_t out_dim, size_t in_dim, int dtype, float* y);

/* ------------------------------------------- INT8 KV swap slots */
/* Bytes of one swap slot: the reference's SwapQuantMode::Int8 slot
 * (src/ssd/block_swap.rs:148-170): K codes, V codes (block_size * kv_dim i8
 * each), K scales, V scales (block_size f32 each), num_filled (u32). */
size_t ssdq_kv_slot_bytes(size_t block_size, size_t kv_dim);
/* Swap-out of paged INT8 KV blocks: slot i (at slots + i * slot_bytes) gets
 * physical block block_ids[i] of the pools (rows block_id * block_size ..,
 * as ssdq_paged_kv_append_dev writes them) and num_filled[i] (NULL: 0).  The
 * bytes are those SwapFile::write_block writes in Int8 mode
 * (block_swap.rs:187-252) for the f32 rows the pool was quantized from.
 * slots may be device memory or mapped pinned host memory (hipHostMalloc);
 * ids outside [0, n_pool_blocks) give zero slots. At most 65535 blocks per
 * call; kv_dim % 4 == 0; pointers 4-byte aligned. Replaces the extract +
 * write half of try_swap_out_blocks (paged_attention.rs:755-786). */
int ssdq_kv_swap_out_dev(const int8_t* k_codes, const float* k_scales, const int8_t* v_codes,
                         const float* v_scales, const int32_t* block_ids, const uint32_t* num_filled,
                         size_t n_blocks, size_t block_size, size_t kv_dim, size_t n_pool_blocks, void* slots,
                         ssdq_stream_t stream);
/* Swap-in: the inverse scatter (read_block + restore_block_data,
 * block_swap.rs:283-370, paged_attention.rs:624-630, 788-815); the codes and
 * scales are restored exactly (the reference dequantizes them to f32 on
 * read). num_filled (NULL: not returned) gets each slot's count; ids outside
 * [0, n_pool_blocks) are skipped. */
int ssdq_kv_swap_in_dev(const void* slots, const int32_t* block_ids, size_t n_blocks, size_t block_size,
                        size_t kv_dim, size_t n_pool_blocks, int8_t* k_codes, float* k_scales, int8_t* v_codes,
                        float* v_scales, uint32_t* num_filled, ssdq_stream_t stream);

/* ------------------------------------------------- decode-layer ops */
/* The projections of one decode step on quantized weights, QKV+RoPE and
 * SwiGLU each one kernel launch where the shapes allow it (one matrix type, whole rows of at most 128
 * 64-element units of Q4_0 / Q8_0 / Q4_K / Q6_K, i.e. n_embd up to 8192 for
 * Q4_K; otherwise the same result from separate launches).  Batch 1.
 *
 * q = Wq x, k = Wk x, v = Wv x, then RoPE on q and k (pairs (2i, 2i+1) of each
 * head rotated by position * theta_base^(-2i/head_dim); head_dim 0: no RoPE).
 * Replaces fused_qkv_rope_f32 / fused_qkv_f32 (compute.rs:273-326, gpu.rs:917,
 * 997; CPU fused_qkv_rope_f32_cpu 509-534, rope_f32_multi_head 482-507) on
 * quantized weights. q_dim, kv_dim even; head_dim even and dividing both. */
int ssdq_qkv_rope_dev(int dtype_q, const void* wq, int dtype_k, const void* wk, int dtype_v,
                      const void* wv, const float* x, float* q, float* k, float* v, size_t q_dim,
                      size_t kv_dim, size_t n_embd, size_t head_dim, size_t position, float theta_base,
                      ssdq_stream_t stream);
/* h = silu(W_gate x) * (W_up x), silu(v) = v / (1 + exp(-v)): the gate / up
 * half of the SwiGLU feed-forward (src/inference/feed_forward.rs:28-40,
 * silu_f32 compute.rs:641-645; the reference's fused Metal kernel
 * gpu.rs feed_forward_f32) on quantized weights. h has n_ff floats. */
int ssdq_swiglu_dev(int dtype, const void* w_gate, const void* w_up, const float* x, float* h,
                    size_t n_ff, size_t n_embd, ssdq_stream_t stream);
/* y = W (x * inv_rms * norm_weight), inv_rms = 1 / sqrt(mean(x^2) + eps): the
 * output head of fused_rmsnorm_linear_f32 (compute.rs:348-372, CPU 557-578,
 * which fixes eps = 1e-5) on quantized weights, which the reference
 * re-dequantizes every token (src/inference/transformer.rs:688-706). */
int ssdq_rmsnorm_matvec_dev(int dtype, const void* w, const float* x, const float* norm_weight, float eps,
                            float* y, size_t out_dim, size_t n_embd, ssdq_stream_t stream);
/* h = x + residual (residual may be NULL; written to hidden_out unless NULL),
 * out = h * inv_rms * weight: fused_post_attn_norm_f32 (compute.rs:328-346,
 * CPU 536-555); with residual NULL, rmsnorm_f32 (compute.rs:193-202). out and
 * hidden_out may alias x. */
int ssdq_rmsnorm_dev(const float* x, const float* residual, const float* weight, float eps,
                     float* hidden_out, float* out, size_t n, ssdq_stream_t stream);

/* ------------------------------------------------------- prefill GEMM */
/* Y[M, N] f32 = X[M, K] bf16 (row-major) times Q4_K W[N rows, K] (reference
 * layout), fp32 accumulate.  The reference has no GEMM: prefill is one matvec
 * per token (src/inference/transformer.rs:166-196 -> matvec_q4_k_cpu,
 * compute.rs:707-750); this computes the same Y in one pass. K % 256 == 0. */
int ssdq_gemm_q4k_bf16_dev(const void* w, const uint16_t* x_bf16, float* y, size_t M,
                           size_t N, size_t K, ssdq_stream_t stream);
/* The same for count = 1..3 Q4_K matrices that read the same X: Y_i[M, n[i]] =
 * X W_i^T, computed as one GEMM over the concatenated columns with X prepared
 * once.  Replaces the per-token q/k/v (or gate/up) matvecs of one layer's
 * prefill, which the reference runs on one shared input per token
 * (transformer.rs:166-196 -> multi_head_attention_fused_rope; the FFN's gate
 * and up, feed_forward.rs:28-40).  Every n[i] >= 1; K % 256 == 0. */
int ssdq_gemm_q4k_bf16_multi_dev(const void* const* w, const size_t* n, size_t count,
                                 const uint16_t* x_bf16, float* const* y, size_t M, size_t K,
                                 ssdq_stream_t stream);

/* ------------------------------------------------------ INT8 KV cache */
/* Per-row absmax INT8 quantization, bit-exact codes and scales:
 * quantize_vectors_int8 (src/ssd/block_swap.rs:36-60) == QuantizedVec::quantize
 * (src/inference/quantized_kv_cache.rs:23-41). in [n_rows, row_len] f32 ->
 * codes [n_rows, row_len] i8, scales [n_rows] f32. */
int ssdq_kv_quantize_rows_dev(const float* in, int8_t* codes, float* scales, size_t n_rows,
                              size_t row_len, ssdq_stream_t stream);
/* code as f32 * scale: dequantize_vectors_int8 (block_swap.rs:63-74) ==
 * QuantizedVec::dequantize (quantized_kv_cache.rs:44-53). */
int ssdq_kv_dequantize_rows_dev(const int8_t* codes, const float* scales, float* out,
                                size_t n_rows, size_t row_len, ssdq_stream_t stream);
/* Host twins (synchronous, copy in/out): quantize_vectors_int8 /
 * dequantize_vectors_int8 (src/ssd/block_swap.rs:36-74) over n_rows rows of
 * dim elements. */
int ssdq_quantize_vectors_int8(ssdq_ctx* ctx, const float* data, size_t n_rows, size_t dim,
                               int8_t* codes, float* scales);
int ssdq_dequantize_vectors_int8(ssdq_ctx* ctx, const int8_t* codes, const float* scales,
                                 size_t n_rows, size_t dim, float* out);
/* Quantize-on-append into the paged INT8 pool: token t's K and V rows
 * (kv_dim floats each) are quantized like ssdq_kv_quantize_rows_dev and stored
 * at pool row slot_mapping[t] (= physical_block * block_size + slot, see
 * physical_block_for_position, src/inference/paged_attention.rs:113-123);
 * slot_mapping[t] < 0 skips the token. Pool layout: codes
 * [n_blocks * block_size, kv_dim] i8 (PhysicalBlock [block_size, kv_dim],
 * paged_attention.rs:34-35), scales [n_blocks * block_size] f32.
 * Replaces PagedKvCache::append (paged_attention.rs:351-409) composed with
 * QuantizedLayerKvCache::append (quantized_kv_cache.rs:107-110). */
int ssdq_paged_kv_append_dev(const float* k, const float* v, const int32_t* slot_mapping,
                             int8_t* k_codes, float* k_scales, int8_t* v_codes, float* v_scales,
                             size_t n_tokens, size_t kv_dim, ssdq_stream_t stream);

/* ------------------------------------------------------------ attention */
/* GQA decode attention over the paged INT8 cache, one query token per
 * sequence: for each sequence s and head h, online softmax over positions
 * [0, ctx_lens[s]) of K/V = code * row scale, kv head h / (n_head/n_head_kv),
 * scale 1/sqrt(head_dim) (src/inference/flash_attention.rs:70-139), the block
 * table addressing of paged_attention.rs:113-123, zeros when the context is
 * empty. q, out: [n_seq, n_head, head_dim] f32; block_tables
 * [n_seq, max_blocks_per_seq] i32; ctx_lens [n_seq] i32 with
 * ctx_lens[s] <= max_ctx <= max_blocks_per_seq * block_size.
 * head_dim in {64, 128, 256}. The library keeps a per-device workspace. */
int ssdq_paged_attention_int8_dev(const float* q, const int8_t* k_codes, const float* k_scales,
                                  const int8_t* v_codes, const float* v_scales,
                                  const int32_t* block_tables, const int32_t* ctx_lens,
                                  float* out, size_t n_seq, size_t n_head, size_t n_head_kv,
                                  size_t head_dim, size_t block_size, size_t max_blocks_per_seq,
                                  size_t max_ctx, ssdq_stream_t stream);
/* The same paged INT8 decode attention over a position window per sequence:
 * sequence s attends over [max(window_starts[s], 0), min(window_ends[s],
 * ctx_lens[s])), the range flash_attention_windowed takes
 * (src/inference/flash_attention.rs:146-227, effective_end = min(window_end,
 * seq_len)) and MetalCompute::flash_attention_f32 passes to its kernel
 * (compute.rs:217-258), here over the paged INT8 cache; an empty window gives
 * zeros, as the reference's running_sum == 0 case does. Either array may be
 * NULL (start 0, no end bound). The window length is at most max_ctx. */
int ssdq_paged_attention_int8_window_dev(const float* q, const int8_t* k_codes, const float* k_scales,
                                         const int8_t* v_codes, const float* v_scales,
                                         const int32_t* block_tables, const int32_t* ctx_lens,
                                         const int32_t* window_starts, const int32_t* window_ends, float* out,
                                         size_t n_seq, size_t n_head, size_t n_head_kv, size_t head_dim,
                                         size_t block_size, size_t max_blocks_per_seq, size_t max_ctx,
                                         ssdq_stream_t stream);
/* The same paged INT8 decode attention, allocating nothing: no counterpart in
 * the reference. It is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Arguments, kernels and results are those of
 * ssdq_paged_attention_int8_dev; the split partials live in a static device
 * array of 16 MiB that each GPU the library runs on holds until the process
 * ends. A call whose partials need more (n_seq * n_head * splits *
 * (head_dim + 2) * 4 bytes; config 5, 8 x 32 heads at 32k context, needs
 * 4.3 MB) fails with SSDQ_ERR_INVALID_ARG and launches nothing. All calls on
 * one GPU share that array: calls that overlap in time on one GPU (different
 * streams, or host threads) race and must be serialized by the caller. */
int ssdq_paged_attention_int8_noalloc_dev(const float* q, const int8_t* k_codes, const float* k_scales,
                                          const int8_t* v_codes, const float* v_scales,
                                          const int32_t* block_tables, const int32_t* ctx_lens, float* out,
                                          size_t n_seq, size_t n_head, size_t n_head_kv, size_t head_dim,
                                          size_t block_size, size_t max_blocks_per_seq, size_t max_ctx,
                                          ssdq_stream_t stream);
/* MetalCompute::flash_attention_f32 (compute.rs:217-258) / MetalGpu::
 * flash_attention_f32 (gpu.rs:547-599): q [n_head, head_dim], k/v flattened
 * [seq_len, n_head_kv, head_dim] f32, positions [window_start,
 * min(window_end, seq_len)), out [n_head, head_dim]. head_dim in {64,128,256}. */
int ssdq_flash_attention_f32_dev(const float* q, const float* k, const float* v, float* out,
                                 size_t n_head, size_t n_head_kv, size_t head_dim,
                                 size_t seq_len, size_t window_start, size_t window_end,
                                 ssdq_stream_t stream);
/* Host twin (synchronous, copies in/out). Unlike MetalCompute, it never returns
 * "None": the seq_len >= 4 dispatch heuristic of compute.rs:232 is the
 * caller's choice. */
int ssdq_flash_attention_f32(ssdq_ctx* ctx, const float* q, const float* k, const float* v,
                             size_t n_head, size_t n_head_kv, size_t head_dim, size_t seq_len,
                             size_t window_start, size_t window_end, float* out);

/* ------------------------------------------------ resident weight store */
/* Raw GGUF tensor bytes kept in HBM, uploaded once and found by name.
 * Replaces SsdStreamer::load_layer / load_tensor_f32 (src/ssd/streamer.rs:
 * 33-66), which re-read a layer's tensors and dequantize them to f32 on every
 * load (Q4_K to zeros, streamer.rs:119-123): the quantized blocks stay as the
 * file holds them and the dev functions decode them in place. Tensors are
 * placed 256-byte aligned in device arenas of at least 256 MiB. A store
 * belongs to one device; its calls are thread-safe. */
typedef struct ssdq_weights ssdq_weights;
/* device: a HIP ordinal, -1 for the current device. SSDQ_ERR_NO_DEVICE when
 * there is none. */
int ssdq_weights_create(int device, ssdq_weights** out);
/* Waits for the device, then frees every tensor of the store. */
void ssdq_weights_destroy(ssdq_weights* w);
/* Uploads one tensor (TensorInfo, src/model/gguf.rs:216-222): its GGUF name,
 * GgmlType id, dims as GGUF lists them (dims[0] is the row length; a matrix
 * is {in_dim, out_dim}), and data_len bytes from host memory (e.g. the mapped
 * file at the tensor's offset, GgufLoader::get_tensor_data). For the types
 * this library knows, dims[0] must be a whole number of blocks and data_len
 * the size dims and type give. Synchronous. A name already resident, or a
 * size mismatch: SSDQ_ERR_INVALID_ARG. */
int ssdq_weights_put(ssdq_weights* w, const char* name, int dtype, const uint64_t* dims, size_t n_dims,
                     const void* data, size_t data_len);
/* The device address of a resident tensor, NULL when absent (Option, as
 * find_tensor_in_layer returns, transformer.rs:552-559). The out pointers may
 * be NULL; dims gets 4 entries (1 past n_dims). */
const void* ssdq_weights_find(const ssdq_weights* w, const char* name, int* dtype, uint64_t* dims,
                              size_t* n_dims, size_t* n_bytes);
size_t ssdq_weights_count(const ssdq_weights* w);
/* tensor bytes resident (CachedLayer::size_bytes summed, in file bytes) */
size_t ssdq_weights_bytes(const ssdq_weights* w);
int ssdq_weights_device(const ssdq_weights* w);

/* ------------------------------------------------------ decoder layer */
/* One layer's shape. n_head * head_dim is the query width, n_head_kv *
 * head_dim the key / value width (the reference sets head_dim = n_embd /
 * n_head, transformer.rs:295). rope_theta: DEFAULT_ROPE_THETA for Llama;
 * norm_eps: 1e-5 in the reference (transformer.rs:577, 351). */
typedef struct ssdq_layer_config {
  size_t n_embd;
  size_t n_head;
  size_t n_head_kv;
  size_t head_dim; /* 64, 128 or 256 */
  size_t n_ff;
  float rope_theta;
  float norm_eps;
} ssdq_layer_config;

/* Regions of the layer's scratch buffer, in floats of the named step's output:
 * attention input (normed), q, k, v (after RoPE), attention, output
 * projection, FFN input (normed), silu(gate) * up, gate and up (used when
 * their types differ), down projection, widened norm weights (F16 / BF16
 * norms), hidden + attention output (when the FFN norm is folded into the
 * SwiGLU launch). */
#define SSDQ_LAYER_ATTN_IN 0
#define SSDQ_LAYER_Q 1
#define SSDQ_LAYER_K 2
#define SSDQ_LAYER_V 3
#define SSDQ_LAYER_ATTN 4
#define SSDQ_LAYER_ATTN_OUT 5
#define SSDQ_LAYER_FFN_IN 6
#define SSDQ_LAYER_FFN_H 7
#define SSDQ_LAYER_FFN_GATE 8
#define SSDQ_LAYER_FFN_UP 9
#define SSDQ_LAYER_FFN_OUT 10
#define SSDQ_LAYER_NORM_W 11
#define SSDQ_LAYER_HIDDEN_MID 12
#define SSDQ_LAYER_N_STAGES 13
/* Bytes of scratch ssdq_decode_layer_dev needs (0 for a bad config);
 * offsets (NULL, or SSDQ_LAYER_N_STAGES entries) gets each region's byte
 * offset. After a call each region holds that step's output for the token. */
size_t ssdq_decode_layer_scratch_bytes(const ssdq_layer_config* cfg, size_t* offsets);

/* One decoder layer for one token, from the store's tensors
 * "blk.{layer}.{attn_norm, attn_q, attn_k, attn_v, attn_output, ffn_norm,
 * ffn_gate, ffn_up, ffn_down}.weight": the per-layer body of forward_pass
 * (src/inference/transformer.rs:319-397) with multi_head_attention_fused_rope
 * (src/inference/attention.rs:172-240) over the paged INT8 cache and the
 * dense SwiGLU FFN (transformer.rs:470-481, feed_forward.rs:16-71):
 *   x = rms_norm(hidden, attn_norm)
 *   q, k, v = Wq x, Wk x, Wv x; RoPE(q, k) at `position`  (ssdq_qkv_rope_dev)
 *   pool row slot_mapping[0] = int8(k), int8(v)            (ssdq_paged_kv_append_dev)
 *   a = attention of q over ctx_len[0] tokens              (ssdq_paged_attention_int8_dev)
 *   hidden += Wo a; f = rms_norm(hidden, ffn_norm)         (ssdq_matvec_dev, ssdq_rmsnorm_dev)
 *   hidden += W_down (silu(W_gate f) * (W_up f))           (ssdq_swiglu_dev, ssdq_matvec_dev)
 * As in the reference: no attn_norm -> x = hidden; any of the four attention
 * tensors absent -> the layer leaves hidden unchanged; no ffn_norm -> f =
 * hidden after the residual add; any FFN tensor absent -> no FFN. MoE layers
 * (ffn_gate_inp) are not on this path. hidden: n_embd floats on the device,
 * updated in place. The pool arguments are those of the paged append and
 * attention above for one sequence (block_table: max_blocks_per_seq entries;
 * slot_mapping and ctx_len: one int32 each, in device memory). scratch: NULL
 * for the library's per-stream workspace, or a 256-byte aligned buffer of
 * ssdq_decode_layer_scratch_bytes(cfg) bytes; it holds the step outputs
 * listed above. The attention's split partials and the down projection's
 * K-slice partials still come from the per-stream workspace (see
 * ssdq_reserve_workspace), as in the separate entry points. Shapes of every tensor are
 * checked before anything is launched. Status: the worst of the steps
 * (SSDQ_WARN_UNSUPPORTED_ZEROED when a projection's type is unsupported and
 * its output was zero-filled, as the reference's matvec does). */
int ssdq_decode_layer_dev(const ssdq_weights* w, uint32_t layer, const ssdq_layer_config* cfg, float* hidden,
                          size_t position, int8_t* k_codes, float* k_scales, int8_t* v_codes, float* v_scales,
                          size_t block_size, const int32_t* block_table, size_t max_blocks_per_seq,
                          const int32_t* slot_mapping, const int32_t* ctx_len, size_t max_ctx, void* scratch,
                          size_t scratch_bytes, ssdq_stream_t stream);

/* -------------------------------------------------------------- testing */
/* Forces the byte-addressed matvec kernel that unaligned weights take, so the
 * fallback can be checked on aligned inputs. Same contract as ssdq_matvec_dev. */
int ssdq_matvec_generic_dev(int dtype, const void* w, const float* x, float* y, size_t out_dim,
                            size_t in_dim, size_t batch, ssdq_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* SSDQ_H */
