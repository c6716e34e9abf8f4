// Internal launchers shared between the kernel translation units and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ssdq {

hipError_t launch_fill_zero(float* out, size_t n, hipStream_t stream);
// F32 copy / F16 / BF16 widening of n elements (element-aligned input).
hipError_t launch_widen(int dtype, const void* w, size_t n, float* out, hipStream_t stream);
hipError_t launch_dequant(int dtype, const uint8_t* w, size_t n_blocks, float* out,
                          hipStream_t stream);

// y[b*out_dim + r] = sum_k W[r,k] * x[b*in_dim + k], b < batch, over the
// whole blocks of each row (k < (in_dim / block) * block).
hipError_t launch_matvec(int dtype, const uint8_t* w, const float* x, float* y, size_t out_dim,
                         size_t in_dim, size_t batch, hipStream_t stream, void* workspace = nullptr,
                         size_t workspace_bytes = 0);
// acc[r] = acc_in[r] + sum_k W[r,k] x[k] (batch 1; Q4_0 / Q8_0 / Q4_K / Q6_K;
// acc_in null: acc itself), with y receiving the plain product: the residual
// add of a decoder layer folded into the K-sliced matvec's slice reduction
// (the same fp32 add as a separate residual kernel).  acc may not alias x or y.
hipError_t launch_matvec_acc(int dtype, const uint8_t* w, const float* x, float* acc, float* y, size_t out_dim,
                             size_t in_dim, hipStream_t s, void* workspace, size_t workspace_bytes,
                             const float* acc_in = nullptr);
// While one is alive on a host thread, batch-1 matvecs launched from that
// thread treat x as just written by the previous kernel (not resident in this
// XCD's L2) and pick the form that requests it from more waves.  A hint for
// kernel selection only: results are the same bit for bit.
struct FreshX {
  FreshX();
  ~FreshX();
  FreshX(const FreshX&) = delete;
  FreshX& operator=(const FreshX&) = delete;
};
bool fresh_x();
// Device workspace launch_matvec uses for these operands (batch-1 K slices).
size_t matvec_workspace_bytes(int dtype, const void* w, const float* x, size_t out_dim,
                              size_t in_dim, size_t batch);
// Same, forcing the byte-addressed fallback kernel (used by tests to cover it).
hipError_t launch_matvec_generic(int dtype, const uint8_t* w, const float* x, float* y,
                                 size_t out_dim, size_t in_dim, size_t batch, hipStream_t stream);

// The reference's other matvec_quantized types (Q2_K, Q3_K, Q5_K, Q8_K, IQ4_NL,
// IQ4_XS, F16, BF16), same contract as launch_matvec; generic forces the
// byte-addressed kernel.
bool matvec_ext_type(int dtype);
hipError_t launch_matvec_ext(int dtype, const uint8_t* w, const float* x, float* y, size_t out_dim,
                             size_t in_dim, size_t batch, hipStream_t stream, bool generic);

// Decode-layer fusion of the batch-1 matvec: up to three matrices of one type
// and row length sharing x ("segments", virtual rows concatenated; with swiglu
// the rows of gate (w0) and up (w1) alternate and silu(g) * u goes to y0),
// and RoPE on the output pairs of the segments in rope_mask.  Every segment
// has an even row count.
// RoPE of one position: sn[i], cs[i] = sin, cos of the fp32 angle position *
// freq_i, freq_i = theta^(-2i/head_dim) for i < head_dim / 2, all on the host:
// the frequency with the C library's powf (what the reference's f32::powf
// calls), so the angle matches the reference bit for bit, and sin / cos in
// double, rounded once to fp32.  The kernels only read the table.
struct RopeTable {
  float sn[128];
  float cs[128];
};

struct MatvecFuse {
  const uint8_t* w0;
  const uint8_t* w1;
  const uint8_t* w2;
  float* y0;
  float* y1;
  float* y2;
  int start1, start2;  // first virtual row of segments 1 and 2 (INT_MAX: absent)
  int swiglu;
  unsigned rope_mask;
  int head_dim;
  RopeTable rope;
  // RMSNorm of x in the kernel's staging (the norm-fused variants): x' = (x +
  // norm_res) * inv_rms * norm_w, inv_rms = 1 / sqrt(mean((x + norm_res)^2) +
  // norm_eps); workgroup 0 writes x + norm_res to hidden_out and x' to xn_out
  // (either may be null).  norm_w null: no norm.
  const float* norm_w;
  const float* norm_res;
  float norm_eps;
  float* hidden_out;
  float* xn_out;
};
// One fused launch when the shapes allow it (Q4_0 / Q8_0 / Q4_K / Q6_K, whole
// rows of at most 128 units, aligned operands); *used = false otherwise.
// Digit-plane kernels (mv_b1 at batch 1, mv_bn for batches) for the matvec_ext
// types that have them (Q5_K, Q2_K, Q3_K, Q8_K); sets *used = false (nothing
// launched) when the type, alignment or workspace does not fit, and the caller
// takes launch_matvec_ext.
size_t matvec_digit_ext_workspace_bytes(int dtype, const void* w, const float* x, size_t out_dim, size_t in_dim,
                                        size_t batch);
hipError_t launch_matvec_digit_ext(int dtype, const uint8_t* w, const float* x, float* y, size_t out_dim,
                                   size_t in_dim, size_t batch, hipStream_t s, void* workspace,
                                   size_t workspace_bytes, bool* used);
hipError_t launch_matvec_fused(int dtype, const MatvecFuse& f, int total_rows, const float* x,
                               size_t in_dim, hipStream_t stream, bool* used);
// Pieces of the unfused decode layer.
// RoPE on n values (heads of head_dim), pairs (2i, 2i+1): rope_f32_multi_head.
hipError_t launch_rope(float* v, int n, int head_dim, const RopeTable& rope, hipStream_t stream);
// h = silu(g) * u
hipError_t launch_swiglu(const float* g, const float* u, float* h, int n, hipStream_t stream);
// h += a (n floats)
hipError_t launch_residual_add(float* h, const float* a, int n, hipStream_t stream);
// out = a + b (n floats; out may alias a or b)
hipError_t launch_add(float* out, const float* a, const float* b, int n, hipStream_t stream);
// hsum = x + residual (residual may be null; hidden_out may be null), then
// out = hsum * inv_rms * w with inv_rms = 1 / sqrt(mean(hsum^2) + eps).
hipError_t launch_rmsnorm(const float* x, const float* residual, const float* w, float eps,
                          float* hidden_out, float* out, int n, hipStream_t stream);

hipError_t launch_kv_quantize(const float* in, int8_t* codes, float* scales, size_t n_rows,
                              size_t row_len, hipStream_t stream);
hipError_t launch_kv_dequantize(const int8_t* codes, const float* scales, float* out,
                                size_t n_rows, size_t row_len, hipStream_t stream);
hipError_t launch_paged_kv_append(const float* k, const float* v, const int32_t* slot_mapping,
                                  int8_t* k_codes, float* k_scales, int8_t* v_codes,
                                  float* v_scales, size_t n_tokens, size_t kv_dim,
                                  hipStream_t stream);

// INT8 swap-file slots of paged KV blocks (the reference's Int8 slot format):
// slot bytes, gather of pool blocks ids[0..n) into consecutive slots (ids out
// of [0, n_pool) give zero slots), and the scatter back (such ids ignored).
size_t kv_slot_bytes(size_t block_size, size_t kv_dim);
hipError_t launch_kv_swap_out(const int8_t* k_codes, const float* k_scales, const int8_t* v_codes,
                              const float* v_scales, const int32_t* ids, const uint32_t* num_filled,
                              size_t n_blocks, size_t block_size, size_t kv_dim, size_t n_pool, void* slots,
                              hipStream_t stream);
hipError_t launch_kv_swap_in(const void* slots, const int32_t* ids, size_t n_blocks, size_t block_size,
                             size_t kv_dim, size_t n_pool, int8_t* k_codes, float* k_scales, int8_t* v_codes,
                             float* v_scales, uint32_t* num_filled, hipStream_t stream);

struct PagedAttnArgs {
  const float* q;
  const int8_t* k_codes;
  const float* k_scales;
  const int8_t* v_codes;
  const float* v_scales;
  const int32_t* block_tables;
  const int32_t* ctx_lens;
  float* out;
  int n_seq, n_head, n_head_kv, head_dim, block_size, max_blocks_per_seq;
  int max_ctx;  // upper bound on ctx_lens (sizes the split-KV grid)
  // Optional per-sequence position window (flash_attention_windowed,
  // src/inference/flash_attention.rs:146-227): sequence s attends over
  // [max(win_lo[s], 0), min(win_hi[s], ctx_lens[s])); null means 0 / no bound.
  const int32_t* win_lo = nullptr;
  const int32_t* win_hi = nullptr;
  // Optional new token of each sequence (a decode step's INT8 append folded
  // into the attention launch; no window): the K / V rows new_k[s], new_v[s]
  // (kv_dim floats each) are quantized in the kernel, bit-identical to
  // ssdq_kv_quantize_rows_dev, written to pool row new_slot[s] (< 0: not
  // written), and the token at position ctx_lens[s] - 1 is taken from those
  // codes instead of being read from the pool.
  const float* new_k = nullptr;
  const float* new_v = nullptr;
  const int32_t* new_slot = nullptr;
};
// Bytes of device workspace the split-KV attention needs for these shapes.
size_t paged_attn_workspace_bytes(const PagedAttnArgs& a, int* n_splits_out);
hipError_t launch_paged_attn(const PagedAttnArgs& a, void* workspace, hipStream_t stream);
// The same with a.new_k / a.new_v / a.new_slot set: one launch (plus the
// combine) where the matrix-core kernel applies (no window, head_dim <= 128,
// kv_dim a multiple of 64 up to 1024, 16-byte aligned new rows); otherwise the
// INT8 append kernel, then the attention.
hipError_t launch_paged_attn_append(const PagedAttnArgs& a, void* workspace, hipStream_t stream);
// Paged attention with its split partials in the library's static device
// scratch (kNoAllocScratchBytes per device): allocates nothing.  *need gets the
// scratch the call requires; hipErrorInvalidValue when that exceeds the maximum.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
hipError_t launch_paged_attn_noalloc(const PagedAttnArgs& a, hipStream_t stream, size_t* need);

size_t flash_attn_f32_workspace_bytes(int n_head, int n_head_kv, int head_dim, int len,
                                      int* n_splits_out);
hipError_t launch_flash_attn_f32(const float* q, const float* k, const float* v, float* out,
                                 int n_head, int n_head_kv, int head_dim, int seq_len,
                                 int window_start, int window_end, void* workspace,
                                 hipStream_t stream);

// Q8_0 matvec of 2-8 activation rows on the matrix cores (matvec_mfma.hip);
// hipErrorNotSupported when the shape or alignment does not fit it.
bool q8_mfma_supported(const void* w, const float* x, size_t in_dim, size_t batch);
hipError_t launch_q8_mfma(const uint8_t* w, const float* x, float* y, size_t out_dim, size_t in_dim, size_t batch,
                          hipStream_t s);

// Prefill GEMM: Y_i[M,n_i] f32 = X[M,K] bf16 x W_i[n_i,K] Q4_K (reference
// layout) for count = 1..3 matrices sharing X, computed as one GEMM.
hipError_t launch_gemm_q4k(const uint8_t* const* w, const size_t* n, int count, const uint16_t* x,
                           float* const* y, size_t M, size_t K, void* workspace, size_t workspace_bytes,
                           hipStream_t stream);
size_t gemm_q4k_workspace_bytes(const void* const* w, const size_t* n, int count, const void* x, size_t M,
                                size_t K);

int device_cu_count();

// The C ABI's status plumbing, for entry points defined outside capi.cpp:
// api_fail records the thread's last error message and returns code;
// api_workspace hands out the per-(device, stream, slot) grow-only workspace.
int api_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int api_hip_fail(hipError_t e, const char* what);
int api_ok();
hipError_t api_workspace(size_t bytes, hipStream_t stream, void** out, int slot);
int api_paged_attention_append(const float* q, int8_t* k_codes, float* k_scales, int8_t* v_codes, float* v_scales,
                               const int32_t* block_tables, const int32_t* ctx_lens, const float* new_k,
                               const float* new_v, const int32_t* new_slot, float* out, size_t n_seq, size_t n_head,
                               size_t n_head_kv, size_t head_dim, size_t block_size, size_t max_blocks_per_seq,
                               size_t max_ctx, hipStream_t stream);
// theta^(-2i/head_dim) with the C library's powf, as the reference computes them
void api_rope_table(RopeTable* r, int head_dim, float theta, int position);

}  // namespace ssdq
