// INT8 per-row KV quantization (bit-exact with the reference) and the paged
// append that writes quantized rows into the block pool.
//
// Reference: quantize_vectors_int8, src/ssd/block_swap.rs:36-60
//   == QuantizedVec::quantize, src/inference/quantized_kv_cache.rs:23-41:
//   absmax = fold(0.0, f32::max) of |v|      (NaN ignored, as fmaxf)
//   absmax == 0  ->  scale 0, codes 0
//   inv = 127 / absmax, scale = absmax / 127 (two correctly rounded divisions)
//   code = clamp(round_half_away(v * inv), -127, 127) as i8   (NaN -> 0)
// Dequant: code as f32 * scale (block_swap.rs:63-74, quantized_kv_cache.rs:44-53).
// A row is one token's K (or V) vector over kv_dim = n_kv_heads * head_dim
// (quantized_kv_cache.rs:107-110, block_swap.rs:232-233).
//
// One wavefront per row; a row is read once from HBM (kept in registers for
// rows up to 64*32 floats, re-read from L2 otherwise) and its codes are written
// as packed dwords.
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"

namespace ssdq {
namespace {

__device__ __forceinline__ uint32_t code_of(float v, float inv) { return kv_code_of(v, inv); }

__device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d, float inv) {
  return kv_pack4(a, b, c, d, inv);
}

// Quantizes the row `in` (len floats, 16-byte aligned when len % 4 == 0) into
// codes/scale.  Executed by one full wavefront.
template <int NV>  // float4 registers per lane kept resident (0: stream twice)
__device__ __forceinline__ void quantize_row(const float* __restrict__ in, int len,
                                             int8_t* __restrict__ codes, float* __restrict__ scale) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  float amax = 0.0f;
  const bool vec = (len & 3) == 0 && (((uintptr_t)in) & 15) == 0 && (((uintptr_t)codes) & 3) == 0;
  if (vec && NV > 0 && len <= NV * 4 * 64) {
    float4 r[NV > 0 ? NV : 1];
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int e = (i * 64 + lane) * 4;
      r[i] = e < len ? *reinterpret_cast<const float4*>(in + e) : make_float4(0.f, 0.f, 0.f, 0.f);
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(r[i].x), fabsf(r[i].y)), fmaxf(fabsf(r[i].z), fabsf(r[i].w))));
    }
    amax = wave_max(amax);
    float inv = 0.0f;
    if (amax != 0.0f) inv = 127.0f / amax;
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int e = (i * 64 + lane) * 4;
      if (e < len) {
        const uint32_t p = amax == 0.0f ? 0u : pack4(r[i].x, r[i].y, r[i].z, r[i].w, inv);
        *reinterpret_cast<uint32_t*>(codes + e) = p;
      }
    }
    if (lane == 0) *scale = amax == 0.0f ? 0.0f : amax / 127.0f;
    return;
  }
  // general path: element-wise, two passes
  for (int e = lane; e < len; e += 64) amax = fmaxf(amax, fabsf(in[e]));
  amax = wave_max(amax);
  const float inv = amax != 0.0f ? 127.0f / amax : 0.0f;
  for (int e = lane; e < len; e += 64) codes[e] = amax == 0.0f ? (int8_t)0 : (int8_t)code_of(in[e], inv);
  if (lane == 0) *scale = amax == 0.0f ? 0.0f : amax / 127.0f;
}

// Rows of len <= NV*256 floats (len % 4 == 0, 16-byte aligned rows): each
// wavefront quantizes RPW consecutive rows, with the loads of all of them
// issued first.  Straight-line code (rows past the end are clamped to the
// last row, quantized again to the same bits; FULL = len == NV*256 drops the
// per-lane bounds tests): a loop or a memory access under a branch makes the
// compiler wait for every outstanding load.  Every input and code byte is
// touched once, by one instruction per 1 KB or 256 B, so loads and stores are
// nontemporal: at config 5a (2 GiB in, 512 MiB out) 492 -> 430 us, and one row
// per wave is faster than four (464 against 492 us with ordinary loads).
constexpr int kRowsPerWave = 1;
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int NV, bool FULL>
__global__ __launch_bounds__(256) void kv_quantize_pipe_kernel(const float* __restrict__ in,
                                                               int8_t* __restrict__ codes,
                                                               float* __restrict__ scales,
                                                               size_t n_rows, int len) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const size_t w = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const size_t r0 = w * kRowsPerWave;
  if (r0 >= n_rows) return;
  float4 rv[kRowsPerWave][NV];
#pragma unroll
  for (int k = 0; k < kRowsPerWave; k++) {
    const size_t row = min(r0 + k, n_rows - 1);
    const float* src = in + row * (size_t)len;
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int e = (i * 64 + lane) * 4;
      if (FULL || e < len) {
        const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + e));
        rv[k][i] = make_float4(t.x, t.y, t.z, t.w);
      } else {
        rv[k][i] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < kRowsPerWave; k++) {
    const size_t row = min(r0 + k, n_rows - 1);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; i++)
      amax = fmaxf(amax, fmaxf(fmaxf(fabsf(rv[k][i].x), fabsf(rv[k][i].y)),
                               fmaxf(fabsf(rv[k][i].z), fabsf(rv[k][i].w))));
    amax = wave_max_dpp(amax);
    const float inv = amax != 0.0f ? 127.0f / amax : 0.0f;
    int8_t* dst = codes + row * (size_t)len;
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int e = (i * 64 + lane) * 4;
      // amax == 0 gives inv == 0 and so codes 0 (NaN inputs map to 0 too):
      // no branch needed
      if (FULL || e < len)
        __builtin_nontemporal_store(pack4(rv[k][i].x, rv[k][i].y, rv[k][i].z, rv[k][i].w, inv),
                                    reinterpret_cast<uint32_t*>(dst + e));
    }
    if (lane == 0) scales[row] = amax / 127.0f;  // 0 when amax == 0
  }
}

template <int NV>
__global__ __launch_bounds__(256) void kv_quantize_kernel(const float* __restrict__ in,
                                                          int8_t* __restrict__ codes,
                                                          float* __restrict__ scales,
                                                          size_t n_rows, int row_len) {
  const size_t waves = (size_t)gridDim.x * (blockDim.x >> 6);
  for (size_t r = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); r < n_rows; r += waves)
    quantize_row<NV>(in + r * row_len, row_len, codes + r * row_len, scales + r);
}

// slot_mapping[t] = physical row (block * block_size + slot) of token t, or < 0 to skip.
template <int NV>
__global__ __launch_bounds__(256) void paged_append_kernel(
    const float* __restrict__ k, const float* __restrict__ v, const int32_t* __restrict__ slots,
    int8_t* __restrict__ kc, float* __restrict__ ks, int8_t* __restrict__ vc,
    float* __restrict__ vs, size_t n_tokens, int kv_dim) {
  const size_t waves = (size_t)gridDim.x * (blockDim.x >> 6);
  for (size_t i = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); i < 2 * n_tokens; i += waves) {
    const size_t t = i >> 1;
    const int32_t slot = slots[t];
    if (slot < 0) continue;
    const bool is_v = (i & 1) != 0;
    const float* src = (is_v ? v : k) + t * kv_dim;
    int8_t* dst = (is_v ? vc : kc) + (size_t)slot * kv_dim;
    float* sc = (is_v ? vs : ks) + slot;
    quantize_row<NV>(src, kv_dim, dst, sc);
  }
}

__global__ __launch_bounds__(256) void kv_dequantize_kernel(const int8_t* __restrict__ codes,
                                                            const float* __restrict__ scales,
                                                            float* __restrict__ out, size_t n_rows,
                                                            int row_len) {
  const size_t total = n_rows * (size_t)row_len;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride)
    out[i] = (float)codes[i] * scales[i / row_len];
}

unsigned grid_waves(size_t rows) {
  size_t g = (rows + 3) / 4;
  const size_t cap = (size_t)device_cu_count() * 16;
  if (g > cap) g = cap;
  return (unsigned)(g ? g : 1);
}

// INT8 swap-file slots (the reference's SwapQuantMode::Int8 format,
// src/ssd/block_swap.rs:148-370): K codes [bs*kv] | V codes [bs*kv] |
// K scales [bs] f32 | V scales [bs] f32 | num_filled u32.  The pool already
// holds the bit-exact codes and scales, so swap-out is a gather of physical
// blocks into consecutive slots and swap-in the scatter back.  Slots are
// 2*bs*kv + 8*bs + 4 bytes apart (4-byte aligned), so the copies go a dword
// per lane; slots may live in device memory or in mapped pinned host memory.
// grid.y = slot, grid.x strides over its dwords.
__global__ __launch_bounds__(256) void kv_swap_out_kernel(const int8_t* __restrict__ kc, const float* __restrict__ ks,
                                                          const int8_t* __restrict__ vc, const float* __restrict__ vs,
                                                          const int32_t* __restrict__ ids,
                                                          const uint32_t* __restrict__ nfill, int bs, int kv,
                                                          long n_pool, uint8_t* __restrict__ slots,
                                                          size_t slot_bytes) {
  const int blk = blockIdx.y;
  const long b = ids[blk];
  const bool valid = b >= 0 && b < n_pool;  // other ids give a zero slot
  uint32_t* dst = reinterpret_cast<uint32_t*>(slots + (size_t)blk * slot_bytes);
  const size_t nc = (size_t)bs * kv / 4, base = valid ? (size_t)b * bs : 0;
  const uint32_t* kd = reinterpret_cast<const uint32_t*>(kc) + base * kv / 4;
  const uint32_t* vd = reinterpret_cast<const uint32_t*>(vc) + base * kv / 4;
  const size_t total = 2 * nc + 2 * (size_t)bs + 1;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    uint32_t v = 0;
    if (valid) {
      if (i < nc) v = kd[i];
      else if (i < 2 * nc) v = vd[i - nc];
      else if (i < 2 * nc + bs) v = __float_as_uint(ks[base + (i - 2 * nc)]);
      else if (i < 2 * nc + 2 * bs) v = __float_as_uint(vs[base + (i - 2 * nc - bs)]);
      else v = nfill ? nfill[blk] : 0u;
    }
    dst[i] = v;
  }
}

__global__ __launch_bounds__(256) void kv_swap_in_kernel(const uint8_t* __restrict__ slots, size_t slot_bytes,
                                                         const int32_t* __restrict__ ids, int bs, int kv, long n_pool,
                                                         int8_t* __restrict__ kc, float* __restrict__ ks,
                                                         int8_t* __restrict__ vc, float* __restrict__ vs,
                                                         uint32_t* __restrict__ nfill) {
  const int blk = blockIdx.y;
  const long b = ids[blk];
  if (b < 0 || b >= n_pool) return;  // ignored
  const uint32_t* src = reinterpret_cast<const uint32_t*>(slots + (size_t)blk * slot_bytes);
  const size_t nc = (size_t)bs * kv / 4, base = (size_t)b * bs;
  uint32_t* kd = reinterpret_cast<uint32_t*>(kc) + base * kv / 4;
  uint32_t* vd = reinterpret_cast<uint32_t*>(vc) + base * kv / 4;
  const size_t total = 2 * nc + 2 * (size_t)bs + 1;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const uint32_t v = src[i];
    if (i < nc) kd[i] = v;
    else if (i < 2 * nc) vd[i - nc] = v;
    else if (i < 2 * nc + bs) ks[base + (i - 2 * nc)] = __uint_as_float(v);
    else if (i < 2 * nc + 2 * bs) vs[base + (i - 2 * nc - bs)] = __uint_as_float(v);
    else if (nfill) nfill[blk] = v;
  }
}

}  // namespace

hipError_t launch_kv_quantize(const float* in, int8_t* codes, float* scales, size_t n_rows,
                              size_t row_len, hipStream_t s) {
  if (n_rows == 0) return hipSuccess;
  const bool vec = row_len % 4 == 0 && ((uintptr_t)in & 15) == 0 && ((uintptr_t)codes & 3) == 0;
  if (vec && row_len <= 64 * 4 * 4) {
    const size_t waves = (n_rows + kRowsPerWave - 1) / kRowsPerWave;
    const size_t g = (waves + 3) / 4;
    if (g > 0x7FFFFFFF) return hipErrorInvalidValue;
    const dim3 grid((unsigned)g);
    if (row_len == 64 * 4 * 4)
      hipLaunchKernelGGL((kv_quantize_pipe_kernel<4, true>), grid, dim3(256), 0, s, in, codes, scales,
                         n_rows, (int)row_len);
    else
      hipLaunchKernelGGL((kv_quantize_pipe_kernel<4, false>), grid, dim3(256), 0, s, in, codes, scales,
                         n_rows, (int)row_len);
    return hipGetLastError();
  }
  if (row_len <= 64 * 4 * 4)
    hipLaunchKernelGGL(kv_quantize_kernel<4>, dim3(grid_waves(n_rows)), dim3(256), 0, s, in, codes,
                       scales, n_rows, (int)row_len);
  else
    hipLaunchKernelGGL(kv_quantize_kernel<8>, dim3(grid_waves(n_rows)), dim3(256), 0, s, in, codes,
                       scales, n_rows, (int)row_len);
  return hipGetLastError();
}

hipError_t launch_paged_kv_append(const float* k, const float* v, const int32_t* slot_mapping,
                                  int8_t* k_codes, float* k_scales, int8_t* v_codes,
                                  float* v_scales, size_t n_tokens, size_t kv_dim, hipStream_t s) {
  if (n_tokens == 0) return hipSuccess;
  if (kv_dim <= 64 * 4 * 4)
    hipLaunchKernelGGL(paged_append_kernel<4>, dim3(grid_waves(2 * n_tokens)), dim3(256), 0, s, k,
                       v, slot_mapping, k_codes, k_scales, v_codes, v_scales, n_tokens, (int)kv_dim);
  else
    hipLaunchKernelGGL(paged_append_kernel<8>, dim3(grid_waves(2 * n_tokens)), dim3(256), 0, s, k,
                       v, slot_mapping, k_codes, k_scales, v_codes, v_scales, n_tokens, (int)kv_dim);
  return hipGetLastError();
}

hipError_t launch_kv_dequantize(const int8_t* codes, const float* scales, float* out,
                                size_t n_rows, size_t row_len, hipStream_t s) {
  const size_t total = n_rows * row_len;
  if (total == 0) return hipSuccess;
  size_t g = (total + 255) / 256;
  if (g > 65536) g = 65536;
  hipLaunchKernelGGL(kv_dequantize_kernel, dim3((unsigned)g), dim3(256), 0, s, codes, scales, out,
                     n_rows, (int)row_len);
  return hipGetLastError();
}

size_t kv_slot_bytes(size_t bs, size_t kv) { return 2 * bs * kv + 8 * bs + 4; }

static dim3 swap_grid(size_t n_blocks, size_t bs, size_t kv) {
  const size_t dwords = (2 * bs * kv + 8 * bs + 4) / 4;
  const size_t per = 256 * 8;  // about eight dwords per lane
  return dim3((unsigned)std::min<size_t>((dwords + per - 1) / per, 1024), (unsigned)n_blocks);
}

hipError_t launch_kv_swap_out(const int8_t* kc, const float* ks, const int8_t* vc, const float* vs,
                              const int32_t* ids, const uint32_t* nfill, size_t n_blocks, size_t bs, size_t kv,
                              size_t n_pool, void* slots, hipStream_t s) {
  if (n_blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(kv_swap_out_kernel, swap_grid(n_blocks, bs, kv), dim3(256), 0, s, kc, ks, vc, vs, ids, nfill,
                     (int)bs, (int)kv, (long)n_pool, (uint8_t*)slots, kv_slot_bytes(bs, kv));
  return hipGetLastError();
}

hipError_t launch_kv_swap_in(const void* slots, const int32_t* ids, size_t n_blocks, size_t bs, size_t kv,
                             size_t n_pool, int8_t* kc, float* ks, int8_t* vc, float* vs, uint32_t* nfill,
                             hipStream_t s) {
  if (n_blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(kv_swap_in_kernel, swap_grid(n_blocks, bs, kv), dim3(256), 0, s, (const uint8_t*)slots,
                     kv_slot_bytes(bs, kv), ids, (int)bs, (int)kv, (long)n_pool, kc, ks, vc, vs, nfill);
  return hipGetLastError();
}

}  // namespace ssdq
