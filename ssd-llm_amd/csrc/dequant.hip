// Bit-exact GGUF block dequantization to f32 (the check path for the fused
// kernels, and the device replacement for the load-time dequantizers).
//
// Element values follow the reference exactly, one IEEE rounding per Rust op:
//   Q4_0  (q - 8) * d                      src/ssd/streamer.rs:153-178
//   Q8_0  (i8) * d                         src/ssd/streamer.rs:128-150
//   Q6_K  (d * scale) * q                  src/ssd/streamer.rs:182-220
//   Q4_K  (d * s) * q - dmin * m           src/metal/compute.rs:716-744
// Contraction is switched off in every function that rounds twice, so
// (d*s)*q - M is never fused into an FMA.
#include "common.hpp"
#include "launch.hpp"

namespace ssdq {
namespace {

constexpr int kElemsPerThread = 8;

template <int F>
__device__ __forceinline__ void dequant8(const uint8_t* __restrict__ w, size_t e0, float* v) {
#pragma clang fp contract(off)
  constexpr int bs = Geom<F>::bs, bb = Geom<F>::bb;
  const size_t b = e0 / bs;
  const int r = (int)(e0 % bs);  // multiple of 8
  const uint8_t* blk = w + b * bb;
  if constexpr (F == kQ4_0) {
    const float d = f16_to_f32(ld_u16(blk));
    const uint8_t* qs = blk + 2 + r / 2;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t byte = qs[j];
      v[2 * j] = (float)((int)(byte & 15u) - 8) * d;
      v[2 * j + 1] = (float)((int)(byte >> 4) - 8) * d;
    }
  } else if constexpr (F == kQ8_0) {
    const float d = f16_to_f32(ld_u16(blk));
    const uint8_t* qs = blk + 2 + r;
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = (float)(int8_t)qs[j] * d;
  } else if constexpr (F == kQ4_K) {
    const float d = f16_to_f32(ld_u16(blk));
    const float dmin = f16_to_f32(ld_u16(blk + 2));
    const uint8_t* sc = blk + 4;
    const int sb = r / 32;
    uint32_t s, m;
    if (sb < 4) {
      s = sc[sb] & 63u;
      m = sc[sb + 4] & 63u;
    } else {
      s = ((uint32_t)sc[sb - 4] >> 6) | (((uint32_t)sc[sb + 4] & 15u) << 2);
      m = ((uint32_t)sc[sb] >> 6) | (((uint32_t)sc[sb + 4] >> 4) << 2);
    }
    const float S = d * (float)s;
    const float M = dmin * (float)m;
    const uint8_t* qs = blk + 16 + sb * 16 + (r % 32) / 2;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t byte = qs[j];
      const float p0 = S * (float)(byte & 15u);
      const float p1 = S * (float)(byte >> 4);
      v[2 * j] = p0 - M;
      v[2 * j + 1] = p1 - M;
    }
  } else {  // kQ6_K
    const float d = f16_to_f32(ld_u16(blk + 208));
    const float sc = (float)(int8_t)blk[192 + r / 16];
    const float ds = d * sc;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int idx = r + j;
      const uint32_t qlb = blk[idx / 2];
      const uint32_t lo4 = (idx & 1) ? (qlb >> 4) : (qlb & 15u);
      const uint32_t hi2 = ((uint32_t)blk[128 + idx / 4] >> (2 * (idx % 4))) & 3u;
      const int q = (int)(lo4 | (hi2 << 4)) - 32;
      v[j] = ds * (float)q;
    }
  }
}

template <int F>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w,
                                                      size_t n_groups, float* __restrict__ out) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < n_groups; g += stride) {
    float v[kElemsPerThread];
    dequant8<F>(w, g * kElemsPerThread, v);
    float* o = out + g * kElemsPerThread;
#pragma unroll
    for (int j = 0; j < kElemsPerThread; j++) o[j] = v[j];
  }
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ out, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = 0.0f;
}

// F32 / F16 / BF16 tensors (streamer.rs:95-115): copy, IEEE half widening,
// bf16 bits << 16.  4 elements per thread where the input allows it.
enum : int { kF32 = 0, kF16 = 1, kBF16 = 30 };

template <int T>
__device__ __forceinline__ float widen1(const uint8_t* __restrict__ w, size_t i) {
  if constexpr (T == kF32) return reinterpret_cast<const float*>(w)[i];
  else {
    const uint32_t h = reinterpret_cast<const uint16_t*>(w)[i];
    if constexpr (T == kF16) return f16_to_f32(h);
    else return __uint_as_float(h << 16);
  }
}

template <int T>
__global__ __launch_bounds__(256) void widen_kernel(const uint8_t* __restrict__ w, size_t n,
                                                    float* __restrict__ out) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = widen1<T>(w, i);
}

unsigned grid_for(size_t work, unsigned block) {
  size_t g = (work + block - 1) / block;
  if (g > 65536) g = 65536;
  if (g == 0) g = 1;
  return (unsigned)g;
}

}  // namespace

hipError_t launch_widen(int dtype, const void* w, size_t n, float* out, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const uint8_t* p = (const uint8_t*)w;
  const dim3 g(grid_for(n, 256)), b(256);
  switch (dtype) {
    case kF32: hipLaunchKernelGGL(widen_kernel<kF32>, g, b, 0, stream, p, n, out); break;
    case kF16: hipLaunchKernelGGL(widen_kernel<kF16>, g, b, 0, stream, p, n, out); break;
    case kBF16: hipLaunchKernelGGL(widen_kernel<kBF16>, g, b, 0, stream, p, n, out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_fill_zero(float* out, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, out, n);
  return hipGetLastError();
}

// Dequantizes n_elements (whole blocks only; the caller zero-fills the
// remainder like the reference's `resize`) of dtype into out.
hipError_t launch_dequant(int dtype, const uint8_t* w, size_t n_blocks, float* out,
                          hipStream_t stream) {
  if (n_blocks == 0) return hipSuccess;
  switch (dtype) {
#define SSDQ_DQ(F)                                                                       \
  case F: {                                                                              \
    const size_t groups = n_blocks * (Geom<F>::bs / kElemsPerThread);                    \
    hipLaunchKernelGGL(dequant_kernel<F>, dim3(grid_for(groups, 256)), dim3(256), 0,     \
                       stream, w, groups, out);                                          \
    return hipGetLastError();                                                            \
  }
    SSDQ_DQ(kQ4_0)
    SSDQ_DQ(kQ8_0)
    SSDQ_DQ(kQ4_K)
    SSDQ_DQ(kQ6_K)
#undef SSDQ_DQ
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace ssdq
