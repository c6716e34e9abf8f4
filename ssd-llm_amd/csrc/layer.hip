// Element-wise decode-layer ops around the quantized matvec: RoPE, SwiGLU and
// RMSNorm (with the residual add of the post-attention norm).  Reference
// semantics: rope_f32_multi_head (src/metal/compute.rs:482-507), silu_f32
// (641-645) times up (src/inference/feed_forward.rs:28-40),
// fused_post_attn_norm_f32_cpu (compute.rs:536-555).  These are the unfused
// path; the fused matvec (matvec.hip) applies the same epilogues in-kernel.
#include "common.hpp"
#include "launch.hpp"

namespace ssdq {
namespace {

__global__ __launch_bounds__(256) void rope_kernel(float* __restrict__ v, int n, int head_dim, RopeTable rope) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;  // pair index
  const int r = 2 * p;
  if (r + 1 >= n) return;  // the reference's idx1 < len guard
  const int i = (r % head_dim) >> 1;
  const float sn = rope.sn[i], cs = rope.cs[i];
  const float x0 = v[r], x1 = v[r + 1];
  v[r] = x0 * cs - x1 * sn;
  v[r + 1] = x0 * sn + x1 * cs;
}

__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                     float* __restrict__ h, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    const float a = g[i];
    h[i] = (a / (1.0f + expf(-a))) * u[i];
  }
}

// out = a + b: the FFN residual add of the decoder layer (transformer.rs:378-380);
// out may alias a or b (each thread reads its element before writing it).
__global__ __launch_bounds__(256) void residual_add_kernel(float* out, const float* a, const float* b, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = a[i] + b[i];
}

// One workgroup: the whole vector (n is a hidden size, a few thousand).  Up to
// 8 elements per thread are kept in registers with their norm weights, so x,
// the residual and w are all requested before the reduction (one memory round
// trip); longer vectors take a second pass.
// x, res, hidden_out and out are not __restrict__: out and hidden_out may
// alias x (the in-place post-attention form).
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float* x, const float* res,
                                                       const float* __restrict__ w, float eps,
                                                       float* hidden_out, float* out, int n) {
  __shared__ float part[16];
  constexpr int KEEP = 8;
  float hv[KEEP], wv[KEEP];
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < KEEP; j++) {
    const int i = threadIdx.x + j * blockDim.x;
    const bool in = i < n;
    const float xv = in ? x[i] : 0.f;
    const float rv = (in && res) ? res[i] : 0.f;
    wv[j] = in ? w[i] : 0.f;
    hv[j] = xv + rv;
    q = fmaf(hv[j], hv[j], q);
  }
  for (int i = threadIdx.x + KEEP * blockDim.x; i < n; i += blockDim.x) {
    const float h = res ? x[i] + res[i] : x[i];
    q = fmaf(h, h, q);
  }
  q = wave_sum_l63(q);  // valid in lane 63
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 63) part[wave] = q;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); i++) t += part[i];
  const float inv = 1.0f / sqrtf(t / (float)n + eps);
  // each thread rewrites only the elements it read (out / hidden_out may alias x)
#pragma unroll
  for (int j = 0; j < KEEP; j++) {
    const int i = threadIdx.x + j * blockDim.x;
    if (i < n) {
      if (hidden_out) hidden_out[i] = hv[j];
      out[i] = hv[j] * inv * wv[j];
    }
  }
  for (int i = threadIdx.x + KEEP * blockDim.x; i < n; i += blockDim.x) {
    const float h = res ? x[i] + res[i] : x[i];
    if (hidden_out) hidden_out[i] = h;
    out[i] = h * inv * w[i];
  }
}

}  // namespace

hipError_t launch_rope(float* v, int n, int head_dim, const RopeTable& rope, hipStream_t s) {
  if (n <= 1) return hipSuccess;
  const int pairs = n / 2;
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, s, v, n, head_dim, rope);
  return hipGetLastError();
}

hipError_t launch_swiglu(const float* g, const float* u, float* h, int n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, u, h, n);
  return hipGetLastError();
}

hipError_t launch_add(float* out, const float* a, const float* b, int n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(residual_add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, a, b, n);
  return hipGetLastError();
}

hipError_t launch_residual_add(float* h, const float* a, int n, hipStream_t s) { return launch_add(h, h, a, n, s); }

hipError_t launch_rmsnorm(const float* x, const float* residual, const float* w, float eps, float* hidden_out,
                          float* out, int n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(1), dim3(1024), 0, s, x, residual, w, eps, hidden_out, out, n);
  return hipGetLastError();
}

}  // namespace ssdq
