// Prefill GEMM: Y[M,N] f32 = X[M,K] bf16 x W[N,K] (Q4_K, reference layout).
//
// The reference has no GEMM: prefill runs one matvec per token
// (src/inference/transformer.rs:166-196 -> matvec_q4_k_cpu,
// src/metal/compute.rs:707-750), so Y[t,:] = matvec(W, widen_bf16(X[t,:])).
// This first version widens X to f32 once (bf16 -> f32 is exact,
// src/ssd/streamer.rs:108-114) and runs the batched matvec kernel, which reads
// W once per group of up to 8 tokens.
#include "common.hpp"
#include "launch.hpp"

namespace ssdq {
namespace {

__global__ __launch_bounds__(256) void widen_bf16_kernel(const uint16_t* __restrict__ x,
                                                         float* __restrict__ out, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = __uint_as_float((uint32_t)x[i] << 16);
}

}  // namespace

size_t gemm_q4k_workspace_bytes(size_t M, size_t N, size_t K) {
  (void)N;
  return M * K * sizeof(float);
}

hipError_t launch_gemm_q4k(const uint8_t* w, const uint16_t* x, float* y, size_t M, size_t N,
                           size_t K, void* workspace, size_t workspace_bytes, hipStream_t s) {
  if (workspace_bytes < gemm_q4k_workspace_bytes(M, N, K)) return hipErrorInvalidValue;
  float* xf = static_cast<float*>(workspace);
  size_t n = M * K, g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  hipLaunchKernelGGL(widen_bf16_kernel, dim3((unsigned)g), dim3(256), 0, s, x, xf, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_matvec(kQ4_K, w, xf, y, N, K, M, s);
}

}  // namespace ssdq
