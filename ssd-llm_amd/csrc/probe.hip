// Measurement kernels for bench.py (libssdq_probe.so, not part of libssdq.so
// or its C ABI): a plain streaming read, which sets the HBM read ceiling the
// matvec kernels are compared with, and an empty kernel, which sets the fixed
// cost of one launch.  No reference counterpart.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

// Each workgroup reads one contiguous slice with 16-byte loads, UNROLL loads
// in flight per thread, and XOR-reduces it; the result is stored only if it
// equals a constant no input produces in practice (keeps the loads live).
template <int UNROLL>
__global__ __launch_bounds__(1024) void stream_read(const uint4* __restrict__ p, size_t n16,
                                                    uint32_t* __restrict__ sink) {
  const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const size_t b = (size_t)blockIdx.x * per, e = b + per < n16 ? b + per : n16;
  uint32_t acc = 0;
  for (size_t i = b + threadIdx.x; i < e; i += (size_t)blockDim.x * UNROLL) {
    uint4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; u++) {
      const size_t j = i + (size_t)u * blockDim.x;
      v[u] = j < e ? p[j] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < UNROLL; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

__global__ void empty_kernel() {}

}  // namespace

extern "C" {

// Streams `bytes` (a multiple of 16, 16-byte aligned) with `grid` x `block`
// threads; returns a hipError_t.
int ssdq_probe_read(const void* p, size_t bytes, uint32_t* sink, int grid, int block, void* stream) {
  if (!p || !sink || (bytes & 15) || ((uintptr_t)p & 15) || grid <= 0 || block <= 0 || block > 1024)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(stream_read<4>, dim3((unsigned)grid), dim3((unsigned)block), 0, (hipStream_t)stream,
                     static_cast<const uint4*>(p), bytes / 16, sink);
  return (int)hipGetLastError();
}

int ssdq_probe_empty(int grid, int block, void* stream) {
  if (grid <= 0 || block <= 0 || block > 1024) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(empty_kernel, dim3((unsigned)grid), dim3((unsigned)block), 0, (hipStream_t)stream);
  return (int)hipGetLastError();
}

}  // extern "C"
