// Measurement kernels for bench.py (libssdq_probe.so, not part of libssdq.so
// or its C ABI): a plain streaming read (ordinary or nontemporal loads), which
// sets the HBM read ceiling the matvec kernels are compared with; an empty
// kernel, which sets the fixed cost of one launch; and an fp16 MFMA loop with
// operands in registers, which sets the matrix-core rate the prefill GEMM is
// compared with.  No reference counterpart.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// Each workgroup reads one contiguous slice with 16-byte loads, UNROLL loads
// in flight per thread, and XOR-reduces it; the result is stored only if it
// equals a constant no input produces in practice (keeps the loads live).
// NT: nontemporal loads.
template <int UNROLL, bool NT>
__global__ __launch_bounds__(1024) void stream_read(const u32x4* __restrict__ p, size_t n16,
                                                    uint32_t* __restrict__ sink) {
  const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const size_t b = (size_t)blockIdx.x * per, e = b + per < n16 ? b + per : n16;
  uint32_t acc = 0;
  for (size_t i = b + threadIdx.x; i < e; i += (size_t)blockDim.x * UNROLL) {
    u32x4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; u++) {
      const size_t j = i + (size_t)u * blockDim.x;
      if (j < e) v[u] = NT ? __builtin_nontemporal_load(p + j) : p[j];
      else v[u] = u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < UNROLL; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

__global__ void empty_kernel() {}

// Eight independent accumulator chains of v_mfma_f32_16x16x32_f16 per wave,
// iters rounds, operands from 8 fp16 vectors per lane read once from src
// (4096 entries: random or zero values decide the switching activity), and NV
// pairs of independent integer VALU instructions (permute, xor) after each
// MFMA.  FLOP per launch: 16384 x 8 x iters x waves.
template <int NV>
__global__ __launch_bounds__(512) void mfma_loop(const h8* __restrict__ src, float* __restrict__ out, int iters) {
  const int t = threadIdx.x + blockIdx.x * blockDim.x;
  h8 a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    a[i] = src[(t * 8 + i) & 4095];
    b[i] = src[(t * 8 + 4 + i) & 4095];
  }
  f4 acc[8];
  uint32_t x[8];
#pragma unroll
  for (int c = 0; c < 8; c++) {
    acc[c] = f4{0.f, 0.f, 0.f, 0.f};
    x[c] = (uint32_t)(t * 7 + c);
  }
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int c = 0; c < 8; c++) {
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c & 3], b[(c >> 2) & 3], acc[c], 0, 0, 0);
#pragma unroll
      for (int v = 0; v < NV; v++)
        x[(c + v) & 7] = __builtin_amdgcn_perm(x[(c + v) & 7], x[(c + v + 1) & 7], 0x05040100u + v) ^ (uint32_t)it;
    }
  }
  float s = 0.f;
  uint32_t xs = 0;
#pragma unroll
  for (int c = 0; c < 8; c++) {
    s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
    xs ^= x[c];
  }
  out[t] = s + (float)(xs & 1u);
}

}  // namespace

extern "C" {

// Streams `bytes` (a multiple of 16, 16-byte aligned) with `grid` x `block`
// threads; returns a hipError_t.
int ssdq_probe_read(const void* p, size_t bytes, uint32_t* sink, int grid, int block, void* stream) {
  if (!p || !sink || (bytes & 15) || ((uintptr_t)p & 15) || grid <= 0 || block <= 0 || block > 1024)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL((stream_read<4, false>), dim3((unsigned)grid), dim3((unsigned)block), 0, (hipStream_t)stream,
                     static_cast<const u32x4*>(p), bytes / 16, sink);
  return (int)hipGetLastError();
}

// As ssdq_probe_read, with nontemporal loads.
int ssdq_probe_read_nt(const void* p, size_t bytes, uint32_t* sink, int grid, int block, void* stream) {
  if (!p || !sink || (bytes & 15) || ((uintptr_t)p & 15) || grid <= 0 || block <= 0 || block > 1024)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL((stream_read<4, true>), dim3((unsigned)grid), dim3((unsigned)block), 0, (hipStream_t)stream,
                     static_cast<const u32x4*>(p), bytes / 16, sink);
  return (int)hipGetLastError();
}

// mfma_loop<nv> (nv in 0..2 pairs of VALU instructions per MFMA) with `grid` x
// `block` threads (block a multiple of 64, at most 512); src: 4096 x 8 fp16
// values (64 KB), out: grid x block floats.
int ssdq_probe_mfma(const void* src, float* out, int iters, int nv, int grid, int block, void* stream) {
  if (!src || !out || iters <= 0 || nv < 0 || nv > 2 || grid <= 0 || block <= 0 || block > 512 || (block & 63))
    return (int)hipErrorInvalidValue;
  const h8* sp = static_cast<const h8*>(src);
  hipStream_t s = (hipStream_t)stream;
  if (nv == 0) hipLaunchKernelGGL(mfma_loop<0>, dim3((unsigned)grid), dim3((unsigned)block), 0, s, sp, out, iters);
  else if (nv == 1) hipLaunchKernelGGL(mfma_loop<1>, dim3((unsigned)grid), dim3((unsigned)block), 0, s, sp, out, iters);
  else hipLaunchKernelGGL(mfma_loop<2>, dim3((unsigned)grid), dim3((unsigned)block), 0, s, sp, out, iters);
  return (int)hipGetLastError();
}

int ssdq_probe_empty(int grid, int block, void* stream) {
  if (grid <= 0 || block <= 0 || block > 1024) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(empty_kernel, dim3((unsigned)grid), dim3((unsigned)block), 0, (hipStream_t)stream);
  return (int)hipGetLastError();
}

}  // extern "C"
