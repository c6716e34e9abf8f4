// Prefill GEMM: Y[M,N] f32 = X[M,K] bf16 x W[N,K]^T, W in Q4_K (reference layout).
//
// The reference has no GEMM: prefill runs one matvec per token
// (src/inference/transformer.rs:166-196 -> matvec_q4_k_cpu,
// src/metal/compute.rs:707-750), so Y[t,:] = matvec(W, widen_bf16(X[t,:])).
// This computes the same Y on the matrix cores:
//   * every weight is dequantized exactly as the reference does it,
//     w = fl(fl(d*s) * q) - fl(dmin*m) in fp32 (compute.rs:716-744), then split
//     into fp16 hi + lo parts (hi = w with the low 13 mantissa bits cleared,
//     lo = w - hi), so w is carried to ~22 bits.  One fp16 part alone would
//     leave ~1e-4 relative error per output, too close to the 1e-3 / 1e-4
//     tolerance on rows with cancellation;
//   * X is bf16, exactly representable in fp16 inside fp16's normal range;
//   * v_mfma_f32_16x16x32_f16 accumulates X*hi + X*lo in fp32.
// Tiling: a workgroup of 4 waves computes a 128 (M) x 128 (N) tile.  X tiles
// (128 x 32) are converted to fp16 once per workgroup and double-buffered in
// LDS; each wave owns 32 columns of N and dequantizes its own weights straight
// into MFMA B fragments (no weight traffic through LDS), reusing each fragment
// for the 8 M sub-tiles.  Weights and X are prefetched two K steps ahead.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace ssdq {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int XS = BK + 8;   // LDS row stride in halves (80 B keeps 16-byte reads conflict free)
constexpr int MT = BM / 16;  // M sub-tiles per wave
constexpr int NT = 2;        // N sub-tiles (of 16 columns) per wave
constexpr int PF = 2;        // K steps in flight

__global__ __launch_bounds__(256) void widen_bf16_kernel(const uint16_t* __restrict__ x,
                                                         float* __restrict__ out, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = __uint_as_float((uint32_t)x[i] << 16);
}

// 8 bf16 (one uint4, element order) -> 8 fp16 at dst.
__device__ __forceinline__ void bf16x8_to_f16(uint4 v, _Float16* dst) {
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
  h8 h;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    h[2 * i] = (_Float16)__uint_as_float(d[i] << 16);
    h[2 * i + 1] = (_Float16)__uint_as_float(d[i] & 0xFFFF0000u);
  }
  *reinterpret_cast<h8*>(dst) = h;
}

// Dequantizes the 8 codes of one packed dword (nibble i = element i of the
// lane's 8-element k range) with scale S and offset Mn exactly as the
// reference, and splits each value into fp16 hi / lo.
__device__ __forceinline__ void dequant8_split(uint32_t q, float S, float Mn, h8& hi, h8& lo) {
#pragma clang fp contract(off)
  const uint32_t ql = opaque(q & 0x0F0F0F0Fu), qh = opaque((q >> 4) & 0x0F0F0F0Fu);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float w0 = S * (float)byte_of(ql, i) - Mn;  // fl(fl(S*q) - M)
    const float w1 = S * (float)byte_of(qh, i) - Mn;
    const float h0 = __uint_as_float(__float_as_uint(w0) & 0xFFFFE000u);
    const float h1 = __uint_as_float(__float_as_uint(w1) & 0xFFFFE000u);
    hi[2 * i] = (_Float16)h0;
    hi[2 * i + 1] = (_Float16)h1;
    lo[2 * i] = (_Float16)(w0 - h0);
    lo[2 * i + 1] = (_Float16)(w1 - h1);
  }
}

// blockIdx.z selects split z of the K range (split = gridDim.z); split z
// writes its partial product to y + z * M * N (a workspace when split > 1).
__global__ __launch_bounds__(256, 2) void gemm_q4k_mfma(const uint8_t* __restrict__ w,
                                                        const uint16_t* __restrict__ x,
                                                        float* __restrict__ y, int M, int N, int K) {
  __shared__ __align__(16) _Float16 xs[2][BM * XS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int blocks = K / 256, z = blockIdx.z, nz = gridDim.z;
  const int b_begin = (int)((long)blocks * z / nz), b_end = (int)((long)blocks * (z + 1) / nz);
  const int s0 = b_begin * 8, steps = (b_end - b_begin) * 8;  // K steps of this split
  y += (size_t)z * M * N;
  const size_t row_bytes = (size_t)(K / 256) * 144;
  const int c = lane >> 4;  // this lane holds k = 8c .. 8c+7 of each 32-wide step

  // weight rows of this lane's B fragments (clamped; columns past N are not stored)
  const uint8_t* wrow[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) {
    const int n = min(n0 + 32 * wave + 16 * j + (lane & 15), N - 1);
    wrow[j] = w + (size_t)n * row_bytes;
  }
  // X staging: thread t converts row t/2, k half (t&1)*16 of each step
  const int xr = threadIdx.x >> 1, xk = (threadIdx.x & 1) * 16;
  const uint16_t* xrow = x + (size_t)min(m0 + xr, M - 1) * K + xk;

  // register queues for steps s .. s+PF-1
  uint4 xq[PF][2];
  uint32_t hq[PF][NT][4];  // block header: d|dmin, scale bytes 0-3, 4-7, 8-11
  uint32_t qq[PF][NT];     // this lane's 8 codes of the step's sub-block
  auto fetch = [&](int s, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    const int ss = s0 + min(s, steps - 1);
    const uint16_t* xp = xrow + (size_t)ss * BK;
    xq[slot][0] = *reinterpret_cast<const uint4*>(xp);
    xq[slot][1] = *reinterpret_cast<const uint4*>(xp + 8);
    const int blk = ss >> 3, sb = ss & 7;
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const uint8_t* b = wrow[j] + (size_t)blk * 144;
      const u32x4a4 h = *reinterpret_cast<const u32x4a4*>(b);
      hq[slot][j][0] = h.x;
      hq[slot][j][1] = h.y;
      hq[slot][j][2] = h.z;
      hq[slot][j][3] = h.w;
      qq[slot][j] = *reinterpret_cast<const uint32_t*>(b + 16 + 16 * sb + 4 * c);
    }
  };

  f4 acc[MT][NT];

  fetch(0, std::integral_constant<int, 0>{});
  fetch(1, std::integral_constant<int, 1>{});
  bf16x8_to_f16(xq[0][0], &xs[0][xr * XS + xk]);
  bf16x8_to_f16(xq[0][1], &xs[0][xr * XS + xk + 8]);
  __syncthreads();

  // Step s uses queue slot and LDS buffer s % 2; the loop is unrolled by two so
  // every register-array index is a compile-time constant.  The matrix-core
  // accumulators restart at every super-block (8 steps; the first MFMA of a
  // chain takes C = 0) and are added into fp32 VALU sums, so no accumulator
  // carries a long chain of roundings at the magnitude of the full dot product
  // (measured at K = 4096: rms error against the exact sum 7e-5 without
  // restarts, 2e-5 with; the serial fp32 reference itself is at 1e-4).
  f4 tot[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) tot[i][j] = f4{0.f, 0.f, 0.f, 0.f};
  auto step = [&](auto slot, int s, auto first_c) {
    constexpr int cur = decltype(slot)::value;
    constexpr bool first = decltype(first_c)::value;
    const int sb = s & 7;
    // B fragments of this step
    h8 bhi[NT], blo[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const float d = f16_to_f32(hq[cur][j][0] & 0xFFFFu), dmin = f16_to_f32(hq[cur][j][0] >> 16);
      uint32_t sc, mn;
      q4k_scale_min(hq[cur][j][1], hq[cur][j][2], hq[cur][j][3], sb, sc, mn);
      float S, Mn;
      {
#pragma clang fp contract(off)
        S = d * (float)sc;
        Mn = dmin * (float)mn;
      }
      dequant8_split(qq[cur][j], S, Mn, bhi[j], blo[j]);
    }
    // X of step s+1 goes to the other LDS buffer (its readers finished at the
    // barrier that ended step s-1); this queue slot is refilled with step s+2
    const uint4 nx0 = xq[cur ^ 1][0], nx1 = xq[cur ^ 1][1];
    fetch(s + PF, slot);
    // all hi products first, then all lo products: the two MFMAs into one
    // accumulator are MT*NT instructions apart instead of back to back
    h8 a[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
      a[mt] = *reinterpret_cast<const h8*>(&xs[cur][(mt * 16 + (lane & 15)) * XS + 8 * c]);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int j = 0; j < NT; j++)
        acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            a[mt], bhi[j], first ? f4{0.f, 0.f, 0.f, 0.f} : acc[mt][j], 0, 0, 0);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int j = 0; j < NT; j++)
        acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt], blo[j], acc[mt][j], 0, 0, 0);
    if (s + 1 < steps) {
      bf16x8_to_f16(nx0, &xs[cur ^ 1][xr * XS + xk]);
      bf16x8_to_f16(nx1, &xs[cur ^ 1][xr * XS + xk + 8]);
    }
    // LDS-only barrier: the prefetched global loads stay in flight
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using T = std::true_type;
  using Fa = std::false_type;
  for (int s = 0; s < steps; s += 8) {  // one super-block per iteration
    step(I0{}, s, T{});
    step(I1{}, s + 1, Fa{});
    step(I0{}, s + 2, Fa{});
    step(I1{}, s + 3, Fa{});
    step(I0{}, s + 4, Fa{});
    step(I1{}, s + 5, Fa{});
    step(I0{}, s + 6, Fa{});
    step(I1{}, s + 7, Fa{});
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int j = 0; j < NT; j++) tot[i][j] += acc[i][j];
  }

  // C fragment layout: element i of acc[mt][j] is row 4*(lane/16)+i, column lane%16
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const int n = n0 + 32 * wave + 16 * j + (lane & 15);
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = m0 + mt * 16 + 4 * c + i;
        if (m < M) y[(size_t)m * N + n] = tot[mt][j][i];
      }
    }
}

// Sums split-K partials in a fixed order (deterministic results).
__global__ __launch_bounds__(256) void splitk_reduce(const float* __restrict__ part, float* __restrict__ y,
                                                     size_t mn, int split) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn; i += stride) {
    float s = part[i];
    for (int z = 1; z < split; z++) s += part[(size_t)z * mn + i];
    y[i] = s;
  }
}

}  // namespace

bool gemm_q4k_mfma_ok(const void* w, const void* x) {
  return ((uintptr_t)w & 3) == 0 && ((uintptr_t)x & 15) == 0;
}

// K splits for a GEMM: enough workgroups for two per CU, at most 8 splits and
// never more than one split per 256-element block.
int gemm_q4k_split(size_t M, size_t N, size_t K) {
  const size_t tiles = ((N + BN - 1) / BN) * ((M + BM - 1) / BM);
  const size_t want = 2 * (size_t)device_cu_count();
  size_t split = tiles >= want ? 1 : (want + tiles - 1) / tiles;
  split = std::min<size_t>(split, 8);
  split = std::min<size_t>(split, K / 256);
  return (int)std::max<size_t>(split, 1);
}

size_t gemm_q4k_workspace_bytes(const void* w, const void* x, size_t M, size_t N, size_t K) {
  if (!gemm_q4k_mfma_ok(w, x)) return M * K * sizeof(float);
  const int split = gemm_q4k_split(M, N, K);
  return split > 1 ? (size_t)split * M * N * sizeof(float) : 0;
}

hipError_t launch_gemm_q4k(const uint8_t* w, const uint16_t* x, float* y, size_t M, size_t N,
                           size_t K, void* workspace, size_t workspace_bytes, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  if (K % 256 != 0) return hipErrorInvalidValue;
  if (gemm_q4k_mfma_ok(w, x)) {
    const int split = gemm_q4k_split(M, N, K);
    const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM), (unsigned)split);
    if (grid.y > 65535) return hipErrorInvalidValue;
    if (split == 1) {
      hipLaunchKernelGGL(gemm_q4k_mfma, grid, dim3(256), 0, s, w, x, y, (int)M, (int)N, (int)K);
      return hipGetLastError();
    }
    if (workspace_bytes < (size_t)split * M * N * sizeof(float)) return hipErrorInvalidValue;
    float* part = static_cast<float*>(workspace);
    hipLaunchKernelGGL(gemm_q4k_mfma, grid, dim3(256), 0, s, w, x, part, (int)M, (int)N, (int)K);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const size_t mn = M * N;
    const unsigned g = (unsigned)std::min<size_t>((mn + 255) / 256, 8192);
    hipLaunchKernelGGL(splitk_reduce, dim3(g), dim3(256), 0, s, part, y, mn, split);
    return hipGetLastError();
  }
  // Misaligned operands: widen X to f32 (exact) and run the batched matvec,
  // which reads W once per group of up to 8 tokens.
  if (workspace_bytes < M * K * sizeof(float)) return hipErrorInvalidValue;
  float* xf = static_cast<float*>(workspace);
  size_t n = M * K, g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  hipLaunchKernelGGL(widen_bf16_kernel, dim3((unsigned)g), dim3(256), 0, s, x, xf, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_matvec(kQ4_K, w, xf, y, N, K, M, s);
}

}  // namespace ssdq
