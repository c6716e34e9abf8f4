// Small-batch Q8_0 matmul (2 <= B <= 16 activation rows) on the matrix cores.
//
// Reference semantics: B independent matvec_q8_0_cpu calls
// (src/inference/batch_scheduler.rs:242-276 -> src/metal/compute.rs:904-925):
// y[b, r] = sum over blocks of sum_k fl(d * q) * x[b, k].
// A workgroup owns 16 weight rows; its 4 wavefronts split K and their results
// meet in LDS (fixed order).  Per 32-element block, two
// v_mfma_f32_16x16x32_f16 multiply A = the 16 rows' int8 codes (exact in
// fp16) by B = the block of x, column b = x row b, split into fp16 hi + lo
// parts (x carried to ~22 bits) that accumulate into one result; every
// product is exact in fp32.  Each block's 16x16 result is scaled by the rows'
// d (f16, exact in f32) and accumulated in fp32.  Weights are read as
// dword-aligned pairs of blocks (68 bytes).
#include "common.hpp"
#include "launch.hpp"

namespace ssdq {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3a4 __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));

// 8 int8 codes (two dwords, element order) -> 8 fp16
__device__ __forceinline__ h8 codes_f16(uint32_t lo, uint32_t hi) {
  h8 a;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    a[i] = (_Float16)(float)(int8_t)(lo >> (8 * i));
    a[4 + i] = (_Float16)(float)(int8_t)(hi >> (8 * i));
  }
  return a;
}

// Registers of one block pair for one lane: codes of both blocks (k = 8c ..
// 8c+7), the two d words, and x of both blocks for this lane's column.
struct Q8Pair {
  u32x3a4 a0;
  u32x2a4 a1;
  uint32_t dw0, dw8;
  float4 xa0, xa1, xb0, xb1;
};

constexpr int kQ8Waves = 4;  // K splits of a 16-row tile (one per wavefront)

__global__ __launch_bounds__(64 * kQ8Waves) void mv_q8_0_mfma(const uint8_t* __restrict__ w,
                                                             const float* __restrict__ x,
                                                             float* __restrict__ y, int out_dim,
                                                             int in_dim, int bpr, int B) {
  __shared__ f4 red[kQ8Waves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m0 = blockIdx.x * 16;
  const int r = lane & 15, c = lane >> 4;  // A row / C column, k group / C row group
  const uint8_t* wr = w + (size_t)min(m0 + r, out_dim - 1) * ((size_t)bpr * 34);
  const int b = r;  // this lane's B column: x row b
  const bool xv = b < B;
  const float* xr = x + (size_t)(xv ? b : 0) * in_dim + 8 * c;
  const int scale_src = 16 * c + 4 * c;  // lane holding the d of C row 4c (+i)
  const int pairs = bpr / 2;
  const int p_begin = pairs * wave / kQ8Waves, p_end = pairs * (wave + 1) / kQ8Waves;

  auto load = [&](int p, Q8Pair& q) {
    p = min(p, p_end - 1);
    const uint8_t* pp = wr + (size_t)p * 68;
    q.a0 = *reinterpret_cast<const u32x3a4*>(pp + 8 * c);       // block 0: bytes 8c .. 8c+11
    q.a1 = *reinterpret_cast<const u32x2a4*>(pp + 36 + 8 * c);  // block 1 codes 8c .. 8c+7
    q.dw0 = *reinterpret_cast<const uint32_t*>(pp);             // d0 | codes
    q.dw8 = *reinterpret_cast<const uint32_t*>(pp + 32);        // codes | d1
    const float4* xp = reinterpret_cast<const float4*>(xr + (size_t)p * 64);
    q.xa0 = xp[0]; q.xa1 = xp[1]; q.xb0 = xp[8]; q.xb1 = xp[9];
  };
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const Q8Pair& q) {
#pragma unroll
    for (int blk = 0; blk < 2; blk++) {
      const h8 a = blk == 0 ? codes_f16(__builtin_amdgcn_alignbit(q.a0.y, q.a0.x, 16),
                                        __builtin_amdgcn_alignbit(q.a0.z, q.a0.y, 16))
                            : codes_f16(q.a1.x, q.a1.y);
      const float4 u0 = blk == 0 ? q.xa0 : q.xb0, u1 = blk == 0 ? q.xa1 : q.xb1;
      const float xs[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
      h8 bh, bl;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const _Float16 hi = (_Float16)xs[i];
        bh[i] = xv ? hi : (_Float16)0.f;
        bl[i] = xv ? (_Float16)(xs[i] - (float)hi) : (_Float16)0.f;
      }
      f4 cm = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bh, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      cm = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bl, cm, 0, 0, 0);
      const float d = f16_to_f32(blk == 0 ? (q.dw0 & 0xFFFFu) : (q.dw8 >> 16));  // d of A row r
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float ds = __shfl(d, scale_src + i, 64);  // d of C row 4c+i
        acc[i] = fmaf(ds, cm[i], acc[i]);
      }
    }
  };
  if (p_begin < p_end) {  // three pairs in flight: compute pair p while p+1, p+2 load
    Q8Pair q0, q1, q2;
    load(p_begin, q0);
    load(p_begin + 1, q1);
    int p = p_begin;
    for (; p + 2 < p_end; p += 3) {
      load(p + 2, q2);
      compute(q0);
      load(p + 3, q0);
      compute(q1);
      load(p + 4, q1);
      compute(q2);
    }
    if (p < p_end) compute(q0);
    if (p + 1 < p_end) compute(q1);
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    f4 s = red[0][lane];
#pragma unroll
    for (int k = 1; k < kQ8Waves; k++) s += red[k][lane];
    if (xv) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = m0 + 4 * c + i;
        if (row < out_dim) y[(size_t)b * out_dim + row] = s[i];
      }
    }
  }
}

}  // namespace

bool mv_q8_0_mfma_ok(const void* w, const float* x, int in_dim, int bpr) {
  return ((uintptr_t)w & 3) == 0 && ((uintptr_t)x & 15) == 0 && (in_dim & 3) == 0 && bpr % 2 == 0;
}

hipError_t launch_mv_q8_0_mfma(const uint8_t* w, const float* x, float* y, int out_dim, int in_dim,
                               int bpr, int batch, hipStream_t s) {
  for (int b0 = 0; b0 < batch; b0 += 16) {
    const int B = batch - b0 < 16 ? batch - b0 : 16;
    const int tiles = (out_dim + 15) / 16;
    hipLaunchKernelGGL(mv_q8_0_mfma, dim3((unsigned)tiles), dim3(64 * kQ8Waves), 0, s, w,
                       x + (size_t)b0 * in_dim, y + (size_t)b0 * out_dim, out_dim, in_dim, bpr, B);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace ssdq
