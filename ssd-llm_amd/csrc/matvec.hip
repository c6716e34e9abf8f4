// Fused GGUF dequant + matvec / small-batch matmul for gfx950.
//
// Reference semantics: matvec_q4_0_cpu / matvec_q4_k_cpu / matvec_q6_k_cpu /
// matvec_q8_0_cpu (src/metal/compute.rs:680-925): y[r] = sum_k elem(W[r,k]) * x[k]
// over the whole blocks of each row, with the reference's element order
// (Q4_0/Q4_K: low nibble of byte j -> element 2j, high nibble -> 2j+1;
// Q6_K: low nibble of ql[i/2] by parity, 2-bit field (i%4) of qh[i/4]).
// Batch B > 1 is B independent matvecs sharing one pass over W
// (src/inference/batch_scheduler.rs:242-276 calls the matvec once per row).
//
// The batch-1 decode matvec is HBM-bound, so the design keeps the weight
// stream the only HBM traffic and the VALU work per weight byte minimal:
//  * x is staged once per workgroup in LDS, pre-scaled per format (odd
//    elements of the 4-bit formats by 1/16, so the high nibble can be
//    converted in place with v_cvt_f32_ubyteN on (w & 0xF0F0F0F0) without a
//    shift), with per-unit padding so 16 consecutive lanes read disjoint banks.
//    For B = 1 each lane then copies its units' x into registers once.
//  * Every lane owns fixed "units" of each row (a Q4_K sub-block, a pair of
//    Q4_0 / Q8_0 blocks, a 32-element quarter of a Q6_K block) and loads them
//    with dword-aligned 128-bit loads; a wave sweeps R rows at a time.
//  * Offsets and centres are folded out of the inner loop:
//    sum (S*q - M) x = S * sum q x - M * sum x, with sum x per sub-block
//    precomputed once per workgroup (Q8_0 codes are biased by +128 and
//    Q6_K codes by +32 the same way).
//  * Rows of unaligned matrices fall back to a byte-addressed kernel.
// Results agree with the reference to fp32 rounding (different summation
// order); the element values themselves are bit-exact in dequant.hip.
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"

namespace ssdq {
namespace {

// ------------------------------------------------------------ unit geometry
template <int F> struct FastUnit;
template <> struct FastUnit<kQ4_K> {
  static constexpr int E = 32, NSUM = 1, SUMG = 32, NW = 8;
  static constexpr bool prescale = true;
};
template <> struct FastUnit<kQ4_0> {
  static constexpr int E = 64, NSUM = 2, SUMG = 32, NW = 9;
  static constexpr bool prescale = true;
};
template <> struct FastUnit<kQ8_0> {
  static constexpr int E = 64, NSUM = 2, SUMG = 32, NW = 17;
  static constexpr bool prescale = false;
};
template <> struct FastUnit<kQ6_K> {
  static constexpr int E = 32, NSUM = 2, SUMG = 16, NW = 10;
  static constexpr bool prescale = false;
};

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x3a4 __attribute__((ext_vector_type(3), aligned(4)));

__device__ __forceinline__ void ld4(const uint8_t* p, uint32_t* d) {
  const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(p);
  d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
}
__device__ __forceinline__ void ld3(const uint8_t* p, uint32_t* d) {
  const u32x3a4 v = *reinterpret_cast<const u32x3a4*>(p);
  d[0] = v.x; d[1] = v.y; d[2] = v.z;
}
__device__ __forceinline__ uint32_t ld1(const uint8_t* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}
__device__ __forceinline__ uint32_t ldh(const uint8_t* p) {
  return *reinterpret_cast<const uint16_t*>(p);
}

// Loads unit u of one row into registers (all loads stay inside the row's
// blocks, or the immediately preceding block for the Q6_K realignment).
template <int F>
__device__ __forceinline__ void load_unit(const uint8_t* __restrict__ row, int u, uint32_t* raw) {
  if constexpr (F == kQ4_K) {
    const uint8_t* blk = row + (size_t)(u >> 3) * 144;
    ld4(blk, raw);                          // d, dmin, scales[12]
    ld4(blk + 16 + 16 * (u & 7), raw + 4);  // qs of sub-block u&7
  } else if constexpr (F == kQ4_0) {
    const uint8_t* p = row + (size_t)u * 36;  // two 18-byte blocks, dword aligned
    ld4(p, raw);
    ld4(p + 16, raw + 4);
    raw[8] = ld1(p + 32);
  } else if constexpr (F == kQ8_0) {
    const uint8_t* p = row + (size_t)u * 68;  // two 34-byte blocks, dword aligned
    ld4(p, raw);
    ld4(p + 16, raw + 4);
    ld4(p + 32, raw + 8);
    ld4(p + 48, raw + 12);
    raw[16] = ld1(p + 64);
  } else {  // kQ6_K: quarter q of block u>>3; blocks are 2-byte aligned
    const uint8_t* blk = row + (size_t)(u >> 3) * 210;
    const int q = u & 7;
    const uint32_t mis = (uint32_t)(uintptr_t)blk & 2u;  // 0 or 2
    ld4(blk + 16 * q - mis, raw);         // ql[16q .. 16q+16) (+ slack)
    raw[4] = ld1(blk + 16 * q - mis + 16);
    ld3(blk + 128 + 8 * q - mis, raw + 5);  // qh[8q .. 8q+8) (+ slack)
    raw[8] = ldh(blk + 192 + 2 * q) | (ldh(blk + 208) << 16);  // scales pair | d
    raw[9] = mis * 8u;                                        // realignment shift
  }
}

// Decodes one unit into per-element integer-valued floats (offsets folded
// out) and applies it to B activations.  xg(b, e): x' of element e of the unit,
// sg(b, g): sum of the raw x over sum-group g of the unit.
template <int F, int B, class XG, class SG>
__device__ __forceinline__ void accumulate(const uint32_t* raw, int u, XG xg, SG sg, float* acc) {
  constexpr int E = FastUnit<F>::E;
  float q[E];
  if constexpr (F == kQ4_K || F == kQ4_0) {
    uint32_t qd[E / 8];
    if constexpr (F == kQ4_K) {
#pragma unroll
      for (int k = 0; k < 4; k++) qd[k] = raw[4 + k];
    } else {
#pragma unroll
      for (int k = 0; k < 4; k++) qd[k] = __builtin_amdgcn_alignbit(raw[k + 1], raw[k], 16);
#pragma unroll
      for (int k = 0; k < 4; k++) qd[4 + k] = raw[5 + k];
    }
#pragma unroll
    for (int k = 0; k < E / 8; k++) {
      const uint32_t lo = qd[k] & 0x0F0F0F0Fu;
      const uint32_t hi = qd[k] & 0xF0F0F0F0u;  // 16 * nibble; x' of odd elements is x/16
#pragma unroll
      for (int i = 0; i < 4; i++) {
        q[8 * k + 2 * i] = (float)byte_of(lo, i);
        q[8 * k + 2 * i + 1] = (float)byte_of(hi, i);
      }
    }
  } else if constexpr (F == kQ8_0) {
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const uint32_t v = __builtin_amdgcn_alignbit(raw[c + 1], raw[c], 16) ^ 0x80808080u;
#pragma unroll
      for (int i = 0; i < 4; i++) q[4 * c + i] = (float)byte_of(v, i);  // code + 128
    }
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const uint32_t v = raw[9 + c] ^ 0x80808080u;
#pragma unroll
      for (int i = 0; i < 4; i++) q[32 + 4 * c + i] = (float)byte_of(v, i);
    }
  } else {  // kQ6_K
    const uint32_t sh = raw[9];
    uint32_t ql[4], qh[2];
#pragma unroll
    for (int k = 0; k < 4; k++) ql[k] = __builtin_amdgcn_alignbit(raw[k + 1], raw[k], sh);
#pragma unroll
    for (int j = 0; j < 2; j++) qh[j] = __builtin_amdgcn_alignbit(raw[6 + j], raw[5 + j], sh);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      // bytes [b0, b0, b1, b1] with b0/b1 = qh bytes 2k, 2k+1
      const uint32_t p =
          __builtin_amdgcn_perm(qh[k >> 1], qh[k >> 1], (k & 1) ? 0x03030202u : 0x01010000u);
      const uint32_t he = ((p << 4) & 0x00300030u) | (p & 0x30003000u);
      const uint32_t ho = ((p << 2) & 0x00300030u) | ((p >> 2) & 0x30003000u);
      const uint32_t ee = (ql[k] & 0x0F0F0F0Fu) | he;          // elements 8k+2i
      const uint32_t eo = ((ql[k] >> 4) & 0x0F0F0F0Fu) | ho;   // elements 8k+2i+1
#pragma unroll
      for (int i = 0; i < 4; i++) {
        q[8 * k + 2 * i] = (float)byte_of(ee, i);   // q + 32
        q[8 * k + 2 * i + 1] = (float)byte_of(eo, i);
      }
    }
  }

  // Per-unit scales
  float sA, oA, sB = 0.f, oB = 0.f;  // acc += sA*(pxA - oA*sumA) + sB*(pxB - oB*sumB)
  if constexpr (F == kQ4_K) {
    const float d = f16_to_f32(raw[0] & 0xFFFFu), dmin = f16_to_f32(raw[0] >> 16);
    uint32_t s, m;
    q4k_scale_min(raw[1], raw[2], raw[3], u & 7, s, m);
    sA = d * (float)s;
    oA = dmin * (float)m;  // used as acc += S*px - M*sum
  } else if constexpr (F == kQ4_0) {
    sA = f16_to_f32(raw[0] & 0xFFFFu);
    sB = f16_to_f32(raw[4] >> 16);
    oA = oB = 8.0f;
  } else if constexpr (F == kQ8_0) {
    sA = f16_to_f32(raw[0] & 0xFFFFu);
    sB = f16_to_f32(raw[8] >> 16);
    oA = oB = 128.0f;
  } else {
    const float d = f16_to_f32(raw[8] >> 16);
    sA = d * (float)(int8_t)(raw[8] & 0xFFu);
    sB = d * (float)(int8_t)((raw[8] >> 8) & 0xFFu);
    oA = oB = 32.0f;
  }

#pragma unroll
  for (int b = 0; b < B; b++) {
    if constexpr (F == kQ4_K) {
      float p0 = 0.f, p1 = 0.f;
#pragma unroll
      for (int e = 0; e < E; e += 2) {
        p0 = fmaf(q[e], xg(b, e), p0);
        p1 = fmaf(q[e + 1], xg(b, e + 1), p1);
      }
      acc[b] = fmaf(sA, p0 + p1, fmaf(-oA, sg(b, 0), acc[b]));
    } else {
      float pa = 0.f, pb = 0.f;
#pragma unroll
      for (int e = 0; e < E / 2; e++) pa = fmaf(q[e], xg(b, e), pa);
#pragma unroll
      for (int e = E / 2; e < E; e++) pb = fmaf(q[e], xg(b, e), pb);
      acc[b] = fmaf(sA, fmaf(-oA, sg(b, 0), pa), acc[b]);
      acc[b] = fmaf(sB, fmaf(-oB, sg(b, 1), pb), acc[b]);
    }
  }
}

template <int F>
__host__ __device__ constexpr size_t lds_floats(int U, int B) {
  return (size_t)B * U * (FastUnit<F>::E + 4) + (size_t)B * U * FastUnit<F>::NSUM;
}

// UPL > 0: B must be 1; each lane keeps x for its UPL units in registers.
// UPL == 0: x read from LDS per use (any B).
template <int F, int B, int R, int UPL>
__global__ __launch_bounds__(256) void mv_fast(const uint8_t* __restrict__ w,
                                               const float* __restrict__ x, float* __restrict__ y,
                                               int out_dim, int in_dim, int bpr,
                                               int rows_per_wg) {
  using FU = FastUnit<F>;
  constexpr int E = FU::E, NS = FU::NSUM, SG = FU::SUMG, ES = E + 4, NW = FU::NW;
  extern __shared__ float smem[];
  const int keff = bpr * Geom<F>::bs;
  const int U = keff / E;
  float* xs = smem;                      // [B][U][ES]
  float* xsum = smem + (size_t)B * U * ES;  // [B][U*NS]

  for (int i = threadIdx.x; i < B * keff; i += blockDim.x) {
    const int b = i / keff, e = i - b * keff;
    float v = x[(size_t)b * in_dim + e];
    const int u = e / E, t = e - u * E;
    if (FU::prescale && (t & 1)) v *= 0.0625f;
    xs[((size_t)b * U + u) * ES + t] = v;
  }
  for (int i = threadIdx.x; i < B * U * NS; i += blockDim.x) {
    const int b = i / (U * NS), g = i - b * (U * NS);
    const float* xp = x + (size_t)b * in_dim + (size_t)g * SG;
    float s = 0.f;
    for (int t = 0; t < SG; t++) s += xp[t];
    xsum[i] = s;
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const size_t row_bytes = (size_t)bpr * Geom<F>::bb;
  const int r_begin = blockIdx.x * rows_per_wg;
  const int r_end = min(out_dim, r_begin + rows_per_wg);

  if constexpr (UPL > 0) {
    static_assert(B == 1, "register-resident x needs B == 1");
    float xr[UPL][E];
    float sr[UPL][NS];
#pragma unroll
    for (int i = 0; i < UPL; i++) {
      const int u = lane + 64 * i;
      const bool ok = u < U;
#pragma unroll
      for (int t = 0; t < E; t++) xr[i][t] = ok ? xs[(size_t)u * ES + t] : 0.f;
#pragma unroll
      for (int g = 0; g < NS; g++) sr[i][g] = ok ? xsum[(size_t)u * NS + g] : 0.f;
    }
    for (int r0 = r_begin + wave * R; r0 < r_end; r0 += nwaves * R) {
      uint32_t raw[R][UPL][NW];
#pragma unroll
      for (int rr = 0; rr < R; rr++) {
        const int row = min(r0 + rr, r_end - 1);
        const uint8_t* rp = w + (size_t)row * row_bytes;
#pragma unroll
        for (int i = 0; i < UPL; i++) {
          const int u = lane + 64 * i;
          if (u < U) load_unit<F>(rp, u, raw[rr][i]);
        }
      }
      float acc[R];
#pragma unroll
      for (int rr = 0; rr < R; rr++) {
        acc[rr] = 0.f;
#pragma unroll
        for (int i = 0; i < UPL; i++) {
          const int u = lane + 64 * i;
          if (u < U)
            accumulate<F, 1>(
                raw[rr][i], u, [&](int, int e) { return xr[i][e]; },
                [&](int, int g) { return sr[i][g]; }, &acc[rr]);
        }
      }
#pragma unroll
      for (int rr = 0; rr < R; rr++) {
        const float s = wave_sum(acc[rr]);
        if (lane == 0 && r0 + rr < r_end) y[r0 + rr] = s;
      }
    }
  } else {
    for (int r0 = r_begin + wave * R; r0 < r_end; r0 += nwaves * R) {
      float acc[R][B];
#pragma unroll
      for (int rr = 0; rr < R; rr++)
#pragma unroll
        for (int b = 0; b < B; b++) acc[rr][b] = 0.f;
      for (int u = lane; u < U; u += 64) {
        uint32_t raw[R][NW];
#pragma unroll
        for (int rr = 0; rr < R; rr++) {
          const int row = min(r0 + rr, r_end - 1);
          load_unit<F>(w + (size_t)row * row_bytes, u, raw[rr]);
        }
        const float* xu = xs + (size_t)u * ES;
        const float* su = xsum + (size_t)u * NS;
#pragma unroll
        for (int rr = 0; rr < R; rr++)
          accumulate<F, B>(
              raw[rr], u,
              [&](int b, int e) { return xu[(size_t)b * U * ES + e]; },
              [&](int b, int g) { return su[(size_t)b * U * NS + g]; }, acc[rr]);
      }
#pragma unroll
      for (int rr = 0; rr < R; rr++)
#pragma unroll
        for (int b = 0; b < B; b++) {
          const float s = wave_sum(acc[rr][b]);
          if (lane == 0 && r0 + rr < r_end) y[(size_t)b * out_dim + r0 + rr] = s;
        }
    }
  }
}

// ------------------------------------------------ byte-addressed fallback
// One wave per row; lanes stride over 32-element groups (16 for Q6_K); any
// alignment of w, x read straight from global memory.
template <int F, int B>
__device__ __forceinline__ void generic_group(const uint8_t* __restrict__ row, int g,
                                              const float* __restrict__ x, int in_dim,
                                              float* acc) {
  if constexpr (F == kQ4_0 || F == kQ8_0) {
    const uint8_t* blk = row + (size_t)g * Geom<F>::bb;
    const float d = f16_to_f32(ld_u16(blk));
    const int x0 = g * 32;
#pragma unroll
    for (int b = 0; b < B; b++) {
      const float* xb = x + (size_t)b * in_dim + x0;
      float p = 0.f;
      if constexpr (F == kQ4_0) {
        for (int j = 0; j < 16; j++) {
          const uint32_t byte = blk[2 + j];
          p = fmaf((float)((int)(byte & 15u) - 8), xb[2 * j], p);
          p = fmaf((float)((int)(byte >> 4) - 8), xb[2 * j + 1], p);
        }
      } else {
        for (int j = 0; j < 32; j++) p = fmaf((float)(int8_t)blk[2 + j], xb[j], p);
      }
      acc[b] = fmaf(d, p, acc[b]);
    }
  } else if constexpr (F == kQ4_K) {
    const uint8_t* blk = row + (size_t)(g >> 3) * 144;
    const int sb = g & 7;
    const float d = f16_to_f32(ld_u16(blk)), dmin = f16_to_f32(ld_u16(blk + 2));
    const uint8_t* sc = blk + 4;
    uint32_t s, m;
    if (sb < 4) {
      s = sc[sb] & 63u;
      m = sc[sb + 4] & 63u;
    } else {
      s = ((uint32_t)sc[sb - 4] >> 6) | (((uint32_t)sc[sb + 4] & 15u) << 2);
      m = ((uint32_t)sc[sb] >> 6) | (((uint32_t)sc[sb + 4] >> 4) << 2);
    }
    const float S = d * (float)s, M = dmin * (float)m;
    const uint8_t* qs = blk + 16 + sb * 16;
#pragma unroll
    for (int b = 0; b < B; b++) {
      const float* xb = x + (size_t)b * in_dim + g * 32;
      float p = 0.f, sx = 0.f;
      for (int j = 0; j < 16; j++) {
        const uint32_t byte = qs[j];
        p = fmaf((float)(byte & 15u), xb[2 * j], p);
        p = fmaf((float)(byte >> 4), xb[2 * j + 1], p);
        sx += xb[2 * j] + xb[2 * j + 1];
      }
      acc[b] = fmaf(S, p, fmaf(-M, sx, acc[b]));
    }
  } else {  // kQ6_K, group of 16 elements
    const uint8_t* blk = row + (size_t)(g >> 4) * 210;
    const int gi = g & 15;
    const float d = f16_to_f32(ld_u16(blk + 208));
    const float sc = d * (float)(int8_t)blk[192 + gi];
#pragma unroll
    for (int b = 0; b < B; b++) {
      const float* xb = x + (size_t)b * in_dim + (size_t)(g >> 4) * 256;
      float p = 0.f;
      for (int t = 0; t < 16; t++) {
        const int idx = gi * 16 + t;
        const uint32_t qlb = blk[idx / 2];
        const uint32_t lo4 = (idx & 1) ? (qlb >> 4) : (qlb & 15u);
        const uint32_t hi2 = ((uint32_t)blk[128 + idx / 4] >> (2 * (idx % 4))) & 3u;
        p = fmaf((float)((int)(lo4 | (hi2 << 4)) - 32), xb[idx], p);
      }
      acc[b] = fmaf(sc, p, acc[b]);
    }
  }
}

template <int F, int B>
__global__ __launch_bounds__(256) void mv_generic(const uint8_t* __restrict__ w,
                                                  const float* __restrict__ x,
                                                  float* __restrict__ y, int out_dim, int in_dim,
                                                  int bpr) {
  const int lane = threadIdx.x & 63;
  const int groups = (F == kQ6_K) ? bpr * 16 : (F == kQ4_K ? bpr * 8 : bpr);
  const size_t row_bytes = (size_t)bpr * Geom<F>::bb;
  for (int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); row < out_dim;
       row += gridDim.x * (blockDim.x >> 6)) {
    float acc[B];
#pragma unroll
    for (int b = 0; b < B; b++) acc[b] = 0.f;
    const uint8_t* rp = w + (size_t)row * row_bytes;
    for (int g = lane; g < groups; g += 64) generic_group<F, B>(rp, g, x, in_dim, acc);
#pragma unroll
    for (int b = 0; b < B; b++) {
      const float s = wave_sum(acc[b]);
      if (lane == 0) y[(size_t)b * out_dim + row] = s;
    }
  }
}

// ------------------------------------------------------------------ host
int g_lds_limit = -1;

int lds_limit() {
  if (g_lds_limit < 0) {
    int dev = 0, v = 65536;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess)
      g_lds_limit = v;
    else
      g_lds_limit = 65536;
  }
  return g_lds_limit;
}

template <int F, int B>
hipError_t run_generic(const uint8_t* w, const float* x, float* y, int out_dim, int in_dim,
                       int bpr, hipStream_t s) {
  const int rows_per_block = 4;
  int grid = (out_dim + rows_per_block - 1) / rows_per_block;
  grid = std::min(grid, 65535);
  hipLaunchKernelGGL((mv_generic<F, B>), dim3(grid), dim3(256), 0, s, w, x, y, out_dim, in_dim,
                     bpr);
  return hipGetLastError();
}

template <int F>
hipError_t generic_dispatch(const uint8_t* w, const float* x, float* y, int out_dim, int in_dim,
                            int bpr, int batch, hipStream_t s) {
  // process the batch in chunks of 8 / 4 / 2 / 1 rows of x
  int b0 = 0;
  while (b0 < batch) {
    const int left = batch - b0;
    const float* xb = x + (size_t)b0 * in_dim;
    float* yb = y + (size_t)b0 * out_dim;
    hipError_t e;
    int take;
    if (left >= 8) { e = run_generic<F, 8>(w, xb, yb, out_dim, in_dim, bpr, s); take = 8; }
    else if (left >= 4) { e = run_generic<F, 4>(w, xb, yb, out_dim, in_dim, bpr, s); take = 4; }
    else if (left >= 2) { e = run_generic<F, 2>(w, xb, yb, out_dim, in_dim, bpr, s); take = 2; }
    else { e = run_generic<F, 1>(w, xb, yb, out_dim, in_dim, bpr, s); take = 1; }
    if (e != hipSuccess) return e;
    b0 += take;
  }
  return hipSuccess;
}

template <int F, int B, int R, int UPL>
hipError_t run_fast(const uint8_t* w, const float* x, float* y, int out_dim, int in_dim, int bpr,
                    size_t lds_bytes, hipStream_t s) {
  auto kern = mv_fast<F, B, R, UPL>;
  static bool attr_set = false;
  if (!attr_set && lds_bytes > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       lds_limit());
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int cus = device_cu_count();
  const int waves_per_wg = 4;
  // Enough workgroups to fill every CU twice; each takes a contiguous row range.
  const int rows_per_pass = waves_per_wg * R;
  int n_wg = std::max(1, std::min((out_dim + rows_per_pass - 1) / rows_per_pass, 2 * cus));
  int rows_per_wg = (out_dim + n_wg - 1) / n_wg;
  rows_per_wg = (rows_per_wg + rows_per_pass - 1) / rows_per_pass * rows_per_pass;
  n_wg = (out_dim + rows_per_wg - 1) / rows_per_wg;
  hipLaunchKernelGGL(kern, dim3(n_wg), dim3(64 * waves_per_wg), lds_bytes, s, w, x, y, out_dim,
                     in_dim, bpr, rows_per_wg);
  return hipGetLastError();
}

template <int F>
bool fast_aligned(const uint8_t* w, int bpr) {
  const uintptr_t a = (uintptr_t)w;
  if constexpr (F == kQ4_K) return (a & 15u) == 0;
  else return (a & 3u) == 0 && (bpr % 2) == 0;  // Q4_0 / Q8_0 pairs, Q6_K dword rows
}

template <int F>
hipError_t fast_dispatch(const uint8_t* w, const float* x, float* y, int out_dim, int in_dim,
                         int bpr, int batch, hipStream_t s, bool* used) {
  *used = false;
  if (!fast_aligned<F>(w, bpr)) return hipSuccess;
  const int keff = bpr * Geom<F>::bs;
  const int U = keff / FastUnit<F>::E;
  const int limit = lds_limit();
  if (batch == 1 && U <= 128) {
    const size_t lds = lds_floats<F>(U, 1) * 4;
    if (lds > (size_t)limit) return hipSuccess;
    *used = true;
    if (U <= 64) return run_fast<F, 1, 4, 1>(w, x, y, out_dim, in_dim, bpr, lds, s);
    return run_fast<F, 1, 4, 2>(w, x, y, out_dim, in_dim, bpr, lds, s);
  }
  // LDS-resident x; batch processed in chunks of 8/4/2/1 that each fit LDS
  int b0 = 0;
  while (b0 < batch) {
    const int left = batch - b0;
    int take = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
    while (take > 1 && lds_floats<F>(U, take) * 4 > (size_t)limit) take >>= 1;
    const size_t lds = lds_floats<F>(U, take) * 4;
    if (lds > (size_t)limit) return b0 == 0 ? hipSuccess : hipErrorInvalidValue;
    const float* xb = x + (size_t)b0 * in_dim;
    float* yb = y + (size_t)b0 * out_dim;
    hipError_t e;
    switch (take) {
      case 8: e = run_fast<F, 8, 2, 0>(w, xb, yb, out_dim, in_dim, bpr, lds, s); break;
      case 4: e = run_fast<F, 4, 2, 0>(w, xb, yb, out_dim, in_dim, bpr, lds, s); break;
      case 2: e = run_fast<F, 2, 2, 0>(w, xb, yb, out_dim, in_dim, bpr, lds, s); break;
      default: e = run_fast<F, 1, 4, 0>(w, xb, yb, out_dim, in_dim, bpr, lds, s); break;
    }
    if (e != hipSuccess) return e;
    *used = true;
    b0 += take;
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_matvec_generic(int dtype, const uint8_t* w, const float* x, float* y,
                                 size_t out_dim, size_t in_dim, size_t batch, hipStream_t s) {
  if (out_dim == 0 || batch == 0) return hipSuccess;
  switch (dtype) {
    case kQ4_0: return generic_dispatch<kQ4_0>(w, x, y, (int)out_dim, (int)in_dim, (int)(in_dim / 32), (int)batch, s);
    case kQ8_0: return generic_dispatch<kQ8_0>(w, x, y, (int)out_dim, (int)in_dim, (int)(in_dim / 32), (int)batch, s);
    case kQ4_K: return generic_dispatch<kQ4_K>(w, x, y, (int)out_dim, (int)in_dim, (int)(in_dim / 256), (int)batch, s);
    case kQ6_K: return generic_dispatch<kQ6_K>(w, x, y, (int)out_dim, (int)in_dim, (int)(in_dim / 256), (int)batch, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_matvec(int dtype, const uint8_t* w, const float* x, float* y, size_t out_dim,
                         size_t in_dim, size_t batch, hipStream_t s) {
  if (out_dim == 0 || batch == 0) return hipSuccess;
  bool used = false;
  hipError_t e = hipSuccess;
  const int od = (int)out_dim, id = (int)in_dim, b = (int)batch;
  switch (dtype) {
    case kQ4_0: e = fast_dispatch<kQ4_0>(w, x, y, od, id, id / 32, b, s, &used); break;
    case kQ8_0: e = fast_dispatch<kQ8_0>(w, x, y, od, id, id / 32, b, s, &used); break;
    case kQ4_K: e = fast_dispatch<kQ4_K>(w, x, y, od, id, id / 256, b, s, &used); break;
    case kQ6_K: e = fast_dispatch<kQ6_K>(w, x, y, od, id, id / 256, b, s, &used); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess || used) return e;
  return launch_matvec_generic(dtype, w, x, y, out_dim, in_dim, batch, s);
}

}  // namespace ssdq
