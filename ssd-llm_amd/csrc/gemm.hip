// Prefill GEMM: Y[M,N] f32 = X[M,K] bf16 x W[N,K]^T, W in Q4_K (reference layout).
//
// The reference has no GEMM: prefill runs one matvec per token
// (src/inference/transformer.rs:166-196 -> matvec_q4_k_cpu,
// src/metal/compute.rs:707-750), so Y[t,:] = matvec(W, widen_bf16(X[t,:])).
// The reference weight is w = fl(fl(S*q) - Mn) with S = fl(d*s), Mn =
// fl(dmin*m) (compute.rs:716-744): d, dmin fp16 per 256-element super-block,
// s, m 6-bit integers per 32-element sub-block, q a 4-bit code.  Here the
// product is taken in factored form on the matrix cores:
//   P[t,n] = sum over the super-block of X[t,k] * (s*q)[n,k]
//   Q[t,n] = sum over its 8 sub-blocks of XS[t,sb] * m[n,sb]
//   Y[t,n] = sum over super-blocks of d*P - dmin*Q            (fp32 FMAs)
// where XS is the sum of X over a sub-block.  Each (row, super-block) of X is
// first scaled by a power of two into fp16's range (undone on the fp32 result
// of that super-block), where bf16 values are exact unless they lie more than
// 2^26 below the super-block's largest magnitude; s*q is an integer <= 945,
// exact in fp16; so every product inside P is exact and
// v_mfma_f32_16x16x32_f16 only rounds the fp32 sums of one super-block (the
// accumulators restart at every super-block).  XS is carried as an fp16
// hi + lo pair (about 22 bits).  The result differs from the reference's serial
// fp32 chain by rounding only (measured: closer to the exact sum than the
// reference itself).  Rows whose range does not fit that window (or that hold
// NaN / infinity, or values beyond 65504) are recomputed in the reference's own
// fp32 order.
//
// A prep kernel writes X as fp16 in MFMA fragment order, plus XS: in a
// super-block, MFMA step t (32 k values) gives lane group c (lanes
// 16c .. 16c+15) the 8 values of sub-block 4*(t/4) + c at offset 8*(t%4), so
// one 16-byte load hands a lane the codes of a whole sub-block, and a 1 KB
// chunk of the prepared X is one A fragment.
// Tiling: a workgroup of 8 waves computes a 128 x 256 tile, one workgroup per
// CU; each wave owns 32 columns and all 128 rows, and builds its B fragments
// from the codes in registers.  K runs in stages of four MFMA steps; each
// stage's X fragments go straight from global memory into LDS (one 16-byte
// load per lane, issued a stage ahead into the other of two buffers), the
// weights of a stage are loaded into registers a stage ahead, and one wait
// plus one barrier per stage publishes both.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace ssdq {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
// native 16-byte vector (HIP's uint4 is a struct whose copies become memcpy
// calls that keep register arrays of it in memory)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int NT = 2;    // N sub-tiles (of 16 columns) per wave

__global__ __launch_bounds__(256) void widen_bf16_kernel(const uint16_t* __restrict__ x,
                                                         float* __restrict__ out, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = __uint_as_float((uint32_t)x[i] << 16);
}

// X prepared for the main kernel: fp16 in MFMA fragment order.  Chunk
// (m16, s) is 1 KB: lane 16 c + r holds the 8 values of row 16 m16 + r that
// K step s gives lane group c (sub-block 4 (t / 4) + c of super-block s / 8,
// at offset 8 (t % 4), t = s % 8).  Rows are padded to a multiple of 16 with
// copies of row M - 1.  Sub-block sums: chunk (m16, super-block) is 512 B:
// lane r holds the fp16 hi parts of row 16 m16 + r's 8 sums, lane 16 + r their
// lo parts.  One workgroup per (16 rows, super-block): each thread reads 8
// consecutive values of a row (coalesced), the tile is reordered in LDS, and
// the 8 chunks of the super-block, contiguous in xp, are written as one 8 KB
// run.
//
// Range: each (row, super-block) is scaled by a power of two 2^sh so that its
// largest magnitude lies in [2^9, 2^10); the sub-block sums then stay below
// 2^15 and every bf16 value at most 2^26 below that maximum is exact in fp16
// (bf16 has 8 significant bits, fp16 keeps them down to 2^-17).  xe holds
// 2^-sh per (m16, super-block, row), which the main kernel applies to the
// super-block's fp32 result.  A (row, super-block) whose values lose more than
// 2^-20 in total to the fp16 rounding (a range wider than the window), that
// holds a value beyond fp16's largest finite 65504 (whose products are too
// large for the fp32 partial sums to resolve the other terms to the
// tolerance: the reference's own serial chain misses the exact sum there), or
// that holds a NaN or an infinity, is flagged in fm (bit r of word (m16,
// super-block)); the main kernel recomputes flagged rows in the reference's
// order.
constexpr float kLossLimit = 0x1p-20f;

__global__ __launch_bounds__(512) void gemm_prep_x(const uint16_t* __restrict__ x, _Float16* __restrict__ xp,
                                                   _Float16* __restrict__ xsp, float* __restrict__ xe,
                                                   uint32_t* __restrict__ fm, int M, int K) {
  __shared__ h8 tile[512];
  __shared__ uint32_t flags[8];
  const int blk = blockIdx.x, m16 = blockIdx.y, nblk = K / 256;
  const int r = threadIdx.x >> 5, p = threadIdx.x & 31;  // row in the tile, 8-value piece of the super-block
  const int sb = p >> 2, q = p & 3;
  const uint4 v = *reinterpret_cast<const uint4*>(x + (size_t)min(16 * m16 + r, M - 1) * K + (size_t)blk * 256 + 8 * p);
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
  float a[8];
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    a[2 * i] = __uint_as_float(d[i] << 16);
    a[2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
  }
  bool bad = false;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    mx = fmaxf(mx, fabsf(a[i]));
    bad |= !(fabsf(a[i]) < INFINITY);
  }
  // the 32 threads of a row are one half of a wave
  mx = half_wave_max(mx);
  int e = 10;
  if (mx > 0.f && mx < INFINITY) (void)frexpf(mx, &e);  // mx < 2^e
  const int sh = 10 - e;
  h8 h;
  float sum = 0.f, lost = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float xs = ldexpf(a[i], sh);  // exact: a power of two, no overflow (|xs| < 2^10)
    const _Float16 hv = (_Float16)xs;
    h[((i & 3) << 1) | (i >> 2)] = hv;  // the element order of codes_times_s: 0, 4, 1, 5, 2, 6, 3, 7
    lost += fabsf(ldexpf(xs - (float)hv, -sh));  // the difference is exact in fp32
    sum += xs;
  }
  lost = half_wave_sum(lost);
  bad = half_wave_max(bad ? 1.f : 0.f) != 0.f;
  const bool flag = bad || mx > 65504.0f || !(lost <= kLossLimit);
  const int t = 4 * (sb >> 2) + q, c = sb & 3;
  tile[t * 64 + 16 * c + r] = h;
  // lanes 4i .. 4i+3 hold one sub-block; a + b is commutative, so all four
  // lanes end with the same sum
  sum += dpp_mov<0xB1>(sum);  // the pairings of shfl_xor 1, 2
  sum += dpp_mov<0x4E>(sum);
  const _Float16 hi = (_Float16)sum;
  const _Float16 lo = (_Float16)(sum - (float)hi);
  _Float16* o = xsp + ((size_t)m16 * nblk + blk) * 256;
  if (q == 0) o[r * 8 + sb] = hi;
  if (q == 1) o[(16 + r) * 8 + sb] = lo;
  const size_t chunk = (size_t)m16 * nblk + blk;
  if (p == 0) xe[chunk * 16 + r] = ldexpf(1.0f, -sh);
  // row flags of the tile: each wave holds two rows (lanes 0 and 32)
  const uint64_t fb = __ballot(flag);
  if ((threadIdx.x & 63) == 0)
    flags[threadIdx.x >> 6] = (uint32_t)(fb & 1u) | ((uint32_t)((fb >> 32) & 1u) << 1);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t m = 0;
#pragma unroll
    for (int w = 0; w < 8; w++) m |= flags[w] << (2 * w);
    fm[chunk] = m;
  }
  reinterpret_cast<h8*>(xp)[((size_t)m16 * (K / 32) + (size_t)blk * 8) * 64 + threadIdx.x] = tile[threadIdx.x];
}

// The scale constants of codes_times_s for one (column, sub-block) with
// 6-bit scale s: fp16 pairs (s, s), (-1024 s, -1024 s), (s/16, s/16) and
// (-64 s, -64 s), all exact.
struct SubScale {
  uint32_t s1, c1, s2, c2;
};
__device__ __forceinline__ SubScale sub_scale(uint32_t s) {
  // fp16 bits 0x6400 + s are 1024 + s exactly (s < 1024)
  const h2 sv = __builtin_bit_cast(h2, (s | (s << 16)) | 0x64006400u) - (h2){(_Float16)1024.f, (_Float16)1024.f};
  SubScale k;
  k.s1 = __builtin_bit_cast(uint32_t, sv);
  k.c1 = __builtin_bit_cast(uint32_t, sv * (h2){(_Float16)-1024.f, (_Float16)-1024.f});
  k.s2 = __builtin_bit_cast(uint32_t, sv * (h2){(_Float16)0.0625f, (_Float16)0.0625f});
  k.c2 = __builtin_bit_cast(uint32_t, sv * (h2){(_Float16)-64.f, (_Float16)-64.f});
  return k;
}

// One dword of codes (8 elements: byte i holds element 2i in its low nibble
// and 2i+1 in its high nibble) -> the 8 fp16 values s*q in the order
// 0, 4, 1, 5, 2, 6, 3, 7 (the prepared X uses the same order; the MFMA sums
// over k in any order).  Each fp16 pair is one mask-and-bias of the codes:
// bits 0x6400 + v are 1024 + v exactly for v < 1024, with v = q (low nibbles)
// or 16 q (high nibbles), and one fma takes it to s*q: s (1024 + q) - 1024 s
// and (s/16) (1024 + 16 q) - 64 s are exact before the fma's single rounding,
// and their value s*q <= 945 is an fp16 integer, so the result is exact.
// (a & m) | b in one instruction: VOP3 takes no literal here and one scalar
// operand, so the mask comes in a scalar register and the bias in a vector
// register (written with two literals, the compiler emits an and and an or).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t b) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(b));
  return r;
}

__device__ __forceinline__ h8 codes_times_s(uint32_t qd, const SubScale& k, uint32_t bias) {
  const uint32_t q8 = qd >> 8;
  const h2 b0 = __builtin_bit_cast(h2, and_or(qd, 0x000F000Fu, bias));  // elements 0, 4
  const h2 b1 = __builtin_bit_cast(h2, and_or(qd, 0x00F000F0u, bias));  // 1, 5 (16 q)
  const h2 b2 = __builtin_bit_cast(h2, and_or(q8, 0x000F000Fu, bias));  // 2, 6
  const h2 b3 = __builtin_bit_cast(h2, and_or(q8, 0x00F000F0u, bias));  // 3, 7 (16 q)
  const h2 s1 = __builtin_bit_cast(h2, k.s1), c1 = __builtin_bit_cast(h2, k.c1);
  const h2 s2 = __builtin_bit_cast(h2, k.s2), c2 = __builtin_bit_cast(h2, k.c2);
  const h2 r0 = __builtin_elementwise_fma(s1, b0, c1), r1 = __builtin_elementwise_fma(s2, b1, c2);
  const h2 r2 = __builtin_elementwise_fma(s1, b2, c1), r3 = __builtin_elementwise_fma(s2, b3, c2);
  return h8{r0.x, r0.y, r1.x, r1.y, r2.x, r2.y, r3.x, r3.y};
}

// 4 bytes (values < 1024) -> fp16 values: bytes 0, 1 -> r[0], bytes 2, 3 -> r[1]
__device__ __forceinline__ void bytes_to_f16(uint32_t b, uint32_t* r) {
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const uint32_t u = __builtin_amdgcn_perm(0u, b, (uint32_t)(2 * i) | 0x0C00u | ((uint32_t)(2 * i + 1) << 16) | 0x0C000000u);
    const h2 hv = __builtin_bit_cast(h2, u | 0x64006400u) - (h2){(_Float16)1024.f, (_Float16)1024.f};
    r[i] = __builtin_bit_cast(uint32_t, hv);
  }
}

// One 16-byte load per lane straight into LDS: lane l writes bytes
// [16 l, 16 l + 16) above the wave-uniform LDS offset lds.  Written as inline
// assembly so that the compiler, which cannot tell which LDS buffer such a load
// fills, does not wait for it before every LDS read; the kernel waits for its
// own loads (vmcnt(0)) before the barrier that publishes a stage.  One wait
// state (s_nop) separates the M0 write from the LDS-DMA load that reads M0.  M0
// is restored.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  uint32_t keep;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
               : "=&s"(keep)
               : "s"(lds), "v"(g)
               : "memory");
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// This wave's LDS loads have landed, and so have all of its register loads
// except the N issued last (the weights of the stage after next, requested
// after the stage's LDS loads); then every wave's have.  The scheduling
// barriers keep the next stage's work (which consumes registers loaded
// earlier) from being hoisted above the wait: the compiler does not count the
// inline-assembly loads, so an early wait it placed for a register load could
// also drain the next stage's LDS loads.
template <int N>
__device__ __forceinline__ void publish_stage() {
  static_assert(N >= 0 && N < 16, "vmcnt range");
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(N | (7 << 4) | (15 << 8));  // vmcnt(N)
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  __builtin_amdgcn_sched_barrier(0);
}

// Up to three Q4_K matrices with the same K that share X, as one GEMM over
// their concatenated columns: matrix i has columns start_i .. start_{i+1} - 1
// (start_0 = 0, start_3 = N; absent matrices have start = N).  The kernels take
// the fields as separate scalar arguments: inside one aggregate, the selects
// below fold into a run-time index, which puts the arguments in private
// memory.
struct GemmMats {
  const uint8_t* w0;
  const uint8_t* w1;
  const uint8_t* w2;
  float* y0;
  float* y1;
  float* y2;
  int start1, start2;
};
#define GEMM_MATS_PARAMS                                                                            \
  const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, const uint8_t *__restrict__ w2, \
      float *__restrict__ y0, float *__restrict__ y1, float *__restrict__ y2, int start1, int start2
#define GEMM_MATS_ARGS(m) m.w0, m.w1, m.w2, m.y0, m.y1, m.y2, m.start1, m.start2
// column c (< N) -> matrix, its first column, its weights and output
#define GEMM_SEGMENT(c) (MULTI ? ((c) >= start1) + ((c) >= start2) : 0)
#define GEMM_FIRST(sg) ((sg) == 0 ? 0 : (sg) == 1 ? start1 : (sg) == 2 ? start2 : N)
#define GEMM_WEIGHTS(sg) ((sg) == 0 ? w0 : (sg) == 1 ? w1 : w2)
#define GEMM_OUT(sg) ((sg) == 0 ? y0 : (sg) == 1 ? y1 : y2)

// Exact recomputation of one flagged row (see gemm_prep_x): every column of
// the workgroup's tile gets the reference's serial fp32 sum over the super-blocks
// b_begin .. b_end - 1 (all of K, or none: 0), in the order of
// matvec_q4_k_cpu (compute.rs:707-750, elements of bf16 X widened as
// streamer.rs:108-114 does): one thread per column, pairs of products added
// before the running sum, no contraction.  The row's bf16 values pass through
// LDS one super-block at a time (xs, 256 floats).  The result is the oracle's
// bit for bit.
template <bool MULTI>
__device__ __noinline__ void gemm_exact_row(GEMM_MATS_PARAMS, const uint16_t* __restrict__ xraw,
                                            float* __restrict__ part, float* xs, int row, int n0, int BN, int N,
                                            int K, int M, int b_begin, int b_end, int nz) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x;
  const int n = n0 + tid;
  const bool col = tid < BN && n < N;
  const int sg = col ? GEMM_SEGMENT(n) : 0;
  const size_t row_bytes = (size_t)(K / 256) * 144;
  const uint8_t* wr = col ? GEMM_WEIGHTS(sg) + (size_t)(n - GEMM_FIRST(sg)) * row_bytes : nullptr;
  float sum = 0.0f;
  for (int b = b_begin; b < b_end; b++) {
    __syncthreads();
    if (tid < 256) xs[tid] = __uint_as_float((uint32_t)xraw[(size_t)row * K + (size_t)b * 256 + tid] << 16);
    __syncthreads();
    if (col) {
      const uint8_t* blk = wr + (size_t)b * 144;
      const float d = f16_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
      const float dmin = f16_to_f32((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
      const uint8_t* sc = blk + 4;
      const uint8_t* qs = blk + 16;
      for (int sb = 0; sb < 8; sb++) {
        uint32_t sv, mv;
        if (sb < 4) {
          sv = sc[sb] & 63u;
          mv = sc[sb + 4] & 63u;
        } else {
          sv = (uint32_t)(sc[sb - 4] >> 6) | ((uint32_t)(sc[sb + 4] & 15) << 2);
          mv = (uint32_t)(sc[sb] >> 6) | ((uint32_t)(sc[sb + 4] >> 4) << 2);
        }
        const float scale = d * (float)sv;
        const float mn = dmin * (float)mv;
        for (int j = 0; j < 16; j++) {
          const uint32_t bv = qs[sb * 16 + j];
          const float v0 = scale * (float)(bv & 15u) - mn;
          const float v1 = scale * (float)(bv >> 4) - mn;
          const float p0 = v0 * xs[sb * 32 + 2 * j];
          const float p1 = v1 * xs[sb * 32 + 2 * j + 1];
          sum = sum + (p0 + p1);
        }
      }
    }
  }
  if (col && row < M) {
    if (nz > 1)
      part[(size_t)row * N + n] = sum;
    else
      GEMM_OUT(sg)[(size_t)row * (GEMM_FIRST(sg + 1) - GEMM_FIRST(sg)) + (n - GEMM_FIRST(sg))] = sum;
  }
}

// Workgroup tile (16 MT) x (32 WAVES): each wave owns 32 columns and all
// 16 MT rows.  K runs in stages of 4 MFMA steps (half a super-block); the X
// chunks of a stage (MT per step), the sub-block sums and the row scales of a
// super-block are loaded straight into LDS one stage ahead, double-buffered,
// and the weights of a stage are loaded into registers one stage ahead, so one
// wait and one barrier per stage cover every load.  The N columns are those of
// up to three matrices that share X, concatenated (GemmMats).  blockIdx.z
// selects split z of the K range (split = gridDim.z); with one split the
// results go to the matrices' own outputs, otherwise split z writes its partial
// product of the concatenated columns to part + z * M * N.  Rows that the prep
// kernel flagged (range wider than the fp16 window, or non-finite values) are
// not stored from the matrix cores but recomputed by gemm_exact_row.
template <int MT, int WAVES, bool MULTI>
__global__ __launch_bounds__(64 * WAVES, 8 / WAVES) void gemm_q4k_mfma(GEMM_MATS_PARAMS,
                                                        const _Float16* __restrict__ xp,
                                                        const _Float16* __restrict__ xsp,
                                                        const float* __restrict__ xe,
                                                        const uint32_t* __restrict__ fm,
                                                        const uint16_t* __restrict__ xraw,
                                                        float* __restrict__ part, int M, int N, int K) {
  static_assert(MT == 8 && WAVES == 8, "the waves move the 8 X chunks of a step evenly, wave 4 the row scales");
  constexpr int BM = 16 * MT, BN = 32 * WAVES;
  constexpr int XPW = MT / WAVES;  // X chunks each wave moves per step
  constexpr int CH = MT * 64;  // h8 slots of one step's X in LDS
  __shared__ __align__(16) h8 xa[4 * CH];  // stages 2b (first half of a super-block)
  __shared__ __align__(16) h8 xb[4 * CH];  // stages 2b + 1
  __shared__ __align__(16) h8 xsl[2][MT / 2 * 64];
  __shared__ __align__(16) f4 xel[2][64];  // row scales 2^-sh of a super-block: [mt][16 rows] (first 512 B)
  __shared__ uint32_t rowflags[MT];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int c = lane >> 4;  // lane group: k = 8c .. 8c+7 of each step
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int nblk = K / 256, S = K / 32, z = blockIdx.z, nz = gridDim.z;
  const int b_begin = (int)((long)nblk * z / nz), b_end = (int)((long)nblk * (z + 1) / nz);
  const int nb = b_end - b_begin, last_step = 8 * nb - 1;
  part += (size_t)z * M * N;
  const size_t row_bytes = (size_t)nblk * 144;
  const int m16 = m0 >> 4, M16 = (M + 15) >> 4;

  // flag words of this wave's row tile (m16 + wave) over all super-blocks of
  // K (every split must agree on the flagged rows), requested first and
  // reduced after the main loop
  const size_t fbase = (size_t)min(m16 + wave, M16 - 1) * nblk;
  uint32_t fw0 = fm[fbase + min(lane, nblk - 1)], fw1 = fm[fbase + min(lane + 64, nblk - 1)];

  // weight rows of this lane's B fragments (clamped; columns past N are not stored)
  const uint8_t* wrow[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) {
    const int n = min(n0 + 32 * wave + 16 * j + (lane & 15), N - 1);
    const int sg = GEMM_SEGMENT(n);
    wrow[j] = GEMM_WEIGHTS(sg) + (size_t)(n - GEMM_FIRST(sg)) * row_bytes;
  }
  // this wave moves X chunks XPW wave .. XPW wave + XPW - 1 of every step
  // (row tiles past the padded M are clamped: their rows are never stored);
  // waves 0-3 move the sum chunks of a super-block, wave w chunks 2 w (lanes
  // 0-31) and 2 w + 1 (lanes 32-63); wave 4 moves the row scales (lane l:
  // tile (l / 4) % 8, rows 4 (l % 4) .. +3; lanes 32-63 repeat lanes 0-31 into
  // the unused second half of the buffer)
  const _Float16* xsrc[XPW];
#pragma unroll
  for (int i = 0; i < XPW; i++) xsrc[i] = xp + (size_t)min(m16 + XPW * wave + i, M16 - 1) * S * 512 + lane * 8;
  const _Float16* ssrc = xsp + (size_t)min(m16 + 2 * (wave & 3) + (lane >> 5), M16 - 1) * nblk * 256 + (lane & 31) * 8;
  const float* esrc = xe + (size_t)min(m16 + ((lane >> 2) & 7), M16 - 1) * nblk * 16 + (lane & 3) * 4;
  const uint32_t lds_a = lds_offset(xa) + wave * XPW * 1024, lds_b = lds_offset(xb) + wave * XPW * 1024;
  auto stage_x = [&](int g, uint32_t base) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const size_t s = (size_t)(8 * b_begin + min(4 * g + t, last_step)) * 512;
#pragma unroll
      for (int i = 0; i < XPW; i++) dma16(xsrc[i] + s, base + t * 8192 + i * 1024);
    }
  };
  auto stage_sums = [&](int b) {
    const int bb = b_begin + min(b, nb - 1);
    if (wave < 4)
      dma16(ssrc + (size_t)bb * 256, lds_offset(&xsl[b & 1][0]) + wave * 1024);
    else if (wave == 4)
      dma16(esrc + (size_t)bb * 16, lds_offset(&xel[b & 1][0]));
  };

  // Weights of super-block b, two stages ahead: the header (d|dmin, scale
  // bytes 0-3, 4-7, 8-11) and the 16 code bytes of sub-block c (steps 0-3,
  // two loads per column) are requested during the first stage of super-block
  // b - 1; the code bytes of sub-block 4 + c (steps 4-7, one load per column)
  // during its second stage.  Each stage requests its weights after its X and
  // sums copies, so the stage's wait leaves exactly those weight loads in
  // flight.  (With the weights one stage ahead the fused gate / up GEMM spent
  // a quarter of its time waiting for them: 166.6 us against 123.7 us for a
  // timing copy that loads no weights.)
  using WRegs = u32x4a4[NT];
  struct WSet {
    WRegs hdr, cd0, cd1;
  };
  WSet wa, wb;  // ping-pong: super-block b computes from one set and loads b + 1 into the other
  // fetch_first issues exactly two 16-byte loads per column (2 NT) and
  // fetch_second one (NT): the stage waits publish_stage<NT> and <2 NT> below
  // count them, so a change here must change those waits
  auto wptr = [&](int j, int b) { return wrow[j] + (size_t)(b_begin + min(b, nb - 1)) * 144; };
  auto fetch_first = [&](int b, WSet& w) {
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const uint8_t* p = wptr(j, b);
      w.hdr[j] = *reinterpret_cast<const u32x4a4*>(p);
      w.cd0[j] = *reinterpret_cast<const u32x4a4*>(p + 16 + 16 * c);
    }
  };
  auto fetch_second = [&](int b, WSet& w) {
#pragma unroll
    for (int j = 0; j < NT; j++) w.cd1[j] = *reinterpret_cast<const u32x4a4*>(wptr(j, b) + 16 + 16 * (4 + c));
  };

  f4 acc[MT][NT], tot[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) tot[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const uint32_t bias = opaque(0x64006400u);  // fp16 pair (1024, 1024), kept in a register
  // One MFMA step t (0-7) of a super-block, X from LDS stage buffer xs
  auto step = [&](auto t_c, const h8* xs, const SubScale (&s2)[NT][2], const u32x4a4 (&cd)[NT]) {
    constexpr int t = decltype(t_c)::value;
    h8 bf[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const uint32_t qd = (t & 3) == 0 ? cd[j].x : (t & 3) == 1 ? cd[j].y : (t & 3) == 2 ? cd[j].z : cd[j].w;
      bf[j] = codes_times_s(qd, s2[j][t >> 2], bias);
    }
#pragma unroll
    for (int m4 = 0; m4 < MT; m4 += 4) {
      h8 a[4];
#pragma unroll
      for (int u = 0; u < 4; u++) a[u] = xs[((t & 3) * MT + m4 + u) * 64 + lane];
#pragma unroll
      for (int u = 0; u < 4; u++)
#pragma unroll
        for (int j = 0; j < NT; j++)
          acc[m4 + u][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              a[u], bf[j], t == 0 ? f4{0.f, 0.f, 0.f, 0.f} : acc[m4 + u][j], 0, 0, 0);
    }
  };

  // One super-block: steps 0-7 from the weights in cur, requesting the next
  // super-block's into nxt.
  auto superblock = [&](int b, WSet& cur, WSet& nxt) {
    // ---- first stage of super-block b (steps 0-3, buffer xa); the code
    // bytes of its second stage may still be in flight
    publish_stage<NT>();
    stage_x(2 * b + 1, lds_b);
    // this super-block's scales (reference unpacking, compute.rs:724-735):
    // s[0..3] = sc[0..3] & 63, s[4..7] = sc[0..3] >> 6 | (sc[8..11] & 15) << 2,
    // m[0..3] = sc[4..7] & 63, m[4..7] = sc[4..7] >> 6 | (sc[8..11] >> 4) << 2
    SubScale s2[NT][2];
    uint32_t mlo[NT], mhi[NT], dbits[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const u32x4a4 hdr = cur.hdr[j];
      const uint32_t h1 = hdr.y, h2v = hdr.z, h3 = hdr.w;
      const uint32_t slo = h1 & 0x3F3F3F3Fu;
      const uint32_t shi = ((h1 >> 6) & 0x03030303u) | ((h3 & 0x0F0F0F0Fu) << 2);
      mlo[j] = h2v & 0x3F3F3F3Fu;
      mhi[j] = ((h2v >> 6) & 0x03030303u) | (((h3 >> 4) & 0x0F0F0F0Fu) << 2);
      const uint32_t sa = (slo >> (8 * c)) & 0xFFu, sb = (shi >> (8 * c)) & 0xFFu;
      s2[j][0] = sub_scale(sa);
      s2[j][1] = sub_scale(sb);
      dbits[j] = hdr.x;
    }
    fetch_first(b + 1, nxt);
    __builtin_amdgcn_sched_barrier(0);  // requested here, not sunk towards the next stage
    step(std::integral_constant<int, 0>{}, xa, s2, cur.cd0);
    step(std::integral_constant<int, 1>{}, xa, s2, cur.cd0);
    step(std::integral_constant<int, 2>{}, xa, s2, cur.cd0);
    step(std::integral_constant<int, 3>{}, xa, s2, cur.cd0);
    // ---- second stage (steps 4-7, buffer xb); the first stage's weights of
    // super-block b + 1 may still be in flight
    publish_stage<2 * NT>();
    stage_x(2 * b + 2, lds_a);
    stage_sums(b + 1);
    fetch_second(b + 1, nxt);
    __builtin_amdgcn_sched_barrier(0);
    step(std::integral_constant<int, 4>{}, xb, s2, cur.cd1);
    step(std::integral_constant<int, 5>{}, xb, s2, cur.cd1);
    step(std::integral_constant<int, 6>{}, xb, s2, cur.cd1);
    step(std::integral_constant<int, 7>{}, xb, s2, cur.cd1);
    // Min term on the matrix cores, added to d*P by the MFMA itself:
    //   v = d*P + sum over the 8 sub-blocks of XS * (-dmin*m),
    // with A = XS hi (lanes 0-15) / lo (16-31) / hi, lo again (32-63) and B =
    // the hi part of D = -dmin*m in lanes 0-31, its lo part in lanes 32-63, so
    // the four products hi*hi, lo*hi, hi*lo, lo*lo fill the 32 k lanes.  D is
    // exactly hi + lo in fp16: the product of an fp16 dmin and a 6-bit m has at
    // most 17 significant bits, none below 2^-24, so the fma's remainder lo is
    // exact, while |D| < 65504, that is |dmin| < 1024.  A column with a larger
    // finite dmin (never seen in real weights) has D and d*P scaled by 2^-10
    // (dmin >= 1024 keeps every bit of D at or above 2^-10, and |D| 2^-10 <
    // 4096), and its running totals are scaled by 2^-10 before the update and
    // by 2^10 after it: exact powers of two, so the update rounds as it would
    // unscaled.  A row's XS are finite unless the row is flagged, and a
    // flagged row's MFMA results are never stored.
    h8 bmin[NT];
    float ds[NT];
    bool wj[NT], wide = false;
#pragma unroll
    for (int j = 0; j < NT; j++) {
      uint32_t mv[4];
      bytes_to_f16(mlo[j], mv);
      bytes_to_f16(mhi[j], mv + 2);
      const uint32_t dmb = dbits[j] >> 16;
      wj[j] = (dmb & 0x7FFFu) >= 0x6400u && (dmb & 0x7C00u) != 0x7C00u;
      wide |= wj[j];
      // -dmin, times 2^-10 for a wide column (its exponent field is >= 25)
      const h2 nd = __builtin_bit_cast(h2, ((wj[j] ? dmb - 0x2800u : dmb) ^ 0x8000u) * 0x10001u);
      uint32_t dv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const h2 m2 = __builtin_bit_cast(h2, mv[i]);
        const h2 hi = m2 * nd;
        const h2 lo = __builtin_elementwise_fma(m2, nd, -hi);
        dv[i] = __builtin_bit_cast(uint32_t, lane < 32 ? hi : lo);
      }
      bmin[j] = __builtin_bit_cast(h8, u32x4{dv[0], dv[1], dv[2], dv[3]});
      // opaque: kept as f32 values, not folded into v_fma_mix_f32 (slower here)
      const float d = __uint_as_float(opaque(__float_as_uint(f16_to_f32(dbits[j] & 0xFFFFu))));
      ds[j] = wj[j] ? d * 0x1p-10f : d;
    }
    const bool any_wide = __builtin_amdgcn_ballot_w64(wide) != 0;
    if (any_wide) {
#pragma unroll
      for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
          for (int i = 0; i < 4; i++) tot[mt][j][i] *= wj[j] ? 0x1p-10f : 1.0f;
    }
    const h8* sums = &xsl[b & 1][0];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      const h8 amin = sums[(mt >> 1) * 64 + (mt & 1) * 32 + (lane & 31)];
      const f4 rs = xel[b & 1][mt * 4 + c];  // 2^-sh of rows 4c .. 4c+3
#pragma unroll
      for (int j = 0; j < NT; j++) {
        f4 dp;
#pragma unroll
        for (int i = 0; i < 4; i++) dp[i] = ds[j] * acc[mt][j][i];
        const f4 v = __builtin_amdgcn_mfma_f32_16x16x32_f16(amin, bmin[j], dp, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) tot[mt][j][i] = __builtin_fmaf(v[i], rs[i], tot[mt][j][i]);
      }
    }
    if (any_wide) {
#pragma unroll
      for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
          for (int i = 0; i < 4; i++) tot[mt][j][i] *= wj[j] ? 1024.0f : 1.0f;
    }
  };
  stage_x(0, lds_a);
  stage_sums(0);
  fetch_first(0, wa);
  fetch_second(0, wa);
  // two super-blocks per iteration, so that no weight register is carried
  // (copied) across the loop's back edge: such a copy waits for its load
  int b = 0;
  for (; b + 1 < nb; b += 2) {
    superblock(b, wa, wb);
    superblock(b + 1, wb, wa);
  }
  if (b < nb) superblock(b, wa, wb);
  // the last stage's loads (clamped repeats) land before the workgroup's LDS is released
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));

  // flagged rows of this wave's tile (words past the first 128 super-blocks
  // are read here)
  {
    uint32_t f = (lane < nblk ? fw0 : 0u) | (lane + 64 < nblk ? fw1 : 0u);
    for (int l = lane + 128; l < nblk; l += 64) f |= fm[fbase + l];
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) f |= __shfl_xor(f, o, 64);
    if (lane == 0) rowflags[wave] = m16 + wave < M16 ? f : 0u;
  }
  __syncthreads();

  // C fragment layout: element i of acc[mt][j] is row 4*(lane/16)+i, column lane%16
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const uint32_t rf = rowflags[mt];
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const int n = n0 + 32 * wave + 16 * j + (lane & 15);
      if (n >= N) continue;
      const int sg = GEMM_SEGMENT(n);
      const int ncols = GEMM_FIRST(sg + 1) - GEMM_FIRST(sg);
      float* dst = nz > 1 ? part + n : GEMM_OUT(sg) + (n - GEMM_FIRST(sg));
      const int ld = nz > 1 ? N : ncols;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int m = m0 + mt * 16 + 4 * c + i;
        if (m < M && !((rf >> (4 * c + i)) & 1u)) dst[(size_t)m * ld] = tot[mt][j][i];
      }
    }
  }
  // exact path for flagged rows (uniform over the workgroup: the flags are in
  // LDS).  Split 0 computes the whole K range in the reference's order and the
  // other splits contribute exact zeros, so the split-K sum is that serial
  // chain itself.
  const int exact_end = z == 0 ? nblk : 0;
  for (int mt = 0; mt < MT; mt++) {
    uint32_t rf = rowflags[mt];
    while (rf) {
      const int r = __builtin_ctz(rf);
      rf &= rf - 1;
      if (m0 + 16 * mt + r >= M) break;  // padding rows (copies of row M - 1) and beyond
      gemm_exact_row<MULTI>(w0, w1, w2, y0, y1, y2, start1, start2, xraw, part,
                            reinterpret_cast<float*>(xa), m0 + 16 * mt + r, n0, BN, N, K, M, 0, exact_end, nz);
    }
  }
}

// Sums split-K partials (M x N, concatenated columns) in a fixed order
// (deterministic results) into the matrices' outputs.  The split count is a
// template parameter so that every partial's load issues before the first add;
// the kernel is bound by HBM either way (split 4 of a 512 x 4096 output moves
// 40 MB in about 7.5 us).
template <bool MULTI, int S>
__global__ __launch_bounds__(256) void splitk_reduce(const float* __restrict__ part, GEMM_MATS_PARAMS, int M,
                                                     int N) {
  const int mn = M * N;
  const int stride = gridDim.x * blockDim.x;
  if (!MULTI && (mn & 3) == 0 && ((uintptr_t)y0 & 15) == 0) {  // one matrix: 16-byte loads and stores
    const int mn4 = mn >> 2;
    const float4* p4 = reinterpret_cast<const float4*>(part);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < mn4; i += stride) {
      float4 v[S];
#pragma unroll
      for (int z = 0; z < S; z++) v[z] = p4[(size_t)z * mn4 + i];
      float4 t = v[0];
#pragma unroll
      for (int z = 1; z < S; z++) {
        t.x += v[z].x;
        t.y += v[z].y;
        t.z += v[z].z;
        t.w += v[z].w;
      }
      reinterpret_cast<float4*>(y0)[i] = t;
    }
    return;
  }
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < mn; i += stride) {
    float v[S];
#pragma unroll
    for (int z = 0; z < S; z++) v[z] = part[(size_t)z * mn + i];
    float t = v[0];
#pragma unroll
    for (int z = 1; z < S; z++) t += v[z];
    if (!MULTI) {
      y0[i] = t;
      continue;
    }
    const int m = i / N, n = i - m * N;
    const int sg = GEMM_SEGMENT(n);
    GEMM_OUT(sg)[(size_t)m * (GEMM_FIRST(sg + 1) - GEMM_FIRST(sg)) + (n - GEMM_FIRST(sg))] = t;
  }
}

#undef GEMM_SEGMENT
#undef GEMM_FIRST
#undef GEMM_WEIGHTS
#undef GEMM_OUT
#undef GEMM_MATS_PARAMS

}  // namespace

bool gemm_q4k_mfma_ok(const void* w, const void* x) {
  return ((uintptr_t)w & 3) == 0 && ((uintptr_t)x & 15) == 0;
}

namespace {

// Workgroup tiles are 128 (M) x 256 (N): eight waves, each 128 rows x 32
// columns, one workgroup per CU.  Sharing each X tile among 256 columns halves
// the X traffic from L2 of 128-column tiles (measured slightly faster than
// those at two workgroups per CU).
constexpr int kMT = 8, kWaves = 8, kBN = 32 * kWaves;

// K splits for a GEMM: none while the tiles fill at least half of the
// workgroup slots (8 / kWaves per CU), since a split costs a partial product
// per split written and summed again; below that, as many as still fit one
// round of slots (at most 8, at most one per 256-element block).
int gemm_split(size_t M, size_t N, size_t K) {
  const size_t bm = 16 * (size_t)kMT;
  const size_t tiles = ((N + kBN - 1) / kBN) * ((M + bm - 1) / bm);
  const size_t slots = (size_t)(8 / kWaves) * (size_t)device_cu_count();
  if (2 * tiles >= slots) return 1;
  const size_t split = std::min<size_t>(std::min<size_t>(slots / tiles, 8), K / 256);
  return (int)std::max<size_t>(split, 1);
}

// workspace layout: X in fragment order (M16*K fp16, M16 = M rounded up to
// 16) | sub-block sums (M16*K/256*16 fp16) | row scales (M16*K/256 f32) |
// row-flag words (M16/16*K/256 u32, padded to 16 bytes) | split partials
// (split*M*N f32)
size_t prep_xe_offset(size_t M, size_t K) {
  const size_t M16 = (M + 15) / 16 * 16;
  return M16 * K * 2 + M16 * (K / 256) * 32;
}
size_t prep_fm_offset(size_t M, size_t K) {
  const size_t M16 = (M + 15) / 16 * 16;
  return prep_xe_offset(M, K) + M16 * (K / 256) * 4;
}
size_t prep_bytes(size_t M, size_t K) {
  const size_t M16 = (M + 15) / 16 * 16;
  return prep_fm_offset(M, K) + ((M16 / 16) * (K / 256) * 4 + 15) / 16 * 16;
}

}  // namespace

size_t gemm_q4k_workspace_bytes(const void* const* w, const size_t* n, int count, const void* x, size_t M,
                                size_t K) {
  size_t N = 0;
  bool aligned = ((uintptr_t)x & 15) == 0;
  for (int i = 0; i < count; i++) {
    N += n[i];
    aligned = aligned && gemm_q4k_mfma_ok(w[i], x);
  }
  if (!aligned) return M * K * sizeof(float);
  const int split = gemm_split(M, N, K);
  return prep_bytes(M, K) + (split > 1 ? (size_t)split * M * N * sizeof(float) : 0);
}

hipError_t launch_gemm_q4k(const uint8_t* const* w, const size_t* n, int count, const uint16_t* x,
                           float* const* y, size_t M, size_t K, void* workspace, size_t workspace_bytes,
                           hipStream_t s) {
  if (count < 1 || count > 3) return hipErrorInvalidValue;
  if (K % 256 != 0) return hipErrorInvalidValue;
  size_t N = 0;
  bool aligned = ((uintptr_t)x & 15) == 0;
  const uint8_t* wv[3];
  float* yv[3];
  int st[3];
  for (int i = 0; i < 3; i++) {
    const int j = i < count ? i : count - 1;
    wv[i] = w[j];
    yv[i] = y[j];
    st[i] = (int)N;
    if (i < count) {
      N += n[i];
      aligned = aligned && gemm_q4k_mfma_ok(w[i], x);
    }
  }
  for (int i = count; i < 3; i++) st[i] = (int)N;
  const GemmMats mats{wv[0], wv[1], wv[2], yv[0], yv[1], yv[2], st[1], st[2]};
  if (M == 0 || N == 0) return hipSuccess;
  if (aligned) {
    const int split = gemm_split(M, N, K);
    const size_t need = prep_bytes(M, K) + (split > 1 ? (size_t)split * M * N * sizeof(float) : 0);
    if (workspace_bytes < need) return hipErrorInvalidValue;
    uint8_t* wsb = static_cast<uint8_t*>(workspace);
    _Float16* xp = reinterpret_cast<_Float16*>(wsb);
    _Float16* xsp = xp + (M + 15) / 16 * 16 * K;
    float* xe = reinterpret_cast<float*>(wsb + prep_xe_offset(M, K));
    uint32_t* fm = reinterpret_cast<uint32_t*>(wsb + prep_fm_offset(M, K));
    float* part = reinterpret_cast<float*>(wsb + prep_bytes(M, K));
    const dim3 pgrid((unsigned)(K / 256), (unsigned)((M + 15) / 16));
    if (pgrid.y > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemm_prep_x, pgrid, dim3(512), 0, s, x, xp, xsp, xe, fm, (int)M, (int)K);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int bm = 16 * kMT;
    const dim3 grid((unsigned)((N + kBN - 1) / kBN), (unsigned)((M + bm - 1) / bm), (unsigned)split);
    if (grid.y > 65535) return hipErrorInvalidValue;
    if (count > 1)
      hipLaunchKernelGGL((gemm_q4k_mfma<kMT, kWaves, true>), grid, dim3(64 * kWaves), 0, s, GEMM_MATS_ARGS(mats), xp,
                         xsp, xe, fm, x, part, (int)M, (int)N, (int)K);
    else
      hipLaunchKernelGGL((gemm_q4k_mfma<kMT, kWaves, false>), grid, dim3(64 * kWaves), 0, s, GEMM_MATS_ARGS(mats), xp,
                         xsp, xe, fm, x, part, (int)M, (int)N, (int)K);
    e = hipGetLastError();
    if (e != hipSuccess || split == 1) return e;
    const bool vec = count == 1 && (M * N) % 4 == 0 && ((uintptr_t)y[0] & 15) == 0;
    const unsigned g = (unsigned)std::min<size_t>(((vec ? M * N / 4 : M * N) + 255) / 256, 8192);
    switch (split) {
#define GEMM_REDUCE(S)                                                                                        \
  case S:                                                                                                     \
    if (count > 1)                                                                                            \
      hipLaunchKernelGGL((splitk_reduce<true, S>), dim3(g), dim3(256), 0, s, part, GEMM_MATS_ARGS(mats),      \
                         (int)M, (int)N);                                                                     \
    else                                                                                                      \
      hipLaunchKernelGGL((splitk_reduce<false, S>), dim3(g), dim3(256), 0, s, part, GEMM_MATS_ARGS(mats),     \
                         (int)M, (int)N);                                                                     \
    break;
      GEMM_REDUCE(2)
      GEMM_REDUCE(3)
      GEMM_REDUCE(4)
      GEMM_REDUCE(5)
      GEMM_REDUCE(6)
      GEMM_REDUCE(7)
      GEMM_REDUCE(8)
#undef GEMM_REDUCE
      default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  // Misaligned operands: widen X to f32 (exact) and run the batched matvec,
  // which reads W once per group of up to 8 tokens.
  if (workspace_bytes < M * K * sizeof(float)) return hipErrorInvalidValue;
  float* xf = static_cast<float*>(workspace);
  size_t nx = M * K, g = (nx + 255) / 256;
  if (g > 65536) g = 65536;
  hipLaunchKernelGGL(widen_bf16_kernel, dim3((unsigned)g), dim3(256), 0, s, x, xf, nx);
  hipError_t e = hipGetLastError();
  for (int i = 0; i < count && e == hipSuccess; i++)
    if (n[i]) e = launch_matvec(kQ4_K, w[i], xf, y[i], n[i], K, M, s);
  return e;
}

#undef GEMM_MATS_ARGS

}  // namespace ssdq
