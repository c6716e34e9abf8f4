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
// where XS is the sum of X over a sub-block.  X is bf16, exact in fp16; s*q is
// an integer <= 945, exact in fp16; so every product inside P is exact and
// v_mfma_f32_16x16x32_f16 only rounds the fp32 sums of one super-block (the
// accumulators restart at every super-block).  XS is carried as an fp16
// hi + lo pair (about 22 bits).  The result differs from the reference's serial
// fp32 chain by rounding only (measured: closer to the exact sum than the
// reference itself).
//
// A prep kernel writes X as fp16 in the order the main kernel consumes it,
// plus XS: in a super-block, MFMA step t (32 k values) gives lane group c
// (lanes 16c .. 16c+15) the 8 values of sub-block 4*(t/4) + c at offset
// 8*(t%4), so one 16-byte load hands a lane the codes of a whole sub-block.
// Tiling: a workgroup of 4 waves computes a (16*MT) x 128 tile, two
// workgroups per CU.  X tiles are staged through LDS (double-buffered, fed
// from a register ring one super-block deep); weights are prefetched a
// super-block ahead; each wave owns 32 columns and builds its B fragments from
// the codes in registers.  Every global load is consumed outside branches, so
// the compiler's waits stay partial (a load consumed under a branch costs a
// full vmcnt(0) drain).
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

constexpr int BN = 128, BK = 32;
constexpr int XS = BK + 8;  // LDS row stride in halves (80 B keeps 16-byte reads conflict free)
constexpr int NT = 2;       // N sub-tiles (of 16 columns) per wave
constexpr int PF = 8;       // X staging: K steps in flight (one super-block)

__global__ __launch_bounds__(256) void widen_bf16_kernel(const uint16_t* __restrict__ x,
                                                         float* __restrict__ out, size_t n) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = __uint_as_float((uint32_t)x[i] << 16);
}

// One thread per 8 consecutive X values: writes them as fp16 at their place in
// the step order, and (lanes q = 0 / 1 of each sub-block's four) the sub-block
// sum's fp16 hi / lo parts: xsp[t][blk][0..7] = hi, [8..15] = lo.
__global__ __launch_bounds__(256) void gemm_prep_x(const uint16_t* __restrict__ x,
                                                   _Float16* __restrict__ xp,
                                                   _Float16* __restrict__ xsp, int M, int K) {
  const long groups = K / 8, total = (long)M * groups;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = gid < total;
  const long g = live ? gid : total - 1;  // every lane takes part in the shuffles
  const int m = (int)(g / groups), e8 = (int)(g % groups);
  const int q = e8 & 3, sbg = e8 >> 2, blk = sbg >> 3, gl = sbg & 7;
  const uint4 v = *reinterpret_cast<const uint4*>(x + (size_t)m * K + (size_t)e8 * 8);
  const uint32_t d[4] = {v.x, v.y, v.z, v.w};
  h8 h;
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float a = __uint_as_float(d[i] << 16), b = __uint_as_float(d[i] & 0xFFFF0000u);
    h[2 * i] = (_Float16)a;
    h[2 * i + 1] = (_Float16)b;
    sum += a;
    sum += b;
  }
  const int t = 4 * (gl >> 2) + q, c = gl & 3;
  if (live) *reinterpret_cast<h8*>(xp + (size_t)m * K + (size_t)blk * 256 + t * 32 + c * 8) = h;
  // lanes 4i .. 4i+3 hold one sub-block (groups is a multiple of 4); a + b is
  // commutative, so all four lanes end with the same sum
  sum += __shfl_xor(sum, 1);
  sum += __shfl_xor(sum, 2);
  const _Float16 hi = (_Float16)sum;
  const _Float16 lo = (_Float16)(sum - (float)hi);
  _Float16* o = xsp + ((size_t)m * (K / 256) + blk) * 16;
  if (live && q == 0) o[gl] = hi;
  if (live && q == 1) o[8 + gl] = lo;
}

// Two 4-bit codes per byte -> 8 fp16 values s*q in element order (byte i:
// low nibble = element 2i, high nibble = element 2i+1).  fp16 bits 0x6400 + v
// are 1024 + v exactly for v < 1024, and s*q <= 945.
__device__ __forceinline__ h8 codes_times_s(uint32_t qd, uint32_t s2) {
  const uint32_t ql = qd & 0x0F0F0F0Fu, qh = (qd >> 4) & 0x0F0F0F0Fu;
  const u16x2 sv = __builtin_bit_cast(u16x2, s2);
  h8 r;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    // bytes: low nibble of byte i, 0, high nibble of byte i, 0
    const uint32_t u = __builtin_amdgcn_perm(qh, ql, (uint32_t)i | 0x0C00u | ((uint32_t)(4 + i) << 16) | 0x0C000000u);
    const u16x2 vv = __builtin_bit_cast(u16x2, u) * sv + (u16x2){0x6400, 0x6400};
    const h2 hv = __builtin_bit_cast(h2, vv) - (h2){(_Float16)1024.f, (_Float16)1024.f};
    r[2 * i] = hv.x;
    r[2 * i + 1] = hv.y;
  }
  return r;
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

// blockIdx.z selects split z of the K range (split = gridDim.z); split z
// writes its partial product to y + z * M * N (a workspace when split > 1).
template <int MT>
__global__ __launch_bounds__(256, 2) void gemm_q4k_mfma(const uint8_t* __restrict__ w,
                                                        const _Float16* __restrict__ xp,
                                                        const _Float16* __restrict__ xsp,
                                                        float* __restrict__ y, int M, int N, int K) {
  constexpr int BM = 16 * MT;
  constexpr int XCH = BM * 4 / 256;  // 16-byte X chunks per thread per step
  constexpr int SS = 32;                   // LDS row stride (halves) of the sub-block sums
  constexpr int SCH = BM * 4 / 256;        // 8-byte pieces of sub-block sums per thread
  __shared__ __align__(16) _Float16 xs[2][BM * XS];
  __shared__ __align__(16) _Float16 xsum[BM * SS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int nblk = K / 256, z = blockIdx.z, nz = gridDim.z;
  const int b_begin = (int)((long)nblk * z / nz), b_end = (int)((long)nblk * (z + 1) / nz);
  const int s0 = b_begin * 8, steps = (b_end - b_begin) * 8;  // K steps of this split
  y += (size_t)z * M * N;
  const size_t row_bytes = (size_t)nblk * 144;
  const int c = lane >> 4;  // lane group: k = 8c .. 8c+7 of each step

  // weight rows of this lane's B fragments (clamped; columns past N are not stored)
  const uint8_t* wrow[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) {
    const int n = min(n0 + 32 * wave + 16 * j + (lane & 15), N - 1);
    wrow[j] = w + (size_t)n * row_bytes;
  }
  // X staging: chunk i of thread t is row (t + 256 i) / 4, 16-byte piece t % 4
  const _Float16* xsrc[XCH];
  int xdst[XCH];
#pragma unroll
  for (int i = 0; i < XCH; i++) {
    const int ch = threadIdx.x + 256 * i, r = ch >> 2, pc = ch & 3;
    xsrc[i] = xp + (size_t)min(m0 + r, M - 1) * K + 8 * pc;
    xdst[i] = r * XS + 8 * pc;
  }
  u32x4 xq[PF][XCH];
  auto fetch_x = [&](int s, auto slot_c) {
    constexpr int slot = decltype(slot_c)::value;
    const size_t off = (size_t)(s0 + min(s, steps - 1)) * BK;
#pragma unroll
    for (int i = 0; i < XCH; i++) xq[slot][i] = *reinterpret_cast<const u32x4*>(xsrc[i] + off);
  };
  auto store_x = [&](auto slot_c, auto buf_c) {
    constexpr int slot = decltype(slot_c)::value, buf = decltype(buf_c)::value;
#pragma unroll
    for (int i = 0; i < XCH; i++) *reinterpret_cast<u32x4*>(&xs[buf][xdst[i]]) = xq[slot][i];
  };

  // Sub-block sums of the current super-block: loaded at step 0, written to
  // LDS at step 6, read after step 7 (piece i of thread t: row (t + 256 i) / 4,
  // halves 4 * (t % 4) .. +4 of hi[8] | lo[8])
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  u32x2 sq[SCH];
  auto fetch_sums = [&](int b) {
#pragma unroll
    for (int i = 0; i < SCH; i++) {
      const int ch = threadIdx.x + 256 * i, r = ch >> 2;
      sq[i] = *reinterpret_cast<const u32x2*>(xsp + ((size_t)min(m0 + r, M - 1) * nblk + b_begin + b) * 16 + 4 * (ch & 3));
    }
  };
  auto store_sums = [&]() {
#pragma unroll
    for (int i = 0; i < SCH; i++) {
      const int ch = threadIdx.x + 256 * i;
      *reinterpret_cast<u32x2*>(&xsum[(ch >> 2) * SS + 4 * (ch & 3)]) = sq[i];
    }
  };

  // Weights, loaded a whole super-block (8 steps) ahead into queue registers:
  // the header (d|dmin, scale bytes 0-3, 4-7, 8-11) with the 16 code bytes of
  // sub-block c (used in steps 0-3) at step 0 of the previous super-block, the
  // 16 code bytes of sub-block 4+c (steps 4-7) at its step 4.
  u32x4a4 hdrq[NT], code0q[NT], code1q[NT], code0[NT], code1[NT];
  auto wptr = [&](int j, int b) { return wrow[j] + (size_t)(b_begin + min(b, b_end - b_begin - 1)) * 144; };
  auto fetch_head = [&](int b) {
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const uint8_t* p = wptr(j, b);
      hdrq[j] = *reinterpret_cast<const u32x4a4*>(p);
      code0q[j] = *reinterpret_cast<const u32x4a4*>(p + 16 + 16 * c);
    }
  };
  auto fetch_tail = [&](int b) {
#pragma unroll
    for (int j = 0; j < NT; j++) code1q[j] = *reinterpret_cast<const u32x4a4*>(wptr(j, b) + 16 + 16 * (4 + c));
  };

  f4 acc[MT][NT], tot[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) tot[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  // halves 16..31 of every sub-block-sum row stay zero: lanes 32-63 read them
  // as their part of the min-term A operand
  for (int r = threadIdx.x; r < BM; r += 256)
    *reinterpret_cast<u32x4*>(&xsum[r * SS + 16]) = *reinterpret_cast<u32x4*>(&xsum[r * SS + 24]) = u32x4{0u, 0u, 0u, 0u};
  fetch_head(0);
  fetch_tail(0);
  fetch_x(0, std::integral_constant<int, 0>{});
  fetch_x(1, std::integral_constant<int, 1>{});
  fetch_x(2, std::integral_constant<int, 2>{});
  fetch_x(3, std::integral_constant<int, 3>{});
  fetch_x(4, std::integral_constant<int, 4>{});
  fetch_x(5, std::integral_constant<int, 5>{});
  fetch_x(6, std::integral_constant<int, 6>{});
  fetch_x(7, std::integral_constant<int, 7>{});
  store_x(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
  __syncthreads();

  // One MFMA step t of super-block b (K step s = 8b + t); X of step s is in LDS
  // buffer t % 2; queue slot t holds X of step s until step s-1 stored it.
  auto step = [&](auto t_c, int s, int b, const uint32_t (&s2)[NT][2]) {
    constexpr int t = decltype(t_c)::value, slot = t & 1;
    if (t == 4) {  // sub-block 4+c codes arrive for steps 4-7; queue the next ones
#pragma unroll
      for (int j = 0; j < NT; j++) code1[j] = code1q[j];
      fetch_tail(b + 1);
    }
    h8 bf[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const u32x4a4 cw = t < 4 ? code0[j] : code1[j];
      const uint32_t qd = (t & 3) == 0 ? cw.x : (t & 3) == 1 ? cw.y : (t & 3) == 2 ? cw.z : cw.w;
      bf[j] = codes_times_s(qd, s2[j][t >> 2]);
    }
    if (t == 0) fetch_sums(b);
    if (t == 6) store_sums();
    // X of step s+1 goes to the other LDS buffer (its readers finished at the
    // barrier that ended step s-1; after the last step it is never read, and
    // the clamped fetch kept it in bounds); queue slot t is refilled with step
    // s+8.  No branch here: a load consumed under a branch costs a full
    // vmcnt(0) wait.
    store_x(std::integral_constant<int, (t + 1) & 7>{}, std::integral_constant<int, slot ^ 1>{});
    fetch_x(s + PF, std::integral_constant<int, t>{});
    // A fragments in groups of four (fewer registers live at once)
#pragma unroll
    for (int m4 = 0; m4 < MT; m4 += 4) {
      h8 a[4];
#pragma unroll
      for (int u = 0; u < 4; u++)
        a[u] = *reinterpret_cast<const h8*>(&xs[slot][((m4 + u) * 16 + (lane & 15)) * XS + 8 * c]);
#pragma unroll
      for (int u = 0; u < 4; u++)
#pragma unroll
        for (int j = 0; j < NT; j++)
          acc[m4 + u][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              a[u], bf[j], t == 0 ? f4{0.f, 0.f, 0.f, 0.f} : acc[m4 + u][j], 0, 0, 0);
    }
    // LDS-only barrier: the prefetched global loads stay in flight
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  };

  const int nb = b_end - b_begin;
  for (int b = 0; b < nb; b++) {
    const int s = 8 * b;
    // this super-block's scales (reference unpacking, compute.rs:724-735):
    // s[0..3] = sc[0..3] & 63, s[4..7] = sc[0..3] >> 6 | (sc[8..11] & 15) << 2,
    // m[0..3] = sc[4..7] & 63, m[4..7] = sc[4..7] >> 6 | (sc[8..11] >> 4) << 2
    uint32_t s2[NT][2], mlo[NT], mhi[NT], dbits[NT];
    u32x4a4 hdr[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) {
      hdr[j] = hdrq[j];
      code0[j] = code0q[j];
    }
    fetch_head(b + 1);
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const uint32_t h1 = hdr[j].y, h2v = hdr[j].z, h3 = hdr[j].w;
      const uint32_t slo = h1 & 0x3F3F3F3Fu;
      const uint32_t shi = ((h1 >> 6) & 0x03030303u) | ((h3 & 0x0F0F0F0Fu) << 2);
      mlo[j] = h2v & 0x3F3F3F3Fu;
      mhi[j] = ((h2v >> 6) & 0x03030303u) | (((h3 >> 4) & 0x0F0F0F0Fu) << 2);
      const uint32_t sa = (slo >> (8 * c)) & 0xFFu, sb = (shi >> (8 * c)) & 0xFFu;
      s2[j][0] = sa | (sa << 16);
      s2[j][1] = sb | (sb << 16);
      dbits[j] = hdr[j].x;
    }
    step(std::integral_constant<int, 0>{}, s, b, s2);
    step(std::integral_constant<int, 1>{}, s + 1, b, s2);
    step(std::integral_constant<int, 2>{}, s + 2, b, s2);
    step(std::integral_constant<int, 3>{}, s + 3, b, s2);
    step(std::integral_constant<int, 4>{}, s + 4, b, s2);
    step(std::integral_constant<int, 5>{}, s + 5, b, s2);
    step(std::integral_constant<int, 6>{}, s + 6, b, s2);
    step(std::integral_constant<int, 7>{}, s + 7, b, s2);
    // min term: A = XS hi (lanes 0-15) / lo (16-31) / zeros (32-63), B = the
    // 8 mins m in every lane group (finite, so the zero A lanes add 0)
    h8 bmin[NT];
    float dd[NT], dm[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) {
      uint32_t mv[4];
      bytes_to_f16(mlo[j], mv);
      bytes_to_f16(mhi[j], mv + 2);
      bmin[j] = __builtin_bit_cast(h8, u32x4{mv[0], mv[1], mv[2], mv[3]});
      dd[j] = f16_to_f32(dbits[j] & 0xFFFFu);
      dm[j] = f16_to_f32(dbits[j] >> 16);
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      const h8 amin = *reinterpret_cast<const h8*>(&xsum[(mt * 16 + (lane & 15)) * SS + 8 * c]);
#pragma unroll
      for (int j = 0; j < NT; j++) {
        const f4 qm = __builtin_amdgcn_mfma_f32_16x16x32_f16(amin, bmin[j], f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          tot[mt][j][i] = __builtin_fmaf(dd[j], acc[mt][j][i], tot[mt][j][i]);
          tot[mt][j][i] = __builtin_fmaf(-dm[j], qm[i], tot[mt][j][i]);
        }
      }
    }
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

namespace {

// Workgroup tiles are 64 (M) x 128 (N): 16 x 4 = 64 rows per wave.  128-row
// tiles would halve the B-fragment work per MFMA but need more than the 256
// registers two waves per SIMD allow (measured: 31 spilled).
constexpr int kMT = 4;

// K splits for a GEMM: enough workgroups for two per CU, at most 8 splits and
// never more than one split per 256-element block.
int gemm_split(size_t M, size_t N, size_t K) {
  const size_t bm = 16 * (size_t)kMT;
  const size_t tiles = ((N + BN - 1) / BN) * ((M + bm - 1) / bm);
  const size_t want = 2 * (size_t)device_cu_count();
  size_t split = tiles >= want ? 1 : (want + tiles - 1) / tiles;
  split = std::min<size_t>(split, 8);
  split = std::min<size_t>(split, K / 256);
  return (int)std::max<size_t>(split, 1);
}

// workspace layout: X in step order (M*K fp16) | sub-block sums (M*K/256*16
// fp16) | split partials (split*M*N f32)
size_t prep_bytes(size_t M, size_t K) { return M * K * 2 + M * (K / 256) * 32; }

}  // namespace

size_t gemm_q4k_workspace_bytes(const void* w, const void* x, size_t M, size_t N, size_t K) {
  if (!gemm_q4k_mfma_ok(w, x)) return M * K * sizeof(float);
  const int split = gemm_split(M, N, K);
  return prep_bytes(M, K) + (split > 1 ? (size_t)split * M * N * sizeof(float) : 0);
}

hipError_t launch_gemm_q4k(const uint8_t* w, const uint16_t* x, float* y, size_t M, size_t N,
                           size_t K, void* workspace, size_t workspace_bytes, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  if (K % 256 != 0) return hipErrorInvalidValue;
  if (gemm_q4k_mfma_ok(w, x)) {
    const int split = gemm_split(M, N, K);
    const size_t need = prep_bytes(M, K) + (split > 1 ? (size_t)split * M * N * sizeof(float) : 0);
    if (workspace_bytes < need) return hipErrorInvalidValue;
    _Float16* xp = static_cast<_Float16*>(workspace);
    _Float16* xsp = xp + M * K;
    float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + prep_bytes(M, K));
    const size_t groups = M * K / 8;
    hipLaunchKernelGGL(gemm_prep_x, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, s, x, xp, xsp,
                       (int)M, (int)K);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int bm = 16 * kMT;
    const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + bm - 1) / bm), (unsigned)split);
    if (grid.y > 65535) return hipErrorInvalidValue;
    float* dst = split > 1 ? part : y;
    hipLaunchKernelGGL(gemm_q4k_mfma<kMT>, grid, dim3(256), 0, s, w, xp, xsp, dst, (int)M, (int)N, (int)K);
    e = hipGetLastError();
    if (e != hipSuccess || split == 1) return e;
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
