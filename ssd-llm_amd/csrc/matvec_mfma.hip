// Small-batch Q8_0 matvec (2-8 activation rows) on the matrix cores.
//
// Reference semantics: matvec_q8_0_cpu (src/metal/compute.rs:904-925) once per
// activation row (src/inference/batch_scheduler.rs:242-276):
// y[b][r] = sum over blocks j of sum_k fl(d_rj * q_rjk) * x[b][32 j + k].
//
// x is carried as in the other digit-plane kernels: each 32-element block of
// an activation row is scaled by a power of two so its largest magnitude sits
// just under 2^22, rounded to integers xi, and written as three balanced
// base-256 digits (signed bytes).  One Q8_0 block is one K = 32 step of
// v_mfma_i32_16x16x32_i8:
//   A (16 x 32 i8): row 4 b' + t is digit t of activation row 4 m + b' (t = 3
//                   is zero), m = 0 for rows 0-3, 1 for rows 4-7;
//   B (32 x 16 i8): column c is the 32 codes of weight row c of the group;
//   D (16 x 16 i32): lane l holds the exact integer sums of digits 0, 1, 2 of
//                   activation row 4 m + l / 16 against weight row l % 16,
// so every lane recombines its own digits (I0 + 256 I1 + 65536 I2), scales by
// the block's d and the x block's power of two, and accumulates in fp32.
//
// Layout: a workgroup of 8 waves owns groups of 16 consecutive weight rows (one
// contiguous run of 16 * row_bytes in HBM), each taken as two stages (the
// first and second halves of the 16 rows).  A stage's half rows are loaded
// straight into LDS (direct loads, four buffers, three stages in flight) and
// each wave reads its B operands there: wave w takes blocks [w K/512, (w + 1)
// K/512) of each half, with its x digit planes in registers.  The eight partial
// sums of an output are added in wave order in LDS.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace ssdq {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kGRows = 16;   // weight rows per group (the MFMA's 16 columns)
constexpr int kWaves = 8;    // waves per workgroup (K eighths)
constexpr int kRowPad = 16;  // LDS bytes after each row (spreads the rows over banks)

__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  uint32_t keep;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
               : "=&s"(keep)
               : "s"(lds), "v"(g)
               : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// byte d of a, b, c, e -> bytes 0, 1, 2, 3
__device__ __forceinline__ uint32_t gather_byte(uint32_t a, uint32_t b, uint32_t c, uint32_t e, int d) {
  const uint32_t lo = __builtin_amdgcn_perm(b, a, (uint32_t)d | ((uint32_t)(4 + d) << 8) | 0x0C0C0000u);
  const uint32_t hi = __builtin_amdgcn_perm(e, c, 0x00000C0Cu | ((uint32_t)d << 16) | ((uint32_t)(4 + d) << 24));
  return lo | hi;
}

template <int NBLK>
struct Q8Geom {
  static_assert(NBLK % (2 * kWaves) == 0, "whole blocks per wave and half row");
  static constexpr int row_bytes = NBLK * 34;
  static constexpr int half_bytes = row_bytes / 2;             // one stage: half of each row
  static constexpr int stride = half_bytes + kRowPad;
  static constexpr int pieces = half_bytes / 16;               // 16-byte loads per half row
  static constexpr int full = pieces / 64, rem = pieces % 64;
  static constexpr int dma_per_row = full + (rem ? 1 : 0);
  static constexpr int rows_per_wave = kGRows / kWaves;
  static constexpr int dma_per_wave = rows_per_wave * dma_per_row;  // per stage
  static constexpr int bw = NBLK / (2 * kWaves);                    // blocks per wave per stage
  static constexpr int buf_bytes = kGRows * stride;
  static constexpr int nbuf = 4;                                   // stages in LDS (3 in flight)
  static_assert(half_bytes % 16 == 0, "half rows of whole 16-byte pieces");
  static_assert(2 * dma_per_wave < 63, "vmcnt range");
};

// x staging through one stage buffer: blocks per pass (A fragments of NM
// MFMAs and NB scales per block), a power of two dividing the row
template <int NB, int NBLK>
struct Q8Staging {
  static constexpr int per_block = (NB + 3) / 4 * 64 * 8 + NB * 4;
  // one buffer (three stages in flight) when half a row's planes fit it, else
  // two buffers (two stages in flight): fewer passes and barriers
  static constexpr int nbuf = Q8Geom<NBLK>::buf_bytes / per_block >= NBLK / 2 ? 1 : 2;
  static constexpr int fit = nbuf * Q8Geom<NBLK>::buf_bytes / per_block;
  static constexpr int pow2_floor(int v) { return v >= 64 ? 64 : v >= 32 ? 32 : v >= 16 ? 16 : v >= 8 ? 8 : v >= 4 ? 4 : 1; }
  static constexpr int pbk = pow2_floor(fit) < NBLK / 2 ? pow2_floor(fit) : NBLK / 2;
  static_assert(pbk >= 1 && pbk <= fit && (NBLK / 2) % pbk == 0, "pass geometry");
};

template <int NB, int NBLK>
constexpr size_t q8_lds_bytes() {
  constexpr int NM = (NB + 3) / 4;
  return (size_t)Q8Geom<NBLK>::nbuf * Q8Geom<NBLK>::buf_bytes + (size_t)kWaves * NM * 64 * sizeof(float);
}

// Stage s of a workgroup is half s & 1 of its group s >> 1 (groups blockIdx.x,
// blockIdx.x + gridDim.x, ...); its 16 half rows go to LDS buffer s % 4.  Wave w
// takes blocks [h NBLK/2 + w bw, + bw) of half h.
template <int NB, int NBLK>
__global__ __launch_bounds__(512, 1) void mv_q8_mfma(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                      float* __restrict__ y, int out_dim, int n_groups) {
  using G = Q8Geom<NBLK>;
  constexpr int NM = (NB + 3) / 4;  // MFMAs per block (activation rows 0-3, 4-7)
  constexpr int BW = G::bw;
  constexpr int HB = NBLK / 2;      // blocks per half row
  extern __shared__ __align__(16) uint8_t smem[];
  float* red = reinterpret_cast<float*>(smem + G::nbuf * G::buf_bytes);  // [wave][NM][64]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int my_groups = blockIdx.x < n_groups ? (n_groups - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
  const int n_stages = 2 * my_groups;

  // ---- x: every chunk of 8 elements this thread converts, requested before any weight.
  // Pass h (half h) has NB * HB * 4 chunks; thread t takes chunks t + 512 k.
  constexpr int CPP = (NB * HB * 4 + 511) / 512;  // chunks per thread per pass
  float4 xv[2][CPP][2];
#pragma unroll
  for (int h = 0; h < 2; h++)
#pragma unroll
    for (int k = 0; k < CPP; k++) {
      const int c = min((int)threadIdx.x + 512 * k, NB * HB * 4 - 1);
      const int b = c / (HB * 4), jj = (c % (HB * 4)) >> 2, kg = c & 3;
      const float* xp = x + (size_t)b * (NBLK * 32) + (size_t)(h * HB + jj) * 32 + 8 * kg;
      xv[h][k][0] = *reinterpret_cast<const float4*>(xp);
      xv[h][k][1] = *reinterpret_cast<const float4*>(xp + 4);
    }

  // one stage (16 half rows) into its LDS buffer: wave w loads rows 2w, 2w + 1
  // (rows past out_dim repeat the last row; their sums are not stored)
  auto dma_stage = [&](int st) {
    const int g = (int)blockIdx.x + (st >> 1) * (int)gridDim.x, h = st & 1;
    uint8_t* buf = smem + (st % G::nbuf) * G::buf_bytes;
#pragma unroll
    for (int rr = 0; rr < G::rows_per_wave; rr++) {
      const int r = wave * G::rows_per_wave + rr;
      const int grow = min(g * kGRows + r, out_dim - 1);
      const uint8_t* src = w + (size_t)grow * G::row_bytes + h * G::half_bytes + 16 * lane;
      const uint32_t dst = __builtin_amdgcn_readfirstlane(lds_addr(buf + r * G::stride));  // uniform
#pragma unroll
      for (int i = 0; i < G::full; i++) dma16(src + 1024 * i, dst + 1024 * i);
      if (G::rem) {
        if (lane < G::rem) dma16(src + 1024 * G::full, dst + 1024 * G::full);
      }
    }
  };
  // Pad loads: the compiler counts only its own loads when it waits for x
  // (in-order vmcnt), so KPAD of them between the x loads and the stage loads
  // keep its counts from covering the stage loads issued after them: the
  // stages stay in flight while x is converted.  They read the start of x
  // (cached: x is read anyway).
  constexpr int SBUF = Q8Staging<NB, NBLK>::nbuf;  // stage buffers the x staging uses
  constexpr int PRE = 4 - SBUF;                      // stages in flight meanwhile
  constexpr int KPAD = PRE * G::dma_per_wave;
  uint32_t pad = 0;
#pragma unroll
  for (int i = 0; i < KPAD; i++) pad += reinterpret_cast<const uint32_t*>(x)[64 * i + lane];  // distinct: not merged
  // PRE stages in flight while x is staged (it passes through the last SBUF buffers)
#pragma unroll
  for (int st = 0; st < PRE; st++)
    if (n_stages > st) dma_stage(st);

  // ---- x digit planes: A fragments [block of the pass][m][lane][8 bytes] and
  // block scales [block][activation row], PBK blocks per pass through buffer 3;
  // a wave copies the fragments of its blocks into registers
  int64_t afrag[2][BW][NM];
  float xsc[2][BW][NM];
  {
    constexpr int PBK = Q8Staging<NB, NBLK>::pbk;  // blocks per pass
    constexpr int NPASS = NBLK / PBK;
    uint2* frag = reinterpret_cast<uint2*>(smem + (4 - SBUF) * G::buf_bytes);
    float* scl = reinterpret_cast<float*>(smem + (4 - SBUF) * G::buf_bytes + (size_t)PBK * NM * 64 * 8);
#pragma unroll
    for (int p = 0; p < NPASS; p++) {
      const int h = (p * PBK) / HB;  // the half these blocks belong to
#pragma unroll
      for (int k = 0; k < CPP; k++) {
        const int c0 = (int)threadIdx.x + 512 * k;
        const bool live = c0 < NB * HB * 4;
        const int c = min(c0, NB * HB * 4 - 1);
        const int b = c / (HB * 4), jh = (c % (HB * 4)) >> 2, kg = c & 3;
        const int jp = h * HB + jh - p * PBK;  // block within the pass
        if (jp < 0 || jp >= PBK) continue;     // uniform over the 4 lanes of a block
        const float v[8] = {xv[h][k][0].x, xv[h][k][0].y, xv[h][k][0].z, xv[h][k][0].w,
                            xv[h][k][1].x, xv[h][k][1].y, xv[h][k][1].z, xv[h][k][1].w};
        float m = 0.f;
        bool bad = false;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          m = fmaxf(m, fabsf(v[i]));
          bad |= !(fabsf(v[i]) < INFINITY);
        }
        // the four chunks of a block are the lanes of one DPP quad
        m = fmaxf(m, dpp_mov<0xB1>(m));
        m = fmaxf(m, dpp_mov<0x4E>(m));
        float badf = bad ? 1.f : 0.f;
        badf = fmaxf(badf, dpp_mov<0xB1>(badf));
        badf = fmaxf(badf, dpp_mov<0x4E>(badf));
        int e = 0;
        if (m > 0.f) (void)frexpf(m, &e);  // m < 2^e
        const int sh = 22 - e;             // the values are scaled (2^sh itself may overflow)
        uint32_t u[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const int xi = (int)rintf(ldexpf(v[i], sh));     // |xi| <= 2^22
          u[i] = ((uint32_t)(xi + 0x808080)) ^ 0x808080u;  // bytes 0-2: balanced digits
        }
        if (live) {
          const int m4 = b >> 2, bb = b & 3;
          uint2* f = frag + ((size_t)jp * NM + m4) * 64 + 16 * kg + 4 * bb;
#pragma unroll
          for (int d = 0; d < 3; d++)
            f[d] = make_uint2(gather_byte(u[0], u[1], u[2], u[3], d), gather_byte(u[4], u[5], u[6], u[7], d));
          f[3] = make_uint2(0u, 0u);
          if (kg == 0) scl[jp * NB + b] = badf != 0.f ? __builtin_nanf("") : ldexpf(1.0f, e - 22);
        }
      }
      // activation rows NB .. 4 NM - 1 of the last MFMA are zero
      if (NB < 4 * NM) {
        for (int c = threadIdx.x; c < PBK * 4 * (4 * NM - NB); c += 512) {
          const int jp = c / (4 * (4 * NM - NB)), q = c % (4 * (4 * NM - NB));
          const int b = NB + (q >> 2), kg = q & 3;
          uint2* f = frag + ((size_t)jp * NM + (b >> 2)) * 64 + 16 * kg + 4 * (b & 3);
#pragma unroll
          for (int d = 0; d < 4; d++) f[d] = make_uint2(0u, 0u);
        }
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < BW; i++) {
        const int jp = h * HB + wave * BW + i - p * PBK;
        if (jp >= 0 && jp < PBK) {  // uniform per wave
#pragma unroll
          for (int m4 = 0; m4 < NM; m4++) {
            const uint2 f = frag[((size_t)jp * NM + m4) * 64 + lane];
            afrag[h][i][m4] = (int64_t)(((uint64_t)f.y << 32) | f.x);
            const int b = 4 * m4 + (lane >> 4);
            xsc[h][i][m4] = b < NB ? scl[jp * NB + b] : 0.f;
          }
        }
      }
      __syncthreads();
    }
  }

#pragma unroll
  for (int st = PRE; st < 3; st++)
    if (n_stages > st) dma_stage(st);

  const int r16 = lane & 15, kg = lane >> 4;
  float acc[NM];
  for (int st = 0; st < n_stages; st++) {
    // this stage's loads have landed (at most two later stages still in flight)
    const int ahead = min(n_stages - 1 - st, 2);
    if (ahead == 2)
      __builtin_amdgcn_s_waitcnt((((2 * G::dma_per_wave) & 15) | (((2 * G::dma_per_wave) >> 4) << 14)) | (7 << 4) |
                                 (15 << 8));
    else if (ahead == 1)
      __builtin_amdgcn_s_waitcnt(((G::dma_per_wave & 15) | ((G::dma_per_wave >> 4) << 14)) | (7 << 4) | (15 << 8));
    else
      __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
    __syncthreads();  // every wave's loads of this stage have landed, and the
                      // buffer of stage st - 1 is no longer read
    if (st + 3 < n_stages) dma_stage(st + 3);

    const int h = st & 1;
    if (h == 0) {
#pragma unroll
      for (int m4 = 0; m4 < NM; m4++) acc[m4] = 0.f;
    }
    const uint8_t* rowp = smem + (st % G::nbuf) * G::buf_bytes + r16 * G::stride;
    auto run_half = [&](auto hc) {
      constexpr int H = decltype(hc)::value;
      // all of the stage's LDS reads first (one wait), then the MFMAs.  The
      // block's parity (its 34-byte alignment) is that of i: H HB and wave BW
      // are even.
      static_assert((HB % 2) == 0 && (BW % 2) == 0, "block parity follows i");
      uint32_t raw[BW][4];
#pragma unroll
      for (int i = 0; i < BW; i++) {
        const uint8_t* blk = rowp + 34 * (wave * BW + i);
        if ((i & 1) == 0) {  // block at a 4-byte boundary: d, then codes 2 bytes in
          const uint32_t* p = reinterpret_cast<const uint32_t*>(blk + 8 * kg);
          raw[i][0] = p[0];
          raw[i][1] = p[1];
          raw[i][2] = p[2];
          raw[i][3] = *reinterpret_cast<const uint32_t*>(blk);
        } else {  // block 2 bytes past a boundary: codes 4-byte aligned
          const uint32_t* p = reinterpret_cast<const uint32_t*>(blk + 2 + 8 * kg);
          raw[i][0] = p[0];
          raw[i][1] = p[1];
          raw[i][2] = 0u;
          raw[i][3] = *reinterpret_cast<const uint32_t*>(blk - 2);
        }
      }
#pragma unroll
      for (int i = 0; i < BW; i++) {
        uint32_t lo, hi, dbits;
        if ((i & 1) == 0) {
          lo = __builtin_amdgcn_alignbit(raw[i][1], raw[i][0], 16);
          hi = __builtin_amdgcn_alignbit(raw[i][2], raw[i][1], 16);
          dbits = raw[i][3] & 0xFFFFu;
        } else {
          lo = raw[i][0];
          hi = raw[i][1];
          dbits = raw[i][3] >> 16;
        }
        const int64_t bop = (int64_t)(((uint64_t)hi << 32) | lo);
        const float d = f16_to_f32(dbits);
#pragma unroll
        for (int m4 = 0; m4 < NM; m4++) {
          const i32x4 c = __builtin_amdgcn_mfma_i32_16x16x32_i8(afrag[H][i][m4], bop, i32x4{0, 0, 0, 0}, 0, 0, 0);
          // I0 + 256 I1 exactly in int (|I1| <= 2^16), then one rounding with 65536 I2
          const float f = fmaf(65536.0f, (float)c.z, (float)(c.x + (c.y << 8)));
          acc[m4] = fmaf(d, f * xsc[H][i][m4], acc[m4]);
        }
      }
    };
    if (h == 0) run_half(std::integral_constant<int, 0>{});
    else run_half(std::integral_constant<int, 1>{});
    if (h == 1) {
#pragma unroll
      for (int m4 = 0; m4 < NM; m4++) red[(wave * NM + m4) * 64 + lane] = acc[m4];
      __syncthreads();
      if (threadIdx.x < NM * 64) {
        const int m4 = threadIdx.x >> 6, l = threadIdx.x & 63;
        float s = 0.f;
#pragma unroll
        for (int wv = 0; wv < kWaves; wv++) s += red[(wv * NM + m4) * 64 + l];
        const int g = (int)blockIdx.x + (st >> 1) * (int)gridDim.x;
        const int b = 4 * m4 + (l >> 4), row = g * kGRows + (l & 15);
        if (b < NB && row < out_dim) y[(size_t)b * out_dim + row] = s;
      }
    }
  }
  asm volatile("" ::"v"(pad));  // the pad loads are used (kept), after everything else
}

template <int NB, int NBLK>
hipError_t run_q8_mfma(const uint8_t* w, const float* x, float* y, int out_dim, hipStream_t s) {
  auto kern = mv_q8_mfma<NB, NBLK>;
  constexpr size_t lds = q8_lds_bytes<NB, NBLK>();
  static std::mutex mu;
  static bool attr_set = false;
  {
    std::lock_guard<std::mutex> lk(mu);
    if (!attr_set) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
      attr_set = true;
    }
  }
  const int n_groups = (out_dim + kGRows - 1) / kGRows;
  const int grid = std::min(n_groups, device_cu_count());
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * kWaves), lds, s, w, x, y, out_dim, n_groups);
  return hipGetLastError();
}

template <int NBLK>
hipError_t q8_mfma_nb(int nb, const uint8_t* w, const float* x, float* y, int out_dim, hipStream_t s) {
  switch (nb) {
    case 2: return run_q8_mfma<2, NBLK>(w, x, y, out_dim, s);
    case 3: return run_q8_mfma<3, NBLK>(w, x, y, out_dim, s);
    case 4: return run_q8_mfma<4, NBLK>(w, x, y, out_dim, s);
    case 5: return run_q8_mfma<5, NBLK>(w, x, y, out_dim, s);
    case 6: return run_q8_mfma<6, NBLK>(w, x, y, out_dim, s);
    case 7: return run_q8_mfma<7, NBLK>(w, x, y, out_dim, s);
    case 8: return run_q8_mfma<8, NBLK>(w, x, y, out_dim, s);
    default: return hipErrorNotSupported;
  }
}

}  // namespace

bool q8_mfma_supported(const void* w, const float* x, size_t in_dim, size_t batch) {
  return batch >= 2 && batch <= 8 && (in_dim == 4096 || in_dim == 2048 || in_dim == 1024) &&
         ((uintptr_t)w & 15) == 0 && ((uintptr_t)x & 15) == 0;
}

hipError_t launch_q8_mfma(const uint8_t* w, const float* x, float* y, size_t out_dim, size_t in_dim, size_t batch,
                          hipStream_t s) {
  if (!q8_mfma_supported(w, x, in_dim, batch) || out_dim == 0 || out_dim > (size_t)INT_MAX)
    return hipErrorNotSupported;
  switch (in_dim) {
    case 4096: return q8_mfma_nb<128>((int)batch, w, x, y, (int)out_dim, s);
    case 2048: return q8_mfma_nb<64>((int)batch, w, x, y, (int)out_dim, s);
    case 1024: return q8_mfma_nb<32>((int)batch, w, x, y, (int)out_dim, s);
    default: return hipErrorNotSupported;
  }
}

}  // namespace ssdq
