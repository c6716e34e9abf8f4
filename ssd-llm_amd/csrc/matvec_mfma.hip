// Small-batch Q8_0 matvec (2-8 activation rows) on the matrix cores.
//
// Reference semantics: matvec_q8_0_cpu (src/metal/compute.rs:904-925) once per
// activation row (src/inference/batch_scheduler.rs:242-276):
// y[b][r] = sum over blocks j of sum_k fl(d_rj * q_rjk) * x[b][32 j + k].
//
// x is carried as in the other digit-plane kernels: each 32-element block of
// an activation row is scaled by a power of two so its largest magnitude sits
// just under 2^30, rounded to integers xi, and written as four balanced
// base-256 digits (signed bytes).  One Q8_0 block is one K = 32 step of
// v_mfma_i32_16x16x32_i8:
//   A (16 x 32 i8): row 4 b' + t is digit t of activation row 4 m + b',
//                   m = 0 for rows 0-3, 1 for rows 4-7;
//   B (32 x 16 i8): column c is the 32 codes of weight row c of the group;
//   D (16 x 16 i32): lane l holds the exact integer sums of digits 0-3 of
//                   activation row 4 m + l / 16 against weight row l % 16,
// so every lane recombines its own digits (I0 + 256 I1 + 2^16 I2 + 2^24 I3),
// scales by the block's d and the x block's power of two, and accumulates in
// fp32.
//
// Layout: a workgroup of 12 waves owns a run of at most 48 rows (three
// groups of 16; runs are spread evenly over the CUs, 43 rows each for 11008
// rows on 256 CUs); the four waves of a group take a quarter of K each.  Lane
// (n = l % 16, q = l / 16) of a wave loads, per step of 8 blocks, the
// dword-aligned 68-byte unit q (blocks 2q, 2q + 1) of row n straight into
// registers, as the batch-1 kernel loads its units.  A 4 x 4 transpose of
// 8-byte chunks across the four 16-lane rows (v_permlane16_swap, then
// v_permlane32_swap) leaves lane row q holding chunk q (codes 8q .. 8q + 7) of
// each of the step's 8 blocks: the B operand for every block.  The x digit
// planes of the whole row are built once per workgroup in LDS (the A operands)
// while the first steps stream, and the four partial sums of an output are
// added in K order in LDS.
#include <algorithm>
#include <mutex>

#include "common.hpp"
#include "launch.hpp"

namespace ssdq {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int kGRows = 16;  // weight rows per group (the MFMA's 16 columns)
constexpr int kRq = 4;      // K quarters per group
constexpr int kRgpw = 3;    // groups per workgroup

template <int NB, int NBLK>
struct Q8R {
  static constexpr int NM = (NB + 3) / 4;
  // steps of 8 blocks in flight per wave (one for 5-8 rows: their x staging
  // is longer, and the stream waits less for it)
  static constexpr int D = NB > 4 ? 1 : 2;
  static constexpr int TB = NBLK / kRq;  // blocks per wave
  static constexpr int STEPS = TB / 8;
  static_assert(TB % 8 == 0, "whole steps of 8 blocks per wave");
  static constexpr int THREADS = 64 * kRq * kRgpw;
  static constexpr int CHUNKS = NB * NBLK * 4;  // 8-element pieces of x
  static constexpr int CPT = (CHUNKS + THREADS - 1) / THREADS;
  // A fragments of block j at j * FS (NM of 512 bytes), padded by 16 bytes
  // so that the staging writes of consecutive blocks fall in different banks
  static constexpr int FS = NM * 512 + 16;
  static constexpr size_t frag_bytes = (size_t)NBLK * FS;
  static constexpr size_t scl_bytes = (size_t)NBLK * NB * 4;
  static constexpr size_t red_bytes = (size_t)kRgpw * kRq * NM * 64 * 8;  // double partial sums
  static constexpr size_t lds = frag_bytes + scl_bytes + red_bytes;
};

// 4 x 4 transpose of one dword of four chunks held by the four 16-lane rows:
// on entry lane row r holds c[i] = chunk i of source r; on exit c[i] = chunk r
// of source i.
__device__ __forceinline__ void transpose_rows4(uint32_t (&c)[4]) {
  // rows 2i + 1 of c0 <-> rows 2i of c1 (likewise c2, c3)
  const auto p01 = __builtin_amdgcn_permlane16_swap(c[0], c[1], false, false);
  const auto p23 = __builtin_amdgcn_permlane16_swap(c[2], c[3], false, false);
  // rows 2, 3 of c0 <-> rows 0, 1 of c2 (likewise c1, c3)
  const auto q02 = __builtin_amdgcn_permlane32_swap(p01[0], p23[0], false, false);
  const auto q13 = __builtin_amdgcn_permlane32_swap(p01[1], p23[1], false, false);
  c[0] = q02[0];
  c[1] = q13[0];
  c[2] = q02[1];
  c[3] = q13[1];
}

// Workgroup b owns rows [b rpw, min((b + 1) rpw, out_dim)), rpw <= 48.
template <int NB, int NBLK>
__global__ __launch_bounds__(768, 1) void mv_q8r(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                  float* __restrict__ y, int out_dim, int rpw) {
  using P = Q8R<NB, NBLK>;
  constexpr int NM = P::NM;
  extern __shared__ __align__(16) uint8_t smem[];
  uint8_t* frag = smem;                                                         // [block][m][lane] (uint2)
  float* scl = reinterpret_cast<float*>(smem + P::frag_bytes);                  // [block][activation row]
  double* red = reinterpret_cast<double*>(smem + P::frag_bytes + P::scl_bytes);  // [group][quarter][m][lane]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int gl = wave / kRq, kq = wave % kRq;
  const int wg_row0 = (int)blockIdx.x * rpw, wg_end = min(wg_row0 + rpw, out_dim);
  const int g_row0 = wg_row0 + gl * kGRows;
  const bool busy = g_row0 < wg_end;  // uniform per wave
  const int kg = lane >> 4;
  constexpr int chunks = P::CHUNKS;

  // ---- x chunks this thread converts (chunk c: activation row c / (4 NBLK),
  // block (c / 4) % NBLK, elements 8 (c % 4) ..), requested first
  float4 xv[P::CPT][2];
#pragma unroll
  for (int k = 0; k < P::CPT; k++) {
    const int c = min((int)threadIdx.x + P::THREADS * k, chunks - 1);
    const float* xp = x + (size_t)(c / (NBLK * 4)) * (NBLK * 32) + (size_t)((c >> 2) % NBLK) * 32 + 8 * (c & 3);
    xv[k][0] = *reinterpret_cast<const float4*>(xp);
    xv[k][1] = *reinterpret_cast<const float4*>(xp + 4);
  }

  // ---- this wave's weights: step s is unit 4 s + kg of its quarter of row
  // g_row0 + n (rows past the workgroup's run repeat its last row, and idle
  // waves load that row too: their sums are not stored).  D steps are
  // requested before x is staged and each later one as the step D before it
  // is taken up: a workgroup keeps about 50-100 KB in flight, what one CU
  // sustains (with every step requested at once the waves stall at issue for
  // microseconds and the x staging and all of the arithmetic come after the
  // stream).
  uint32_t raw[P::STEPS][17];
  const uint8_t* rp = w + (size_t)min(g_row0 + (lane & 15), wg_end - 1) * (NBLK * 34) +
                      (size_t)(kq * P::TB) * 34 + 68 * kg;
  auto load_step = [&](int s) {
    const uint8_t* p = rp + 272 * s;
    const u32x4a4 a = *reinterpret_cast<const u32x4a4*>(p);
    const u32x4a4 b = *reinterpret_cast<const u32x4a4*>(p + 16);
    const u32x4a4 c = *reinterpret_cast<const u32x4a4*>(p + 32);
    const u32x4a4 d = *reinterpret_cast<const u32x4a4*>(p + 48);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      raw[s][i] = a[i];
      raw[s][4 + i] = b[i];
      raw[s][8 + i] = c[i];
      raw[s][12 + i] = d[i];
    }
    raw[s][16] = *reinterpret_cast<const uint32_t*>(p + 64);
  };
#pragma unroll
  for (int s = 0; s < P::STEPS && s < P::D; s++) load_step(s);
  // the loads above are issued before anything waits for one
  __builtin_amdgcn_sched_barrier(0);

  // ---- x digit planes of the whole row into LDS (A rows 4 b' + t: digits
  // 0-3; the rows of activation rows past NB are never read)
#pragma unroll
  for (int k = 0; k < P::CPT; k++) {
    const int c0 = (int)threadIdx.x + P::THREADS * k;
    const int c = min(c0, chunks - 1);
    const int b = c / (NBLK * 4), j = (c >> 2) % NBLK, q = c & 3;
    const float v[8] = {xv[k][0].x, xv[k][0].y, xv[k][0].z, xv[k][0].w,
                        xv[k][1].x, xv[k][1].y, xv[k][1].z, xv[k][1].w};
    float m = 0.f, z = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      m = fmaxf(m, fabsf(v[i]));
      z = fmaf(v[i], 0.f, z);  // NaN when an element is NaN or infinite
    }
    // the four chunks of a block are the lanes of one DPP quad
    m = fmaxf(m, dpp_mov<0xB1>(m));
    m = fmaxf(m, dpp_mov<0x4E>(m));
    z += dpp_mov<0xB1>(z);
    z += dpp_mov<0x4E>(z);
    int e = 0;
    if (m > 0.f) (void)frexpf(m, &e);  // m < 2^e
    const int sh = min(30 - e, 149);  // 2^-sh stays a (subnormal) fp32 value
    // xi = rint(v 2^sh), |xi| <= 2^30 (one rounding, to nearest even); u = xi +
    // 0x80808080 lies in [0, 2^32), and its bytes xor 0x80 are the balanced
    // digits
    uint32_t u[8];
#pragma unroll
    for (int i = 0; i < 8; i++) u[i] = ((uint32_t)(int)rintf(ldexpf(v[i], sh)) + 0x80808080u) ^ 0x80808080u;
    if (c0 < chunks) {
      uint2* f = reinterpret_cast<uint2*>(frag + (size_t)j * P::FS + (b >> 2) * 512) + 16 * q + 4 * (b & 3);
      uint32_t p0[4], p1[4];
      planes4(u[0], u[1], u[2], u[3], p0);
      planes4(u[4], u[5], u[6], u[7], p1);
#pragma unroll
      for (int d = 0; d < 4; d++) f[d] = make_uint2(p0[d], p1[d]);
      if (q == 0) scl[j * NB + b] = z != z ? __builtin_nanf("") : ldexpf(1.0f, -sh);
    }
  }
  __syncthreads();

  // A row lane % 16 of MFMA m is digit lane % 4 of activation row 4 m +
  // lane % 16 / 4; D rows 4 q .. 4 q + 3 are activation row 4 m + q.  Rows of
  // activation rows past NB (batches that are not a multiple of 4) are masked
  // to zero, as bits: a select here becomes a branch around the LDS reads
  uint64_t amask[NM];
  uint32_t xmask[NM];
#pragma unroll
  for (int m4 = 0; m4 < NM; m4++) {
    amask[m4] = 4 * m4 + ((lane & 15) >> 2) < NB ? ~0ull : 0ull;
    xmask[m4] = 4 * m4 + kg < NB ? ~0u : 0u;
  }
  // per-lane sums in double: terms of very different sizes (massive
  // activation channels) cancel without fp32 rounding
  double acc[NM];
#pragma unroll
  for (int m4 = 0; m4 < NM; m4++) acc[m4] = 0.0;
  if (busy) {
#pragma unroll
    for (int s = 0; s < P::STEPS; s++) {
      if (s + P::D < P::STEPS) load_step(s + P::D);
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t* R = raw[s];
      // chunk i of the even block (codes 2 bytes into the unit) and of the odd
      // block (codes at dword 9), low and high dwords
      uint32_t el[4], eh[4], ol[4], oh[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        el[i] = __builtin_amdgcn_alignbit(R[2 * i + 1], R[2 * i], 16);
        eh[i] = __builtin_amdgcn_alignbit(R[2 * i + 2], R[2 * i + 1], 16);
        ol[i] = R[9 + 2 * i];
        oh[i] = R[10 + 2 * i];
      }
      transpose_rows4(el);
      transpose_rows4(eh);
      transpose_rows4(ol);
      transpose_rows4(oh);
      // the block scales of lane row r (blocks 2 r, 2 r + 1) to every row
      const uint32_t dd = (R[0] & 0xFFFFu) | (R[8] & 0xFFFF0000u);
      const auto t = __builtin_amdgcn_permlane16_swap(dd, dd, false, false);  // {rows 0 0 2 2, 1 1 3 3}
      const auto t0 = __builtin_amdgcn_permlane32_swap(t[0], t[0], false, false);
      const auto t1 = __builtin_amdgcn_permlane32_swap(t[1], t[1], false, false);
      const uint32_t dr[4] = {t0[0], t1[0], t0[1], t1[1]};
#pragma unroll
      for (int bk = 0; bk < 8; bk++) {
        const int r = bk >> 1;
        const uint32_t lo = (bk & 1) ? ol[r] : el[r], hi = (bk & 1) ? oh[r] : eh[r];
        const int64_t bop = (int64_t)(((uint64_t)hi << 32) | lo);
        const float d = f16_to_f32((bk & 1) ? dr[r] >> 16 : dr[r] & 0xFFFFu);
        const int j = kq * P::TB + 8 * s + bk;
#pragma unroll
        for (int m4 = 0; m4 < NM; m4++) {
          const uint2 fa = reinterpret_cast<const uint2*>(frag + (size_t)j * P::FS + m4 * 512)[lane];
          const uint64_t av = ((uint64_t)fa.y << 32) | fa.x;
          const int64_t aop = (int64_t)(NB % 4 == 0 ? av : av & amask[m4]);
          const float xs = __uint_as_float(__float_as_uint(scl[j * NB + min(4 * m4 + kg, NB - 1)]) & xmask[m4]);
          const i32x4 c = __builtin_amdgcn_mfma_i32_16x16x32_i8(aop, bop, i32x4{0, 0, 0, 0}, 0, 0, 0);
          // I0 + 256 I1 and I2 + 256 I3 exactly in int (|I1|, |I3| < 2^20), then
          // the exact digit sum (below 2^53) and the exact scales in double
          const double f = fma(65536.0, (double)(c.z + (c.w << 8)), (double)(c.x + (c.y << 8)));
          acc[m4] = fma((double)d, f * (double)xs, acc[m4]);
        }
        if (bk & 1) __builtin_amdgcn_sched_barrier(0);  // two blocks at a time: bounded registers
      }
      __builtin_amdgcn_sched_barrier(0);  // a step waits only for its own loads
    }
  }
#pragma unroll
  for (int m4 = 0; m4 < NM; m4++) red[((gl * kRq + kq) * NM + m4) * 64 + lane] = acc[m4];
  __syncthreads();
  for (int t = threadIdx.x; t < kRgpw * NM * 64; t += P::THREADS) {
    const int g2 = t / (NM * 64), m4 = (t >> 6) % NM, l = t & 63;
    double sum = 0.0;
#pragma unroll
    for (int q = 0; q < kRq; q++) sum += red[((g2 * kRq + q) * NM + m4) * 64 + l];
    const int b = 4 * m4 + (l >> 4), row = wg_row0 + g2 * kGRows + (l & 15);
    if (b < NB && row < wg_end) y[(size_t)b * out_dim + row] = (float)sum;
  }
}

template <int NB, int NBLK>
hipError_t run_q8r(const uint8_t* w, const float* x, float* y, int out_dim, hipStream_t s) {
  auto kern = mv_q8r<NB, NBLK>;
  constexpr size_t lds = Q8R<NB, NBLK>::lds;
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
  // rows spread evenly over the CUs (runs of at most 48 rows)
  const long cus = device_cu_count();
  const long wg0 = std::max<long>(1, std::min<long>(cus, (out_dim + kGRows - 1) / kGRows));
  const int rpw = (int)std::min<long>(kRgpw * kGRows, (out_dim + wg0 - 1) / wg0);
  const int grid = (out_dim + rpw - 1) / rpw;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(Q8R<NB, NBLK>::THREADS), lds, s, w, x, y, out_dim, rpw);
  return hipGetLastError();
}

template <int NBLK>
hipError_t q8r_nb(int nb, const uint8_t* w, const float* x, float* y, int out_dim, hipStream_t s) {
  switch (nb) {
    case 2: return run_q8r<2, NBLK>(w, x, y, out_dim, s);
    case 3: return run_q8r<3, NBLK>(w, x, y, out_dim, s);
    case 4: return run_q8r<4, NBLK>(w, x, y, out_dim, s);
    case 5: return run_q8r<5, NBLK>(w, x, y, out_dim, s);
    case 6: return run_q8r<6, NBLK>(w, x, y, out_dim, s);
    case 7: return run_q8r<7, NBLK>(w, x, y, out_dim, s);
    case 8: return run_q8r<8, NBLK>(w, x, y, out_dim, s);
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
    case 4096: return q8r_nb<128>((int)batch, w, x, y, (int)out_dim, s);
    case 2048: return q8r_nb<64>((int)batch, w, x, y, (int)out_dim, s);
    case 1024: return q8r_nb<32>((int)batch, w, x, y, (int)out_dim, s);
    default: return hipErrorNotSupported;
  }
}

}  // namespace ssdq
