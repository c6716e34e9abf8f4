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
#include <climits>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace ssdq {
namespace {

// ------------------------------------------------------------ unit geometry
// A "unit" is the slice of one row a lane owns:
//   Q4_K: two sub-blocks of one super-block (64 elements, one 16-byte header)
//   Q4_0 / Q8_0: two consecutive 18- / 34-byte blocks (64 elements, dword aligned)
//   Q6_K: a 32-element quarter of a 210-byte block
//   Q5_K (batch-1 kernel only): two sub-blocks (header, 8 high-bit bytes, 32 code bytes)
//   Q2_K (batch-1 kernel only): four 16-element sub-blocks (d|dmin, 4 scale bytes, 16 code bytes)
//   Q3_K (batch-1 kernel only): four 16-element sub-blocks (8 high-bit bytes, 16 code bytes, scales, d)
//   Q8_K (batch-1 kernel only): 64 int8 codes and the block's f32 scale
// E elements, NSUM x-sum groups of SUMG elements, NW dwords of raw data.
template <int F> struct FastUnit;
template <> struct FastUnit<kQ4_K> {
  static constexpr int E = 64, NSUM = 2, SUMG = 32, NW = 12;
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
template <> struct FastUnit<kQ5_K> {
  static constexpr int E = 64, NSUM = 2, SUMG = 32, NW = 14;
  static constexpr bool prescale = true;
};
template <> struct FastUnit<kQ2_K> {
  static constexpr int E = 64, NSUM = 4, SUMG = 16, NW = 6;
  static constexpr bool prescale = false;
};
template <> struct FastUnit<kQ3_K> {
  static constexpr int E = 64, NSUM = 4, SUMG = 16, NW = 12;
  static constexpr bool prescale = false;
};
template <> struct FastUnit<kQ8_K> {
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
    const uint8_t* blk = row + (size_t)(u >> 2) * 144;
    ld4(blk, raw);                          // d, dmin, scales[12]
    ld4(blk + 16 + 32 * (u & 3), raw + 4);  // qs of sub-block 2*(u&3)
    ld4(blk + 32 + 32 * (u & 3), raw + 8);  // qs of sub-block 2*(u&3)+1
  } else if constexpr (F == kQ5_K) {
    // block (compute.rs:855-860): d, dmin, scales[12] | qh[32] | ql[128]
    const uint8_t* blk = row + (size_t)(u >> 2) * 176;
    ld4(blk, raw);                          // d, dmin, scales[12]
    ld4(blk + 48 + 32 * (u & 3), raw + 4);  // low nibbles of sub-block 2*(u&3)
    ld4(blk + 64 + 32 * (u & 3), raw + 8);  // low nibbles of sub-block 2*(u&3)+1
    const uint2 h = *reinterpret_cast<const uint2*>(blk + 16 + 8 * (u & 3));  // high bits of the 64 elements
    raw[12] = h.x;
    raw[13] = h.y;
  } else if constexpr (F == kQ2_K) {
    // block (compute.rs:940-944): d, dmin | scales[16] | qs[64]; dword aligned
    const uint8_t* blk = row + (size_t)(u >> 2) * 84;
    raw[0] = ld1(blk);                       // d | dmin
    raw[1] = ld1(blk + 4 + 4 * (u & 3));     // scale|min bytes of sub-blocks 4*(u&3) .. +3
    ld4(blk + 20 + 16 * (u & 3), raw + 2);  // one code dword per 16-element sub-block
  } else if constexpr (F == kQ3_K) {
    // block (compute.rs:807-810): hmask[32] | qs[64] | scales[12] | d; 110 bytes,
    // 2-byte aligned: dwords are read from 0 or 2 bytes below and realigned
    const uint8_t* blk = row + (size_t)(u >> 2) * 110;
    const int j = u & 3;
    const uint32_t mis = (uint32_t)(uintptr_t)blk & 2u;  // 0 or 2
    ld3(blk + 8 * j - mis, raw);           // hmask[8j .. 8j+8) (+ slack)
    ld4(blk + 32 + 16 * j - mis, raw + 3);  // qs[16j .. 16j+16) (+ slack)
    raw[7] = ld1(blk + 48 + 16 * j - mis);
    raw[8] = ldh(blk + 96 + 2 * j) | (ldh(blk + 104 + (j & 2)) << 16);  // low-nibble scale bytes | high-bit bytes
    raw[9] = ldh(blk + 108);                                              // d
    raw[10] = mis * 8u;                                                   // realignment shift
    raw[11] = 0;
  } else if constexpr (F == kQ8_K) {
    // block (compute.rs:981-987): f32 d | int8 qs[256] | bsums (unused); dword aligned
    const uint8_t* blk = row + (size_t)(u >> 2) * 292;
    raw[0] = ld1(blk);
    const uint8_t* q = blk + 4 + 64 * (u & 3);
    ld4(q, raw + 1);
    ld4(q + 16, raw + 5);
    ld4(q + 32, raw + 9);
    ld4(q + 48, raw + 13);
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

// 4-bit codes of one dword: q[2i] = low nibble of byte i, q[2i+1] = 16 * high nibble
__device__ __forceinline__ void nibbles8(uint32_t w, float* q) {
  const uint32_t lo = opaque(w & 0x0F0F0F0Fu);
  const uint32_t hi = opaque(w & 0xF0F0F0F0u);  // x' of odd elements is x / 16
#pragma unroll
  for (int i = 0; i < 4; i++) {
    q[2 * i] = (float)byte_of(lo, i);
    q[2 * i + 1] = (float)byte_of(hi, i);
  }
}

// 6-bit scale / min of sub-block sb, branch-free form of the reference unpacking
// (compute.rs:724-731): sb < 4 -> low six bits of sc[sb] / sc[sb+4]; sb >= 4 ->
// bits 6-7 of sc[sb-4] / sc[sb] as the LOW two bits, sc[sb+4] nibbles as the high four.
__device__ __forceinline__ void q4k_sm(uint32_t sc1, uint32_t sc2, uint32_t sc3, int sb,
                                       float& s, float& m) {
  const uint32_t i = sb & 3, hi = sb >> 2;
  const uint32_t off = 8 * i + 6 * hi, wl = hi ? 2u : 6u, wh = hi ? 4u : 0u;
  const uint32_t si = __builtin_amdgcn_ubfe(sc1, off, wl) | (__builtin_amdgcn_ubfe(sc3, 8 * i, wh) << 2);
  const uint32_t mi = __builtin_amdgcn_ubfe(sc2, off, wl) | (__builtin_amdgcn_ubfe(sc3, 8 * i + 4, wh) << 2);
  s = (float)si;
  m = (float)mi;
}

// Decodes one unit into integer-valued floats (offsets folded out) and
// applies it to B activations.  xg(b, e): x' of element e of the unit;
// sg(b, g): sum of the raw x over sum-group g of the unit.
template <int F, int B, class XG, class SG>
__device__ __forceinline__ void accumulate(const uint32_t* raw, int u, XG xg, SG sg, float* acc) {
  constexpr int E = FastUnit<F>::E;
  float q[E];
  if constexpr (F == kQ4_K) {
#pragma unroll
    for (int k = 0; k < 8; k++) nibbles8(raw[4 + k], q + 8 * k);
  } else if constexpr (F == kQ4_0) {
#pragma unroll
    for (int k = 0; k < 4; k++) nibbles8(__builtin_amdgcn_alignbit(raw[k + 1], raw[k], 16), q + 8 * k);
#pragma unroll
    for (int k = 0; k < 4; k++) nibbles8(raw[5 + k], q + 32 + 8 * k);
  } else if constexpr (F == kQ8_0) {
#pragma unroll
    for (int c = 0; c < 16; c++) {
      const uint32_t src = c < 8 ? __builtin_amdgcn_alignbit(raw[c + 1], raw[c], 16) : raw[1 + c];
      const uint32_t v = opaque(src ^ 0x80808080u);  // code + 128
#pragma unroll
      for (int i = 0; i < 4; i++) q[4 * c + i] = (float)byte_of(v, i);
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
      const uint32_t ee = opaque((ql[k] & 0x0F0F0F0Fu) | he);         // q + 32, elements 8k+2i
      const uint32_t eo = opaque(((ql[k] >> 4) & 0x0F0F0F0Fu) | ho);  // elements 8k+2i+1
#pragma unroll
      for (int i = 0; i < 4; i++) {
        q[8 * k + 2 * i] = (float)byte_of(ee, i);
        q[8 * k + 2 * i + 1] = (float)byte_of(eo, i);
      }
    }
  }

  // per-half scale and offset: acc += sA * pA - oA * sum_A + sB * pB - oB * sum_B
  float sA, sB, oA, oB;
  if constexpr (F == kQ4_K) {
    const float d = f16_to_f32(raw[0] & 0xFFFFu), dmin = f16_to_f32(raw[0] >> 16);
    const int sb = 2 * (u & 3);
    float s0, m0, s1, m1;
    q4k_sm(raw[1], raw[2], raw[3], sb, s0, m0);
    q4k_sm(raw[1], raw[2], raw[3], sb + 1, s1, m1);
    sA = d * s0;
    sB = d * s1;
    oA = dmin * m0;
    oB = dmin * m1;
  } else if constexpr (F == kQ4_0) {
    sA = f16_to_f32(raw[0] & 0xFFFFu);
    sB = f16_to_f32(raw[4] >> 16);
    oA = 8.0f * sA;
    oB = 8.0f * sB;
  } else if constexpr (F == kQ8_0) {
    sA = f16_to_f32(raw[0] & 0xFFFFu);
    sB = f16_to_f32(raw[8] >> 16);
    oA = 128.0f * sA;
    oB = 128.0f * sB;
  } else {
    const float d = f16_to_f32(raw[8] >> 16);
    sA = d * (float)(int8_t)(raw[8] & 0xFFu);
    sB = d * (float)(int8_t)((raw[8] >> 8) & 0xFFu);
    oA = 32.0f * sA;
    oB = 32.0f * sB;
  }

#pragma unroll
  for (int b = 0; b < B; b++) {
    float pa = 0.f, pb = 0.f;
#pragma unroll
    for (int e = 0; e < E / 2; e++) pa = fmaf(q[e], xg(b, e), pa);
#pragma unroll
    for (int e = E / 2; e < E; e++) pb = fmaf(q[e], xg(b, e), pb);
    float a = fmaf(-oA, sg(b, 0), acc[b]);
    a = fmaf(-oB, sg(b, 1), a);
    a = fmaf(sA, pa, a);
    acc[b] = fmaf(sB, pb, a);
  }
}

template <int F>
__host__ __device__ constexpr size_t lds_floats(int U, int B) {
  return (size_t)B * U * (FastUnit<F>::E + 4) + (size_t)B * U * FastUnit<F>::NSUM;
}

// Stages x' (pre-scaled, per-unit padded) for B activations into LDS.
template <int F, int B>
__device__ __forceinline__ void stage_x(const float* __restrict__ x, int in_dim, int keff, int U,
                                        float* xs) {
  using FU = FastUnit<F>;
  constexpr int E = FU::E, ES = E + 4;
  const int n4 = keff >> 2;  // keff is a multiple of 32
  for (int i = threadIdx.x; i < B * n4; i += blockDim.x) {
    const int b = i / n4, e = (i - b * n4) * 4;
    float4 v = *reinterpret_cast<const float4*>(x + (size_t)b * in_dim + e);
    if (FU::prescale) {  // elements e+1, e+3 are odd
      v.y *= 0.0625f;
      v.w *= 0.0625f;
    }
    const int u = e / E, t = e - u * E;
    *reinterpret_cast<float4*>(xs + ((size_t)b * U + u) * ES + t) = v;
  }
}

// ---------------------------------------------------------- batch 1 path
// Integer dot products on "digit planes" of x.  Each 32-element group of x is
// scaled by a power of two so its largest magnitude sits just under 2^30 and
// rounded to an integer xi (|xi| <= 2^30: the rounding error is at most 2^-31
// of the group maximum, so an element 2^k below its group's largest keeps
// 30 - k bits; with 22 bits, a group holding a channel 10^4 times the rest put
// some Llama-shaped outputs outside the stated tolerance).  xi is written in
// kDigits = 4 balanced base-256 digits (signed bytes), and the digits of the
// elements that meet one weight dword are packed into "planes" of four bytes.
// A weight dword of 4-bit codes then costs two masks and eight v_dot4_i32_i8;
// the four per-digit integer sums of a group are recombined (I0 + 256 I1
// exactly in int, then 2^16 I2 and 2^24 I3 in two fp32 FMAs), and scaled by
// the group's power of two.  Per element this is ~2 VALU instructions instead
// of a float conversion plus an FMA.  Each group's term (exact integer sum x
// scales) and a lane's running sum are taken in double precision, and so is
// the cross-lane row sum: with terms of very different sizes (massive
// activation channels) an output that cancels to a small value keeps its
// accuracy, where fp32 partial sums would each round at the terms' size.
//
// Group record in LDS (GW dwords): 32 plane dwords [k][parity][digit] for the
// four 8-element weight dwords k (parity 0 = elements 8k+0,2,4,6, parity 1 =
// 8k+1,3,5,7; Q8_0 instead uses elements 8k+0..3 / 8k+4..7), then at kDigScale
// the scale 2^-sh and at kDigSum the sum of the group's integers xi as a double
// (exact: below 2^36; two half sums for the 16-element scales of Q6_K / Q2_K
// / Q3_K, the second at kDigSum + 2).  A group's term is then 2^-sh (S F - M
// X) with F its digit sum and X that sum, both exact: the offset term uses
// the same rounded x as the codes' term.
constexpr int kDigits = 4;
constexpr int kDigScale = 8 * kDigits, kDigSum = kDigScale + 1;
// A unit's record holds NG group records of GW dwords; records of consecutive
// units are US dwords apart, 4 more than NG GW: every lane reads its own
// unit's record with 16-byte LDS loads, and a stride of 72 or 40 dwords (8 mod
// 32) put lanes l and l + 4 on the same banks, a 2-way conflict over the ~18
// KB each row wave reads before its first row.  Strides of 76, 44 and 84
// dwords (12, 12 and 20 mod 32) give any 8 consecutive lanes distinct banks
// (the readers load the 4 padding dwords too: trimming them measured no
// faster).  Measured (row-slot kernels, A/B, two runs): 14336 x 4096 Q4_K 8.16-8.25 ->
// 7.71-7.89 us, 4096 x 4096 Q4_0 4.46 -> 4.38 us, 4096 x 14336 Q4_K 10.67 ->
// 10.35 us, the decode layer 54.0 -> 52.9 us.
template <int F> struct Dig;
template <> struct Dig<kQ4_K> { static constexpr int NG = 2, GW = 36, US = 76; static constexpr bool contig = false; };
template <> struct Dig<kQ4_0> { static constexpr int NG = 2, GW = 36, US = 76; static constexpr bool contig = false; };
template <> struct Dig<kQ5_K> { static constexpr int NG = 2, GW = 36, US = 76; static constexpr bool contig = false; };
template <> struct Dig<kQ8_0> { static constexpr int NG = 2, GW = 36, US = 76; static constexpr bool contig = true; };
template <> struct Dig<kQ8_K> { static constexpr int NG = 2, GW = 36, US = 76; static constexpr bool contig = true; };
template <> struct Dig<kQ6_K> { static constexpr int NG = 1, GW = 40, US = 44; static constexpr bool contig = false; };
// Q2_K: a group record holds two 16-element sub-blocks, each as 4 phase planes
// (elements p, p+4, p+8, p+12: the bytes a code dword yields for shift 2p) x 4
// digits, then the scale and the two sub-block sums as for Q6_K.
template <> struct Dig<kQ2_K> { static constexpr int NG = 2, GW = 40, US = 84; static constexpr bool contig = false; };
template <> struct Dig<kQ3_K> { static constexpr int NG = 2, GW = 40, US = 84; static constexpr bool contig = false; };

// A double kept in two dwords of a group record.
__device__ __forceinline__ double pair_value(uint32_t lo, uint32_t hi) {
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ void pair_store(uint32_t* p, double d) {
  const uint64_t b = __builtin_bit_cast(uint64_t, d);
  p[0] = (uint32_t)b;
  p[1] = (uint32_t)(b >> 32);
}

// Staging of x in two phases so the x loads can be issued before the weight
// prefetch: vector loads return in order, so x fetched after the weights would
// wait for them.  One thread per 8 elements (the four threads of a 32-element
// group are adjacent lanes); each thread holds up to kStageIt chunks.
constexpr int kStageIt = 4;  // largest chunk count per thread the kernels instantiate

template <int SIT>
struct XChunks {
  float v[SIT][8];
};

// rows > 1: the chunks of rows x rows of x (row stride x_stride floats) form
// one sequence (a row's chunk count is a multiple of 4, so no 32-element group
// straddles two rows).
template <int SIT>
__device__ __forceinline__ void stage_load(const float* __restrict__ x, int keff, XChunks<SIT>& st,
                                           int nthreads, int rows = 1, size_t x_stride = 0) {
  const int nchunk = keff >> 3, total = rows * nchunk;
#pragma unroll
  for (int it = 0; it < SIT; it++) {
    const int c = it * nthreads + threadIdx.x;
    if (c < total) {
      const int r = rows > 1 ? c / nchunk : 0, cc = c - r * nchunk;
      const float* xp = x + (size_t)r * x_stride + 8 * cc;
      const float4 a = *reinterpret_cast<const float4*>(xp);
      const float4 b = *reinterpret_cast<const float4*>(xp + 4);
      st.v[it][0] = a.x; st.v[it][1] = a.y; st.v[it][2] = a.z; st.v[it][3] = a.w;
      st.v[it][4] = b.x; st.v[it][5] = b.y; st.v[it][6] = b.z; st.v[it][7] = b.w;
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) st.v[it][j] = 0.f;
    }
  }
}

// rows > 1: row r's planes start lds_stride dwords after row r-1's.
template <int F, int SIT>
__device__ __forceinline__ void stage_store(const XChunks<SIT>& st, int keff, uint32_t* lds, int nthreads,
                                            int rows = 1, int lds_stride = 0) {
  using D = Dig<F>;
  const int nchunk = keff >> 3, total = rows * nchunk;
#pragma unroll
  for (int it = 0; it < SIT; it++) {
    if (it * nthreads >= total) break;  // uniform across the staging waves
    const int c0 = it * nthreads + threadIdx.x;
    const bool live = c0 < total;
    const int r = rows > 1 ? c0 / nchunk : 0, c = c0 - r * nchunk;
    const float* v = st.v[it];
    float m = 0.f, z = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      m = fmaxf(m, fabsf(v[j]));
      z = fmaf(v[j], 0.f, z);  // NaN when an element is NaN or infinite
    }
    m = fmaxf(m, dpp_mov<0xB1>(m));
    m = fmaxf(m, dpp_mov<0x4E>(m));
    z += dpp_mov<0xB1>(z);  // the group's four chunks
    z += dpp_mov<0x4E>(z);
    const int k = c & 3;
    int e = 0;
    if (m > 0.f) (void)frexpf(m, &e);  // m < 2^e
    // the value is scaled, not multiplied by 2^(30 - e): that factor overflows
    // for groups whose largest magnitude is below 2^-97; and the shift stops
    // at 149, so that the scale 2^-sh stays a (subnormal) fp32 value: groups
    // below 2^-119 keep fp32's subnormal resolution instead
    const int sh = min(30 - e, 149);
    uint32_t u[8];
    double s = 0.0;  // the chunk's integers, summed exactly
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int xi = (int)rintf(ldexpf(v[j], sh));  // |xi| <= 2^30
      s += (double)xi;
      // xi + 0x80808080 lies in [0, 2^32): its bytes are the balanced digits + 128
      u[j] = ((uint32_t)xi + 0x80808080u) ^ 0x80808080u;
    }
    const double s_half = s + dpp_mov_d<0xB1>(s);  // sum over this 16-element half of the group
    s = s_half + dpp_mov_d<0x4E>(s_half);
    const bool gbad = z != z;
    if (live) {
      const int g = c >> 2;
      uint32_t* rec = lds + (size_t)r * lds_stride + (size_t)(g / D::NG) * D::US + (g % D::NG) * D::GW;
      uint32_t* pl = rec + 2 * kDigits * k;
      if constexpr (F == kQ2_K || F == kQ3_K) {
        // chunk k is half k & 1 of sub-block k >> 1: bytes 2 (k & 1), +1 of its
        // phase planes (elements p and p + 4 of this chunk)
        uint16_t* pb = reinterpret_cast<uint16_t*>(rec + 4 * kDigits * (k >> 1)) + (k & 1);
#pragma unroll
        for (int ph = 0; ph < 4; ph++)
#pragma unroll
          for (int d = 0; d < kDigits; d++)
            pb[2 * (kDigits * ph + d)] =
                (uint16_t)__builtin_amdgcn_perm(u[4 + ph], u[ph], (uint32_t)d | ((uint32_t)(4 + d) << 8) | 0x0C0C0000u);
      } else {
        static_assert(kDigits == 4, "one 4 x 4 byte transpose per half chunk");
        uint32_t p0[4], p1[4];
        if (D::contig) {
          planes4(u[0], u[1], u[2], u[3], p0);
          planes4(u[4], u[5], u[6], u[7], p1);
        } else {
          planes4(u[0], u[2], u[4], u[6], p0);
          planes4(u[1], u[3], u[5], u[7], p1);
        }
#pragma unroll
        for (int d = 0; d < kDigits; d++) {
          pl[d] = p0[d];
          pl[kDigits + d] = p1[d];
        }
      }
      constexpr bool halves = D::GW == 40;  // two 16-element sums per record
      if (k == 0) {
        // a non-finite input poisons its group's result instead of being rounded
        rec[kDigScale] = __float_as_uint(gbad ? __builtin_nanf("") : ldexpf(1.0f, -sh));
        pair_store(rec + kDigSum, halves ? s_half : s);
      }
      if (halves && k == 2) pair_store(rec + kDigSum + 2, s_half);
    }
  }
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// I0 + 256 I1 + 2^16 (I2 + 256 I3), exactly (|I1|, |I3| < 2^20, so the pairs
// combine exactly in int; the whole stays below 2^53)
__device__ __forceinline__ double digits_value(int i0, int i1, int i2, int i3) {
  return fma(65536.0, (double)(i2 + (i3 << 8)), (double)(i0 + (i1 << 8)));
}

// Applies one unit (raw weight dwords) to x given as digit planes pl[] (the
// unit's US dwords).
// The fifth bits of a Q5_K weight dword's 8 elements (bits 0-7 of one qh byte,
// element 2i at bit 2i) as bit 4 of four bytes, for the even (elements 0, 2,
// 4, 6) and the odd elements.  A 24-bit multiply spreads the four bits: the
// copies of the byte land 6 bits apart, so each target bit 8j+4 receives only
// bit 2j (2j+1) and the carries where copies overlap stay below it.
__device__ __forceinline__ uint32_t q5_high_even(uint32_t hb) {
  return __umul24(hb & 0x55u, 0x00410410u) & 0x10101010u;
}
__device__ __forceinline__ uint32_t q5_high_odd(uint32_t hb) {
  return __umul24(hb & 0xAAu, 0x00208208u) & 0x10101010u;
}

template <int F, class PL>
__device__ __forceinline__ void accumulate_dig(const uint32_t* raw, int u, PL pl, double& acc) {
  using D = Dig<F>;
  if constexpr (F == kQ4_K || F == kQ4_0 || F == kQ5_K) {
    float sc[2], off[2];
    if constexpr (F == kQ4_K || F == kQ5_K) {
      const float d = f16_to_f32(raw[0] & 0xFFFFu), dmin = f16_to_f32(raw[0] >> 16);
      const int sb = 2 * (u & 3);
#pragma unroll
      for (int h = 0; h < 2; h++) {
        float s, m;
        q4k_sm(raw[1], raw[2], raw[3], sb + h, s, m);
        sc[h] = d * s;
        off[h] = dmin * m;  // acc += S * sum(q x) - M * sum(x)
      }
    } else {
      sc[0] = f16_to_f32(raw[0] & 0xFFFFu);
      sc[1] = f16_to_f32(raw[4] >> 16);
      off[0] = 8.0f * sc[0];  // value (q - 8) d
      off[1] = 8.0f * sc[1];
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
      int i0 = 0, i1 = 0, i2 = 0, i3 = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t wd;
        if constexpr (F == kQ4_K || F == kQ5_K) wd = raw[4 + 4 * h + k];
        else wd = h == 0 ? __builtin_amdgcn_alignbit(raw[k + 1], raw[k], 16) : raw[5 + k];
        uint32_t lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;
        if constexpr (F == kQ5_K) {  // codes 0..31 (compute.rs:882-892)
          const uint32_t hb = raw[12 + h] >> (8 * k);
          lo |= q5_high_even(hb);
          hi |= q5_high_odd(hb);
        }
        const int b = h * D::GW + 2 * kDigits * k;
        i0 = dot4(lo, pl(b + 0), i0);
        i1 = dot4(lo, pl(b + 1), i1);
        i2 = dot4(lo, pl(b + 2), i2);
        i3 = dot4(lo, pl(b + 3), i3);
        i0 = dot4(hi, pl(b + 4), i0);
        i1 = dot4(hi, pl(b + 5), i1);
        i2 = dot4(hi, pl(b + 6), i2);
        i3 = dot4(hi, pl(b + 7), i3);
      }
      // the scales d * s, dmin * m are exact products of fp32 values
      const double xs = pair_value(pl(h * D::GW + kDigSum), pl(h * D::GW + kDigSum + 1));
      const double t = fma((double)sc[h], digits_value(i0, i1, i2, i3), -(double)off[h] * xs);
      acc = fma(t, (double)__uint_as_float(pl(h * D::GW + kDigScale)), acc);
    }
  } else if constexpr (F == kQ8_0) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const float d = h == 0 ? f16_to_f32(raw[0] & 0xFFFFu) : f16_to_f32(raw[8] >> 16);
      int i0 = 0, i1 = 0, i2 = 0, i3 = 0;
#pragma unroll
      for (int c = 0; c < 8; c++) {
        const uint32_t wd = h == 0 ? __builtin_amdgcn_alignbit(raw[c + 1], raw[c], 16) : raw[9 + c];
        const int b = h * D::GW + 2 * kDigits * (c >> 1) + kDigits * (c & 1);
        i0 = dot4(wd, pl(b + 0), i0);
        i1 = dot4(wd, pl(b + 1), i1);
        i2 = dot4(wd, pl(b + 2), i2);
        i3 = dot4(wd, pl(b + 3), i3);
      }
      const double xscale = (double)__uint_as_float(pl(h * D::GW + kDigScale));
      acc = fma((double)d, digits_value(i0, i1, i2, i3) * xscale, acc);
    }
  } else if constexpr (F == kQ8_K) {
    const float d = __uint_as_float(raw[0]);
#pragma unroll
    for (int h = 0; h < 2; h++) {
      int i0 = 0, i1 = 0, i2 = 0, i3 = 0;
#pragma unroll
      for (int c = 0; c < 8; c++) {
        const uint32_t wd = raw[1 + 8 * h + c];
        const int b = h * D::GW + 2 * kDigits * (c >> 1) + kDigits * (c & 1);
        i0 = dot4(wd, pl(b + 0), i0);
        i1 = dot4(wd, pl(b + 1), i1);
        i2 = dot4(wd, pl(b + 2), i2);
        i3 = dot4(wd, pl(b + 3), i3);
      }
      const double xscale = (double)__uint_as_float(pl(h * D::GW + kDigScale));
      acc = fma((double)d, digits_value(i0, i1, i2, i3) * xscale, acc);
    }
  } else if constexpr (F == kQ2_K) {
    // 16 sub-blocks of 16 elements; scale / min = low / high nibble of the
    // sub-block's byte (compute.rs:948-960): value d*s*q - dmin*m
    const float d = f16_to_f32(raw[0] & 0xFFFFu), dmin = f16_to_f32(raw[0] >> 16);
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const double xscale = (double)__uint_as_float(pl(h * D::GW + kDigScale));
#pragma unroll
      for (int sb = 0; sb < 2; sb++) {
        const uint32_t wd = raw[2 + 2 * h + sb];
        const uint32_t scb = (raw[1] >> (8 * (2 * h + sb))) & 0xFFu;
        int i0 = 0, i1 = 0, i2 = 0, i3 = 0;
#pragma unroll
        for (int ph = 0; ph < 4; ph++) {
          const uint32_t q = (wd >> (2 * ph)) & 0x03030303u;
          const int b = h * D::GW + 4 * kDigits * sb + kDigits * ph;
          i0 = dot4(q, pl(b + 0), i0);
          i1 = dot4(q, pl(b + 1), i1);
          i2 = dot4(q, pl(b + 2), i2);
          i3 = dot4(q, pl(b + 3), i3);
        }
        const float S = d * (float)(scb & 15u), Mn = dmin * (float)(scb >> 4);  // exact products
        const double xs = pair_value(pl(h * D::GW + kDigSum + 2 * sb), pl(h * D::GW + kDigSum + 2 * sb + 1));
        acc = fma(fma((double)S, digits_value(i0, i1, i2, i3), -(double)Mn * xs), xscale, acc);
      }
    }
  } else if constexpr (F == kQ3_K) {
    // 3-bit codes q = low2 | hbit << 2, value d * scale * (q - 4) with a
    // signed 6-bit scale (compute.rs:813-833): sum = S (sum q x - 4 sum x)
    const uint32_t sh = raw[10];
    const uint32_t hm0 = __builtin_amdgcn_alignbit(raw[1], raw[0], sh);
    const uint32_t hm1 = __builtin_amdgcn_alignbit(raw[2], raw[1], sh);
    uint32_t qd[4];
#pragma unroll
    for (int k = 0; k < 4; k++) qd[k] = __builtin_amdgcn_alignbit(raw[4 + k], raw[3 + k], sh);
    const float d = f16_to_f32(raw[9] & 0xFFFFu);
    const int j = u & 3;
    const uint32_t hi2byte = (raw[8] >> (16 + 8 * (j & 1))) & 0xFFu;  // scales[8 + j]
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const double xscale = (double)__uint_as_float(pl(h * D::GW + kDigScale));
#pragma unroll
      for (int sb = 0; sb < 2; sb++) {
        const int s4 = 2 * h + sb;  // sub-block 4j + s4
        // high bits of its 16 elements: bytes 2 s4, 2 s4 + 1 of hmask[8j ..]
        const uint32_t hw = ((s4 < 2 ? hm0 : hm1) >> (16 * (s4 & 1))) & 0xFFFFu;
        // bytes: A, A >> 4, B, B >> 4 (A, B the two hmask bytes): bit p of
        // byte i is the high bit of element 4 i + p
        const uint32_t nib = (hw >> 4) & 0x0F0Fu;
        const uint32_t hr = __builtin_amdgcn_perm(nib, hw, 0x05010400u);
        int i0 = 0, i1 = 0, i2 = 0, i3 = 0;
#pragma unroll
        for (int ph = 0; ph < 4; ph++) {
          const uint32_t q = ((qd[s4] >> (2 * ph)) & 0x03030303u) | (((hr >> ph) & 0x01010101u) << 2);
          const int b = h * D::GW + 4 * kDigits * sb + kDigits * ph;
          i0 = dot4(q, pl(b + 0), i0);
          i1 = dot4(q, pl(b + 1), i1);
          i2 = dot4(q, pl(b + 2), i2);
          i3 = dot4(q, pl(b + 3), i3);
        }
        const uint32_t lo4 = (raw[8] >> (8 * h + 4 * sb)) & 15u;  // scales[2j + h] nibble sb
        const uint32_t hi2 = (hi2byte >> (2 * s4)) & 3u;
        const int sv = (int)((lo4 | (hi2 << 4)) ^ 32u) - 32;  // sign-extended 6 bits
        const float S = d * (float)sv;  // exact product
        const double xs = pair_value(pl(h * D::GW + kDigSum + 2 * sb), pl(h * D::GW + kDigSum + 2 * sb + 1));
        acc = fma((double)S * fma(-4.0, xs, digits_value(i0, i1, i2, i3)), xscale, acc);
      }
    }
  } else {  // kQ6_K quarter: 6-bit codes + 32 as bytes, two 16-element scale groups
    const uint32_t sh = raw[9];
    uint32_t ql[4], qh[2];
#pragma unroll
    for (int k = 0; k < 4; k++) ql[k] = __builtin_amdgcn_alignbit(raw[k + 1], raw[k], sh);
#pragma unroll
    for (int j = 0; j < 2; j++) qh[j] = __builtin_amdgcn_alignbit(raw[6 + j], raw[5 + j], sh);
    const float d = f16_to_f32(raw[8] >> 16);
    const double xscale = (double)__uint_as_float(pl(kDigScale));
#pragma unroll
    for (int h = 0; h < 2; h++) {
      int i0 = 0, i1 = 0, i2 = 0, i3 = 0;
#pragma unroll
      for (int kk = 0; kk < 2; kk++) {
        const int k = 2 * h + kk;
        const uint32_t p =
            __builtin_amdgcn_perm(qh[k >> 1], qh[k >> 1], (k & 1) ? 0x03030202u : 0x01010000u);
        const uint32_t he = ((p << 4) & 0x00300030u) | (p & 0x30003000u);
        const uint32_t ho = ((p << 2) & 0x00300030u) | ((p >> 2) & 0x30003000u);
        const uint32_t ee = (ql[k] & 0x0F0F0F0Fu) | he;
        const uint32_t eo = ((ql[k] >> 4) & 0x0F0F0F0Fu) | ho;
        const int b = 2 * kDigits * k;
        i0 = dot4(ee, pl(b + 0), i0);
        i1 = dot4(ee, pl(b + 1), i1);
        i2 = dot4(ee, pl(b + 2), i2);
        i3 = dot4(ee, pl(b + 3), i3);
        i0 = dot4(eo, pl(b + 4), i0);
        i1 = dot4(eo, pl(b + 5), i1);
        i2 = dot4(eo, pl(b + 6), i2);
        i3 = dot4(eo, pl(b + 7), i3);
      }
      const float sg = d * (float)(int8_t)((raw[8] >> (8 * h)) & 0xFFu);  // exact product
      const double xs = pair_value(pl(kDigSum + 2 * h), pl(kDigSum + 2 * h + 1));
      acc = fma((double)sg * fma(-32.0, xs, digits_value(i0, i1, i2, i3)), xscale, acc);
    }
  }
}

// Barrier for LDS data only.  __syncthreads() also orders global memory, which
// makes every wave wait for all of its outstanding weight loads first.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Vector memory instructions one load_unit issues.
template <int F> constexpr int loads_per_unit() {
  return (F == kQ4_K || F == kQ4_0 || F == kQ2_K) ? 3 : F == kQ5_K ? 4 : F == kQ3_K ? 6 : 5;  // Q8_0 / Q8_K / Q6_K: 5
}

// rows whose weight loads are in flight at once in a wave (measured at
// 14336 x 4096 Q4_K: depth 1 9.8 us, 2 8.5 us, 3 9.2 us, 5 11.2 us)
template <int RMAX> constexpr int kB1Depth = RMAX < 2 ? RMAX : 2;

// RMSNorm of the staged x (the norm-fused decode-layer launches): h = x (+ the
// residual), x' = h * inv_rms * w with inv_rms = 1 / sqrt(mean(h^2) + eps),
// the sum of squares reduced over the staging threads (each workgroup computes
// the same value: the same data in the same order).  Workgroup 0 writes h and
// x'.  norm_sumsq forms h in place and returns the thread's sum of squares;
// norm_apply scales by inv_rms and the norm weights.
template <int SIT, bool RES>
__device__ __forceinline__ float norm_sumsq(XChunks<SIT>& st, const XChunks<SIT>& st_r) {
  float q = 0.f;
#pragma unroll
  for (int it = 0; it < SIT; it++)
#pragma unroll
    for (int j = 0; j < 8; j++) {
      if (RES) st.v[it][j] = st.v[it][j] + st_r.v[it][j];
      q = fmaf(st.v[it][j], st.v[it][j], q);  // chunks past the end are zeros
    }
  return q;
}

template <int SIT>
__device__ __forceinline__ void norm_apply(XChunks<SIT>& st, const XChunks<SIT>& st_w, float inv, int keff,
                                           int nthreads, const MatvecFuse& fu) {
  const int nchunk = keff >> 3;
#pragma unroll
  for (int it = 0; it < SIT; it++) {
    const int c = it * nthreads + (int)threadIdx.x;
    const bool live = c < nchunk;
    float h[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      h[j] = st.v[it][j];
      st.v[it][j] = h[j] * inv * st_w.v[it][j];
    }
    if (blockIdx.x == 0 && live) {
      if (fu.hidden_out) {
        *reinterpret_cast<float4*>(fu.hidden_out + 8 * c) = make_float4(h[0], h[1], h[2], h[3]);
        *reinterpret_cast<float4*>(fu.hidden_out + 8 * c + 4) = make_float4(h[4], h[5], h[6], h[7]);
      }
      if (fu.xn_out) {
        const float* v = st.v[it];
        *reinterpret_cast<float4*>(fu.xn_out + 8 * c) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(fu.xn_out + 8 * c + 4) = make_float4(v[4], v[5], v[6], v[7]);
      }
    }
  }
}

// The norm over every thread of the workgroup (mv_b1: all waves stage x).
template <int SIT, bool RES>
__device__ __forceinline__ void stage_norm(XChunks<SIT>& st, const XChunks<SIT>& st_r, const XChunks<SIT>& st_w,
                                           int keff, const MatvecFuse& fu) {
  __shared__ float part[16];
  const float q = wave_sum(norm_sumsq<SIT, RES>(st, st_r));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (lane == 0) part[wave] = q;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; i++) t += part[i];
  norm_apply<SIT>(st, st_w, 1.0f / sqrtf(t / (float)keff + fu.norm_eps), keff, (int)blockDim.x, fu);
}

// Decode-layer fusion of the batch-1 kernel (FUSE = true).  Up to three
// weight matrices of one type and row length share x ("segments", virtual
// rows concatenated; for SwiGLU the rows of gate and up alternate).  Row runs
// are handed out in pairs so each wave finishes both rows of a RoPE pair or of
// a (gate, up) pair in its epilogue.  (An RMSNorm of x folded into the staging
// measured slower than a separate norm kernel: the norm weights queue ahead of
// every workgroup's first weight rows.)
// The plain kernel takes an empty argument in the fuse descriptor's place.
struct NoFuse {};
// FUSE: 0 plain; 2 segments in row pairs with the RoPE / SwiGLU epilogue; 3
// and 4 the same with an RMSNorm of x (4: of x + a residual) in the staging.
template <int FUSE> using FuseArg = typename std::conditional<FUSE != 0, MatvecFuse, NoFuse>::type;

__device__ __forceinline__ int fuse_seg(const MatvecFuse& f, int v, int& r) {
  if (f.swiglu) {
    r = v >> 1;
    return v & 1;
  }
  const int sg = (v >= f.start1 ? 1 : 0) + (v >= f.start2 ? 1 : 0);
  r = v - (sg == 0 ? 0 : sg == 1 ? f.start1 : f.start2);
  return sg;
}

// Epilogue of the row pair at virtual rows v, v + 1 with dot products a0, a1:
// silu(gate) * up, or the two outputs, rotated when their segment is in
// rope_mask (rows r, r + 1 are pair i of a head).
__device__ __forceinline__ void fuse_store_pair(const MatvecFuse& fu, int v, float a0, float a1) {
  int r;
  const int sg = fuse_seg(fu, v, r);
  if (fu.swiglu) {
    fu.y0[r] = (a0 / (1.0f + expf(-a0))) * a1;
    return;
  }
  float o0 = a0, o1 = a1;
  if ((fu.rope_mask >> sg) & 1u) {
    const int i = (r % fu.head_dim) >> 1;
    const float sn = fu.rope.sn[i], cs = fu.rope.cs[i];
    o0 = a0 * cs - a1 * sn;
    o1 = a0 * sn + a1 * cs;
  }
  float* yo = sg == 0 ? fu.y0 : sg == 1 ? fu.y1 : fu.y2;
  yo[r] = o0;
  yo[r + 1] = o1;
}

// Every lane keeps the digit planes of its units in registers.  KS waves split
// each row's units (KS > 1 for long rows; partial sums meet in LDS); the
// workgroup's other waves take other rows.  Rows are spread evenly over all
// row streams of the grid (at most RMAX per stream).  One workgroup runs per
// CU.
//
// Schedule, from timelines of the kernel phases on MI355X (vector memory
// returns in order per wave, and a wave stalls at issue when the memory
// pipeline is full):
//   1. x and the first row are requested.  More weight traffic ahead of x
//      delays x, and nothing can be computed before x is staged.
//   2. When x has arrived, the second row is requested, then x is turned into
//      digit planes in LDS (LDS-only barrier: the weight loads stay in flight).
//   3. Each row is computed while the next one is in flight (lookahead 1; a
//      deeper lookahead stalls the issuing wave).  Rows are computed in
//      straight-line code with clamped addresses, so the compiler's in-order
//      wait counts stay exact, and the cross-lane sums of all rows are taken
//      together at the end.
//
// Long rows are cut into K slices (blockIdx.y; slice_bpr blocks each, the last
// one may be shorter): every workgroup stages only its slice of x, and slice z
// writes its partial dot products to y + z * out_dim, summed by
// slice_reduce_kernel in slice order.
template <int F, int UPL, int RMAX, bool FULL, int SIT, int FUSE = 0>
__global__ __launch_bounds__(768) void mv_b1(const uint8_t* __restrict__ w,
                                             const float* __restrict__ x, float* __restrict__ y,
                                             int out_dim, int row_bpr, int slice_bpr, int ks,
                                             bool interleave, FuseArg<FUSE> fu) {
  static_assert(FUSE < 2 || RMAX % 2 == 0, "fused rows come in pairs");
  using FU = FastUnit<F>;
  using D = Dig<F>;
  constexpr int NW = FU::NW, US = D::US;
  static_assert(US % 4 == 0, "unit records are read as 16-byte vectors");
  extern __shared__ uint4 lds4[];
  uint32_t* lds = reinterpret_cast<uint32_t*>(lds4);
  const int blk0 = blockIdx.y * slice_bpr;
  const int bpr = min(slice_bpr, row_bpr - blk0);  // blocks of this slice
  w += (size_t)blk0 * Geom<F>::bb;
  x += (size_t)blk0 * Geom<F>::bs;
  // slice z of a K-sliced row writes its partial sums as doubles to
  // ((double*)y)[z * out_dim + row] (the slice reduction adds them in order)
  const bool sliced = gridDim.y > 1;
  double* yp = reinterpret_cast<double*>(y) + (size_t)blockIdx.y * out_dim;
  const int keff = bpr * Geom<F>::bs;
  const int U = keff / FU::E;
  double* red = reinterpret_cast<double*>(lds + (size_t)U * US);  // [stream][RMAX][ks]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6, kw = wave % ks, stream = wave / ks, rs = nw / ks;
  const size_t row_bytes = (size_t)row_bpr * Geom<F>::bb;
  const long n_streams = (long)gridDim.x * rs, gs = (long)blockIdx.x * rs + stream;
  // Rows of a stream are either one contiguous run or, interleaved, rows
  // gs, gs + n_streams, ... (all waves then sweep the matrix together).
  int r_begin, r_step, n_rows;  // n_rows <= RMAX either way
  if (FUSE >= 2) {  // runs of row pairs
    const long P = out_dim / 2;
    const long p0 = gs * P / n_streams, p1 = (gs + 1) * P / n_streams;
    r_begin = (int)(2 * p0);
    r_step = 1;
    n_rows = (int)(2 * (p1 - p0));
  } else if (interleave) {
    r_begin = (int)gs;
    r_step = (int)n_streams;
    n_rows = gs < out_dim ? (int)((out_dim - 1 - gs) / n_streams) + 1 : 0;
  } else {
    r_begin = (int)(gs * out_dim / n_streams);
    r_step = 1;
    n_rows = (int)((gs + 1) * out_dim / n_streams) - r_begin;
  }
  const int ubase = kw * 64 * UPL + lane;
  // The segments' weight pointers as a base and two offsets: selecting an
  // offset per row is register arithmetic, where a select of the three
  // pointers is compiled as an indexed load of the kernel argument.
  [[maybe_unused]] const uint8_t* fw0 = nullptr;
  [[maybe_unused]] ptrdiff_t fd1 = 0, fd2 = 0;
  if constexpr (FUSE >= 2) {
    fw0 = fu.w0;
    fd1 = fu.w1 - fu.w0;
    fd2 = fu.w2 - fu.w0;
  }

  uint32_t buf[RMAX][UPL][NW];
  auto load_row = [&](int rr) {
    const int row = max(0, min(r_begin + rr * r_step, out_dim - 1));
    const uint8_t* rp;
    if constexpr (FUSE >= 2) {
      // The row is wave-uniform: taken as a scalar, the segment's weight
      // pointer is scalar arithmetic.  A load of the pointer would need a
      // wait that drains the rows still in flight.
      int r;
      const int sg = fuse_seg(fu, __builtin_amdgcn_readfirstlane(row), r);
      rp = fw0 + (sg == 0 ? 0 : sg == 1 ? fd1 : fd2) + (size_t)r * row_bytes;
    } else {
      rp = w + (size_t)row * row_bytes;
    }
#pragma unroll
    for (int i = 0; i < UPL; i++) {
      const int u = ubase + 64 * i;
      if (FULL || u < U) load_unit<F>(rp, u, buf[rr][i]);
    }
  };

  XChunks<SIT> st;
  stage_load<SIT>(x, keff, st, blockDim.x);  // 1.
  [[maybe_unused]] XChunks<SIT> st_r, st_w;
  if constexpr (FUSE >= 3) {  // the norm's operands, also before any weight
    if constexpr (FUSE == 4) stage_load<SIT>(fu.norm_res, keff, st_r, blockDim.x);
    stage_load<SIT>(fu.norm_w, keff, st_w, blockDim.x);
  }
#pragma unroll
  for (int rr = 0; rr < kB1Depth<RMAX>; rr++) load_row(rr);
  {
    // 2. wait for x only (the weight loads issued after it may stay in flight)
    constexpr int N = kB1Depth<RMAX> * UPL * loads_per_unit<F>();
    static_assert(N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  }
  if constexpr (FUSE >= 3) stage_norm<SIT, FUSE == 4>(st, st_r, st_w, keff, fu);
  stage_store<F, SIT>(st, keff, lds, blockDim.x);
  lds_barrier();

  uint32_t pr[UPL][US];
#pragma unroll
  for (int i = 0; i < UPL; i++) {
    const int u = ubase + 64 * i;
    const bool ok = FULL || u < U;
#pragma unroll
    for (int t = 0; t < US; t += 4) {
      const uint4 v = ok ? lds4[(size_t)u * (US / 4) + t / 4] : make_uint4(0, 0, 0, 0);
      pr[i][t] = v.x; pr[i][t + 1] = v.y; pr[i][t + 2] = v.z; pr[i][t + 3] = v.w;
    }
  }

  double acc[RMAX];
#pragma unroll
  for (int rr = 0; rr < RMAX; rr++) {  // 3.
    if (rr >= 1 && rr + kB1Depth<RMAX> - 1 < RMAX) load_row(rr + kB1Depth<RMAX> - 1);
    double a = 0.0;
    if (ks > 1 || rr < n_rows) {  // uniform per wave: padding rows are not computed
#pragma unroll
      for (int i = 0; i < UPL; i++) {
        const int u = ubase + 64 * i;
        if (FULL || u < U) accumulate_dig<F>(buf[rr][i], u, [&](int t) { return pr[i][t]; }, a);
      }
    }
    acc[rr] = a;
  }
#pragma unroll
  for (int rr = 0; rr < RMAX; rr++) acc[rr] = wave_sum_l63_d(acc[rr]);
  if constexpr (FUSE >= 2) {
    if (lane == 63) {
#pragma unroll
      for (int rr = 0; rr < RMAX; rr += 2)
        if (rr < n_rows) fuse_store_pair(fu, r_begin + rr, (float)acc[rr], (float)acc[rr + 1]);
    }
    return;
  }
  if (lane == 63) {
    if (ks == 1) {
#pragma unroll
      for (int rr = 0; rr < RMAX; rr++)
        if (rr < n_rows) {
          if (sliced) yp[r_begin + rr * r_step] = acc[rr];
          else y[r_begin + rr * r_step] = (float)acc[rr];
        }
    } else {
#pragma unroll
      for (int rr = 0; rr < RMAX; rr++) red[(stream * RMAX + rr) * ks + kw] = acc[rr];
    }
  }
  if (ks > 1) {
    __syncthreads();
    if (kw == 0 && lane < n_rows) {  // the first wave of each row stream
      double s = 0.0;
      for (int k = 0; k < ks; k++) s += red[(stream * RMAX + lane) * ks + k];
      if (sliced) yp[r_begin + lane * r_step] = s;
      else y[r_begin + lane * r_step] = (float)s;
    }
  }
}

// Batch-1 matvec as long per-wave row streams, for matrices that would take
// more than one round of mv_b1 workgroups: one workgroup per CU and K slice,
// wave w of workgroup b a run of consecutive rows (any length, balanced to one
// row), one unit per lane, D rows in flight in a rolling window of registers
// (the loop is unrolled by D so every window index is a constant).  Loads past
// the run repeat its last row (cached, results not stored).  Each row's sum is
// reduced and stored as soon as it is done.
template <int F, int D, bool FULL, int SIT>
__global__ __launch_bounds__(768) void mv_b1s(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                              float* __restrict__ y, int out_dim, int row_bpr, int slice_bpr) {
  using FU = FastUnit<F>;
  using DG = Dig<F>;
  constexpr int NW = FU::NW, US = DG::US;
  extern __shared__ uint4 lds4[];
  uint32_t* lds = reinterpret_cast<uint32_t*>(lds4);
  const int blk0 = blockIdx.y * slice_bpr;
  const int bpr = min(slice_bpr, row_bpr - blk0);
  w += (size_t)blk0 * Geom<F>::bb;
  x += (size_t)blk0 * Geom<F>::bs;
  const bool sliced = gridDim.y > 1;  // partial sums as doubles (see mv_b1)
  double* yp = reinterpret_cast<double*>(y) + (size_t)blockIdx.y * out_dim;
  const int keff = bpr * Geom<F>::bs;
  const int U = keff / FU::E;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const size_t row_bytes = (size_t)row_bpr * Geom<F>::bb;
  const long n_streams = (long)gridDim.x * (blockDim.x >> 6), gs = (long)blockIdx.x * (blockDim.x >> 6) + wave;
  const int r_begin = (int)(gs * out_dim / n_streams);
  const int n_rows = (int)((gs + 1) * out_dim / n_streams) - r_begin;
  const int r_last = r_begin + max(n_rows, 1) - 1;
  const int u = FULL ? lane : min(lane, U - 1);  // partial rows: the spare lanes repeat the last unit

  uint32_t buf[D][NW];
  auto load_row = [&](int rr, uint32_t* b) { load_unit<F>(w + (size_t)min(r_begin + rr, r_last) * row_bytes, u, b); };

  XChunks<SIT> st;
  stage_load<SIT>(x, keff, st, blockDim.x);
#pragma unroll
  for (int i = 0; i < D; i++) load_row(i, buf[i]);
  {
    constexpr int N = D * loads_per_unit<F>();  // wait for x only
    static_assert(N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  }
  stage_store<F, SIT>(st, keff, lds, blockDim.x);
  lds_barrier();
  uint32_t pr[US];
#pragma unroll
  for (int t = 0; t < US; t += 4) {
    const uint4 v = lds4[(size_t)u * (US / 4) + t / 4];
    pr[t] = v.x; pr[t + 1] = v.y; pr[t + 2] = v.z; pr[t + 3] = v.w;
  }
  const bool live = FULL || lane < U;
  for (int r0 = 0; r0 < n_rows; r0 += D) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      double a = 0.0;
      accumulate_dig<F>(buf[i], u, [&](int t) { return pr[t]; }, a);
      load_row(r0 + i + D, buf[i]);
      a = wave_sum_l63_d(live ? a : 0.0);
      if (lane == 63 && r0 + i < n_rows) {
        if (sliced) yp[r_begin + r0 + i] = a;
        else y[r_begin + r0 + i] = (float)a;
      }
    }
  }
}

// One 16-byte nontemporal load per lane straight into LDS: lane l writes
// bytes [16 l, 16 l + 16) above the wave-uniform LDS offset lds.  Inline
// assembly, so the compiler neither counts nor waits for it: the kernel waits
// for these loads itself.  One wait state (s_nop) separates the M0 write from
// the LDS-DMA load that reads M0, as the ISA requires and as the compiler's
// hazard recognizer, which does not look inside inline assembly, would insert.
// M0 is restored.
__device__ __forceinline__ void dma16_nt(const void* g, uint32_t lds) {
  uint32_t keep;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off nt\n\ts_mov_b32 m0, %0"
               : "=&s"(keep)
               : "s"(lds), "v"(g)
               : "memory");
}

// Row streams as mv_b1s, with each row slice (at most 64 units) copied into a
// per-wave LDS slot by contiguous 1 KB nontemporal loads, so every 128-byte
// line of the matrix is requested once, by one instruction (the overlapping
// per-unit loads of load_unit hit a line up to three times, which only the
// vector cache absorbs, and the nontemporal hint bypasses it); load_unit then
// reads the unit from the slot at the same byte offsets.  The slice must start
// 16-byte aligned in memory (the slot keeps its alignment, which the Q6_K
// realignment reads).  D slots form the rolling window; a row's copies are
// waited for with an exact count (NC per later row), so the loop holds no
// other vector memory instruction: row sums go to LDS and are stored after
// the loop.  (The compiler's wait for x, which does not count the copies,
// drains the first rows' copies before x is staged; staging x through the
// same LDS copies instead measured slower.)  Used for long row streams only:
// 28672 x 8192 Q4_K (19 rows per wave) 27.4 -> 26.2 us, while 4096 x 14336
// (5 rows per wave) was 3% slower than mv_b1s.
template <int F, int UPL = 1>
struct LdsSlot {
  static constexpr int unit_bytes = Geom<F>::bb * FastUnit<F>::E / Geom<F>::bs;
  static constexpr int NC = (UPL * 64 * unit_bytes + 1023) / 1024;  // 1 KB copies per row slice
  static constexpr int SLOT = 1024 * NC;
};

// UPL units per lane: rows of up to 64 UPL units run whole (UPL = 2: rows of
// 65-128 units without K slices, whose partials would need a second launch).
template <int F, int UPL, int D, bool FULL, int SIT>
__global__ __launch_bounds__(768) void mv_b1s_lds(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                  float* __restrict__ y, int out_dim, int row_bpr, int slice_bpr,
                                                  int rows_cap) {
  constexpr int US = Dig<F>::US, SLOT = LdsSlot<F, UPL>::SLOT, NC = LdsSlot<F, UPL>::NC;
  extern __shared__ uint4 lds4[];
  uint32_t* lds = reinterpret_cast<uint32_t*>(lds4);
  const int blk0 = blockIdx.y * slice_bpr;
  const int bpr = min(slice_bpr, row_bpr - blk0);
  w += (size_t)blk0 * Geom<F>::bb;
  x += (size_t)blk0 * Geom<F>::bs;
  const bool sliced = gridDim.y > 1;  // partial sums as doubles (see mv_b1)
  double* yp = reinterpret_cast<double*>(y) + (size_t)blockIdx.y * out_dim;
  const int keff = bpr * Geom<F>::bs;
  const int U = keff / FastUnit<F>::E;
  const int nbytes = bpr * Geom<F>::bb;  // <= SLOT
  const int lane = threadIdx.x & 63, nwaves = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // scalar: the LDS slots' M0 base
  const size_t row_bytes = (size_t)row_bpr * Geom<F>::bb;
  const long n_streams = (long)gridDim.x * nwaves, gs = (long)blockIdx.x * nwaves + wave;
  const int r_begin = (int)(gs * out_dim / n_streams);
  const int n_rows = (int)((gs + 1) * out_dim / n_streams) - r_begin;
  const int r_last = r_begin + max(n_rows, 1) - 1;
  int u[UPL];
#pragma unroll
  for (int i = 0; i < UPL; i++) u[i] = FULL ? lane + 64 * i : min(lane + 64 * i, U - 1);
  uint8_t* wl = reinterpret_cast<uint8_t*>(lds4) + (size_t)U * US * sizeof(uint32_t);
  double* red = reinterpret_cast<double*>(wl + (size_t)nwaves * D * SLOT) + (size_t)wave * rows_cap;
  wl += (size_t)wave * D * SLOT;
  const uint32_t wl_off = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)wl;

  // Copy k of a row slice: lanes whose 16 bytes lie in the slice, and lane 0
  // always (a dummy copy of the row's first bytes into the unused part of the
  // slot when the slice ends before 1024 k), so that every row issues NC
  // copies.
  auto copy_row = [&](int rr, int sl) {
    const uint8_t* rp = w + (size_t)min(r_begin + rr, r_last) * row_bytes;
#pragma unroll
    for (int k = 0; k < NC; k++) {
      const int o = 1024 * k + 16 * lane;
      if (o < nbytes || lane == 0) dma16_nt(rp + (o < nbytes ? o : 0), wl_off + sl * SLOT + 1024 * k);
    }
  };

  XChunks<SIT> st;
  stage_load<SIT>(x, keff, st, blockDim.x);
#pragma unroll
  for (int i = 0; i < D; i++) copy_row(i, i);
  stage_store<F, SIT>(st, keff, lds, blockDim.x);
  lds_barrier();
  uint32_t pr[UPL][US];
#pragma unroll
  for (int j = 0; j < UPL; j++)
#pragma unroll
    for (int t = 0; t < US; t += 4) {
      const uint4 v = lds4[(size_t)u[j] * (US / 4) + t / 4];
      pr[j][t] = v.x; pr[j][t + 1] = v.y; pr[j][t + 2] = v.z; pr[j][t + 3] = v.w;
    }
  static_assert(D <= 2, "the wait below counts one later row");
  for (int r0 = 0; r0 < n_rows; r0 += D) {
#pragma unroll
    for (int i = 0; i < D; i++) {
      // the copies of row r0 + i have landed once only those of row r0 + i + 1
      // may be pending (issued unless past the run and past the first D rows:
      // refills past the run are not issued, the first D rows are, clamped)
      __builtin_amdgcn_sched_barrier(0);
      if (D == 1 || r0 + i + 1 >= max(D, n_rows)) wait_vmcnt<0>();
      else wait_vmcnt<NC * (D - 1)>();
      __builtin_amdgcn_sched_barrier(0);
      double a = 0.0;
#pragma unroll
      for (int j = 0; j < UPL; j++) {
        uint32_t raw[FastUnit<F>::NW];
        load_unit<F>(wl + i * SLOT, u[j], raw);
        double aj = 0.0;
        accumulate_dig<F>(raw, u[j], [&](int t) { return pr[j][t]; }, aj);
        a += (FULL || lane + 64 * j < U) ? aj : 0.0;
      }
      // The slot's LDS reads complete before its next copy is requested: the
      // compiler may issue the copy (inline assembly) right after the read
      // instructions, and a copy served from the cache can land before reads
      // still queued in the LDS pipeline.
      __builtin_amdgcn_sched_barrier(0);
      wait_lgkmcnt0();
      __builtin_amdgcn_sched_barrier(0);
      // no refill past the run (a nontemporal copy of a repeated row is
      // fetched from HBM again)
      if (r0 + i + D < n_rows) copy_row(r0 + i + D, i);
      a = wave_sum_l63_d(a);
      if (lane == 63 && r0 + i < n_rows) red[r0 + i] = a;
    }
  }
  // the window's last copies land before the workgroup's LDS is released
  wait_vmcnt<0>();
  for (int r = lane; r < n_rows; r += 64) {
    if (sliced) yp[r_begin + r] = red[r];
    else y[r_begin + r] = (float)red[r];
  }
}

// Batch-1 matvec of whole rows (at most 64 units) with the rows copied into
// LDS and x staged by waves of its own.  One workgroup per CU of XW "x waves"
// (kB1rXW, or kB1rXWCold where x is cold) and NRW "row waves".  The
// workgroup owns a contiguous range of rows; row wave v takes rows v, v + NRW,
// v + 2 NRW, ... of it, so the workgroup's
// copies in flight cover consecutive rows.  Each row wave keeps D row slots of
// NCR KB and copies a row into a slot with NCR contiguous 1 KB nontemporal
// copies (lanes past the row masked off; lane 0 always issues, so every row
// issues NCR copies).  The first D rows are copied even past a short run
// (clamped repeats, not stored); later rows past the run are not.
//
// Schedule (per-wave wall-clock timelines on MI355X, 14336 x 4096 Q4_K):
//   1. The x waves request x; the row waves sleep a few hundred cycles first,
//      so the x loads are queued in the CU ahead of the weight copies (x lands
//      at ~0.55 us from the first wave's start instead of ~1 us).  A barrier
//      there instead made the x waves wait for the last row wave to launch
//      before converting (measured: 14336 x 4096 Q4_K 8.10 -> 8.07 us, 4096 x
//      4096 Q4_0 4.50 -> 4.47, 11008 x 4096 Q8_0 9.20 -> 9.11, and with the
//      longer sleep of the norm-fused launches, whose x waves also request the
//      residual and the norm weights, the decode layer 55.5 -> 54.9 us).
//   2. The row waves copy their first D rows.  The x waves wait for x, write
//      the digit planes and meet the row waves at an LDS-only barrier.
//      x is fetched by waves that issue no copies, so the compiler's wait for
//      x, which cannot count the copies (inline assembly), drains nothing of
//      the weight stream; staging x (~0.8 us) hides under the first rows'
//      memory latency.
//   3. Each row is computed once its copies have landed (exact wait counts:
//      the loop issues no other vector memory instruction), and its slot takes
//      the copies of row r + D as soon as the slot's LDS reads are done.  Row
//      sums go to LDS and are stored after the loop.
// Measured (kernel alone, graph replays): 14336 x 4096 Q4_K 8.45 -> 7.99 us
// (D 1, 12 row waves), 4096 x 4096 4.81 -> 4.56 us (D 2, 8 row waves); 1024
// rows (4 per CU) stay on mv_b1 (3.6 against 3.9 us).  Slots of one whole row each beat a contiguous 1 KB ring of the
// wave's run (8.2-8.8 us) and requesting every row of the run at the start
// (10.4 us: the copies stall at issue and the stream slows).
constexpr int kB1rXW = 4;
// x waves where x is cold: the fused decode-layer launches with 8 row waves
// (their x is the layer input, just written) and plain launches under FreshX.
// With x resident in L2 (a matvec repeated on one x) four x waves are faster:
// 4096 x 4096 Q4_0 4.49 against 4.56 us with eight; where x was just written
// by the previous kernel, eight request it sooner: the decode layer's output
// projection and QKV + RoPE launches, 54.9 -> 54.0 us per layer (A/B, two runs).
constexpr int kB1rXWCold = 8;

// Waits until at most pend rows of NCR copies each are pending (pend <= P,
// wave-uniform; vmcnt takes an immediate, so one branch per count).
template <int NCR, int P>
__device__ __forceinline__ void wait_rows(int pend) {
  if constexpr (P == 0) {
    wait_vmcnt<0>();
  } else {
    if (pend >= P) wait_vmcnt<NCR * P>();
    else wait_rows<NCR, P - 1>(pend);
  }
}

// The body of mv_b1r and of its decode-layer fusion mv_b1r_fused (FUSE as in
// mv_b1: 2 row pairs with the RoPE / SwiGLU epilogue, 3 and 4 the same with an
// RMSNorm of x, 4 of x + a residual).  Fused, the workgroup's units are row
// pairs (out_dim virtual rows, q and rem count pairs): row wave v takes pairs
// v, v + NRW, ... and copies both rows of each, so it holds both dot products
// of its pairs for the epilogue.  With the norm, the x waves also load the
// residual and the norm weights, and the row waves sleep longer before their
// first copies.
template <int F, int NCR, int D, int NRW, int FUSE, int XW = kB1rXW>
__device__ __forceinline__ void b1r_body(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                         float* __restrict__ y, int out_dim, int row_bpr, int slice_bpr, int q,
                                         int rem, int rows_cap, const FuseArg<FUSE>& fu) {
  constexpr int US = Dig<F>::US, NW = FastUnit<F>::NW, SLOT = 1024 * NCR, SIT = 8 / XW;
  static_assert(NCR * (D - 1) < 64, "vmcnt range");
  extern __shared__ uint4 lds4[];
  uint32_t* lds = reinterpret_cast<uint32_t*>(lds4);
  // K slice blockIdx.y of the rows (slice_bpr blocks; the whole row when
  // gridDim.y == 1): a sliced row writes its partial sums as doubles to
  // ((double*)y)[z * out_dim + row] (slice_reduce_kernel adds them in order)
  const int blk0 = blockIdx.y * slice_bpr;
  const int bpr = min(slice_bpr, row_bpr - blk0);
  w += (size_t)blk0 * Geom<F>::bb;
  x += (size_t)blk0 * Geom<F>::bs;
  const bool sliced = gridDim.y > 1;
  const int keff = bpr * Geom<F>::bs;  // at most 4096: 512 chunks of 8, two per x-wave thread
  const int U = keff / FastUnit<F>::E;
  const int nbytes = bpr * Geom<F>::bb;  // at most SLOT
  const size_t row_bytes = (size_t)row_bpr * Geom<F>::bb;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  uint8_t* const slots = reinterpret_cast<uint8_t*>(lds4) + (size_t)U * US * sizeof(uint32_t);
  double* const red_all = reinterpret_cast<double*>(slots + (size_t)NRW * D * SLOT);
  // norm-fused: the x waves' sums of squares and staging exponents, after the
  // row sums of every row wave
  [[maybe_unused]] float* const part = reinterpret_cast<float*>(red_all + (size_t)NRW * rows_cap);
  if (wave < XW) {
    XChunks<SIT> st;
    stage_load<SIT>(x, keff, st, 64 * XW);
    [[maybe_unused]] XChunks<SIT> st_r, st_w;
    if constexpr (FUSE >= 3) {
      if constexpr (FUSE == 4) stage_load<SIT>(fu.norm_res, keff, st_r, 64 * XW);
      stage_load<SIT>(fu.norm_w, keff, st_w, 64 * XW);
    }
    if constexpr (FUSE >= 3) {
      // Every output is linear in x' = h inv_rms w, so the x waves stage h w
      // at once and the row waves multiply their dot products by inv_rms,
      // which needs the sums of squares of all x waves only after the loop.
      // Where a product of finite h and w overflows fp32 (for x' itself finite
      // or, the sum of squares overflowing, zero), the wave stages h w 2^-k
      // instead (k from its largest product, rounded once from double), and
      // the row waves scale the partial sums of its units by 2^k.
      // st is h from here; the wave's sum of squares is valid in lane 63
      const float qs = wave_sum_l63(norm_sumsq<SIT, FUSE == 4>(st, st_r));
      XChunks<SIT> hw;
      float zz = 0.f;  // NaN when a product is infinite or NaN (rare: then the test below)
#pragma unroll
      for (int it = 0; it < SIT; it++)
#pragma unroll
        for (int j = 0; j < 8; j++) {
          hw.v[it][j] = st.v[it][j] * st_w.v[it][j];
          zz = fmaf(hw.v[it][j], 0.f, zz);
        }
      bool ovf = false;
      if (__any(zz != zz)) {
#pragma unroll
        for (int it = 0; it < SIT; it++)
#pragma unroll
          for (int j = 0; j < 8; j++)
            ovf |= isinf(hw.v[it][j]) && isfinite(st.v[it][j]) && isfinite(st_w.v[it][j]);
      }
      int k = 0;
      if (__any(ovf)) {
        float e = -1000.f;  // bound on the exponent of every finite product
#pragma unroll
        for (int it = 0; it < SIT; it++)
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const float h = st.v[it][j], g = st_w.v[it][j];
            if (isfinite(h) && isfinite(g) && h != 0.f && g != 0.f) e = fmaxf(e, (float)(ilogbf(h) + ilogbf(g) + 2));
          }
        k = max(0, (int)wave_max(e) - 127);
        const double sc = ldexp(1.0, -k);
#pragma unroll
        for (int it = 0; it < SIT; it++)
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const float h = st.v[it][j], g = st_w.v[it][j];
            if (isfinite(h) && isfinite(g)) hw.v[it][j] = (float)((double)h * (double)g * sc);
          }
      }
      if (lane == 63) {
        part[wave] = qs;
        reinterpret_cast<int*>(part)[XW + wave] = k;
      }
      stage_store<F, SIT>(hw, keff, lds, 64 * XW);
      lds_barrier();  // 2.
      if (blockIdx.x == 0) {  // h and x' to the step outputs
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < XW; i++) t += part[i];
        norm_apply<SIT>(st, st_w, 1.0f / sqrtf(t / (float)keff + fu.norm_eps), keff, 64 * XW, fu);
      }
      return;
    }
    stage_store<F, SIT>(st, keff, lds, 64 * XW);
    lds_barrier();  // 2.
    return;
  }
  __builtin_amdgcn_s_sleep(FUSE >= 3 ? 6 : 2);  // 1. (64 cycles per unit)
  const int rw = wave - XW;
  const int b = (int)blockIdx.x;
  constexpr int UR = FUSE != 0 ? 2 : 1;  // rows per unit of work
  const int wg_begin = b * q + min(b, rem), wg_units = q + (b < rem ? 1 : 0);
  const int nu = wg_units > rw ? (wg_units - 1 - rw) / NRW + 1 : 0;
  const int nr = UR * nu;  // <= rows_cap
  uint8_t* wl = slots + (size_t)rw * D * SLOT;
  double* red = red_all + (size_t)rw * rows_cap;
  const uint32_t wl_off = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)wl;
  // The segments' weight pointers as a base and two offsets (scalar
  // arithmetic per row, as in mv_b1).
  [[maybe_unused]] const uint8_t* fw0 = nullptr;
  [[maybe_unused]] ptrdiff_t fd1 = 0, fd2 = 0;
  if constexpr (FUSE != 0) {
    fw0 = fu.w0;
    fd1 = fu.w1 - fu.w0;
    fd2 = fu.w2 - fu.w0;
  }
  auto copy_row = [&](int k, int sl) {
    const int kk = min(k, max(nr, 1) - 1);
    const uint8_t* rp;
    if constexpr (FUSE != 0) {
      const int pair = min(wg_begin + rw + (kk >> 1) * NRW, out_dim / 2 - 1);
      int r;
      const int sg = fuse_seg(fu, __builtin_amdgcn_readfirstlane(2 * pair + (kk & 1)), r);
      rp = fw0 + (sg == 0 ? 0 : sg == 1 ? fd1 : fd2) + (size_t)r * row_bytes;
    } else {
      const int row = min(wg_begin + rw + kk * NRW, out_dim - 1);
      rp = w + (size_t)row * row_bytes;
    }
#pragma unroll
    for (int c = 0; c < NCR; c++) {
      const int o = 1024 * c + 16 * lane;
      if (o < nbytes || lane == 0) dma16_nt(rp + (o < nbytes ? o : 0), wl_off + sl * SLOT + 1024 * c);
    }
  };
#pragma unroll
  for (int i = 0; i < D; i++) copy_row(i, i);  // 2.
  lds_barrier();                                // 2.
  const int u = min(lane, U - 1);
  uint32_t pr[US];
#pragma unroll
  for (int t = 0; t < US; t += 4) {
    const uint4 v = lds4[(size_t)u * (US / 4) + t / 4];
    pr[t] = v.x; pr[t + 1] = v.y; pr[t + 2] = v.z; pr[t + 3] = v.w;
  }
  // norm-fused: 2^k of the x wave that staged unit u (its 8-element chunks
  // c went to thread c mod 64 XW)
  [[maybe_unused]] double unit_sc = 1.0;
  if constexpr (FUSE >= 3) {
    const int c0 = (FastUnit<F>::E / 8) * u;
    unit_sc = ldexp(1.0, reinterpret_cast<const int*>(part)[XW + (c0 % (64 * XW)) / 64]);
  }
  for (int r0 = 0; r0 < nr; r0 += D) {  // 3.
#pragma unroll
    for (int i = 0; i < D; i++) {
      // Row r0 + i has landed once only the copies issued after it are
      // pending: those of rows r0 + i + 1 .. r0 + i + D - 1 that were issued
      // (the first D rows always are, clamped; refills past the run are not),
      // that is min(D - 1, max(D, nr) - 1 - (r0 + i)) rows.
      __builtin_amdgcn_sched_barrier(0);
      wait_rows<NCR, D - 1>(min(D - 1, max(D, nr) - 1 - (r0 + i)));
      __builtin_amdgcn_sched_barrier(0);
      uint32_t raw[NW];
      load_unit<F>(wl + i * SLOT, u, raw);
      // The slot's LDS reads complete before its next copies are requested (a
      // copy served from the cache can land before reads still queued in the
      // LDS pipeline).
      __builtin_amdgcn_sched_barrier(0);
      wait_lgkmcnt0();
      __builtin_amdgcn_sched_barrier(0);
      // no refill past the run: nontemporal copies of a repeated row are
      // fetched from HBM again (1.07x the headline's bytes, 1.18x at Q8_0
      // 11008 x 4096)
      if (r0 + i + D < nr) copy_row(r0 + i + D, i);
      double a = 0.0;
      accumulate_dig<F>(raw, u, [&](int t) { return pr[t]; }, a);
      if constexpr (FUSE >= 3) a *= unit_sc;
      a = wave_sum_l63_d(lane < U ? a : 0.0);
      if (lane == 63 && r0 + i < nr) red[r0 + i] = a;
    }
  }
  wait_vmcnt<0>();  // the last copies land before the workgroup's LDS is released
  if constexpr (FUSE != 0) {
    double inv = 1.0;
    if constexpr (FUSE >= 3) {
      float t = 0.f;
#pragma unroll
      for (int i = 0; i < XW; i++) t += part[i];
      inv = (double)(1.0f / sqrtf(t / (float)keff + fu.norm_eps));
    }
    for (int k = lane; k < nu; k += 64)
      fuse_store_pair(fu, 2 * (wg_begin + rw + k * NRW), (float)(red[2 * k] * inv), (float)(red[2 * k + 1] * inv));
    return;
  }
  double* yp = reinterpret_cast<double*>(y) + (size_t)blockIdx.y * out_dim;
  for (int r = lane; r < nr; r += 64) {
    if (sliced) yp[wg_begin + rw + r * NRW] = red[r];
    else y[wg_begin + rw + r * NRW] = (float)red[r];
  }
}

template <int F, int NCR, int D, int NRW, int XW = kB1rXW>
__global__ __launch_bounds__(64 * (XW + NRW)) void mv_b1r(const uint8_t* __restrict__ w,
                                                              const float* __restrict__ x, float* __restrict__ y,
                                                              int out_dim, int row_bpr, int slice_bpr, int q, int rem,
                                                              int rows_cap) {
  b1r_body<F, NCR, D, NRW, 0, XW>(w, x, y, out_dim, row_bpr, slice_bpr, q, rem, rows_cap, NoFuse{});
}

// Whole rows only (one K slice); vrows virtual rows, q and rem in row pairs.
template <int F, int NCR, int D, int NRW, int FUSE, int XW = kB1rXW>
__global__ __launch_bounds__(64 * (XW + NRW)) void mv_b1r_fused(const float* __restrict__ x, int vrows, int bpr,
                                                                    int q, int rem, int rows_cap, MatvecFuse fu) {
  b1r_body<F, NCR, D, NRW, FUSE, XW>(nullptr, x, nullptr, vrows, bpr, bpr, q, rem, rows_cap, fu);
}

// Sums the K-slice partials (doubles, [slices][n]) in slice order and rounds
// once.  With res non-null, y = res + (the slice sum), the residual add of a
// decoder layer (y may alias res: each thread reads its element before
// writing it), and the slice sum itself also goes to sum_out.
__global__ __launch_bounds__(256) void slice_reduce_kernel(const double* __restrict__ part, float* y, int n,
                                                           int slices, const float* res, float* sum_out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  // Eight slice loads are in flight together (addresses clamped, so the
  // loads are unconditional); the sum still runs in slice order.
  double s = 0.0;
  for (int z0 = 0; z0 < slices; z0 += 8) {
    double v[8];
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = part[(size_t)min(z0 + k, slices - 1) * n + i];
#pragma unroll
    for (int k = 0; k < 8; k++)
      if (z0 + k < slices) s = z0 + k == 0 ? v[k] : s + v[k];
  }
  const float sf = (float)s;
  if (res) {
    y[i] = res[i] + sf;
    sum_out[i] = sf;
  } else {
    y[i] = sf;
  }
}

// Small batches (NB = 2..8 activation rows) on the digit-plane scheme.  The
// planes of all NB rows of x sit in LDS (row b at b * U * US dwords); each
// wave streams its weight rows through registers once, as mv_b1 does, and
// applies every row to all NB activations, so W is read once per call.  One
// unit per lane (rows longer than 64 units are cut into K slices; slice z
// writes partials [z][NB][out_dim]).
template <int F, int NB, int RMAX, int RG, bool FULL, int SIT>
__global__ __launch_bounds__(512) void mv_bn(const uint8_t* __restrict__ w,
                                             const float* __restrict__ x, float* __restrict__ y,
                                             int out_dim, int in_dim, int row_bpr, int slice_bpr,
                                             bool interleave) {
  using FU = FastUnit<F>;
  using D = Dig<F>;
  constexpr int NW = FU::NW, US = D::US;
  static_assert(US % 4 == 0, "unit records are read as 16-byte vectors");
  extern __shared__ uint4 lds4[];
  uint32_t* lds = reinterpret_cast<uint32_t*>(lds4);
  const int blk0 = blockIdx.y * slice_bpr;
  const int bpr = min(slice_bpr, row_bpr - blk0);
  w += (size_t)blk0 * Geom<F>::bb;
  x += (size_t)blk0 * Geom<F>::bs;
  const bool sliced = gridDim.y > 1;  // partial sums as doubles (see mv_b1)
  double* yp = reinterpret_cast<double*>(y) + (size_t)blockIdx.y * NB * out_dim;
  const int keff = bpr * Geom<F>::bs;
  const int U = keff / FU::E;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const size_t row_bytes = (size_t)row_bpr * Geom<F>::bb;
  const long n_streams = (long)gridDim.x * nw, gs = (long)blockIdx.x * nw + wave;
  int r_begin, r_step, n_rows;  // n_rows <= RMAX
  if (interleave) {
    r_begin = (int)gs;
    r_step = (int)n_streams;
    n_rows = gs < out_dim ? (int)((out_dim - 1 - gs) / n_streams) + 1 : 0;
  } else {
    r_begin = (int)(gs * out_dim / n_streams);
    r_step = 1;
    n_rows = (int)((gs + 1) * out_dim / n_streams) - r_begin;
  }
  const int u = lane;
  const bool ok = FULL || u < U;

  uint32_t buf[RMAX][NW];
  auto load_row = [&](int rr) {
    const int row = max(0, min(r_begin + rr * r_step, out_dim - 1));
    if (ok) load_unit<F>(w + (size_t)row * row_bytes, u, buf[rr]);
  };

  static_assert(RMAX % RG == 0, "rows come in groups of RG");
  XChunks<SIT> st;
  stage_load<SIT>(x, keff, st, blockDim.x, NB, (size_t)in_dim);
#pragma unroll
  for (int rr = 0; rr < RG; rr++) load_row(rr);
  {
    constexpr int N = RG * loads_per_unit<F>();
    static_assert(N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
  }
  stage_store<F, SIT>(st, keff, lds, blockDim.x, NB, U * US);
  lds_barrier();

  // Groups of RG rows: the next group's rows are requested before this one is
  // computed; each activation row's planes are read from LDS once per group.
  double acc[RMAX][NB];
#pragma unroll
  for (int g0 = 0; g0 < RMAX; g0 += RG) {
    if (g0 + RG < RMAX) {
#pragma unroll
      for (int r = 0; r < RG; r++) load_row(g0 + RG + r);
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
      uint32_t pr[US];
#pragma unroll
      for (int t = 0; t < US; t += 4) {
        const uint4 v = lds4[((size_t)b * U + u) * (US / 4) + t / 4];
        pr[t] = v.x; pr[t + 1] = v.y; pr[t + 2] = v.z; pr[t + 3] = v.w;
      }
#pragma unroll
      for (int r = 0; r < RG; r++) {
        double a = 0.0;
        if (g0 + r < n_rows && ok)  // uniform per wave except the last units of a partial row
          accumulate_dig<F>(buf[g0 + r], u, [&](int t) { return pr[t]; }, a);
        acc[g0 + r][b] = a;
      }
    }
  }
#pragma unroll
  for (int rr = 0; rr < RMAX; rr++)
#pragma unroll
    for (int b = 0; b < NB; b++) acc[rr][b] = wave_sum_l63_d(acc[rr][b]);
  if (lane == 63) {
#pragma unroll
    for (int rr = 0; rr < RMAX; rr++)
      if (rr < n_rows) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
          if (sliced) yp[(size_t)b * out_dim + r_begin + rr * r_step] = acc[rr][b];
          else y[(size_t)b * out_dim + r_begin + rr * r_step] = (float)acc[rr][b];
        }
      }
  }
}

// ------------------------------------------------------ batched (B > 1) path
// x' for all B activations lives in LDS; each lane reads its unit's x' per use
// and applies one decoded unit to R rows x B activations.
template <int F, int B, int R>
__global__ __launch_bounds__(256) void mv_lds(const uint8_t* __restrict__ w,
                                              const float* __restrict__ x, float* __restrict__ y,
                                              int out_dim, int in_dim, int bpr, int rows_per_wg) {
  using FU = FastUnit<F>;
  constexpr int E = FU::E, NS = FU::NSUM, SG = FU::SUMG, ES = E + 4, NW = FU::NW;
  extern __shared__ float smem[];
  const int keff = bpr * Geom<F>::bs;
  const int U = keff / E;
  float* xs = smem;                          // [B][U][ES]
  float* xsum = smem + (size_t)B * U * ES;   // [B][U*NS]
  stage_x<F, B>(x, in_dim, keff, U, xs);
  for (int i = threadIdx.x; i < B * U * NS; i += blockDim.x) {
    const int b = i / (U * NS), g = i - b * (U * NS);
    const float* xp = x + (size_t)b * in_dim + (size_t)g * SG;
    float s = 0.f;
    for (int t = 0; t < SG; t += 4) {
      const float4 v = *reinterpret_cast<const float4*>(xp + t);
      s += (v.x + v.y) + (v.z + v.w);
    }
    xsum[i] = s;
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const size_t row_bytes = (size_t)bpr * Geom<F>::bb;
  const int r_begin = blockIdx.x * rows_per_wg;
  const int r_end = min(out_dim, r_begin + rows_per_wg);
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
            raw[rr], u, [&](int b, int e) { return xu[(size_t)b * U * ES + e]; },
            [&](int b, int g) { return su[(size_t)b * U * NS + g]; }, acc[rr]);
    }
#pragma unroll
    for (int rr = 0; rr < R; rr++)
#pragma unroll
      for (int b = 0; b < B; b++) {
        const float s = wave_sum_dpp(acc[rr][b]);
        if (lane == 0 && r0 + rr < r_end) y[(size_t)b * out_dim + r0 + rr] = s;
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

template <class K>
hipError_t set_lds_attr(K kern, size_t lds_bytes) {
  if (lds_bytes <= 65536) return hipSuccess;
  return hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                             lds_limit());
}

// Splits out_dim into contiguous row ranges, a multiple of `quantum` rows each,
// for about `target` workgroups.
void row_split(int out_dim, int quantum, int target, int* n_wg, int* rows_per_wg) {
  int n = std::max(1, std::min((out_dim + quantum - 1) / quantum, target));
  int r = (out_dim + n - 1) / n;
  r = (r + quantum - 1) / quantum * quantum;
  *rows_per_wg = r;
  *n_wg = (out_dim + r - 1) / r;
}

template <int F, int UPL, int RMAX, bool FULL, int SIT>
hipError_t run_b1_sit(const uint8_t* w, const float* x, float* y, int out_dim, int row_bpr,
                      int slice_bpr, int slices, int ks, int rs, size_t lds, hipStream_t s) {
  auto kern = mv_b1<F, UPL, RMAX, FULL, SIT>;
  hipError_t e = set_lds_attr(kern, lds);
  if (e != hipSuccess) return e;
  const int threads = 64 * ks * rs;
  // Q8_0 rows (68 bytes per unit) run faster with interleaved rows (11008 x
  // 4096: 11.0 us vs 11.5 us); the other formats with contiguous runs.
  const bool interleave = F == kQ8_0;
  const long streams_needed = (out_dim + RMAX - 1) / RMAX;
  // about one workgroup per CU over all slices (rounded down, so that the
  // slices together do not spill a few workgroups into a second round)
  long n_wg = std::max<long>(device_cu_count() / slices, (streams_needed + rs - 1) / rs);
  n_wg = std::max<long>(1, std::min<long>(n_wg, (out_dim + rs - 1) / rs));
  hipLaunchKernelGGL(kern, dim3((unsigned)n_wg, (unsigned)slices), dim3(threads), lds, s, w, x, y,
                     out_dim, row_bpr, slice_bpr, ks, interleave, NoFuse{});
  return hipGetLastError();
}

template <int F, int UPL, int RMAX, bool FULL>
hipError_t run_b1(const uint8_t* w, const float* x, float* y, int out_dim, int row_bpr,
                  int slice_bpr, int slices, int ks, hipStream_t s) {
  const int U = slice_bpr * Geom<F>::bs / FastUnit<F>::E;
  // x planes, then the per-wave row sums of every row stream (at most 12 waves)
  const size_t lds = ((size_t)U * Dig<F>::US + (size_t)2 * RMAX * 12) * sizeof(uint32_t);  // planes, double sums
  if (lds > (size_t)lds_limit()) return hipErrorInvalidValue;
  // One workgroup per CU holding as many waves as fit (ks waves per row
  // stream); the occupancy is the same for every staging depth.
  // The answer depends on (device, ks, lds) only and is cached: a launch then
  // costs no runtime query.
  static std::mutex mu;
  static std::map<std::tuple<int, int, size_t>, int> rs_cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  const auto key = std::make_tuple(dev, ks, lds);
  int rs = 0;
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = rs_cache.find(key);
    if (it != rs_cache.end()) rs = it->second;
  }
  if (rs == 0) {
    auto probe = mv_b1<F, UPL, RMAX, FULL, kStageIt>;
    hipError_t e = set_lds_attr(probe, lds);
    if (e != hipSuccess) return e;
    rs = 1;
    for (int cand = 768 / (64 * ks); cand >= 1; cand--) {
      int per_cu = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, probe, 64 * ks * cand, lds) == hipSuccess &&
          per_cu >= 1) {
        rs = cand;
        break;
      }
    }
    std::lock_guard<std::mutex> lk(mu);
    rs_cache[key] = rs;
  }
  const int threads = 64 * ks * rs;
  const int nchunk = slice_bpr * Geom<F>::bs / 8;
  const int sit = (nchunk + threads - 1) / threads;
  switch (sit) {
    case 0:
    case 1: return run_b1_sit<F, UPL, RMAX, FULL, 1>(w, x, y, out_dim, row_bpr, slice_bpr, slices, ks, rs, lds, s);
    case 2: return run_b1_sit<F, UPL, RMAX, FULL, 2>(w, x, y, out_dim, row_bpr, slice_bpr, slices, ks, rs, lds, s);
    case 3:
    case 4: return run_b1_sit<F, UPL, RMAX, FULL, 4>(w, x, y, out_dim, row_bpr, slice_bpr, slices, ks, rs, lds, s);
    default: return hipErrorNotSupported;  // x too long to stage
  }
}

template <int F, int B, int R>
hipError_t run_lds(const uint8_t* w, const float* x, float* y, int out_dim, int in_dim, int bpr,
                   size_t lds, hipStream_t s) {
  auto kern = mv_lds<F, B, R>;
  hipError_t e = set_lds_attr(kern, lds);
  if (e != hipSuccess) return e;
  int n_wg, rows;
  row_split(out_dim, 4 * R, 2 * device_cu_count(), &n_wg, &rows);
  hipLaunchKernelGGL(kern, dim3(n_wg), dim3(256), lds, s, w, x, y, out_dim, in_dim, bpr, rows);
  return hipGetLastError();
}

template <int F>
bool fast_aligned(const uint8_t* w, const float* x, int in_dim, int bpr) {
  const uintptr_t a = (uintptr_t)w;
  if ((((uintptr_t)x) & 15) || (in_dim & 3)) return false;  // float4 staging of x
  if constexpr (F == kQ4_K || F == kQ5_K) return (a & 15u) == 0;
  else if constexpr (F == kQ2_K || F == kQ3_K || F == kQ8_K) return (a & 3u) == 0;
  else return (a & 3u) == 0 && (bpr % 2) == 0;  // Q4_0 / Q8_0 pairs, Q6_K dword rows
}

// Two units per lane keep two units' digit planes in registers: only Q6_K's
// 40-dword records (80 VGPRs; 126-150 VGPRs per kernel) fit beside the row
// buffers without spilling; the 72- and 80-dword records of the other types
// (144-160 VGPRs) spill, and scratch accesses would also break the exact wait
// counts of the kernels that stream rows through LDS.
template <int F>
constexpr bool kTwoUnits = Dig<F>::NG == 1;

// Row geometry of the batch-1 kernel: rows of up to 128 units run whole (one
// wave per row stream); longer rows are cut into slices of at most 64 units.
template <int F>
struct B1Plan {
  int upl = 1, slice_bpr = 0, slices = 1;
  bool full = true;
};

template <int F>
B1Plan<F> b1_plan(int bpr, int out_dim) {
  const int U = bpr * Geom<F>::bs / FastUnit<F>::E;
  B1Plan<F> p;
  // Rows of 65-128 units run whole with two units per lane (3 rows per wave)
  // while that fits one round of workgroups and the kernel fits its registers
  // (kTwoUnits: Q6_K); otherwise as two K slices of one unit per lane, which
  // fit more rows per wave (14336 x 4096 Q6_K: 18.4 -> 15.2 us)
  if (U <= 64 || (U <= 128 && kTwoUnits<F> && out_dim <= 3 * 12 * device_cu_count())) {
    p.upl = U <= 64 ? 1 : 2;
    p.slice_bpr = bpr;
    p.full = (U == p.upl * 64);
    return p;
  }
  p.slices = (U + 63) / 64;
  int sb;
  if constexpr (Geom<F>::bs == 32) {  // Q4_0 / Q8_0: two blocks per unit
    sb = (bpr + p.slices - 1) / p.slices;
    sb += sb & 1;
  } else {
    sb = (bpr + p.slices - 1) / p.slices;
  }
  p.slice_bpr = sb;
  p.slices = (bpr + sb - 1) / sb;
  p.full = (bpr % sb == 0) && sb * Geom<F>::bs / FastUnit<F>::E == 64;
  return p;
}

// Types whose long row streams take mv_b1s_lds.
template <int F>
constexpr bool kLdsRowStreams = F == kQ4_K || F == kQ6_K || F == kQ4_0 || F == kQ8_0;

// mv_b1s launch: one workgroup of 12 waves per CU and K slice (at least one
// row per wave), two rows in flight per wave.
template <int F, bool FULL>
hipError_t run_b1s(const uint8_t* w, const float* x, float* y, int out_dim, int row_bpr, int slice_bpr,
                   int slices, hipStream_t s) {
  const int U = slice_bpr * Geom<F>::bs / FastUnit<F>::E;
  const size_t lds = (size_t)U * Dig<F>::US * sizeof(uint32_t);
  if (lds > (size_t)lds_limit()) return hipErrorNotSupported;
  const int sit = (slice_bpr * Geom<F>::bs / 8 + 767) / 768;
  const long n_wg = std::max<long>(1, std::min<long>(device_cu_count() / slices, (out_dim + 11) / 12));
  auto go = [&](auto kern) {
    hipError_t e = set_lds_attr(kern, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3((unsigned)n_wg, (unsigned)slices), dim3(768), lds, s, w, x, y, out_dim, row_bpr,
                       slice_bpr);
    return hipGetLastError();
  };
  if constexpr (kLdsRowStreams<F>) {
    // weights through LDS (mv_b1s_lds): two slots per wave and the row sums;
    // slices that start 16-byte aligned in memory
    const long n_streams = n_wg * 12;
    const int rows_cap = (int)((out_dim + n_streams - 1) / n_streams) + 1;
    const size_t lds2 = lds + (size_t)12 * 2 * LdsSlot<F, 1>::SLOT + (size_t)12 * rows_cap * sizeof(double);
    const bool aligned16 = ((uintptr_t)w % 16) == 0 && ((size_t)row_bpr * Geom<F>::bb) % 16 == 0 &&
                           ((size_t)slice_bpr * Geom<F>::bb) % 16 == 0;
    if (aligned16 && lds2 <= (size_t)lds_limit() && sit <= 2 && rows_cap > 12) {
      auto go2 = [&](auto kern) {
        hipError_t e = set_lds_attr(kern, lds2);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(kern, dim3((unsigned)n_wg, (unsigned)slices), dim3(768), lds2, s, w, x, y, out_dim,
                           row_bpr, slice_bpr, rows_cap);
        return hipGetLastError();
      };
      return sit <= 1 ? go2(mv_b1s_lds<F, 1, 2, FULL, 1>) : go2(mv_b1s_lds<F, 1, 2, FULL, 2>);
    }
  }
  switch (sit) {
    case 0:
    case 1: return go(mv_b1s<F, 2, FULL, 1>);
    case 2: return go(mv_b1s<F, 2, FULL, 2>);
    case 3:
    case 4: return go(mv_b1s<F, 2, FULL, 4>);
    default: return hipErrorNotSupported;
  }
}

// Rows of 65-128 units as whole-row LDS streams (mv_b1s_lds, two units per
// lane, one workgroup per CU): no K slices, so no partials and no second
// launch.  hipErrorNotSupported when the shape does not qualify (short
// streams, unaligned rows, LDS).
template <int F>
hipError_t run_b1s_lds_rows(const uint8_t* w, const float* x, float* y, int out_dim, int bpr, hipStream_t s) {
  if constexpr (!kLdsRowStreams<F> || !kTwoUnits<F>) {
    return hipErrorNotSupported;
  } else {
    const int U = bpr * Geom<F>::bs / FastUnit<F>::E;
    if (U <= 64 || U > 128) return hipErrorNotSupported;
    if (((uintptr_t)w % 16) != 0 || ((size_t)bpr * Geom<F>::bb) % 16 != 0) return hipErrorNotSupported;
    const int sit = (bpr * Geom<F>::bs / 8 + 767) / 768;
    if (sit > 2) return hipErrorNotSupported;
    const long n_wg = std::max<long>(1, std::min<long>(device_cu_count(), (out_dim + 11) / 12));
    const long n_streams = n_wg * 12;
    const int rows_cap = (int)((out_dim + n_streams - 1) / n_streams) + 1;
    if (rows_cap <= 12) return hipErrorNotSupported;
    const size_t lds = (size_t)U * Dig<F>::US * sizeof(uint32_t) + (size_t)12 * 2 * LdsSlot<F, 2>::SLOT +
                       (size_t)12 * rows_cap * sizeof(double);
    if (lds > (size_t)lds_limit()) return hipErrorNotSupported;
    auto go = [&](auto kern) {
      hipError_t e = set_lds_attr(kern, lds);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(kern, dim3((unsigned)n_wg), dim3(768), lds, s, w, x, y, out_dim, bpr, bpr, rows_cap);
      return hipGetLastError();
    };
    const bool full = U == 128;
    if (sit <= 1) return full ? go(mv_b1s_lds<F, 2, 2, true, 1>) : go(mv_b1s_lds<F, 2, 2, false, 1>);
    return full ? go(mv_b1s_lds<F, 2, 2, true, 2>) : go(mv_b1s_lds<F, 2, 2, false, 2>);
  }
}

thread_local int g_fresh_x = 0;

}  // namespace

FreshX::FreshX() { ++g_fresh_x; }
FreshX::~FreshX() { --g_fresh_x; }
bool fresh_x() { return g_fresh_x > 0; }

namespace {

// Types whose whole rows of 4096 elements take mv_b1r (LDS row slots).
template <int F>
constexpr bool kRowSlots = F == kQ4_K || F == kQ4_0 || F == kQ8_0;

// mv_b1r launch: whole rows of 3584-4096 elements (3 KB slots for Q4_K and
// Q4_0, 5 KB for Q8_0), 16-byte aligned, from 8 rows per CU up to one round of
// mv_b1 workgroups (10 rows per wave).  One row in flight per wave with 12 row
// waves from 24 rows per CU, else two with 8 row waves (measured on 256 CUs:
// 4096, 14336 and 28672 rows; at 28672 x 4096 Q4_K, 112 rows per CU, 12 waves
// 14.02-14.14 us against 14.18-14.20 us with 8; at 28672 x 8192 in two K
// slices, 224 rows per CU, 26.87-27.10 against 27.93-27.94 us).
// hipErrorNotSupported when the shape does not qualify.
template <int F>
hipError_t run_b1r(const uint8_t* w, const float* x, float* y, int out_dim, int bpr, hipStream_t s) {
  if constexpr (!kRowSlots<F>) {
    return hipErrorNotSupported;
  } else {
    constexpr int NCR = F == kQ8_0 ? 5 : 3;
    const int keff = bpr * Geom<F>::bs, U = keff / FastUnit<F>::E;
    const size_t row_bytes = (size_t)bpr * Geom<F>::bb;
    if (U > 64 || keff > 4096 || row_bytes <= (size_t)1024 * (NCR - 1) || row_bytes > (size_t)1024 * NCR)
      return hipErrorNotSupported;
    if (((uintptr_t)w % 16) != 0 || row_bytes % 16 != 0) return hipErrorNotSupported;
    const int cu = device_cu_count();
    if ((long)out_dim < 8L * cu || (long)out_dim > 10L * 12 * cu) return hipErrorNotSupported;
    const bool one = (long)out_dim >= 24L * cu;
    const int nrw = one ? 12 : 8, d = one ? 1 : 2;
    const int n_wg = cu, q = out_dim / n_wg, rem = out_dim % n_wg;
    const int slice_bpr = bpr;
    const int rows_cap = (q + (rem ? 1 : 0) + nrw - 1) / nrw;
    const size_t lds = (size_t)U * Dig<F>::US * sizeof(uint32_t) + (size_t)nrw * d * 1024 * NCR +
                       (size_t)nrw * rows_cap * sizeof(double);
    if (lds > (size_t)lds_limit()) return hipErrorNotSupported;
    auto go = [&](auto kern, int threads) {
      hipError_t e = set_lds_attr(kern, lds);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(kern, dim3((unsigned)n_wg), dim3((unsigned)threads), lds, s, w, x, y, out_dim, bpr, slice_bpr,
                         q, rem, rows_cap);
      return hipGetLastError();
    };
    if (!one && fresh_x()) return go(mv_b1r<F, NCR, 2, 8, kB1rXWCold>, 64 * (kB1rXWCold + 8));
    return one ? go(mv_b1r<F, NCR, 1, 12>, 64 * (kB1rXW + 12)) : go(mv_b1r<F, NCR, 2, 8>, 64 * (kB1rXW + 8));
  }
}

// Fused decode-layer launch on the LDS row slots (mv_b1r_fused): whole rows as
// run_b1r takes them, every segment 16-byte aligned, at least one row pair per
// CU.  hipErrorNotSupported when the shape does not qualify.
template <int F, int MODE>
hipError_t run_b1r_fused(const MatvecFuse& f, const float* x, int vrows, int bpr, hipStream_t s) {
  if constexpr (!kRowSlots<F>) {
    return hipErrorNotSupported;
  } else {
    constexpr int NCR = F == kQ8_0 ? 5 : 3;
    const int keff = bpr * Geom<F>::bs, U = keff / FastUnit<F>::E;
    const size_t row_bytes = (size_t)bpr * Geom<F>::bb;
    if (U > 64 || keff > 4096 || row_bytes <= (size_t)1024 * (NCR - 1) || row_bytes > (size_t)1024 * NCR)
      return hipErrorNotSupported;
    for (const uint8_t* w : {f.w0, f.w1, f.w2})
      if (w && (uintptr_t)w % 16 != 0) return hipErrorNotSupported;
    if (row_bytes % 16 != 0) return hipErrorNotSupported;
    const int cu = device_cu_count();
    const int pairs = vrows / 2;
    if (pairs < cu) return hipErrorNotSupported;
    const int q = pairs / cu, rem = pairs % cu;
    // Row waves and rows in flight per wave, measured (kernel in a HIP graph,
    // Q4_K rows of 4096; (row waves, rows in flight) = (8, 2) / (12, 2) /
    // (8, 1) / (12, 1)): QKV + RoPE 6144 rows, 24 per CU, 6.81 / 8.09 / 7.34 /
    // 7.63 us; SwiGLU 2 x 14336 rows, 112 per CU, 14.83 / 13.94 / 16.02 /
    // 13.82 us.  mv_b1 took 8.00 and 16.47 us.
    const bool many = q >= 24;  // at least 48 rows per workgroup
    const int nrw = many ? 12 : 8, d = many ? 1 : 2;
    const int rows_cap = 2 * ((q + (rem ? 1 : 0) + nrw - 1) / nrw);
    const size_t lds = (size_t)U * Dig<F>::US * sizeof(uint32_t) + (size_t)nrw * d * 1024 * NCR +
                       (size_t)nrw * rows_cap * sizeof(double) + 2 * kB1rXWCold * sizeof(float);
    if (lds > (size_t)lds_limit()) return hipErrorNotSupported;
    auto go = [&](auto kern, int threads) {
      hipError_t e = set_lds_attr(kern, lds);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(kern, dim3((unsigned)cu), dim3((unsigned)threads), lds, s, x, vrows, bpr, q, rem, rows_cap,
                         f);
      return hipGetLastError();
    };
    return many ? go(mv_b1r_fused<F, NCR, 1, 12, MODE>, 64 * (kB1rXW + 12))
                : go(mv_b1r_fused<F, NCR, 2, 8, MODE, kB1rXWCold>, 64 * (kB1rXWCold + 8));
  }
}

// Types whose K-sliced rows (slices of at most 2 KB) take mv_b1r.
template <int F>
constexpr bool kSliceSlots = F == kQ6_K || F == kQ4_K;

template <int F, int NCR>
hipError_t run_b1r_sliced_ncr(const uint8_t* w, const float* x, double* part, int out_dim, int row_bpr,
                              int slice_bpr, int slices, hipStream_t s);

// mv_b1r over K slices of slice_bpr blocks (partials as doubles in part,
// [slice][row], for slice_reduce_kernel): one workgroup per CU and slice, each
// owning a run of rows of its slice, 2 KB slots, or 3 KB for slices of up to
// 3 KB (slices start 16-byte aligned in memory; 28672 x 8192 Q4_K, two slices
// of 2304 bytes: 27.6 us on the LDS row streams of mv_b1s_lds, 26.9 us here).
// Rows per workgroup decide the wave layout as in run_b1r.
// hipErrorNotSupported when the shape does not qualify.
template <int F>
hipError_t run_b1r_sliced(const uint8_t* w, const float* x, double* part, int out_dim, int row_bpr, int slice_bpr,
                          int slices, hipStream_t s) {
  if constexpr (!kSliceSlots<F>) {
    return hipErrorNotSupported;
  } else {
    const size_t slice_bytes = (size_t)slice_bpr * Geom<F>::bb;
    if (slice_bytes > 2048) return run_b1r_sliced_ncr<F, 3>(w, x, part, out_dim, row_bpr, slice_bpr, slices, s);
    return run_b1r_sliced_ncr<F, 2>(w, x, part, out_dim, row_bpr, slice_bpr, slices, s);
  }
}

template <int F, int NCR>
hipError_t run_b1r_sliced_ncr(const uint8_t* w, const float* x, double* part, int out_dim, int row_bpr,
                              int slice_bpr, int slices, hipStream_t s) {
  {
    const int keff = slice_bpr * Geom<F>::bs, U = keff / FastUnit<F>::E;
    const size_t slice_bytes = (size_t)slice_bpr * Geom<F>::bb, row_bytes = (size_t)row_bpr * Geom<F>::bb;
    if (slices < 2 || U > 64 || keff > 4096 || slice_bytes > (size_t)1024 * NCR) return hipErrorNotSupported;
    if (((uintptr_t)w % 16) != 0 || row_bytes % 16 != 0 || slice_bytes % 16 != 0) return hipErrorNotSupported;
    const int cu = device_cu_count();
    const int n_wg = std::max(1, cu / slices), q = out_dim / n_wg, rem = out_dim % n_wg;
    if (q < 8) return hipErrorNotSupported;
    const bool one = q >= 24;
    const int nrw = one ? 12 : 8, d = one ? 1 : 2;
    const int rows_cap = (q + (rem ? 1 : 0) + nrw - 1) / nrw;
    const size_t lds = (size_t)U * Dig<F>::US * sizeof(uint32_t) + (size_t)nrw * d * 1024 * NCR +
                       (size_t)nrw * rows_cap * sizeof(double);
    if (lds > (size_t)lds_limit()) return hipErrorNotSupported;
    auto go = [&](auto kern, int threads) {
      hipError_t e = set_lds_attr(kern, lds);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(kern, dim3((unsigned)n_wg, (unsigned)slices), dim3((unsigned)threads), lds, s, w, x,
                         reinterpret_cast<float*>(part), out_dim, row_bpr, slice_bpr, q, rem, rows_cap);
      return hipGetLastError();
    };
    return one ? go(mv_b1r<F, NCR, 1, 12>, 64 * (kB1rXW + 12)) : go(mv_b1r<F, NCR, 2, 8>, 64 * (kB1rXW + 8));
  }
}

template <int F>
size_t b1_workspace_floats(int out_dim, int bpr) {
  const B1Plan<F> p = b1_plan<F>(bpr, out_dim);
  return p.slices > 1 ? (size_t)2 * p.slices * out_dim : 0;  // double partials
}

// acc non-null: acc = acc_in + W x (acc_in null: acc itself) instead of y =
// W x, with y receiving W x (K-sliced rows add acc_in in the slice reduction).
template <int F>
hipError_t b1_dispatch(const uint8_t* w, const float* x, float* y, int out_dim, int bpr,
                       hipStream_t s, float* ws, size_t ws_floats, bool* used, float* acc = nullptr,
                       const float* acc_in = nullptr) {
  if (acc && !acc_in) acc_in = acc;
  const int U = bpr * Geom<F>::bs / FastUnit<F>::E;
  if (U == 0) return hipSuccess;
  {
    hipError_t e = run_b1s_lds_rows<F>(w, x, y, out_dim, bpr, s);
    if (e == hipErrorNotSupported) e = run_b1r<F>(w, x, y, out_dim, bpr, s);
    if (e != hipErrorNotSupported) {
      *used = e == hipSuccess;
      if (e != hipSuccess) return e;
      return acc ? launch_add(acc, acc_in, y, out_dim, s) : hipSuccess;
    }
  }
  const B1Plan<F> p = b1_plan<F>(bpr, out_dim);
  // K-slice partials are doubles: an 8-byte aligned workspace of two floats each
  if (p.slices > 1 && (!ws || ((uintptr_t)ws & 7) || ws_floats < (size_t)2 * p.slices * out_dim)) return hipSuccess;
  float* dst = p.slices > 1 ? ws : y;
  *used = true;
  hipError_t e;
  if (p.slices > 1 && p.upl == 1) {  // K slices through LDS row slots
    e = run_b1r_sliced<F>(w, x, reinterpret_cast<double*>(ws), out_dim, bpr, p.slice_bpr, p.slices, s);
    if (e != hipErrorNotSupported) {
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(slice_reduce_kernel, dim3((unsigned)((out_dim + 255) / 256)), dim3(256), 0, s,
                         reinterpret_cast<const double*>(ws), acc ? acc : y, out_dim, p.slices, acc_in, y);
      return hipGetLastError();
    }
  }
  // (Four waves sharing each row of 129-256 units, summed in LDS, avoid the
  // slices' partials and second launch, but every workgroup then stages the
  // whole x: 4096 x 14336 Q4_K took 15.6 us against 14.0 us sliced.)
  // Rows per wave (one unit per lane): the fewest of 2, 4, 5, 6, 8, 10 whose
  // workgroups (one per CU, 12 row streams each, as run_b1_sit sizes the grid)
  // fit one round, else the fewest rounds x rows.  Rows past a wave's share are
  // still loaded (clamped), so spare capacity costs bandwidth; a second round
  // costs a whole round.  4096 x 4096 Q4_0: 2 rows, 5.55 -> 4.92 us; 4096 x
  // 14336 Q4_K (4 slices): 8 rows, 18.2 -> 14.0 us; 14336 x 4096: 5 rows.
  auto rounds = [&](int rmax) {
    const long cu = device_cu_count(), streams = (out_dim + rmax - 1) / rmax;
    long n_wg = std::max<long>(cu / p.slices, (streams + 11) / 12);
    n_wg = std::max<long>(1, std::min<long>(n_wg, (out_dim + 11) / 12));
    return (n_wg * p.slices + cu - 1) / cu;
  };
  int rsl = 0;
  for (int cand : {2, 4, 5, 6, 8, 10})
    if (!rsl && rounds(cand) == 1) rsl = cand;
  // Rows cut into 2-4 K slices of one unit per lane, and matrices that take
  // more than one round of mv_b1 workgroups, run as long per-wave row streams
  // (mv_b1s), kernel alone: 4096 x 14336 Q4_K 12.9 -> 9.5 us, 8192 x 8192 Q4_K
  // 11.3 -> 9.8 us, 14336 x 4096 Q6_K 14.1 -> 12.9 us, 28672 x 8192 Q4_K 30.2 ->
  // 25.6 us.  Whole rows that fit one round (14336 x 4096 Q4_K: 8.4 against
  // 9.2 us) and rows of 7 slices (4096 x 14336 Q6_K: no gain) stay on mv_b1.
  if (p.upl == 1 && ((p.slices > 1 && p.slices <= 4) || !rsl)) {
    e = p.full ? run_b1s<F, true>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, s)
               : run_b1s<F, false>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, s);
    if (e != hipErrorNotSupported) {
      if (e != hipSuccess) return e;
      if (p.slices == 1) return acc ? launch_add(acc, acc_in, y, out_dim, s) : hipSuccess;
      hipLaunchKernelGGL(slice_reduce_kernel, dim3((unsigned)((out_dim + 255) / 256)), dim3(256), 0, s,
                         reinterpret_cast<const double*>(ws), acc ? acc : y, out_dim, p.slices, acc_in, y);
      return hipGetLastError();
    }
  }
  if (!rsl) {
    rsl = 5;
    for (int cand : {8, 10})
      if (rounds(cand) * cand < rounds(rsl) * rsl) rsl = cand;
  }
  if (p.upl == 1 && rsl == 10)
    e = p.full ? run_b1<F, 1, 10, true>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s)
               : run_b1<F, 1, 10, false>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s);
  else if (p.upl == 1 && rsl == 8)
    e = p.full ? run_b1<F, 1, 8, true>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s)
               : run_b1<F, 1, 8, false>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s);
  else if (p.upl == 1 && rsl == 4)
    e = p.full ? run_b1<F, 1, 4, true>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s)
               : run_b1<F, 1, 4, false>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s);
  else if (p.upl == 1 && rsl == 6)
    e = p.full ? run_b1<F, 1, 6, true>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s)
               : run_b1<F, 1, 6, false>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s);
  else if (p.upl == 1 && rsl == 2)
    e = p.full ? run_b1<F, 1, 2, true>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s)
               : run_b1<F, 1, 2, false>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s);
  else if (p.upl == 1)
    e = p.full ? run_b1<F, 1, 5, true>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s)
               : run_b1<F, 1, 5, false>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s);
  else if constexpr (kTwoUnits<F>)
    e = p.full ? run_b1<F, 2, 3, true>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s)
               : run_b1<F, 2, 3, false>(w, x, dst, out_dim, bpr, p.slice_bpr, p.slices, 1, s);
  else
    e = hipErrorNotSupported;  // b1_plan gives these types one unit per lane
  if (e == hipErrorNotSupported) {  // not launched: the caller takes the batched path
    *used = false;
    return hipSuccess;
  }
  if (e != hipSuccess) return e;
  if (p.slices == 1) return acc ? launch_add(acc, acc_in, y, out_dim, s) : hipSuccess;
  hipLaunchKernelGGL(slice_reduce_kernel, dim3((unsigned)((out_dim + 255) / 256)), dim3(256), 0, s,
                     reinterpret_cast<const double*>(ws), acc ? acc : y, out_dim, p.slices, acc_in, y);
  return hipGetLastError();
}

// Fused decode-layer launch: whole rows (one slice), pairs of rows per wave.
template <int F, int UPL, int RMAX, int SIT, int MODE>
hipError_t run_fused_sit(const MatvecFuse& f, const float* x, int vrows, int bpr, int rs, size_t lds,
                         hipStream_t s) {
  auto kern = mv_b1<F, UPL, RMAX, true, SIT, MODE>;
  hipError_t e = set_lds_attr(kern, lds);
  if (e != hipSuccess) return e;
  // streams of row pairs, at most RMAX rows each
  const long units = vrows / 2, per = RMAX / 2;
  const long streams_needed = (units + per - 1) / per;
  long n_wg = std::max<long>(device_cu_count(), (streams_needed + rs - 1) / rs);
  n_wg = std::max<long>(1, std::min<long>(n_wg, (units + rs - 1) / rs));
  if (n_wg > device_cu_count()) {
    // paired rows in more than one round of workgroups measured slower than
    // the separate launches (one row chain per wave grows too long)
    return hipErrorNotSupported;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)n_wg), dim3(64 * rs), lds, s, nullptr, x, nullptr, vrows, bpr,
                     bpr, 1, false, f);
  return hipGetLastError();
}

template <int F, int UPL, int RMAX, int MODE>
hipError_t run_fused(const MatvecFuse& f, const float* x, int vrows, int bpr, hipStream_t s, bool* used) {
  const int U = bpr * Geom<F>::bs / FastUnit<F>::E;
  const size_t lds = ((size_t)U * Dig<F>::US + RMAX) * sizeof(uint32_t);
  if (lds > (size_t)lds_limit()) return hipSuccess;
  static std::mutex mu;
  static std::map<std::pair<int, size_t>, int> rs_cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  int rs = 0;
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = rs_cache.find({dev, lds});
    if (it != rs_cache.end()) rs = it->second;
  }
  if (rs == 0) {
    auto probe = mv_b1<F, UPL, RMAX, true, MODE >= 3 ? 1 : 2, MODE>;
    hipError_t e = set_lds_attr(probe, lds);
    if (e != hipSuccess) return e;
    rs = 1;
    for (int cand = 12; cand >= 1; cand--) {  // launch bounds: 768 threads
      int per_cu = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, probe, 64 * cand, lds) == hipSuccess && per_cu >= 1) {
        rs = cand;
        break;
      }
    }
    std::lock_guard<std::mutex> lk(mu);
    rs_cache[{dev, lds}] = rs;
  }
  const int nchunk = bpr * Geom<F>::bs / 8;
  const int sit = (nchunk + 64 * rs - 1) / (64 * rs);
  hipError_t e;
  if (sit <= 1) e = run_fused_sit<F, UPL, RMAX, 1, MODE>(f, x, vrows, bpr, rs, lds, s);
  else if constexpr (MODE >= 3) return hipSuccess;  // the norm-fused forms stage x in one chunk per thread
  else if (sit <= 2) e = run_fused_sit<F, UPL, RMAX, 2, MODE>(f, x, vrows, bpr, rs, lds, s);
  else return hipSuccess;  // x too long to stage in two chunks per thread
  if (e == hipErrorNotSupported) return hipSuccess;  // more rows than one round: not fused
  *used = (e == hipSuccess);
  return e;
}

template <int F>
hipError_t fused_dispatch(const MatvecFuse& f, int vrows, const float* x, int in_dim, hipStream_t s,
                          bool* used) {
  *used = false;
  if (in_dim % Geom<F>::bs) return hipSuccess;
  const int bpr = in_dim / Geom<F>::bs;
  const int U = bpr * Geom<F>::bs / FastUnit<F>::E;
  if (U == 0 || (U != 64 && U != 128)) return hipSuccess;  // whole units per lane, one slice
  for (const uint8_t* w : {f.w0, f.w1, f.w2})
    if (w && !fast_aligned<F>(w, x, in_dim, bpr)) return hipSuccess;
  {  // whole Q4_K / Q4_0 / Q8_0 rows of 3584-4096 elements: the LDS row slots
    hipError_t e = !f.norm_w   ? run_b1r_fused<F, 2>(f, x, vrows, bpr, s)
                   : f.norm_res ? run_b1r_fused<F, 4>(f, x, vrows, bpr, s)
                                : run_b1r_fused<F, 3>(f, x, vrows, bpr, s);
    if (e != hipErrorNotSupported) {
      *used = e == hipSuccess;
      return e;
    }
  }
  if (f.norm_w) {
    // the norm-fused forms: the row counts of the Llama-3-8B-sized layers (QKV
    // 6144 rows: 2 per wave; SwiGLU 2 x 14336: 10), one unit per lane; other
    // shapes take a separate norm launch and the plain fused kernel
    if (U != 64) return hipSuccess;
    hipError_t e = f.norm_res ? run_fused<F, 1, 2, 4>(f, x, vrows, bpr, s, used)
                              : run_fused<F, 1, 2, 3>(f, x, vrows, bpr, s, used);
    if (e != hipSuccess || *used) return e;
    // more rows: 10 per wave, but only where that is the fewest that fit one
    // round (12 waves per workgroup, one workgroup per CU)
    for (int rmax : {4, 6})
      if ((vrows / 2 + rmax / 2 - 1) / (rmax / 2) <= 12L * device_cu_count()) return hipSuccess;
    return f.norm_res ? run_fused<F, 1, 10, 4>(f, x, vrows, bpr, s, used)
                      : run_fused<F, 1, 10, 3>(f, x, vrows, bpr, s, used);
  }
  if (U == 64) {
    // the fewest rows per wave that still fit one round of workgroups: rows
    // past a wave's share are still loaded (clamped), so spare capacity costs
    // bandwidth (SwiGLU 2 x 14336: 10 rows 9.3 in use; QKV 6144: 2 rows)
    hipError_t e = run_fused<F, 1, 2, 2>(f, x, vrows, bpr, s, used);
    if (e != hipSuccess || *used) return e;
    e = run_fused<F, 1, 4, 2>(f, x, vrows, bpr, s, used);
    if (e != hipSuccess || *used) return e;
    e = run_fused<F, 1, 6, 2>(f, x, vrows, bpr, s, used);
    if (e != hipSuccess || *used) return e;
    e = run_fused<F, 1, 10, 2>(f, x, vrows, bpr, s, used);
    if (e != hipSuccess || *used) return e;
    return run_fused<F, 1, 12, 2>(f, x, vrows, bpr, s, used);
  }
  // two units per lane (kTwoUnits: Q6_K); the other types' rows take the
  // separate launches
  if constexpr (kTwoUnits<F>) return run_fused<F, 2, 4, 2>(f, x, vrows, bpr, s, used);
  return hipSuccess;
}

// K slices of the small-batch kernel: one unit per lane, at most 64 per slice.
template <int F>
B1Plan<F> bn_plan(int bpr) {
  const int U = bpr * Geom<F>::bs / FastUnit<F>::E;
  B1Plan<F> p;
  if (U == 0) {  // rows shorter than one unit: one empty slice
    p.slice_bpr = bpr;
    p.full = false;
    return p;
  }
  p.slices = (U + 63) / 64;
  int sb = (bpr + p.slices - 1) / p.slices;
  if constexpr (Geom<F>::bs == 32) sb += sb & 1;  // Q4_0 / Q8_0: two blocks per unit
  p.slice_bpr = sb;
  p.slices = (bpr + sb - 1) / sb;
  p.full = (bpr % sb == 0) && sb * Geom<F>::bs / FastUnit<F>::E == 64;
  return p;
}

template <int F>
size_t bn_workspace_floats(int out_dim, int bpr, int nb) {
  const B1Plan<F> p = bn_plan<F>(bpr);
  return p.slices > 1 ? (size_t)2 * p.slices * nb * out_dim : 0;  // double partials
}

// Rows per wave of mv_bn and rows per group (planes read once per group); 4-8
// activation rows keep 3 rows per wave, so that the double row sums fit the
// registers beside the row buffers
template <int NB> constexpr int kBnRows = NB >= 4 ? 3 : 6;
template <int NB> constexpr int kBnGroup = NB >= 4 ? 3 : 2;

template <int F, int NB, int RMAX, int RG, bool FULL>
hipError_t run_bn(const uint8_t* w, const float* x, float* dst, int out_dim, int in_dim, int row_bpr,
                  int slice_bpr, int slices, hipStream_t s) {
  const int U = slice_bpr * Geom<F>::bs / FastUnit<F>::E;
  const size_t lds = (size_t)NB * U * Dig<F>::US * sizeof(uint32_t);
  if (lds > (size_t)lds_limit()) return hipErrorNotSupported;
  // waves per workgroup: as many as fit with one workgroup per CU (cached per
  // device and LDS size, probed on the deepest staging instantiation)
  static std::mutex mu;
  static std::map<std::pair<int, size_t>, int> rs_cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  int rs = 0;
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = rs_cache.find({dev, lds});
    if (it != rs_cache.end()) rs = it->second;
  }
  if (rs == 0) {
    auto probe = mv_bn<F, NB, RMAX, RG, FULL, 8>;
    hipError_t e = set_lds_attr(probe, lds);
    if (e != hipSuccess) return e;
    rs = 1;
    for (int cand = 8; cand >= 1; cand--) {  // launch bounds: 512 threads
      int per_cu = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, probe, 64 * cand, lds) == hipSuccess && per_cu >= 1) {
        rs = cand;
        break;
      }
    }
    std::lock_guard<std::mutex> lk(mu);
    rs_cache[{dev, lds}] = rs;
  }
  const int threads = 64 * rs;
  const int nchunk = NB * (slice_bpr * Geom<F>::bs / 8);
  const int sit = (nchunk + threads - 1) / threads;
  const long streams_needed = (out_dim + RMAX - 1) / RMAX;
  long n_wg = std::max<long>(device_cu_count() / slices, (streams_needed + rs - 1) / rs);  // as in run_b1_sit
  n_wg = std::max<long>(1, std::min<long>(n_wg, (out_dim + rs - 1) / rs));
  const bool interleave = F == kQ8_0;
  auto launch = [&](auto kern) {
    hipError_t e = set_lds_attr(kern, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3((unsigned)n_wg, (unsigned)slices), dim3(threads), lds, s, w, x, dst,
                       out_dim, in_dim, row_bpr, slice_bpr, interleave);
    return hipGetLastError();
  };
  if (sit <= 1) return launch(mv_bn<F, NB, RMAX, RG, FULL, 1>);
  if (sit <= 2) return launch(mv_bn<F, NB, RMAX, RG, FULL, 2>);
  if (sit <= 4) return launch(mv_bn<F, NB, RMAX, RG, FULL, 4>);
  if (sit <= 8) return launch(mv_bn<F, NB, RMAX, RG, FULL, 8>);
  return hipErrorNotSupported;
}

// One chunk of NB activation rows; *used = false when the kernel cannot take it.
template <int F, int NB>
hipError_t bn_dispatch(const uint8_t* w, const float* x, float* y, int out_dim, int in_dim, int bpr,
                       hipStream_t s, float* ws, size_t ws_floats, bool* used) {
  const B1Plan<F> p = bn_plan<F>(bpr);
  *used = false;
  if (p.slices > 1 && (!ws || ((uintptr_t)ws & 7) || ws_floats < (size_t)2 * p.slices * NB * out_dim))
    return hipSuccess;
  float* dst = p.slices > 1 ? ws : y;
  constexpr int R = kBnRows<NB>, G = kBnGroup<NB>;
  hipError_t e = p.full ? run_bn<F, NB, R, G, true>(w, x, dst, out_dim, in_dim, bpr, p.slice_bpr, p.slices, s)
                        : run_bn<F, NB, R, G, false>(w, x, dst, out_dim, in_dim, bpr, p.slice_bpr, p.slices, s);
  if (e == hipErrorNotSupported) return hipSuccess;
  if (e != hipSuccess) return e;
  *used = true;
  if (p.slices == 1) return hipSuccess;
  const int n = NB * out_dim;
  hipLaunchKernelGGL(slice_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     reinterpret_cast<const double*>(ws), y, n, p.slices, nullptr, nullptr);
  return hipGetLastError();
}

// The batch-1 digit-plane kernel alone, for the types whose float path is
// mv_ext (their batches stay on mv_ext): *used = false when it does not apply.
template <int F>
hipError_t digit_dispatch(const uint8_t* w, const float* x, float* y, int out_dim, int in_dim, int bpr,
                          int batch, hipStream_t s, float* ws, size_t ws_floats, bool* used) {
  *used = false;
  if (batch != 1 || bpr == 0 || !fast_aligned<F>(w, x, in_dim, bpr)) return hipSuccess;
  return b1_dispatch<F>(w, x, y, out_dim, bpr, s, ws, ws_floats, used);
}

template <int F>
hipError_t fast_dispatch(const uint8_t* w, const float* x, float* y, int out_dim, int in_dim,
                         int bpr, int batch, hipStream_t s, float* ws, size_t ws_floats,
                         bool* used) {
  *used = false;
  // rows shorter than one block: the generic path writes the (zero) sums
  if (bpr == 0 || !fast_aligned<F>(w, x, in_dim, bpr)) return hipSuccess;
  const int keff = bpr * Geom<F>::bs;
  const int U = keff / FastUnit<F>::E;
  const int limit = lds_limit();
  if (batch == 1) {
    hipError_t e = b1_dispatch<F>(w, x, y, out_dim, bpr, s, ws, ws_floats, used);
    if (e != hipSuccess || *used) return e;
  } else {
    // chunks of 8 / 4 / 2 activation rows on mv_bn, a last single row on mv_b1
    // (the first chunk decides: every chunk has the same row geometry); Q8_0
    // chunks of 2-8 rows at K = 1024 / 2048 / 4096 run on the matrix cores
    int b0 = 0;
    while (b0 < batch) {
      const int left = batch - b0;
      const float* xb = x + (size_t)b0 * in_dim;
      float* yb = y + (size_t)b0 * out_dim;
      bool u = false;
      hipError_t e;
      int take;
      if (F == kQ8_0 && left >= 2 && q8_mfma_supported(w, xb, in_dim, std::min(left, 8))) {
        take = std::min(left, 8);
        e = launch_q8_mfma(w, xb, yb, out_dim, in_dim, take, s);
        u = e == hipSuccess;
        if (e == hipErrorNotSupported) e = hipSuccess;
      }
      else if (left >= 8) { take = 8; e = bn_dispatch<F, 8>(w, xb, yb, out_dim, in_dim, bpr, s, ws, ws_floats, &u); }
      else if (left >= 4) { take = 4; e = bn_dispatch<F, 4>(w, xb, yb, out_dim, in_dim, bpr, s, ws, ws_floats, &u); }
      else if (left >= 2) { take = 2; e = bn_dispatch<F, 2>(w, xb, yb, out_dim, in_dim, bpr, s, ws, ws_floats, &u); }
      else { take = 1; e = b1_dispatch<F>(w, xb, yb, out_dim, bpr, s, ws, ws_floats, &u); }
      if (e != hipSuccess) return e;
      if (!u) {
        if (b0 == 0) break;  // nothing launched: the paths below take the whole batch
        return hipErrorInvalidValue;
      }
      b0 += take;
    }
    if (b0 == batch) {
      *used = true;
      return hipSuccess;
    }
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
      case 8: e = run_lds<F, 8, 2>(w, xb, yb, out_dim, in_dim, bpr, lds, s); break;
      case 4: e = run_lds<F, 4, 2>(w, xb, yb, out_dim, in_dim, bpr, lds, s); break;
      case 2: e = run_lds<F, 2, 2>(w, xb, yb, out_dim, in_dim, bpr, lds, s); break;
      default: e = run_lds<F, 1, 4>(w, xb, yb, out_dim, in_dim, bpr, lds, s); break;
    }
    if (e != hipSuccess) return e;
    *used = true;
    b0 += take;
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_matvec_fused(int dtype, const MatvecFuse& f, int total_rows, const float* x,
                               size_t in_dim, hipStream_t s, bool* used) {
  *used = false;
  if (total_rows <= 0 || (total_rows & 1) || in_dim > (size_t)INT_MAX) return hipSuccess;
  switch (dtype) {
    case kQ4_0: return fused_dispatch<kQ4_0>(f, total_rows, x, (int)in_dim, s, used);
    case kQ8_0: return fused_dispatch<kQ8_0>(f, total_rows, x, (int)in_dim, s, used);
    case kQ4_K: return fused_dispatch<kQ4_K>(f, total_rows, x, (int)in_dim, s, used);
    case kQ6_K: return fused_dispatch<kQ6_K>(f, total_rows, x, (int)in_dim, s, used);
    default: return hipSuccess;
  }
}

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

template <int F>
size_t ws_floats_for(int od, int bpr, size_t batch) {
  size_t n = b1_workspace_floats<F>(od, bpr);  // batch 1, or the last single row of a batch
  if (batch > 1) n = std::max(n, bn_workspace_floats<F>(od, bpr, (int)std::min<size_t>(batch, 8)));
  return n;
}

size_t matvec_digit_ext_workspace_bytes(int dtype, const void* w, const float* x, size_t out_dim, size_t in_dim,
                                        size_t batch) {
  if (out_dim == 0 || batch == 0) return 0;
  const int od = (int)out_dim, id = (int)in_dim, bpr = id / 256;
  const uint8_t* wb = (const uint8_t*)w;
  switch (dtype) {
    case kQ5_K: return fast_aligned<kQ5_K>(wb, x, id, bpr) ? ws_floats_for<kQ5_K>(od, bpr, batch) * 4 : 0;
    case kQ2_K: return fast_aligned<kQ2_K>(wb, x, id, bpr) ? ws_floats_for<kQ2_K>(od, bpr, batch) * 4 : 0;
    case kQ3_K: return fast_aligned<kQ3_K>(wb, x, id, bpr) ? ws_floats_for<kQ3_K>(od, bpr, batch) * 4 : 0;
    case kQ8_K: return 0;  // whole rows only (see launch_matvec_digit_ext)
    default: return 0;
  }
}

hipError_t launch_matvec_digit_ext(int dtype, const uint8_t* w, const float* x, float* y, size_t out_dim,
                                   size_t in_dim, size_t batch, hipStream_t s, void* workspace,
                                   size_t workspace_bytes, bool* used) {
  *used = false;
  if (out_dim == 0 || batch == 0) return hipSuccess;
  const int od = (int)out_dim, id = (int)in_dim, bpr = id / 256, b = (int)batch;
  float* ws = static_cast<float*>(workspace);
  const size_t wf = workspace_bytes / sizeof(float);
  switch (dtype) {
    case kQ5_K: return digit_dispatch<kQ5_K>(w, x, y, od, id, bpr, b, s, ws, wf, used);
    case kQ2_K: return digit_dispatch<kQ2_K>(w, x, y, od, id, bpr, b, s, ws, wf, used);
    case kQ3_K: return digit_dispatch<kQ3_K>(w, x, y, od, id, bpr, b, s, ws, wf, used);
    case kQ8_K:
      // rows of up to 128 units without workspace: K-sliced Q8_K rows (4096 x
      // 14336) measured no faster than mv_ext (20.6 against 19.6 us); 14336 x
      // 4096 at batch 1: 16.8 -> 14.3 us
      if (bpr * 4 > 128) return hipSuccess;
      return digit_dispatch<kQ8_K>(w, x, y, od, id, bpr, b, s, nullptr, 0, used);
    default: return hipSuccess;
  }
}

size_t matvec_workspace_bytes(int dtype, const void* w, const float* x, size_t out_dim,
                              size_t in_dim, size_t batch) {
  if (batch == 0 || out_dim == 0) return 0;
  const uint8_t* wb = (const uint8_t*)w;
  const int od = (int)out_dim, id = (int)in_dim;
  size_t n = 0;
  switch (dtype) {
    case kQ4_0: if (fast_aligned<kQ4_0>(wb, x, id, id / 32)) n = ws_floats_for<kQ4_0>(od, id / 32, batch); break;
    case kQ8_0: if (fast_aligned<kQ8_0>(wb, x, id, id / 32)) n = ws_floats_for<kQ8_0>(od, id / 32, batch); break;
    case kQ4_K: if (fast_aligned<kQ4_K>(wb, x, id, id / 256)) n = ws_floats_for<kQ4_K>(od, id / 256, batch); break;
    case kQ6_K: if (fast_aligned<kQ6_K>(wb, x, id, id / 256)) n = ws_floats_for<kQ6_K>(od, id / 256, batch); break;
    default: break;
  }
  return n * sizeof(float);
}

hipError_t launch_matvec_acc(int dtype, const uint8_t* w, const float* x, float* acc, float* y, size_t out_dim,
                             size_t in_dim, hipStream_t s, void* workspace, size_t workspace_bytes,
                             const float* acc_in) {
  if (!acc_in) acc_in = acc;
  if (out_dim == 0) return hipSuccess;
  bool used = false;
  hipError_t e = hipSuccess;
  const int od = (int)out_dim, id = (int)in_dim;
  float* ws = static_cast<float*>(workspace);
  const size_t wf = workspace_bytes / sizeof(float);
  auto go = [&](auto f_c, int bpr) {
    constexpr int F = decltype(f_c)::value;
    if (bpr == 0 || !fast_aligned<F>(w, x, id, bpr)) return hipSuccess;
    return b1_dispatch<F>(w, x, y, od, bpr, s, ws, wf, &used, acc, acc_in);
  };
  switch (dtype) {
    case kQ4_0: e = go(std::integral_constant<int, kQ4_0>{}, id / 32); break;
    case kQ8_0: e = go(std::integral_constant<int, kQ8_0>{}, id / 32); break;
    case kQ4_K: e = go(std::integral_constant<int, kQ4_K>{}, id / 256); break;
    case kQ6_K: e = go(std::integral_constant<int, kQ6_K>{}, id / 256); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess || used) return e;
  e = launch_matvec(dtype, w, x, y, out_dim, in_dim, 1, s, workspace, workspace_bytes);
  if (e != hipSuccess) return e;
  return launch_add(acc, acc_in, y, od, s);
}

hipError_t launch_matvec(int dtype, const uint8_t* w, const float* x, float* y, size_t out_dim,
                         size_t in_dim, size_t batch, hipStream_t s, void* workspace,
                         size_t workspace_bytes) {
  if (out_dim == 0 || batch == 0) return hipSuccess;
  bool used = false;
  hipError_t e = hipSuccess;
  const int od = (int)out_dim, id = (int)in_dim, b = (int)batch;
  float* ws = static_cast<float*>(workspace);
  const size_t wf = workspace_bytes / sizeof(float);
  switch (dtype) {
    case kQ4_0: e = fast_dispatch<kQ4_0>(w, x, y, od, id, id / 32, b, s, ws, wf, &used); break;
    case kQ8_0: e = fast_dispatch<kQ8_0>(w, x, y, od, id, id / 32, b, s, ws, wf, &used); break;
    case kQ4_K: e = fast_dispatch<kQ4_K>(w, x, y, od, id, id / 256, b, s, ws, wf, &used); break;
    case kQ6_K: e = fast_dispatch<kQ6_K>(w, x, y, od, id, id / 256, b, s, ws, wf, &used); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess || used) return e;
  return launch_matvec_generic(dtype, w, x, y, out_dim, in_dim, batch, s);
}

}  // namespace ssdq
