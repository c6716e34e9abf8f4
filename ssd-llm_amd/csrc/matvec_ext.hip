// Dequant-matvec for the reference's other matvec_quantized types: Q2_K,
// Q3_K, Q5_K, Q8_K, IQ4_NL, IQ4_XS, F16 and BF16 (src/metal/compute.rs:
// 796-1077 and 2249-2285, dispatched at 655-671).  Same contract as the four
// main types: y[b*out_dim + r] = sum over the whole blocks of row r of
// elem(W[r,k]) * x[b*in_dim + k], with the reference's block layouts and
// element order.
//
// Design: HBM-bound like the main matvec, but these formats trade fewer bits
// for more decode work, so the per-element VALU cost is what is kept small:
//  * x for up to 8 activations is staged once per workgroup in LDS (32-float
//    groups padded to 36 so 16 consecutive lanes hit disjoint banks), with the
//    sum of each 16-element half precomputed.
//  * A lane owns 32-element groups of every row it visits and loads them with
//    dword loads (2-byte-aligned blocks, Q3_K and IQ4_NL, are read from the
//    dword below and realigned with v_alignbit).
//  * Codes are widened a dword at a time (masks / shifts leave one code per
//    byte, v_cvt_f32_ubyteN converts), so the inner loop is one conversion and
//    one FMA per element; scales and offsets apply once per 16-element half:
//    acc += S * sum(u x) - O * sum(x).  Signed codes and the IQ4 code book are
//    biased by +128 (O = 128 S) so every code converts from an unsigned byte.
//  * IQ4 code-book lookups are two v_perm_b32 over the table held in four
//    dwords, merged on bit 3 of the index.
// A byte-addressed fallback kernel takes unaligned operands.
#include <algorithm>

#include "common.hpp"
#include "launch.hpp"
#define SSDQ_IQ_GRIDS_DEVICE_ONLY
#include "iq_grids.h"

namespace ssdq {
namespace {

enum : int {
  kF16 = 1, kIQ2_XXS = 16, kIQ2_XS = 17, kIQ3_XXS = 18,
  kIQ4_NL = 20, kIQ3_S = 21, kIQ4_XS = 23, kBF16 = 30
};

// IQ2 / IQ3 lattice code books (device copies; each workgroup stages its
// type's table into LDS)
__constant__ uint64_t k_iq2xxs_grid[256] = SSDQ_IQ2XXS_GRID_INIT;
__constant__ uint64_t k_iq2xs_grid[512] = SSDQ_IQ2XS_GRID_INIT;
__constant__ uint32_t k_iq3xxs_grid[256] = SSDQ_IQ3XXS_GRID_INIT;
__constant__ uint32_t k_iq3s_grid[512] = SSDQ_IQ3S_GRID_INIT;

template <int F> constexpr bool is_iq_lattice = F == kIQ2_XXS || F == kIQ2_XS || F == kIQ3_XXS || F == kIQ3_S;
// bytes of the type's code book in LDS
template <int F> constexpr int tab_bytes = F == kIQ2_XXS ? 2048 : F == kIQ2_XS ? 4096 : F == kIQ3_XXS ? 1024
                                         : F == kIQ3_S ? 2048 : 0;
template <int F>
__device__ __forceinline__ const uint32_t* tab_src() {
  if constexpr (F == kIQ2_XXS) return reinterpret_cast<const uint32_t*>(k_iq2xxs_grid);
  else if constexpr (F == kIQ2_XS) return reinterpret_cast<const uint32_t*>(k_iq2xs_grid);
  else if constexpr (F == kIQ3_XXS) return k_iq3xxs_grid;
  else return k_iq3s_grid;
}

// KSIGNS_IQ2XS (compute.rs:1964-1973): the 7-bit index with its parity as bit 7
__device__ __forceinline__ uint32_t ksigns(uint32_t i) { return i | ((__popc(i) & 1u) << 7); }

// bs elements / bb bytes per block; NW raw dwords per 32-element group.
template <int F> struct XG;
template <> struct XG<kQ2_K> { static constexpr int bs = 256, bb = 84, NW = 4; };
template <> struct XG<kQ3_K> { static constexpr int bs = 256, bb = 110, NW = 6; };
template <> struct XG<kQ5_K> { static constexpr int bs = 256, bb = 176, NW = 9; };
template <> struct XG<kQ8_K> { static constexpr int bs = 256, bb = 292, NW = 9; };
template <> struct XG<kIQ4_NL> { static constexpr int bs = 32, bb = 18, NW = 6; };
template <> struct XG<kIQ4_XS> { static constexpr int bs = 256, bb = 148, NW = 6; };
template <> struct XG<kF16> { static constexpr int bs = 1, bb = 2, NW = 16; };
template <> struct XG<kBF16> { static constexpr int bs = 1, bb = 2, NW = 16; };
template <> struct XG<kIQ2_XXS> { static constexpr int bs = 256, bb = 66, NW = 3; };
template <> struct XG<kIQ2_XS> { static constexpr int bs = 256, bb = 74, NW = 4; };
template <> struct XG<kIQ3_XXS> { static constexpr int bs = 256, bb = 98, NW = 4; };
template <> struct XG<kIQ3_S> { static constexpr int bs = 256, bb = 110, NW = 6; };

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ void ld4(const uint8_t* p, uint32_t* d) {
  const u32x4a4 v = *reinterpret_cast<const u32x4a4*>(p);
  d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
}
__device__ __forceinline__ uint32_t ld1(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
__device__ __forceinline__ uint32_t ldh(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }

// IQ4_NL code book (compute.rs:997-999), biased by +128 and packed four
// entries per dword for v_perm_b32.
constexpr int kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
constexpr uint32_t lut_dword(int i) {
  return (uint32_t)(kIq4nl[4 * i] + 128) | ((uint32_t)(kIq4nl[4 * i + 1] + 128) << 8) |
         ((uint32_t)(kIq4nl[4 * i + 2] + 128) << 16) | ((uint32_t)(kIq4nl[4 * i + 3] + 128) << 24);
}

// Four 4-bit indices (one per byte) -> four biased code-book bytes.
__device__ __forceinline__ uint32_t iq4_lookup(uint32_t idx4) {
  const uint32_t sel = idx4 & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(lut_dword(1), lut_dword(0), sel);
  const uint32_t hi = __builtin_amdgcn_perm(lut_dword(3), lut_dword(2), sel);
  const uint32_t b3 = idx4 & 0x08080808u;
  const uint32_t mask = (b3 << 5) - (b3 >> 3);  // 0xFF in the bytes whose index is >= 8
  return (hi & mask) | (lo & ~mask);
}

// Loads 32-element group g of one row (raw dwords; every load stays inside the
// group's block, or the two bytes below a 2-byte-aligned block).
template <int F>
__device__ __forceinline__ void load_group(const uint8_t* __restrict__ row, int g, uint32_t* raw) {
  if constexpr (F == kF16 || F == kBF16) {
    const uint8_t* p = row + (size_t)g * 64;
    ld4(p, raw); ld4(p + 16, raw + 4); ld4(p + 32, raw + 8); ld4(p + 48, raw + 12);
  } else if constexpr (F == kQ2_K) {
    const uint8_t* blk = row + (size_t)(g >> 3) * 84;
    const int gi = g & 7;
    raw[0] = ld1(blk);                         // d, dmin
    raw[1] = ld1(blk + 4 + 4 * (gi >> 1));     // sc[2gi], sc[2gi+1] among four
    raw[2] = ld1(blk + 20 + 8 * gi);           // qs of sub-block 2gi
    raw[3] = ld1(blk + 24 + 8 * gi);           // qs of sub-block 2gi+1
  } else if constexpr (F == kQ3_K) {
    const uint8_t* blk = row + (size_t)(g >> 3) * 110;
    const int gi = g & 7;
    const uint32_t mis = (uint32_t)(uintptr_t)blk & 2u;  // 0 or 2
    const uint8_t* b = blk - mis;
    const uint32_t sh = mis * 8u;
    const uint32_t h0 = ld1(b + 4 * gi), h1 = ld1(b + 4 * gi + 4);
    const uint32_t q0 = ld1(b + 32 + 8 * gi), q1 = ld1(b + 36 + 8 * gi), q2 = ld1(b + 40 + 8 * gi);
    raw[0] = __builtin_amdgcn_alignbit(h1, h0, sh);  // hmask bits of the 32 elements
    raw[1] = __builtin_amdgcn_alignbit(q1, q0, sh);  // low-2-bit codes, sub-block 2gi
    raw[2] = __builtin_amdgcn_alignbit(q2, q1, sh);  // sub-block 2gi+1
    raw[3] = ldh(blk + 96 + (gi & ~1)) | (ldh(blk + 104 + ((gi >> 1) & ~1)) << 16);
    raw[4] = ldh(blk + 108);  // d
    raw[5] = 0;
  } else if constexpr (F == kQ5_K) {
    const uint8_t* blk = row + (size_t)(g >> 3) * 176;
    const int sb = g & 7;
    ld4(blk, raw);                      // d, dmin, sc[12]
    raw[4] = ld1(blk + 16 + 4 * sb);    // fifth bits of the 32 elements
    ld4(blk + 48 + 16 * sb, raw + 5);   // nibbles
  } else if constexpr (F == kQ8_K) {
    const uint8_t* blk = row + (size_t)(g >> 3) * 292;
    const int gi = g & 7;
    raw[0] = ld1(blk);  // f32 d
    ld4(blk + 4 + 32 * gi, raw + 1);
    ld4(blk + 20 + 32 * gi, raw + 5);
  } else if constexpr (F == kIQ4_NL) {
    const uint8_t* blk = row + (size_t)g * 18;
    const uint32_t mis = (uint32_t)(uintptr_t)blk & 2u;
    ld4(blk - mis, raw);                               // bytes -mis .. 15-mis
    raw[4] = ldh(blk + 14) | (ldh(blk + 16) << 16);    // bytes 14..17
    raw[5] = mis;
  } else if constexpr (is_iq_lattice<F>) {  // 2-byte-aligned blocks: 16-bit loads
    const uint8_t* blk = row + (size_t)(g >> 3) * XG<F>::bb;
    const int ib = g & 7;
    const uint8_t* q = blk + 2 + 8 * ib;  // grid indices (IQ2_XXS: + signs / scale word)
    raw[0] = ldh(q) | (ldh(q + 2) << 16);
    raw[1] = ldh(q + 4) | (ldh(q + 6) << 16);
    if constexpr (F == kIQ2_XXS) {
      raw[2] = ldh(blk);
    } else if constexpr (F == kIQ2_XS) {
      raw[2] = ldh(blk + 66 + ((ib >> 1) & ~1));  // scale bytes 2(ib/4), 2(ib/4)+1
      raw[3] = ldh(blk);
    } else if constexpr (F == kIQ3_XXS) {
      const uint8_t* a = blk + 66 + 4 * ib;  // scales_and_signs word
      raw[2] = ldh(a) | (ldh(a + 2) << 16);
      raw[3] = ldh(blk);
    } else {  // kIQ3_S
      raw[2] = ldh(blk + 66 + (ib & ~1));            // qh bytes ib&~1, +1
      const uint8_t* sg = blk + 74 + 4 * ib;          // sign bytes of the four 8-groups
      raw[3] = ldh(sg) | (ldh(sg + 2) << 16);
      raw[4] = ldh(blk + 106 + ((ib >> 1) & ~1));     // scale bytes
      raw[5] = ldh(blk);
    }
  } else {  // kIQ4_XS
    const uint8_t* blk = row + (size_t)(g >> 3) * 148;
    const int sb = g & 7;
    raw[0] = ld1(blk);                       // d, scales_h
    raw[1] = ld1(blk + 4 + 4 * (sb >> 2));   // scales_l words 2(sb/4), 2(sb/4)+1
    ld4(blk + 20 + 16 * sb, raw + 2);
  }
}

// Decodes group g: u[e] (integer or code-book values as floats) and per-half
// scale S / offset O, element value = S*u - O.
// Magnitude byte j of a code-book entry, with the sign of bit j of sg.
__device__ __forceinline__ float signed_mag(uint32_t word, int j, uint32_t sg, int sj) {
  const float m = (float)((word >> (8 * j)) & 0xFFu);
  return ((sg >> sj) & 1u) ? -m : m;
}

template <int F>
__device__ __forceinline__ void decode_group(const uint32_t* raw, int g, float* u, float* S, float* O,
                                             const uint32_t* tab = nullptr) {
  if constexpr (F == kF16) {
    // converted explicitly: left to itself the compiler folds the widening
    // into v_fma_mix_f32, which measured 2.5x slower here than cvt + fmac
#pragma unroll
    for (int i = 0; i < 16; i++) {
      u[2 * i] = __uint_as_float(opaque(__float_as_uint(f16_to_f32(raw[i] & 0xFFFFu))));
      u[2 * i + 1] = __uint_as_float(opaque(__float_as_uint(f16_to_f32(raw[i] >> 16))));
    }
    S[0] = S[1] = 1.f;
    O[0] = O[1] = 0.f;
  } else if constexpr (F == kBF16) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      u[2 * i] = __uint_as_float(raw[i] << 16);
      u[2 * i + 1] = __uint_as_float(raw[i] & 0xFFFF0000u);
    }
    S[0] = S[1] = 1.f;
    O[0] = O[1] = 0.f;
  } else if constexpr (F == kQ2_K || F == kQ3_K) {
    // 2-bit fields: byte j of (w >> 2i) & 0x03030303 is element 4j+i of the dword's 16
#pragma unroll
    for (int d = 0; d < 2; d++) {
      const uint32_t w = raw[F == kQ2_K ? 2 + d : 1 + d];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t v = opaque((w >> (2 * i)) & 0x03030303u);
#pragma unroll
        for (int j = 0; j < 4; j++) u[16 * d + 4 * j + i] = (float)byte_of(v, j);
      }
    }
    const int gi = g & 7;
    if constexpr (F == kQ2_K) {
      const float d = f16_to_f32(raw[0] & 0xFFFFu), dmin = f16_to_f32(raw[0] >> 16);
      const uint32_t c = raw[1] >> (16 * (gi & 1));
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const uint32_t ch = (c >> (8 * h)) & 0xFFu;
        S[h] = d * (float)(ch & 15u);
        O[h] = dmin * (float)(ch >> 4);
      }
    } else {
      // high bit of each 3-bit code: + 4 * bit e of the hmask dword
      const uint32_t hm = raw[0];
#pragma unroll
      for (int e = 0; e < 32; e++) u[e] += (float)(4u * ((hm >> e) & 1u));
      const float d = f16_to_f32(raw[4]);
      const uint32_t lo = ((raw[3] & 0xFFFFu) >> (8 * (gi & 1))) & 0xFFu;  // sc[gi]
      const uint32_t hi = ((raw[3] >> 16) >> (8 * ((gi >> 1) & 1))) & 0xFFu;  // sc[8 + gi/2]
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const uint32_t s6 = ((lo >> (4 * h)) & 15u) | (((hi >> (2 * (2 * (gi & 1) + h))) & 3u) << 4);
        const int sv = (int)(s6 << 26) >> 26;  // 6-bit two's complement
        S[h] = d * (float)sv;
        O[h] = 4.0f * S[h];  // codes stored as q + 4
      }
    }
  } else if constexpr (F == kQ5_K) {
    const float d = f16_to_f32(raw[0] & 0xFFFFu), dmin = f16_to_f32(raw[0] >> 16);
    uint32_t s, m;
    q4k_scale_min(raw[1], raw[2], raw[3], g & 7, s, m);
    S[0] = S[1] = d * (float)s;
    O[0] = O[1] = dmin * (float)m;
    const uint32_t qh = raw[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {  // nibble dword k: elements 8k..8k+7
      const uint32_t w = raw[5 + k];
      // bits 8k+p, 8k+p+2, 8k+p+4, 8k+p+6 of qh -> bit 4 of bytes 0..3 (the
      // multiply by 2^4 + 2^10 + 2^16 + 2^22 moves bit 2i to 8i + 4; no two
      // shifted copies meet inside the mask)
      const uint32_t te = (qh >> (8 * k)) & 0x55u, to = (qh >> (8 * k + 1)) & 0x55u;
      const uint32_t he = (te * 0x410410u) & 0x10101010u;
      const uint32_t ho = (to * 0x410410u) & 0x10101010u;
      const uint32_t ve = opaque((w & 0x0F0F0F0Fu) | he);
      const uint32_t vo = opaque(((w >> 4) & 0x0F0F0F0Fu) | ho);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        u[8 * k + 2 * i] = (float)byte_of(ve, i);
        u[8 * k + 2 * i + 1] = (float)byte_of(vo, i);
      }
    }
  } else if constexpr (F == kQ8_K) {
    const float d = __uint_as_float(raw[0]);
#pragma unroll
    for (int c = 0; c < 8; c++) {
      const uint32_t v = opaque(raw[1 + c] ^ 0x80808080u);  // code + 128
#pragma unroll
      for (int i = 0; i < 4; i++) u[4 * c + i] = (float)byte_of(v, i);
    }
    S[0] = S[1] = d;
    O[0] = O[1] = 128.0f * d;
  } else if constexpr (F == kIQ2_XXS || F == kIQ2_XS) {
    // four 8-element groups: a 64-bit grid row (tab, two dwords) and a sign mask
    const int ib = g & 7;
    float db;
    uint32_t gi[4], sg[4];
    if constexpr (F == kIQ2_XXS) {  // compute.rs:2137-2182
      const uint32_t a0 = raw[0], a1 = raw[1];
      db = f16_to_f32(raw[2]) * (0.5f + (float)(a1 >> 28)) * 0.25f;
#pragma unroll
      for (int l = 0; l < 4; l++) {
        gi[l] = (a0 >> (8 * l)) & 0xFFu;
        sg[l] = ksigns((a1 >> (7 * l)) & 127u);
      }
    } else {  // compute.rs:2192-2238
      const uint32_t sb = (raw[2] >> (8 * ((ib >> 1) & 1))) & 0xFFu;
      db = f16_to_f32(raw[3]) * (0.5f + (float)((sb >> (4 * (ib & 1))) & 15u)) * 0.25f;
#pragma unroll
      for (int l = 0; l < 4; l++) {
        const uint32_t qv = (raw[l >> 1] >> (16 * (l & 1))) & 0xFFFFu;
        gi[l] = qv & 511u;
        sg[l] = ksigns(qv >> 9);
      }
    }
#pragma unroll
    for (int l = 0; l < 4; l++) {
      const uint32_t lo = tab[2 * gi[l]], hi = tab[2 * gi[l] + 1];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        u[8 * l + j] = signed_mag(lo, j, sg[l], j);
        u[8 * l + j + 4] = signed_mag(hi, j, sg[l], j + 4);
      }
    }
    S[0] = S[1] = db;
    O[0] = O[1] = 0.f;
  } else if constexpr (F == kIQ3_XXS || F == kIQ3_S) {
    // four 8-element groups: two 32-bit grid entries and a sign mask each
    const int ib = g & 7;
    float db;
    uint32_t i1[4], i2[4], sg[4];
    if constexpr (F == kIQ3_XXS) {  // compute.rs:1983-2034
      const uint32_t aux = raw[2];
      db = f16_to_f32(raw[3]) * (0.5f + (float)(aux >> 28)) * 0.5f;
#pragma unroll
      for (int l = 0; l < 4; l++) {
        i1[l] = (raw[l >> 1] >> (16 * (l & 1))) & 0xFFu;
        i2[l] = (raw[l >> 1] >> (16 * (l & 1) + 8)) & 0xFFu;
        sg[l] = ksigns((aux >> (7 * l)) & 127u);
      }
    } else {  // compute.rs:2042-2128
      const uint32_t qh = (raw[2] >> (8 * (ib & 1))) & 0xFFu;
      const uint32_t sb = (raw[4] >> (8 * ((ib >> 1) & 1))) & 0xFFu;
      db = f16_to_f32(raw[5]) * (float)(1 + 2 * (int)((sb >> (4 * (ib & 1))) & 15u));
#pragma unroll
      for (int l = 0; l < 4; l++) {
        i1[l] = ((raw[l >> 1] >> (16 * (l & 1))) & 0xFFu) | ((qh << (8 - 2 * l)) & 256u);
        i2[l] = ((raw[l >> 1] >> (16 * (l & 1) + 8)) & 0xFFu) | ((qh << (7 - 2 * l)) & 256u);
        sg[l] = (raw[3] >> (8 * l)) & 0xFFu;
      }
    }
#pragma unroll
    for (int l = 0; l < 4; l++) {
      const uint32_t g1 = tab[i1[l]], g2 = tab[i2[l]];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        u[8 * l + j] = signed_mag(g1, j, sg[l], j);
        u[8 * l + j + 4] = signed_mag(g2, j, sg[l], j + 4);
      }
    }
    S[0] = S[1] = db;
    O[0] = O[1] = 0.f;
  } else {  // IQ4_NL / IQ4_XS: 16 index bytes, element 2j / 2j+1 = low / high nibble of byte j
    uint32_t qs[4];
    float scale;
    if constexpr (F == kIQ4_NL) {
      const uint32_t mis = raw[5];
      // bytes 2..17 of the block: mis == 2 -> raw[1..4]; mis == 0 -> shifted
      // pairs of raw[0..3], the last dword being raw[4] itself
      qs[0] = mis ? raw[1] : __builtin_amdgcn_alignbit(raw[1], raw[0], 16);
      qs[1] = mis ? raw[2] : __builtin_amdgcn_alignbit(raw[2], raw[1], 16);
      qs[2] = mis ? raw[3] : __builtin_amdgcn_alignbit(raw[3], raw[2], 16);
      qs[3] = raw[4];
      scale = f16_to_f32((raw[0] >> (8 * mis)) & 0xFFFFu);
    } else {
      const int sb = g & 7;
      const float d = f16_to_f32(raw[0] & 0xFFFFu);
      const uint32_t slw = (raw[1] >> (16 * ((sb >> 1) & 1))) & 0xFFFFu;
      const uint32_t sl = (slw >> (4 * (sb & 1))) & 15u;
      const uint32_t shv = (raw[0] >> (16 + 2 * sb)) & 3u;
      scale = d * ((float)(sl | (shv << 4)) - 32.0f);
#pragma unroll
      for (int k = 0; k < 4; k++) qs[k] = raw[2 + k];
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t ve = opaque(iq4_lookup(qs[k] & 0x0F0F0F0Fu));
      const uint32_t vo = opaque(iq4_lookup((qs[k] >> 4) & 0x0F0F0F0Fu));
#pragma unroll
      for (int i = 0; i < 4; i++) {
        u[8 * k + 2 * i] = (float)byte_of(ve, i);
        u[8 * k + 2 * i + 1] = (float)byte_of(vo, i);
      }
    }
    S[0] = S[1] = scale;
    O[0] = O[1] = 128.0f * scale;
  }
}

constexpr int kGS = 36;  // LDS stride of a 32-float group

template <int F, int B>
__host__ __device__ constexpr size_t ext_lds_bytes(int G) {
  return (size_t)B * G * (kGS + 2) * sizeof(float) + tab_bytes<F>;
}

// Types whose groups are requested two at a time per lane (see mv_ext).
// Measured at 14336 x 4096, batch 1, 8 workgroups per CU: IQ2_XXS 15.3 -> 14.7
// us, IQ2_XS 16.6 -> 15.8, IQ3_XXS 16.0 -> 14.8, IQ3_S 17.3 -> 16.6, IQ4_NL 12.7
// -> 12.3, F16 23.8 -> 22.4; IQ4_XS (12.4 -> 14.6) and BF16 (21.8 -> 22.4) keep
// one group at a time.
template <int F>
constexpr bool kPairGroups = F != kIQ4_XS && F != kBF16;

template <int F, int B, int R>
__global__ __launch_bounds__(256) void mv_ext(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                              float* __restrict__ y, int out_dim, int in_dim, int G,
                                              size_t row_bytes, int rows_per_wg) {
  extern __shared__ float smem[];
  float* xs = smem;                           // [B][G][kGS]
  float* xsum = smem + (size_t)B * G * kGS;   // [B][G][2]
  uint32_t* tab = reinterpret_cast<uint32_t*>(xsum + (size_t)B * G * 2);  // code book (IQ2 / IQ3)
  if constexpr (is_iq_lattice<F>) {
    const uint32_t* src = tab_src<F>();
    for (int i = threadIdx.x; i < tab_bytes<F> / 4; i += blockDim.x) tab[i] = src[i];
  }
  // stage x: one thread per 8 floats; a group's four chunks sit on adjacent lanes
  const int n8 = B * G * 4;  // multiple of 4, so lanes i and i^1 are both live or both not
  for (int i = threadIdx.x; i < n8; i += blockDim.x) {
    const int b = i / (G * 4), c = i - b * G * 4, g = c >> 2, part = c & 3;
    const float* xp = x + (size_t)b * in_dim + (size_t)g * 32 + part * 8;
    const float4 v0 = *reinterpret_cast<const float4*>(xp);
    const float4 v1 = *reinterpret_cast<const float4*>(xp + 4);
    float* dst = xs + ((size_t)b * G + g) * kGS + part * 8;
    *reinterpret_cast<float4*>(dst) = v0;
    *reinterpret_cast<float4*>(dst + 4) = v1;
    float s = ((v0.x + v0.y) + (v0.z + v0.w)) + ((v1.x + v1.y) + (v1.z + v1.w));
    s += dpp_mov<0xB1>(s);  // lane i ^ 1, as shfl_xor(s, 1)
    if ((part & 1) == 0) xsum[((size_t)b * G + g) * 2 + (part >> 1)] = s;
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int r_begin = blockIdx.x * rows_per_wg;
  const int r_end = min(out_dim, r_begin + rows_per_wg);
  constexpr int NW = XG<F>::NW;
  for (int r0 = r_begin + wave * R; r0 < r_end; r0 += nwaves * R) {
    float acc[R][B];
#pragma unroll
    for (int rr = 0; rr < R; rr++)
#pragma unroll
      for (int b = 0; b < B; b++) acc[rr][b] = 0.f;
    // (the two forms below are written out separately: sharing the group body
    // through a lambda cost the paired form 14-18 VGPRs and a wave per SIMD)
    if constexpr (kPairGroups<F>) {
      // groups g and g + 64 of every row are requested together before either
      // is decoded (the second clamped to the row's last group, and not summed,
      // past the end), so a wave keeps twice the loads in flight
      for (int g0 = lane; g0 < G; g0 += 128) {
        uint32_t raw[2][R][NW];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
          for (int rr = 0; rr < R; rr++) {
            const int row = min(r0 + rr, r_end - 1);
            load_group<F>(w + (size_t)row * row_bytes, min(g0 + 64 * h, G - 1), raw[h][rr]);
          }
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const int g = min(g0 + 64 * h, G - 1);
          const bool live = g0 + 64 * h < G;
#pragma unroll
          for (int rr = 0; rr < R; rr++) {
            float u[32], S[2], O[2];
            decode_group<F>(raw[h][rr], g, u, S, O, tab);
#pragma unroll
            for (int b = 0; b < B; b++) {
              const float* xg = xs + ((size_t)b * G + g) * kGS;
              float pa = 0.f, pb = 0.f;
#pragma unroll
              for (int e = 0; e < 16; e++) pa = fmaf(u[e], xg[e], pa);
#pragma unroll
              for (int e = 16; e < 32; e++) pb = fmaf(u[e], xg[e], pb);
              const float* sg = xsum + ((size_t)b * G + g) * 2;
              float a = fmaf(-O[0], sg[0], acc[rr][b]);
              a = fmaf(-O[1], sg[1], a);
              a = fmaf(S[0], pa, a);
              acc[rr][b] = live ? fmaf(S[1], pb, a) : acc[rr][b];
            }
          }
        }
      }
    } else {
      for (int g = lane; g < G; g += 64) {
        uint32_t raw[R][NW];
#pragma unroll
        for (int rr = 0; rr < R; rr++) {
          const int row = min(r0 + rr, r_end - 1);
          load_group<F>(w + (size_t)row * row_bytes, g, raw[rr]);
        }
#pragma unroll
        for (int rr = 0; rr < R; rr++) {
          float u[32], S[2], O[2];
          decode_group<F>(raw[rr], g, u, S, O, tab);
#pragma unroll
          for (int b = 0; b < B; b++) {
            const float* xg = xs + ((size_t)b * G + g) * kGS;
            float pa = 0.f, pb = 0.f;
#pragma unroll
            for (int e = 0; e < 16; e++) pa = fmaf(u[e], xg[e], pa);
#pragma unroll
            for (int e = 16; e < 32; e++) pb = fmaf(u[e], xg[e], pb);
            const float* sg = xsum + ((size_t)b * G + g) * 2;
            float a = fmaf(-O[0], sg[0], acc[rr][b]);
            a = fmaf(-O[1], sg[1], a);
            a = fmaf(S[0], pa, a);
            acc[rr][b] = fmaf(S[1], pb, a);
          }
        }
      }
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
// Element k of a row, formed as the reference forms it (any alignment).
template <int F>
__device__ __forceinline__ float ext_value(const uint8_t* __restrict__ row, int k) {
  if constexpr (F == kF16) {
    return f16_to_f32(ld_u16(row + 2 * (size_t)k));
  } else if constexpr (F == kBF16) {
    return __uint_as_float(ld_u16(row + 2 * (size_t)k) << 16);
  } else if constexpr (F == kQ2_K) {
    const uint8_t* p = row + (size_t)(k >> 8) * 84;
    const int idx = k & 255, sb = idx >> 4;
    const uint32_t c = p[4 + sb];
    const float scale = f16_to_f32(ld_u16(p)) * (float)(c & 15u);
    const float mn = f16_to_f32(ld_u16(p + 2)) * (float)(c >> 4);
    return scale * (float)((p[20 + idx / 4] >> (2 * (idx % 4))) & 3u) - mn;
  } else if constexpr (F == kQ3_K) {
    const uint8_t* p = row + (size_t)(k >> 8) * 110;
    const int idx = k & 255, sb = idx >> 4;
    const uint32_t low4 = (p[96 + sb / 2] >> ((sb & 1) * 4)) & 15u;
    const uint32_t hi2 = (p[104 + sb / 4] >> ((sb % 4) * 2)) & 3u;
    int sv = (int)(low4 | (hi2 << 4));
    if (sv >= 32) sv -= 64;
    const uint32_t low2 = (p[32 + idx / 4] >> ((idx % 4) * 2)) & 3u;
    const uint32_t hb = (p[idx / 8] >> (idx % 8)) & 1u;
    return (f16_to_f32(ld_u16(p + 108)) * (float)sv) * (float)((int)(low2 | (hb << 2)) - 4);
  } else if constexpr (F == kQ5_K) {
    const uint8_t* p = row + (size_t)(k >> 8) * 176;
    const int idx = k & 255, sb = idx >> 5;
    uint32_t s, m;
    const uint32_t sc1 = p[4] | (p[5] << 8) | (p[6] << 16) | ((uint32_t)p[7] << 24);
    const uint32_t sc2 = p[8] | (p[9] << 8) | (p[10] << 16) | ((uint32_t)p[11] << 24);
    const uint32_t sc3 = p[12] | (p[13] << 8) | (p[14] << 16) | ((uint32_t)p[15] << 24);
    q4k_scale_min(sc1, sc2, sc3, sb, s, m);
    const uint32_t bv = p[48 + sb * 16 + (idx & 31) / 2];
    const uint32_t lo = (idx & 1) ? (bv >> 4) : (bv & 15u);
    const uint32_t hb = (p[16 + idx / 8] >> (idx % 8)) & 1u;
    return (f16_to_f32(ld_u16(p)) * (float)s) * (float)(lo | (hb << 4)) - f16_to_f32(ld_u16(p + 2)) * (float)m;
  } else if constexpr (F == kQ8_K) {
    const uint8_t* p = row + (size_t)(k >> 8) * 292;
    const uint32_t db = p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24);
    return __uint_as_float(db) * (float)(int8_t)p[4 + (k & 255)];
  } else if constexpr (F == kIQ4_NL) {
    const uint8_t* p = row + (size_t)(k >> 5) * 18;
    const int j = k & 31;
    const uint32_t bv = p[2 + j / 2];
    return f16_to_f32(ld_u16(p)) * (float)kIq4nl[(j & 1) ? (bv >> 4) : (bv & 15u)];
  } else if constexpr (is_iq_lattice<F>) {
    const uint8_t* p = row + (size_t)(k >> 8) * XG<F>::bb;
    const int idx = k & 255, ib = idx >> 5, l = (idx >> 3) & 3, j = idx & 7;
    const float d = f16_to_f32(ld_u16(p));
    auto u32at = [](const uint8_t* q) {
      return (uint32_t)q[0] | ((uint32_t)q[1] << 8) | ((uint32_t)q[2] << 16) | ((uint32_t)q[3] << 24);
    };
    if constexpr (F == kIQ2_XXS) {
      const uint32_t a1 = u32at(p + 2 + 8 * ib + 4);
      const float db = d * (0.5f + (float)(a1 >> 28)) * 0.25f;
      const uint64_t gr = k_iq2xxs_grid[p[2 + 8 * ib + l]];
      const uint32_t sg = ksigns((a1 >> (7 * l)) & 127u);
      return db * (float)((gr >> (8 * j)) & 0xFFu) * (((sg >> j) & 1u) ? -1.0f : 1.0f);
    } else if constexpr (F == kIQ2_XS) {
      const uint32_t sb = p[66 + ib / 2];
      const float db = d * (0.5f + (float)((ib % 2 == 0) ? (sb & 15u) : (sb >> 4))) * 0.25f;
      const uint32_t qv = ld_u16(p + 2 + (ib * 4 + l) * 2);
      const uint64_t gr = k_iq2xs_grid[qv & 511u];
      const uint32_t sg = ksigns(qv >> 9);
      return db * (float)((gr >> (8 * j)) & 0xFFu) * (((sg >> j) & 1u) ? -1.0f : 1.0f);
    } else if constexpr (F == kIQ3_XXS) {
      const uint32_t aux = u32at(p + 66 + 4 * ib);
      const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
      const uint32_t gw = k_iq3xxs_grid[p[2 + 8 * ib + 2 * l + (j >> 2)]];
      const uint32_t sg = ksigns((aux >> (7 * l)) & 127u);
      return db * (float)((gw >> (8 * (j & 3))) & 0xFFu) * (((sg >> j) & 1u) ? -1.0f : 1.0f);
    } else {  // kIQ3_S
      const uint32_t sb = p[106 + ib / 2];
      const float db = d * (float)(1 + 2 * (int)((ib % 2 == 0) ? (sb & 15u) : (sb >> 4)));
      const uint32_t qh = p[66 + ib];
      const int h = j >> 2;  // 0: first grid word of the pair, 1: second
      const uint32_t gi = p[2 + 8 * ib + 2 * l + h] | ((qh << (8 - 2 * l - h)) & 256u);
      const uint32_t gw = k_iq3s_grid[gi];
      const uint32_t sg = p[74 + 4 * ib + l];
      return db * (float)((gw >> (8 * (j & 3))) & 0xFFu) * (((sg >> j) & 1u) ? -1.0f : 1.0f);
    }
  } else {  // kIQ4_XS
    const uint8_t* p = row + (size_t)(k >> 8) * 148;
    const int idx = k & 255, sb = idx >> 5, j = idx & 31;
    const uint32_t slw = ld_u16(p + 4 + (sb / 2) * 2);
    const uint32_t sl = (sb % 2 == 0) ? (slw & 15u) : ((slw >> 4) & 15u);
    const uint32_t shv = (ld_u16(p + 2) >> (2 * sb)) & 3u;
    const float scale = (float)(sl | (shv << 4)) - 32.0f;
    const uint32_t bv = p[20 + sb * 16 + j / 2];
    return f16_to_f32(ld_u16(p)) * scale * (float)kIq4nl[(j & 1) ? (bv >> 4) : (bv & 15u)];
  }
}

template <int F, int B>
__global__ __launch_bounds__(256) void mv_ext_generic(const uint8_t* __restrict__ w, const float* __restrict__ x,
                                                      float* __restrict__ y, int out_dim, int in_dim, int keff,
                                                      size_t row_bytes) {
  const int lane = threadIdx.x & 63;
  for (int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); row < out_dim;
       row += gridDim.x * (blockDim.x >> 6)) {
    const uint8_t* rp = w + (size_t)row * row_bytes;
    float acc[B];
#pragma unroll
    for (int b = 0; b < B; b++) acc[b] = 0.f;
    for (int k = lane; k < keff; k += 64) {
      const float v = ext_value<F>(rp, k);
#pragma unroll
      for (int b = 0; b < B; b++) acc[b] = fmaf(v, x[(size_t)b * in_dim + k], acc[b]);
    }
#pragma unroll
    for (int b = 0; b < B; b++) {
      const float s = wave_sum(acc[b]);
      if (lane == 0) y[(size_t)b * out_dim + row] = s;
    }
  }
}

// ------------------------------------------------------------------ host
int ext_lds_limit() {
  int dev = 0, v = 65536;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
    v = 65536;
  return v;
}

template <int F, int B, int R>
hipError_t run_ext(const uint8_t* w, const float* x, float* y, int out_dim, int in_dim, int G,
                   size_t row_bytes, size_t lds, hipStream_t s) {
  auto kern = mv_ext<F, B, R>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  // about eight workgroups per CU, rows in multiples of 4R.  Each wave walks
  // its groups one load-and-decode at a time, so the waves in flight carry the
  // latency: with two workgroups per CU (and four rows per wave at batch 1)
  // 14336 x 4096 took IQ4_NL 15.4 -> 12.7 us, IQ4_XS 15.3 -> 12.3, BF16 25.2 ->
  // 21.7, IQ2_XXS 17.4 -> 15.2, IQ3_S 18.9 -> 17.2, F16 24.7 -> 23.8.
  const int target = 8 * device_cu_count();
  const int q = 4 * R;
  int n = std::max(1, std::min((out_dim + q - 1) / q, target));
  int rows = (out_dim + n - 1) / n;
  rows = (rows + q - 1) / q * q;
  n = (out_dim + rows - 1) / rows;
  hipLaunchKernelGGL(kern, dim3(n), dim3(256), lds, s, w, x, y, out_dim, in_dim, G, row_bytes, rows);
  return hipGetLastError();
}

template <int F>
hipError_t ext_fast(const uint8_t* w, const float* x, float* y, int out_dim, int in_dim, int keff,
                    size_t row_bytes, int batch, hipStream_t s, bool* used) {
  *used = false;
  const int G = keff / 32;
  if (((uintptr_t)w & 3) || ((uintptr_t)x & 15) || (in_dim & 3) || (keff & 31) || G == 0) return hipSuccess;
  if ((F == kF16 || F == kBF16) && (row_bytes & 3)) return hipSuccess;
  const size_t limit = (size_t)ext_lds_limit();
  if (ext_lds_bytes<F, 1>(G) > limit) return hipSuccess;
  int b0 = 0;
  while (b0 < batch) {
    const int left = batch - b0;
    int take = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
    while (take > 1 && (size_t)take * ext_lds_bytes<F, 1>(G) > limit) take >>= 1;  // (table counted per take)
    const float* xb = x + (size_t)b0 * in_dim;
    float* yb = y + (size_t)b0 * out_dim;
    hipError_t e;
    switch (take) {
      case 8: e = run_ext<F, 8, 1>(w, xb, yb, out_dim, in_dim, G, row_bytes, ext_lds_bytes<F, 8>(G), s); break;
      case 4: e = run_ext<F, 4, 1>(w, xb, yb, out_dim, in_dim, G, row_bytes, ext_lds_bytes<F, 4>(G), s); break;
      case 2: e = run_ext<F, 2, 2>(w, xb, yb, out_dim, in_dim, G, row_bytes, ext_lds_bytes<F, 2>(G), s); break;
      default: e = run_ext<F, 1, 2>(w, xb, yb, out_dim, in_dim, G, row_bytes, ext_lds_bytes<F, 1>(G), s); break;
    }
    if (e != hipSuccess) return e;
    b0 += take;
  }
  *used = true;
  return hipSuccess;
}

template <int F>
hipError_t ext_generic(const uint8_t* w, const float* x, float* y, int out_dim, int in_dim, int keff,
                       size_t row_bytes, int batch, hipStream_t s) {
  const int grid = std::min((out_dim + 3) / 4, 65535);
  int b0 = 0;
  while (b0 < batch) {
    const int left = batch - b0;
    const float* xb = x + (size_t)b0 * in_dim;
    float* yb = y + (size_t)b0 * out_dim;
    int take;
    if (left >= 4) {
      take = 4;
      hipLaunchKernelGGL((mv_ext_generic<F, 4>), dim3(grid), dim3(256), 0, s, w, xb, yb, out_dim, in_dim, keff, row_bytes);
    } else if (left >= 2) {
      take = 2;
      hipLaunchKernelGGL((mv_ext_generic<F, 2>), dim3(grid), dim3(256), 0, s, w, xb, yb, out_dim, in_dim, keff, row_bytes);
    } else {
      take = 1;
      hipLaunchKernelGGL((mv_ext_generic<F, 1>), dim3(grid), dim3(256), 0, s, w, xb, yb, out_dim, in_dim, keff, row_bytes);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    b0 += take;
  }
  return hipSuccess;
}

template <int F>
hipError_t ext_dispatch(const uint8_t* w, const float* x, float* y, size_t out_dim, size_t in_dim,
                        size_t batch, hipStream_t s, bool generic) {
  constexpr int bs = XG<F>::bs;
  const size_t bpr = in_dim / bs, keff = bpr * bs, row_bytes = bpr * XG<F>::bb;
  if (keff == 0) return launch_fill_zero(y, out_dim * batch, s);  // no whole block: the sum is 0
  if (!generic) {
    bool used = false;
    hipError_t e = ext_fast<F>(w, x, y, (int)out_dim, (int)in_dim, (int)keff, row_bytes, (int)batch, s, &used);
    if (e != hipSuccess || used) return e;
  }
  return ext_generic<F>(w, x, y, (int)out_dim, (int)in_dim, (int)keff, row_bytes, (int)batch, s);
}

}  // namespace

bool matvec_ext_type(int dtype) {
  switch (dtype) {
    case kQ2_K: case kQ3_K: case kQ5_K: case kQ8_K: case kIQ4_NL: case kIQ4_XS: case kF16: case kBF16:
    case kIQ2_XXS: case kIQ2_XS: case kIQ3_XXS: case kIQ3_S:
      return true;
    default:
      return false;
  }
}

hipError_t launch_matvec_ext(int dtype, const uint8_t* w, const float* x, float* y, size_t out_dim,
                             size_t in_dim, size_t batch, hipStream_t s, bool generic) {
  if (out_dim == 0 || batch == 0) return hipSuccess;
  switch (dtype) {
    case kQ2_K: return ext_dispatch<kQ2_K>(w, x, y, out_dim, in_dim, batch, s, generic);
    case kQ3_K: return ext_dispatch<kQ3_K>(w, x, y, out_dim, in_dim, batch, s, generic);
    case kQ5_K: return ext_dispatch<kQ5_K>(w, x, y, out_dim, in_dim, batch, s, generic);
    case kQ8_K: return ext_dispatch<kQ8_K>(w, x, y, out_dim, in_dim, batch, s, generic);
    case kIQ4_NL: return ext_dispatch<kIQ4_NL>(w, x, y, out_dim, in_dim, batch, s, generic);
    case kIQ4_XS: return ext_dispatch<kIQ4_XS>(w, x, y, out_dim, in_dim, batch, s, generic);
    case kF16: return ext_dispatch<kF16>(w, x, y, out_dim, in_dim, batch, s, generic);
    case kBF16: return ext_dispatch<kBF16>(w, x, y, out_dim, in_dim, batch, s, generic);
    case kIQ2_XXS: return ext_dispatch<kIQ2_XXS>(w, x, y, out_dim, in_dim, batch, s, generic);
    case kIQ2_XS: return ext_dispatch<kIQ2_XS>(w, x, y, out_dim, in_dim, batch, s, generic);
    case kIQ3_XXS: return ext_dispatch<kIQ3_XXS>(w, x, y, out_dim, in_dim, batch, s, generic);
    case kIQ3_S: return ext_dispatch<kIQ3_S>(w, x, y, out_dim, in_dim, batch, s, generic);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ssdq
