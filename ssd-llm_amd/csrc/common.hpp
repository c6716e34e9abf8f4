// Shared device helpers for the ssdq gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ssdq {

constexpr int kWave = 64;  // CDNA wavefront width

// GgmlType ids (src/model/gguf.rs:17-48) and block geometry (gguf.rs:87-135).
enum : int { kQ4_0 = 2, kQ8_0 = 8, kQ2_K = 10, kQ3_K = 11, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kQ8_K = 15 };

template <int F> struct Geom;
template <> struct Geom<kQ4_0> { static constexpr int bs = 32, bb = 18; };
template <> struct Geom<kQ8_0> { static constexpr int bs = 32, bb = 34; };
template <> struct Geom<kQ2_K> { static constexpr int bs = 256, bb = 84; };
template <> struct Geom<kQ3_K> { static constexpr int bs = 256, bb = 110; };
template <> struct Geom<kQ4_K> { static constexpr int bs = 256, bb = 144; };
template <> struct Geom<kQ5_K> { static constexpr int bs = 256, bb = 176; };
template <> struct Geom<kQ6_K> { static constexpr int bs = 256, bb = 210; };
template <> struct Geom<kQ8_K> { static constexpr int bs = 256, bb = 292; };

// IEEE binary16 -> binary32 (exact widening, v_cvt_f32_f16).
__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (float)h;
}

__device__ __forceinline__ uint32_t ld_u8(const uint8_t* p) { return *p; }
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
  // p may be only 1-byte aligned in the generic paths
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8);
}

// s_waitcnt vmcnt(N) as inline assembly with a memory clobber.  The builtin
// s_waitcnt is a no-memory intrinsic at IR level, so LDS reads placed after it
// may be moved above it; after loads the compiler does not track (LDS DMA
// issued from inline assembly) the wait must also order those reads.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// s_waitcnt lgkmcnt(0) with a memory clobber (every LDS read issued so far has
// returned its data).
__device__ __forceinline__ void wait_lgkmcnt0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Byte k (0..3) of a dword.
__device__ __forceinline__ uint32_t byte_of(uint32_t v, int k) { return (v >> (8 * k)) & 0xFFu; }

// Hides a value from the optimizer so byte extractions of it map onto
// v_cvt_f32_ubyte{0..3} instead of being folded into bit-field extracts.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm("" : "+v"(v));
  return v;
}

// DPP lane moves within rows of 16 lanes (quad_perm / row_ror controls).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Sum across the 64 lanes of a wavefront (result valid in every lane): four
// DPP steps inside each 16-lane row, then two cross-row exchanges.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x124>(v);  // row_ror:4
  v += dpp_mov<0x128>(v);  // row_ror:8
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// DPP move whose disabled rows (ROW_MASK) read as 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_upd(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               ROW_MASK, 0xF, false));
}

// Sum across the 64 lanes of a wavefront, valid in lane 63 only: DPP steps
// inside each 16-lane row, then row_bcast:15 / row_bcast:31 (no LDS traffic).
__device__ __forceinline__ float wave_sum_l63(float v) {
  v += dpp_mov<0xB1>(v);        // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);        // quad_perm [2,3,0,1]
  v += dpp_mov<0x124>(v);       // row_ror:4
  v += dpp_mov<0x128>(v);       // row_ror:8: every lane holds its row's sum
  v += dpp_upd<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_upd<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// DPP moves of a double (both halves moved with the same control).
template <int CTRL>
__device__ __forceinline__ double dpp_mov_d(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)b, CTRL, 0xF, 0xF, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, true);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_upd_d(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROW_MASK, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROW_MASK, 0xF, false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// wave_sum_l63 in double precision (the matvec kernels' row sums: terms of
// very different sizes, as massive activation channels make them, cancel
// without fp32 rounding).
__device__ __forceinline__ double wave_sum_l63_d(double v) {
  v += dpp_mov_d<0xB1>(v);
  v += dpp_mov_d<0x4E>(v);
  v += dpp_mov_d<0x124>(v);
  v += dpp_mov_d<0x128>(v);
  v += dpp_upd_d<0x142, 0xA>(v);
  v += dpp_upd_d<0x143, 0xC>(v);
  return v;
}

// Sum across the 64 lanes of a wavefront (result valid in every lane).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Maximum over the wavefront with DPP only, returned in every lane.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_mov<0x124>(v));  // row_ror:4
  v = fmaxf(v, dpp_mov<0x128>(v));  // row_ror:8: every lane holds its row's maximum
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                   __builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                   __builtin_bit_cast(int, v), __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false)));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Sum / maximum over each 32-lane half of a wavefront, in every lane, with
// the pairings of the steps x op shfl_xor(x, o), o = 1, 2, 4, 8, 16 (so a sum
// is bit for bit the one those steps give): DPP quad_perm for o = 1, 2; after
// them the four lanes of a quad agree, so row_half_mirror (lane i of 8 to
// 7 - i) pairs the same quads as o = 4, and row_mirror the same halves of a
// row as o = 8; v_permlane16_swap of a register with itself for o = 16.
__device__ __forceinline__ float half_wave_sum(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float half_wave_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  v = fmaxf(v, dpp_mov<0x140>(v));
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

// Bytes d of a, b, c, e to bytes 0-3 of out[d], d = 0..3: a 4 x 4 byte
// transpose in eight byte permutes (the digit planes of four 32-bit integers).
__device__ __forceinline__ void planes4(uint32_t a, uint32_t b, uint32_t c, uint32_t e, uint32_t out[4]) {
  const uint32_t ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
  const uint32_t ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
  const uint32_t ce_lo = __builtin_amdgcn_perm(e, c, 0x05010400u);
  const uint32_t ce_hi = __builtin_amdgcn_perm(e, c, 0x07030602u);
  out[0] = __builtin_amdgcn_perm(ce_lo, ab_lo, 0x05040100u);  // a0 b0 c0 e0
  out[1] = __builtin_amdgcn_perm(ce_lo, ab_lo, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(ce_hi, ab_hi, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(ce_hi, ab_hi, 0x07060302u);
}

// INT8 code of one KV element (quantize_vectors_int8, src/ssd/block_swap.rs:36-60
// = QuantizedVec::quantize, src/inference/quantized_kv_cache.rs:23-41):
// clamp(round_half_away(v * inv), -127, 127), NaN -> 0 (Rust `as i8`), as a
// byte.  inv = 127 / absmax of the row (0 for an all-zero row, which gives
// codes 0); the row's scale is absmax / 127.
__device__ __forceinline__ uint32_t kv_code_of(float v, float inv) {
#pragma clang fp contract(off)
  const float t = roundf(v * inv);  // round half away from zero
  int c;
  if (t != t) {
    c = 0;
  } else {
    c = (int)fminf(fmaxf(t, -127.0f), 127.0f);
  }
  return (uint32_t)(c & 0xFF);
}

__device__ __forceinline__ uint32_t kv_pack4(float a, float b, float c, float d, float inv) {
  return kv_code_of(a, inv) | (kv_code_of(b, inv) << 8) | (kv_code_of(c, inv) << 16) | (kv_code_of(d, inv) << 24);
}

// 6-bit scale s and min m of Q4_K sub-block sb from the 12 packed bytes, in the
// reference's bit order (src/metal/compute.rs:724-731): for sb >= 4 the two bits
// taken from sc[sb-4] / sc[sb] are the LOW bits.  sc1/sc2/sc3 are bytes 0-3,
// 4-7 and 8-11 of the packed area as little-endian dwords.
__device__ __forceinline__ void q4k_scale_min(uint32_t sc1, uint32_t sc2, uint32_t sc3, int sb,
                                              uint32_t& s, uint32_t& m) {
  if (sb < 4) {
    s = byte_of(sc1, sb) & 63u;
    m = byte_of(sc2, sb) & 63u;
  } else {
    const int i = sb - 4;
    const uint32_t hi = byte_of(sc3, i);
    s = (byte_of(sc1, i) >> 6) | ((hi & 0x0Fu) << 2);
    m = (byte_of(sc2, i) >> 6) | ((hi >> 4) << 2);
  }
}

}  // namespace ssdq
