// Single-query GQA decode attention with online softmax, split over the
// context ("flash-decoding") so one (sequence, KV head) pair fills many CUs.
//
// Reference semantics (src/inference/flash_attention.rs:70-139, the
// MetalCompute::flash_attention_f32 contract, src/metal/compute.rs:217-258):
//   kv_h = h / max(n_head / n_head_kv, 1), scale = 1/sqrt(head_dim),
//   online softmax over the positions, out = acc / sum, zeros when sum == 0.
// Two KV sources share the kernel:
//   * the paged INT8 cache: token t of a sequence lives in physical block
//     block_table[t / block_size], slot t % block_size
//     (src/inference/paged_attention.rs:113-123); a block is
//     [block_size, kv_dim] codes (paged_attention.rs:34-35) plus one f32 scale
//     per token row (quantized_kv_cache.rs:23-53); K = code * scale.
//   * flattened f32 KV [seq, n_head_kv, head_dim] with a position window
//     (kernels.metal:1350-1355 layout, window [start, min(end, seq_len))).
//
// Pass 1 (one workgroup per (split, kv head, sequence)) computes, for the G
// query heads sharing the KV head, the split's running max m, sum l and
// unnormalised acc[head_dim]; every K/V byte of the split is read once for all
// G heads.  Pass 2 merges the splits with the usual log-sum-exp rescaling.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include <climits>

#include "common.hpp"
#include "launch.hpp"

namespace ssdq {
namespace {

constexpr int kTile = 64;     // tokens per tile
constexpr int kThreads = 256;
constexpr int kMaxG = 8;      // query heads per KV head handled in one workgroup pass

struct PagedSrc {
  const int8_t* kc;
  const float* ks;
  const int8_t* vc;
  const float* vs;
  const int32_t* table;  // this sequence's block table
  int block_size;
  int kv_dim;
  __device__ __forceinline__ size_t row(int t) const {
    return (size_t)table[t / block_size] * block_size + (t % block_size);
  }
};

struct FlatSrc {
  const float* k;
  const float* v;
  int kv_dim;
};

// Partial record layout per (seq, head, split): [m, l, acc[head_dim]]
template <int HD, class Src>
__global__ __launch_bounds__(kThreads) void attn_split_kernel(
    const float* __restrict__ q, Src src, const int32_t* __restrict__ block_tables,
    const int32_t* __restrict__ ctx_lens, const int32_t* __restrict__ win_lo, const int32_t* __restrict__ win_hi,
    int max_blocks_per_seq, int n_head, int n_head_kv, int pos_begin_flat, int pos_end_flat, int split_len,
    int n_splits, float* __restrict__ partial) {
  constexpr int QK_PARTS = kThreads / kTile;     // threads per token in the QK phase
  constexpr int QK_DIMS = HD / QK_PARTS;
  constexpr int PV_THREADS_PER_TOK = HD / 2;     // 2 dims per thread
  constexpr int PV_GROUPS = kThreads / PV_THREADS_PER_TOK;
  constexpr int PV_TOKS = kTile / PV_GROUPS;
  static_assert(QK_DIMS % 4 == 0, "head_dim must split into dword parts");

  const int split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int group = max(n_head / n_head_kv, 1);
  const int G = min(group, kMaxG);
  const int h0 = kvh * group;  // first query head of this KV head (handled in chunks of kMaxG)

  int p_begin, p_end;
  if constexpr (std::is_same<Src, PagedSrc>::value) {
    src.table = block_tables + (size_t)seq * max_blocks_per_seq;
    // the window [lo, hi) of this sequence; never address past the block
    // table, whatever ctx_lens holds
    p_begin = win_lo ? max(win_lo[seq], 0) : 0;
    p_end = min(ctx_lens[seq], max_blocks_per_seq * src.block_size);
    if (win_hi) p_end = min(p_end, win_hi[seq]);
  } else {
    p_begin = pos_begin_flat;
    p_end = pos_end_flat;
  }
  const int s_begin = p_begin + split * split_len;
  const int s_end = min(p_end, s_begin + split_len);

  __shared__ float q_s[kMaxG][HD];
  __shared__ float sc_s[kMaxG][kTile];
  __shared__ float p_s[kMaxG][kTile];
  __shared__ float corr_s[kMaxG];
  __shared__ float red_s[PV_GROUPS][kMaxG][HD];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float inv_sqrt = 1.0f / sqrtf((float)HD);

  for (int hc = 0; hc < group; hc += kMaxG) {  // query-head chunks (group > kMaxG only)
    const int gn = min(G, group - hc);
    for (int i = tid; i < kMaxG * HD; i += kThreads) {
      const int g = i / HD, d = i % HD;
      q_s[g][d] = g < gn ? q[((size_t)seq * n_head + h0 + hc + g) * HD + d] : 0.f;
    }
    float run_m[2] = {-INFINITY, -INFINITY}, run_l[2] = {0.f, 0.f};  // heads wave, wave+4
    float acc[kMaxG][2];
#pragma unroll
    for (int g = 0; g < kMaxG; g++) acc[g][0] = acc[g][1] = 0.f;
    __syncthreads();

    for (int t0 = s_begin; t0 < s_end; t0 += kTile) {
      // ---- QK: 4 threads per token
      {
        const int j = tid / QK_PARTS, part = tid % QK_PARTS;
        const int t = t0 + j;
        float dot[kMaxG];
#pragma unroll
        for (int g = 0; g < kMaxG; g++) dot[g] = 0.f;
        float kscale = 1.0f;
        if (t < s_end) {
          float kf[QK_DIMS];
          if constexpr (std::is_same<Src, PagedSrc>::value) {
            const size_t r = src.row(t);
            const int8_t* kp = src.kc + r * src.kv_dim + (size_t)kvh * HD + part * QK_DIMS;
#pragma unroll
            for (int d = 0; d < QK_DIMS; d += 4) {
              const uint32_t w4 = *reinterpret_cast<const uint32_t*>(kp + d);
#pragma unroll
              for (int i = 0; i < 4; i++) kf[d + i] = (float)(int8_t)(w4 >> (8 * i));
            }
            kscale = src.ks[r];
          } else {
            const float* kp = src.k + (size_t)t * src.kv_dim + (size_t)kvh * HD + part * QK_DIMS;
#pragma unroll
            for (int d = 0; d < QK_DIMS; d += 4) {
              const float4 f = *reinterpret_cast<const float4*>(kp + d);
              kf[d] = f.x; kf[d + 1] = f.y; kf[d + 2] = f.z; kf[d + 3] = f.w;
            }
          }
#pragma unroll
          for (int g = 0; g < kMaxG; g++) {
            if (g < gn) {
              float a = 0.f;
#pragma unroll
              for (int d = 0; d < QK_DIMS; d++) a = fmaf(q_s[g][part * QK_DIMS + d], kf[d], a);
              dot[g] = a;
            }
          }
        }
#pragma unroll
        for (int g = 0; g < kMaxG; g++) {
          float v = dot[g];
#pragma unroll
          for (int off = 1; off < QK_PARTS; off <<= 1) v += __shfl_xor(v, off, kWave);
          dot[g] = v;
        }
        if (part == 0) {
#pragma unroll
          for (int g = 0; g < kMaxG; g++)
            sc_s[g][j] = (t < s_end && g < gn) ? dot[g] * kscale * inv_sqrt : -INFINITY;
        }
      }
      __syncthreads();
      // ---- online softmax per head: wave w owns heads w and w+4, lane = token
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const int g = wave + 4 * k;
        if (g < gn) {
          const float s = sc_s[g][lane];
          const float tmax = wave_max(s);
          const float m_new = fmaxf(run_m[k], tmax);
          float corr, p;
          if (m_new == -INFINITY) {
            corr = 1.f;
            p = 0.f;
          } else {
            corr = __expf(run_m[k] - m_new);
            p = __expf(s - m_new);
          }
          run_l[k] = run_l[k] * corr + wave_sum(p);
          run_m[k] = m_new;
          float vscale = 1.0f;
          const int t = t0 + lane;
          if constexpr (std::is_same<Src, PagedSrc>::value)
            if (t < s_end) vscale = src.vs[src.row(t)];
          p_s[g][lane] = p * vscale;
          if (lane == 0) corr_s[g] = corr;
        }
      }
      __syncthreads();
      // ---- PV: thread owns 2 dims for PV_TOKS tokens of the tile
      {
        const int dpair = tid % PV_THREADS_PER_TOK, tg = tid / PV_THREADS_PER_TOK;
#pragma unroll
        for (int g = 0; g < kMaxG; g++) {
          if (g < gn) {
            const float c = corr_s[g];
            acc[g][0] *= c;
            acc[g][1] *= c;
          }
        }
        for (int jj = 0; jj < PV_TOKS; jj++) {
          const int j = tg * PV_TOKS + jj;
          const int t = t0 + j;
          if (t >= s_end) break;
          float v0, v1;
          if constexpr (std::is_same<Src, PagedSrc>::value) {
            const size_t r = src.row(t);
            const uint32_t two =
                *reinterpret_cast<const uint16_t*>(src.vc + r * src.kv_dim + (size_t)kvh * HD + 2 * dpair);
            v0 = (float)(int8_t)(two & 0xFF);
            v1 = (float)(int8_t)(two >> 8);
          } else {
            const float2 f = *reinterpret_cast<const float2*>(src.v + (size_t)t * src.kv_dim +
                                                              (size_t)kvh * HD + 2 * dpair);
            v0 = f.x;
            v1 = f.y;
          }
#pragma unroll
          for (int g = 0; g < kMaxG; g++) {
            if (g < gn) {
              const float p = p_s[g][j];
              acc[g][0] = fmaf(p, v0, acc[g][0]);
              acc[g][1] = fmaf(p, v1, acc[g][1]);
            }
          }
        }
      }
      __syncthreads();
    }

    // ---- reduce the PV token groups and write the split's partial records
    {
      const int dpair = tid % PV_THREADS_PER_TOK, tg = tid / PV_THREADS_PER_TOK;
#pragma unroll
      for (int g = 0; g < kMaxG; g++) {
        red_s[tg][g][2 * dpair] = acc[g][0];
        red_s[tg][g][2 * dpair + 1] = acc[g][1];
      }
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int g = wave + 4 * k;
      if (g < gn && lane == 0) {
        float* rec = partial + (((size_t)seq * n_head + h0 + hc + g) * n_splits + split) * (HD + 2);
        rec[0] = run_m[k];
        rec[1] = run_l[k];
      }
    }
    __syncthreads();
    for (int i = tid; i < gn * HD; i += kThreads) {
      const int g = i / HD, d = i % HD;
      float s = 0.f;
#pragma unroll
      for (int tg = 0; tg < PV_GROUPS; tg++) s += red_s[tg][g][d];
      partial[(((size_t)seq * n_head + h0 + hc + g) * n_splits + split) * (HD + 2) + 2 + d] = s;
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------------
// Paged INT8 decode attention on the matrix cores (QK) and the VALU (PV).
//
// One wavefront owns one split of one (sequence, KV head, chunk of up to 4
// query heads); there are no workgroup barriers.  Per 64-token tile:
//  * QK^T on v_mfma_i32_16x16x64_i8.  The A operand holds q as integer digit
//    planes: q of head h is scaled by a power of two so |q| < 2^30, rounded,
//    and written as four balanced base-256 signed digits; A row 4h+j is digit
//    j of head h.  The B operand is the K codes as stored (int8, head_dim
//    contiguous per token), so each lane loads 16 contiguous bytes per MFMA.
//    With the MFMA output layout (lane l holds rows 4*(l/16)..+3 of column
//    l%16) every lane ends up with the four exact digit sums of one (head,
//    token) pair: score = (I0 + 256 I1 + 2^16 I2 + 2^24 I3) * 2^(e-30) *
//    k_scale * 1/sqrt(head_dim).  The only rounding beyond the reference's is
//    q's 31-bit rounding relative to its head's maximum.
//  * online softmax per head inside each 16-lane row (DPP reductions).
//  * PV on the VALU: p * v_scale goes through LDS to a lane layout where each
//    lane owns head_dim/16 dimensions of one token per round; each V code is
//    converted once (v_cvt_f32_i32 of a sign-extended byte) and accumulated
//    for all 4 heads.
// Partial records (m, l, acc[head_dim]) per split go to the combine kernel.
// A tile is KT = 64 tokens, or 32 when the context is short enough that each
// wave would hold a single 64-token tile (its chain of K / V load, QK,
// softmax and PV then sets the time, and half a tile halves it).
constexpr int kAt = 64;     // tokens per tile
constexpr int kAtMin = 32;  // short contexts

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// max / sum over the 16 lanes of a DPP row, result in every lane of the row
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x124>(v));
  return fmaxf(v, dpp_f<0x128>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x124>(v);
  return v + dpp_f<0x128>(v);
}

// Sums and maxima over the same lane of the four 16-lane rows (lanes l, l ^ 16,
// l ^ 32, l ^ 48), in every lane: the rows are exchanged by v_permlane16_swap
// and v_permlane32_swap of a register with itself (VALU, no LDS), and the
// operands of each step are those of x + shfl_xor(x, 16), then 32, so the
// results are bit for bit the same.
__device__ __forceinline__ float rows4_sum(float x) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}
__device__ __forceinline__ float rows4_max(float x) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

template <int HD, int NWV, int KT, bool NEW>
__global__ __launch_bounds__(64 * NWV, HD == 256 ? 1 : 8 / NWV) void paged_attn_mfma_kernel(
    const float* __restrict__ q, const int8_t* __restrict__ kc, const float* __restrict__ ks,
    const int8_t* __restrict__ vc, const float* __restrict__ vs, const int32_t* __restrict__ tables,
    const int32_t* __restrict__ ctx_lens, const int32_t* __restrict__ win_lo, const int32_t* __restrict__ win_hi,
    int max_blocks, int bs_log2, int n_head, int n_head_kv, int n_hchunks, int split_len, int n_splits,
    bool kv_major, float* __restrict__ partial, const float* __restrict__ new_k, const float* __restrict__ new_v,
    const int32_t* __restrict__ new_slot, int8_t* kc_w, float* ks_w, int8_t* vc_w, float* vs_w) {
  constexpr int NMI = HD / 64;  // MFMAs per 16-token sub-tile
  constexpr int VD = HD / 16;   // dims per lane in the PV layout
  constexpr int VW = VD / 4;    // V dwords per lane per round
  constexpr int NSUB = KT / 16;  // QK sub-tiles of 16 tokens
  constexpr int NRR = KT / 4;    // PV rounds of 4 tokens
  static_assert(KT == 64 || KT == 32, "tile of 64 or 32 tokens");
  __shared__ float p_s[NWV][KT * 4];     // per wave: p * v_scale [token][head]
  __shared__ int row_s[NWV][2 * KT];     // per wave, two tiles: pool row of each token
  __shared__ float ks_s[NWV][2 * KT], vs_s[NWV][2 * KT];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // kv_major: the NWV waves take NWV KV heads of one split, so the slices of
  // each token row they read (adjacent in the pool row) are fetched together
  // (measured at config 5b: 129 us with 4 splits of one KV head per workgroup,
  // 110 us with 4 KV heads); otherwise NWV splits of one KV head
  const int split = kv_major ? blockIdx.x : blockIdx.x * NWV + wave;
  const int hc = blockIdx.y % n_hchunks, seq = blockIdx.z;
  const int kvh = kv_major ? (blockIdx.y / n_hchunks) * NWV + wave : blockIdx.y / n_hchunks;
  if (split >= n_splits || kvh >= n_head_kv) return;  // no barriers follow: the wave can leave
  const int group = n_head / n_head_kv;
  const int h0 = kvh * group + hc * 4;
  const int G = min(4, group - hc * 4);
  const int kv_dim = n_head_kv * HD;
  const int32_t* table = tables + (size_t)seq * max_blocks;
  // positions [lo, p_end): the sequence's window (ctx_lens and the block
  // table bound it); the splits tile it from lo (its length is at most max_ctx)
  const int lo = win_lo ? max(win_lo[seq], 0) : 0;
  const int p_end = min(min(ctx_lens[seq], win_hi ? win_hi[seq] : INT_MAX), max_blocks << bs_log2);
  const int s_begin = lo + split * split_len;
  const int s_end = min(p_end, s_begin + split_len);
  float* pw = p_s[wave];
  int* rw = row_s[wave];
  float* ksw = ks_s[wave];
  float* vsw = vs_s[wave];

  // ---- the sequence's new token (NEW: a decode step's INT8 append folded
  // into this launch).  It sits at position ctx_len - 1, the last of the last
  // split, so of that split's last tile.  Each wave of that split quantizes
  // its KV head's slice of the token's K and V rows against the rows' scales
  // (the absmax over all KV heads, kv_dim <= 1024; the arithmetic of
  // kv_quantize_pipe_kernel): lanes 0 .. HD/4 - 1 four K elements each,
  // lanes 32 .. 32 + HD/4 - 1 four V elements.  The codes reach the operand
  // layouts below through the wave's LDS: the lanes that hold the token in
  // the last tile take them, and its scales, instead of what the pool held.
  // The same dwords are written to pool row new_slot[seq] at the end of the
  // kernel (a store earlier would make the wave's later loads wait for it:
  // vector memory counts both in order).  Waves that read that row before
  // (clamped repeats of the last token) only read it into lanes that are
  // masked out and take the new scales.  The rows are requested here, with q,
  // so that both arrive in one round trip.
  constexpr int kNewC = 4;  // float4 chunks per lane of a whole new row
  const int pos_new = NEW ? ctx_lens[seq] - 1 : -1;
  const bool has_new = NEW && pos_new >= s_begin && pos_new < s_end;
  const bool nv_lane = lane >= 32;           // this lane's four new elements: V (else K)
  const int nj = min(lane & 31, HD / 4 - 1);  // ... dims 4 nj .. 4 nj + 3 of head kvh
  float4 kA[kNewC], vA[kNewC], nown;
  if (has_new) {
    const float* kr = new_k + (size_t)seq * kv_dim;
    const float* vr = new_v + (size_t)seq * kv_dim;
#pragma unroll
    for (int i = 0; i < kNewC; i++) {  // chunks past kv_dim repeat the last one (masked below)
      const int e = min(4 * lane + 256 * i, kv_dim - 4);
      kA[i] = *reinterpret_cast<const float4*>(kr + e);
      vA[i] = *reinterpret_cast<const float4*>(vr + e);
    }
    nown = *reinterpret_cast<const float4*>((nv_lane ? vr : kr) + (size_t)kvh * HD + 4 * nj);
  }

  // ---- q digit planes (A operand): row r = lane%16 is digit r%4 of head r/4,
  // lane group c = lane/16 holds dims 64*mi + 16c .. +16 of MFMA mi
  const int r = lane & 15, c = lane >> 4;
  i32x4 qa[NMI];
  float qscale;  // 2^-sh of head c (the head of this lane's scores)
  {
    const int qh = r >> 2, qj = r & 3;
    const bool hv = qh < G;
    const float* qp = q + ((size_t)seq * n_head + h0 + (hv ? qh : 0)) * HD;
    float qv[NMI][16];
    float m = 0.f;
    bool bad = false;
#pragma unroll
    for (int mi = 0; mi < NMI; mi++)
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        const float4 f = hv ? *reinterpret_cast<const float4*>(qp + 64 * mi + 16 * c + i)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
        qv[mi][i] = f.x; qv[mi][i + 1] = f.y; qv[mi][i + 2] = f.z; qv[mi][i + 3] = f.w;
      }
#pragma unroll
    for (int mi = 0; mi < NMI; mi++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        m = fmaxf(m, fabsf(qv[mi][i]));
        bad |= !(fabsf(qv[mi][i]) < INFINITY);
      }
    m = rows4_max(m);  // same head, the other dims
    const int badi = rows4_max(bad ? 1.f : 0.f) != 0.f;
    int e = 0;
    if (m > 0.f) (void)frexpf(m, &e);  // m < 2^e
    // the values are scaled (2^(30 - e) itself overflows below 2^-97); the
    // shift stops at 149, so that 2^-sh stays a (subnormal) fp32 value
    const int sh = min(30 - e, 149);
    const float qs_row = badi ? __builtin_nanf("") : ldexpf(1.0f, -sh);
#pragma unroll
    for (int mi = 0; mi < NMI; mi++) {
      uint32_t dw[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t acc = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
          const int qi = (int)rintf(ldexpf(qv[mi][4 * k + b], sh));  // |qi| <= 2^30
          const uint32_t u = ((uint32_t)qi + 0x80808080u) ^ 0x80808080u;  // balanced digits
          acc |= ((u >> (8 * (qj & 3))) & 0xFFu) << (8 * b);
        }
        dw[k] = hv ? acc : 0u;
      }
      qa[mi] = i32x4{(int)dw[0], (int)dw[1], (int)dw[2], (int)dw[3]};
    }
    qscale = __shfl(qs_row, 4 * c, 64);  // lane 4c holds digit 0 of head c
  }
  i32x4 knew[NMI];
  uint32_t vnew[VW];
  float ksc_new = 0.f, vsc_new = 0.f;
  uint32_t ncode = 0;
  if (has_new) {
    float ka = 0.f, va = 0.f;
#pragma unroll
    for (int i = 0; i < kNewC; i++) {
      if (4 * lane + 256 * i < kv_dim) {
        ka = fmaxf(ka, fmaxf(fmaxf(fabsf(kA[i].x), fabsf(kA[i].y)), fmaxf(fabsf(kA[i].z), fabsf(kA[i].w))));
        va = fmaxf(va, fmaxf(fmaxf(fabsf(vA[i].x), fabsf(vA[i].y)), fmaxf(fabsf(vA[i].z), fabsf(vA[i].w))));
      }
    }
    ka = wave_max_dpp(ka);
    va = wave_max_dpp(va);
    const float kinv = ka != 0.0f ? 127.0f / ka : 0.0f, vinv = va != 0.0f ? 127.0f / va : 0.0f;
    ksc_new = ka / 127.0f;  // 0 for an all-zero row
    vsc_new = va / 127.0f;
    ncode = kv_pack4(nown.x, nown.y, nown.z, nown.w, nv_lane ? vinv : kinv);
    // K code dwords 0 .. HD/4 - 1, V code dwords 32 .. 32 + HD/4 - 1 (the
    // wave's p_s is free until its first tile)
    uint32_t* xw = reinterpret_cast<uint32_t*>(p_s[wave]);
    xw[lane] = ncode;
#pragma unroll
    for (int mi = 0; mi < NMI; mi++) {  // K: dims 64 mi + 16 c .. + 16
      const uint4 t = *reinterpret_cast<const uint4*>(xw + 16 * mi + 4 * (lane >> 4));
      knew[mi] = i32x4{(int)t.x, (int)t.y, (int)t.z, (int)t.w};
    }
#pragma unroll
    for (int w4 = 0; w4 < VW; w4++) vnew[w4] = xw[32 + VW * (lane & 15) + w4];  // V: dims VD dg .. + VD
  }
  const float inv_sqrt = 1.0f / sqrtf((float)HD);
  const int bs_mask = (1 << bs_log2) - 1;

  float run_m = -INFINITY, run_l = 0.f;  // head c, replicated over the 16-lane row
  const int tg = lane >> 4, dg = lane & 15;  // PV layout: token group, dimension group
  float acc[4][VD];
#pragma unroll
  for (int h = 0; h < 4; h++)
#pragma unroll
    for (int d = 0; d < VD; d++) acc[h][d] = 0.f;

  // Software pipeline over the split's tiles (two register / LDS slots):
  // while tile i is computed, the K and V of tile i+1 and the block-table
  // entries of tile i+2 are in flight.
  const int n_tiles = s_end > s_begin ? (s_end - s_begin + KT - 1) / KT : 0;
  auto tok_row = [&](int tab, int t) { return tab * (1 << bs_log2) + (t & bs_mask); };
  // token of lane l < KT in tile i (lanes past KT repeat a valid token; only
  // lanes < KT store rows and scales)
  auto tile_tok = [&](int i) { return min(s_begin + i * KT + lane, s_end - 1); };
  int tab_n = 0, row_n = 0;
  float ks_n = 0.f, vs_n = 0.f;
  i32x4 kb[2][NSUB][NMI];
  uint32_t vraw[2][NRR][VW];
  auto issue_kv = [&](auto slot_c) {  // K and V of the tile whose rows sit in rw[slot]
    constexpr int sl = decltype(slot_c)::value;
    const int* rws = rw + sl * KT;
#pragma unroll
    for (int sub = 0; sub < NSUB; sub++) {
      const int8_t* kp = kc + (size_t)rws[16 * sub + r] * kv_dim + (size_t)kvh * HD + 16 * c;
#pragma unroll
      for (int mi = 0; mi < NMI; mi++) kb[sl][sub][mi] = *reinterpret_cast<const i32x4*>(kp + 64 * mi);
    }
#pragma unroll
    for (int rr = 0; rr < NRR; rr++) {
      // One instruction reads whole pool-row slices of V (16 lanes x VD
      // bytes per token), each once per step: nontemporal (config 5b 103.4 ->
      // 93.4 us).  K slices are read by NMI instructions each, where the hint
      // costs more than it saves (97.9 us with K too).
      const int8_t* vp = vc + (size_t)rws[4 * rr + tg] * kv_dim + (size_t)kvh * HD + VD * dg;
      if constexpr (VW == 1) {
        vraw[sl][rr][0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(vp));
      } else if constexpr (VW == 2) {
        const u32x2 v2 = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(vp));
        vraw[sl][rr][0] = v2.x; vraw[sl][rr][1] = v2.y;
      } else {
        const u32x4v v4 = __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(vp));
        vraw[sl][rr][0] = v4.x; vraw[sl][rr][1] = v4.y; vraw[sl][rr][2] = v4.z; vraw[sl][rr][3] = v4.w;
      }
    }
  };
  if (n_tiles > 0) {  // prologue: rows and K / V of tile 0, table entry of tile 1
    const int t = tile_tok(0);
    row_n = tok_row(table[t >> bs_log2], t);
    if (lane < KT) rw[lane] = row_n;
    ks_n = ks[row_n];
    vs_n = vs[row_n];
    const int t1 = tile_tok(1);
    tab_n = table[t1 >> bs_log2];
    issue_kv(std::integral_constant<int, 0>{});
  }

  auto tile = [&](auto slot_c, int i) {
    constexpr int sl = decltype(slot_c)::value;
    const int t0 = s_begin + i * KT;
    float* ksl = ksw + sl * KT;
    float* vsl = vsw + sl * KT;
    if (lane < KT) {  // scales of tile i (loaded one iteration ago)
      const bool nt = has_new && tile_tok(i) == pos_new;
      ksl[lane] = nt ? ksc_new : ks_n;
      vsl[lane] = nt ? vsc_new : vs_n;
    }
    if (has_new && i == n_tiles - 1) {
      // the new token's codes into this tile's operands (the tile's loads
      // land first; the next tile's loads, issued below, are clamped repeats)
      const int jr = pos_new - t0;
#pragma unroll
      for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
        for (int mi = 0; mi < NMI; mi++)
          if (16 * sub + r == jr) kb[sl][sub][mi] = knew[mi];
#pragma unroll
      for (int rr = 0; rr < NRR; rr++)
#pragma unroll
        for (int w4 = 0; w4 < VW; w4++)
          if (4 * rr + tg == jr) vraw[sl][rr][w4] = vnew[w4];
    }
    {  // rows of tile i+1, their scales, the table entry of tile i+2, then K and V of tile i+1
      const int t = tile_tok(i + 1);
      row_n = tok_row(tab_n, t);
      if (lane < KT) rw[(sl ^ 1) * KT + lane] = row_n;
      ks_n = ks[row_n];
      vs_n = vs[row_n];
      const int t2 = tile_tok(i + 2);
      tab_n = table[t2 >> bs_log2];
      issue_kv(std::integral_constant<int, sl ^ 1>{});
    }
    // scores of head c, tokens 16*sub + r
    float sc[NSUB];
#pragma unroll
    for (int sub = 0; sub < NSUB; sub++) {
      i32x4 cacc = i32x4{0, 0, 0, 0};
#pragma unroll
      for (int mi = 0; mi < NMI; mi++)
        cacc = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[mi], kb[sl][sub][mi], cacc, 0, 0, 0);
      const float sv =
          fmaf(16777216.0f, (float)cacc[3], fmaf(65536.0f, (float)cacc[2], (float)(cacc[0] + (cacc[1] << 8))));
      const bool valid = (t0 + 16 * sub + r < s_end) && c < G;
      sc[sub] = valid ? sv * qscale * ksl[16 * sub + r] * inv_sqrt : -INFINITY;
    }
    // online softmax of head c over the tile
    float tm = fmaxf(sc[0], sc[1]);
    if constexpr (NSUB == 4) tm = fmaxf(tm, fmaxf(sc[2], sc[3]));
    const float tmax = row16_max(tm);
    const float m_new = fmaxf(run_m, tmax);
    float corr = 1.0f, p[NSUB];
#pragma unroll
    for (int sub = 0; sub < NSUB; sub++) p[sub] = 0.f;
    if (m_new != -INFINITY) {
      corr = __expf(run_m - m_new);
#pragma unroll
      for (int sub = 0; sub < NSUB; sub++) p[sub] = __expf(sc[sub] - m_new);
    }
    float ps = p[0] + p[1];
    if constexpr (NSUB == 4) ps = ps + (p[2] + p[3]);
    run_l = run_l * corr + row16_sum(ps);
    run_m = m_new;
#pragma unroll
    for (int sub = 0; sub < NSUB; sub++) pw[(16 * sub + r) * 4 + c] = p[sub] * vsl[16 * sub + r];
    // rescale the PV accumulators by each head's correction
#pragma unroll
    for (int h = 0; h < 4; h++) {
      const float ch = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, corr), 16 * h));
#pragma unroll
      for (int d = 0; d < VD; d++) acc[h][d] *= ch;
    }
    // PV
#pragma unroll
    for (int rr = 0; rr < NRR; rr++) {
      const float4 pv = *reinterpret_cast<const float4*>(&pw[(4 * rr + tg) * 4]);
      const float ph[4] = {pv.x, pv.y, pv.z, pv.w};
      float f[VD];
#pragma unroll
      for (int w = 0; w < VW; w++)
#pragma unroll
        for (int b = 0; b < 4; b++)  // one v_cvt_f32_i32 with a sign-extended byte select
          f[4 * w + b] = (float)(int8_t)(vraw[sl][rr][w] >> (8 * b));
#pragma unroll
      for (int h = 0; h < 4; h++)
#pragma unroll
        for (int d = 0; d < VD; d++) acc[h][d] = fmaf(ph[h], f[d], acc[h][d]);
    }
  };
  for (int i = 0; i < n_tiles; i += 2) {
    tile(std::integral_constant<int, 0>{}, i);
    if (i + 1 < n_tiles) tile(std::integral_constant<int, 1>{}, i + 1);
  }

  // sum the four token groups, write the split's records
#pragma unroll
  for (int h = 0; h < 4; h++)
#pragma unroll
    for (int d = 0; d < VD; d++) {
      acc[h][d] = rows4_sum(acc[h][d]);
    }
  if (tg == 0) {
#pragma unroll
    for (int h = 0; h < 4; h++) {
      if (h < G) {
        float* rec = partial + (((size_t)seq * n_head + h0 + h) * n_splits + split) * (HD + 2);
#pragma unroll
        for (int d = 0; d < VD; d++) rec[2 + VD * dg + d] = acc[h][d];
      }
    }
  }
  if (r == 0 && c < G) {
    float* rec = partial + (((size_t)seq * n_head + h0 + c) * n_splits + split) * (HD + 2);
    rec[0] = run_m;
    rec[1] = run_l;
  }
  if (has_new && hc == 0) {  // the new token's row slices and scales into the pool
    const int32_t slot = new_slot[seq];
    if (slot >= 0) {
      if ((lane & 31) < HD / 4)
        *reinterpret_cast<uint32_t*>((nv_lane ? vc_w : kc_w) + (size_t)slot * kv_dim + (size_t)kvh * HD + 4 * nj) =
            ncode;
      if (kvh == 0 && lane == 0) {
        ks_w[slot] = ksc_new;
        vs_w[slot] = vsc_new;
      }
    }
  }
}

// Log-sum-exp merge of the split partials of one (sequence, head).  The block
// is CG groups of HD threads: thread (g, d) folds splits g, g + CG, g + 2 CG,
// ... into a running (max, sum, acc[d]), a chunk of 8 splits at a time with
// the next chunk's loads issued before the current one is folded (indices
// clamped, so every load is unconditional; splits past the end are masked
// after loading).  The CG running triples are then merged through LDS.  One
// memory round trip for up to 8 CG splits, where a max / weights / sum pass
// over the partials would take three.  CG fills 1024 threads, so the 129
// splits of a 4097-token context (32-token tiles) take three round trips per
// group.
constexpr int kMaxSplits = 1024;

template <int HD>
constexpr int combine_groups() {
  return 1024 / HD;
}

template <int HD>
__global__ __launch_bounds__(HD * combine_groups<HD>()) void attn_combine_kernel(const float* __restrict__ partial,
                                                                               int n_splits, int n_head,
                                                                               float* __restrict__ out) {
  constexpr int CG = combine_groups<HD>(), CH = 8;
  __shared__ float m_s[CG], l_s[CG];
  __shared__ float a_s[CG][HD];
  const int h = blockIdx.x, seq = blockIdx.y;
  const int d = threadIdx.x % HD, g = threadIdx.x / HD;
  const float* rec = partial + ((size_t)seq * n_head + h) * n_splits * (HD + 2);
  float M = -INFINITY, L = 0.f, A = 0.f;
  float mc[CH], lc[CH], ac[CH];
  auto load = [&](float (&m)[CH], float (&l)[CH], float (&a)[CH], int c0) {
#pragma unroll
    for (int u = 0; u < CH; u++) {
      const int sp = g + (c0 + u) * CG;
      const float* r = rec + (size_t)min(sp, n_splits - 1) * (HD + 2);
      m[u] = r[0];
      l[u] = r[1];
      a[u] = r[2 + d];
    }
#pragma unroll
    for (int u = 0; u < CH; u++)
      if (g + (c0 + u) * CG >= n_splits) m[u] = -INFINITY;
  };
  const int per = g < n_splits ? (n_splits - g + CG - 1) / CG : 0;  // this group's splits
  load(mc, lc, ac, 0);
  for (int c0 = 0; c0 < per; c0 += CH) {
    float mn[CH], ln[CH], an[CH];
    load(mn, ln, an, c0 + CH);
    float cm = M;
#pragma unroll
    for (int u = 0; u < CH; u++) cm = fmaxf(cm, mc[u]);
    const float f = cm == -INFINITY ? 1.f : __expf(M - cm);
    L *= f;
    A *= f;
#pragma unroll
    for (int u = 0; u < CH; u++) {
      const float w = mc[u] == -INFINITY ? 0.f : __expf(mc[u] - cm);
      L = fmaf(w, lc[u], L);
      A = fmaf(w, ac[u], A);
    }
    M = cm;
#pragma unroll
    for (int u = 0; u < CH; u++) {
      mc[u] = mn[u];
      lc[u] = ln[u];
      ac[u] = an[u];
    }
  }
  if (d == 0) {
    m_s[g] = M;  // every thread of the group holds the same M and L
    l_s[g] = L;
  }
  a_s[g][d] = A;
  __syncthreads();
  if (g == 0) {
    float mx = m_s[0];
#pragma unroll
    for (int i = 1; i < CG; i++) mx = fmaxf(mx, m_s[i]);
    float lt = 0.f, at = 0.f;
#pragma unroll
    for (int i = 0; i < CG; i++) {
      const float w = m_s[i] == -INFINITY ? 0.f : __expf(m_s[i] - mx);
      lt = fmaf(w, l_s[i], lt);
      at = fmaf(w, a_s[i][d], at);
    }
    out[((size_t)seq * n_head + h) * HD + d] = lt > 0.f ? at * (1.0f / lt) : 0.f;
  }
}

int pick_splits(int units, int max_len) {
  // aim for ~4 workgroups per CU, splits of at least one tile
  const int target = device_cu_count() * 4;
  int splits = std::max(1, (target + units - 1) / units);
  const int max_splits = std::max(1, (max_len + kTile - 1) / kTile);
  return std::min(std::min(splits, max_splits), kMaxSplits);
}

template <int HD, class Src>
hipError_t run_attn(const float* q, Src src, const int32_t* tables, const int32_t* ctx, const int32_t* win_lo,
                    const int32_t* win_hi, int max_blocks, int n_seq, int n_head, int n_head_kv, int pb, int pe,
                    int max_len, int n_splits, float* partial, float* out, hipStream_t s) {
  int split_len = (max_len + n_splits - 1) / n_splits;
  split_len = std::max(kTile, (split_len + kTile - 1) / kTile * kTile);
  hipLaunchKernelGGL((attn_split_kernel<HD, Src>), dim3(n_splits, n_head_kv, n_seq),
                     dim3(kThreads), 0, s, q, src, tables, ctx, win_lo, win_hi, max_blocks, n_head, n_head_kv, pb,
                     pe, split_len, n_splits, partial);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3(n_head, n_seq), dim3(HD * combine_groups<HD>()), 0, s, partial,
                     n_splits, n_head, out);
  return hipGetLastError();
}

}  // namespace

namespace {

int log2_exact(int v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int l = 0;
  while ((1 << l) < v) l++;
  return l;
}

// The matrix-core kernel needs a power-of-two block size and 16-byte aligned
// q and code pools (16-byte K / q loads).
bool paged_mfma_ok(const PagedAttnArgs& a) {
  return log2_exact(a.block_size) >= 0 && ((uintptr_t)a.k_codes & 15) == 0 &&
         ((uintptr_t)a.v_codes & 15) == 0 && ((uintptr_t)a.q & 15) == 0;
}

// Splits of the context for the matrix-core kernel: about 8 wavefronts per CU,
// whole 64-token tiles.
// Split length (a multiple of the tile) for about 8 waves per CU; the
// 32-token tile when even 64-token splits leave fewer waves than that.
void paged_mfma_splits(const PagedAttnArgs& a, int* n_splits, int* split_len, int* tile) {
  const int group = a.n_head / a.n_head_kv;
  const int units = a.n_seq * a.n_head_kv * ((group + 3) / 4);
  const int target = device_cu_count() * 8;
  const int want = std::max(1, (target + units - 1) / units);
  const int raw = (a.max_ctx + want - 1) / want;
  const int kt = raw <= kAtMin && (a.max_ctx + kAtMin - 1) / kAtMin <= kMaxSplits ? kAtMin : kAt;
  int len = std::max(kt, (raw + kt - 1) / kt * kt);
  len = std::max(len, (a.max_ctx + kMaxSplits - 1) / kMaxSplits);
  len = (len + kt - 1) / kt * kt;
  *split_len = len;
  *n_splits = std::max(1, (a.max_ctx + len - 1) / len);
  *tile = kt;
}

}  // namespace

size_t paged_attn_workspace_bytes(const PagedAttnArgs& a, int* n_splits_out) {
  int n;
  if (paged_mfma_ok(a)) {
    int len, kt;
    paged_mfma_splits(a, &n, &len, &kt);
  } else {
    n = pick_splits(a.n_seq * a.n_head_kv, a.max_ctx);
  }
  if (n_splits_out) *n_splits_out = n;
  return (size_t)a.n_seq * a.n_head * n * (a.head_dim + 2) * sizeof(float);
}

template <int HD>
hipError_t run_paged_mfma(const PagedAttnArgs& a, float* part, hipStream_t s) {
  int n_splits, split_len, kt;
  paged_mfma_splits(a, &n_splits, &split_len, &kt);
  const int group = a.n_head / a.n_head_kv, n_hchunks = (group + 3) / 4;
  // one workgroup per split over 8 (else 4) KV heads when they divide n_head_kv
  auto launch = [&](auto nwv_c, auto new_c, bool kv_major) {
    constexpr int NWV = decltype(nwv_c)::value;
    constexpr bool NEW = decltype(new_c)::value;
    const dim3 grid = kv_major
        ? dim3((unsigned)n_splits, (unsigned)(a.n_head_kv / NWV * n_hchunks), (unsigned)a.n_seq)
        : dim3((unsigned)((n_splits + NWV - 1) / NWV), (unsigned)(a.n_head_kv * n_hchunks), (unsigned)a.n_seq);
    if (grid.y > 65535 || grid.z > 65535) return hipErrorInvalidValue;
    auto kern = kt == kAtMin ? paged_attn_mfma_kernel<HD, NWV, kAtMin, NEW> : paged_attn_mfma_kernel<HD, NWV, kAt, NEW>;
    hipLaunchKernelGGL(kern, grid, dim3(64 * NWV), 0, s, a.q, a.k_codes, a.k_scales, a.v_codes, a.v_scales,
                       a.block_tables, a.ctx_lens, a.win_lo, a.win_hi, a.max_blocks_per_seq, log2_exact(a.block_size),
                       a.n_head, a.n_head_kv, n_hchunks, split_len, n_splits, kv_major, part, a.new_k, a.new_v,
                       a.new_slot, const_cast<int8_t*>(a.k_codes), const_cast<float*>(a.k_scales),
                       const_cast<int8_t*>(a.v_codes), const_cast<float*>(a.v_scales));
    return hipGetLastError();
  };
  auto go = [&](auto nwv_c, bool kv_major) {
    return a.new_k ? launch(nwv_c, std::true_type{}, kv_major) : launch(nwv_c, std::false_type{}, kv_major);
  };
  hipError_t e0;
  if constexpr (HD < 256) {  // head_dim 256 fits one wave per SIMD only: 4 waves
    // 8 KV heads per workgroup, unless that leaves CUs without a workgroup
    const long wg8 = (long)n_splits * (a.n_head_kv / 8) * n_hchunks * a.n_seq;
    e0 = a.n_head_kv % 8 == 0 && wg8 >= device_cu_count()
             ? go(std::integral_constant<int, 8>{}, true)
             : go(std::integral_constant<int, 4>{}, a.n_head_kv % 4 == 0);
  } else {
    e0 = go(std::integral_constant<int, 4>{}, a.n_head_kv % 4 == 0);
  }
  if (e0 != hipSuccess) return e0;
  hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3(a.n_head, a.n_seq), dim3(HD * combine_groups<HD>()), 0, s, part,
                     n_splits, a.n_head, a.out);
  return hipGetLastError();
}

hipError_t launch_paged_attn_append(const PagedAttnArgs& a, void* workspace, hipStream_t s) {
  const int kv_dim = a.n_head_kv * a.head_dim;
  const bool fused = paged_mfma_ok(a) && !a.win_lo && !a.win_hi && kv_dim % 64 == 0 && kv_dim <= 1024 &&
                     a.head_dim <= 128 && ((uintptr_t)a.new_k & 15) == 0 && ((uintptr_t)a.new_v & 15) == 0;
  if (!fused) {
    hipError_t e = launch_paged_kv_append(a.new_k, a.new_v, a.new_slot, const_cast<int8_t*>(a.k_codes),
                                          const_cast<float*>(a.k_scales), const_cast<int8_t*>(a.v_codes),
                                          const_cast<float*>(a.v_scales), (size_t)a.n_seq, (size_t)kv_dim, s);
    if (e != hipSuccess) return e;
    PagedAttnArgs b = a;
    b.new_k = b.new_v = nullptr;
    b.new_slot = nullptr;
    return launch_paged_attn(b, workspace, s);
  }
  float* part = static_cast<float*>(workspace);
  switch (a.head_dim) {
    case 64: return run_paged_mfma<64>(a, part, s);
    case 128: return run_paged_mfma<128>(a, part, s);
    case 256: return run_paged_mfma<256>(a, part, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_paged_attn(const PagedAttnArgs& a, void* workspace, hipStream_t s) {
  if (a.new_k) return hipErrorInvalidValue;  // launch_paged_attn_append
  float* part = static_cast<float*>(workspace);
  if (paged_mfma_ok(a)) {
    switch (a.head_dim) {
      case 64: return run_paged_mfma<64>(a, part, s);
      case 128: return run_paged_mfma<128>(a, part, s);
      case 256: return run_paged_mfma<256>(a, part, s);
      default: return hipErrorInvalidValue;
    }
  }
  int n_splits = 0;
  paged_attn_workspace_bytes(a, &n_splits);
  PagedSrc src{a.k_codes, a.k_scales, a.v_codes, a.v_scales, nullptr, a.block_size,
               a.n_head_kv * a.head_dim};
  switch (a.head_dim) {
    case 64:
      return run_attn<64>(a.q, src, a.block_tables, a.ctx_lens, a.win_lo, a.win_hi, a.max_blocks_per_seq, a.n_seq,
                          a.n_head, a.n_head_kv, 0, 0, a.max_ctx, n_splits, part, a.out, s);
    case 128:
      return run_attn<128>(a.q, src, a.block_tables, a.ctx_lens, a.win_lo, a.win_hi, a.max_blocks_per_seq, a.n_seq,
                           a.n_head, a.n_head_kv, 0, 0, a.max_ctx, n_splits, part, a.out, s);
    case 256:
      return run_attn<256>(a.q, src, a.block_tables, a.ctx_lens, a.win_lo, a.win_hi, a.max_blocks_per_seq, a.n_seq,
                           a.n_head, a.n_head_kv, 0, 0, a.max_ctx, n_splits, part, a.out, s);
    default:
      return hipErrorInvalidValue;
  }
}

// Scratch of the allocation-free entry point (ssdq_paged_attention_int8_noalloc_dev):
// the split partials of paged attention live in this file-scope device array,
// which every GPU the library runs on holds until the process ends.  Host code
// never passes the array's name to a kernel (on the host it is only a stand-in
// for the symbol): it uses the device address hipGetSymbolAddress returns for
// the current device, looked up once per device.
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

hipError_t scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}
}  // namespace

hipError_t launch_paged_attn_noalloc(const PagedAttnArgs& a, hipStream_t s, size_t* need) {
  const size_t bytes = paged_attn_workspace_bytes(a, nullptr);
  if (need) *need = bytes;
  if (bytes > kNoAllocScratchBytes) return hipErrorInvalidValue;
  void* p = nullptr;
  hipError_t e = scratch_address(&p);
  if (e != hipSuccess) return e;
  // every (sequence, head, split) record the combine reads is written by the
  // split kernel of the same call (empty splits write m = -inf, l = 0): the
  // scratch needs no clearing
  return launch_paged_attn(a, p, s);
}

size_t flash_attn_f32_workspace_bytes(int n_head, int n_head_kv, int head_dim, int len,
                                      int* n_splits_out) {
  const int n_splits = pick_splits(n_head_kv, std::max(len, 1));
  if (n_splits_out) *n_splits_out = n_splits;
  return (size_t)n_head * n_splits * (head_dim + 2) * sizeof(float);
}

hipError_t launch_flash_attn_f32(const float* q, const float* k, const float* v, float* out,
                                 int n_head, int n_head_kv, int head_dim, int seq_len,
                                 int window_start, int window_end, void* workspace,
                                 hipStream_t s) {
  const int pe = std::min(window_end, seq_len);
  const int pb = window_start;
  const int len = std::max(0, pe - pb);
  int n_splits = 1;
  flash_attn_f32_workspace_bytes(n_head, n_head_kv, head_dim, len, &n_splits);
  float* ws = static_cast<float*>(workspace);
  FlatSrc src{k, v, n_head_kv * head_dim};
  switch (head_dim) {
    case 64:
      return run_attn<64>(q, src, nullptr, nullptr, nullptr, nullptr, 0, 1, n_head, n_head_kv, pb, pe, len,
                          n_splits, ws, out, s);
    case 128:
      return run_attn<128>(q, src, nullptr, nullptr, nullptr, nullptr, 0, 1, n_head, n_head_kv, pb, pe, len,
                           n_splits, ws, out, s);
    case 256:
      return run_attn<256>(q, src, nullptr, nullptr, nullptr, nullptr, 0, 1, n_head, n_head_kv, pb, pe, len,
                           n_splits, ws, out, s);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace ssdq
