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
#include <type_traits>

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
    const int32_t* __restrict__ ctx_lens, int max_blocks_per_seq, int n_head, int n_head_kv,
    int pos_begin_flat, int pos_end_flat, int split_len, int n_splits,
    float* __restrict__ partial) {
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
    p_begin = 0;
    // never address past the block table, whatever ctx_lens holds
    p_end = min(ctx_lens[seq], max_blocks_per_seq * src.block_size);
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

template <int HD>
__global__ __launch_bounds__(HD) void attn_combine_kernel(const float* __restrict__ partial,
                                                          int n_splits, int n_head,
                                                          float* __restrict__ out) {
  const int h = blockIdx.x, seq = blockIdx.y, d = threadIdx.x;
  const float* rec = partial + ((size_t)seq * n_head + h) * n_splits * (HD + 2);
  float M = -INFINITY;
  for (int s = 0; s < n_splits; s++) M = fmaxf(M, rec[(size_t)s * (HD + 2)]);
  float l = 0.f, a = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < n_splits; s++) {
      const float* r = rec + (size_t)s * (HD + 2);
      if (r[0] == -INFINITY) continue;
      const float w = __expf(r[0] - M);
      l = fmaf(w, r[1], l);
      a = fmaf(w, r[2 + d], a);
    }
  }
  out[((size_t)seq * n_head + h) * HD + d] = l > 0.f ? a * (1.0f / l) : 0.f;
}

int pick_splits(int units, int max_len) {
  // aim for ~4 workgroups per CU, splits of at least one tile
  const int target = device_cu_count() * 4;
  int splits = std::max(1, (target + units - 1) / units);
  const int max_splits = std::max(1, (max_len + kTile - 1) / kTile);
  return std::min(splits, max_splits);
}

template <int HD, class Src>
hipError_t run_attn(const float* q, Src src, const int32_t* tables, const int32_t* ctx,
                    int max_blocks, int n_seq, int n_head, int n_head_kv, int pb, int pe,
                    int max_len, int n_splits, float* partial, float* out, hipStream_t s) {
  int split_len = (max_len + n_splits - 1) / n_splits;
  split_len = std::max(kTile, (split_len + kTile - 1) / kTile * kTile);
  hipLaunchKernelGGL((attn_split_kernel<HD, Src>), dim3(n_splits, n_head_kv, n_seq),
                     dim3(kThreads), 0, s, q, src, tables, ctx, max_blocks, n_head, n_head_kv, pb,
                     pe, split_len, n_splits, partial);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((attn_combine_kernel<HD>), dim3(n_head, n_seq), dim3(HD), 0, s, partial,
                     n_splits, n_head, out);
  return hipGetLastError();
}

}  // namespace

size_t paged_attn_workspace_bytes(const PagedAttnArgs& a, int* n_splits_out) {
  const int n = pick_splits(a.n_seq * a.n_head_kv, a.max_ctx);
  if (n_splits_out) *n_splits_out = n;
  return (size_t)a.n_seq * a.n_head * n * (a.head_dim + 2) * sizeof(float);
}

hipError_t launch_paged_attn(const PagedAttnArgs& a, void* workspace, hipStream_t s) {
  int n_splits = 0;
  paged_attn_workspace_bytes(a, &n_splits);
  PagedSrc src{a.k_codes, a.k_scales, a.v_codes, a.v_scales, nullptr, a.block_size,
               a.n_head_kv * a.head_dim};
  float* part = static_cast<float*>(workspace);
  switch (a.head_dim) {
    case 64:
      return run_attn<64>(a.q, src, a.block_tables, a.ctx_lens, a.max_blocks_per_seq, a.n_seq,
                          a.n_head, a.n_head_kv, 0, 0, a.max_ctx, n_splits, part, a.out, s);
    case 128:
      return run_attn<128>(a.q, src, a.block_tables, a.ctx_lens, a.max_blocks_per_seq, a.n_seq,
                           a.n_head, a.n_head_kv, 0, 0, a.max_ctx, n_splits, part, a.out, s);
    case 256:
      return run_attn<256>(a.q, src, a.block_tables, a.ctx_lens, a.max_blocks_per_seq, a.n_seq,
                           a.n_head, a.n_head_kv, 0, 0, a.max_ctx, n_splits, part, a.out, s);
    default:
      return hipErrorInvalidValue;
  }
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
      return run_attn<64>(q, src, nullptr, nullptr, 0, 1, n_head, n_head_kv, pb, pe, len,
                          n_splits, ws, out, s);
    case 128:
      return run_attn<128>(q, src, nullptr, nullptr, 0, 1, n_head, n_head_kv, pb, pe, len,
                           n_splits, ws, out, s);
    case 256:
      return run_attn<256>(q, src, nullptr, nullptr, 0, 1, n_head, n_head_kv, pb, pe, len,
                           n_splits, ws, out, s);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace ssdq
