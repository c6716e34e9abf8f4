// Device-resident GGUF weights and the decoder-layer step that reads them.
//
// ssdq_weights keeps each tensor's raw file bytes in HBM, uploaded once and
// found by its GGUF name.  It replaces SsdStreamer::load_layer /
// load_tensor_f32 (src/ssd/streamer.rs:33-66), which re-read a layer's
// tensors and dequantize them to f32 on every load (Q4_K to zeros,
// streamer.rs:119-123); here the quantized blocks stay as the file has them
// and the matvec kernels decode them in place.
//
// ssdq_decode_layer_dev is one layer of forward_pass for one token
// (src/inference/transformer.rs:319-397) on those tensors, with the KV cache
// in the paged INT8 pool: RMSNorm, QKV + RoPE, INT8 append, paged GQA
// attention, output projection, residual + RMSNorm, SwiGLU, down projection,
// residual.  Every step is an existing dev entry point; this file only wires
// them, so each step keeps the parity its own tests establish.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ssdq.h"
#include "launch.hpp"

using ssdq::api_fail;
using ssdq::api_hip_fail;
using ssdq::api_ok;

namespace {

constexpr size_t kArenaBytes = 256ull << 20;  // device memory is taken in pieces of at least this
constexpr size_t kAlign = 256;                // every tensor starts on a 256-byte boundary
constexpr size_t kMaxDims = 4;                // GGML_MAX_DIMS

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct Tensor {
  void* dev = nullptr;
  int dtype = 0;
  uint64_t dims[kMaxDims] = {0, 0, 0, 0};
  size_t n_dims = 0;
  size_t bytes = 0;
};

// Restores the caller's current device on scope exit.
struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

}  // namespace

struct ssdq_weights {
  mutable std::mutex mu;
  int device = 0;
  hipStream_t stream = nullptr;  // uploads
  std::vector<void*> arenas;
  size_t arena_cap = 0;   // capacity of the last arena
  size_t arena_used = 0;  // bytes used in the last arena
  std::unordered_map<std::string, Tensor> tensors;
  size_t total = 0;  // tensor bytes resident
};

namespace {

// Bump allocation from the store's arenas; a tensor larger than an arena gets
// an arena of its own size.
hipError_t store_alloc(ssdq_weights* w, size_t bytes, void** out) {
  size_t off = align_up(w->arena_used, kAlign);
  if (w->arenas.empty() || off + bytes > w->arena_cap) {
    const size_t cap = bytes > kArenaBytes ? align_up(bytes, 2u << 20) : kArenaBytes;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, cap);
    if (e != hipSuccess) return e;
    w->arenas.push_back(p);
    w->arena_cap = cap;
    off = 0;
  }
  *out = (char*)w->arenas.back() + off;
  w->arena_used = off + bytes;
  return hipSuccess;
}

const Tensor* find(const ssdq_weights* w, const std::string& name) {
  auto it = w->tensors.find(name);
  return it == w->tensors.end() ? nullptr : &it->second;
}

}  // namespace

extern "C" {

int ssdq_weights_create(int device, ssdq_weights** out) {
  if (!out) return api_fail(SSDQ_ERR_INVALID_ARG, "ssdq_weights_create: out is NULL");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
    return api_fail(SSDQ_ERR_NO_DEVICE, "ssdq_weights_create: no HIP device");
  if (device < 0 && hipGetDevice(&device) != hipSuccess) device = 0;
  if (device >= n) return api_fail(SSDQ_ERR_NO_DEVICE, "ssdq_weights_create: device %d of %d", device, n);
  DeviceGuard g(device);
  auto* w = new ssdq_weights();
  w->device = device;
  hipError_t e = hipStreamCreateWithFlags(&w->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete w;
    return api_hip_fail(e, "ssdq_weights_create");
  }
  *out = w;
  return api_ok();
}

void ssdq_weights_destroy(ssdq_weights* w) {
  if (!w) return;
  {
    DeviceGuard g(w->device);
    (void)hipDeviceSynchronize();  // kernels queued on any stream may still read the tensors
    for (void* p : w->arenas) (void)hipFree(p);
    if (w->stream) (void)hipStreamDestroy(w->stream);
  }
  delete w;
}

int ssdq_weights_put(ssdq_weights* w, const char* name, int dtype, const uint64_t* dims, size_t n_dims,
                     const void* data, size_t data_len) {
  const char* fn = "ssdq_weights_put";
  if (!w || !name || !dims) return api_fail(SSDQ_ERR_INVALID_ARG, "%s: NULL pointer", fn);
  if (n_dims == 0 || n_dims > kMaxDims) return api_fail(SSDQ_ERR_INVALID_ARG, "%s: %zu dims (1-4)", fn, n_dims);
  uint64_t n_el = 1;
  for (size_t i = 0; i < n_dims; i++) {
    if (dims[i] == 0 || n_el > UINT64_MAX / dims[i])
      return api_fail(SSDQ_ERR_INVALID_ARG, "%s: %s: bad dimension %zu", fn, name, i);
    n_el *= dims[i];
  }
  // the size the type gives (GgmlType::block_size / type_size); types this
  // library does not know are kept as the bytes given
  const size_t bs = ssdq_block_size(dtype), ts = ssdq_type_size(dtype);
  if (bs) {
    if (dims[0] % bs)
      return api_fail(SSDQ_ERR_INVALID_ARG, "%s: %s: row length %llu is not a multiple of the block (%zu)", fn,
                      name, (unsigned long long)dims[0], bs);
    const uint64_t want = n_el / bs * ts;
    if (data_len != want)
      return api_fail(SSDQ_ERR_INVALID_ARG, "%s: %s: %zu bytes given, dims and type %d give %llu", fn, name,
                      data_len, dtype, (unsigned long long)want);
  }
  if (data_len && !data) return api_fail(SSDQ_ERR_INVALID_ARG, "%s: %s: data is NULL", fn, name);
  std::lock_guard<std::mutex> lk(w->mu);
  if (w->tensors.count(name)) return api_fail(SSDQ_ERR_INVALID_ARG, "%s: %s is already resident", fn, name);
  DeviceGuard g(w->device);
  Tensor t;
  t.dtype = dtype;
  t.n_dims = n_dims;
  for (size_t i = 0; i < n_dims; i++) t.dims[i] = dims[i];
  t.bytes = data_len;
  hipError_t e = store_alloc(w, data_len ? data_len : 1, &t.dev);
  if (e != hipSuccess) return api_hip_fail(e, "ssdq_weights_put: device memory");
  if (data_len) {
    e = hipMemcpyAsync(t.dev, data, data_len, hipMemcpyHostToDevice, w->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
    if (e != hipSuccess) return api_hip_fail(e, "ssdq_weights_put: upload");
  }
  w->tensors.emplace(name, t);
  w->total += data_len;
  return api_ok();
}

const void* ssdq_weights_find(const ssdq_weights* w, const char* name, int* dtype, uint64_t* dims,
                              size_t* n_dims, size_t* n_bytes) {
  if (!w || !name) return nullptr;
  std::lock_guard<std::mutex> lk(w->mu);
  const Tensor* t = find(w, name);
  if (!t) return nullptr;
  if (dtype) *dtype = t->dtype;
  if (dims)
    for (size_t i = 0; i < kMaxDims; i++) dims[i] = i < t->n_dims ? t->dims[i] : 1;
  if (n_dims) *n_dims = t->n_dims;
  if (n_bytes) *n_bytes = t->bytes;
  return t->dev;
}

size_t ssdq_weights_count(const ssdq_weights* w) {
  if (!w) return 0;
  std::lock_guard<std::mutex> lk(w->mu);
  return w->tensors.size();
}

size_t ssdq_weights_bytes(const ssdq_weights* w) {
  if (!w) return 0;
  std::lock_guard<std::mutex> lk(w->mu);
  return w->total;
}

int ssdq_weights_device(const ssdq_weights* w) { return w ? w->device : -1; }

}  // extern "C"

// ------------------------------------------------------------ decode layer

namespace {

// Scratch layout: one region per stage output, each 256-byte aligned.
size_t layer_layout(const ssdq_layer_config* c, size_t* off) {
  const size_t q_dim = c->n_head * c->head_dim, kv_dim = c->n_head_kv * c->head_dim;
  const size_t n[SSDQ_LAYER_N_STAGES] = {c->n_embd, q_dim,  kv_dim, kv_dim,    q_dim,         c->n_embd, c->n_embd,
                                         c->n_ff,   c->n_ff, c->n_ff, c->n_embd, 2 * c->n_embd, c->n_embd};
  size_t at = 0;
  for (int i = 0; i < SSDQ_LAYER_N_STAGES; i++) {
    if (off) off[i] = at;
    at += align_up(n[i] * sizeof(float), kAlign);
  }
  return at;
}

bool config_ok(const ssdq_layer_config* c) {
  if (!c || !c->n_embd || !c->n_head || !c->n_head_kv || !c->n_ff) return false;
  // the paged attention kernels' head sizes
  if (c->n_head % c->n_head_kv || (c->head_dim != 64 && c->head_dim != 128 && c->head_dim != 256)) return false;
  const size_t lim = (size_t)INT_MAX / 4;
  return c->n_embd < lim && c->n_ff < lim && c->n_head < lim / 256 && c->n_head_kv <= 65535;
}

// A projection's tensor must have GGUF dims {in, out}.
int check_proj(const Tensor* t, const std::string& name, size_t in, size_t out) {
  if (t->n_dims != 2 || t->dims[0] != in || t->dims[1] != out)
    return api_fail(SSDQ_ERR_INVALID_ARG,
                    "ssdq_decode_layer_dev: %s has dims [%llu, %llu] (%zu dims), the layer needs [%zu, %zu]",
                    name.c_str(), (unsigned long long)t->dims[0], (unsigned long long)(t->n_dims > 1 ? t->dims[1] : 1),
                    t->n_dims, in, out);
  return SSDQ_OK;
}

// A norm weight as f32: the resident bytes when F32, else widened into `tmp`.
int norm_weight(const Tensor* t, const std::string& name, size_t n, float* tmp, hipStream_t s, const float** out) {
  if (t->n_dims != 1 || t->dims[0] != n)
    return api_fail(SSDQ_ERR_INVALID_ARG, "ssdq_decode_layer_dev: %s has %llu elements, the layer needs %zu",
                    name.c_str(), (unsigned long long)t->dims[0], n);
  if (t->dtype == SSDQ_TYPE_F32) {
    *out = (const float*)t->dev;
    return SSDQ_OK;
  }
  if (t->dtype != SSDQ_TYPE_F16 && t->dtype != SSDQ_TYPE_BF16)
    return api_fail(SSDQ_ERR_UNSUPPORTED, "ssdq_decode_layer_dev: %s has type %d (F32, F16 or BF16 expected)",
                    name.c_str(), t->dtype);
  hipError_t e = ssdq::launch_widen(t->dtype, t->dev, n, tmp, s);
  if (e != hipSuccess) return api_hip_fail(e, "ssdq_decode_layer_dev: norm weight");
  *out = tmp;
  return SSDQ_OK;
}

}  // namespace

extern "C" {

size_t ssdq_decode_layer_scratch_bytes(const ssdq_layer_config* cfg, size_t* offsets) {
  if (!config_ok(cfg)) return 0;
  return layer_layout(cfg, offsets);
}

int ssdq_decode_layer_dev(const ssdq_weights* w, uint32_t layer, const ssdq_layer_config* cfg, float* hidden,
                          size_t position, int8_t* k_codes, float* k_scales, int8_t* v_codes, float* v_scales,
                          size_t block_size, const int32_t* block_table, size_t max_blocks_per_seq,
                          const int32_t* slot_mapping, const int32_t* ctx_len, size_t max_ctx, void* scratch,
                          size_t scratch_bytes, ssdq_stream_t stream) {
  const char* fn = "ssdq_decode_layer_dev";
  if (!w || !hidden) return api_fail(SSDQ_ERR_INVALID_ARG, "%s: NULL store or hidden state", fn);
  if (!config_ok(cfg))
    return api_fail(SSDQ_ERR_INVALID_ARG,
                    "%s: bad config (all sizes positive, n_head a multiple of n_head_kv, head_dim 64, 128 or 256)",
                    fn);
  if (position > (size_t)INT_MAX) return api_fail(SSDQ_ERR_INVALID_ARG, "%s: position exceeds 2^31", fn);
  hipStream_t s = (hipStream_t)stream;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != w->device)
    return api_fail(SSDQ_ERR_INVALID_ARG, "%s: the store is on device %d, the current device is %d", fn, w->device,
                    dev);
  const size_t n_embd = cfg->n_embd, n_ff = cfg->n_ff;
  const size_t q_dim = cfg->n_head * cfg->head_dim, kv_dim = cfg->n_head_kv * cfg->head_dim;

  // find_tensor_in_layer (transformer.rs:552-559): "blk.{layer}.{suffix}"
  const std::string pre = "blk." + std::to_string(layer) + ".";
  const Tensor *t_an, *t_q, *t_k, *t_v, *t_o, *t_fn, *t_g, *t_u, *t_d;
  {
    std::lock_guard<std::mutex> lk(w->mu);
    t_an = find(w, pre + "attn_norm.weight");
    t_q = find(w, pre + "attn_q.weight");
    t_k = find(w, pre + "attn_k.weight");
    t_v = find(w, pre + "attn_v.weight");
    t_o = find(w, pre + "attn_output.weight");
    t_fn = find(w, pre + "ffn_norm.weight");
    t_g = find(w, pre + "ffn_gate.weight");
    t_u = find(w, pre + "ffn_up.weight");
    t_d = find(w, pre + "ffn_down.weight");
  }
  const bool attn = t_q && t_k && t_v && t_o;
  const bool ffn = t_g && t_u && t_d;
  // shapes first, so a mismatch launches nothing
  int rc = SSDQ_OK;
  if (attn && ((rc = check_proj(t_q, pre + "attn_q.weight", n_embd, q_dim)) ||
               (rc = check_proj(t_k, pre + "attn_k.weight", n_embd, kv_dim)) ||
               (rc = check_proj(t_v, pre + "attn_v.weight", n_embd, kv_dim)) ||
               (rc = check_proj(t_o, pre + "attn_output.weight", q_dim, n_embd))))
    return rc;
  if (attn && ffn && ((rc = check_proj(t_g, pre + "ffn_gate.weight", n_embd, n_ff)) ||
                      (rc = check_proj(t_u, pre + "ffn_up.weight", n_embd, n_ff)) ||
                      (rc = check_proj(t_d, pre + "ffn_down.weight", n_ff, n_embd))))
    return rc;
  if (attn && (!k_codes || !k_scales || !v_codes || !v_scales || !block_table || !slot_mapping || !ctx_len))
    return api_fail(SSDQ_ERR_INVALID_ARG, "%s: NULL KV pool, block table, slot mapping or context length", fn);
  if (attn && (((uintptr_t)k_codes & 3) || ((uintptr_t)v_codes & 3)))
    return api_fail(SSDQ_ERR_INVALID_ARG, "%s: the code pools must be 4-byte aligned", fn);
  if (attn && (block_size == 0 || max_blocks_per_seq == 0 || max_ctx == 0 ||
               max_ctx > max_blocks_per_seq * block_size || max_ctx > (size_t)INT_MAX ||
               max_blocks_per_seq > (size_t)INT_MAX))
    return api_fail(SSDQ_ERR_INVALID_ARG,
                    "%s: block geometry (block_size, max_blocks_per_seq > 0; 0 < max_ctx <= their product)", fn);

  size_t off[SSDQ_LAYER_N_STAGES];
  const size_t need = layer_layout(cfg, off);
  if (scratch) {
    if (scratch_bytes < need)
      return api_fail(SSDQ_ERR_INVALID_ARG, "%s: scratch of %zu bytes, the layer needs %zu", fn, scratch_bytes, need);
    if ((uintptr_t)scratch % kAlign)
      return api_fail(SSDQ_ERR_INVALID_ARG, "%s: scratch must be 256-byte aligned", fn);
  } else {
    hipError_t e = ssdq::api_workspace(need, s, &scratch, 2);
    if (e != hipSuccess) return api_hip_fail(e, "ssdq_decode_layer_dev: workspace");
  }
  char* base = (char*)scratch;
  float* xn = (float*)(base + off[SSDQ_LAYER_ATTN_IN]);
  float* q = (float*)(base + off[SSDQ_LAYER_Q]);
  float* k = (float*)(base + off[SSDQ_LAYER_K]);
  float* v = (float*)(base + off[SSDQ_LAYER_V]);
  float* att = (float*)(base + off[SSDQ_LAYER_ATTN]);
  float* ao = (float*)(base + off[SSDQ_LAYER_ATTN_OUT]);
  float* fin = (float*)(base + off[SSDQ_LAYER_FFN_IN]);
  float* h = (float*)(base + off[SSDQ_LAYER_FFN_H]);
  float* gate = (float*)(base + off[SSDQ_LAYER_FFN_GATE]);
  float* up = (float*)(base + off[SSDQ_LAYER_FFN_UP]);
  float* fo = (float*)(base + off[SSDQ_LAYER_FFN_OUT]);
  float* nw = (float*)(base + off[SSDQ_LAYER_NORM_W]);
  float* hmid = (float*)(base + off[SSDQ_LAYER_HIDDEN_MID]);
  int worst = SSDQ_OK;
  // keeps the worst status of the steps: a failure ends the layer, the
  // unsupported-type warning (that projection zero-filled) is passed on
  auto take = [&](int r) {
    if (r < 0) {
      worst = r;
      return true;
    }
    if (r > worst) worst = r;
    return false;
  };

  // 1-2. attn_input = rms_norm(hidden, attn_norm) (transformer.rs:319-323),
  // then multi_head_attention_fused_rope's QKV + RoPE (attention.rs:190-198):
  // one launch when the norm folds into the fused QKV kernel's staging of x
  hipError_t e = hipSuccess;
  const float* g_attn = nullptr;
  if (t_an && (rc = norm_weight(t_an, pre + "attn_norm.weight", n_embd, nw, s, &g_attn))) return rc;
  bool qkv_done = false;
  if (g_attn && attn && t_q->dtype == t_k->dtype && t_k->dtype == t_v->dtype) {
    ssdq::MatvecFuse f{};
    f.w0 = (const uint8_t*)t_q->dev;
    f.w1 = (const uint8_t*)t_k->dev;
    f.w2 = (const uint8_t*)t_v->dev;
    f.y0 = q;
    f.y1 = k;
    f.y2 = v;
    f.start1 = (int)q_dim;
    f.start2 = (int)(q_dim + kv_dim);
    f.rope_mask = 3u;
    f.head_dim = (int)cfg->head_dim;
    ssdq::api_rope_table(&f.rope, (int)cfg->head_dim, cfg->rope_theta, (int)position);
    f.norm_w = g_attn;
    f.norm_eps = cfg->norm_eps;
    f.xn_out = xn;
    e = ssdq::launch_matvec_fused(t_q->dtype, f, (int)(q_dim + 2 * kv_dim), hidden, n_embd, s, &qkv_done);
    if (e != hipSuccess) return api_hip_fail(e, "ssdq_decode_layer_dev: norm + QKV");
  }
  if (!qkv_done) {
    if (g_attn)
      e = ssdq::launch_rmsnorm(hidden, nullptr, g_attn, cfg->norm_eps, nullptr, xn, (int)n_embd, s);
    else
      e = hipMemcpyAsync(xn, hidden, n_embd * sizeof(float), hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess) return api_hip_fail(e, "ssdq_decode_layer_dev: attention norm");
  }
  // without all four attention tensors the reference skips the rest of the
  // layer (transformer.rs:326-331)
  if (!attn) {
    api_ok();
    return SSDQ_OK;
  }

  // 2-5. multi_head_attention_fused_rope (attention.rs:172-240) over the paged
  // INT8 cache: QKV + RoPE (unless done above), append, attention, output
  // projection
  if (!qkv_done && take(ssdq_qkv_rope_dev(t_q->dtype, t_q->dev, t_k->dtype, t_k->dev, t_v->dtype, t_v->dev, xn, q,
                                          k, v, q_dim, kv_dim, n_embd, cfg->head_dim, position, cfg->rope_theta,
                                          stream)))
    return worst;
  // append + attention: one launch (and the combine) on the matrix cores
  if (take(ssdq::api_paged_attention_append(q, k_codes, k_scales, v_codes, v_scales, block_table, ctx_len, k, v,
                                      slot_mapping, att, 1, cfg->n_head, cfg->n_head_kv, cfg->head_dim, block_size,
                                      max_blocks_per_seq, max_ctx, s)))
    return worst;
  {
    const ssdq::FreshX fresh;  // att was just written by the attention combine
    if (take(ssdq_matvec_dev(t_o->dtype, t_o->dev, att, ao, n_embd, q_dim, 1, stream))) return worst;
  }

  // 6. hidden += attn_output, ffn_input = rms_norm(hidden, ffn_norm)
  // (fused_post_attn_norm_f32, transformer.rs:346-359); without ffn_norm the
  // FFN reads the updated hidden state itself (transformer.rs:381-386).
  // 7-8. dense SwiGLU FFN (run_ffn_or_moe_gpu, transformer.rs:470-481 ->
  // feed_forward.rs:16-45) and its residual add (transformer.rs:369-373);
  // absent FFN tensors leave hidden as hidden + attn_output.
  const float* g_ffn = nullptr;
  if (t_fn && (rc = norm_weight(t_fn, pre + "ffn_norm.weight", n_embd, nw + n_embd, s, &g_ffn))) return rc;
  // The norm folds into the fused SwiGLU kernel's staging: every workgroup
  // reads hidden and attn_output, so the updated hidden state goes to hmid
  // (not in place) and the down projection writes hidden = hmid + W_down h.
  bool ffn_done = false;
  if (g_ffn && ffn && t_g->dtype == t_u->dtype) {
    ssdq::MatvecFuse f{};
    f.w0 = (const uint8_t*)t_g->dev;
    f.w1 = (const uint8_t*)t_u->dev;
    f.y0 = h;
    f.start1 = f.start2 = INT_MAX;
    f.swiglu = 1;
    f.head_dim = 2;
    f.norm_w = g_ffn;
    f.norm_res = ao;
    f.norm_eps = cfg->norm_eps;
    f.hidden_out = hmid;
    f.xn_out = fin;
    e = ssdq::launch_matvec_fused(t_g->dtype, f, (int)(2 * n_ff), hidden, n_embd, s, &ffn_done);
    if (e != hipSuccess) return api_hip_fail(e, "ssdq_decode_layer_dev: norm + SwiGLU");
  }
  const float* ffn_in = fin;
  const float* h_res = hidden;  // the hidden state the FFN output is added to
  if (ffn_done) {
    h_res = hmid;
  } else {
    if (g_ffn) {
      e = ssdq::launch_rmsnorm(hidden, ao, g_ffn, cfg->norm_eps, hidden, fin, (int)n_embd, s);
    } else {
      e = ssdq::launch_residual_add(hidden, ao, (int)n_embd, s);
      ffn_in = hidden;
    }
    if (e != hipSuccess) return api_hip_fail(e, "ssdq_decode_layer_dev: residual norm");
    if (ffn) {
      if (t_g->dtype == t_u->dtype) {
        if (take(ssdq_swiglu_dev(t_g->dtype, t_g->dev, t_u->dev, ffn_in, h, n_ff, n_embd, stream))) return worst;
      } else {
        // gate and up of different types: two projections, then the product
        if (take(ssdq_matvec_dev(t_g->dtype, t_g->dev, ffn_in, gate, n_ff, n_embd, 1, stream))) return worst;
        if (take(ssdq_matvec_dev(t_u->dtype, t_u->dev, ffn_in, up, n_ff, n_embd, 1, stream))) return worst;
        if ((e = ssdq::launch_swiglu(gate, up, h, (int)n_ff, s)) != hipSuccess)
          return api_hip_fail(e, "ssdq_decode_layer_dev: swiglu");
      }
    }
  }
  if (ffn) {
    const int dd = t_d->dtype;
    if (dd == SSDQ_TYPE_Q4_0 || dd == SSDQ_TYPE_Q8_0 || dd == SSDQ_TYPE_Q4_K || dd == SSDQ_TYPE_Q6_K) {
      // hidden = h_res + W_down h inside the K-sliced matvec's slice reduction
      // (fo still receives W_down h)
      const size_t wsb = ssdq::matvec_workspace_bytes(dd, t_d->dev, h, n_embd, n_ff, 1);
      void* ws = nullptr;
      if (wsb && (e = ssdq::api_workspace(wsb, s, &ws, 0)) != hipSuccess)
        return api_hip_fail(e, "ssdq_decode_layer_dev: workspace");
      e = ssdq::launch_matvec_acc(dd, (const uint8_t*)t_d->dev, h, hidden, fo, n_embd, n_ff, s, ws, wsb, h_res);
      if (e != hipSuccess) return api_hip_fail(e, "ssdq_decode_layer_dev: down projection");
    } else {
      if (take(ssdq_matvec_dev(dd, t_d->dev, h, fo, n_embd, n_ff, 1, stream))) return worst;
      if ((e = ssdq::launch_add(hidden, h_res, fo, (int)n_embd, s)) != hipSuccess)
        return api_hip_fail(e, "ssdq_decode_layer_dev: residual");
    }
  }
  if (worst == SSDQ_OK) api_ok();
  return worst;
}

}  // extern "C"
