// extern "C" boundary of libssdq.so: argument checking, status codes,
// per-device workspaces and the synchronous host-pointer twins.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <tuple>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/ssdq.h"
#include "launch.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
    return fail(SSDQ_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
  return fail(SSDQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int ok() {
  g_err[0] = '\0';
  return SSDQ_OK;
}

bool supported_quant(int dtype) {
  return dtype == SSDQ_TYPE_Q4_0 || dtype == SSDQ_TYPE_Q8_0 || dtype == SSDQ_TYPE_Q4_K ||
         dtype == SSDQ_TYPE_Q6_K;
}

// matvec_quantized_cpu's match arms (compute.rs:655-671)
bool supported_matvec(int dtype) { return supported_quant(dtype) || ssdq::matvec_ext_type(dtype); }

bool float_type(int dtype) {
  return dtype == SSDQ_TYPE_F32 || dtype == SSDQ_TYPE_F16 || dtype == SSDQ_TYPE_BF16;
}

bool fits_int(size_t v) { return v <= (size_t)INT_MAX; }

// Grow-only device buffers keyed by (device, stream), so calls on different
// streams never share scratch memory.
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
  bool captured = false;  // handed out while its stream was being captured into a graph
};
// slot 0: the kernels' own scratch; slot 1: intermediates of the unfused
// decode-layer paths, which call kernels that use slot 0; slot 2: the
// activations of ssdq_decode_layer_dev, which calls entry points that use
// slots 0 and 1.
std::mutex g_ws_mu;
std::map<std::tuple<int, void*, int>, Workspace> g_ws;
// Buffers replaced by a larger one that a HIP graph captured on their stream
// may still hold: never freed on growth, only by ssdq_release_workspaces()
// (device, pointer).
std::vector<std::pair<int, void*>> g_ws_retired;

// Growth is geometric (at least twice the old size, in 2 MiB steps), so a
// caller whose request creeps up (the decode attention's split count as the
// context grows) replaces its buffer O(log n) times.  A replaced buffer that
// was never handed out during a graph capture is freed after the stream
// drains the work already queued with it; one that was is retired.
hipError_t workspace_get(size_t bytes, hipStream_t stream, void** out, int slot = 0) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(g_ws_mu);
  Workspace& w = g_ws[std::make_tuple(dev, (void*)stream, slot)];
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  const bool capturing =
      stream && hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
  if (w.bytes < bytes) {
    // No allocation while the stream is being captured into a graph (it would
    // invalidate the capture): run the call once on this stream beforehand,
    // or reserve with ssdq_reserve_workspace().
    if (capturing) return hipErrorStreamCaptureUnsupported;
    constexpr size_t kStep = (size_t)2 << 20;
    size_t want = bytes > 2 * w.bytes ? bytes : 2 * w.bytes;
    want = (want + kStep - 1) / kStep * kStep;
    void* p = nullptr;
    e = hipMalloc(&p, want);
    if (e != hipSuccess) {
      want = bytes;  // the geometric size does not fit: the exact one may
      e = hipMalloc(&p, want);
      if (e != hipSuccess) return e;
    }
    if (w.ptr) {
      if (w.captured) {
        g_ws_retired.emplace_back(dev, w.ptr);
      } else {
        // work already queued on the stream may still use the old buffer
        e = hipStreamSynchronize(stream);
        if (e == hipSuccess) e = hipFree(w.ptr);
        if (e != hipSuccess) {
          (void)hipFree(p);
          return e;
        }
      }
    }
    w.ptr = p;
    w.bytes = want;
    w.captured = false;
  }
  if (capturing) w.captured = true;
  *out = w.ptr;
  return hipSuccess;
}

}  // namespace

namespace ssdq {

int api_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}
int api_hip_fail(hipError_t e, const char* what) { return hip_fail(e, what); }
int api_ok() { return ok(); }
void api_rope_table(RopeTable* r, int head_dim, float theta, int position) {
  for (int i = 0; i < 128; i++) {
    const float freq = i < head_dim / 2 ? 1.0f / powf(theta, 2.0f * (float)i / (float)head_dim) : 0.0f;
    const float ang = (float)position * freq;
    r->sn[i] = (float)sin((double)ang);
    r->cs[i] = (float)cos((double)ang);
  }
}
hipError_t api_workspace(size_t bytes, hipStream_t stream, void** out, int slot) {
  return workspace_get(bytes, stream, out, slot);
}

int device_cu_count() {
  static std::mutex mu;
  static std::map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  cache[dev] = cus;
  return cus;
}

}  // namespace ssdq

struct ssdq_ctx {
  std::mutex mu;  // host twins on one context run one at a time
  int device = 0;
  hipStream_t stream = nullptr;
  void* buf[4] = {nullptr, nullptr, nullptr, nullptr};
  size_t cap[4] = {0, 0, 0, 0};
};

namespace {

hipError_t ctx_buf(ssdq_ctx* c, int i, size_t bytes, void** out) {
  if (c->cap[i] < bytes) {
    if (c->buf[i]) (void)hipFree(c->buf[i]);
    c->buf[i] = nullptr;
    c->cap[i] = 0;
    hipError_t e = hipMalloc(&c->buf[i], bytes ? bytes : 4);
    if (e != hipSuccess) return e;
    c->cap[i] = bytes;
  }
  *out = c->buf[i];
  return hipSuccess;
}

}  // namespace

extern "C" {

int ssdq_abi_version(void) { return SSDQ_ABI_VERSION; }

const char* ssdq_last_error(void) { return g_err; }

size_t ssdq_block_size(int dtype) {
  switch (dtype) {
    case SSDQ_TYPE_F32: case SSDQ_TYPE_F16: case SSDQ_TYPE_BF16: return 1;
    case SSDQ_TYPE_Q4_0: case SSDQ_TYPE_Q8_0: case SSDQ_TYPE_IQ4_NL: return 32;
    case SSDQ_TYPE_Q2_K: case SSDQ_TYPE_Q3_K: case SSDQ_TYPE_Q4_K: case SSDQ_TYPE_Q5_K:
    case SSDQ_TYPE_Q6_K: case SSDQ_TYPE_Q8_K: case SSDQ_TYPE_IQ4_XS: case SSDQ_TYPE_IQ2_XXS:
    case SSDQ_TYPE_IQ2_XS: case SSDQ_TYPE_IQ3_XXS: case SSDQ_TYPE_IQ3_S: return 256;
    default: return 0;
  }
}

size_t ssdq_type_size(int dtype) {
  switch (dtype) {
    case SSDQ_TYPE_F32: return 4;
    case SSDQ_TYPE_F16: case SSDQ_TYPE_BF16: return 2;
    case SSDQ_TYPE_Q4_0: return 18;
    case SSDQ_TYPE_Q8_0: return 34;
    case SSDQ_TYPE_Q4_K: return 144;
    case SSDQ_TYPE_Q6_K: return 210;
    case SSDQ_TYPE_Q2_K: return 84;
    case SSDQ_TYPE_Q3_K: return 110;  // the matvec's block; gguf.rs:127 computes 174
    case SSDQ_TYPE_Q5_K: return 176;
    case SSDQ_TYPE_Q8_K: return 292;
    case SSDQ_TYPE_IQ4_NL: return 18;
    case SSDQ_TYPE_IQ4_XS: return 148;
    case SSDQ_TYPE_IQ2_XXS: return 66;
    case SSDQ_TYPE_IQ2_XS: return 74;
    case SSDQ_TYPE_IQ3_XXS: return 98;
    case SSDQ_TYPE_IQ3_S: return 110;
    default: return 0;
  }
}

size_t ssdq_row_bytes(int dtype, size_t in_dim) {
  const size_t bs = ssdq_block_size(dtype);
  return bs ? (in_dim / bs) * ssdq_type_size(dtype) : 0;
}

int ssdq_ctx_create(int device, ssdq_ctx** out) {
  if (!out) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_ctx_create: out is NULL");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
    return fail(SSDQ_ERR_NO_DEVICE, "ssdq_ctx_create: no HIP device");
  if (device < 0) {
    if (hipGetDevice(&device) != hipSuccess) device = 0;
  }
  if (device >= n) return fail(SSDQ_ERR_NO_DEVICE, "ssdq_ctx_create: device %d of %d", device, n);
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, "ssdq_ctx_create: hipSetDevice");
  ssdq_ctx* c = new (std::nothrow) ssdq_ctx();
  if (!c) return fail(SSDQ_ERR_OUT_OF_MEMORY, "ssdq_ctx_create: host allocation");
  c->device = device;
  e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(e, "ssdq_ctx_create: hipStreamCreate");
  }
  *out = c;
  return ok();
}

void ssdq_ctx_destroy(ssdq_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  for (int i = 0; i < 4; i++)
    if (c->buf[i]) (void)hipFree(c->buf[i]);
  (void)hipStreamDestroy(c->stream);
  delete c;
}

int ssdq_ctx_device(const ssdq_ctx* c) { return c ? c->device : -1; }

int ssdq_reserve_workspace(size_t bytes, ssdq_stream_t stream) {
  void* p = nullptr;
  hipError_t e = workspace_get(bytes ? bytes : 1, (hipStream_t)stream, &p);
  if (e != hipSuccess) return hip_fail(e, "ssdq_reserve_workspace");
  return ok();
}

int ssdq_release_workspaces(void) {
  std::vector<std::pair<int, void*>> retired;
  {
    std::lock_guard<std::mutex> lk(g_ws_mu);
    retired.swap(g_ws_retired);
  }
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) cur = -1;
  for (auto& r : retired) {
    hipError_t e = hipSetDevice(r.first);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipFree(r.second);
    if (e != hipSuccess) {
      if (cur >= 0) (void)hipSetDevice(cur);
      return hip_fail(e, "ssdq_release_workspaces");
    }
  }
  if (cur >= 0) (void)hipSetDevice(cur);
  return ok();
}

int ssdq_dequant_dev(int dtype, const void* w, size_t n_elements, float* out,
                     ssdq_stream_t stream) {
  if (n_elements == 0) return ok();
  if (!out) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_dequant_dev: out is NULL");
  hipStream_t s = (hipStream_t)stream;
  if (float_type(dtype)) {
    if (!w) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_dequant_dev: w is NULL");
    if ((uintptr_t)w % ssdq_type_size(dtype) || ((uintptr_t)out & 3))
      return fail(SSDQ_ERR_INVALID_ARG, "ssdq_dequant_dev: w / out not element aligned");
    hipError_t e = ssdq::launch_widen(dtype, w, n_elements, out, s);
    if (e != hipSuccess) return hip_fail(e, "ssdq_dequant_dev: widen");
    return ok();
  }
  if (!supported_quant(dtype)) {
    hipError_t e = ssdq::launch_fill_zero(out, n_elements, s);
    if (e != hipSuccess) return hip_fail(e, "ssdq_dequant_dev: fill");
    fail(SSDQ_WARN_UNSUPPORTED_ZEROED, "ssdq_dequant_dev: dtype %d unsupported, zero-filled", dtype);
    return SSDQ_WARN_UNSUPPORTED_ZEROED;
  }
  if (!w) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_dequant_dev: w is NULL");
  const size_t bs = ssdq_block_size(dtype);
  const size_t n_blocks = n_elements / bs;
  hipError_t e = ssdq::launch_dequant(dtype, (const uint8_t*)w, n_blocks, out, s);
  if (e != hipSuccess) return hip_fail(e, "ssdq_dequant_dev");
  if (n_blocks * bs < n_elements) {
    e = ssdq::launch_fill_zero(out + n_blocks * bs, n_elements - n_blocks * bs, s);
    if (e != hipSuccess) return hip_fail(e, "ssdq_dequant_dev: tail");
  }
  return ok();
}

static int matvec_common(int dtype, const void* w, const float* x, float* y, size_t out_dim,
                         size_t in_dim, size_t batch, ssdq_stream_t stream, bool generic) {
  const char* fn = generic ? "ssdq_matvec_generic_dev" : "ssdq_matvec_dev";
  if (out_dim == 0 || batch == 0) return ok();
  if (!y) return fail(SSDQ_ERR_INVALID_ARG, "%s: y is NULL", fn);
  if (!fits_int(out_dim) || !fits_int(in_dim) || !fits_int(batch) ||
      !fits_int(out_dim * batch) || !fits_int(in_dim * batch))
    return fail(SSDQ_ERR_INVALID_ARG, "%s: dimensions exceed 2^31", fn);
  hipStream_t s = (hipStream_t)stream;
  if (!supported_matvec(dtype)) {
    hipError_t e = ssdq::launch_fill_zero(y, out_dim * batch, s);
    if (e != hipSuccess) return hip_fail(e, fn);
    fail(SSDQ_WARN_UNSUPPORTED_ZEROED, "%s: dtype %d unsupported, zero-filled", fn, dtype);
    return SSDQ_WARN_UNSUPPORTED_ZEROED;
  }
  const size_t keff = (in_dim / ssdq_block_size(dtype)) * ssdq_block_size(dtype);
  if (keff > 0 && (!w || !x)) return fail(SSDQ_ERR_INVALID_ARG, "%s: w or x is NULL", fn);
  if (((uintptr_t)x & 3) || ((uintptr_t)y & 3))
    return fail(SSDQ_ERR_INVALID_ARG, "%s: x and y must be 4-byte aligned", fn);
  hipError_t e = hipSuccess;
  if (ssdq::matvec_ext_type(dtype)) {
    bool used = false;
    // batch 1 on the digit-plane kernel, where the type has one.  (Batches stay
    // on mv_ext: on synthetic rows that cancel to 1e-5 of their terms, the
    // factored S*sum(q x) - M*sum(x) of mv_bn strayed 4e-4 from the exact sum
    // on one output, past the tolerance the float path met.)
    if (!generic && batch == 1) {
      const size_t wsb = ssdq::matvec_digit_ext_workspace_bytes(dtype, w, x, out_dim, in_dim, batch);
      void* ws = nullptr;
      if (wsb && (e = workspace_get(wsb, s, &ws)) != hipSuccess) return hip_fail(e, "ssdq_matvec_dev: workspace");
      e = ssdq::launch_matvec_digit_ext(dtype, (const uint8_t*)w, x, y, out_dim, in_dim, batch, s, ws, wsb, &used);
      if (e != hipSuccess) return hip_fail(e, fn);
    }
    if (!used) e = ssdq::launch_matvec_ext(dtype, (const uint8_t*)w, x, y, out_dim, in_dim, batch, s, generic);
  } else if (generic) {
    e = ssdq::launch_matvec_generic(dtype, (const uint8_t*)w, x, y, out_dim, in_dim, batch, s);
  } else {
    const size_t wsb = ssdq::matvec_workspace_bytes(dtype, w, x, out_dim, in_dim, batch);
    void* ws = nullptr;
    if (wsb && (e = workspace_get(wsb, s, &ws)) != hipSuccess) return hip_fail(e, "ssdq_matvec_dev: workspace");
    e = ssdq::launch_matvec(dtype, (const uint8_t*)w, x, y, out_dim, in_dim, batch, s, ws, wsb);
  }
  if (e != hipSuccess) return hip_fail(e, fn);
  return ok();
}

int ssdq_matvec_dev(int dtype, const void* w, const float* x, float* y, size_t out_dim,
                    size_t in_dim, size_t batch, ssdq_stream_t stream) {
  return matvec_common(dtype, w, x, y, out_dim, in_dim, batch, stream, false);
}

int ssdq_matvec_generic_dev(int dtype, const void* w, const float* x, float* y, size_t out_dim,
                            size_t in_dim, size_t batch, ssdq_stream_t stream) {
  return matvec_common(dtype, w, x, y, out_dim, in_dim, batch, stream, true);
}

int ssdq_matvec_quantized(ssdq_ctx* c, const uint8_t* w_raw, size_t w_len, const float* x,
                          size_t x_len, size_t out_dim, size_t in_dim, int dtype, float* y) {
  if (!c) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_matvec_quantized: ctx is NULL");
  if (out_dim == 0) return ok();
  if (!y) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_matvec_quantized: y is NULL");
  if (!supported_matvec(dtype)) {
    memset(y, 0, out_dim * sizeof(float));
    fail(SSDQ_WARN_UNSUPPORTED_ZEROED, "ssdq_matvec_quantized: dtype %d unsupported, zeros", dtype);
    return SSDQ_WARN_UNSUPPORTED_ZEROED;
  }
  const size_t rb = ssdq_row_bytes(dtype, in_dim);
  const size_t keff = (in_dim / ssdq_block_size(dtype)) * ssdq_block_size(dtype);
  // The reference indexes w[row*row_bytes + ...] and x[..keff) and panics when
  // they are short; this reports an error instead.
  if (w_len < out_dim * rb)
    return fail(SSDQ_ERR_INVALID_ARG, "ssdq_matvec_quantized: w has %zu bytes, need %zu", w_len,
                out_dim * rb);
  if (x_len < keff)
    return fail(SSDQ_ERR_INVALID_ARG, "ssdq_matvec_quantized: x has %zu floats, need %zu", x_len, keff);
  if ((rb && !w_raw) || (keff && !x)) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_matvec_quantized: NULL input");
  std::lock_guard<std::mutex> lk(c->mu);
  hipError_t e = hipSetDevice(c->device);
  if (e != hipSuccess) return hip_fail(e, "ssdq_matvec_quantized: hipSetDevice");
  void *dw, *dx, *dy;
  if ((e = ctx_buf(c, 0, out_dim * rb, &dw)) != hipSuccess ||
      (e = ctx_buf(c, 1, (keff ? keff : 1) * sizeof(float), &dx)) != hipSuccess ||
      (e = ctx_buf(c, 2, out_dim * sizeof(float), &dy)) != hipSuccess)
    return hip_fail(e, "ssdq_matvec_quantized: staging allocation");
  if (rb && (e = hipMemcpyAsync(dw, w_raw, out_dim * rb, hipMemcpyHostToDevice, c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_matvec_quantized: copy w");
  if (keff && (e = hipMemcpyAsync(dx, x, keff * sizeof(float), hipMemcpyHostToDevice, c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_matvec_quantized: copy x");
  int rc = ssdq_matvec_dev(dtype, dw, (const float*)dx, (float*)dy, out_dim, keff ? keff : in_dim,
                           1, c->stream);
  if (rc < 0) return rc;
  if ((e = hipMemcpyAsync(y, dy, out_dim * sizeof(float), hipMemcpyDeviceToHost, c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_matvec_quantized: copy y");
  if ((e = hipStreamSynchronize(c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_matvec_quantized: sync");
  return ok();
}

/* -------------------------------------------- INT8 KV swap slots */

size_t ssdq_kv_slot_bytes(size_t block_size, size_t kv_dim) { return ssdq::kv_slot_bytes(block_size, kv_dim); }

static int swap_args_ok(const char* fn, const void* kc, const void* ks, const void* vc, const void* vs,
                        const void* ids, const void* slots, size_t n_blocks, size_t bs, size_t kv, size_t n_pool) {
  if (!kc || !ks || !vc || !vs || !ids || !slots) return fail(SSDQ_ERR_INVALID_ARG, "%s: NULL pointer", fn);
  if (bs == 0 || kv == 0 || kv % 4) return fail(SSDQ_ERR_INVALID_ARG, "%s: kv_dim must be a positive multiple of 4", fn);
  if (((uintptr_t)kc | (uintptr_t)vc | (uintptr_t)ks | (uintptr_t)vs | (uintptr_t)slots) & 3)
    return fail(SSDQ_ERR_INVALID_ARG, "%s: pools and slots must be 4-byte aligned", fn);
  if (n_blocks > 65535 || !fits_int(bs * kv) || n_pool > (size_t)LONG_MAX / (bs * kv))
    return fail(SSDQ_ERR_INVALID_ARG, "%s: too many blocks per call (at most 65535) or blocks too large", fn);
  return SSDQ_OK;
}

int ssdq_kv_swap_out_dev(const int8_t* k_codes, const float* k_scales, const int8_t* v_codes,
                         const float* v_scales, const int32_t* block_ids, const uint32_t* num_filled,
                         size_t n_blocks, size_t block_size, size_t kv_dim, size_t n_pool_blocks, void* slots,
                         ssdq_stream_t stream) {
  if (n_blocks == 0) return ok();
  int rc = swap_args_ok("ssdq_kv_swap_out_dev", k_codes, k_scales, v_codes, v_scales, block_ids, slots, n_blocks,
                        block_size, kv_dim, n_pool_blocks);
  if (rc) return rc;
  hipError_t e = ssdq::launch_kv_swap_out(k_codes, k_scales, v_codes, v_scales, block_ids, num_filled, n_blocks,
                                          block_size, kv_dim, n_pool_blocks, slots, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "ssdq_kv_swap_out_dev");
  return ok();
}

int ssdq_kv_swap_in_dev(const void* slots, const int32_t* block_ids, size_t n_blocks, size_t block_size,
                        size_t kv_dim, size_t n_pool_blocks, int8_t* k_codes, float* k_scales, int8_t* v_codes,
                        float* v_scales, uint32_t* num_filled, ssdq_stream_t stream) {
  if (n_blocks == 0) return ok();
  int rc = swap_args_ok("ssdq_kv_swap_in_dev", k_codes, k_scales, v_codes, v_scales, block_ids, slots, n_blocks,
                        block_size, kv_dim, n_pool_blocks);
  if (rc) return rc;
  hipError_t e = ssdq::launch_kv_swap_in(slots, block_ids, n_blocks, block_size, kv_dim, n_pool_blocks, k_codes,
                                         k_scales, v_codes, v_scales, num_filled, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "ssdq_kv_swap_in_dev");
  return ok();
}

/* ------------------------------------------------- decode-layer ops */

namespace {
// 1 / theta^(2i/head_dim) with the C library's powf, the call the reference's
// rope_f32_multi_head makes (compute.rs:494)
void rope_table(ssdq::RopeTable* r, int head_dim, float theta, int position) {
  ssdq::api_rope_table(r, head_dim, theta, position);
}
}  // namespace

int ssdq_rmsnorm_dev(const float* x, const float* residual, const float* weight, float eps,
                     float* hidden_out, float* out, size_t n, ssdq_stream_t stream) {
  if (n == 0) return ok();
  if (!x || !weight || !out) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_rmsnorm_dev: NULL pointer");
  if (!fits_int(n)) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_rmsnorm_dev: n exceeds 2^31");
  hipError_t e = ssdq::launch_rmsnorm(x, residual, weight, eps, hidden_out, out, (int)n, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "ssdq_rmsnorm_dev");
  return ok();
}

int ssdq_qkv_rope_dev(int dtype_q, const void* wq, int dtype_k, const void* wk, int dtype_v,
                      const void* wv, const float* x, float* q, float* k, float* v, size_t q_dim,
                      size_t kv_dim, size_t n_embd, size_t head_dim, size_t position, float theta_base,
                      ssdq_stream_t stream) {
  const char* fn = "ssdq_qkv_rope_dev";
  if (!wq || !wk || !wv || !x || !q || !k || !v) return fail(SSDQ_ERR_INVALID_ARG, "%s: NULL pointer", fn);
  if (q_dim == 0 || kv_dim == 0 || (q_dim & 1) || (kv_dim & 1) || !fits_int(q_dim + 2 * kv_dim) ||
      !fits_int(n_embd) || !fits_int(position))
    return fail(SSDQ_ERR_INVALID_ARG, "%s: q_dim / kv_dim must be positive and even", fn);
  if (head_dim && ((head_dim & 1) || head_dim > 256 || q_dim % head_dim || kv_dim % head_dim))
    return fail(SSDQ_ERR_INVALID_ARG, "%s: head_dim must be even, at most 256 and divide q_dim and kv_dim", fn);
  hipStream_t s = (hipStream_t)stream;
  ssdq::RopeTable rope;
  rope_table(&rope, head_dim ? (int)head_dim : 2, theta_base, (int)position);
  if (dtype_q == dtype_k && dtype_k == dtype_v && supported_quant(dtype_q)) {
    ssdq::MatvecFuse f{};
    f.w0 = (const uint8_t*)wq; f.w1 = (const uint8_t*)wk; f.w2 = (const uint8_t*)wv;
    f.y0 = q; f.y1 = k; f.y2 = v;
    f.start1 = (int)q_dim;
    f.start2 = (int)(q_dim + kv_dim);
    f.rope_mask = head_dim ? 3u : 0u;
    f.head_dim = head_dim ? (int)head_dim : 2;
    f.rope = rope;
    bool used = false;
    hipError_t e = ssdq::launch_matvec_fused(dtype_q, f, (int)(q_dim + 2 * kv_dim), x, n_embd, s, &used);
    if (e != hipSuccess) return hip_fail(e, fn);
    if (used) return ok();
  }
  // unfused: three projections, then the rotation of q and k
  int worst = SSDQ_OK;
  const int dts[3] = {dtype_q, dtype_k, dtype_v};
  const void* ws[3] = {wq, wk, wv};
  float* ys[3] = {q, k, v};
  const size_t rows[3] = {q_dim, kv_dim, kv_dim};
  for (int i = 0; i < 3; i++) {
    int rc = ssdq_matvec_dev(dts[i], ws[i], x, ys[i], rows[i], n_embd, 1, stream);
    if (rc < 0) return rc;
    if (rc > worst) worst = rc;
  }
  if (head_dim) {
    hipError_t e = ssdq::launch_rope(q, (int)q_dim, (int)head_dim, rope, s);
    if (e == hipSuccess) e = ssdq::launch_rope(k, (int)kv_dim, (int)head_dim, rope, s);
    if (e != hipSuccess) return hip_fail(e, fn);
  }
  if (worst != SSDQ_OK) {
    fail(worst, "%s: a projection dtype is unsupported, its output zero-filled", fn);
    return worst;
  }
  return ok();
}

int ssdq_swiglu_dev(int dtype, const void* w_gate, const void* w_up, const float* x, float* h,
                    size_t n_ff, size_t n_embd, ssdq_stream_t stream) {
  const char* fn = "ssdq_swiglu_dev";
  if (n_ff == 0) return ok();
  if (!w_gate || !w_up || !x || !h) return fail(SSDQ_ERR_INVALID_ARG, "%s: NULL pointer", fn);
  if (!fits_int(2 * n_ff) || !fits_int(n_embd)) return fail(SSDQ_ERR_INVALID_ARG, "%s: dimensions exceed 2^31", fn);
  hipStream_t s = (hipStream_t)stream;
  if (supported_quant(dtype)) {
    ssdq::MatvecFuse f{};
    f.w0 = (const uint8_t*)w_gate; f.w1 = (const uint8_t*)w_up;
    f.y0 = h;
    f.start1 = f.start2 = INT_MAX;
    f.swiglu = 1;
    f.head_dim = 2;
    bool used = false;
    hipError_t e = ssdq::launch_matvec_fused(dtype, f, (int)(2 * n_ff), x, n_embd, s, &used);
    if (e != hipSuccess) return hip_fail(e, fn);
    if (used) return ok();
  }
  void* tmp = nullptr;
  hipError_t e = workspace_get(2 * n_ff * sizeof(float), s, &tmp, 1);
  if (e != hipSuccess) return hip_fail(e, "ssdq_swiglu_dev: workspace");
  float* g = (float*)tmp;
  float* u = g + n_ff;
  int rc = ssdq_matvec_dev(dtype, w_gate, x, g, n_ff, n_embd, 1, stream);
  if (rc < 0) return rc;
  rc = ssdq_matvec_dev(dtype, w_up, x, u, n_ff, n_embd, 1, stream);
  if (rc < 0) return rc;
  e = ssdq::launch_swiglu(g, u, h, (int)n_ff, s);
  if (e != hipSuccess) return hip_fail(e, fn);
  if (rc != SSDQ_OK) {
    fail(rc, "%s: dtype %d unsupported, zeros", fn, dtype);
    return rc;
  }
  return ok();
}

int ssdq_rmsnorm_matvec_dev(int dtype, const void* w, const float* x, const float* norm_weight, float eps,
                            float* y, size_t out_dim, size_t n_embd, ssdq_stream_t stream) {
  const char* fn = "ssdq_rmsnorm_matvec_dev";
  if (out_dim == 0) return ok();
  if (!w || !x || !norm_weight || !y) return fail(SSDQ_ERR_INVALID_ARG, "%s: NULL pointer", fn);
  if (!fits_int(out_dim) || !fits_int(n_embd)) return fail(SSDQ_ERR_INVALID_ARG, "%s: dimensions exceed 2^31", fn);
  hipStream_t s = (hipStream_t)stream;
  // A separate norm kernel and the plain matvec: folding the norm into the
  // matvec's staging of x measured slower (the norm weights queue ahead of
  // every workgroup's first weight rows).
  void* tmp = nullptr;
  hipError_t e = workspace_get((n_embd ? n_embd : 1) * sizeof(float), s, &tmp, 1);
  if (e != hipSuccess) return hip_fail(e, "ssdq_rmsnorm_matvec_dev: workspace");
  if (n_embd) {
    e = ssdq::launch_rmsnorm(x, nullptr, norm_weight, eps, nullptr, (float*)tmp, (int)n_embd, s);
    if (e != hipSuccess) return hip_fail(e, fn);
  }
  return ssdq_matvec_dev(dtype, w, (const float*)tmp, y, out_dim, n_embd, 1, stream);
}

namespace {
int gemm_multi(const char* fn, const void* const* w, const size_t* n, size_t count, const uint16_t* x,
               float* const* y, size_t M, size_t K, ssdq_stream_t stream) {
  if (count < 1 || count > 3) return fail(SSDQ_ERR_INVALID_ARG, "%s: count must be 1, 2 or 3", fn);
  if (!w || !n || !y || !x) return fail(SSDQ_ERR_INVALID_ARG, "%s: NULL pointer", fn);
  size_t N = 0;
  for (size_t i = 0; i < count; i++) {
    if (!w[i] || !y[i]) return fail(SSDQ_ERR_INVALID_ARG, "%s: NULL pointer", fn);
    if (n[i] == 0) return fail(SSDQ_ERR_INVALID_ARG, "%s: every matrix needs at least one row", fn);
    N += n[i];
  }
  if (M == 0) return ok();
  if (K == 0 || K % 256) return fail(SSDQ_ERR_INVALID_ARG, "%s: K must be a positive multiple of 256", fn);
  if (!fits_int(M) || !fits_int(N) || !fits_int(K) || !fits_int(M * K) || !fits_int(M * N))
    return fail(SSDQ_ERR_INVALID_ARG, "%s: dimensions exceed 2^31", fn);
  hipStream_t s = (hipStream_t)stream;
  const uint8_t* const* wb = reinterpret_cast<const uint8_t* const*>(w);
  const size_t wsb = ssdq::gemm_q4k_workspace_bytes(w, n, (int)count, x, M, K);
  void* ws = nullptr;
  hipError_t e = hipSuccess;
  if (wsb && (e = workspace_get(wsb, s, &ws)) != hipSuccess) return hip_fail(e, "ssdq_gemm_q4k_bf16 workspace");
  e = ssdq::launch_gemm_q4k(wb, n, (int)count, x, y, M, K, ws, wsb, s);
  if (e != hipSuccess) return hip_fail(e, fn);
  return ok();
}
}  // namespace

int ssdq_gemm_q4k_bf16_dev(const void* w, const uint16_t* x, float* y, size_t M, size_t N,
                           size_t K, ssdq_stream_t stream) {
  if (M == 0 || N == 0) return ok();
  return gemm_multi("ssdq_gemm_q4k_bf16_dev", &w, &N, 1, x, &y, M, K, stream);
}

int ssdq_gemm_q4k_bf16_multi_dev(const void* const* w, const size_t* n, size_t count, const uint16_t* x_bf16,
                                 float* const* y, size_t M, size_t K, ssdq_stream_t stream) {
  return gemm_multi("ssdq_gemm_q4k_bf16_multi_dev", w, n, count, x_bf16, y, M, K, stream);
}

int ssdq_kv_quantize_rows_dev(const float* in, int8_t* codes, float* scales, size_t n_rows,
                              size_t row_len, ssdq_stream_t stream) {
  if (n_rows == 0) return ok();
  if (!scales || (row_len && (!in || !codes)))
    return fail(SSDQ_ERR_INVALID_ARG, "ssdq_kv_quantize_rows_dev: NULL pointer");
  if (!fits_int(row_len)) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_kv_quantize_rows_dev: row_len too large");
  hipError_t e = ssdq::launch_kv_quantize(in, codes, scales, n_rows, row_len, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "ssdq_kv_quantize_rows_dev");
  return ok();
}

int ssdq_kv_dequantize_rows_dev(const int8_t* codes, const float* scales, float* out,
                                size_t n_rows, size_t row_len, ssdq_stream_t stream) {
  if (n_rows == 0 || row_len == 0) return ok();
  if (!codes || !scales || !out) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_kv_dequantize_rows_dev: NULL pointer");
  if (!fits_int(row_len)) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_kv_dequantize_rows_dev: row_len too large");
  hipError_t e = ssdq::launch_kv_dequantize(codes, scales, out, n_rows, row_len, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "ssdq_kv_dequantize_rows_dev");
  return ok();
}

int ssdq_paged_kv_append_dev(const float* k, const float* v, const int32_t* slot_mapping,
                             int8_t* k_codes, float* k_scales, int8_t* v_codes, float* v_scales,
                             size_t n_tokens, size_t kv_dim, ssdq_stream_t stream) {
  if (n_tokens == 0) return ok();
  if (!k || !v || !slot_mapping || !k_codes || !k_scales || !v_codes || !v_scales)
    return fail(SSDQ_ERR_INVALID_ARG, "ssdq_paged_kv_append_dev: NULL pointer");
  if (kv_dim == 0 || !fits_int(kv_dim)) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_paged_kv_append_dev: bad kv_dim");
  hipError_t e = ssdq::launch_paged_kv_append(k, v, slot_mapping, k_codes, k_scales, v_codes,
                                              v_scales, n_tokens, kv_dim, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "ssdq_paged_kv_append_dev");
  return ok();
}

static bool head_dim_ok(size_t hd) { return hd == 64 || hd == 128 || hd == 256; }

// Argument checks shared by the paged-attention entry points; 0 with *a filled
// in, or the failure status.
static int paged_attention_args(const char* fn, const float* q, const int8_t* k_codes, const float* k_scales,
                                const int8_t* v_codes, const float* v_scales, const int32_t* block_tables,
                                const int32_t* ctx_lens, float* out, size_t n_seq, size_t n_head,
                                size_t n_head_kv, size_t head_dim, size_t block_size,
                                size_t max_blocks_per_seq, size_t max_ctx, ssdq::PagedAttnArgs* a) {
  if (!q || !k_codes || !k_scales || !v_codes || !v_scales || !block_tables || !ctx_lens || !out)
    return fail(SSDQ_ERR_INVALID_ARG, "%s: NULL pointer", fn);
  if (!head_dim_ok(head_dim)) return fail(SSDQ_ERR_UNSUPPORTED, "%s: head_dim %zu not in {64,128,256}", fn, head_dim);
  if (n_head_kv == 0 || n_head % n_head_kv) return fail(SSDQ_ERR_INVALID_ARG, "%s: n_head must be a multiple of n_head_kv", fn);
  if (((uintptr_t)k_codes & 3) || ((uintptr_t)v_codes & 3) || ((uintptr_t)q & 3) || ((uintptr_t)out & 3))
    return fail(SSDQ_ERR_INVALID_ARG, "%s: q, out and the code pools must be 4-byte aligned", fn);
  if (block_size == 0 || max_blocks_per_seq == 0) return fail(SSDQ_ERR_INVALID_ARG, "%s: empty block geometry", fn);
  if (max_ctx > max_blocks_per_seq * block_size)
    return fail(SSDQ_ERR_INVALID_ARG, "%s: max_ctx exceeds the block tables", fn);
  if (!fits_int(n_seq) || n_seq > 65535 || n_head_kv > 65535 || !fits_int(max_ctx) ||
      !fits_int(n_seq * max_blocks_per_seq))
    return fail(SSDQ_ERR_INVALID_ARG, "%s: dimensions too large", fn);
  *a = ssdq::PagedAttnArgs{q, k_codes, k_scales, v_codes, v_scales, block_tables, ctx_lens, out,
                           (int)n_seq, (int)n_head, (int)n_head_kv, (int)head_dim, (int)block_size,
                           (int)max_blocks_per_seq, (int)(max_ctx ? max_ctx : 1)};
  return SSDQ_OK;
}

int ssdq_paged_attention_int8_dev(const float* q, const int8_t* k_codes, const float* k_scales,
                                  const int8_t* v_codes, const float* v_scales,
                                  const int32_t* block_tables, const int32_t* ctx_lens,
                                  float* out, size_t n_seq, size_t n_head, size_t n_head_kv,
                                  size_t head_dim, size_t block_size, size_t max_blocks_per_seq,
                                  size_t max_ctx, ssdq_stream_t stream) {
  const char* fn = "ssdq_paged_attention_int8_dev";
  if (n_seq == 0 || n_head == 0) return ok();
  ssdq::PagedAttnArgs a;
  int rc = paged_attention_args(fn, q, k_codes, k_scales, v_codes, v_scales, block_tables, ctx_lens, out, n_seq,
                                n_head, n_head_kv, head_dim, block_size, max_blocks_per_seq, max_ctx, &a);
  if (rc != SSDQ_OK) return rc;
  hipStream_t s = (hipStream_t)stream;
  const size_t wsb = ssdq::paged_attn_workspace_bytes(a, nullptr);
  void* ws = nullptr;
  hipError_t e = workspace_get(wsb, s, &ws);
  if (e != hipSuccess) return hip_fail(e, "ssdq_paged_attention_int8_dev: workspace");
  e = ssdq::launch_paged_attn(a, ws, s);
  if (e != hipSuccess) return hip_fail(e, fn);
  return ok();
}

int ssdq_paged_attention_int8_window_dev(const float* q, const int8_t* k_codes, const float* k_scales,
                                         const int8_t* v_codes, const float* v_scales,
                                         const int32_t* block_tables, const int32_t* ctx_lens,
                                         const int32_t* window_starts, const int32_t* window_ends, float* out,
                                         size_t n_seq, size_t n_head, size_t n_head_kv, size_t head_dim,
                                         size_t block_size, size_t max_blocks_per_seq, size_t max_ctx,
                                         ssdq_stream_t stream) {
  const char* fn = "ssdq_paged_attention_int8_window_dev";
  if (n_seq == 0 || n_head == 0) return ok();
  ssdq::PagedAttnArgs a;
  int rc = paged_attention_args(fn, q, k_codes, k_scales, v_codes, v_scales, block_tables, ctx_lens, out, n_seq,
                                n_head, n_head_kv, head_dim, block_size, max_blocks_per_seq, max_ctx, &a);
  if (rc != SSDQ_OK) return rc;
  a.win_lo = window_starts;
  a.win_hi = window_ends;
  hipStream_t s = (hipStream_t)stream;
  const size_t wsb = ssdq::paged_attn_workspace_bytes(a, nullptr);
  void* ws = nullptr;
  hipError_t e = workspace_get(wsb, s, &ws);
  if (e != hipSuccess) return hip_fail(e, "ssdq_paged_attention_int8_window_dev: workspace");
  e = ssdq::launch_paged_attn(a, ws, s);
  if (e != hipSuccess) return hip_fail(e, fn);
  return ok();
}

int ssdq_paged_attention_int8_noalloc_dev(const float* q, const int8_t* k_codes, const float* k_scales,
                                          const int8_t* v_codes, const float* v_scales,
                                          const int32_t* block_tables, const int32_t* ctx_lens, float* out,
                                          size_t n_seq, size_t n_head, size_t n_head_kv, size_t head_dim,
                                          size_t block_size, size_t max_blocks_per_seq, size_t max_ctx,
                                          ssdq_stream_t stream) {
  const char* fn = "ssdq_paged_attention_int8_noalloc_dev";
  if (n_seq == 0 || n_head == 0) return ok();
  ssdq::PagedAttnArgs a;
  int rc = paged_attention_args(fn, q, k_codes, k_scales, v_codes, v_scales, block_tables, ctx_lens, out, n_seq,
                                n_head, n_head_kv, head_dim, block_size, max_blocks_per_seq, max_ctx, &a);
  if (rc != SSDQ_OK) return rc;
  size_t need = 0;
  hipError_t e = ssdq::launch_paged_attn_noalloc(a, (hipStream_t)stream, &need);
  if (need > ssdq::kNoAllocScratchBytes)
    return fail(SSDQ_ERR_INVALID_ARG, "%s: the call needs %zu bytes of scratch, the static maximum is %zu", fn,
                need, ssdq::kNoAllocScratchBytes);
  if (e != hipSuccess) return hip_fail(e, fn);
  return ok();
}

int ssdq_flash_attention_f32_dev(const float* q, const float* k, const float* v, float* out,
                                 size_t n_head, size_t n_head_kv, size_t head_dim,
                                 size_t seq_len, size_t window_start, size_t window_end,
                                 ssdq_stream_t stream) {
  const char* fn = "ssdq_flash_attention_f32_dev";
  if (n_head == 0) return ok();
  if (!q || !out || (seq_len && (!k || !v))) return fail(SSDQ_ERR_INVALID_ARG, "%s: NULL pointer", fn);
  if (!head_dim_ok(head_dim)) return fail(SSDQ_ERR_UNSUPPORTED, "%s: head_dim %zu not in {64,128,256}", fn, head_dim);
  if (n_head_kv == 0 || n_head % n_head_kv) return fail(SSDQ_ERR_INVALID_ARG, "%s: n_head must be a multiple of n_head_kv", fn);
  if (!fits_int(seq_len) || !fits_int(n_head) || n_head_kv > 65535)
    return fail(SSDQ_ERR_INVALID_ARG, "%s: dimensions too large", fn);
  if (((uintptr_t)k & 15) || ((uintptr_t)v & 15))
    return fail(SSDQ_ERR_INVALID_ARG, "%s: k and v must be 16-byte aligned", fn);
  const size_t we = window_end < seq_len ? window_end : seq_len;
  const size_t ws = window_start < we ? window_start : we;
  hipStream_t s = (hipStream_t)stream;
  const size_t wsb = ssdq::flash_attn_f32_workspace_bytes((int)n_head, (int)n_head_kv,
                                                          (int)head_dim, (int)(we - ws), nullptr);
  void* wsp = nullptr;
  hipError_t e = workspace_get(wsb, s, &wsp);
  if (e != hipSuccess) return hip_fail(e, "ssdq_flash_attention_f32_dev: workspace");
  e = ssdq::launch_flash_attn_f32(q, k, v, out, (int)n_head, (int)n_head_kv, (int)head_dim,
                                  (int)seq_len, (int)ws, (int)we, wsp, s);
  if (e != hipSuccess) return hip_fail(e, fn);
  return ok();
}

int ssdq_flash_attention_f32(ssdq_ctx* c, const float* q, const float* k, const float* v,
                             size_t n_head, size_t n_head_kv, size_t head_dim, size_t seq_len,
                             size_t window_start, size_t window_end, float* out) {
  if (!c) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_flash_attention_f32: ctx is NULL");
  if (n_head == 0) return ok();
  if (!q || !out || (seq_len && (!k || !v))) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_flash_attention_f32: NULL pointer");
  std::lock_guard<std::mutex> lk(c->mu);
  hipError_t e = hipSetDevice(c->device);
  if (e != hipSuccess) return hip_fail(e, "ssdq_flash_attention_f32: hipSetDevice");
  const size_t qn = n_head * head_dim, kvn = seq_len * n_head_kv * head_dim;
  void *dq, *dk, *dv, *dout;
  if ((e = ctx_buf(c, 0, qn * 4, &dq)) != hipSuccess || (e = ctx_buf(c, 1, kvn * 4, &dk)) != hipSuccess ||
      (e = ctx_buf(c, 2, kvn * 4, &dv)) != hipSuccess || (e = ctx_buf(c, 3, qn * 4, &dout)) != hipSuccess)
    return hip_fail(e, "ssdq_flash_attention_f32: staging allocation");
  if ((e = hipMemcpyAsync(dq, q, qn * 4, hipMemcpyHostToDevice, c->stream)) != hipSuccess ||
      (kvn && (e = hipMemcpyAsync(dk, k, kvn * 4, hipMemcpyHostToDevice, c->stream)) != hipSuccess) ||
      (kvn && (e = hipMemcpyAsync(dv, v, kvn * 4, hipMemcpyHostToDevice, c->stream)) != hipSuccess))
    return hip_fail(e, "ssdq_flash_attention_f32: copy in");
  int rc = ssdq_flash_attention_f32_dev((const float*)dq, (const float*)dk, (const float*)dv,
                                        (float*)dout, n_head, n_head_kv, head_dim, seq_len,
                                        window_start, window_end, c->stream);
  if (rc < 0) return rc;
  if ((e = hipMemcpyAsync(out, dout, qn * 4, hipMemcpyDeviceToHost, c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_flash_attention_f32: copy out");
  if ((e = hipStreamSynchronize(c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_flash_attention_f32: sync");
  return ok();
}

// ------------------------------------------------------------ host twins
// dequantize_to_f32 (src/ssd/streamer.rs:93-125): F32 / F16 / BF16 widen,
// Q4_0 / Q8_0 / Q6_K per the load-time dequantizers and Q4_K per the matvec
// element values; only whole blocks present in data_len are decoded, the rest
// of the n_elements outputs is zero (the dequantizers' `break` + `resize`).
int ssdq_dequantize_to_f32(ssdq_ctx* c, int dtype, const uint8_t* data, size_t data_len,
                           size_t n_elements, float* out) {
  if (!c) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_dequantize_to_f32: ctx is NULL");
  if (n_elements == 0) return ok();
  if (!out) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_dequantize_to_f32: out is NULL");
  if (!float_type(dtype) && !supported_quant(dtype)) {
    memset(out, 0, n_elements * sizeof(float));
    fail(SSDQ_WARN_UNSUPPORTED_ZEROED, "ssdq_dequantize_to_f32: dtype %d unsupported, zeros", dtype);
    return SSDQ_WARN_UNSUPPORTED_ZEROED;
  }
  const size_t bs = ssdq_block_size(dtype), tsz = ssdq_type_size(dtype);
  size_t units = n_elements / bs;  // whole blocks (elements for float types)
  if (float_type(dtype)) {
    // the reference reads n_elements values unconditionally and would read
    // past a short slice; that is an error here
    if (data_len < n_elements * tsz)
      return fail(SSDQ_ERR_INVALID_ARG, "ssdq_dequantize_to_f32: data has %zu bytes, need %zu",
                  data_len, n_elements * tsz);
  } else if (units > data_len / tsz) {
    units = data_len / tsz;
  }
  const size_t in_bytes = units * tsz, decoded = units * bs;
  if (in_bytes && !data) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_dequantize_to_f32: data is NULL");
  std::lock_guard<std::mutex> lk(c->mu);
  hipError_t e = hipSetDevice(c->device);
  if (e != hipSuccess) return hip_fail(e, "ssdq_dequantize_to_f32: hipSetDevice");
  void *dw, *dy;
  if ((e = ctx_buf(c, 0, in_bytes, &dw)) != hipSuccess ||
      (e = ctx_buf(c, 2, n_elements * sizeof(float), &dy)) != hipSuccess)
    return hip_fail(e, "ssdq_dequantize_to_f32: staging allocation");
  if (in_bytes && (e = hipMemcpyAsync(dw, data, in_bytes, hipMemcpyHostToDevice, c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_dequantize_to_f32: copy in");
  int rc = ssdq_dequant_dev(dtype, dw, decoded, (float*)dy, c->stream);
  if (rc < 0) return rc;
  if ((e = hipMemcpyAsync(out, dy, decoded * sizeof(float), hipMemcpyDeviceToHost, c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_dequantize_to_f32: copy out");
  if ((e = hipStreamSynchronize(c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_dequantize_to_f32: sync");
  if (decoded < n_elements) memset(out + decoded, 0, (n_elements - decoded) * sizeof(float));
  return ok();
}

// quantize_vectors_int8 (src/ssd/block_swap.rs:36-60): n_rows = data_len / dim
// whole rows; codes [n_rows * dim], scales [n_rows].
int ssdq_quantize_vectors_int8(ssdq_ctx* c, const float* data, size_t n_rows, size_t dim,
                               int8_t* codes, float* scales) {
  if (!c) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_quantize_vectors_int8: ctx is NULL");
  if (n_rows == 0) return ok();
  if (!scales || (dim && (!data || !codes)))
    return fail(SSDQ_ERR_INVALID_ARG, "ssdq_quantize_vectors_int8: NULL pointer");
  if (!fits_int(dim)) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_quantize_vectors_int8: dim too large");
  std::lock_guard<std::mutex> lk(c->mu);
  hipError_t e = hipSetDevice(c->device);
  if (e != hipSuccess) return hip_fail(e, "ssdq_quantize_vectors_int8: hipSetDevice");
  const size_t n = n_rows * dim;
  void *din, *dc, *ds;
  if ((e = ctx_buf(c, 0, n * sizeof(float), &din)) != hipSuccess ||
      (e = ctx_buf(c, 1, n, &dc)) != hipSuccess ||
      (e = ctx_buf(c, 2, n_rows * sizeof(float), &ds)) != hipSuccess)
    return hip_fail(e, "ssdq_quantize_vectors_int8: staging allocation");
  if (n && (e = hipMemcpyAsync(din, data, n * sizeof(float), hipMemcpyHostToDevice, c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_quantize_vectors_int8: copy in");
  int rc = ssdq_kv_quantize_rows_dev((const float*)din, (int8_t*)dc, (float*)ds, n_rows, dim, c->stream);
  if (rc < 0) return rc;
  if ((n && (e = hipMemcpyAsync(codes, dc, n, hipMemcpyDeviceToHost, c->stream)) != hipSuccess) ||
      (e = hipMemcpyAsync(scales, ds, n_rows * sizeof(float), hipMemcpyDeviceToHost, c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_quantize_vectors_int8: copy out");
  if ((e = hipStreamSynchronize(c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_quantize_vectors_int8: sync");
  return ok();
}

// dequantize_vectors_int8 (src/ssd/block_swap.rs:63-74): out [n_rows * dim].
int ssdq_dequantize_vectors_int8(ssdq_ctx* c, const int8_t* codes, const float* scales,
                                 size_t n_rows, size_t dim, float* out) {
  if (!c) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_dequantize_vectors_int8: ctx is NULL");
  if (n_rows == 0 || dim == 0) return ok();
  if (!codes || !scales || !out)
    return fail(SSDQ_ERR_INVALID_ARG, "ssdq_dequantize_vectors_int8: NULL pointer");
  if (!fits_int(dim)) return fail(SSDQ_ERR_INVALID_ARG, "ssdq_dequantize_vectors_int8: dim too large");
  std::lock_guard<std::mutex> lk(c->mu);
  hipError_t e = hipSetDevice(c->device);
  if (e != hipSuccess) return hip_fail(e, "ssdq_dequantize_vectors_int8: hipSetDevice");
  const size_t n = n_rows * dim;
  void *dc, *ds, *dout;
  if ((e = ctx_buf(c, 1, n, &dc)) != hipSuccess ||
      (e = ctx_buf(c, 2, n_rows * sizeof(float), &ds)) != hipSuccess ||
      (e = ctx_buf(c, 3, n * sizeof(float), &dout)) != hipSuccess)
    return hip_fail(e, "ssdq_dequantize_vectors_int8: staging allocation");
  if ((e = hipMemcpyAsync(dc, codes, n, hipMemcpyHostToDevice, c->stream)) != hipSuccess ||
      (e = hipMemcpyAsync(ds, scales, n_rows * sizeof(float), hipMemcpyHostToDevice, c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_dequantize_vectors_int8: copy in");
  int rc = ssdq_kv_dequantize_rows_dev((const int8_t*)dc, (const float*)ds, (float*)dout, n_rows, dim,
                                       c->stream);
  if (rc < 0) return rc;
  if ((e = hipMemcpyAsync(out, dout, n * sizeof(float), hipMemcpyDeviceToHost, c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_dequantize_vectors_int8: copy out");
  if ((e = hipStreamSynchronize(c->stream)) != hipSuccess)
    return hip_fail(e, "ssdq_dequantize_vectors_int8: sync");
  return ok();
}

}  // extern "C"

// The decode step's INT8 append and paged attention as one launch (plus the
// combine) where the matrix-core kernel applies (launch_paged_attn_append):
// the token at position ctx_lens[s] - 1 is the new one, quantized from new_k /
// new_v rows and written to pool row new_slot[s].  Same arguments and checks
// as ssdq_paged_kv_append_dev followed by ssdq_paged_attention_int8_dev.
int ssdq::api_paged_attention_append(const float* q, int8_t* k_codes, float* k_scales, int8_t* v_codes, float* v_scales,
                               const int32_t* block_tables, const int32_t* ctx_lens, const float* new_k,
                               const float* new_v, const int32_t* new_slot, float* out, size_t n_seq, size_t n_head,
                               size_t n_head_kv, size_t head_dim, size_t block_size, size_t max_blocks_per_seq,
                               size_t max_ctx, hipStream_t s) {
  const char* fn = "paged INT8 append + attention";
  if (n_seq == 0 || n_head == 0) return ok();
  if (!new_k || !new_v || !new_slot) return fail(SSDQ_ERR_INVALID_ARG, "%s: NULL pointer", fn);
  ssdq::PagedAttnArgs a;
  int rc = paged_attention_args(fn, q, k_codes, k_scales, v_codes, v_scales, block_tables, ctx_lens, out, n_seq,
                                n_head, n_head_kv, head_dim, block_size, max_blocks_per_seq, max_ctx, &a);
  if (rc != SSDQ_OK) return rc;
  a.new_k = new_k;
  a.new_v = new_v;
  a.new_slot = new_slot;
  const size_t wsb = ssdq::paged_attn_workspace_bytes(a, nullptr);
  void* ws = nullptr;
  hipError_t e = workspace_get(wsb, s, &ws);
  if (e != hipSuccess) return hip_fail(e, "paged INT8 append + attention: workspace");
  e = ssdq::launch_paged_attn_append(a, ws, s);
  if (e != hipSuccess) return hip_fail(e, fn);
  return ok();
}
