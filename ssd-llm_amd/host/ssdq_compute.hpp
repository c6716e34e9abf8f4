// C++ host mirror of the reference's kernel-dispatch surface for the quantized
// path, written over the C ABI of libssdq.so (include/ssdq.h) only.
//
// The reference host is Rust: MetalCompute (src/metal/compute.rs:29-373) and
// the free dequant / INT8 helpers of src/ssd/streamer.rs and
// src/ssd/block_swap.rs.  This header keeps their names, argument meaning and
// error behaviour so the host side reads like the reference:
//   MetalCompute::new() -> Option<Self>         GpuCompute::create() -> std::optional
//   matvec_quantized(..) -> Vec<f32>             matvec_quantized(..) -> std::vector<float>
//   flash_attention_f32(..) -> Option<Vec<f32>>  flash_attention_f32(..) -> std::optional
//   dequantize_to_f32(..) -> Result<Vec<f32>>    dequantize_to_f32(..) (throws ssdq::Error)
//   quantize_vectors_int8 / dequantize_vectors_int8
// Differences, all deliberate: a context is created once and reused (the
// reference builds a MetalCompute per forward pass, transformer.rs:301-302);
// a short weight or activation slice raises ssdq::Error where the reference
// would panic on an out-of-range index; Q4_K dequantizes where the reference's
// loader yields zeros (streamer.rs:119-123).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "../../include/ssdq.h"

namespace ssdq {

// GgmlType ids (src/model/gguf.rs:17-48) of the types this path handles.
enum class GgmlType : int {
  F32 = SSDQ_TYPE_F32,
  F16 = SSDQ_TYPE_F16,
  Q4_0 = SSDQ_TYPE_Q4_0,
  Q8_0 = SSDQ_TYPE_Q8_0,
  Q4K = SSDQ_TYPE_Q4_K,
  Q6K = SSDQ_TYPE_Q6_K,
  BF16 = SSDQ_TYPE_BF16,
};

class Error : public std::runtime_error {
 public:
  Error(const std::string& fn, int status)
      : std::runtime_error(fn + " failed (" + std::to_string(status) + "): " + ssdq_last_error()),
        status_(status) {}
  int status() const { return status_; }

 private:
  int status_;
};

namespace detail {
// Negative status -> exception; SSDQ_OK and SSDQ_WARN_UNSUPPORTED_ZEROED pass
// (the latter is the reference's "unsupported type yields zeros").
inline int check(const char* fn, int rc) {
  if (rc < 0) throw Error(fn, rc);
  return rc;
}
struct CtxDeleter {
  void operator()(ssdq_ctx* c) const { ssdq_ctx_destroy(c); }
};
}  // namespace detail

// MetalCompute counterpart (compute.rs:29-373) for the quantized path.
class GpuCompute {
 public:
  // MetalCompute::new() -> Option<Self> (compute.rs:47-71): std::nullopt when
  // no usable GPU exists, and the caller keeps its CPU path.
  static std::optional<GpuCompute> create(int device = -1) {
    ssdq_ctx* c = nullptr;
    if (ssdq_ctx_create(device, &c) != SSDQ_OK) return std::nullopt;
    return GpuCompute(c);
  }

  // MetalCompute::has_gpu (compute.rs:262-264)
  bool has_gpu() const { return static_cast<bool>(ctx_); }
  int device() const { return ssdq_ctx_device(ctx_.get()); }
  ssdq_ctx* raw() const { return ctx_.get(); }

  // MetalCompute::matvec_quantized (compute.rs:157-191): y[out_dim] for one
  // activation vector; unsupported dtypes give zeros.
  std::vector<float> matvec_quantized(const uint8_t* w_raw, size_t w_len, const float* x,
                                      size_t x_len, size_t out_dim, size_t in_dim,
                                      GgmlType dtype) const {
    std::vector<float> y(out_dim);
    detail::check("ssdq_matvec_quantized",
                  ssdq_matvec_quantized(ctx_.get(), w_raw, w_len, x, x_len, out_dim, in_dim,
                                        static_cast<int>(dtype), y.data()));
    return y;
  }
  std::vector<float> matvec_quantized(const std::vector<uint8_t>& w_raw, const std::vector<float>& x,
                                      size_t out_dim, size_t in_dim, GgmlType dtype) const {
    return matvec_quantized(w_raw.data(), w_raw.size(), x.data(), x.size(), out_dim, in_dim, dtype);
  }

  // MetalCompute::flash_attention_f32 (compute.rs:217-258): std::nullopt below
  // the reference's GPU threshold (seq_len >= 4, compute.rs:232), where the
  // caller runs its CPU attention, exactly as with the reference.
  std::optional<std::vector<float>> flash_attention_f32(
      const std::vector<float>& q_heads, const std::vector<float>& k_cache,
      const std::vector<float>& v_cache, size_t n_head, size_t n_head_kv, size_t head_dim,
      size_t seq_len, size_t window_start, size_t window_end) const {
    if (seq_len < 4) return std::nullopt;
    if (q_heads.size() < n_head * head_dim || k_cache.size() < seq_len * n_head_kv * head_dim ||
        v_cache.size() < seq_len * n_head_kv * head_dim)
      throw Error("flash_attention_f32: slices shorter than the shapes", SSDQ_ERR_INVALID_ARG);
    std::vector<float> out(n_head * head_dim);
    detail::check("ssdq_flash_attention_f32",
                  ssdq_flash_attention_f32(ctx_.get(), q_heads.data(), k_cache.data(),
                                           v_cache.data(), n_head, n_head_kv, head_dim, seq_len,
                                           window_start, window_end, out.data()));
    return out;
  }

  // dequantize_to_f32 (src/ssd/streamer.rs:93-125)
  std::vector<float> dequantize_to_f32(const std::vector<uint8_t>& data, GgmlType dtype,
                                       size_t n_elements) const {
    std::vector<float> out(n_elements);
    detail::check("ssdq_dequantize_to_f32",
                  ssdq_dequantize_to_f32(ctx_.get(), static_cast<int>(dtype), data.data(),
                                         data.size(), n_elements, out.data()));
    return out;
  }

  // quantize_vectors_int8 (src/ssd/block_swap.rs:36-60): rows of `dim`
  // elements, one absmax scale per row.
  std::pair<std::vector<int8_t>, std::vector<float>> quantize_vectors_int8(
      const std::vector<float>& data, size_t dim) const {
    const size_t n_rows = dim ? data.size() / dim : 0;
    std::pair<std::vector<int8_t>, std::vector<float>> r;
    r.first.resize(n_rows * dim);
    r.second.resize(n_rows);
    detail::check("ssdq_quantize_vectors_int8",
                  ssdq_quantize_vectors_int8(ctx_.get(), data.data(), n_rows, dim, r.first.data(),
                                             r.second.data()));
    return r;
  }

  // dequantize_vectors_int8 (src/ssd/block_swap.rs:63-74)
  std::vector<float> dequantize_vectors_int8(const std::vector<int8_t>& quantized,
                                             const std::vector<float>& scales, size_t dim) const {
    if (quantized.size() < scales.size() * dim)
      throw Error("dequantize_vectors_int8: codes shorter than scales * dim", SSDQ_ERR_INVALID_ARG);
    std::vector<float> out(scales.size() * dim);
    detail::check("ssdq_dequantize_vectors_int8",
                  ssdq_dequantize_vectors_int8(ctx_.get(), quantized.data(), scales.data(),
                                               scales.size(), dim, out.data()));
    return out;
  }

 private:
  explicit GpuCompute(ssdq_ctx* c) : ctx_(c, detail::CtxDeleter()) {}
  std::shared_ptr<ssdq_ctx> ctx_;  // shared: copies of a GpuCompute use one context
};

}  // namespace ssdq
