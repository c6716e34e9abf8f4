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
//   SsdStreamer::load_layer -> CachedLayer        ResidentWeights::load_layer (tensors stay in HBM)
//   find_tensor_in_layer(..) -> Option<&Vec<f32>> ResidentWeights::find_tensor_in_layer -> std::optional
//   forward_pass's per-layer body                 forward_layer (device buffers, paged INT8 KV)
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

// TensorInfo (src/model/gguf.rs:216-222): what the GGUF parser lists for a
// tensor; offset is from the start of the file's data section.
struct TensorInfo {
  std::string name;
  std::vector<uint64_t> dimensions;  // row length first
  int dtype = 0;                     // GgmlType id
  uint64_t offset = 0;
  uint64_t size_bytes = 0;
};

// SsdStreamer::load_layer (src/ssd/streamer.rs:43-66) with the tensors kept
// as their raw GGUF bytes in HBM (uploaded once) instead of dequantized f32
// vectors per load; find_tensor_in_layer (transformer.rs:552-559) returns
// the resident tensor.
class ResidentWeights {
 public:
  struct Tensor {
    const void* data;  // device address
    int dtype;
    std::vector<uint64_t> dims;
    size_t bytes;
  };

  // std::nullopt when no usable GPU exists (as GpuCompute::create)
  static std::optional<ResidentWeights> create(int device = -1) {
    ssdq_weights* w = nullptr;
    if (ssdq_weights_create(device, &w) != SSDQ_OK) return std::nullopt;
    return ResidentWeights(w);
  }

  // load_tensor_f32 without the dequantization: the tensor's bytes at
  // data_section + offset (the mapped file, GgufLoader::get_tensor_data)
  void put(const TensorInfo& t, const uint8_t* data_section) {
    detail::check("ssdq_weights_put",
                  ssdq_weights_put(w_.get(), t.name.c_str(), t.dtype, t.dimensions.data(), t.dimensions.size(),
                                   data_section + t.offset, t.size_bytes));
  }

  // load_layer: every tensor named "blk.{layer_idx}." (GgufFile::layer_tensors,
  // gguf.rs:410-416); returns the bytes made resident (CachedLayer::size_bytes)
  size_t load_layer(const std::vector<TensorInfo>& tensors, const uint8_t* data_section, uint32_t layer_idx) {
    const std::string prefix = "blk." + std::to_string(layer_idx) + ".";
    size_t total = 0;
    for (const auto& t : tensors) {
      if (t.name.compare(0, prefix.size(), prefix) != 0) continue;
      put(t, data_section);
      total += t.size_bytes;
    }
    return total;
  }

  std::optional<Tensor> find(const std::string& name) const {
    int dt = 0;
    uint64_t dims[4];
    size_t nd = 0, nb = 0;
    const void* p = ssdq_weights_find(w_.get(), name.c_str(), &dt, dims, &nd, &nb);
    if (!p) return std::nullopt;
    return Tensor{p, dt, std::vector<uint64_t>(dims, dims + nd), nb};
  }

  std::optional<Tensor> find_tensor_in_layer(const std::string& suffix, uint32_t layer_idx) const {
    return find("blk." + std::to_string(layer_idx) + "." + suffix);
  }

  size_t size() const { return ssdq_weights_count(w_.get()); }
  size_t size_bytes() const { return ssdq_weights_bytes(w_.get()); }
  ssdq_weights* raw() const { return w_.get(); }

 private:
  struct Deleter {
    void operator()(ssdq_weights* w) const { ssdq_weights_destroy(w); }
  };
  explicit ResidentWeights(ssdq_weights* w) : w_(w, Deleter()) {}
  std::shared_ptr<ssdq_weights> w_;
};

// One sequence's view of a layer's paged INT8 KV pool (device memory):
// PagedKvCache's block table and the pool rows of PhysicalBlock
// (src/inference/paged_attention.rs:34-35, 113-123).
struct PagedKvView {
  int8_t* k_codes;
  float* k_scales;
  int8_t* v_codes;
  float* v_scales;
  size_t block_size;
  const int32_t* block_table;  // max_blocks_per_seq entries
  size_t max_blocks_per_seq;
  const int32_t* slot_mapping;  // 1 entry: the pool row of this token
  const int32_t* ctx_len;       // 1 entry: tokens after the append
  size_t max_ctx;
};

// One layer of forward_pass (transformer.rs:319-397) for one token on device
// buffers: hidden (n_embd floats) is updated in place.  Returns the status
// (SSDQ_WARN_UNSUPPORTED_ZEROED passes, as the reference's zeros do).
inline int forward_layer(const ResidentWeights& w, uint32_t layer_idx, const ssdq_layer_config& cfg,
                         float* hidden, size_t position, const PagedKvView& kv, void* stream = nullptr,
                         void* scratch = nullptr, size_t scratch_bytes = 0) {
  return detail::check("ssdq_decode_layer_dev",
                       ssdq_decode_layer_dev(w.raw(), layer_idx, &cfg, hidden, position, kv.k_codes, kv.k_scales,
                                             kv.v_codes, kv.v_scales, kv.block_size, kv.block_table,
                                             kv.max_blocks_per_seq, kv.slot_mapping, kv.ctx_len, kv.max_ctx,
                                             scratch, scratch_bytes, stream));
}

}  // namespace ssdq
