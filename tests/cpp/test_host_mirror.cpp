// GPU test of the C++ host mirror (ssd-llm_amd/host/ssdq_compute.hpp) against
// the CPU oracle on the same seeded inputs.  Exit status 0 = every check
// passed.  The oracle is the checker only.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "../../oracle/ssdq_oracle.h"
#include "../../ssd-llm_amd/host/ssdq_compute.hpp"

using ssdq::GgmlType;

static int g_fail = 0, g_checks = 0;

#define CHECK(cond, ...)                          \
  do {                                            \
    g_checks++;                                   \
    if (!(cond)) {                                \
      g_fail++;                                   \
      std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
      std::printf(__VA_ARGS__);                   \
      std::printf("\n");                          \
    }                                             \
  } while (0)

static bool same_bits(const float* a, const float* b, size_t n) {
  return std::memcmp(a, b, n * sizeof(float)) == 0;
}

// |gpu - ref| <= 1e-4 + 1e-3 |ref|, or the same bound against the exact sum
// when the serial fp32 reference itself is that far from it.
static size_t count_out_of_tol(const std::vector<float>& g, const std::vector<float>& ref,
                               const std::vector<double>* exact) {
  size_t bad = 0;
  for (size_t i = 0; i < g.size(); i++) {
    const double t = 1e-4 + 1e-3 * std::fabs((double)ref[i]);
    if (std::fabs((double)g[i] - ref[i]) <= t) continue;
    if (exact && std::fabs((double)g[i] - (*exact)[i]) <= 1e-4 + 1e-3 * std::fabs((*exact)[i])) continue;
    bad++;
  }
  return bad;
}

// scale_exp sets the f16 block scales' exponent; signed: each block's scales
// get a random sign (zero-mean weights)
static std::vector<uint8_t> random_blocks(GgmlType t, size_t rows, size_t cols, uint64_t seed,
                                          uint16_t scale_exp = 0x1C00, bool signed_blocks = false) {
  std::mt19937_64 g(seed);
  const size_t bs = ssdq_block_size((int)t), bb = ssdq_type_size((int)t);
  const size_t nb = rows * (cols / bs);
  std::vector<uint8_t> w(nb * bb);
  for (auto& b : w) b = (uint8_t)g();
  std::uniform_real_distribution<float> u(0.001f, 0.01f);
  for (size_t i = 0; i < nb; i++) {
    uint8_t* blk = w.data() + i * bb;
    const uint16_t sign = signed_blocks && (g() & 1) ? 0x8000 : 0;
    // f16 scales of moderate size (exponent bits forced into range)
    auto put_f16 = [&](uint8_t* p) {
      // default exponent: ~[0.0039, 0.0078)
      const uint16_t h = (uint16_t)(sign | scale_exp | (g() & 0x03FF));
      p[0] = h & 0xFF;
      p[1] = h >> 8;
    };
    if (t == GgmlType::Q6K) {
      put_f16(blk + 208);
      for (int j = 0; j < 16; j++) blk[192 + j] = (uint8_t)(int8_t)((int)(g() % 64) - 32);
    } else {
      put_f16(blk);
      if (t == GgmlType::Q4K) put_f16(blk + 2);
    }
  }
  return w;
}

int main() {
  setvbuf(stdout, nullptr, _IONBF, 0);
  // create(): a device ordinal far past the last one -> nullopt (MetalCompute::new() == None)
  CHECK(!ssdq::GpuCompute::create(1 << 20).has_value(), "create(bad device) must be nullopt");
  auto gc = ssdq::GpuCompute::create();
  CHECK(gc.has_value() && gc->has_gpu(), "create() failed: %s", ssdq_last_error());
  if (!gc) return 1;
  std::mt19937_64 rng(12345);
  std::normal_distribution<float> nd(0.f, 1.f);

  // matvec_quantized for every supported type
  for (GgmlType t : {GgmlType::Q4_0, GgmlType::Q8_0, GgmlType::Q4K, GgmlType::Q6K}) {
    const size_t out_dim = 96, in_dim = 1024;
    auto w = random_blocks(t, out_dim, in_dim, 7 + (int)t);
    std::vector<float> x(in_dim);
    for (auto& v : x) v = nd(rng);
    auto y = gc->matvec_quantized(w, x, out_dim, in_dim, t);
    std::vector<float> ref(out_dim);
    std::vector<double> exact(out_dim);
    ssdo_matvec_quantized(w.data(), x.data(), out_dim, in_dim, (int)t, ref.data());
    ssdo_matvec_exact(w.data(), x.data(), out_dim, in_dim, (int)t, exact.data());
    CHECK(y.size() == out_dim, "matvec size");
    CHECK(count_out_of_tol(y, ref, &exact) == 0, "matvec type %d out of tolerance", (int)t);
  }
  {  // unsupported type -> zeros; short weight slice -> Error(SSDQ_ERR_INVALID_ARG)
    std::vector<uint8_t> w(64 * 20, 0x11);
    std::vector<float> x(64, 1.f);
    auto y = gc->matvec_quantized(w.data(), w.size(), x.data(), x.size(), 4, 64,
                                  static_cast<GgmlType>(3));
    bool zeros = true;
    for (float v : y) zeros &= (v == 0.f);
    CHECK(zeros, "unsupported dtype must give zeros");
    int status = 0;
    try {
      gc->matvec_quantized(w.data(), 10, x.data(), x.size(), 4, 64, GgmlType::Q4_0);
    } catch (const ssdq::Error& e) {
      status = e.status();
    }
    CHECK(status == SSDQ_ERR_INVALID_ARG, "short w must raise INVALID_ARG, got %d", status);
  }

  // flash_attention_f32: below the GPU threshold -> nullopt; else within tolerance
  {
    const size_t nh = 8, nkv = 2, hd = 128;
    for (size_t seq : {size_t(3), size_t(300)}) {
      std::vector<float> q(nh * hd), k(seq * nkv * hd), v(seq * nkv * hd);
      for (auto& a : q) a = nd(rng);
      for (auto& a : k) a = nd(rng);
      for (auto& a : v) a = nd(rng);
      auto out = gc->flash_attention_f32(q, k, v, nh, nkv, hd, seq, 0, seq);
      if (seq < 4) {
        CHECK(!out.has_value(), "seq_len %zu must return nullopt", seq);
        continue;
      }
      CHECK(out.has_value(), "attention returned nullopt");
      std::vector<float> ref(nh * hd);
      ssdo_flash_attention_f32(q.data(), k.data(), v.data(), nh, nkv, hd, seq, 0, seq, ref.data());
      CHECK(out && count_out_of_tol(*out, ref, nullptr) == 0, "attention out of tolerance");
    }
  }

  // dequantize_to_f32: bit-exact, including a truncated slice
  for (GgmlType t : {GgmlType::Q4_0, GgmlType::Q8_0, GgmlType::Q4K, GgmlType::Q6K}) {
    auto w = random_blocks(t, 4, 512, 99 + (int)t);
    const size_t n = 4 * 512;
    for (size_t len : {w.size(), w.size() / 2 + 3}) {
      std::vector<uint8_t> part(w.begin(), w.begin() + len);
      auto got = gc->dequantize_to_f32(part, t, n);
      std::vector<float> ref(n);
      ssdo_dequantize_to_f32((int)t, part.data(), part.size(), n, ref.data());
      CHECK(same_bits(got.data(), ref.data(), n), "dequantize type %d len %zu not bit-exact", (int)t, len);
    }
  }

  // quantize_vectors_int8 / dequantize_vectors_int8: bit-exact
  {
    const size_t dim = 1024, rows = 33;
    std::vector<float> d(rows * dim);
    for (auto& a : d) a = nd(rng);
    for (size_t i = 0; i < dim; i++) d[5 * dim + i] = 0.f;  // zero row
    auto qs = gc->quantize_vectors_int8(d, dim);
    std::vector<int8_t> rc(rows * dim);
    std::vector<float> rs(rows);
    ssdo_quantize_rows_int8(d.data(), rows, dim, rc.data(), rs.data());
    CHECK(qs.first == rc, "int8 codes differ");
    CHECK(same_bits(qs.second.data(), rs.data(), rows), "int8 scales differ");
    auto back = gc->dequantize_vectors_int8(qs.first, qs.second, dim);
    std::vector<float> rb(rows * dim);
    ssdo_dequantize_rows_int8(rc.data(), rs.data(), rows, dim, rb.data());
    CHECK(same_bits(back.data(), rb.data(), rows * dim), "int8 dequant differs");
  }

  // ResidentWeights::load_layer + forward_layer: one decoder layer for one
  // token from device-resident tensors, against the oracle's composition
  {
    const size_t n_embd = 512, n_head = 4, n_kv = 2, hd = 128, n_ff = 1024;
    const size_t q_dim = n_head * hd, kv_dim = n_kv * hd;
    const size_t bs = 16, max_blocks = 8, n_phys = 12, pos = 37;  // 37 tokens already cached
    const uint32_t layer = 5;
    const float theta = 500000.f, eps = 1e-5f;
    // a GGUF data section: the tensors back to back, listed by TensorInfo;
    // block scales +-[0.00049, 0.00098) keep the activations O(1)
    std::vector<uint8_t> section;
    std::vector<ssdq::TensorInfo> infos;
    auto add = [&](const std::string& name, int dtype, std::vector<uint64_t> dims, const uint8_t* p, size_t n) {
      while (section.size() % 32) section.push_back(0);  // GGUF aligns tensor data
      infos.push_back({name, dims, dtype, (uint64_t)section.size(), (uint64_t)n});
      section.insert(section.end(), p, p + n);
    };
    const std::string pre = "blk." + std::to_string(layer) + ".";
    struct Proj { const char* name; GgmlType t; size_t in, out; std::vector<uint8_t> w; };
    std::vector<Proj> proj = {{"attn_q", GgmlType::Q4K, n_embd, q_dim, {}},
                              {"attn_k", GgmlType::Q4K, n_embd, kv_dim, {}},
                              {"attn_v", GgmlType::Q6K, n_embd, kv_dim, {}},
                              {"attn_output", GgmlType::Q4K, q_dim, n_embd, {}},
                              {"ffn_gate", GgmlType::Q4K, n_embd, n_ff, {}},
                              {"ffn_up", GgmlType::Q4K, n_embd, n_ff, {}},
                              {"ffn_down", GgmlType::Q6K, n_ff, n_embd, {}}};
    for (size_t i = 0; i < proj.size(); i++) {
      auto& p = proj[i];
      p.w = random_blocks(p.t, p.out, p.in, 500 + i, 0x1000, true);
      add(pre + p.name + ".weight", (int)p.t, {p.in, p.out}, p.w.data(), p.w.size());
    }
    std::uniform_real_distribution<float> un(0.5f, 1.5f);
    std::vector<float> attn_norm(n_embd), ffn_norm(n_embd), hidden(n_embd);
    for (auto& a : attn_norm) a = un(rng);
    for (auto& a : ffn_norm) a = un(rng);
    for (auto& a : hidden) a = nd(rng);
    add(pre + "attn_norm.weight", SSDQ_TYPE_F32, {n_embd}, (const uint8_t*)attn_norm.data(), n_embd * 4);
    add(pre + "ffn_norm.weight", SSDQ_TYPE_F32, {n_embd}, (const uint8_t*)ffn_norm.data(), n_embd * 4);
    add("blk.6.attn_q.weight", (int)GgmlType::Q4K, {n_embd, q_dim}, proj[0].w.data(), proj[0].w.size());
    add("output_norm.weight", SSDQ_TYPE_F32, {n_embd}, (const uint8_t*)ffn_norm.data(), n_embd * 4);

    auto rw = ssdq::ResidentWeights::create();
    CHECK(rw.has_value(), "ResidentWeights::create failed: %s", ssdq_last_error());
    if (!rw) return 1;
    size_t want = 0;
    for (const auto& t : infos)
      if (t.name.compare(0, pre.size(), pre) == 0) want += t.size_bytes;
    const size_t got_bytes = rw->load_layer(infos, section.data(), layer);
    CHECK(got_bytes == want && rw->size_bytes() == want && rw->size() == 9, "load_layer: %zu bytes, %zu tensors",
          got_bytes, rw->size());
    auto tq = rw->find_tensor_in_layer("attn_q.weight", layer);
    CHECK(tq && tq->dtype == (int)GgmlType::Q4K && tq->dims == std::vector<uint64_t>({n_embd, q_dim}),
          "find_tensor_in_layer(attn_q)");
    CHECK(!rw->find_tensor_in_layer("attn_q.weight", layer + 1), "another layer's tensor must not be loaded");

    // the pool: 37 earlier tokens, quantized by the oracle, at rows given by a
    // shuffled block table
    std::vector<int32_t> table(max_blocks);
    for (size_t i = 0; i < max_blocks; i++) table[i] = (int32_t)((i * 5 + 3) % n_phys);
    const size_t rows = n_phys * bs;
    std::vector<int8_t> kc(rows * kv_dim, 0), vc(rows * kv_dim, 0);
    std::vector<float> ks(rows, 0.f), vs(rows, 0.f);
    auto row_of = [&](size_t p) { return (size_t)table[p / bs] * bs + p % bs; };
    std::vector<float> kv(kv_dim);
    for (size_t p = 0; p < pos; p++) {
      const size_t r = row_of(p);
      for (auto& a : kv) a = nd(rng);
      ssdo_quantize_rows_int8(kv.data(), 1, kv_dim, &kc[r * kv_dim], &ks[r]);
      for (auto& a : kv) a = nd(rng);
      ssdo_quantize_rows_int8(kv.data(), 1, kv_dim, &vc[r * kv_dim], &vs[r]);
    }
    const int32_t slot = (int32_t)row_of(pos), ctx_len = (int32_t)(pos + 1);

    // device buffers
    void *d_hidden, *d_kc, *d_ks, *d_vc, *d_vs, *d_table, *d_slot, *d_ctx;
    bool ok = hipMalloc(&d_hidden, n_embd * 4) == hipSuccess && hipMalloc(&d_kc, kc.size()) == hipSuccess &&
              hipMalloc(&d_vc, vc.size()) == hipSuccess && hipMalloc(&d_ks, rows * 4) == hipSuccess &&
              hipMalloc(&d_vs, rows * 4) == hipSuccess && hipMalloc(&d_table, max_blocks * 4) == hipSuccess &&
              hipMalloc(&d_slot, 4) == hipSuccess && hipMalloc(&d_ctx, 4) == hipSuccess;
    CHECK(ok, "hipMalloc");
    if (!ok) return 1;
    auto copy = [&](void* dst, const void* src, size_t n, hipMemcpyKind kind) {
      ok = ok && hipMemcpy(dst, src, n, kind) == hipSuccess;
    };
    copy(d_hidden, hidden.data(), n_embd * 4, hipMemcpyHostToDevice);
    copy(d_kc, kc.data(), kc.size(), hipMemcpyHostToDevice);
    copy(d_vc, vc.data(), vc.size(), hipMemcpyHostToDevice);
    copy(d_ks, ks.data(), rows * 4, hipMemcpyHostToDevice);
    copy(d_vs, vs.data(), rows * 4, hipMemcpyHostToDevice);
    copy(d_table, table.data(), max_blocks * 4, hipMemcpyHostToDevice);
    copy(d_slot, &slot, 4, hipMemcpyHostToDevice);
    copy(d_ctx, &ctx_len, 4, hipMemcpyHostToDevice);
    CHECK(ok, "hipMemcpy to the device");
    const ssdq_layer_config cfg{n_embd, n_head, n_kv, hd, n_ff, theta, eps};
    const ssdq::PagedKvView view{(int8_t*)d_kc, (float*)d_ks, (int8_t*)d_vc, (float*)d_vs, bs,
                                 (const int32_t*)d_table, max_blocks, (const int32_t*)d_slot,
                                 (const int32_t*)d_ctx, max_blocks * bs};
    const int rc = ssdq::forward_layer(*rw, layer, cfg, (float*)d_hidden, pos, view);
    std::vector<float> out(n_embd);
    CHECK(rc == SSDQ_OK && hipDeviceSynchronize() == hipSuccess, "forward_layer: %s", ssdq_last_error());
    copy(out.data(), d_hidden, n_embd * 4, hipMemcpyDeviceToHost);
    CHECK(ok, "hipMemcpy from the device");

    // the oracle composition (transformer.rs:319-397 over the paged INT8 cache)
    std::vector<float> x = hidden, q(q_dim), k(kv_dim), v(kv_dim), att(q_dim), ao(n_embd), fin(n_embd);
    ssdo_rmsnorm(x.data(), attn_norm.data(), n_embd, eps);
    ssdo_matvec_quantized(proj[0].w.data(), x.data(), q_dim, n_embd, (int)proj[0].t, q.data());
    ssdo_matvec_quantized(proj[1].w.data(), x.data(), kv_dim, n_embd, (int)proj[1].t, k.data());
    ssdo_matvec_quantized(proj[2].w.data(), x.data(), kv_dim, n_embd, (int)proj[2].t, v.data());
    ssdo_rope_multi_head(q.data(), q_dim, hd, n_head, pos, theta);
    ssdo_rope_multi_head(k.data(), kv_dim, hd, n_kv, pos, theta);
    ssdo_quantize_rows_int8(k.data(), 1, kv_dim, &kc[slot * kv_dim], &ks[slot]);
    ssdo_quantize_rows_int8(v.data(), 1, kv_dim, &vc[slot * kv_dim], &vs[slot]);
    ssdo_paged_attention_int8(q.data(), kc.data(), ks.data(), vc.data(), vs.data(), table.data(), &ctx_len, 1,
                              n_head, n_kv, hd, bs, max_blocks, att.data());
    ssdo_matvec_quantized(proj[3].w.data(), att.data(), n_embd, q_dim, (int)proj[3].t, ao.data());
    std::vector<float> ref = hidden;
    ssdo_fused_post_attn_norm(ref.data(), ao.data(), ffn_norm.data(), n_embd, eps, fin.data());
    std::vector<float> g(n_ff), u(n_ff), dn(n_embd);
    ssdo_matvec_quantized(proj[4].w.data(), fin.data(), n_ff, n_embd, (int)proj[4].t, g.data());
    ssdo_matvec_quantized(proj[5].w.data(), fin.data(), n_ff, n_embd, (int)proj[5].t, u.data());
    ssdo_silu(g.data(), n_ff);
    for (size_t i = 0; i < n_ff; i++) g[i] *= u[i];
    ssdo_matvec_quantized(proj[6].w.data(), g.data(), n_embd, n_ff, (int)proj[6].t, dn.data());
    for (size_t i = 0; i < n_embd; i++) ref[i] += dn[i];
    // an output can be a near-cancellation of hidden + Wo a + W_down h, so the
    // bar is relative to the magnitude of those terms, S = |hidden| + |Wo||a| +
    // |W_down||h| over the dequantized elements: |gpu - ref| <= 1e-4 + 1e-4 S
    // (a K-term fp32 sum carries about sqrt(K) 2^-24 S of rounding)
    std::vector<double> scale(n_embd);
    for (size_t i = 0; i < n_embd; i++) scale[i] = std::fabs((double)hidden[i]);
    auto add_abs = [&](const Proj& p, const std::vector<float>& in) {
      std::vector<float> e(p.out * p.in);
      ssdo_matvec_elements(p.w.data(), p.out, p.in, (int)p.t, e.data());
      for (size_t r = 0; r < p.out; r++)
        for (size_t c = 0; c < p.in; c++) scale[r] += std::fabs((double)e[r * p.in + c] * in[c]);
    };
    add_abs(proj[3], att);
    add_abs(proj[6], g);
    size_t bad = 0;
    double worst = 0;
    for (size_t i = 0; i < n_embd; i++) {
      const double err = std::fabs((double)out[i] - ref[i]);
      worst = std::fmax(worst, err / scale[i]);
      bad += err > 1e-4 + 1e-4 * scale[i];
    }
    CHECK(bad == 0, "forward_layer: %zu outputs differ from the oracle composition", bad);
    std::printf("forward_layer: max |gpu - ref| / term scale %.2e\n", worst);
    for (void* p : {d_hidden, d_kc, d_ks, d_vc, d_vs, d_table, d_slot, d_ctx}) (void)hipFree(p);
    double mx = 0;
    for (float a : ref) mx = std::fmax(mx, std::fabs(a));
    std::printf("forward_layer: %zu outputs, max |ref| %.3g\n", ref.size(), mx);
  }

  std::printf("%s: %d checks, %d failed\n", g_fail ? "FAIL" : "PASS", g_checks, g_fail);
  return g_fail ? 1 : 0;
}
