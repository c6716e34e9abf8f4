// GPU test of the C++ host mirror (ssd-llm_amd/host/ssdq_compute.hpp) against
// the CPU oracle on the same seeded inputs.  Exit status 0 = every check
// passed.  The oracle is the checker only.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

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

static std::vector<uint8_t> random_blocks(GgmlType t, size_t rows, size_t cols, uint64_t seed) {
  std::mt19937_64 g(seed);
  const size_t bs = ssdq_block_size((int)t), bb = ssdq_type_size((int)t);
  const size_t nb = rows * (cols / bs);
  std::vector<uint8_t> w(nb * bb);
  for (auto& b : w) b = (uint8_t)g();
  std::uniform_real_distribution<float> u(0.001f, 0.01f);
  for (size_t i = 0; i < nb; i++) {
    uint8_t* blk = w.data() + i * bb;
    // f16 scales of moderate size (exponent bits forced into range)
    auto put_f16 = [&](uint8_t* p) {
      const uint16_t h = (uint16_t)(0x1C00 | (g() & 0x03FF));  // ~[0.0039, 0.0078)
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

  std::printf("%s: %d checks, %d failed\n", g_fail ? "FAIL" : "PASS", g_checks, g_fail);
  return g_fail ? 1 : 0;
}
