// test_host.cpp — tests of the C++ host side (hearth_amd/host/hearth_host.hpp),
// written the way the reference's inline Rust tests read, through the C ABI and
// checked against the CPU oracle (oracle/hearth_oracle.h, linked as the
// checker only).
//
//   test_host --cpu    tests that need no device (the CPU suite runs these)
//   test_host          every test (on a GPU box)
//   --gguf PATH --seed N   also load PATH, a GGUF written from a model synthesized with seed N
//
// Each test prints "ok <name>" or "FAIL <name>: <reason>"; the exit status is
// the number of failures (capped at 100).
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <array>
#include <functional>
#include <random>
#include <string>
#include <vector>

#include "../../hearth_amd/host/hearth_host.hpp"
#include "../../oracle/hearth_oracle.h"

using namespace hearth;

namespace {

struct Failure {
  std::string msg;
};
struct TestCase {
  const char* name;
  bool gpu;
  std::function<void()> fn;
};
std::vector<TestCase>& registry() {
  static std::vector<TestCase> r;
  return r;
}
struct Reg {
  Reg(const char* n, bool gpu, std::function<void()> f) { registry().push_back({n, gpu, std::move(f)}); }
};
#define TEST_CPU(name) \
  static void name();  \
  static Reg reg_##name(#name, false, name); \
  static void name()
#define TEST_GPU(name) \
  static void name();  \
  static Reg reg_##name(#name, true, name); \
  static void name()
#define REQUIRE(cond, ...)                                          \
  do {                                                              \
    if (!(cond)) {                                                  \
      char buf_[512];                                               \
      snprintf(buf_, sizeof buf_, __VA_ARGS__);                     \
      throw Failure{std::string(#cond) + " -- " + buf_};            \
    }                                                               \
  } while (0)

template <class T> T must(std::optional<T> o, const char* what) {
  if (!o) throw Failure{std::string(what) + " returned None: " + (hh_last_error() ? hh_last_error() : "")};
  return std::move(*o);
}
template <class T> T must(Result<T> r, const char* what) {
  if (!r) throw Failure{std::string(what) + ": " + r.error()};
  return std::move(r.value());
}

GpuCompute& gpu() {
  static std::optional<GpuCompute> g = GpuCompute::create(0);
  if (!g) throw Failure{"GpuCompute::create(0) returned None"};
  return *g;
}

uint16_t f16(float x) { return ho_f32_to_f16(x); }
bool same_bits(float a, float b) { return std::memcmp(&a, &b, 4) == 0; }

// q2_0.rs:939-986 / q1_0g128.rs:1504-1551 paired-vs-single fixtures.
std::vector<uint8_t> ref_q2_weights(size_t n) {
  const size_t nb = n / 128;
  std::vector<uint8_t> w(nb * 34);
  for (size_t b = 0; b < nb; ++b) {
    const uint16_t s = f16(((float)(b % 7) + 0.5f) * 0.25f);
    std::memcpy(&w[b * 34], &s, 2);
    for (size_t j = 0; j < 32; ++j) w[b * 34 + 2 + j] = (uint8_t)(((b * 32 + j) * 37) ^ 0xAB);
  }
  return w;
}
std::vector<uint8_t> ref_q1_weights(size_t n) {
  const size_t nb = n / 128;
  std::vector<uint8_t> w(nb * 18);
  for (size_t b = 0; b < nb; ++b) {
    const uint16_t s = f16(((float)(b % 7) + 0.5f) * 0.25f);
    std::memcpy(&w[b * 18], &s, 2);
    for (size_t j = 0; j < 16; ++j) w[b * 18 + 2 + j] = (uint8_t)(((b * 16 + j) * 37) ^ 0xAB);
  }
  return w;
}
std::vector<uint8_t> ref_act(size_t n, uint32_t salt) {
  const size_t nb = n / 32;
  std::vector<uint8_t> a(nb * 34);
  for (size_t b = 0; b < nb; ++b) {
    const uint16_t s = f16(((float)(b % 5) + 0.5f) * 0.125f);
    std::memcpy(&a[b * 34], &s, 2);
    const uint8_t v = (uint8_t)((uint32_t)b * salt * 2654435761u);
    for (size_t j = 0; j < 32; ++j) a[b * 34 + 2 + j] = v;
  }
  return a;
}

// ------------------------------------------------------------------ CPU tests

// new() -> Option<Self> (lib.rs:126): no such device is None, not an abort.
TEST_CPU(test_gpu_compute_new_without_device_is_none) {
  auto g = GpuCompute::create(4096);
  REQUIRE(!g.has_value(), "device 4096 opened");
  const char* e = hh_last_error();
  REQUIRE(e && e[0], "no error message for the failed open");
}

// QuantKind::from_gguf_dtype (lib.rs:37-49): this path's formats, None otherwise.
TEST_CPU(test_quant_kind_from_gguf_dtype) {
  REQUIRE(from_gguf_dtype(8) == QuantKind::Q8_0, "8");
  REQUIRE(from_gguf_dtype(41) == QuantKind::Q1_0, "41");
  REQUIRE(from_gguf_dtype(42) == QuantKind::Q2_0, "42");
  REQUIRE(from_gguf_dtype(43) == QuantKind::Q1_0G128, "43");
  REQUIRE(from_gguf_dtype(142) == QuantKind::PQ2_0, "142");
  REQUIRE(from_gguf_dtype(143) == QuantKind::PTQ1_0, "143");
  for (int t : {0, 1, 2, 3, 12, 200}) REQUIRE(!from_gguf_dtype(t).has_value(), "dtype %d", t);
  REQUIRE(row_bytes(QuantKind::Q2_0, 4096) == 4096 / 128 * 34, "Q2_0 row");
  REQUIRE(row_bytes(QuantKind::Q1_0, 2048) == 2048 / 128 * 18, "Q1_0 row");
  REQUIRE(row_bytes(QuantKind::Q8_0, 4096) == 4096 / 32 * 34, "Q8_0 row");
}

// RopeCache::new (ops.rs:78-138): the same table as the oracle's restatement.
TEST_CPU(test_rope_cache_table) {
  for (int rd : {64, 128, 256}) {
    RopeCache r = RopeCache::build(300, rd, 1e6f);
    std::vector<float> want((size_t)300 * rd);
    ho_rope_table(300, rd, 1e6f, want.data());
    REQUIRE(std::memcmp(r.table.data(), want.data(), want.size() * 4) == 0, "rope_dim %d", rd);
  }
}

// Result<_, String>: a failing call carries the library's message.
TEST_CPU(test_status_carries_message) {
  hh_ctx* c = nullptr;
  Status s = check(hh_ctx_create(-1, &c), "open");
  REQUIRE(s.is_err() && s.error().rfind("open: ", 0) == 0 && s.error().size() > 6, "%s", s.error().c_str());
}

// ------------------------------------------------------------------ GPU tests

// q8_0.rs:177-195 test_roundtrip_q8_0: quantize then dequantize within 1.0,
// and the bytes equal the oracle's quantizer (q8_0.rs:20-51).
TEST_GPU(test_roundtrip_q8_0) {
  std::vector<float> src(64);
  for (int i = 0; i < 64; ++i) src[i] = ((float)i - 32.0f) * 0.5f;
  auto x = must(gpu().upload_f32(src), "upload");
  auto q = must(gpu().quantize_q8_0(x, 64), "quantize");
  auto d = must(gpu().dequantize(q, QuantKind::Q8_0, 64), "dequantize");
  auto back = gpu().readback_f32(d, 64);
  for (int i = 0; i < 64; ++i) REQUIRE(std::fabs(src[i] - back[i]) < 1.0f, "i=%d src=%g deq=%g", i, src[i], back[i]);
  std::vector<uint8_t> want(2 * 34);
  ho_quantize_q8_0(src.data(), 64, want.data());
  REQUIRE(gpu().readback_bytes(q, want.size()) == want, "bytes differ from q8_0::quantize");
}

// Known answers of the quantizer: an all-zero block has scale 1.0 (f16 0x3C00)
// and codes 0; a block whose max is 127 has scale 1.0 and codes x.  Random
// vectors match the oracle byte for byte.
TEST_GPU(test_q8_0_known_answers_and_random) {
  std::vector<float> v(64, 0.0f);
  for (int i = 0; i < 32; ++i) v[32 + i] = (float)(i * 4 - 127);   // -127 .. -3
  v[32 + 31] = 127.0f;
  auto x = must(gpu().upload_f32(v), "upload");
  auto q = gpu().readback_bytes(must(gpu().quantize_q8_0(x, 64), "quantize"), 68);
  REQUIRE(q[0] == 0x00 && q[1] == 0x3C, "zero block scale %02x%02x", q[1], q[0]);
  for (int i = 0; i < 32; ++i) REQUIRE(q[2 + i] == 0, "zero block code %d", i);
  REQUIRE(q[34] == 0x00 && q[35] == 0x3C, "max-127 block scale %02x%02x", q[35], q[34]);
  for (int i = 0; i < 32; ++i) REQUIRE((int8_t)q[36 + i] == (int8_t)v[32 + i], "code %d", i);
  std::mt19937 rng(11);
  std::normal_distribution<float> nd(0.0f, 3.0f);
  std::vector<float> r(4096 + 32 * 7);
  for (auto& e : r) e = nd(rng);
  auto xr = must(gpu().upload_f32(r), "upload");
  auto got = gpu().readback_bytes(must(gpu().quantize_q8_0(xr, r.size()), "quantize"), r.size() / 32 * 34);
  std::vector<uint8_t> want(r.size() / 32 * 34);
  ho_quantize_q8_0(r.data(), (int64_t)r.size(), want.data());
  REQUIRE(got == want, "random vector bytes differ");
}

// q2_0.rs:738-766 test_q2_0_dequantize: byte 0b00100100 at d = 2.0 is -2, 0, +2, -2.
TEST_GPU(test_q2_0_dequantize) {
  std::vector<uint8_t> data(34 * 2, 0);
  const uint16_t s = f16(2.0f);
  std::memcpy(&data[0], &s, 2);
  data[2] = 0b00100100;
  auto w = must(gpu().upload_bytes(data.data(), data.size()), "upload");
  auto out = gpu().readback_f32(must(gpu().dequantize(w, QuantKind::Q2_0, 256), "dequantize"), 256);
  REQUIRE(out[0] == -2.0f && out[1] == 0.0f && out[2] == 2.0f && out[3] == -2.0f, "%g %g %g %g", out[0], out[1],
          out[2], out[3]);
}

// q2_0.rs:913-934 test_q2_0_dot_f32: 0xAA codes are all +1, so the dot is the sum
// of the activation.  Here through the Q8_0 path, over two blocks (the device
// dots take whole 256-value units): within 0.01 per value of the f32 sum.
TEST_GPU(test_q2_0_dot_all_plus_one) {
  std::vector<uint8_t> w(2 * 34, 0xAA);
  const uint16_t s = f16(1.0f);
  std::memcpy(&w[0], &s, 2);
  std::memcpy(&w[34], &s, 2);
  std::vector<float> v(256);
  float expected = 0.0f;
  for (int i = 0; i < 256; ++i) { v[i] = (float)(i % 128) * 0.01f; expected += v[i]; }
  auto wb = must(gpu().upload_bytes(w.data(), w.size()), "upload");
  auto xb = must(gpu().upload_f32(v), "upload");
  auto y = gpu().readback_f32(must(gpu().dequant_matmul_fused(wb, QuantKind::Q2_0, xb, 1, 1, 256), "matmul"), 1);
  REQUIRE(std::fabs(y[0] - expected) < 0.01f * 256, "dot %g vs %g", y[0], expected);
  // n != 1 is None, as the plugin's dequant_matmul_fused; so is a k the units do not tile
  REQUIRE(!gpu().dequant_matmul_fused(wb, QuantKind::Q2_0, xb, 1, 2, 256).has_value(), "n = 2 accepted");
  REQUIRE(!gpu().dequant_matmul_fused(wb, QuantKind::Q2_0, xb, 1, 1, 128).has_value(), "k = 128 accepted");
}

// q1_0g128.rs:1459-1502: all bits 1 is +d, all bits 0 is -d.
TEST_GPU(test_q1_0_dequantize_all_ones_all_zeros) {
  for (uint8_t bits : {(uint8_t)0xFF, (uint8_t)0x00}) {
    std::vector<uint8_t> w(18, bits);
    const uint16_t s = f16(1.5f);
    std::memcpy(&w[0], &s, 2);
    auto wb = must(gpu().upload_bytes(w.data(), w.size()), "upload");
    auto out = gpu().readback_f32(must(gpu().dequantize(wb, QuantKind::Q1_0, 128), "dequantize"), 128);
    for (int i = 0; i < 128; ++i) REQUIRE(out[i] == (bits ? 1.5f : -1.5f), "bits %02x i=%d %g", bits, i, out[i]);
  }
}

// q2_0.rs:939-986 / q1_0g128.rs:1504-1551 (the paired kernel equals the single
// one): here the batched GEMM over both tokens equals the GEMV of each, and both
// equal the reference's scalar DotFn bit for bit, on the reference's fixtures
// (n = 256, 2048, 6144; the fixtures' n = 128 is below the device unit).
TEST_GPU(test_dot_q8_0x2_matches_single) {
  for (QuantKind k : {QuantKind::Q2_0, QuantKind::Q1_0}) {
    for (size_t n : {256u, 2048u, 6144u}) {
      auto w = k == QuantKind::Q2_0 ? ref_q2_weights(n) : ref_q1_weights(n);
      auto a0 = ref_act(n, 53), a1 = ref_act(n, 97);
      std::vector<uint8_t> both(a0);
      both.insert(both.end(), a1.begin(), a1.end());
      auto wb = must(gpu().upload_bytes(w.data(), w.size()), "upload");
      auto ab = must(gpu().upload_bytes(both.data(), both.size()), "upload");
      auto a0b = must(gpu().upload_bytes(a0.data(), a0.size()), "upload");
      auto a1b = must(gpu().upload_bytes(a1.data(), a1.size()), "upload");
      auto pair = gpu().readback_f32(must(gpu().dot_rows_q8_batch(wb, k, ab, 1, (uint32_t)n, 2), "gemm"), 2);
      const float g0 = gpu().readback_f32(must(gpu().dot_rows_q8(wb, k, a0b, 1, (uint32_t)n), "gemv"), 1)[0];
      const float g1 = gpu().readback_f32(must(gpu().dot_rows_q8(wb, k, a1b, 1, (uint32_t)n), "gemv"), 1)[0];
      const float w0 = k == QuantKind::Q2_0 ? ho_dot_q2_0_q8_0(w.data(), a0.data(), (int64_t)n)
                                            : ho_dot_q1_0_q8_0(w.data(), a0.data(), (int64_t)n);
      const float w1 = k == QuantKind::Q2_0 ? ho_dot_q2_0_q8_0(w.data(), a1.data(), (int64_t)n)
                                            : ho_dot_q1_0_q8_0(w.data(), a1.data(), (int64_t)n);
      REQUIRE(same_bits(pair[0], g0) && same_bits(pair[1], g1), "kind %d n=%zu paired %g %g single %g %g", (int)k, n,
              pair[0], pair[1], g0, g1);
      REQUIRE(same_bits(g0, w0) && same_bits(g1, w1), "kind %d n=%zu device %g %g DotFn %g %g", (int)k, n, g0, g1,
              w0, w1);
      REQUIRE(std::fabs(w0) > 1e-6f && std::fabs(w1) > 1e-6f, "n=%zu fixture", n);
    }
  }
}

// dequant_matmul_fused over many rows equals LlamaModel::matmul's CPU path
// (quantize x, then par_dot_rows with the scalar DotFn) for every format.
TEST_GPU(test_matmul_equals_dot_fn_rows) {
  std::mt19937 rng(3);
  const uint32_t m = 300, k = 2048;
  std::vector<float> x(k);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  for (auto& e : x) e = nd(rng);
  std::vector<uint8_t> xq(k / 32 * 34);
  ho_quantize_q8_0(x.data(), k, xq.data());
  for (QuantKind kind : {QuantKind::Q2_0, QuantKind::PQ2_0, QuantKind::Q1_0, QuantKind::Q8_0, QuantKind::PTQ1_0}) {
    std::vector<uint8_t> w(row_bytes(kind, k) * m);
    ho_synth_tensor((int)kind, 77, "blk.0.ffn_up.weight", m, k, 0.02f, 0.0f, w.data(), 8);
    auto wb = must(gpu().upload_bytes(w.data(), w.size()), "upload");
    auto xb = must(gpu().upload_f32(x), "upload");
    auto got = gpu().readback_f32(must(gpu().dequant_matmul_fused(wb, kind, xb, m, 1, k), "matmul"), m);
    std::vector<float> want(m);
    REQUIRE(ho_gemv((int)kind, w.data(), m, k, xq.data(), want.data(), 8, 0) == 0, "oracle gemv");
    for (uint32_t r = 0; r < m; ++r)
      REQUIRE(same_bits(got[r], want[r]), "kind %d row %u: %.9g vs %.9g", (int)kind, r, got[r], want[r]);
  }
}

// hearth-sampler lib.rs:214-233 test_greedy_argmax / test_temperature_zero_equiv_greedy,
// and the two tie rules: the dense sampler keeps the last maximum (max_by), the
// qwen35 loop and argmax_f32 the first.
TEST_GPU(test_greedy_argmax) {
  auto a = must(gpu().upload_f32({-1.0f, -2.0f, 5.0f, 0.5f}), "upload");
  REQUIRE(must(gpu().sample_greedy(a, 4, nullptr, 0, 1.1f, 0), "sample") == 2u, "greedy");
  auto b = must(gpu().upload_f32({0.1f, 0.2f, 0.7f, 0.05f}), "upload");
  REQUIRE(must(gpu().sample_greedy(b, 4, nullptr, 0, 1.1f, 0), "sample") == 2u, "temperature 0");
  auto t = must(gpu().upload_f32({1.0f, 3.0f, 0.5f, 3.0f, 2.0f}), "upload");
  REQUIRE(must(gpu().sample_greedy(t, 5, nullptr, 0, 1.0f, 0), "sample") == 3u, "dense tie: last max");
  REQUIRE(must(gpu().sample_greedy(t, 5, nullptr, 0, 1.0f, 1), "sample") == 1u, "hybrid tie: first max");
  REQUIRE(must(gpu().argmax_f32(t, 5), "argmax") == 1u, "argmax_f32: first max");
  // apply_repetition_penalty (lib.rs:26-40): a past token's positive logit is divided
  auto past = must(gpu().upload_bytes(std::vector<uint32_t>{3}.data(), 4), "upload");
  REQUIRE(must(gpu().sample_greedy(t, 5, &past, 1, 2.0f, 0), "sample") == 1u, "penalised 3 -> 1.5, max at 1");
}

// rms_norm (ops.rs:8-35) within 1e-5 of the oracle, rope_combined (ops.rs:140-164)
// bit for bit, decode attention (ops.rs:353-406) within 1e-4.
TEST_GPU(test_rms_norm_rope_attention) {
  std::mt19937 rng(5);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  const uint32_t n = 4096;
  std::vector<float> x(n), w(n);
  for (auto& e : x) e = nd(rng);
  for (auto& e : w) e = 1.0f + 0.02f * nd(rng);
  auto xb = must(gpu().upload_f32(x), "upload");
  auto wb = must(gpu().upload_f32(w), "upload");
  auto ob = must(gpu().create_storage_buffer(n * 4), "alloc");
  REQUIRE(gpu().rms_norm(xb, wb, ob, n, 1e-6f), "rms_norm");
  auto got = gpu().readback_f32(ob, n);
  std::vector<float> want(n);
  ho_rms_norm(x.data(), w.data(), 1e-6f, n, want.data());
  double md = 0, mw = 0;
  for (uint32_t i = 0; i < n; ++i) { md = std::fmax(md, std::fabs((double)got[i] - want[i])); mw = std::fmax(mw, std::fabs((double)want[i])); }
  REQUIRE(md / mw < 1e-5, "rms_norm rel %g", md / mw);

  const int hd = 128, max_seq = 256, nh = 8;
  RopeCache rc = RopeCache::build(max_seq, hd, 1e6f);
  auto tab = must(gpu().upload_f32(rc.table), "upload");
  std::vector<float> q((size_t)nh * hd);
  for (auto& e : q) e = nd(rng);
  auto qb = must(gpu().upload_f32(q), "upload");
  RopeConfig cfg{nh, hd, hd, max_seq, &tab};
  REQUIRE(gpu().rope_combined(qb, cfg, 77), "rope");
  auto qr = gpu().readback_f32(qb, q.size());
  for (int h = 0; h < nh; ++h) ho_rope_apply(rc.table.data(), max_seq, hd, q.data() + (size_t)h * hd, 77);
  REQUIRE(std::memcmp(qr.data(), q.data(), q.size() * 4) == 0, "rope differs from ops.rs");

  const int nkv = 8, nq = 32, seq = 2049, ms = seq + 7;
  std::vector<float> qv((size_t)nq * hd), kc((size_t)nkv * ms * hd), vc((size_t)nkv * ms * hd);
  for (auto& e : qv) e = nd(rng);
  for (auto& e : kc) e = nd(rng);
  for (auto& e : vc) e = nd(rng);
  auto qd = must(gpu().upload_f32(qv), "upload");
  auto kd = must(gpu().upload_f32(kc), "upload");
  auto vd = must(gpu().upload_f32(vc), "upload");
  auto od = must(gpu().flash_attention(qd, kd, vd, FlashAttnShape{nq, nkv, hd, ms, seq}), "attention");
  auto o = gpu().readback_f32(od, (size_t)nq * hd);
  double md2 = 0, mw2 = 0;
  for (int h = 0; h < nq; ++h) {
    std::vector<float> oh(hd), scratch(seq);
    const int kv = h / (nq / nkv);
    ho_attention(qv.data() + (size_t)h * hd, kc.data() + (size_t)kv * ms * hd, vc.data() + (size_t)kv * ms * hd, seq,
                 hd, oh.data(), scratch.data());
    for (int d = 0; d < hd; ++d) {
      md2 = std::fmax(md2, std::fabs((double)o[(size_t)h * hd + d] - oh[d]));
      mw2 = std::fmax(mw2, std::fabs((double)oh[d]));
    }
  }
  REQUIRE(md2 / mw2 < 1e-4, "attention rel %g", md2 / mw2);
}

// flash_attention_prefill (lib.rs:599-668; forward_batch's per-token attention,
// mod.rs:1101-1140): the split/merge form gives each token's row bit for bit as
// the decode operator at seq_len pos0 + t + 1; the fp32-MFMA form agrees to fp32
// rounding (1e-5 of the largest output).
TEST_GPU(test_flash_attention_prefill_modes) {
  std::mt19937 rng(9);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  for (auto geo : {std::array<int, 3>{32, 8, 128}, std::array<int, 3>{16, 4, 256}}) {
    const int nh = geo[0], nkv = geo[1], hd = geo[2], pos0 = 37, ntok = 45, ms = 96;
    std::vector<float> q((size_t)ntok * nh * hd), kc((size_t)nkv * ms * hd), vc((size_t)nkv * ms * hd);
    for (auto& e : q) e = nd(rng);
    for (auto& e : kc) e = nd(rng);
    for (auto& e : vc) e = nd(rng);
    auto qd = must(gpu().upload_f32(q), "upload");
    auto kd = must(gpu().upload_f32(kc), "upload");
    auto vd = must(gpu().upload_f32(vc), "upload");
    auto o0 = gpu().readback_f32(
        must(gpu().flash_attention_prefill(qd, kd, vd, PrefillAttnShape{nh, nkv, hd, ms, pos0, ntok, 0}), "prefill"),
        q.size());
    auto o1 = gpu().readback_f32(
        must(gpu().flash_attention_prefill(qd, kd, vd, PrefillAttnShape{nh, nkv, hd, ms, pos0, ntok, 1}), "prefill"),
        q.size());
    double md = 0, mx = 0;
    for (size_t i = 0; i < q.size(); ++i) {
      md = std::fmax(md, std::fabs((double)o0[i] - o1[i]));
      mx = std::fmax(mx, std::fabs((double)o0[i]));
    }
    REQUIRE(md <= 1e-5 * mx, "hd %d: flash form differs by %g of %g", hd, md, mx);
    for (int t : {0, 17, ntok - 1}) {
      std::vector<float> qt(q.begin() + (size_t)t * nh * hd, q.begin() + (size_t)(t + 1) * nh * hd);
      auto qtd = must(gpu().upload_f32(qt), "upload");
      auto dec = gpu().readback_f32(
          must(gpu().flash_attention(qtd, kd, vd, FlashAttnShape{nh, nkv, hd, ms, pos0 + t + 1}), "attention"),
          qt.size());
      REQUIRE(std::memcmp(dec.data(), o0.data() + (size_t)t * nh * hd, dec.size() * 4) == 0,
              "hd %d token %d: prefill row differs from the decode operator", hd, t);
    }
  }
}

hh_model_config tiny_dense() {
  hh_model_config c{};
  c.arch = 0; c.d_model = 1024; c.n_layers = 2; c.n_heads = 8; c.n_kv_heads = 4; c.head_dim = 128;
  c.d_ffn = 2048; c.vocab = 4096; c.eps = 1e-6f; c.rope_theta = 1e6f; c.max_seq = 128;
  c.wtype = HH_Q2_0; c.head_type = HH_Q8_0; c.qk_norm = 1; c.full_attn_interval = 4; c.ssm_head_dim = 128;
  c.ssm_conv_kernel = 4;
  return c;
}
hh_model_config tiny_hybrid() {
  hh_model_config c = tiny_dense();
  c.arch = 1; c.n_layers = 4; c.n_heads = 4; c.n_kv_heads = 2; c.head_dim = 256; c.rope_dim = 64;
  c.ssm_n_k_heads = 2; c.ssm_n_v_heads = 4; c.attn_out_gate = 1;
  return c;
}
ho_config to_oracle(const hh_model_config& c) {
  ho_config o{};
  o.arch = c.arch; o.d_model = c.d_model; o.n_layers = c.n_layers; o.n_heads = c.n_heads; o.n_kv_heads = c.n_kv_heads;
  o.head_dim = c.head_dim; o.d_ffn = c.d_ffn; o.vocab = c.vocab; o.eps = c.eps; o.rope_theta = c.rope_theta;
  o.rope_dim = c.rope_dim; o.max_seq = c.max_seq; o.wtype = c.wtype; o.head_type = c.head_type; o.qk_norm = c.qk_norm;
  o.full_attn_interval = c.full_attn_interval; o.ssm_n_k_heads = c.ssm_n_k_heads; o.ssm_n_v_heads = c.ssm_n_v_heads;
  o.ssm_head_dim = c.ssm_head_dim; o.ssm_conv_kernel = c.ssm_conv_kernel; o.attn_out_gate = c.attn_out_gate;
  o.kv_type = c.kv_type; o.had_block = c.had_block; o.had_flags = c.had_flags;
  return o;
}

// generate_text's token loop (mod.rs:2718-3012 / qwen35.rs:1654-1804) on a
// synthesized model (dense, hybrid, dense with a Q8_0 KV cache): tokens equal
// the oracle's in the device's association order.
TEST_GPU(test_generate_matches_oracle) {
  hh_model_config q8kv = tiny_dense();
  q8kv.kv_type = HH_Q8_0;   // KVStorage::Q8_0 (kvcache.rs:41-57)
  for (const hh_model_config& cfg : {tiny_dense(), tiny_hybrid(), q8kv}) {
    Model m = must(Model::create(gpu(), cfg), "create");
    must(m.synthesize(1234), "synthesize");
    const ho_config oc = to_oracle(cfg);
    ho_model* o = ho_model_new(&oc);
    ho_model_synth(o, 1234, 16);
    ho_model_set_order(o, 1);
    std::vector<uint32_t> prompt;
    for (int i = 0; i < 9; ++i) prompt.push_back(ho_synth_token(99, i, cfg.vocab));
    const float pen = cfg.arch == 0 ? 1.1f : 1.0f;
    Generation g = must(m.generate(prompt, 12, SamplerConfig{pen}), "generate");
    std::vector<uint32_t> want(12);
    std::vector<float> wl((size_t)cfg.vocab);
    ho_generate(o, prompt.data(), (int)prompt.size(), 0, 12, pen, want.data(), wl.data());
    ho_model_free(o);
    REQUIRE(g.tokens == want, "arch %d tokens differ from the oracle", cfg.arch);
    REQUIRE(g.decode_ms > 0.0 && g.prefill_ms > 0.0, "arch %d timing %g %g", cfg.arch, g.prefill_ms, g.decode_ms);
  }
}

// forward_batch then forward (mod.rs:899-1221, :451-860): the batched prefill
// leaves the state token-by-token feeding leaves, so the next step's logits agree.
TEST_GPU(test_prefill_then_forward) {
  const hh_model_config cfg = tiny_dense();
  std::vector<uint32_t> prompt;
  for (int i = 0; i < 40; ++i) prompt.push_back(ho_synth_token(7, i, cfg.vocab));
  Model a = must(Model::create(gpu(), cfg), "create");
  Model b = must(Model::create(gpu(), cfg), "create");
  must(a.synthesize(5), "synthesize");
  must(b.synthesize(5), "synthesize");
  must(a.prefill(std::vector<uint32_t>(prompt.begin(), prompt.end() - 1), 0), "prefill");
  std::vector<float> la = must(a.forward(prompt.back(), (int)prompt.size() - 1, cfg.vocab), "forward");
  std::vector<float> lb;
  for (size_t i = 0; i < prompt.size(); ++i) lb = must(b.forward(prompt[i], (int)i, cfg.vocab), "forward");
  REQUIRE(std::memcmp(la.data(), lb.data(), la.size() * 4) == 0, "batched prefill differs from token by token");
}

// Errors as the reference words them: an unknown tensor (matmul.rs:59-62), a
// cancelled step (mod.rs:461), a position past the cache.
TEST_GPU(test_model_errors) {
  const hh_model_config cfg = tiny_dense();
  Model m = must(Model::create(gpu(), cfg), "create");
  std::vector<uint8_t> bytes(34);
  Status s = m.upload_tensor("blk.99.no_such.weight", QuantKind::Q2_0, 128, 1, bytes.data(), bytes.size());
  REQUIRE(s.is_err() && s.error().find("not found") != std::string::npos, "%s", s.error().c_str());
  must(m.synthesize(1), "synthesize");
  must(m.set_cancel(true), "cancel");
  auto f = m.forward(1, 0, cfg.vocab);
  REQUIRE(f.is_err() && f.error().find("Cancelled") != std::string::npos, "%s", f.error().c_str());
  must(m.set_cancel(false), "uncancel");
  auto g = m.forward(1, cfg.max_seq + 5, cfg.vocab);
  REQUIRE(g.is_err(), "position past max_seq accepted");
  auto h = m.forward(1, 0, cfg.vocab);
  REQUIRE(h.is_ok(), "forward after the errors: %s", h.error().c_str());
}

std::string g_gguf;     // --gguf PATH: a model file written from a synthesized model
uint64_t g_gguf_seed = 0;

// LlamaModel::load (mod.rs:103-150) of a GGUF file written from a model
// synthesized with g_gguf_seed: the configuration reads back, and logits and
// greedy tokens equal the synthesized model's bit for bit.
TEST_GPU(test_load_gguf_matches_synthesized) {
  if (g_gguf.empty()) return;   // run by tests/test_host_cpp.py with --gguf
  hh_model_config cfg = must(read_config(g_gguf, 128), "read_config");
  REQUIRE(cfg.max_seq == 128 && cfg.d_model > 0 && cfg.vocab > 0, "config %d %d %d", cfg.max_seq, cfg.d_model,
          cfg.vocab);
  Model ref = must(Model::create(gpu(), cfg), "create");
  must(ref.synthesize(g_gguf_seed), "synthesize");
  Model m = must(Model::load(gpu(), g_gguf, 128), "load");
  std::vector<float> la = must(ref.forward(11, 0, cfg.vocab), "forward");
  std::vector<float> lb = must(m.forward(11, 0, cfg.vocab), "forward");
  REQUIRE(std::memcmp(la.data(), lb.data(), la.size() * 4) == 0, "logits differ");
  must(ref.reset(), "reset");
  must(m.reset(), "reset");
  const std::vector<uint32_t> prompt = {11, 400, 7, 123};
  Generation a = must(ref.generate(prompt, 8, SamplerConfig{1.0f}), "generate");
  Generation b = must(m.generate(prompt, 8, SamplerConfig{1.0f}), "generate");
  REQUIRE(a.tokens == b.tokens, "tokens differ");
  auto missing = Model::load(gpu(), g_gguf + ".missing", 128);
  REQUIRE(missing.is_err(), "a missing file loaded");
}

}  // namespace

int main(int argc, char** argv) {
  bool cpu_only = false;
  for (int i = 1; i < argc; ++i) {
    if (std::strcmp(argv[i], "--cpu") == 0) cpu_only = true;
    else if (std::strcmp(argv[i], "--gguf") == 0 && i + 1 < argc) g_gguf = argv[++i];
    else if (std::strcmp(argv[i], "--seed") == 0 && i + 1 < argc) g_gguf_seed = std::strtoull(argv[++i], nullptr, 10);
  }
  int failed = 0, ran = 0;
  for (const TestCase& t : registry()) {
    if (cpu_only && t.gpu) continue;
    ++ran;
    try {
      t.fn();
      printf("ok %s\n", t.name);
    } catch (const Failure& f) {
      ++failed;
      printf("FAIL %s: %s\n", t.name, f.msg.c_str());
    }
    fflush(stdout);
  }
  printf("%d passed, %d failed\n", ran - failed, failed);
  return failed > 100 ? 100 : failed;
}
