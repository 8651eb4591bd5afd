// hearth_host.hpp — C++17 host side of the MI355X decode path, above the C ABI
// of include/hearth_hip.h (libhearth_hip.so).  Header-only: include it and link
// the library.
//
// It restates, with the same names, argument meaning and error behaviour, the
// Rust interfaces a Hearth build calls on this path:
//  * GpuCompute: the GPU plugin hearth_compute::GpuCompute
//    (crates/hearth-compute/src/lib.rs:103-1552).  create() is `new() ->
//    Option<Self>` (lib.rs:126), so no device means std::nullopt and the
//    caller keeps its CPU path.  The operators return std::optional or bool
//    where the plugin returns Option or bool.
//  * Model: the decode model, LlamaModel (crates/hearth-llm/src/model/mod.rs:59-3012)
//    and the qwen35 hybrid (model/qwen35.rs).  load() is LlamaModel::load
//    (mod.rs:103-150), forward() is one decode step (mod.rs:451-860), prefill()
//    is forward_batch (mod.rs:899-1221), and generate() is the greedy token loop
//    of generate_text (mod.rs:2718-3012, qwen35.rs:1654-1804).  Token ids go in
//    and out, because the tokenizer is not on this path.
//  * Result<T>: Rust's Result<T, String>.  Each failing call carries the
//    library's message (hh_last_error), e.g. "Tensor not found: ..." as
//    matmul.rs:59-62 words it, or "Cancelled" (mod.rs:461).
//  * RopeCache: the host RoPE table of ops.rs:78-138.
//
// Arithmetic is the reference CPU path's, not the wgpu shaders'.
// dequant_matmul_fused quantizes x to Q8_0 (q8_0.rs:20-51) and runs the
// DotFn row dots (pool.rs:510-566) bit for bit.  The plugin's fp32 dequant
// shader (matmul.rs of hearth-compute) would give different bits.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <optional>
#include <string>
#include <utility>
#include <vector>

#include "../../include/hearth_hip.h"

namespace hearth {

// ---------------------------------------------------------------- Result<T>
struct Unit {};

template <class T>
class Result {
 public:
  static Result ok(T v) {
    Result r;
    r.v_ = std::move(v);
    return r;
  }
  static Result err(std::string e) {
    Result r;
    r.e_ = std::move(e);
    return r;
  }
  bool is_ok() const { return v_.has_value(); }
  bool is_err() const { return !v_.has_value(); }
  explicit operator bool() const { return is_ok(); }
  T& value() { return *v_; }
  const T& value() const { return *v_; }
  const std::string& error() const { return e_; }

 private:
  std::optional<T> v_;
  std::string e_;
};
using Status = Result<Unit>;

// A non-zero library status as the Err side: "<what>: <hh_last_error()>".
inline std::string last_error(const char* what) {
  const char* e = hh_last_error();
  return std::string(what) + ": " + (e && e[0] ? e : "error");
}
inline Status check(int rc, const char* what) {
  return rc == HH_OK ? Status::ok({}) : Status::err(last_error(what));
}

// ---------------------------------------------------------------- QuantKind
// hearth_compute::QuantKind (lib.rs:25-50), by GGUF dtype id.  from_gguf_dtype
// returns nullopt for a dtype the device path does not take (lib.rs:37-49).
enum class QuantKind : int {
  Q8_0 = HH_Q8_0,
  Q1_0 = HH_Q1_0,
  Q2_0 = HH_Q2_0,
  Q1_0G128 = HH_Q1_0_G128,
  PQ2_0 = HH_PQ2_0,
  PTQ1_0 = HH_PTQ1_0,
};
inline std::optional<QuantKind> from_gguf_dtype(int dtype) {
  switch (dtype) {
    case HH_Q8_0: return QuantKind::Q8_0;
    case HH_Q1_0: return QuantKind::Q1_0;
    case HH_Q2_0: return QuantKind::Q2_0;
    case HH_Q1_0_G128: return QuantKind::Q1_0G128;
    case HH_PQ2_0: return QuantKind::PQ2_0;
    case HH_PTQ1_0: return QuantKind::PTQ1_0;
  }
  return std::nullopt;
}
// Bytes of a row of n_cols values (ggml.rs:105-171 block sizes).
inline size_t row_bytes(QuantKind k, size_t n_cols) {
  switch (k) {
    case QuantKind::Q8_0: return n_cols / 32 * 34;
    case QuantKind::Q1_0: case QuantKind::Q1_0G128: return n_cols / 128 * 18;
    case QuantKind::Q2_0: case QuantKind::PQ2_0: return n_cols / 128 * 34;
    case QuantKind::PTQ1_0: return n_cols / 128 * 28;
  }
  return 0;
}

// ---------------------------------------------------------------- context, buffers
using CtxPtr = std::shared_ptr<hh_ctx>;

// Device memory owned by one context (hearth_compute GpuBuffer): freed on
// destruction; move-only.
class GpuBuffer {
 public:
  GpuBuffer() = default;
  GpuBuffer(CtxPtr ctx, void* p, size_t n) : ctx_(std::move(ctx)), p_(p), n_(n) {}
  GpuBuffer(const GpuBuffer&) = delete;
  GpuBuffer& operator=(const GpuBuffer&) = delete;
  GpuBuffer(GpuBuffer&& o) noexcept : ctx_(std::move(o.ctx_)), p_(o.p_), n_(o.n_) { o.p_ = nullptr; o.n_ = 0; }
  GpuBuffer& operator=(GpuBuffer&& o) noexcept {
    if (this != &o) {
      release();
      ctx_ = std::move(o.ctx_);
      p_ = o.p_;
      n_ = o.n_;
      o.p_ = nullptr;
      o.n_ = 0;
    }
    return *this;
  }
  ~GpuBuffer() { release(); }
  void* data() const { return p_; }
  size_t size() const { return n_; }
  template <class T> T* as() const { return static_cast<T*>(p_); }
  explicit operator bool() const { return p_ != nullptr; }

 private:
  void release() {
    if (p_ && ctx_) hh_free(ctx_.get(), p_);
    p_ = nullptr;
  }
  CtxPtr ctx_;
  void* p_ = nullptr;
  size_t n_ = 0;
};

// The RoPE table of RopeCache::new (ops.rs:78-138): rows of [sin(half) | cos(half)]
// for positions 0..max_seq, inv_freq = 1 / theta^(2i / rope_dim), host libm in f32.
struct RopeCache {
  int max_seq = 0, rope_dim = 0;
  std::vector<float> table;
  static RopeCache build(int max_seq, int rope_dim, float theta) {
    RopeCache r;
    r.max_seq = max_seq;
    r.rope_dim = rope_dim;
    const int half = rope_dim / 2;
    std::vector<float> inv(half);
    for (int i = 0; i < half; ++i) inv[i] = 1.0f / powf(theta, 2.0f * (float)i / (float)rope_dim);
    r.table.resize((size_t)max_seq * rope_dim);
    for (int p = 0; p < max_seq; ++p)
      for (int i = 0; i < half; ++i) {
        const float f = (float)p * 1.0f * inv[i];
        r.table[(size_t)p * rope_dim + i] = sinf(f);
        r.table[(size_t)p * rope_dim + half + i] = cosf(f);
      }
    return r;
  }
};

// hearth_compute::RopeConfig (lib.rs:911-925): NeoX rotate-half on the first
// rope_dim dims of each head.  The table is the device copy of a RopeCache.
struct RopeConfig {
  int n_heads = 0, head_dim = 0, rope_dim = 0, max_seq = 0;
  const GpuBuffer* table = nullptr;
};

// Decode attention shape (FlashAttnShape, lib.rs:530-540).  The cache is
// [n_kv_heads][max_seq][head_dim] f32 per K and V (kvcache.rs:11-22), and the
// query attends positions 0..seq_len_kv-1.
struct FlashAttnShape {
  int n_heads = 0, n_kv_heads = 0, head_dim = 0, max_seq = 0, seq_len_kv = 0;
};
// Prefill attention shape (PrefillAttnShape, lib.rs:599-612): seq_len_q tokens at
// positions pos0.., each attending 0..pos0+t (causal).  flash: 0 = the
// split/merge kernels (bit-identical per token to the decode operator), 1 = the
// fp32-MFMA flash form.
struct PrefillAttnShape {
  int n_heads = 0, n_kv_heads = 0, head_dim = 0, max_seq = 0, pos0 = 0, seq_len_q = 0, flash = 0;
};

class GpuCompute {
 public:
  // new() -> Option<Self> (lib.rs:126-183): nullopt when the device cannot be opened.
  static std::optional<GpuCompute> create(int device_ordinal = 0) {
    hh_ctx* c = nullptr;
    if (hh_ctx_create(device_ordinal, &c) != HH_OK || !c) return std::nullopt;
    return GpuCompute(CtxPtr(c, [](hh_ctx* p) { hh_ctx_destroy(p); }));
  }
  hh_ctx* raw() const { return ctx_.get(); }
  const CtxPtr& ctx() const { return ctx_; }

  // has_dequant (lib.rs:186-191): every format of this path has a device dot.
  bool has_dequant(QuantKind) const { return true; }

  // create_storage_buffer / upload_f32 / upload_bytes / readback_f32 (lib.rs:226-253)
  std::optional<GpuBuffer> create_storage_buffer(size_t nbytes) const {
    void* p = nullptr;
    if (hh_malloc(raw(), nbytes, &p) != HH_OK) return std::nullopt;
    if (hh_memset(raw(), p, 0, nbytes) != HH_OK) {
      hh_free(raw(), p);
      return std::nullopt;
    }
    return GpuBuffer(ctx_, p, nbytes);
  }
  std::optional<GpuBuffer> upload_bytes(const void* data, size_t nbytes) const {
    auto b = create_storage_buffer(nbytes);
    if (!b || hh_memcpy_h2d(raw(), b->data(), data, nbytes) != HH_OK) return std::nullopt;
    return b;
  }
  std::optional<GpuBuffer> upload_f32(const std::vector<float>& v) const {
    return upload_bytes(v.data(), v.size() * sizeof(float));
  }
  std::vector<float> readback_f32(const GpuBuffer& b, size_t n) const {
    std::vector<float> out(n);
    if (n * sizeof(float) > b.size() || hh_memcpy_d2h(raw(), out.data(), b.data(), n * sizeof(float)) != HH_OK)
      return {};
    return out;
  }
  std::vector<uint8_t> readback_bytes(const GpuBuffer& b, size_t n) const {
    std::vector<uint8_t> out(n);
    if (n > b.size() || hh_memcpy_d2h(raw(), out.data(), b.data(), n) != HH_OK) return {};
    return out;
  }

  // begin_batch / end_batch (lib.rs:206-224): work queues on the context's
  // stream in order; end_batch waits for it.
  void begin_batch() const {}
  bool end_batch() const { return hh_ctx_synchronize(raw()) == HH_OK; }

  // argmax_f32 (lib.rs:338-420): index of the first maximum.
  std::optional<uint32_t> argmax_f32(const GpuBuffer& data, size_t n) const {
    return sample_greedy(data, n, nullptr, 0, 1.0f, 1);
  }
  // The greedy choices of the decode loop: rule 0 is hearth_sampler::sample at
  // temperature 0 (repetition penalty over past, then the last maximum,
  // lib.rs:26-40, :156-207); rule 1 is the qwen35 inline argmax (first
  // maximum, no penalty, qwen35.rs:1735-1745).
  std::optional<uint32_t> sample_greedy(const GpuBuffer& logits, size_t n, const GpuBuffer* past, size_t n_past,
                                        float repeat_pen, int rule) const {
    auto d = create_storage_buffer(sizeof(uint32_t));   // the index is written on the device
    uint32_t idx = 0;
    if (!d || hh_argmax(raw(), logits.as<float>(), (int64_t)n, past ? past->as<uint32_t>() : nullptr,
                        (int64_t)n_past, repeat_pen, rule, d->as<uint32_t>()) != HH_OK ||
        hh_memcpy_d2h(raw(), &idx, d->data(), sizeof idx) != HH_OK)
      return std::nullopt;
    return idx;
  }

  // q8_0::quantize (q8_0.rs:20-51) of n f32 values into n/32 Q8_0 blocks.
  std::optional<GpuBuffer> quantize_q8_0(const GpuBuffer& x, size_t n) const {
    auto out = create_storage_buffer(n / 32 * 34);
    if (!out || hh_quantize_q8_0(raw(), x.as<float>(), (int64_t)n, out->as<uint8_t>()) != HH_OK) return std::nullopt;
    return out;
  }
  // dequantize (quant lib.rs:169-239): n values of a weight row run.
  std::optional<GpuBuffer> dequantize(const GpuBuffer& w, QuantKind kind, size_t n) const {
    auto out = create_storage_buffer(n * sizeof(float));
    if (!out || hh_dequantize(raw(), (int)kind, w.data(), (int64_t)n, out->as<float>()) != HH_OK) return std::nullopt;
    return out;
  }

  // dequant_matmul_fused(quant_buf, kind, x_buf, m, n, k) (lib.rs:483-507): y[m] =
  // W[m x k] . x[k] for one column (n == 1, else None, as the plugin).  x is
  // quantized to Q8_0 and each row is the DotFn dot (see the file comment).
  // The device dots take k in whole 256-value units (every width of this path
  // is); other k are None, as an unsupported shape is for the plugin.
  std::optional<GpuBuffer> dequant_matmul_fused(const GpuBuffer& quant_buf, QuantKind kind, const GpuBuffer& x_buf,
                                                uint32_t m, uint32_t n, uint32_t k) const {
    if (n != 1) return std::nullopt;
    auto xq = quantize_q8_0(x_buf, k);
    if (!xq) return std::nullopt;
    return dot_rows_q8(quant_buf, kind, *xq, m, k);
  }
  // par_dot_rows with a caller-quantized activation (the x_q8 argument of
  // LlamaModel::matmul, matmul.rs:50-58): y[r] = DotFn(w + r * row_bytes, x_q8, k).
  std::optional<GpuBuffer> dot_rows_q8(const GpuBuffer& w, QuantKind kind, const GpuBuffer& x_q8, uint32_t m,
                                       uint32_t k) const {
    auto y = create_storage_buffer((size_t)m * sizeof(float));
    if (!y || hh_gemv_q8(raw(), (int)kind, w.data(), m, k, x_q8.as<uint8_t>(), y->as<float>()) != HH_OK)
      return std::nullopt;
    return y;
  }
  // The batched form (matmul_batch / par_dot_rows_batched, matmul.rs:580-674):
  // seq_len Q8_0 rows of k values, out[s * m + r].
  std::optional<GpuBuffer> dot_rows_q8_batch(const GpuBuffer& w, QuantKind kind, const GpuBuffer& x_q8, uint32_t m,
                                             uint32_t k, uint32_t seq_len) const {
    auto y = create_storage_buffer((size_t)m * seq_len * sizeof(float));
    if (!y || hh_gemm_q8(raw(), (int)kind, w.data(), m, k, x_q8.as<uint8_t>(), seq_len, y->as<float>()) != HH_OK)
      return std::nullopt;
    return y;
  }

  // rms_norm(x_buf, w_buf, out_buf, d, eps) (lib.rs:731-768, ops.rs:8-35) over rows of d.
  bool rms_norm(const GpuBuffer& x, const GpuBuffer& w, const GpuBuffer& out, uint32_t d, float eps,
                uint32_t rows = 1) const {
    return hh_rms_norm(raw(), x.as<float>(), w.as<float>(), eps, rows, d, out.as<float>()) == HH_OK;
  }
  // rope_combined(x_buf, config, pos) (lib.rs:911-963, ops.rs:140-164), in place.
  bool rope_combined(const GpuBuffer& x, const RopeConfig& c, uint32_t pos) const {
    if (!c.table) return false;
    return hh_rope(raw(), x.as<float>(), c.n_heads, c.head_dim, c.rope_dim, c.table->as<float>(), c.max_seq,
                   (int)pos) == HH_OK;
  }
  // flash_attention (lib.rs:530-597; ops.rs:353-406 per q head): [n_heads][head_dim] out.
  std::optional<GpuBuffer> flash_attention(const GpuBuffer& q, const GpuBuffer& k_cache, const GpuBuffer& v_cache,
                                           const FlashAttnShape& s) const {
    auto out = create_storage_buffer((size_t)s.n_heads * s.head_dim * sizeof(float));
    if (!out || hh_attention(raw(), q.as<float>(), k_cache.as<float>(), v_cache.as<float>(), s.n_heads,
                             s.n_kv_heads, s.head_dim, s.max_seq, s.seq_len_kv, out->as<float>()) != HH_OK)
      return std::nullopt;
    return out;
  }
  // flash_attention_prefill (lib.rs:599-668; mod.rs:1101-1140): [seq_len_q][n_heads][head_dim] out.
  std::optional<GpuBuffer> flash_attention_prefill(const GpuBuffer& q, const GpuBuffer& k_cache,
                                                   const GpuBuffer& v_cache, const PrefillAttnShape& s) const {
    auto out = create_storage_buffer((size_t)s.seq_len_q * s.n_heads * s.head_dim * sizeof(float));
    if (!out || hh_attention_prefill(raw(), q.as<float>(), k_cache.as<float>(), v_cache.as<float>(), s.n_heads,
                                     s.n_kv_heads, s.head_dim, s.max_seq, s.pos0, s.seq_len_q, s.flash,
                                     out->as<float>()) != HH_OK)
      return std::nullopt;
    return out;
  }

 private:
  explicit GpuCompute(CtxPtr c) : ctx_(std::move(c)) {}
  CtxPtr ctx_;
};

// ---------------------------------------------------------------- Model
// hearth_core::SamplerConfig (core/sampler.rs:2-24) restricted to this path:
// greedy decoding (temperature 0), repeat_pen applied by the dense rule.
struct SamplerConfig {
  float repeat_pen = 1.1f;
};

// What generate() returns: the new token ids and the device clock of the two
// phases (the prompt phase includes the step that yields the first new token).
struct Generation {
  std::vector<uint32_t> tokens;
  double prefill_ms = 0.0, decode_ms = 0.0;
};

// ModelConfig::from_gguf (config.rs:57-217, qwen35.rs:470-530) with the KV
// context cap of kv_budget.rs:19-58 (ctx_cap_override > 0 replaces it).
inline Result<hh_model_config> read_config(const std::string& path, int ctx_cap_override = 0) {
  hh_gguf* g = nullptr;
  if (hh_gguf_open(path.c_str(), &g) != HH_OK) return Result<hh_model_config>::err(last_error("open"));
  hh_model_config c{};
  const int rc = hh_gguf_model_config(g, ctx_cap_override, &c);
  std::string e = rc != HH_OK ? last_error("config") : std::string();
  hh_gguf_close(g);
  if (rc != HH_OK) return Result<hh_model_config>::err(e);
  return Result<hh_model_config>::ok(c);
}

class Model {
 public:
  Model(Model&&) = default;
  Model& operator=(Model&&) = default;

  // LlamaModel::load (mod.rs:103-150) of a GGUF file onto the device.
  static Result<Model> load(const GpuCompute& gpu, const std::string& path, int ctx_cap_override = 0) {
    hh_model* m = nullptr;
    if (hh_model_load_gguf(gpu.raw(), path.c_str(), ctx_cap_override, &m) != HH_OK)
      return Result<Model>::err(last_error("load"));
    return Result<Model>::ok(Model(gpu.ctx(), m));
  }
  // A model of the given geometry with every tensor allocated (weights to be
  // uploaded or synthesized).
  static Result<Model> create(const GpuCompute& gpu, const hh_model_config& cfg) {
    hh_model* m = nullptr;
    if (hh_model_create(gpu.raw(), &cfg, &m) != HH_OK) return Result<Model>::err(last_error("create"));
    return Result<Model>::ok(Model(gpu.ctx(), m));
  }
  hh_model* raw() const { return m_.get(); }

  Status upload_tensor(const std::string& name, QuantKind kind, int64_t n_cols, int64_t n_rows, const void* bytes,
                       size_t nbytes) {
    return check(hh_model_upload_tensor(raw(), name.c_str(), (int)kind, n_cols, n_rows, bytes, nbytes), "upload");
  }
  Status upload_f32(const std::string& name, int64_t n, const float* v) {
    return check(hh_model_upload_tensor(raw(), name.c_str(), HH_F32, n, 1, v, (size_t)n * sizeof(float)), "upload");
  }
  Status synthesize(uint64_t seed) { return check(hh_model_synthesize(raw(), seed), "synthesize"); }
  Status reset() { return check(hh_model_reset(raw()), "reset"); }
  // The per-layer cancel flag (mod.rs:461): the next step fails with "Cancelled".
  Status set_cancel(bool cancel) { return check(hh_model_set_cancel(raw(), cancel ? 1 : 0), "cancel"); }

  // forward (mod.rs:451-860 / qwen35.rs:1028-1236): token at pos, the vocab logits.
  Result<std::vector<float>> forward(uint32_t token, int pos, int vocab) {
    std::vector<float> logits((size_t)vocab);
    if (hh_model_forward(raw(), token, pos, logits.data(), nullptr) != HH_OK)
      return Result<std::vector<float>>::err(last_error("forward"));
    return Result<std::vector<float>>::ok(std::move(logits));
  }
  // forward_batch (mod.rs:899-1221): K/V (and GDN state) of tokens at start_pos.., no logits.
  Status prefill(const std::vector<uint32_t>& tokens, int start_pos) {
    return check(hh_model_prefill(raw(), tokens.data(), (int)tokens.size(), start_pos), "prefill");
  }
  // generate_text's token loop (mod.rs:2718-3012 / qwen35.rs:1654-1804): the
  // prompt from start_pos, then max_new_tokens greedy tokens.
  Result<Generation> generate(const std::vector<uint32_t>& prompt, size_t max_new_tokens, const SamplerConfig& sc,
                              int start_pos = 0) {
    Generation g;
    g.tokens.resize(max_new_tokens);
    if (hh_model_generate(raw(), prompt.data(), (int)prompt.size(), start_pos, (int)max_new_tokens, sc.repeat_pen,
                          g.tokens.data(), nullptr) != HH_OK)
      return Result<Generation>::err(last_error("generate"));
    hh_model_last_prefill_ms(raw(), &g.prefill_ms);
    hh_model_last_decode_ms(raw(), &g.decode_ms);
    return Result<Generation>::ok(std::move(g));
  }

 private:
  Model(CtxPtr ctx, hh_model* m) : ctx_(std::move(ctx)), m_(m, [](hh_model* p) { hh_model_destroy(p); }) {}
  CtxPtr ctx_;   // held so the context outlives the model
  std::unique_ptr<hh_model, void (*)(hh_model*)> m_{nullptr, [](hh_model*) {}};
};

}  // namespace hearth
