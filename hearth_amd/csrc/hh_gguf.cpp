// hh_gguf.cpp — GGUF v2/v3 reader and model loader (host side of the C ABI).
//
// Restates the reference's loading path for the decode model:
//   GgufFile::open            hearth-gguf gguf.rs:138-218 (header, metadata, tensor table,
//                             v3 data-section alignment)
//   MetaValue::as_*           hearth-gguf meta.rs:26-64
//   GgmlDType block table     hearth-gguf ggml.rs:57-171 (tensor byte sizes)
//   ModelConfig::from_gguf    hearth-llm config.rs:57-217 (+ arch prefixes :288-307)
//   qwen35 GDN geometry       hearth-llm model/qwen35.rs:470-530
//   KV context cap            hearth-llm model/kv_budget.rs:19-58
//   tied LM head              hearth-llm model/mod.rs:360-364
// The file is memory-mapped; tensors are uploaded straight from the mapping
// in their native block layout (model/gpu.rs:8-50), so no host copy is made
// of a quantized weight.
#include <errno.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/hearth_hip.h"
#include "hh_host.h"

namespace {

// One metadata value (meta.rs MetaValue): scalar kinds keep their GGUF type id.
struct Meta {
  uint32_t type = 0;
  uint64_t u = 0;       // U8/U16/U32/U64/Bool (zero-extended)
  int64_t i = 0;        // I8/I16/I32/I64 (sign-extended)
  double f = 0.0;       // F32/F64
  std::string s;        // String
  uint32_t elem = 0;    // Array element type
  std::vector<Meta> items;
};

enum : uint32_t {
  GT_U8 = 0, GT_I8 = 1, GT_U16 = 2, GT_I16 = 3, GT_U32 = 4, GT_I32 = 5, GT_F32 = 6, GT_BOOL = 7,
  GT_STRING = 8, GT_ARRAY = 9, GT_U64 = 10, GT_I64 = 11, GT_F64 = 12
};

struct TInfo {
  std::string name;
  std::vector<uint64_t> shape;   // ne0 (fastest) first
  uint32_t type;
  uint64_t offset;               // from the start of the data section
  uint64_t nbytes;
};

// Elements per block and bytes per block of a ggml type id (ggml.rs:57-171);
// false for an id the reference does not know.
bool block_of(uint32_t id, uint64_t* el, uint64_t* by) {
  struct E { uint32_t id; uint32_t el, by; };
  static const E t[] = {
      {0, 1, 4},     {1, 1, 2},      {2, 32, 18},   {3, 32, 20},   {6, 32, 22},   {7, 32, 24},
      {8, 32, 34},   {9, 32, 40},    {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
      {14, 256, 210}, {15, 256, 272}, {16, 256, 66}, {17, 256, 74},  {18, 256, 98},  {19, 256, 50},
      {20, 32, 84},  {21, 256, 110}, {22, 256, 82}, {23, 256, 290}, {24, 1, 1},     {25, 1, 2},
      {26, 1, 4},    {27, 1, 8},     {28, 1, 8},    {29, 256, 54},  {30, 1, 2},     {31, 32, 18},
      {32, 32, 18},  {33, 32, 18},   {34, 32, 34},  {35, 32, 34},   {36, 32, 84},   {37, 32, 84},
      {38, 32, 84},  {39, 128, 18},  {41, 128, 18}, {42, 128, 34},  {43, 128, 18},  {142, 128, 34},
      {143, 128, 28},
  };
  for (const E& e : t)
    if (e.id == id) {
      *el = e.el;
      *by = e.by;
      return true;
    }
  return false;
}

// qwen35.rs:189-201 meta_int: any integer kind
bool meta_int(const Meta& m, int64_t* v) {
  switch (m.type) {
    case GT_U8: case GT_U16: case GT_U32: case GT_U64: *v = (int64_t)m.u; return true;
    case GT_I8: case GT_I16: case GT_I32: case GT_I64: *v = m.i; return true;
  }
  return false;
}

struct Reader {
  const uint8_t* p;
  size_t n, pos = 0;
  bool eof = false;
  bool need(size_t k) {
    if (eof || pos + k > n || pos + k < pos) { eof = true; return false; }
    return true;
  }
  template <typename T> T get() {
    T v{};
    if (!need(sizeof(T))) return v;
    memcpy(&v, p + pos, sizeof(T));   // GGUF is little-endian, as is the host
    pos += sizeof(T);
    return v;
  }
  std::string str() {
    uint64_t len = get<uint64_t>();
    if (!need(len)) return std::string();
    std::string s((const char*)p + pos, (size_t)len);
    pos += len;
    return s;
  }
};

bool read_value(Reader& r, uint32_t type, Meta& m, int depth) {
  m.type = type;
  switch (type) {
    case GT_U8: m.u = r.get<uint8_t>(); break;
    case GT_I8: m.i = r.get<int8_t>(); break;
    case GT_U16: m.u = r.get<uint16_t>(); break;
    case GT_I16: m.i = r.get<int16_t>(); break;
    case GT_U32: m.u = r.get<uint32_t>(); break;
    case GT_I32: m.i = r.get<int32_t>(); break;
    case GT_F32: m.f = r.get<float>(); break;
    case GT_BOOL: m.u = r.get<uint8_t>() != 0; break;
    case GT_STRING: m.s = r.str(); break;
    case GT_U64: m.u = r.get<uint64_t>(); break;
    case GT_I64: m.i = r.get<int64_t>(); break;
    case GT_F64: m.f = r.get<double>(); break;
    case GT_ARRAY: {
      if (depth > 4) return false;
      m.elem = r.get<uint32_t>();
      uint64_t count = r.get<uint64_t>();
      if (r.eof || count > r.n) return false;   // every element takes at least one byte
      m.items.resize((size_t)count);
      for (uint64_t k = 0; k < count; ++k)
        if (!read_value(r, m.elem, m.items[(size_t)k], depth + 1)) return false;
      break;
    }
    default:
      // gguf.rs:125 keeps an unknown type as a placeholder string without
      // consuming bytes; the parse of what follows then fails or misreads, so
      // it is refused here outright.
      return false;
  }
  return !r.eof;
}

}  // namespace

struct hh_gguf {
  void* map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint64_t data_offset = 0, alignment = 32;
  std::map<std::string, Meta> meta;
  std::vector<TInfo> tensors;
  std::map<std::string, int> by_name;
  ~hh_gguf() {
    if (map) munmap(map, size);
  }
  const uint8_t* base() const { return (const uint8_t*)map; }
  const Meta* find(const std::string& k) const {
    auto it = meta.find(k);
    return it == meta.end() ? nullptr : &it->second;
  }
  // MetaValue::as_u32 / as_f32 / as_u64 / as_bool / as_str (meta.rs:26-64)
  bool u32(const std::string& k, uint32_t* v) const {
    const Meta* m = find(k);
    if (!m) return false;
    if (m->type == GT_U32) { *v = (uint32_t)m->u; return true; }
    if (m->type == GT_I32) { *v = (uint32_t)m->i; return true; }
    return false;
  }
  bool f32(const std::string& k, float* v) const {
    const Meta* m = find(k);
    if (!m || m->type != GT_F32) return false;
    *v = (float)m->f;
    return true;
  }
  bool str(const std::string& k, std::string* v) const {
    const Meta* m = find(k);
    if (!m || m->type != GT_STRING) return false;
    *v = m->s;
    return true;
  }
  bool arr_len(const std::string& k, uint64_t* n) const {
    const Meta* m = find(k);
    if (!m || m->type != GT_ARRAY) return false;
    *n = m->items.size();
    return true;
  }
  const TInfo* tensor(const std::string& name) const {
    auto it = by_name.find(name);
    return it == by_name.end() ? nullptr : &tensors[(size_t)it->second];
  }
};

namespace {

int parse(hh_gguf* g) {
  Reader r{g->base(), g->size};
  if (g->size < 4) return hh_set_error(HH_ERR_INVALID, "GGUF: file too small");
  if (memcmp(g->base(), "GGUF", 4) != 0) {
    char b[64];
    snprintf(b, sizeof b, "GGUF: invalid magic %02x %02x %02x %02x", g->base()[0], g->base()[1], g->base()[2],
             g->base()[3]);
    return hh_set_error(HH_ERR_INVALID, b);
  }
  r.pos = 4;
  g->version = r.get<uint32_t>();
  if (!r.eof && g->version != 2 && g->version != 3)
    return hh_set_error(HH_ERR_INVALID, "GGUF: unsupported version " + std::to_string(g->version));
  uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
  if (r.eof) return hh_set_error(HH_ERR_INVALID, "GGUF: unexpected end of file in the header");
  if (n_tensors > g->size || n_kv > g->size) return hh_set_error(HH_ERR_INVALID, "GGUF: implausible counts");
  for (uint64_t k = 0; k < n_kv; ++k) {
    std::string key = r.str();
    uint32_t type = r.get<uint32_t>();
    Meta m;
    if (r.eof || !read_value(r, type, m, 0))
      return hh_set_error(HH_ERR_INVALID, "GGUF: bad metadata value for key '" + key + "' at offset " +
                                              std::to_string(r.pos));
    g->meta[key] = std::move(m);
  }
  uint32_t al = 0;
  if (g->u32("general.alignment", &al) && al > 0) g->alignment = al;   // gguf.rs:165-169
  for (uint64_t k = 0; k < n_tensors; ++k) {
    TInfo t;
    t.name = r.str();
    uint32_t nd = r.get<uint32_t>();
    if (r.eof || nd > 8) return hh_set_error(HH_ERR_INVALID, "GGUF: bad tensor record " + std::to_string(k));
    uint64_t el = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      uint64_t v = r.get<uint64_t>();
      t.shape.push_back(v);
      el *= v;
    }
    t.type = r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    if (r.eof) return hh_set_error(HH_ERR_INVALID, "GGUF: unexpected end of file in the tensor table");
    uint64_t bel, bby;
    if (!block_of(t.type, &bel, &bby))
      return hh_set_error(HH_ERR_DTYPE,
                          "GGUF: unknown dtype id " + std::to_string(t.type) + " for tensor " + t.name);
    t.nbytes = (el + bel - 1) / bel * bby;   // ggml.rs:166-169 byte_size
    g->by_name[t.name] = (int)g->tensors.size();
    g->tensors.push_back(std::move(t));
  }
  uint64_t pos = r.pos;
  if (g->version == 3) pos += (g->alignment - pos % g->alignment) % g->alignment;   // gguf.rs:199-205
  g->data_offset = pos;
  for (const TInfo& t : g->tensors)
    if (g->data_offset + t.offset + t.nbytes > g->size || g->data_offset + t.offset < g->data_offset)
      return hh_set_error(HH_ERR_INVALID, "GGUF: tensor " + t.name + " extends past the end of the file");
  return HH_OK;
}

// config.rs:288-307: the key prefixes tried in order, then "llama."
void prefixes_of(const std::string& arch, std::string out[2]) {
  out[1] = arch;
  if (arch == "llama" || arch == "mistral" || arch == "mixtral" || arch == "gemma") out[0] = "llama";
  else if (arch == "qwen2" || arch == "qwen2.5") out[0] = "qwen2";
  else if (arch == "qwen3" || arch == "qwen3moe" || arch == "qwen3next" || arch == "qwen35" || arch == "qwen35moe")
    out[0] = "qwen3";
  else if (arch == "phi3" || arch == "phi-3") out[0] = "phi3";
  else if (arch == "starcoder2") out[0] = "starcoder2";
  else if (arch == "gemma2") out[0] = "gemma";
  else if (arch == "command-r") out[0] = "command-r";
  else if (arch == "dbrx") out[0] = "dbrx";
  else if (arch == "falcon") out[0] = "falcon";
  else if (arch == "yi") out[0] = "yi";
  else if (arch == "deepseek2") out[0] = "deepseek2";
  else out[0] = "llama";
}

// kv_budget.rs:19-58: the context allocated for a model declaring `declared`.
int ctx_cap(uint64_t declared, uint64_t n_kv_layers, uint64_t n_kv_heads, uint64_t hd, bool dense, int cap_override) {
  const uint64_t budget = 1280ull << 20, min_ctx = 512, dense_cap = 4096;
  uint64_t per_token = 2 * n_kv_layers * n_kv_heads * hd * 4;
  if (per_token == 0) per_token = 1;
  uint64_t by_budget = budget / per_token;
  if (by_budget < min_ctx) by_budget = min_ctx;
  uint64_t def = dense ? (dense_cap < by_budget ? dense_cap : by_budget) : by_budget;
  uint64_t cap = cap_override > 0 ? (uint64_t)cap_override : def;
  return (int)(declared < cap ? declared : cap);
}

// The Hadamard fold metadata of a qwen35 file (qwen35.rs:532-620), with the
// reference loader's checks and messages: block size (0 = unfolded), version 1
// or 2, the normalized Sylvester transform, sign vectors by width (each width a
// multiple of the block, values +-1, the widths covering sign_values exactly),
// a latent token_embd when inverse_weight_names lists it, and the tied-output
// invariants (version 2, no output.weight, latent token_embd).
int hadamard_meta(const hh_gguf* g, hh_model_config* c, std::vector<std::pair<int, std::vector<float>>>* signs) {
  uint32_t hb = 0, ver = 0;
  g->u32("prism.hadamard.block_size", &hb);
  g->u32("prism.hadamard.version", &ver);
  const Meta* tied_m = g->find("prism.hadamard.tied_output");
  const bool tied = tied_m && tied_m->type == GT_BOOL && tied_m->u != 0;
  bool latent = false;
  c->had_block = 0;
  c->had_flags = 0;
  if (hb > 0) {
    if (ver != 1 && ver != 2)
      return hh_set_error(HH_ERR_INVALID, "qwen35: unsupported prism.hadamard.version " + std::to_string(ver));
    std::string tr;
    g->str("prism.hadamard.transform", &tr);
    if (tr != "normalized-sylvester-walsh-hadamard")
      return hh_set_error(HH_ERR_INVALID, "qwen35: unsupported hadamard transform " + tr);
    const Meta* wm = g->find("prism.hadamard.sign_widths");
    if (!wm || wm->type != GT_ARRAY) return hh_set_error(HH_ERR_INVALID, "qwen35: missing prism.hadamard.sign_widths");
    const Meta* vm = g->find("prism.hadamard.sign_values");
    if (!vm || vm->type != GT_ARRAY) return hh_set_error(HH_ERR_INVALID, "qwen35: missing prism.hadamard.sign_values");
    size_t off = 0;
    for (const Meta& w : wm->items) {
      int64_t width = 0;
      if (!meta_int(w, &width)) return hh_set_error(HH_ERR_INVALID, "qwen35: bad sign width");
      if (width <= 0 || width % hb || off + (size_t)width > vm->items.size())
        return hh_set_error(HH_ERR_INVALID, "qwen35: invalid hadamard sign width " + std::to_string(width));
      std::vector<float> v((size_t)width);
      for (int64_t k = 0; k < width; ++k) {
        int64_t x = 0;
        meta_int(vm->items[off + (size_t)k], &x);
        if (x != 1 && x != -1) return hh_set_error(HH_ERR_INVALID, "qwen35: hadamard sign values must be +/-1");
        v[(size_t)k] = (float)x;
      }
      off += (size_t)width;
      signs->push_back({(int)width, std::move(v)});
    }
    if (off != vm->items.size()) return hh_set_error(HH_ERR_INVALID, "qwen35: hadamard sign_values length mismatch");
    const Meta* inv = g->find("prism.hadamard.inverse_weight_names");
    if (inv && inv->type == GT_ARRAY)
      for (const Meta& n : inv->items) latent = latent || (n.type == GT_STRING && n.s == "token_embd.weight");
  }
  if (tied) {
    if (ver != 2 || hb == 0) return hh_set_error(HH_ERR_INVALID, "qwen35: tied output requires prism.hadamard version 2");
    if (g->tensor("output.weight"))
      return hh_set_error(HH_ERR_INVALID, "qwen35: prism.hadamard.tied_output requires output.weight to be absent");
    if (!latent) return hh_set_error(HH_ERR_INVALID, "qwen35: prism.hadamard.tied_output requires a latent token_embd");
  }
  c->had_block = (int)hb;
  c->had_flags = (latent ? HH_HAD_LATENT_EMBD : 0) | (tied ? HH_HAD_TIED_OUTPUT : 0);
  return HH_OK;
}

int model_config(const hh_gguf* g, int cap_override, hh_model_config* c) {
  std::string arch;
  if (!g->str("general.architecture", &arch)) return hh_set_error(HH_ERR_INVALID, "Missing general.architecture");
  std::string pf[2];
  prefixes_of(arch, pf);
  auto pu32 = [&](const char* key, uint32_t* v) {
    for (const std::string& p : pf)
      if (g->u32(p + "." + key, v)) return true;
    return g->u32(std::string("llama.") + key, v);
  };
  auto pf32 = [&](const char* key, float* v) {
    for (const std::string& p : pf)
      if (g->f32(p + "." + key, v)) return true;
    return g->f32(std::string("llama.") + key, v);
  };
  memset(c, 0, sizeof *c);
  const bool hybrid = arch == "qwen35";
  const bool dense = arch == "llama" || arch == "qwen3" || arch == "qwen2" || arch == "mistral";
  if (!hybrid && !dense)
    return hh_set_error(HH_ERR_DTYPE, "GGUF: architecture '" + arch + "' is not on the decode path");
  c->arch = hybrid ? 1 : 0;
  uint32_t v = 0;
  if (!pu32("embedding_length", &v)) return hh_set_error(HH_ERR_INVALID, "Missing embedding_length");
  c->d_model = (int)v;
  if (!pu32("block_count", &v)) return hh_set_error(HH_ERR_INVALID, "Missing block_count");
  c->n_layers = (int)v;
  if (!pu32("attention.head_count", &v)) return hh_set_error(HH_ERR_INVALID, "Missing head_count");
  c->n_heads = (int)v;
  c->n_kv_heads = pu32("attention.head_count_kv", &v) ? (int)v : c->n_heads;
  bool explicit_hd = pu32("attention.head_dim", &v) || pu32("attention.key_length", &v) ||
                     pu32("attention.value_length", &v);
  if (c->n_heads <= 0 || c->n_kv_heads <= 0 || c->d_model <= 0 || c->n_layers <= 0)
    return hh_set_error(HH_ERR_INVALID, "Config validation: zero dimension");
  c->head_dim = explicit_hd ? (int)v : c->d_model / c->n_heads;
  c->d_ffn = pu32("feed_forward_length", &v) ? (int)v : 4 * c->d_model;
  uint64_t nv = 0;
  if (g->u32("tokenizer.ggml.tokens", &v) || g->u32("llama.vocab_size", &v)) c->vocab = (int)v;
  else if (g->arr_len("tokenizer.ggml.tokens", &nv)) c->vocab = (int)nv;
  else return hh_set_error(HH_ERR_INVALID, "Missing vocab_size");
  uint32_t declared = pu32("context_length", &v) ? v : 2048;
  float f = 0.0f;
  c->rope_theta = pf32("rope.freq_base", &f) ? f : 10000.0f;
  c->eps = pf32("attention.layer_norm_rms_epsilon", &f) ? f : 1e-5f;

  const TInfo* q = g->tensor("blk.0.attn_q.weight");
  if (!hybrid) {
    // mod.rs:156-167: head_dim from the Q projection unless stated
    if (!explicit_hd && q && q->shape.size() == 2) {
      uint64_t rows = q->shape[1];
      if (rows % (uint64_t)c->n_heads == 0) c->head_dim = (int)(rows / (uint64_t)c->n_heads);
    }
    c->qk_norm = g->tensor("blk.0.attn_q_norm.weight") != nullptr;
  } else {
    // qwen35.rs:475-488: head_dim from the first attention layer's K rows
    for (int i = 0; i < c->n_layers; ++i) {
      const TInfo* k = g->tensor("blk." + std::to_string(i) + ".attn_k.weight");
      if (k) {
        if (k->shape.size() == 2 && k->shape[1] % (uint64_t)c->n_kv_heads == 0 && k->shape[1] / c->n_kv_heads > 0)
          c->head_dim = (int)(k->shape[1] / (uint64_t)c->n_kv_heads);
        break;
      }
    }
    uint32_t state = 0, groups = 0, rank = 0, kernel = 0, inner = 0, interval = 4;
    if (!g->u32("qwen35.ssm.state_size", &state)) return hh_set_error(HH_ERR_INVALID, "qwen35: missing qwen35.ssm.state_size");
    if (!g->u32("qwen35.ssm.group_count", &groups)) return hh_set_error(HH_ERR_INVALID, "qwen35: missing qwen35.ssm.group_count");
    if (!g->u32("qwen35.ssm.time_step_rank", &rank)) return hh_set_error(HH_ERR_INVALID, "qwen35: missing qwen35.ssm.time_step_rank");
    if (!g->u32("qwen35.ssm.conv_kernel", &kernel)) return hh_set_error(HH_ERR_INVALID, "qwen35: missing qwen35.ssm.conv_kernel");
    if (g->u32("qwen35.ssm.inner_size", &inner) && inner != state * rank)
      return hh_set_error(HH_ERR_INVALID, "qwen35: ssm.inner_size " + std::to_string(inner) +
                                              " != state_size*time_step_rank " + std::to_string(state * rank));
    // config.rs:179-196 / qwen35.rs:520-528: full attention iff (i+1) % interval == 0
    if (g->find("qwen35.attention.recurrent_layers"))
      return hh_set_error(HH_ERR_INVALID, "qwen35: explicit recurrent_layers lists are not supported; "
                                          "the decode path takes the full_attention_interval pattern");
    if (!g->u32(pf[0] + ".full_attention_interval", &interval)) g->u32("qwen35.full_attention_interval", &interval);
    if (interval == 0) return hh_set_error(HH_ERR_INVALID, "qwen35: full_attention_interval is 0");
    c->full_attn_interval = (int)interval;
    c->ssm_head_dim = (int)state;
    c->ssm_n_k_heads = (int)groups;
    c->ssm_n_v_heads = (int)rank;
    c->ssm_conv_kernel = (int)kernel;
    c->attn_out_gate = 1;
    std::vector<std::pair<int, std::vector<float>>> signs;
    int rc = hadamard_meta(g, c, &signs);
    if (rc != HH_OK) return rc;
    for (int i = 0; i < c->n_layers; ++i)
      if ((i + 1) % c->full_attn_interval == 0) {
        c->qk_norm = g->tensor("blk." + std::to_string(i) + ".attn_q_norm.weight") != nullptr;
        break;
      }
  }
  c->rope_dim = pu32("rope.dimension_count", &v) ? (int)v : c->head_dim;

  // weight formats: every layer matmul shares one type; embedding/head Q8_0
  const TInfo* emb = g->tensor("token_embd.weight");
  if (!emb) return hh_set_error(HH_ERR_NOT_FOUND, "Missing token_embd.weight");
  c->head_type = (int)emb->type;
  const TInfo* out = g->tensor("output.weight");
  if (out && out->type != emb->type)
    return hh_set_error(HH_ERR_DTYPE, "GGUF: output.weight and token_embd.weight differ in type");
  const TInfo* w0 = g->tensor("blk.0.ffn_gate.weight");
  if (!w0) return hh_set_error(HH_ERR_NOT_FOUND, "Missing blk.0.ffn_gate.weight");
  c->wtype = (int)w0->type;
  if (c->wtype == 39) c->wtype = HH_Q1_0_G128;   // ggml.rs:97 legacy id

  uint64_t n_kv_layers = 0;
  for (int i = 0; i < c->n_layers; ++i)
    if (!hybrid || (i + 1) % c->full_attn_interval == 0) ++n_kv_layers;
  c->max_seq = ctx_cap(declared, n_kv_layers, (uint64_t)c->n_kv_heads, (uint64_t)c->head_dim, !hybrid, cap_override);
  if (c->eps <= 0.0f || c->rope_theta <= 0.0f) return hh_set_error(HH_ERR_INVALID, "Config validation: eps/theta");
  if (c->n_heads % c->n_kv_heads != 0)
    return hh_set_error(HH_ERR_INVALID, "Config validation: n_heads not divisible by n_kv_heads");
  return HH_OK;
}

}  // namespace

extern "C" {

int hh_gguf_open(const char* path, hh_gguf** out) {
  if (!path || !out) return hh_set_error(HH_ERR_INVALID, "null argument");
  *out = nullptr;
  int fd = open(path, O_RDONLY);
  if (fd < 0) return hh_set_error(HH_ERR_NOT_FOUND, std::string("GGUF: cannot open ") + path + ": " + strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return hh_set_error(HH_ERR_INVALID, std::string("GGUF: cannot stat ") + path);
  }
  std::unique_ptr<hh_gguf> g(new hh_gguf);
  g->size = (size_t)st.st_size;
  if (g->size > 0) {
    g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (g->map == MAP_FAILED) {
      g->map = nullptr;
      close(fd);
      return hh_set_error(HH_ERR_INVALID, std::string("GGUF: mmap failed: ") + strerror(errno));
    }
  }
  close(fd);
  if (!g->map) return hh_set_error(HH_ERR_INVALID, "GGUF: file too small");   // zero-length file
  int rc = parse(g.get());
  if (rc != HH_OK) return rc;
  *out = g.release();
  return HH_OK;
}

int hh_gguf_close(hh_gguf* g) {
  delete g;
  return HH_OK;
}

int hh_gguf_header(hh_gguf* g, uint32_t* version, uint64_t* data_offset, uint64_t* alignment) {
  if (!g) return hh_set_error(HH_ERR_INVALID, "null argument");
  if (version) *version = g->version;
  if (data_offset) *data_offset = g->data_offset;
  if (alignment) *alignment = g->alignment;
  return HH_OK;
}

int hh_gguf_tensor_count(hh_gguf* g) { return g ? (int)g->tensors.size() : -1; }

int hh_gguf_tensor_info(hh_gguf* g, int index, const char** name, int* ggml_type, int* n_dims, int64_t* shape4,
                        uint64_t* offset, uint64_t* nbytes) {
  if (!g) return hh_set_error(HH_ERR_INVALID, "null argument");
  if (index < 0 || index >= (int)g->tensors.size()) return hh_set_error(HH_ERR_RANGE, "tensor index out of range");
  const TInfo& t = g->tensors[(size_t)index];
  if (name) *name = t.name.c_str();
  if (ggml_type) *ggml_type = (int)t.type;
  if (n_dims) *n_dims = (int)t.shape.size();
  if (shape4)
    for (int d = 0; d < 4; ++d) shape4[d] = d < (int)t.shape.size() ? (int64_t)t.shape[(size_t)d] : 1;
  if (offset) *offset = t.offset;
  if (nbytes) *nbytes = t.nbytes;
  return HH_OK;
}

int hh_gguf_meta_u32(hh_gguf* g, const char* key, uint32_t* out) {
  if (!g || !key || !out) return hh_set_error(HH_ERR_INVALID, "null argument");
  if (!g->u32(key, out)) return hh_set_error(HH_ERR_NOT_FOUND, std::string("no u32 metadata ") + key);
  return HH_OK;
}

int hh_gguf_meta_f32(hh_gguf* g, const char* key, float* out) {
  if (!g || !key || !out) return hh_set_error(HH_ERR_INVALID, "null argument");
  if (!g->f32(key, out)) return hh_set_error(HH_ERR_NOT_FOUND, std::string("no f32 metadata ") + key);
  return HH_OK;
}

int hh_gguf_meta_str(hh_gguf* g, const char* key, const char** out) {
  if (!g || !key || !out) return hh_set_error(HH_ERR_INVALID, "null argument");
  const Meta* m = g->find(key);
  if (!m || m->type != GT_STRING) return hh_set_error(HH_ERR_NOT_FOUND, std::string("no string metadata ") + key);
  *out = m->s.c_str();
  return HH_OK;
}

int hh_gguf_meta_array_len(hh_gguf* g, const char* key, uint64_t* out) {
  if (!g || !key || !out) return hh_set_error(HH_ERR_INVALID, "null argument");
  if (!g->arr_len(key, out)) return hh_set_error(HH_ERR_NOT_FOUND, std::string("no array metadata ") + key);
  return HH_OK;
}

int hh_gguf_model_config(hh_gguf* g, int ctx_cap_override, hh_model_config* cfg) {
  if (!g || !cfg) return hh_set_error(HH_ERR_INVALID, "null argument");
  return model_config(g, ctx_cap_override, cfg);
}

int hh_gguf_tensor_data(hh_gguf* g, int index, const void** data) {
  if (!g || !data) return hh_set_error(HH_ERR_INVALID, "null argument");
  if (index < 0 || index >= (int)g->tensors.size()) return hh_set_error(HH_ERR_RANGE, "tensor index out of range");
  *data = g->base() + g->data_offset + g->tensors[(size_t)index].offset;
  return HH_OK;
}

int hh_model_load_gguf(hh_ctx* ctx, const char* path, int ctx_cap_override, hh_model** out) {
  if (!ctx || !path || !out) return hh_set_error(HH_ERR_INVALID, "null argument");
  *out = nullptr;
  hh_gguf* g = nullptr;
  int rc = hh_gguf_open(path, &g);
  if (rc != HH_OK) return rc;
  std::unique_ptr<hh_gguf> hold(g);
  hh_model_config cfg;
  rc = model_config(g, ctx_cap_override, &cfg);
  if (rc != HH_OK) return rc;
  hh_model* m = nullptr;
  rc = hh_model_create(ctx, &cfg, &m);
  if (rc != HH_OK) return rc;
  if (cfg.had_block > 0) {
    std::vector<std::pair<int, std::vector<float>>> signs;
    hh_model_config tmp = cfg;
    hadamard_meta(g, &tmp, &signs);
    for (auto& sv : signs) {
      rc = hh_model_set_hadamard_signs(m, sv.first, sv.second.data());
      if (rc != HH_OK) {
        std::string msg = hh_last_error();
        hh_model_destroy(m);
        return hh_set_error(rc, msg);
      }
    }
  }
  // every tensor the model holds must come from the file (a tied LM head
  // reads token_embd, mod.rs:360-364); extra tensors in the file are ignored
  const int n = hh_model_tensor_count(m);
  std::vector<float> conv;
  for (int i = 0; i < n; ++i) {
    const char* name = nullptr;
    int type = 0;
    int64_t ne0 = 0, ne1 = 0;
    size_t nbytes = 0;
    hh_model_tensor_info(m, i, &name, &type, &ne0, &ne1, &nbytes);
    std::string src = name;
    const TInfo* t = g->tensor(src);
    if (!t && src == "output.weight") t = g->tensor("token_embd.weight");
    if (!t) {
      hh_model_destroy(m);
      return hh_set_error(HH_ERR_NOT_FOUND, "GGUF: missing tensor " + src);
    }
    uint64_t el = 1;
    for (uint64_t d : t->shape) el *= d;
    uint64_t rows = t->shape.size() >= 2 ? el / t->shape[0] : 1;
    uint64_t cols = t->shape.empty() ? 1 : t->shape[0];
    if (cols != (uint64_t)ne0 || rows != (uint64_t)ne1) {
      hh_model_destroy(m);
      return hh_set_error(HH_ERR_DIM, "GGUF: tensor " + src + " is " + std::to_string(cols) + " x " +
                                          std::to_string(rows) + ", the model expects " + std::to_string(ne0) +
                                          " x " + std::to_string(ne1));
    }
    const void* bytes = g->base() + g->data_offset + t->offset;
    size_t len = (size_t)t->nbytes;
    if ((int)t->type != type) {
      // small f32 tensors (norms, GDN parameters) may be stored as F16
      if (type == HH_F32 && t->type == HH_F16) {
        conv.resize((size_t)el);
        const uint16_t* h = (const uint16_t*)bytes;
        for (uint64_t k = 0; k < el; ++k) {
          uint32_t x = h[k], s = (x & 0x8000u) << 16, e = (x >> 10) & 0x1f, mnt = x & 0x3ff, bits;
          if (e == 0) {
            if (mnt == 0) bits = s;
            else {   // subnormal: normalise
              int sh = 0;
              while (!(mnt & 0x400)) { mnt <<= 1; ++sh; }
              bits = s | ((uint32_t)(113 - sh) << 23) | ((mnt & 0x3ff) << 13);
            }
          } else if (e == 31) bits = s | 0x7f800000u | (mnt << 13);
          else bits = s | ((e + 112) << 23) | (mnt << 13);
          memcpy(&conv[(size_t)k], &bits, 4);
        }
        bytes = conv.data();
        len = (size_t)el * 4;
      } else if (!(type == HH_Q1_0_G128 && t->type == 39)) {
        hh_model_destroy(m);
        return hh_set_error(HH_ERR_DTYPE, "GGUF: tensor " + src + " has type " + std::to_string(t->type) +
                                              ", the decode path takes type " + std::to_string(type));
      }
    }
    rc = hh_model_upload_tensor(m, name, type, ne0, ne1, bytes, len);
    if (rc != HH_OK) {
      std::string msg = hh_last_error();
      hh_model_destroy(m);
      return hh_set_error(rc, msg);
    }
  }
  *out = m;
  return HH_OK;
}

}  // extern "C"
