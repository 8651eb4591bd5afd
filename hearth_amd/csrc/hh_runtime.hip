// hh_runtime.hip — C ABI (include/hearth_hip.h): context, operators, model
// storage in HBM, the per-token step as one captured HIP graph, and the
// device-resident token loop.
//
// Host-side restatement of the reference's model/session layer:
//   LlamaModel::forward / generate_text       mod.rs:451-860, :2718-3012
//   Qwen35Core::forward / generate_text       qwen35.rs:1028-1236, :1654-1804
//   upload_tensors_to_gpu (native blocks)     model/gpu.rs:8-50
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <mutex>
#include <vector>

#include "../../include/hearth_hip.h"
#include "hh_host.h"
#include "hh_kernels.h"

namespace {
thread_local std::string g_err;
}  // namespace

int hh_set_error(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

namespace {

int fail(int code, const std::string& msg) { return hh_set_error(code, msg); }

#define HIP_TRY(expr)                                                                \
  do {                                                                               \
    hipError_t e_ = (expr);                                                          \
    if (e_ != hipSuccess)                                                            \
      return fail(HH_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(e_));    \
  } while (0)

#define KTRY(expr)                                                                   \
  do {                                                                               \
    if ((expr) != 0) {                                                               \
      hipError_t e_ = hipGetLastError();                                             \
      return fail(HH_ERR_HIP, std::string("launch failed: ") + #expr + ": " + hipGetErrorString(e_)); \
    }                                                                                \
  } while (0)

size_t row_bytes(int type, int64_t n) {
  switch (type) {
    case HH_F32: return (size_t)n * 4;
    case HH_F16: return (size_t)n * 2;
    case HH_Q8_0: return (size_t)(n / 32) * 34;
    case HH_Q1_0: case HH_Q1_0_G128: return (size_t)(n / 128) * 18;
    case HH_Q2_0: case HH_PQ2_0: return (size_t)(n / 128) * 34;
    case HH_PTQ1_0: return (size_t)(n / 128) * 28;
  }
  return 0;
}

bool is_quant(int t) {
  return t == HH_Q8_0 || t == HH_Q1_0 || t == HH_Q1_0_G128 || t == HH_Q2_0 || t == HH_PQ2_0 || t == HH_PTQ1_0;
}

uint64_t mix64h(uint64_t x) {
  x ^= x >> 30;
  x *= 0xbf58476d1ce4e5b9ull;
  x ^= x >> 27;
  x *= 0x94d049bb133111ebull;
  x ^= x >> 31;
  return x;
}

uint64_t name_key(uint64_t seed, const char* name) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (const unsigned char* p = (const unsigned char*)name; *p; ++p) {
    h ^= *p;
    h *= 0x100000001b3ull;
  }
  return mix64h(seed ^ mix64h(h));
}

}  // namespace

struct hh_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  // scratch for the standalone argmax operator
  float* part_val = nullptr;
  int* part_idx = nullptr;
  int* counter = nullptr;
  int* counts = nullptr;
  int64_t counts_n = 0;
  hipEvent_t ev[8] = {};
  void* attn_scratch = nullptr;     // standalone attention partials + counters
  size_t attn_scratch_bytes = 0;
  void* gemm_scratch = nullptr;     // standalone GEMM: activations in split layout
  size_t gemm_scratch_bytes = 0;
};

namespace {

struct Tensor {
  std::string name;
  int type;
  int64_t rows, cols;
  float std, mean;
  size_t nbytes;
  uint8_t* d;       // device pointer (inside the model arena)
};

struct Layer {
  bool gdn = false;
  int attn_idx = -1;
  // fused matrices (device pointers into the arena)
  uint8_t* w_in = nullptr;    // dense: [q;k;v]  gdn: [qkv;gate]  q35 attn: [q(2nq);k;v]
  int n_in = 0;               // rows of w_in
  uint8_t* w_out = nullptr;   // attn_output / ssm_out
  uint8_t* w_gu = nullptr;    // [gate; up]
  uint8_t* w_down = nullptr;
  float *attn_norm = nullptr, *ffn_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
  float *ssm_conv = nullptr, *ssm_dt = nullptr, *ssm_a = nullptr, *ssm_alpha = nullptr, *ssm_beta = nullptr,
        *ssm_norm = nullptr;
  float *k_cache = nullptr, *v_cache = nullptr;
  float *gdn_state = nullptr, *conv_state = nullptr;
};

}  // namespace

struct hh_model {
  hh_ctx* ctx = nullptr;
  hh_model_config cfg{};
  int rope_dim = 0;
  int wfmt = 0;
  std::vector<Tensor> tensors;
  std::map<std::string, int> by_name;
  std::vector<Layer> layers;
  uint8_t* arena = nullptr;
  size_t arena_bytes = 0;
  Tensor *token_embd = nullptr, *output = nullptr, *output_norm = nullptr;
  // state
  float* kv = nullptr;
  size_t kv_bytes = 0;
  float* rec = nullptr;     // gdn + conv state
  size_t rec_bytes = 0;
  float* rope = nullptr;
  // step buffers
  // KV rows per kv head in the cache (>= max_seq): an odd multiple of 64, so
  // that the per-head stride is no multiple of a large power of two.  Strides
  // of 2^22 B and more (max_seq 8192, 32768) measured ~2% slower decode at 2k
  // context than 8000 or 2300, the kv heads' rows meeting in the same memory
  // channels.  The attention kernels take it as their max_seq (the KV stride;
  // positions stay below the configured max_seq, so the RoPE rows are the same).
  int kv_rows = 0;
  float* hidden = nullptr;
  float* hidden_sq = nullptr;   // RMSNorm tree nodes of hidden, one per 16 elements (GemvArgs::sq_out)
  float* proj = nullptr;        // QKV / GDN projection output
  uint8_t* act_mid = nullptr;   // packed input of attn_output / ssm_out
  uint8_t* act_ffn = nullptr;   // packed input of ffn_down
  float* logits = nullptr;
  float* head_pv = nullptr;
  int* head_pi = nullptr;
  int* counters = nullptr;      // [0] head, [1..] attention per kv head, then gdn
  float* attn_po = nullptr;
  float* attn_pml = nullptr;
  int attn_chunk = 0, attn_splits = 0;
  float* gdn_scratch = nullptr;
  int* counts = nullptr;
  uint32_t* prompt = nullptr;
  uint32_t* out_tokens = nullptr;
  int max_out = 0;
  StepState* state = nullptr;
  // graph
  hipGraph_t graph = nullptr;
  hipGraphExec_t gexec = nullptr;
  hipGraph_t graph_n = nullptr;        // graph_steps consecutive decode steps in one graph
  hipGraphExec_t gexec_n = nullptr;
  hipGraph_t graph_ne = nullptr;       // one decode step without k_embed (the previous step's
  hipGraphExec_t gexec_ne = nullptr;   // k_head_final wrote the embedding)
  int graph_steps = 1;
  hipEvent_t ev0 = nullptr, ev1 = nullptr, ev2 = nullptr, evp = nullptr;
  double last_decode_ms = 0.0, last_prefill_ms = 0.0;
  int cancel = 0;
  // launch geometry
  int rows_in = 16, rows_out = 16, rows_gu = 32, rows_down = 16, rows_head = 64;
  // batched prefill scratch (grown on demand); HH_BATCHED_PREFILL=0 feeds prompts token by token
  uint8_t* pf_buf = nullptr;
  size_t pf_cap = 0;
  int batched_prefill = 1;
  // HH_GDN_CHUNKED=1: the batched prefill runs the GDN recurrence in chunked
  // form (fp32-rounding parity with the sequential rule instead of bit parity)
  int gdn_chunked = 0;
  // the chunked form needs every ssm_a < 0 (its decays exp(G_t - G_s) then stay
  // <= 1): -1 unchecked since the last weight write, 0 some ssm_a >= 0, 1 all negative
  int ssm_a_negative = -1;
  // HH_PREFILL_ATTN=mfma: the batched prefill's attention runs on fp32 MFMA
  // (k_attn_prefill_mfma; fp32-rounding parity instead of bit parity)
  int prefill_attn_mfma = 0;
  // Hadamard fold: one device sign vector per folded width (+1 until set), and
  // the f32 hand-off of the matmul inputs that are rotated in the consumer's prologue
  float* had_signs = nullptr;
  std::vector<std::pair<int, size_t>> sign_off;   // width -> float offset in had_signs
  float* rot_f32 = nullptr;
};

// Scratch of the allocation-free attention entry point (hh_attention_noalloc):
// the split partials live in this file-scope device array, one copy per GPU,
// held until the process ends.  Host code never passes `scratch` itself to a
// kernel (in host code it is a stand-in, not a device address): each device's
// address comes from hipGetSymbolAddress at context set-up, with that device
// current, and is kept in g_scratch_ptr.
constexpr size_t HH_NOALLOC_SCRATCH_BYTES = (size_t)4 << 20;
static __device__ __align__(256) uint8_t scratch[HH_NOALLOC_SCRATCH_BYTES];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];   // by device ordinal

namespace {

Tensor* find(hh_model* m, const std::string& n) {
  auto it = m->by_name.find(n);
  return it == m->by_name.end() ? nullptr : &m->tensors[it->second];
}

// Declares every tensor and where it lives inside the arena.  Matrices that one
// GEMV launch consumes together are adjacent (rows concatenated, native blocks).
void declare(hh_model* m) {
  const hh_model_config& c = m->cfg;
  int d = c.d_model, hd = c.head_dim, nq = c.n_heads * hd, nkv = c.n_kv_heads * hd;
  int kdim = c.ssm_n_k_heads * c.ssm_head_dim, vdim = c.ssm_n_v_heads * c.ssm_head_dim;
  int conv_dim = 2 * kdim + vdim;
  auto add = [&](const std::string& name, int type, int64_t rows, int64_t cols, float sd, float mean) {
    Tensor t{name, type, rows, cols, sd, mean, row_bytes(type, cols) * (size_t)rows, nullptr};
    m->by_name[name] = (int)m->tensors.size();
    m->tensors.push_back(t);
  };
  char b[96];
  add("token_embd.weight", c.head_type, c.vocab, d, 0.02f, 0.0f);
  // a tied head (prism.hadamard.tied_output, qwen35.rs:597-620) has no output.weight
  if (!(c.arch == 1 && c.had_block > 0 && (c.had_flags & HH_HAD_TIED_OUTPUT)))
    add("output.weight", c.head_type, c.vocab, d, 0.02f, 0.0f);
  add("output_norm.weight", HH_F32, 1, d, 0.02f, 1.0f);
  int wt = c.wtype;
  for (int i = 0; i < c.n_layers; ++i) {
    bool gdn = (c.arch == 1) && ((i + 1) % c.full_attn_interval != 0);
#define NM(s) (snprintf(b, sizeof b, "blk.%d." s, i), std::string(b))
    add(NM("attn_norm.weight"), HH_F32, 1, d, 0.02f, 1.0f);
    if (c.arch == 1) add(NM("post_attention_norm.weight"), HH_F32, 1, d, 0.02f, 1.0f);
    else add(NM("ffn_norm.weight"), HH_F32, 1, d, 0.02f, 1.0f);
    if (gdn) {
      add(NM("attn_qkv.weight"), wt, conv_dim, d, 0.02f, 0.0f);
      add(NM("attn_gate.weight"), wt, vdim, d, 0.02f, 0.0f);
      add(NM("ssm_conv1d.weight"), HH_F32, conv_dim, c.ssm_conv_kernel, 0.3f, 0.0f);
      add(NM("ssm_dt.bias"), HH_F32, 1, c.ssm_n_v_heads, 0.5f, 0.0f);
      add(NM("ssm_a"), HH_F32, 1, c.ssm_n_v_heads, 0.1f, -1.0f);
      add(NM("ssm_alpha.weight"), HH_F32, c.ssm_n_v_heads, d, 0.02f, 0.0f);
      add(NM("ssm_beta.weight"), HH_F32, c.ssm_n_v_heads, d, 0.02f, 0.0f);
      add(NM("ssm_norm.weight"), HH_F32, 1, c.ssm_head_dim, 0.02f, 1.0f);
      add(NM("ssm_out.weight"), wt, d, vdim, 0.02f, 0.0f);
    } else {
      int qrows = c.attn_out_gate ? 2 * nq : nq;
      add(NM("attn_q.weight"), wt, qrows, d, 0.02f, 0.0f);
      add(NM("attn_k.weight"), wt, nkv, d, 0.02f, 0.0f);
      add(NM("attn_v.weight"), wt, nkv, d, 0.02f, 0.0f);
      add(NM("attn_output.weight"), wt, d, nq, 0.02f, 0.0f);
      if (c.qk_norm) {
        add(NM("attn_q_norm.weight"), HH_F32, 1, hd, 0.02f, 1.0f);
        add(NM("attn_k_norm.weight"), HH_F32, 1, hd, 0.02f, 1.0f);
      }
    }
    add(NM("ffn_gate.weight"), wt, c.d_ffn, d, 0.02f, 0.0f);
    add(NM("ffn_up.weight"), wt, c.d_ffn, d, 0.02f, 0.0f);
    add(NM("ffn_down.weight"), wt, d, c.d_ffn, 0.02f, 0.0f);
#undef NM
  }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Rows per GEMV workgroup (1024 lanes): enough for one workgroup per CU
// (256), capped so the transposed block products part[2P x (rows+1)] stay
// within 64 KB of LDS.
int gemv_rows_for(int n_rows, int P) {
  int rows = (n_rows + 255) / 256;
  int cap = std::max(1, (64 * 1024) / (8 * P) - 1);
  return std::max(1, std::min(rows, cap));
}

int enqueue_step(hh_model* m, hipStream_t s, int only_layer = -1, unsigned stages = ~0u);

// Device sign vector of a folded width (all +1 until hh_model_set_hadamard_signs).
const float* signs_of(const hh_model* m, int width) {
  for (auto& so : m->sign_off)
    if (so.first == width) return m->had_signs + so.second;
  return nullptr;
}

int capture(hh_model* m) {
  hipStream_t s = m->ctx->stream;
  if (m->gexec) { hipGraphExecDestroy(m->gexec); m->gexec = nullptr; }
  if (m->graph) { hipGraphDestroy(m->graph); m->graph = nullptr; }
  HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  int rc = enqueue_step(m, s);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(s, &g);
  if (rc != 0) { if (g) hipGraphDestroy(g); return rc; }
  if (e != hipSuccess) return fail(HH_ERR_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(e));
  m->graph = g;
  HIP_TRY(hipGraphInstantiate(&m->gexec, g, nullptr, nullptr, 0));
  // continuation graphs: steps whose token the previous step's k_head_final
  // already embedded (every decode step of hh_model_generate after the first);
  // the step advances its own state, so several chain inside one graph
  auto capture_steps = [&](int n, hipGraph_t* gp, hipGraphExec_t* ep) -> int {
    if (*ep) { hipGraphExecDestroy(*ep); *ep = nullptr; }
    if (*gp) { hipGraphDestroy(*gp); *gp = nullptr; }
    HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int rc2 = 0;
    for (int i = 0; i < n && rc2 == 0; ++i) rc2 = enqueue_step(m, s, -1, ~1u);
    hipGraph_t gn = nullptr;
    hipError_t e2 = hipStreamEndCapture(s, &gn);
    if (rc2 != 0) { if (gn) hipGraphDestroy(gn); return rc2; }
    if (e2 != hipSuccess) return fail(HH_ERR_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(e2));
    *gp = gn;
    HIP_TRY(hipGraphInstantiate(ep, gn, nullptr, nullptr, 0));
    return HH_OK;
  };
  int rc3 = capture_steps(1, &m->graph_ne, &m->gexec_ne);
  if (rc3 == HH_OK) rc3 = capture_steps(m->graph_steps, &m->graph_n, &m->gexec_n);
  return rc3;
}

GemvArgs gemv_base(const uint8_t* w, int n_rows, int K, int rows_per_wg) {
  GemvArgs a{};
  a.w = w;
  a.n_rows = n_rows;
  a.K = K;
  a.rows_per_wg = rows_per_wg;
  return a;
}

// One decode step (mod.rs:451-860 / qwen35.rs:1028-1236) as a kernel sequence.
// Stages: 0 embed, 1 input projection, 2 attention / GDN, 3 output projection,
// 4 gate+up, 5 down, 6 LM head + greedy selection.  `only_layer`/`stages`
// restrict the launch (stage timing); the captured graph holds everything.
int enqueue_step(hh_model* m, hipStream_t s, int only_layer, unsigned stages) {
  auto want = [&](int st, int li) { return ((stages >> st) & 1u) && (only_layer < 0 || li == only_layer || li < 0); };
  const hh_model_config& c = m->cfg;
  const int d = c.d_model, hd = c.head_dim, nq = c.n_heads * hd, nkv = c.n_kv_heads * hd;
  const int wf = m->wfmt;
  // Hadamard-folded qwen35 model: every matmul input is rotated before Q8_0
  // (qwen35.rs:881-970); producers then hand f32 vectors to the next prologue
  const bool had = c.had_block > 0;
  const bool latent = had && (c.had_flags & HH_HAD_LATENT_EMBD);
  const int pro_norm = had ? HH_PRO_NORMROT : HH_PRO_RMSNORM;
  auto fold = [&](GemvArgs& g, int width) { g.signs = signs_of(m, width); g.had_block = c.had_block; };
  // The residual-add GEMVs hand the RMSNorm sum-of-squares tree nodes of the
  // hidden state to the next norm prologue (no workgroup barrier there) when
  // their workgroups own whole 16-row groups; layer 0's input comes from the
  // embedding and keeps the in-kernel reduction.
  const bool sq = !had && d % 64 == 0 && d <= 4096 && m->rows_out % 16 == 0 && m->rows_down % 16 == 0;
  if (want(0, -1))
    KTRY(hh_embed_launch(c.head_type, m->token_embd->d, d, m->state, m->hidden, latent ? signs_of(m, d) : nullptr,
                         latent ? c.had_block : 0, s));
  for (int li = 0; li < c.n_layers; ++li) {
    Layer& L = m->layers[li];
    // input projection(s), RMSNorm + Q8_0 fused into the GEMV prologue
    GemvArgs g = gemv_base(L.w_in, L.n_in, d, m->rows_in);
    g.x = m->hidden;
    g.norm_w = L.attn_norm;
    g.eps = c.eps;
    g.y = m->proj;
    if (had) fold(g, d);
    if (sq && li > 0) g.sq_in = m->hidden_sq;
    if (L.gdn) {   // the first 2 n_v workgroups also form the raw alpha / beta dots
      g.ab_wa = L.ssm_alpha;
      g.ab_wb = L.ssm_beta;
      g.ab_n = c.ssm_n_v_heads;
      g.ab_rows = 2 * c.ssm_n_v_heads;
      g.ab_out = m->gdn_scratch;
    }
    if (want(1, li)) KTRY(hh_gemv_launch(wf, pro_norm, HH_EPI_STORE, g, s));
    int k_out;
    if (L.gdn) {
      int kdim = c.ssm_n_k_heads * c.ssm_head_dim, vdim = c.ssm_n_v_heads * c.ssm_head_dim;
      GdnArgs ga{};
      ga.proj = m->proj;
      ga.z = m->proj + (2 * kdim + vdim);
      ga.hidden = m->hidden;
      ga.attn_norm = L.attn_norm;
      ga.w_alpha = L.ssm_alpha;
      ga.w_beta = L.ssm_beta;
      ga.dt_bias = L.ssm_dt;
      ga.ssm_a = L.ssm_a;
      ga.conv_w = L.ssm_conv;
      ga.conv_state = L.conv_state;
      ga.ssm_norm = L.ssm_norm;
      ga.state = L.gdn_state;
      ga.d = d;
      ga.n_k = c.ssm_n_k_heads;
      ga.n_v = c.ssm_n_v_heads;
      ga.hd = c.ssm_head_dim;
      ga.kernel = c.ssm_conv_kernel;
      ga.eps = c.eps;
      ga.act_out = m->act_mid;
      ga.act_fmt = wf;
      ga.ab_raw = m->gdn_scratch;
      ga.st = m->state;
      if (had) ga.out_f32 = m->rot_f32;
      if (want(2, li)) KTRY(hh_gdn_launch(ga, s));
      k_out = vdim;
    } else {
      AttnArgs aa{};
      aa.qkv = m->proj;
      aa.n_heads = c.n_heads;
      aa.n_kv = c.n_kv_heads;
      aa.hd = hd;
      aa.rope_dim = m->rope_dim;
      aa.gated = c.attn_out_gate;
      aa.q_stride_heads = (c.attn_out_gate ? 2 : 1) * nq;
      aa.q_norm = L.q_norm;
      aa.k_norm = L.k_norm;
      aa.eps = c.eps;
      aa.rope = m->rope;
      aa.max_seq = m->kv_rows;
      aa.k_cache = L.k_cache;
      aa.v_cache = L.v_cache;
      aa.state = m->state;
      aa.fixed_seq = 0;
      aa.chunk = m->attn_chunk;
      aa.max_splits = m->attn_splits;
      aa.part_o = m->attn_po;
      aa.part_ml = m->attn_pml;
      aa.counters = m->counters + 1;
      aa.out_f32 = nullptr;
      aa.act_out = m->act_mid;
      aa.act_fmt = wf;
      aa.kv_q8 = c.kv_type == HH_Q8_0;
      if (had) { aa.out_f32 = m->rot_f32; aa.act_out = nullptr; }
      if (want(2, li)) KTRY(hh_attn_launch(aa, s));
      k_out = nq;
      (void)nkv;
    }
    GemvArgs o = gemv_base(L.w_out, d, k_out, m->rows_out);
    o.act = m->act_mid;
    o.y = m->hidden;
    if (sq) o.sq_out = m->hidden_sq;
    if (had) {
      o.x = m->rot_f32;
      fold(o, k_out);
      if (L.gdn) { o.perm_nk = c.ssm_n_k_heads; o.perm_rep = c.ssm_n_v_heads / c.ssm_n_k_heads; }
    }
    if (want(3, li)) KTRY(hh_gemv_launch(wf, had ? HH_PRO_F32ROT : HH_PRO_PACKED, HH_EPI_ADD, o, s));
    GemvArgs gu = gemv_base(L.w_gu, 2 * c.d_ffn, d, m->rows_gu);
    gu.half_rows = c.d_ffn;
    gu.x = m->hidden;
    gu.norm_w = L.ffn_norm;
    gu.eps = c.eps;
    gu.act_out = m->act_ffn;
    gu.act_out_fmt = wf;
    gu.act_out_k = c.d_ffn;
    if (sq) gu.sq_in = m->hidden_sq;
    if (had) { fold(gu, d); gu.y = m->rot_f32; }
    if (want(4, li)) KTRY(hh_gemv_launch(wf, pro_norm, HH_EPI_SILU, gu, s));
    GemvArgs dn = gemv_base(L.w_down, d, c.d_ffn, m->rows_down);
    dn.act = m->act_ffn;
    dn.y = m->hidden;
    if (sq) dn.sq_out = m->hidden_sq;
    if (had) { dn.x = m->rot_f32; fold(dn, c.d_ffn); }
    if (want(5, li)) KTRY(hh_gemv_launch(wf, had ? HH_PRO_F32ROT : HH_PRO_PACKED, HH_EPI_ADD, dn, s));
  }
  GemvArgs h = gemv_base(m->output->d, c.vocab, d, m->rows_head);
  h.x = m->hidden;
  h.norm_w = (const float*)m->output_norm->d;
  if (sq && c.n_layers > 0) h.sq_in = m->hidden_sq;
  h.eps = c.eps;
  h.y = m->logits;
  h.state = m->state;
  h.prompt = m->prompt;
  h.out_tokens = m->out_tokens;
  h.max_out = m->max_out;
  h.counts = m->counts;
  h.pen = 1.0f;   // replaced from the state at run time (see k_gemv EPI_LOGITS)
  h.rule = c.arch == 1 ? 1 : 0;
  h.part_val = m->head_pv;
  h.part_idx = m->head_pi;
  h.counter = m->counters;
  // the next step's embedding, written by k_head_final (steps replayed by
  // hh_model_generate then skip k_embed)
  h.emb_table = m->token_embd->d;
  h.emb_type = c.head_type;
  h.emb_d = d;
  h.emb_had = latent ? c.had_block : 0;
  h.emb_signs = latent ? signs_of(m, d) : nullptr;
  h.emb_out = m->hidden;
  if (had) fold(h, d);
  if (want(6, -1)) KTRY(hh_gemv_launch(hh_fmt_of(c.head_type), pro_norm, HH_EPI_LOGITS, h, s));
  return HH_OK;
}



// Batched prefill of a dense model (forward_batch, mod.rs:899-1221): tokens
// toks[0..S) at positions pos0.. through every layer with the int8-MFMA GEMM
// and row kernels that restate the decode step's arithmetic, writing the KV
// cache; no logits (mod.rs:1201-1218 computes only the last token's, which the
// caller runs through the decode step).
// Batched prefill (forward_batch, mod.rs:899-1221) of S prompt tokens from
// pos0: every projection is one MFMA GEMM over the S token rows.  Dense and
// qwen35 full-attention layers run the split/merge attention per 128-token
// tile; GDN layers run the per-token prep in parallel and the recurrence in
// token order per v-head (the state stays in registers).  The result is the
// state that feeding the tokens one at a time leaves, bit for bit.
#ifndef PF_ATTN_BYTES
#define PF_ATTN_BYTES ((size_t)2 << 30)
#endif
// Whether every GDN layer's ssm_a is negative (read back once per weight write).
int ssm_a_all_negative(hh_model* m, bool* ok) {
  if (m->ssm_a_negative < 0) {
    std::vector<float> a(m->cfg.ssm_n_v_heads);
    int neg = 1;
    for (const Layer& L : m->layers) {
      if (!L.ssm_a) continue;
      HIP_TRY(hipMemcpy(a.data(), L.ssm_a, sizeof(float) * a.size(), hipMemcpyDeviceToHost));
      for (float v : a)
        if (!(v < 0.0f)) neg = 0;
    }
    m->ssm_a_negative = neg;
  }
  *ok = m->ssm_a_negative == 1;
  return HH_OK;
}

int prefill_batched(hh_model* m, const uint32_t* toks, int S, int pos0) {
  const hh_model_config& c = m->cfg;
  hipStream_t s = m->ctx->stream;
  // HH_GDN_CHUNKED applies only where every ssm_a < 0; otherwise the
  // sequential recurrence runs (it stays finite for any ssm_a)
  bool chunked = false;
  if (m->gdn_chunked) {
    const int rc = ssm_a_all_negative(m, &chunked);
    if (rc != HH_OK) return rc;
  }
  const int d = c.d_model, hd = c.head_dim, nq = c.n_heads * hd, F = c.d_ffn;
  // the chunks the prompt reaches (the partials' chunk stride, shared by the
  // split and merge passes), not every chunk of the cache
  // (rounded up to 3 mod 8: the split grid's workgroup ids x + n_chunks * y
  // then put each kv head's chunk x on a different XCD of the round-robin
  // dispatch; measured against the neighbouring strides)
  int n_chunks = (pos0 + S + m->attn_chunk - 1) / m->attn_chunk;
  n_chunks += (3 - n_chunks % 8 + 8) % 8;
  const int G = c.n_heads / c.n_kv_heads;
  // attention tokens per pass: as many as keep the split partials within
  // PF_ATTN_BYTES (all of them up to a few thousand tokens), in 16-token tiles
  const size_t part_per_tok = (size_t)c.n_kv_heads * n_chunks * G * (hd + 2) * 4;
  const int TA = std::max(16, std::min((S + 15) / 16 * 16, (int)(PF_ATTN_BYTES / part_per_tok) / 16 * 16));
  const bool hyb = c.arch == 1;
  const int kv8 = c.kv_type == HH_Q8_0;
  const int kdim = hyb ? c.ssm_n_k_heads * c.ssm_head_dim : 0, vdim = hyb ? c.ssm_n_v_heads * c.ssm_head_dim : 0;
  int n_in_max = 0;
  for (const Layer& L : m->layers) n_in_max = std::max(n_in_max, L.n_in);
  const int kmax = std::max(std::max(d, F), std::max(nq, vdim));
  // scratch layout
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off = align256(off + bytes); return o; };
  const size_t oH = take((size_t)S * d * 4), oXq = take((size_t)S * kmax), oXd = take((size_t)S * (kmax / 32) * 4),
               oQKV = take((size_t)S * n_in_max * 4), oQB = take((size_t)S * nq * 4),
               oT = take((size_t)S * d * 4), oGU = take((size_t)S * 2 * F * 4),
               oPO = take((size_t)TA * c.n_kv_heads * n_chunks * G * hd * 4),
               oPML = take((size_t)TA * c.n_kv_heads * n_chunks * G * 2 * 4),
               oGQK = take(hyb ? (size_t)S * 2 * kdim * 4 : 0), oGV = take(hyb ? (size_t)S * vdim * 4 : 0),
               oGAB = take(hyb ? (size_t)S * 2 * c.ssm_n_v_heads * 4 : 0),
               oGDEC = take(hyb ? (size_t)S * c.ssm_n_v_heads * 4 : 0), oGO = take(hyb ? (size_t)S * vdim * 4 : 0),
               oRot = take(c.had_block > 0 ? (size_t)S * std::max(std::max(vdim, nq), F) * 4 : 0),
               oChunk = take(hyb && chunked ? hh_gdn_chunk_scratch_bytes(c.ssm_n_v_heads, S) : 0);
  if (off > m->pf_cap) {
    if (m->pf_buf) HIP_TRY(hipFree(m->pf_buf));
    m->pf_buf = nullptr;
    m->pf_cap = 0;
    if (hipMalloc(&m->pf_buf, off) != hipSuccess) return fail(HH_ERR_OOM, "prefill scratch allocation failed");
    m->pf_cap = off;
  }
  uint8_t* B = m->pf_buf;
  float* H = (float*)(B + oH);
  int8_t* Xq = (int8_t*)(B + oXq);
  float* Xd = (float*)(B + oXd);
  float* QKV = (float*)(B + oQKV);
  float* QB = (float*)(B + oQB);
  float* T = (float*)(B + oT);
  float* GU = (float*)(B + oGU);
  float* PO = (float*)(B + oPO);
  float* PML = (float*)(B + oPML);
  // Hadamard fold (qwen35.rs:881-970): every matmul input row is rotated
  // before Q8_0; producers write f32 rows to Rot, k_rot_q8_rows quantizes them
  const bool had = c.had_block > 0;
  const bool latent = had && (c.had_flags & HH_HAD_LATENT_EMBD);
  float* Rot = had ? (float*)(B + oRot) : nullptr;
  auto norm_rows = [&](const float* w) -> int {
    if (had) return hh_rot_q8_rows_launch(H, w, c.eps, d, S, signs_of(m, d), c.had_block, 0, 0, Xq, Xd, s);
    return hh_norm_q8_rows_launch(H, w, c.eps, d, S, Xq, Xd, s);
  };
  KTRY(hh_embed_rows_launch(c.head_type, m->token_embd->d, d, toks, S, H, latent ? signs_of(m, d) : nullptr,
                            latent ? c.had_block : 0, s));
  for (int li = 0; li < c.n_layers; ++li) {
    Layer& L = m->layers[li];
    // the previous layer's ffn_down residual add runs here, fused with this
    // layer's input norm where no Hadamard rotation sits between them
    if (li > 0 && !had) {
      KTRY(hh_add_norm_q8_rows_launch(H, T, L.attn_norm, c.eps, d, S, Xq, Xd, s));
    } else {
      if (li > 0) KTRY(hh_add_rows_launch(H, T, (int64_t)S * d, s));
      KTRY(norm_rows(L.attn_norm));
    }
    KTRY(hh_gemm_launch(m->wfmt, L.w_in, L.n_in, d, Xq, Xd, S, QKV, s));
    int k_out;
    if (L.gdn) {
      GdnArgs ga{};
      ga.proj = QKV;
      ga.hidden = H;
      ga.attn_norm = L.attn_norm;
      ga.w_alpha = L.ssm_alpha;
      ga.w_beta = L.ssm_beta;
      ga.dt_bias = L.ssm_dt;
      ga.ssm_a = L.ssm_a;
      ga.conv_w = L.ssm_conv;
      ga.conv_state = L.conv_state;
      ga.ssm_norm = L.ssm_norm;
      ga.state = L.gdn_state;
      ga.d = d;
      ga.n_k = c.ssm_n_k_heads;
      ga.n_v = c.ssm_n_v_heads;
      ga.hd = c.ssm_head_dim;
      ga.kernel = c.ssm_conv_kernel;
      ga.eps = c.eps;
      ga.qk = (float*)(B + oGQK);
      ga.vconv = (float*)(B + oGV);
      ga.ab = (float*)(B + oGAB);
      ga.dec_rows = (float*)(B + oGDEC);
      ga.pos0 = pos0;
      ga.S = S;
      ga.row_in = L.n_in;
      ga.o_rows = (float*)(B + oGO);
      ga.xq = Xq;
      ga.xd = Xd;
      ga.y_rows = Rot;
      KTRY(hh_gdn_rows_launch(ga, chunked ? (float*)(B + oChunk) : nullptr, s));
      if (had)
        KTRY(hh_rot_q8_rows_launch(Rot, nullptr, 0.0f, vdim, S, signs_of(m, vdim), c.had_block, c.ssm_n_k_heads,
                                   c.ssm_n_v_heads / c.ssm_n_k_heads, Xq, Xd, s));
      k_out = vdim;
    } else {
      const int gated = hyb && c.attn_out_gate;
      KTRY(hh_prefill_qk_launch(hd, QKV, L.n_in, c.n_heads, c.n_kv_heads, c.qk_norm ? L.q_norm : nullptr,
                                c.qk_norm ? L.k_norm : nullptr, c.eps, m->rope, m->rope_dim, m->kv_rows, pos0, S,
                                gated, kv8, L.k_cache, L.v_cache, QB, s));
      if (m->prefill_attn_mfma)
        KTRY(hh_prefill_attn_mfma_launch(hd, QB, L.k_cache, L.v_cache, c.n_heads, c.n_kv_heads, m->kv_rows, pos0, 0,
                                         S, gated ? QKV : nullptr, L.n_in, kv8, Xq, Xd, Rot, s));
      else
        for (int t0 = 0; t0 < S; t0 += TA)
          KTRY(hh_prefill_attn_launch(hd, QB, L.k_cache, L.v_cache, c.n_heads, c.n_kv_heads, m->kv_rows, pos0, t0,
                                      std::min(TA, S - t0), n_chunks, PO, PML, gated ? QKV : nullptr, L.n_in, kv8,
                                      Xq, Xd, Rot, s));
      if (had)
        KTRY(hh_rot_q8_rows_launch(Rot, nullptr, 0.0f, nq, S, signs_of(m, nq), c.had_block, 0, 0, Xq, Xd, s));
      k_out = nq;
    }
    KTRY(hh_gemm_launch(m->wfmt, L.w_out, d, k_out, Xq, Xd, S, T, s));
    if (!had) {
      KTRY(hh_add_norm_q8_rows_launch(H, T, L.ffn_norm, c.eps, d, S, Xq, Xd, s));
    } else {
      KTRY(hh_add_rows_launch(H, T, (int64_t)S * d, s));
      KTRY(norm_rows(L.ffn_norm));
    }
    KTRY(hh_gemm_launch(m->wfmt, L.w_gu, 2 * F, d, Xq, Xd, S, GU, s));
    KTRY(hh_silu_q8_rows_launch(GU, F, S, Xq, Xd, Rot, s));
    if (had) KTRY(hh_rot_q8_rows_launch(Rot, nullptr, 0.0f, F, S, signs_of(m, F), c.had_block, 0, 0, Xq, Xd, s));
    KTRY(hh_gemm_launch(m->wfmt, L.w_down, d, F, Xq, Xd, S, T, s));
    // the residual add: fused into the next layer's input norm, plain after the last
    if (li + 1 == c.n_layers) KTRY(hh_add_rows_launch(H, T, (int64_t)S * d, s));
  }
  return HH_OK;
}

}  // namespace

extern "C" {

const char* hh_last_error(void) { return g_err.c_str(); }
const char* hh_version(void) { return "hearth_hip 0.1 gfx950"; }

int hh_ctx_create(int device_ordinal, hh_ctx** out) {
  if (!out) return fail(HH_ERR_INVALID, "out is null");
  int n = 0;
  HIP_TRY(hipGetDeviceCount(&n));
  if (device_ordinal < 0 || device_ordinal >= n) return fail(HH_ERR_INVALID, "no such device");
  HIP_TRY(hipSetDevice(device_ordinal));
  if (device_ordinal >= 64) return fail(HH_ERR_INVALID, "device ordinal beyond 63");
  {
    // once per device, with the device current: the device address of `scratch`
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device_ordinal]) {
      void* p = nullptr;
      hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) return fail(HH_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
      g_scratch_ptr[device_ordinal] = p;
    }
  }
  hh_ctx* c = new hh_ctx();
  c->device = device_ordinal;
  // a failure past this point releases what was created through hh_ctx_destroy
  const int rc = [&]() -> int {
    HIP_TRY(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    HIP_TRY(hipMalloc(&c->part_val, 4096 * sizeof(float)));
    HIP_TRY(hipMalloc(&c->part_idx, 4096 * sizeof(int)));
    HIP_TRY(hipMalloc(&c->counter, 64 * sizeof(int)));
    HIP_TRY(hipMemset(c->counter, 0, 64 * sizeof(int)));
    return HH_OK;
  }();
  if (rc != HH_OK) {
    const std::string msg = hh_last_error();
    hh_ctx_destroy(c);
    return fail(rc, msg);
  }
  *out = c;
  return HH_OK;
}

int hh_ctx_destroy(hh_ctx* c) {
  if (!c) return HH_OK;
  hipSetDevice(c->device);
  if (c->stream) hipStreamSynchronize(c->stream);
  hipFree(c->part_val);
  hipFree(c->part_idx);
  hipFree(c->counter);
  if (c->counts) hipFree(c->counts);
  if (c->attn_scratch) hipFree(c->attn_scratch);
  if (c->gemm_scratch) hipFree(c->gemm_scratch);
  for (hipEvent_t e : c->ev)
    if (e) hipEventDestroy(e);
  if (c->stream) hipStreamDestroy(c->stream);
  delete c;
  return HH_OK;
}

int hh_ctx_synchronize(hh_ctx* c) {
  if (!c) return fail(HH_ERR_INVALID, "ctx is null");
  HIP_TRY(hipStreamSynchronize(c->stream));
  return HH_OK;
}

int hh_ctx_event_record(hh_ctx* c, int slot) {
  if (!c || slot < 0 || slot >= 8) return fail(HH_ERR_INVALID, "bad event slot");
  if (!c->ev[slot]) HIP_TRY(hipEventCreate(&c->ev[slot]));
  HIP_TRY(hipEventRecord(c->ev[slot], c->stream));
  return HH_OK;
}

int hh_ctx_event_elapsed(hh_ctx* c, int a, int b, float* ms) {
  if (!c || !ms || a < 0 || b < 0 || a >= 8 || b >= 8 || !c->ev[a] || !c->ev[b])
    return fail(HH_ERR_INVALID, "bad event slot");
  HIP_TRY(hipEventSynchronize(c->ev[b]));
  HIP_TRY(hipEventElapsedTime(ms, c->ev[a], c->ev[b]));
  return HH_OK;
}

int hh_malloc(hh_ctx* c, size_t n, void** p) {
  if (!c || !p) return fail(HH_ERR_INVALID, "null argument");
  hipError_t e = hipMalloc(p, n ? n : 1);
  if (e != hipSuccess) return fail(HH_ERR_OOM, std::string("hipMalloc: ") + hipGetErrorString(e));
  return HH_OK;
}
int hh_free(hh_ctx* c, void* p) {
  if (!c) return fail(HH_ERR_INVALID, "ctx is null");
  HIP_TRY(hipFree(p));
  return HH_OK;
}
int hh_memcpy_h2d(hh_ctx* c, void* dst, const void* src, size_t n) {
  if (!c) return fail(HH_ERR_INVALID, "ctx is null");
  HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return HH_OK;
}
int hh_memcpy_d2h(hh_ctx* c, void* dst, const void* src, size_t n) {
  if (!c) return fail(HH_ERR_INVALID, "ctx is null");
  HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return HH_OK;
}
int hh_memset(hh_ctx* c, void* dst, int v, size_t n) {
  if (!c) return fail(HH_ERR_INVALID, "ctx is null");
  HIP_TRY(hipMemsetAsync(dst, v, n, c->stream));
  return HH_OK;
}

int hh_quantize_q8_0(hh_ctx* c, const float* x, int64_t n, uint8_t* out) {
  if (!c || (!x && n) || (!out && n)) return fail(HH_ERR_INVALID, "null argument");
  if (n < 0) return fail(HH_ERR_DIM, "negative length");
  KTRY(hh_quantize_launch(x, n, out, c->stream));
  return HH_OK;
}

int hh_dequantize(hh_ctx* c, int type, const void* w, int64_t n, float* out) {
  if (!c || (!w && n) || (!out && n)) return fail(HH_ERR_INVALID, "null argument");
  if (!(is_quant(type) || type == HH_F32 || type == HH_F16)) return fail(HH_ERR_DTYPE, "unsupported dtype");
  int64_t blk = type == HH_Q8_0 ? 32 : (is_quant(type) ? 128 : 1);
  if (n % blk) return fail(HH_ERR_DIM, "length is not a whole number of blocks");
  KTRY(hh_dequant_launch(type, w, n, out, c->stream));
  return HH_OK;
}

int hh_gemv_q8(hh_ctx* c, int type, const void* w, int64_t n_rows, int64_t n_cols, const uint8_t* xq8, float* y) {
  if (!c || !w || !xq8 || !y) return fail(HH_ERR_INVALID, "null argument");
  int fmt = hh_fmt_of(type);
  if (fmt < 0) return fail(HH_ERR_DTYPE, "unsupported weight dtype for the Q8_0 GEMV");
  int el = hh_unit_el(fmt);
  if (n_cols <= 0 || n_cols % el != 0)
    return fail(HH_ERR_DIM, "n_cols must be a positive multiple of " + std::to_string(el));
  if (n_cols > 20480) return fail(HH_ERR_DIM, "n_cols above 20480");
  if (n_rows <= 0 || n_rows > (1ll << 30)) return fail(HH_ERR_DIM, "bad n_rows");
  int P = (int)n_cols / el;
  int rows = gemv_rows_for((int)n_rows, P);
  // Where one workgroup per CU would stream more than 4 units per lane, give
  // every lane of a workgroup exactly one unit and launch many more
  // workgroups instead (151936 x 2048 against one workgroup per CU: Q1_0
  // 19.5 -> 14.1 us, Q2_0 24.7 -> 19.0 us; 1024 units per workgroup beat
  // 768: Q1_0 15.6 -> 14.1 us, Q8_0 62.8 -> 58.4 us, and beat 384, 512, 896,
  // 1192, 1536, 2048 and 2376, which leave lanes idle or take the
  // multi-unit kernels).
  if (rows * P > 4 * 1024) rows = std::max(1, 1024 / P);   // 1024 = lanes per GEMV workgroup
  GemvArgs a = gemv_base((const uint8_t*)w, (int)n_rows, (int)n_cols, rows);
  a.act = xq8;
  a.y = y;
  KTRY(hh_gemv_launch(fmt, HH_PRO_STDQ8, HH_EPI_STORE, a, c->stream));
  return HH_OK;
}

int hh_gemm_q8(hh_ctx* c, int type, const void* w, int64_t n_rows, int64_t n_cols, const uint8_t* xq8,
               int64_t seq_len, float* out) {
  if (!c || !w || !xq8 || !out) return fail(HH_ERR_INVALID, "null argument");
  int fmt = hh_fmt_of(type);
  if (fmt < 0) return fail(HH_ERR_DTYPE, "unsupported weight dtype for the Q8_0 GEMM");
  if (n_cols <= 0 || n_cols % 128 != 0) return fail(HH_ERR_DIM, "n_cols must be a positive multiple of 128");
  if (n_rows <= 0 || n_rows > (1ll << 30) || seq_len <= 0 || seq_len > (1ll << 24))
    return fail(HH_ERR_DIM, "bad n_rows or seq_len");
  if ((n_rows + 63) / 64 > 2147483647ll || (seq_len + 63) / 64 > 65535) return fail(HH_ERR_DIM, "grid too large");
  // the GEMM reads its activations as int8 rows plus f32 block scales
  const size_t nq = (size_t)seq_len * n_cols, need = align256(nq) + nq / 32 * 4;
  if (c->gemm_scratch_bytes < need) {
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (c->gemm_scratch) HIP_TRY(hipFree(c->gemm_scratch));
    c->gemm_scratch = nullptr;
    c->gemm_scratch_bytes = 0;
    HIP_TRY(hipMalloc(&c->gemm_scratch, need));
    c->gemm_scratch_bytes = need;
  }
  int8_t* xq = (int8_t*)c->gemm_scratch;
  float* xd = (float*)((char*)c->gemm_scratch + align256(nq));
  KTRY(hh_q8_split_launch(xq8, (int64_t)(nq / 32), xq, xd, c->stream));
  KTRY(hh_gemm_launch(fmt, (const uint8_t*)w, (int)n_rows, (int)n_cols, xq, xd, (int)seq_len, out, c->stream));
  return HH_OK;
}

int hh_rms_norm(hh_ctx* c, const float* x, const float* w, float eps, int64_t rows, int64_t n, float* out) {
  if (!c || !x || !w || !out) return fail(HH_ERR_INVALID, "null argument");
  if (n <= 0 || rows < 0) return fail(HH_ERR_DIM, "bad shape");
  KTRY(hh_rmsnorm_launch(x, w, eps, rows, n, out, c->stream));
  return HH_OK;
}

int hh_rope(hh_ctx* c, float* x, int n_heads, int hd, int rope_dim, const float* table, int max_seq, int pos) {
  if (!c || !x || !table) return fail(HH_ERR_INVALID, "null argument");
  if (rope_dim > hd || rope_dim % 2 || pos < 0) return fail(HH_ERR_DIM, "bad rope shape");
  KTRY(hh_rope_launch(x, n_heads, hd, rope_dim, table, max_seq, pos, c->stream));
  return HH_OK;
}

int hh_attention(hh_ctx* c, const float* q, const float* k, const float* v, int n_heads, int n_kv, int hd,
                 int max_seq, int seq_len, float* out) {
  if (!c || !q || !k || !v || !out) return fail(HH_ERR_INVALID, "null argument");
  if (n_kv <= 0 || n_heads % n_kv || (hd != 128 && hd != 256))
    return fail(HH_ERR_DIM, "unsupported attention geometry (head_dim 128 or 256)");
  if (seq_len <= 0 || seq_len > max_seq) return fail(HH_ERR_RANGE, "seq_len out of range");
  int G = n_heads / n_kv;
  if (G > 8) return fail(HH_ERR_DIM, "more than 8 query heads per kv head (n_heads / n_kv_heads)");
  int chunk = 8192 / hd;
  int splits = (seq_len + chunk - 1) / chunk;
  // split partials live in a context scratch buffer grown on demand; the
  // per-kv-head counters are reset by the kernel itself after use
  size_t need = sizeof(float) * (size_t)n_kv * splits * G * (hd + 2) + sizeof(int) * 1024;
  if (n_kv > 1024) return fail(HH_ERR_DIM, "too many kv heads");
  if (c->attn_scratch_bytes < need) {
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (c->attn_scratch) HIP_TRY(hipFree(c->attn_scratch));
    c->attn_scratch = nullptr;
    c->attn_scratch_bytes = 0;
    HIP_TRY(hipMalloc(&c->attn_scratch, need));
    HIP_TRY(hipMemset(c->attn_scratch, 0, need));
    c->attn_scratch_bytes = need;
  }
  int* cnt = (int*)c->attn_scratch;
  float* po = (float*)((char*)c->attn_scratch + sizeof(int) * 1024);
  float* pml = po + (size_t)n_kv * splits * G * hd;
  AttnArgs a{};
  a.qkv = q;
  a.n_heads = n_heads;
  a.n_kv = n_kv;
  a.hd = hd;
  a.k_cache = const_cast<float*>(k);
  a.v_cache = const_cast<float*>(v);
  a.max_seq = max_seq;
  a.fixed_seq = seq_len;
  a.chunk = chunk;
  a.max_splits = splits;
  a.part_o = po;
  a.part_ml = pml;
  a.counters = cnt;
  a.out_f32 = out;
  int rc = hh_attn_launch(a, c->stream);
  if (rc) return fail(HH_ERR_HIP, std::string("attention launch: ") + hipGetErrorString(hipGetLastError()));
  return HH_OK;
}

int hh_attention_prefill(hh_ctx* c, const float* q, const float* k, const float* v, int n_heads, int n_kv, int hd,
                         int max_seq, int pos0, int n_tok, int mode, float* out) {
  if (!c || !q || !k || !v || !out) return fail(HH_ERR_INVALID, "null argument");
  if (n_kv <= 0 || n_heads % n_kv || (hd != 128 && hd != 256))
    return fail(HH_ERR_DIM, "unsupported attention geometry (head_dim 128 or 256)");
  if (n_heads / n_kv > 8) return fail(HH_ERR_DIM, "more than 8 query heads per kv head (n_heads / n_kv_heads)");
  if (pos0 < 0 || n_tok <= 0 || pos0 + n_tok > max_seq) return fail(HH_ERR_RANGE, "positions out of range");
  if (mode != 0 && mode != 1) return fail(HH_ERR_INVALID, "mode must be 0 (split/merge) or 1 (MFMA)");
  // the output rows go out as f32 (the folded-model hand-off); the Q8_0 row
  // arguments are unused then
  if (mode == 1) {
    if (hh_prefill_attn_mfma_launch(hd, q, k, v, n_heads, n_kv, max_seq, pos0, 0, n_tok, nullptr, 0, 0, nullptr,
                                    nullptr, out, c->stream))
      return fail(HH_ERR_HIP, std::string("prefill attention launch: ") + hipGetErrorString(hipGetLastError()));
    return HH_OK;
  }
  const int G = n_heads / n_kv, n_chunks = (pos0 + n_tok + 8192 / hd - 1) / (8192 / hd);
  const size_t per_tok = (size_t)n_kv * n_chunks * G * (hd + 2) * sizeof(float);
  const int TA = (int)std::max<size_t>(16, std::min<size_t>((n_tok + 15) / 16 * 16, ((size_t)1 << 30) / per_tok / 16 * 16));
  const size_t need = per_tok * TA;
  if (c->attn_scratch_bytes < need) {
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (c->attn_scratch) HIP_TRY(hipFree(c->attn_scratch));
    c->attn_scratch = nullptr;
    c->attn_scratch_bytes = 0;
    HIP_TRY(hipMalloc(&c->attn_scratch, need));
    c->attn_scratch_bytes = need;
  }
  float* po = (float*)c->attn_scratch;
  float* pml = po + (size_t)TA * n_kv * n_chunks * G * hd;
  for (int t0 = 0; t0 < n_tok; t0 += TA)
    if (hh_prefill_attn_launch(hd, q, k, v, n_heads, n_kv, max_seq, pos0, t0, std::min(TA, n_tok - t0), n_chunks, po,
                               pml, nullptr, 0, 0, nullptr, nullptr, out, c->stream))
      return fail(HH_ERR_HIP, std::string("prefill attention launch: ") + hipGetErrorString(hipGetLastError()));
  return HH_OK;
}

int hh_attention_noalloc(hh_ctx* c, const float* q, const float* k, const float* v, int n_heads, int n_kv, int hd,
                         int max_seq, int seq_len, float* out) {
  if (!c || !q || !k || !v || !out) return fail(HH_ERR_INVALID, "null argument");
  if (n_kv <= 0 || n_heads % n_kv || (hd != 128 && hd != 256))
    return fail(HH_ERR_DIM, "unsupported attention geometry (head_dim 128 or 256)");
  if (seq_len <= 0 || seq_len > max_seq) return fail(HH_ERR_RANGE, "seq_len out of range");
  const int G = n_heads / n_kv;
  if (G > 8) return fail(HH_ERR_DIM, "more than 8 query heads per kv head (n_heads / n_kv_heads)");
  const int chunk = 8192 / hd;
  const int splits = (seq_len + chunk - 1) / chunk;
  const size_t need = sizeof(float) * (size_t)n_kv * splits * G * (hd + 2);
  if (need > HH_NOALLOC_SCRATCH_BYTES)
    return fail(HH_ERR_RANGE, "attention partials need " + std::to_string(need) +
                                  " bytes, beyond the 4 MiB scratch of hh_attention_noalloc");
  void* base = g_scratch_ptr[c->device];
  if (!base) return fail(HH_ERR_INVALID, "scratch not set up for this device");
  // every partial that the merge reads is written by the split pass of the
  // same call, so nothing needs clearing between calls
  float* po = (float*)base;
  float* pml = po + (size_t)n_kv * splits * G * hd;
  AttnArgs a{};
  a.qkv = q;
  a.n_heads = n_heads;
  a.n_kv = n_kv;
  a.hd = hd;
  a.k_cache = const_cast<float*>(k);
  a.v_cache = const_cast<float*>(v);
  a.max_seq = max_seq;
  a.fixed_seq = seq_len;
  a.chunk = chunk;
  a.max_splits = splits;
  a.part_o = po;
  a.part_ml = pml;
  a.out_f32 = out;
  int rc = hh_attn_launch(a, c->stream);
  if (rc) return fail(HH_ERR_HIP, std::string("attention launch: ") + hipGetErrorString(hipGetLastError()));
  return HH_OK;
}

int hh_argmax(hh_ctx* c, const float* logits, int64_t n, const uint32_t* past, int64_t n_past, float pen, int rule,
              uint32_t* out) {
  if (!c || !logits || !out || (n_past && !past)) return fail(HH_ERR_INVALID, "null argument");
  if (n <= 0 || n > (1ll << 31) - 1) return fail(HH_ERR_DIM, "bad length");
  if (rule != 0 && rule != 1) return fail(HH_ERR_INVALID, "rule must be 0 or 1");
  const int* counts = nullptr;
  if (rule == 0 && n_past > 0) {
    if (c->counts_n < n) {
      if (c->counts) hipFree(c->counts);
      HIP_TRY(hipMalloc(&c->counts, sizeof(int) * (size_t)n));
      c->counts_n = n;
    }
    KTRY(hh_fill_i32_launch(c->counts, n, 0, c->stream));
    KTRY(hh_count_tokens_launch(past, n_past, c->counts, c->stream));
    counts = c->counts;
  }
  KTRY(hh_argmax_launch(logits, n, counts, pen, rule, c->part_val, c->part_idx, c->counter, out, c->stream));
  return HH_OK;
}

// ---------------------------------------------------------------------------
// model
// ---------------------------------------------------------------------------

int hh_model_create(hh_ctx* ctx, const hh_model_config* cfg, hh_model** out) {
  if (!ctx || !cfg || !out) return fail(HH_ERR_INVALID, "null argument");
  const hh_model_config& c = *cfg;
  if (c.arch != 0 && c.arch != 1) return fail(HH_ERR_INVALID, "arch must be 0 (dense) or 1 (qwen35)");
  int wf = hh_fmt_of(c.wtype);
  if (wf < 0 || wf == 0) return fail(HH_ERR_DTYPE, "layer weights must be Q1_0/Q1_0_G128/Q2_0/PQ2_0/PTQ1_0");
  if (c.head_type != HH_Q8_0) return fail(HH_ERR_DTYPE, "token_embd/output must be Q8_0");
  if (c.d_model % 1024 || c.d_ffn % 1024 || c.n_layers <= 0 || c.vocab <= 0)
    return fail(HH_ERR_DIM, "d_model and d_ffn must be multiples of 1024");
  if (c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads || (c.head_dim != 128 && c.head_dim != 256))
    return fail(HH_ERR_DIM, "unsupported attention geometry (head_dim 128 or 256)");
  if (c.n_heads / c.n_kv_heads > 8)
    return fail(HH_ERR_DIM, "more than 8 query heads per kv head (n_heads / n_kv_heads)");
  if ((c.n_heads * c.head_dim) % 256) return fail(HH_ERR_DIM, "n_heads*head_dim must be a multiple of 256");
  if (c.max_seq <= 0) return fail(HH_ERR_DIM, "max_seq must be positive");
  if (c.kv_type != HH_F32 && c.kv_type != HH_Q8_0) return fail(HH_ERR_DTYPE, "kv_type must be F32 or Q8_0");
  if (c.arch == 1) {
    if (c.full_attn_interval <= 0 || c.ssm_n_k_heads <= 0 || c.ssm_n_v_heads % c.ssm_n_k_heads ||
        c.ssm_head_dim != 128 || c.ssm_conv_kernel < 2 || c.ssm_conv_kernel > 8)
      return fail(HH_ERR_DIM, "unsupported qwen35 recurrent geometry");
  }
  if (c.had_block != 0) {
    // the fold (qwen35.rs:532-610) applies to qwen35 models; every folded
    // width must hold whole chunks and fit the rotation prologues
    const int nq_ = c.n_heads * c.head_dim, vd_ = c.ssm_n_v_heads * c.ssm_head_dim;
    const int ws[4] = {c.d_model, c.d_ffn, nq_, vd_};
    if (c.arch != 1 || c.had_block < 2 || (c.had_block & (c.had_block - 1)))
      return fail(HH_ERR_DIM, "had_block must be a power of two on a qwen35 model");
    for (int w : ws)
      if (w % c.had_block || w % 1024 || w > 20480) return fail(HH_ERR_DIM, "folded width not a multiple of had_block");
  }
  HIP_TRY(hipSetDevice(ctx->device));
  hh_model* m = new hh_model();
  // every early return below releases what was allocated so far
  struct Guard {
    hh_model* m;
    ~Guard() { if (m) hh_model_destroy(m); }
  } guard{m};
  m->ctx = ctx;
  m->cfg = c;
  m->wfmt = wf;
  m->rope_dim = c.rope_dim > 0 ? c.rope_dim : c.head_dim;
  declare(m);
  // arena: every tensor, 256-byte aligned, fused groups contiguous in declaration order
  size_t off = 0;
  std::vector<size_t> offs(m->tensors.size());
  for (size_t i = 0; i < m->tensors.size(); ++i) {
    Tensor& t = m->tensors[i];
    bool fuse_prev = false;
    const std::string& n = t.name;
    auto ends = [&](const char* suf) { return n.size() > strlen(suf) && n.compare(n.size() - strlen(suf), strlen(suf), suf) == 0; };
    if (ends("attn_k.weight") || ends("attn_v.weight") || ends("attn_gate.weight") || ends("ffn_up.weight")) fuse_prev = true;
    if (!fuse_prev) off = align256(off);
    offs[i] = off;
    off += t.nbytes;
  }
  m->arena_bytes = align256(off);
  hipError_t e = hipMalloc(&m->arena, m->arena_bytes);
  if (e != hipSuccess) {
    m->arena = nullptr;
    return fail(HH_ERR_OOM, "weight arena allocation failed (" + std::to_string(m->arena_bytes) + " bytes)");
  }
  for (size_t i = 0; i < m->tensors.size(); ++i) m->tensors[i].d = m->arena + offs[i];
  m->token_embd = find(m, "token_embd.weight");
  m->output = m->cfg.arch == 1 && m->cfg.had_block > 0 && (m->cfg.had_flags & HH_HAD_TIED_OUTPUT)
                  ? m->token_embd
                  : find(m, "output.weight");
  m->output_norm = find(m, "output_norm.weight");
  // layers
  int hd = c.head_dim, nq = c.n_heads * hd, nkv = c.n_kv_heads * hd;
  int kdim = c.ssm_n_k_heads * c.ssm_head_dim, vdim = c.ssm_n_v_heads * c.ssm_head_dim;
  int conv_dim = 2 * kdim + vdim;
  m->layers.resize(c.n_layers);
  int n_attn = 0, n_gdn = 0;
  char b[96];
  for (int i = 0; i < c.n_layers; ++i) {
    Layer& L = m->layers[i];
    L.gdn = (c.arch == 1) && ((i + 1) % c.full_attn_interval != 0);
    auto T = [&](const char* s) -> Tensor* { snprintf(b, sizeof b, "blk.%d.%s", i, s); return find(m, b); };
    L.attn_norm = (float*)T("attn_norm.weight")->d;
    L.ffn_norm = (float*)(c.arch == 1 ? T("post_attention_norm.weight") : T("ffn_norm.weight"))->d;
    if (L.gdn) {
      L.w_in = T("attn_qkv.weight")->d;
      L.n_in = conv_dim + vdim;
      L.w_out = T("ssm_out.weight")->d;
      L.ssm_conv = (float*)T("ssm_conv1d.weight")->d;
      L.ssm_dt = (float*)T("ssm_dt.bias")->d;
      L.ssm_a = (float*)T("ssm_a")->d;
      L.ssm_alpha = (float*)T("ssm_alpha.weight")->d;
      L.ssm_beta = (float*)T("ssm_beta.weight")->d;
      L.ssm_norm = (float*)T("ssm_norm.weight")->d;
      n_gdn++;
    } else {
      L.w_in = T("attn_q.weight")->d;
      L.n_in = (c.attn_out_gate ? 2 * nq : nq) + 2 * nkv;
      L.w_out = T("attn_output.weight")->d;
      if (c.qk_norm) {
        L.q_norm = (float*)T("attn_q_norm.weight")->d;
        L.k_norm = (float*)T("attn_k_norm.weight")->d;
      }
      L.attn_idx = n_attn++;
    }
    L.w_gu = T("ffn_gate.weight")->d;
    L.w_down = T("ffn_down.weight")->d;
  }
  // KV cache: [attn layer][K|V][kv_head][max_seq][hd] f32 (kvcache.rs:11-39), or
  // Q8_0 rows (kvcache.rs:41-57): int8 [kv_head][max_seq][hd], then the f16
  // block scales [kv_head][max_seq][hd/32] (136 B per row at hd 128, as the
  // reference's 34-byte blocks)
  m->kv_rows = (c.max_seq + 63) / 64 * 64;
  if ((m->kv_rows / 64) % 2 == 0) m->kv_rows += 64;
  size_t per = (size_t)c.n_kv_heads * m->kv_rows * hd;
  const size_t cache_bytes = c.kv_type == HH_Q8_0 ? align256(per + per / 32 * 2) : per * sizeof(float);
  m->kv_bytes = cache_bytes * 2 * (size_t)n_attn;
  if (m->kv_bytes) {
    e = hipMalloc(&m->kv, m->kv_bytes);
    if (e != hipSuccess) { m->kv = nullptr; return fail(HH_ERR_OOM, "KV cache allocation failed"); }
  }
  size_t rec_per = 0;
  if (c.arch == 1) {
    // recurrent state, then the conv window in two buffers (the decode step at
    // position p reads buffer p & 1 and writes buffer (p + 1) & 1)
    rec_per = (size_t)c.ssm_n_v_heads * c.ssm_head_dim * c.ssm_head_dim +
              2 * (size_t)conv_dim * (c.ssm_conv_kernel - 1);
    m->rec_bytes = sizeof(float) * rec_per * (size_t)n_gdn;
    e = hipMalloc(&m->rec, m->rec_bytes);
    if (e != hipSuccess) { m->rec = nullptr; return fail(HH_ERR_OOM, "recurrent state allocation failed"); }
  }
  if (m->kv) HIP_TRY(hipMemset(m->kv, 0, m->kv_bytes));
  if (m->rec) HIP_TRY(hipMemset(m->rec, 0, m->rec_bytes));
  int ai = 0, gi = 0;
  for (auto& L : m->layers) {
    if (L.gdn) {
      L.gdn_state = m->rec + rec_per * gi;
      L.conv_state = L.gdn_state + (size_t)c.ssm_n_v_heads * c.ssm_head_dim * c.ssm_head_dim;
      gi++;
    } else {
      L.k_cache = (float*)((uint8_t*)m->kv + cache_bytes * 2 * ai);
      L.v_cache = (float*)((uint8_t*)L.k_cache + cache_bytes);
      ai++;
    }
  }
  // RoPE table (ops.rs:78-138), computed on the host with libm like the reference
  {
    int half = m->rope_dim / 2;
    std::vector<float> inv(half), tab((size_t)c.max_seq * m->rope_dim);
    for (int i = 0; i < half; ++i) inv[i] = 1.0f / powf(c.rope_theta, 2.0f * (float)i / (float)m->rope_dim);
    for (int p = 0; p < c.max_seq; ++p)
      for (int i = 0; i < half; ++i) {
        float f = (float)p * 1.0f * inv[i];
        tab[(size_t)p * half * 2 + i] = sinf(f);
        tab[(size_t)p * half * 2 + half + i] = cosf(f);
      }
    HIP_TRY(hipMalloc(&m->rope, tab.size() * sizeof(float)));
    HIP_TRY(hipMemcpy(m->rope, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice));
  }
  // step buffers
  int wide = std::max(std::max(c.d_model, c.d_ffn), std::max((c.attn_out_gate ? 2 : 1) * nq + 2 * nkv, conv_dim + vdim));
  m->attn_chunk = 8192 / hd;
  m->attn_splits = (c.max_seq + m->attn_chunk - 1) / m->attn_chunk;
  int G = c.n_heads / c.n_kv_heads;
  // launch geometry of the GEMVs
  {
    int el = hh_unit_el(wf);
    int n_in_max = std::max((c.attn_out_gate ? 2 : 1) * nq + 2 * nkv, c.arch == 1 ? conv_dim + vdim : 0);
    m->rows_in = gemv_rows_for(n_in_max, c.d_model / el);
    m->rows_gu = 32;
    m->rows_out = gemv_rows_for(c.d_model, std::max(nq, vdim) / el);
    m->rows_down = gemv_rows_for(c.d_model, c.d_ffn / el);
    m->rows_head = gemv_rows_for(c.vocab, c.d_model / hh_unit_el(hh_fmt_of(c.head_type)));
    // whole 16-row groups per residual-add workgroup, so that it can hand the
    // RMSNorm tree nodes of the hidden state on (GemvArgs::sq_out); 1.7B (d
    // 2048: 8 -> 16 rows, 128 workgroups) 1045 -> 1054 tok/s
    if (c.d_model % 64 == 0 && c.d_model <= 4096 && c.had_block == 0) {
      m->rows_out = (m->rows_out + 15) / 16 * 16;
      m->rows_down = (m->rows_down + 15) / 16 * 16;
    }
  }
  int head_wg = std::max(256, (c.vocab + m->rows_head - 1) / m->rows_head);
  m->max_out = c.max_seq + 8;
  HIP_TRY(hipMalloc(&m->hidden, sizeof(float) * c.d_model));
  HIP_TRY(hipMalloc(&m->hidden_sq, sizeof(float) * (c.d_model / 16 + 4)));
  HIP_TRY(hipMalloc(&m->proj, sizeof(float) * wide));
  HIP_TRY(hipMalloc(&m->act_mid, hh_packed_bytes(std::max(nq, vdim)) + 64));
  HIP_TRY(hipMalloc(&m->act_ffn, hh_packed_bytes(c.d_ffn) + 64));
  HIP_TRY(hipMalloc(&m->logits, sizeof(float) * c.vocab));
  HIP_TRY(hipMalloc(&m->head_pv, sizeof(float) * head_wg));
  HIP_TRY(hipMalloc(&m->head_pi, sizeof(int) * head_wg));
  HIP_TRY(hipMalloc(&m->counters, sizeof(int) * 256));
  HIP_TRY(hipMemset(m->counters, 0, sizeof(int) * 256));
  HIP_TRY(hipMalloc(&m->attn_po, sizeof(float) * (size_t)c.n_kv_heads * m->attn_splits * G * hd));
  HIP_TRY(hipMalloc(&m->attn_pml, sizeof(float) * (size_t)c.n_kv_heads * m->attn_splits * G * 2));
  // raw alpha / beta dots of the GDN input projection, [2 n_v]
  HIP_TRY(hipMalloc(&m->gdn_scratch, sizeof(float) * (size_t)(2 * c.ssm_n_v_heads + 64)));
  if (c.had_block > 0) {
    size_t tot = 0;
    for (int w : {c.d_model, c.d_ffn, nq, vdim}) {
      bool seen = w <= 0;
      for (auto& so : m->sign_off) seen = seen || so.first == w;
      if (!seen) { m->sign_off.push_back({w, tot}); tot += (size_t)w; }
    }
    std::vector<float> ones(tot, 1.0f);
    HIP_TRY(hipMalloc(&m->had_signs, sizeof(float) * tot));
    HIP_TRY(hipMemcpy(m->had_signs, ones.data(), sizeof(float) * tot, hipMemcpyHostToDevice));
    HIP_TRY(hipMalloc(&m->rot_f32, sizeof(float) * (size_t)std::max(std::max(nq, vdim), c.d_ffn)));
  }
  HIP_TRY(hipMalloc(&m->counts, sizeof(int) * c.vocab));
  HIP_TRY(hipMemset(m->counts, 0, sizeof(int) * c.vocab));
  HIP_TRY(hipMalloc(&m->prompt, sizeof(uint32_t) * (c.max_seq + 8)));
  HIP_TRY(hipMalloc(&m->out_tokens, sizeof(uint32_t) * m->max_out));
  HIP_TRY(hipMalloc(&m->state, sizeof(StepState)));
  HIP_TRY(hipMemset(m->state, 0, sizeof(StepState)));
  HIP_TRY(hipEventCreate(&m->ev0));
  HIP_TRY(hipEventCreate(&m->ev1));
  HIP_TRY(hipEventCreate(&m->ev2));
  HIP_TRY(hipEventCreate(&m->evp));
  {
    const char* e = getenv("HH_BATCHED_PREFILL");
    m->batched_prefill = (e && e[0] == '0') ? 0 : 1;
    const char* g = getenv("HH_GDN_CHUNKED");
    m->gdn_chunked = (g && g[0] == '1') ? 1 : 0;
    const char* pa = getenv("HH_PREFILL_ATTN");
    m->prefill_attn_mfma = (pa && strcmp(pa, "mfma") == 0) ? 1 : 0;
    // hh_model_generate replays 8 decode steps per graph launch (the launch
    // boundary costs ~5 us per step otherwise: 8B step 1.662 -> 1.657 ms)
    m->graph_steps = 8;
  }
  HIP_TRY(hipDeviceSynchronize());
  int rc = capture(m);
  if (rc) return fail(rc, "graph capture: " + std::string(g_err));
  guard.m = nullptr;
  *out = m;
  return HH_OK;
}

int hh_model_destroy(hh_model* m) {
  if (!m) return HH_OK;
  hipSetDevice(m->ctx->device);
  hipStreamSynchronize(m->ctx->stream);
  if (m->gexec) hipGraphExecDestroy(m->gexec);
  if (m->graph) hipGraphDestroy(m->graph);
  if (m->gexec_n) hipGraphExecDestroy(m->gexec_n);
  if (m->graph_n) hipGraphDestroy(m->graph_n);
  if (m->gexec_ne) hipGraphExecDestroy(m->gexec_ne);
  if (m->graph_ne) hipGraphDestroy(m->graph_ne);
  void* bufs[] = {m->arena, m->kv, m->rec, m->rope, m->hidden, m->hidden_sq, m->proj, m->act_mid, m->act_ffn, m->logits,
                  m->head_pv, m->head_pi, m->counters, m->attn_po, m->attn_pml, m->gdn_scratch, m->counts,
                  m->prompt, m->out_tokens, m->state, m->had_signs, m->rot_f32};
  for (void* p : bufs)
    if (p) hipFree(p);
  if (m->ev0) hipEventDestroy(m->ev0);
  if (m->ev1) hipEventDestroy(m->ev1);
  if (m->ev2) hipEventDestroy(m->ev2);
  if (m->evp) hipEventDestroy(m->evp);
  if (m->pf_buf) hipFree(m->pf_buf);
  delete m;
  return HH_OK;
}

int hh_model_download_state(hh_model* m, int gdn_index, float* host, size_t n_floats) {
  if (!m || !host) return fail(HH_ERR_INVALID, "null argument");
  const hh_model_config& c = m->cfg;
  const size_t per = (size_t)c.ssm_n_v_heads * c.ssm_head_dim * c.ssm_head_dim;
  int gi = 0;
  for (const Layer& L : m->layers) {
    if (!L.gdn) continue;
    if (gi++ != gdn_index) continue;
    if (n_floats != per) return fail(HH_ERR_DIM, "state holds n_v * hd * hd floats");
    HIP_TRY(hipSetDevice(m->ctx->device));
    HIP_TRY(hipStreamSynchronize(m->ctx->stream));
    HIP_TRY(hipMemcpy(host, L.gdn_state, per * sizeof(float), hipMemcpyDeviceToHost));
    return HH_OK;
  }
  return fail(HH_ERR_RANGE, "no such Gated-DeltaNet layer");
}

int hh_model_set_hadamard_signs(hh_model* m, int width, const float* signs) {
  if (!m || !signs) return fail(HH_ERR_INVALID, "null argument");
  if (m->cfg.had_block <= 0) return fail(HH_ERR_INVALID, "model has no Hadamard fold (had_block 0)");
  for (int i = 0; i < width; ++i)
    if (signs[i] != 1.0f && signs[i] != -1.0f) return fail(HH_ERR_INVALID, "hadamard sign values must be +/-1");
  float* dst = const_cast<float*>(signs_of(m, width));
  if (!dst) return HH_OK;   // a width this model does not fold
  HIP_TRY(hipSetDevice(m->ctx->device));
  HIP_TRY(hipMemcpy(dst, signs, sizeof(float) * (size_t)width, hipMemcpyHostToDevice));
  return HH_OK;
}

int hh_model_upload_tensor(hh_model* m, const char* name, int type, int64_t ne0, int64_t ne1, const void* host,
                           size_t nbytes) {
  if (!m || !name || !host) return fail(HH_ERR_INVALID, "null argument");
  Tensor* t = find(m, name);
  if (!t) return fail(HH_ERR_NOT_FOUND, std::string("Tensor not found: ") + name);
  if (t->type != type) return fail(HH_ERR_DTYPE, std::string("dtype mismatch for ") + name);
  if (t->cols != ne0 || t->rows != ne1 || t->nbytes != nbytes)
    return fail(HH_ERR_DIM, std::string("shape mismatch for ") + name);
  HIP_TRY(hipMemcpyAsync(t->d, host, nbytes, hipMemcpyHostToDevice, m->ctx->stream));
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  m->ssm_a_negative = -1;
  return HH_OK;
}

int hh_model_download_tensor(hh_model* m, const char* name, void* host, size_t nbytes) {
  if (!m || !name || !host) return fail(HH_ERR_INVALID, "null argument");
  Tensor* t = find(m, name);
  if (!t) return fail(HH_ERR_NOT_FOUND, std::string("Tensor not found: ") + name);
  if (nbytes != t->nbytes) return fail(HH_ERR_DIM, "byte size mismatch");
  HIP_TRY(hipMemcpyAsync(host, t->d, nbytes, hipMemcpyDeviceToHost, m->ctx->stream));
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  return HH_OK;
}

int hh_model_tensor_count(hh_model* m) { return m ? (int)m->tensors.size() : 0; }

int hh_model_tensor_info(hh_model* m, int i, const char** name, int* type, int64_t* ne0, int64_t* ne1,
                         size_t* nbytes) {
  if (!m || i < 0 || i >= (int)m->tensors.size()) return fail(HH_ERR_INVALID, "bad tensor index");
  const Tensor& t = m->tensors[i];
  if (name) *name = t.name.c_str();
  if (type) *type = t.type;
  if (ne0) *ne0 = t.cols;
  if (ne1) *ne1 = t.rows;
  if (nbytes) *nbytes = t.nbytes;
  return HH_OK;
}

int hh_model_synthesize(hh_model* m, uint64_t seed) {
  if (!m) return fail(HH_ERR_INVALID, "null model");
  for (const Tensor& t : m->tensors) {
    float cc = t.std / 37837.227f;
    float cq = cc / 128.0f;
    KTRY(hh_synth_launch(t.type, name_key(seed, t.name.c_str()), t.rows, t.cols, cc, cq, t.mean, t.d,
                         m->ctx->stream));
  }
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  m->ssm_a_negative = -1;
  return HH_OK;
}

int hh_model_reset(hh_model* m) {
  if (!m) return fail(HH_ERR_INVALID, "null model");
  hipStream_t s = m->ctx->stream;
  if (m->kv) HIP_TRY(hipMemsetAsync(m->kv, 0, m->kv_bytes, s));
  if (m->rec) HIP_TRY(hipMemsetAsync(m->rec, 0, m->rec_bytes, s));
  HIP_TRY(hipMemsetAsync(m->counts, 0, sizeof(int) * m->cfg.vocab, s));
  HIP_TRY(hipStreamSynchronize(s));
  return HH_OK;
}

int hh_model_prefill_kv_synthetic(hh_model* m, uint64_t seed, int n_pos) {
  if (!m) return fail(HH_ERR_INVALID, "null model");
  if (n_pos < 0 || n_pos > m->cfg.max_seq) return fail(HH_ERR_RANGE, "n_pos beyond max_seq");
  float cs = 1.0f / 37837.227f;
  char b[64];
  for (int i = 0; i < m->cfg.n_layers; ++i) {
    Layer& L = m->layers[i];
    if (L.gdn) continue;
    auto synth = m->cfg.kv_type == HH_Q8_0 ? hh_kv_synth_q8_launch : hh_kv_synth_launch;
    snprintf(b, sizeof b, "blk.%d.kv_k", i);
    KTRY(synth(name_key(seed, b), n_pos, m->cfg.n_kv_heads, m->cfg.head_dim, m->kv_rows, cs, L.k_cache,
               m->ctx->stream));
    snprintf(b, sizeof b, "blk.%d.kv_v", i);
    KTRY(synth(name_key(seed, b), n_pos, m->cfg.n_kv_heads, m->cfg.head_dim, m->kv_rows, cs, L.v_cache,
               m->ctx->stream));
  }
  HIP_TRY(hipStreamSynchronize(m->ctx->stream));
  return HH_OK;
}

int hh_model_set_cancel(hh_model* m, int cancel) {
  if (!m) return fail(HH_ERR_INVALID, "null model");
  m->cancel = cancel;
  return HH_OK;
}

int hh_model_forward(hh_model* m, uint32_t token, int pos, float* logits_host, uint32_t* argmax_host) {
  if (!m) return fail(HH_ERR_INVALID, "null model");
  if (m->cancel) return fail(HH_ERR_CANCELLED, "Cancelled");
  if (token >= (uint32_t)m->cfg.vocab) return fail(HH_ERR_RANGE, "token id out of range");
  if (pos < 0 || pos >= m->cfg.max_seq) return fail(HH_ERR_RANGE, "position beyond max_seq");
  hipStream_t s = m->ctx->stream;
  StepState st{};
  st.pos = pos;
  st.step = 0;
  st.token = (int)token;
  st.n_prompt = 1;
  st.update = 0;
  HIP_TRY(hipMemcpyAsync(m->state, &st, sizeof st, hipMemcpyHostToDevice, s));
  HIP_TRY(hipGraphLaunch(m->gexec, s));
  if (logits_host)
    HIP_TRY(hipMemcpyAsync(logits_host, m->logits, sizeof(float) * m->cfg.vocab, hipMemcpyDeviceToHost, s));
  StepState out{};
  HIP_TRY(hipMemcpyAsync(&out, m->state, sizeof out, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  if (argmax_host) *argmax_host = (uint32_t)out.argmax;
  return HH_OK;
}

int hh_model_generate(hh_model* m, const uint32_t* prompt, int n_prompt, int start_pos, int n_gen, float pen,
                      uint32_t* out_tokens, float* last_logits) {
  if (!m || !prompt || (n_gen > 0 && !out_tokens)) return fail(HH_ERR_INVALID, "null argument");
  if (n_prompt <= 0) return fail(HH_ERR_INVALID, "Empty prompt");
  if (n_gen < 0 || n_gen > m->max_out) return fail(HH_ERR_RANGE, "n_gen out of range");
  if (start_pos < 0 || start_pos + n_prompt + n_gen > m->cfg.max_seq)
    return fail(HH_ERR_RANGE, "sequence exceeds max_seq");
  for (int i = 0; i < n_prompt; ++i)
    if (prompt[i] >= (uint32_t)m->cfg.vocab) return fail(HH_ERR_RANGE, "prompt token out of range");
  if (m->cancel) return fail(HH_ERR_CANCELLED, "Cancelled");
  hipStream_t s = m->ctx->stream;
  HIP_TRY(hipEventRecord(m->evp, s));
  HIP_TRY(hipMemcpyAsync(m->prompt, prompt, sizeof(uint32_t) * n_prompt, hipMemcpyHostToDevice, s));
  // past_tokens = [last prompt token] (mod.rs:2879); counts start from it
  KTRY(hh_fill_i32_launch(m->counts, m->cfg.vocab, 0, s));
  KTRY(hh_count_tokens_launch(m->prompt + (n_prompt - 1), 1, m->counts, s));
  StepState st{};
  st.pos = start_pos;
  st.step = 0;
  st.token = (int)prompt[0];
  st.n_prompt = n_prompt;
  st.update = 1;
  st.pen = pen;
  HIP_TRY(hipMemcpyAsync(m->state, &st, sizeof st, hipMemcpyHostToDevice, s));
  // prompt: all but the last token in one batched pass (the reference feeds
  // hybrids token by token, qwen35.rs:1693-1700; the batched GDN pass leaves
  // the same state); the last prompt token runs the decode step, which yields
  // the first generated token.
  int fed = 0;
  if (m->batched_prefill && n_prompt >= 2) {
    KTRY(prefill_batched(m, m->prompt, n_prompt - 1, start_pos));
    fed = n_prompt - 1;
    st.pos = start_pos + fed;
    st.step = fed;
    st.token = (int)prompt[fed];
    HIP_TRY(hipMemcpyAsync(m->state, &st, sizeof st, hipMemcpyHostToDevice, s));
  }
  for (int i = fed; i < n_prompt; ++i) HIP_TRY(hipGraphLaunch(m->gexec, s));
  HIP_TRY(hipEventRecord(m->ev0, s));
  // decode steps: forward each generated token (the last forward only when its logits are wanted)
  int steps = n_gen - 1 + (last_logits ? 1 : 0);
  // the last prompt step's k_head_final embedded the first generated token
  int i = 0;
  for (; i + m->graph_steps <= steps; i += m->graph_steps) HIP_TRY(hipGraphLaunch(m->gexec_n, s));
  for (; i < steps; ++i) HIP_TRY(hipGraphLaunch(m->gexec_ne, s));
  HIP_TRY(hipEventRecord(m->ev1, s));
  if (n_gen > 0)
    HIP_TRY(hipMemcpyAsync(out_tokens, m->out_tokens, sizeof(uint32_t) * n_gen, hipMemcpyDeviceToHost, s));
  if (last_logits)
    HIP_TRY(hipMemcpyAsync(last_logits, m->logits, sizeof(float) * m->cfg.vocab, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  float ms = 0.0f;
  HIP_TRY(hipEventElapsedTime(&ms, m->ev0, m->ev1));
  m->last_decode_ms = ms;
  HIP_TRY(hipEventElapsedTime(&ms, m->evp, m->ev0));
  m->last_prefill_ms = ms;
  return HH_OK;
}

int hh_read_bandwidth(hh_ctx* c, size_t nbytes, int reps, double* gbps) {
  if (!c || !gbps || reps <= 0) return fail(HH_ERR_INVALID, "null argument");
  const size_t unit = (size_t)16 * 8 * 512 * 1024;   // one pass of the probe's grid
  if (nbytes < unit || nbytes % unit) return fail(HH_ERR_DIM, "nbytes must be a positive multiple of 64 MiB");
  HIP_TRY(hipSetDevice(c->device));
  void* p = nullptr;
  HIP_TRY(hipMalloc(&p, nbytes));
  struct Free {
    void* p;
    ~Free() { hipFree(p); }
  } guard{p};
  HIP_TRY(hipMemsetAsync(p, 1, nbytes, c->stream));
  hipEvent_t a = nullptr, b = nullptr;
  HIP_TRY(hipEventCreate(&a));
  struct FreeEv {
    hipEvent_t e[2];
    ~FreeEv() {
      for (hipEvent_t x : e)
        if (x) hipEventDestroy(x);
    }
  } evs{{a, nullptr}};
  HIP_TRY(hipEventCreate(&b));
  evs.e[1] = b;
  KTRY(hh_read_probe_launch(p, (int64_t)nbytes, c->counter, c->stream));   // warm-up
  HIP_TRY(hipEventRecord(a, c->stream));
  for (int r = 0; r < reps; ++r) KTRY(hh_read_probe_launch(p, (int64_t)nbytes, c->counter, c->stream));
  HIP_TRY(hipEventRecord(b, c->stream));
  HIP_TRY(hipEventSynchronize(b));
  float ms = 0.0f;
  HIP_TRY(hipEventElapsedTime(&ms, a, b));
  *gbps = (double)nbytes * reps / (ms * 1e-3) / 1e9;
  return HH_OK;
}

int hh_model_time_stages(hh_model* m, int layer, int iters, double* out_ms, int n_out) {
  if (!m || !out_ms || iters <= 0) return fail(HH_ERR_INVALID, "bad argument");
  if (layer < 0 || layer >= m->cfg.n_layers) return fail(HH_ERR_RANGE, "layer out of range");
  hipStream_t s = m->ctx->stream;
  // keep the head kernel in decode mode with the state untouched between launches
  StepState st{};
  HIP_TRY(hipMemcpyAsync(&st, m->state, sizeof st, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  StepState fixed = st;
  fixed.update = 0;
  fixed.n_prompt = 1;
  fixed.step = 0;
  HIP_TRY(hipMemcpyAsync(m->state, &fixed, sizeof fixed, hipMemcpyHostToDevice, s));
  // Each stage is launched for every layer in turn (layers of one kind only),
  // so its weights stream from HBM as in a real step rather than from the
  // 256 MB last-level cache a single repeated layer would sit in.
  const bool want_gdn = m->layers[layer].gdn;
  std::vector<int> same;
  for (int li = 0; li < m->cfg.n_layers; ++li)
    if (m->layers[li].gdn == want_gdn) same.push_back(li);
  for (int stg = 0; stg < n_out && stg < 7; ++stg) {
    int rc = enqueue_step(m, s, layer, 1u << stg);   // warm
    if (rc) return rc;
    HIP_TRY(hipEventRecord(m->ev0, s));
    for (int i = 0; i < iters; ++i) {
      rc = enqueue_step(m, s, same[i % same.size()], 1u << stg);
      if (rc) return rc;
    }
    HIP_TRY(hipEventRecord(m->ev1, s));
    HIP_TRY(hipEventSynchronize(m->ev1));
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, m->ev0, m->ev1));
    out_ms[stg] = (double)ms / iters;
  }
  HIP_TRY(hipMemcpyAsync(m->state, &st, sizeof st, hipMemcpyHostToDevice, s));
  HIP_TRY(hipStreamSynchronize(s));
  return HH_OK;
}

int hh_model_prefill(hh_model* m, const uint32_t* tokens, int n, int start_pos) {
  if (!m || !tokens) return fail(HH_ERR_INVALID, "null argument");
  if (n <= 0) return fail(HH_ERR_INVALID, "Empty prompt");
  if (start_pos < 0 || start_pos + n > m->cfg.max_seq) return fail(HH_ERR_RANGE, "sequence exceeds max_seq");
  for (int i = 0; i < n; ++i)
    if (tokens[i] >= (uint32_t)m->cfg.vocab) return fail(HH_ERR_RANGE, "prompt token out of range");
  if (m->cancel) return fail(HH_ERR_CANCELLED, "Cancelled");
  hipStream_t s = m->ctx->stream;
  uint32_t* dt = nullptr;
  HIP_TRY(hipMalloc(&dt, sizeof(uint32_t) * n));
  HIP_TRY(hipMemcpyAsync(dt, tokens, sizeof(uint32_t) * n, hipMemcpyHostToDevice, s));
  HIP_TRY(hipEventRecord(m->evp, s));
  int rc = prefill_batched(m, dt, n, start_pos);
  HIP_TRY(hipEventRecord(m->ev2, s));
  HIP_TRY(hipStreamSynchronize(s));
  hipFree(dt);
  if (rc) return rc;
  float ms = 0.0f;
  HIP_TRY(hipEventElapsedTime(&ms, m->evp, m->ev2));
  m->last_prefill_ms = ms;
  return HH_OK;
}

int hh_model_last_prefill_ms(hh_model* m, double* ms) {
  if (!m || !ms) return fail(HH_ERR_INVALID, "null argument");
  *ms = m->last_prefill_ms;
  return HH_OK;
}

int hh_model_last_decode_ms(hh_model* m, double* ms) {
  if (!m || !ms) return fail(HH_ERR_INVALID, "null argument");
  *ms = m->last_decode_ms;
  return HH_OK;
}

}  // extern "C"
