// hh_kernels.h — launch interface between the runtime (hh_runtime.hip) and the
// gfx950 kernels.  Internal to the library.
#pragma once
#include "hh_device.h"

struct GemvArgs {
  const uint8_t* w;     // matrix base, rows contiguous in native block layout
  int n_rows;           // rows (EPI_SILU: unused; half_rows gives the gate count)
  int K;                // n_cols
  int P;                // units per row (set by the launcher)
  int rows_per_wg;      // rows per workgroup (EPI_SILU: unused, blocks of 32 gate rows)
  int half_rows;        // EPI_SILU: row offset of the up half
  // prologue inputs
  const float* x;       // PRO_RMSNORM: f32 vector
  const float* norm_w;  // PRO_RMSNORM: weight
  float eps;
  const uint8_t* act;   // PRO_PACKED: packed activation; PRO_STDQ8: Q8_0 blocks
  // epilogue outputs
  float* y;             // EPI_STORE / EPI_ADD target, EPI_LOGITS logits (may be null)
  uint8_t* act_out;     // EPI_SILU packed output
  int act_out_fmt;
  int act_out_k;
  // EPI_LOGITS
  StepState* state;
  const uint32_t* prompt;
  uint32_t* out_tokens;
  int max_out;
  int* counts;
  float pen;
  int rule;
  float* part_val;
  int* part_idx;
  int* counter;
  // Hadamard-folded prologues (PRO_NORMROT, PRO_F32ROT): the activation is
  // rotated (signs, then the WHT per had_block chunk) before Q8_0
  const float* signs;   // [K] +-1
  int had_block;
  int perm_nk, perm_rep;   // PRO_F32ROT: GDN grouped head order when perm_rep > 1 (head dim 128)
  // qwen35 GDN input projection (PRO_RMSNORM / PRO_NORMROT, EPI_STORE): workgroup
  // b < ab_rows also writes the f32 dot of the normed (unrotated) activation with
  // row b of [ssm_alpha (ab_n rows); ssm_beta (ab_n rows)] into ab_out[b]
  const float* ab_wa;
  const float* ab_wb;
  int ab_n, ab_rows;
  float* ab_out;
  // EPI_LOGITS: k_head_final also writes the embedding of the next step's token
  // into emb_out (null: not), with R^-1 for a latent table (emb_had > 0)
  const uint8_t* emb_table;
  int emb_type, emb_d, emb_had;
  const float* emb_signs;
  float* emb_out;
  // Sum-of-squares hand-off of the hidden state.  sq_out (EPI_ADD, rows per
  // workgroup a multiple of 16): for every 16 rows 16b.. of y written, the
  // node (s0 + s1) + (s2 + s3) of the RMSNorm tree, s_t = ((y0^2 + y1^2) +
  // y2^2) + y3^2 over rows 16b + 4t ..  sq_in (PRO_RMSNORM, EPI_LOGITS head;
  // K <= 4096): those nodes of x, so each wave finishes the sum by itself.
  float* sq_out;
  const float* sq_in;
};

// PRO_NORMROT: rms_norm(x, norm_w) then the fold, then Q8_0.
// PRO_F32ROT: an f32 vector x (optionally permuted to grouped head order), the fold, then Q8_0.
// EPI_SILU with y != null writes silu(g) * u as f32 into y instead of packed Q8_0.
// (hh_gemv_launch runs PRO_RMSNORM + EPI_STORE launches with small weight shares
// through an all-lanes variant of the same prologue.)
enum { HH_PRO_PACKED = 0, HH_PRO_RMSNORM = 1, HH_PRO_STDQ8 = 2, HH_PRO_NORMROT = 3, HH_PRO_F32ROT = 4 };
enum { HH_EPI_STORE = 0, HH_EPI_ADD = 1, HH_EPI_SILU = 2, HH_EPI_LOGITS = 3 };

int hh_fmt_of(int ggml_type);
int hh_unit_el(int fmt);
size_t hh_gemv_lds(int fmt, int K, int rows_total_per_wg);
int hh_gemv_launch(int fmt, int pro, int epi, GemvArgs a, hipStream_t s);
int hh_gemv_grid(int epi, const GemvArgs& a);

// Packed-activation byte size for a K-vector.
inline size_t hh_packed_bytes(int K) { return (size_t)K + (size_t)(K / 32) * 8; }

// ---- other operators (hh_ops.hip) ----
struct AttnArgs {
  const float* qkv;      // q region (gated: [q_h | gate_h] per head), then k, then v
  int n_heads, n_kv, hd, rope_dim, gated;
  int q_stride_heads;    // offset of k region from qkv start (floats)
  const float* q_norm;   // null = no per-head RMSNorm
  const float* k_norm;
  float eps;
  const float* rope;     // [max_seq][rope_dim] sin|cos (null = no RoPE)
  int max_seq;
  float* k_cache;        // [n_kv][max_seq][hd]
  float* v_cache;
  const StepState* state;  // pos source (null -> fixed_seq)
  int fixed_seq;         // >0: attend this many rows, no KV write / prep
  int chunk;             // positions per workgroup
  int max_splits;
  float* part_o;         // [n_kv][max_splits][G][hd]
  float* part_ml;        // [n_kv][max_splits][G][2]
  int* counters;         // [n_kv]
  float* out_f32;        // optional [n_heads*hd]
  uint8_t* act_out;      // optional packed activation (K = n_heads*hd)
  int act_fmt;
  int kv_q8;             // caches hold Q8_0 rows in 64-row blocks (max_seq a multiple of 64): each
                         // block's 64*hd int8 values, then its f16 scales [64][hd/32], the values
                         // interleaved so one 16-byte load holds 4 bytes of 4 rows (KvQ8::qoff / doff)
};
int hh_attn_launch(const AttnArgs& a, hipStream_t s);
int hh_kv_synth_q8_launch(uint64_t key, int n_pos, int n_kv, int hd, int max_seq, float cs, float* cache,
                          hipStream_t s);

// Batched prefill row kernels (hh_ops.hip).
// signs/had_block: a latent (folded) table's rows get R^-1 = H D after the lookup (had_block 0: none)
int hh_embed_rows_launch(int type, const uint8_t* table, int d, const uint32_t* toks, int S, float* H,
                         const float* signs, int had_block, hipStream_t s);
// Fold + Q8_0 of f32 rows X[S][K] into the split layout: optional rms_norm(x, w)
// first (w != null), optional GDN grouped head order (rep > 1), then signs and
// the WHT per had_block chunk.
int hh_rot_q8_rows_launch(const float* X, const float* w, float eps, int K, int S, const float* signs, int had_block,
                          int perm_nk, int perm_rep, int8_t* xq, float* xd, hipStream_t s);
// Row Q8_0 outputs use the GEMM's split layout: int8 xq[S][K], f32 scales xd[S][K/32].
int hh_norm_q8_rows_launch(const float* X, const float* w, float eps, int K, int S, int8_t* xq, float* xd,
                           hipStream_t s);
// yf != null: silu(g) * u rows as f32 [S][F] instead of Q8_0
int hh_silu_q8_rows_launch(const float* GU, int F, int S, int8_t* xq, float* xd, float* yf, hipStream_t s);
int hh_add_rows_launch(float* H, const float* T, int64_t n, hipStream_t s);
// H += T, then hh_norm_q8_rows_launch's output from the new H, in one pass (K % 1024 == 0, K <= 8192)
int hh_add_norm_q8_rows_launch(float* H, const float* T, const float* w, float eps, int K, int S, int8_t* xq,
                               float* xd, hipStream_t s);
int hh_prefill_qk_launch(int hd, const float* QKV, int n_in, int n_heads, int n_kv, const float* q_norm,
                         const float* k_norm, float eps, const float* rope, int rope_dim, int max_seq, int pos0, int S,
                         int gated, int kv_q8, float* k_cache, float* v_cache, float* QB, hipStream_t s);
int hh_prefill_attn_launch(int hd, const float* QB, const float* k_cache, const float* v_cache, int n_heads, int n_kv,
                           int max_seq, int pos0, int t0, int n, int n_chunks, float* PO, float* PML,
                           const float* gate, int gate_row, int kv_q8, int8_t* yq, float* yd, float* yf,
                           hipStream_t s);
int hh_prefill_attn_mfma_launch(int hd, const float* QB, const float* k_cache, const float* v_cache, int n_heads,
                                int n_kv, int max_seq, int pos0, int t0, int n, const float* gate, int gate_row,
                                int kv_q8, int8_t* yq, float* yd, float* yf, hipStream_t s);
// yf != null: the merged (gated) rows as f32 [S][n_heads*hd] instead of Q8_0
// gate: qwen35 gated attention's projection rows (gate_row floats apart), or null;
// kv_q8: the caches hold Q8_0 rows (quantized on write, dequantized on load)

// Batched Q8_0 GEMM on int8 MFMA (prefill): out[s*n + r], K % 128 == 0, activations
// split (int8 xq[seq][K], f32 xd[seq][K/32]); hh_q8_split_launch converts standard Q8_0 rows.
int hh_gemm_launch(int fmt, const uint8_t* w, int n, int K, const int8_t* xq, const float* xd, int seq, float* out,
                   hipStream_t s);
int hh_q8_split_launch(const uint8_t* x, int64_t nblocks, int8_t* xq, float* xd, hipStream_t s);

int hh_quantize_launch(const float* x, int64_t n, uint8_t* out, hipStream_t s);
int hh_dequant_launch(int type, const void* w, int64_t n, float* out, hipStream_t s);
int hh_rmsnorm_launch(const float* x, const float* w, float eps, int64_t rows, int64_t n, float* out,
                      hipStream_t s);
int hh_rope_launch(float* x, int n_heads, int hd, int rope_dim, const float* table, int max_seq, int pos,
                   hipStream_t s);
int hh_embed_launch(int type, const uint8_t* table, int d, const StepState* st, float* hidden,
                    const float* signs, int had_block, hipStream_t s);
int hh_argmax_launch(const float* logits, int64_t n, const int* counts, float pen, int rule,
                     float* part_val, int* part_idx, int* counter, uint32_t* out, hipStream_t s);
int hh_count_tokens_launch(const uint32_t* past, int64_t n_past, int* counts, hipStream_t s);
int hh_fill_i32_launch(int* p, int64_t n, int v, hipStream_t s);

// synthetic data
int hh_synth_launch(int type, uint64_t key, int64_t rows, int64_t cols, float c, float cq, float mean,
                    void* out, hipStream_t s);
int hh_kv_synth_launch(uint64_t key, int n_pos, int n_kv, int hd, int max_seq, float cs, float* cache,
                       hipStream_t s);

// qwen35 GDN step (hh_gdn.hip)
struct GdnArgs {
  const float* proj;      // [conv_dim] qkv projection (q | k | v), then [v_dim] z gate
  const float* hidden;    // prefill: layer input rows; alpha/beta read rms_norm(hidden, attn_norm)
  const float* attn_norm;
  const float* w_alpha;   // [n_v][d] f32 (prefill; decode forms the dots in the input projection)
  const float* w_beta;    // [n_v][d] f32
  const float* dt_bias;   // [n_v]
  const float* ssm_a;     // [n_v]
  const float* conv_w;    // [conv_dim][kernel]
  float* conv_state;      // [2][conv_dim][kernel-1] (see st / pos0 below)
  const float* ssm_norm;  // [hd]
  float* state;           // [n_v][hd][hd]
  int d, n_k, n_v, hd, kernel;
  float eps;
  uint8_t* act_out;       // packed activation of the gated-norm output (K = v_dim)
  int act_fmt;
  float* out_f32;         // non-null: the gated-norm output as f32 [v_dim] instead (folded models)
  // batched prefill scratch rows (k_gdn_prep_rows -> recurrence): per token
  float* ab;              // [S][2*n_v] g, beta
  float* dec_rows;        // [S][n_v] exp(g), the recurrence's decay (k_gdn_prep_rows -> k_gdn_rec_rows)
  float* qk;              // [S][2*k_dim] conv+silu+l2norm q,k
  float* vconv;           // [S][v_dim] conv+silu v
  const float* z;         // [v_dim] gate projection
  // batched prefill (hh_gdn_rows_launch): qk, vconv, ab, hidden are per-token
  // rows [S][...]; proj rows are row_in floats apart
  int S;
  int row_in;
  float* o_rows;          // [S][v_dim] recurrence outputs
  int8_t* xq;             // [S][v_dim] gated-norm Q8_0 codes (GEMM split layout)
  float* xd;              // [S][v_dim/32] scales
  float* y_rows;          // non-null: gated-norm rows as f32 [S][v_dim] instead of xq/xd
  // conv windows are double-buffered: [2][conv_dim][kernel-1]; the decode step
  // at position p reads buffer p & 1 and writes buffer (p + 1) & 1
  const StepState* st;    // decode: position source
  int pos0;               // batched prefill: position of token 0
  const float* ab_raw;    // decode: [2 n_v] raw alpha / beta dots (from the input projection)
};
int hh_gdn_launch(const GdnArgs& a, hipStream_t s);
// chunk_scratch != null: the recurrence in chunked form (hh_gdn_chunk.hip),
// scratch of hh_gdn_chunk_scratch_bytes(n_v, S) bytes
int hh_gdn_rows_launch(const GdnArgs& a, float* chunk_scratch, hipStream_t s);
size_t hh_gdn_chunk_scratch_bytes(int n_v, int S);
int hh_gdn_chunked_rec_launch(const GdnArgs& a, float* scratch, hipStream_t s);

// Measurement: one read-only pass over nbytes (multiple of 16 * 8 * 512 * 1024).
int hh_read_probe_launch(const void* p, int64_t nbytes, int* sink, hipStream_t s);
