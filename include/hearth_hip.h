/*
 * hearth_hip.h — C ABI of the MI355X (gfx950) decode library for Hearth.
 *
 * Plain pointers and sizes only.  Every entry point returns an int status
 * (HH_OK = 0); on failure hh_last_error() returns a thread-local message, the
 * analogue of the reference's Result<_, String> (matmul.rs:50-73).  A non-zero
 * status lets the caller keep Hearth's "fall back to CPU" behaviour
 * (matmul.rs:83-147, mod.rs:238-282).  No C++ exception crosses this boundary.
 *
 * Threading: an hh_ctx owns one HIP stream; an hh_model is externally
 * synchronised (one forward in flight per model), as Hearth's forward scratch
 * sits behind a Mutex (mod.rs:66-72, :2781-2783).
 *
 * Two granularities are exported:
 *   - operator level (device pointers), replacing the DotFn/par_dot_rows layer
 *     (pool.rs:6, :510-566), the quantizer (q8_0.rs:20-51) and the
 *     hearth_compute::GpuCompute operator set (hearth-compute/src/lib.rs:103-1364);
 *   - model level (hh_model_*), replacing LlamaModel::forward / generate_text
 *     (mod.rs:451-860, :2718-3012) and Qwen35Core::forward / generate_text
 *     (qwen35.rs:1028-1236, :1654-1804).
 */
#ifndef HEARTH_HIP_H
#define HEARTH_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
enum {
  HH_OK = 0,
  HH_ERR_INVALID = 1,   /* null pointer, bad argument */
  HH_ERR_DTYPE = 2,     /* unsupported ggml type (matmul.rs:270-378 error arm) */
  HH_ERR_DIM = 3,       /* dimension mismatch (matmul.rs:66-73) */
  HH_ERR_OOM = 4,       /* device allocation failed */
  HH_ERR_HIP = 5,       /* HIP runtime error */
  HH_ERR_NOT_FOUND = 6, /* unknown tensor name (matmul.rs:59-62) */
  HH_ERR_RANGE = 7,     /* position / token out of range */
  HH_ERR_CANCELLED = 8  /* cancel flag observed (mod.rs:461, :510) */
};

/* GGML type ids (crates/hearth-gguf/src/ggml.rs:49-53, :96-100) */
enum {
  HH_F32 = 0,
  HH_F16 = 1,
  HH_Q8_0 = 8,
  HH_Q1_0 = 41,
  HH_Q2_0 = 42,
  HH_Q1_0_G128 = 43,
  HH_PQ2_0 = 142,
  HH_PTQ1_0 = 143       /* 128 weights in 28 B: 5 trits/byte (ptq1_0.rs:1-13) */
};

typedef struct hh_ctx hh_ctx;
typedef struct hh_model hh_model;

/* Thread-local message of the last failing call on this thread. */
const char* hh_last_error(void);
/* Library version string. */
const char* hh_version(void);

/* ---- context: replaces GpuCompute::new() -> Option<Self> (hearth-compute lib.rs:126) ---- */
int hh_ctx_create(int device_ordinal, hh_ctx** out);
int hh_ctx_destroy(hh_ctx* ctx);
int hh_ctx_synchronize(hh_ctx* ctx);
/* Device memory helpers (GpuCompute::upload_bytes / readback_f32, lib.rs:230-243). */
int hh_malloc(hh_ctx* ctx, size_t nbytes, void** dptr);
int hh_free(hh_ctx* ctx, void* dptr);
int hh_memcpy_h2d(hh_ctx* ctx, void* dst, const void* src, size_t nbytes);
int hh_memcpy_d2h(hh_ctx* ctx, void* dst, const void* src, size_t nbytes);
int hh_memset(hh_ctx* ctx, void* dst, int value, size_t nbytes);
/* Device-clock timing on the context's stream (hipEvents in 8 slots): record
 * a slot, then read the milliseconds between two recorded slots (waits for b). */
int hh_ctx_event_record(hh_ctx* ctx, int slot);
int hh_ctx_event_elapsed(hh_ctx* ctx, int slot_a, int slot_b, float* ms);

/* ---- operators (all pointers are device pointers; enqueued on the ctx stream) ---- */

/* q8_0.rs:20-51 quantize_into: n f32 -> ceil(n/32)*34 bytes, bit-exact. */
int hh_quantize_q8_0(hh_ctx* ctx, const float* x, int64_t n, uint8_t* out_q8);

/* quant lib.rs:169-239 dequantize (Q8_0 q8_0.rs:4-18, Q2_0/PQ2_0 q2_0.rs:66-84,
 * Q1_0/Q1_0_G128 q1_0g128.rs:75-98): n elements -> f32, bit-exact. */
int hh_dequantize(hh_ctx* ctx, int ggml_type, const void* w, int64_t n, float* out);

/* Row-parallel quantized GEMV: y[r] = dot_fn(w + r*row_bytes, x_q8, n_cols) for
 * r < n_rows.  Replaces ThreadPool::par_dot_rows with dot_fn in
 * {dot_q2_0_q8_0_ptr (q2_0.rs:628), dot_q1_0g128_q8_0_ptr (q1_0g128.rs:1000),
 *  dot_q8_0_q8_0_ptr (q8_0.rs:154)} (pool.rs:510-566, matmul.rs:153-269).
 * x_q8: n_cols/32 standard Q8_0 blocks.  n_cols: a multiple of 256 (Q1_0/Q2_0)
 * or 64 (Q8_0), at most 20480. */
int hh_gemv_q8(hh_ctx* ctx, int ggml_type, const void* w, int64_t n_rows, int64_t n_cols,
               const uint8_t* x_q8, float* y);

/* Batched quantized GEMM for prefill: out[s*n_rows + r] = dot_fn(w + r*row_bytes,
 * x_q8 + s*(n_cols/32)*34, n_cols) for every token s < seq_len.  Replaces
 * ThreadPool::par_dot_rows_batched with DotFn / DotFn2 (pool.rs:40-80, :568-618;
 * matmul.rs:580-674 matmul_batch).  Runs on int8 MFMA; each output is bit-identical
 * to hh_gemv_q8 on that token, as the reference's paired kernels are to its
 * single-token dot (q2_0.rs:936-986).  x_q8: seq_len rows of n_cols/32 standard
 * Q8_0 blocks.  n_cols: a positive multiple of 128. */
int hh_gemm_q8(hh_ctx* ctx, int ggml_type, const void* w, int64_t n_rows, int64_t n_cols,
               const uint8_t* x_q8, int64_t seq_len, float* out);

/* ops.rs:8-35 rms_norm over n_rows independent rows of width n. */
int hh_rms_norm(hh_ctx* ctx, const float* x, const float* weight, float eps, int64_t n_rows,
                int64_t n, float* out);

/* ops.rs:140-164 RopeCache::apply on n_heads heads of width head_dim (first
 * rope_dim dims rotated, NeoX halves) at position pos; table as built by
 * RopeCache::new (ops.rs:78-138): [max_seq][rope_dim] = sin | cos. */
int hh_rope(hh_ctx* ctx, float* x, int n_heads, int head_dim, int rope_dim, const float* table,
            int max_seq, int pos);

/* ops.rs:353-406 decode attention, GQA (mod.rs:687-704): q [n_heads][hd];
 * k/v cache [n_kv][max_seq][hd] f32 (kvcache.rs:11-22); attends seq_len rows. */
int hh_attention(hh_ctx* ctx, const float* q, const float* k_cache, const float* v_cache,
                 int n_heads, int n_kv_heads, int head_dim, int max_seq, int seq_len, float* out);

/* Causal attention of a batch of prompt tokens, as forward_batch runs it per
 * token (mod.rs:1101-1140, each token through ops.rs:353-406 over the rows
 * before it): q [n_tokens][n_heads][hd] (already normed and rotated), k/v
 * cache [n_kv][max_seq][hd] f32 holding positions 0 .. pos0 + n_tokens - 1;
 * token t attends positions 0 .. pos0 + t.  out [n_tokens][n_heads][hd] f32.
 * mode 0: the batched prefill's split/merge kernels (each token's row equals
 * hh_attention at seq_len pos0 + t + 1 bit for bit); mode 1: the fp32-MFMA
 * flash form (HH_PREFILL_ATTN=mfma), equal to fp32 rounding. */
int hh_attention_prefill(hh_ctx* ctx, const float* q, const float* k_cache, const float* v_cache, int n_heads,
                         int n_kv_heads, int head_dim, int max_seq, int pos0, int n_tokens, int mode, float* out);

/* hh_attention without any allocation: no counterpart in the reference.  For
 * callers that cannot call hipMalloc (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  Same arguments, kernels
 * and results as hh_attention, but the split partials live in a fixed
 * per-GPU device array of 4 MiB (n_kv * ceil(seq_len / (8192 / head_dim)) *
 * (n_heads / n_kv) * (head_dim + 2) floats at most; larger calls fail with
 * HH_ERR_RANGE).  Every call on one GPU shares that array: calls that overlap
 * in time on the same GPU (any context or stream) race.  Each call writes every
 * partial it reads, so the array's previous contents do not matter. */
int hh_attention_noalloc(hh_ctx* ctx, const float* q, const float* k_cache, const float* v_cache,
                         int n_heads, int n_kv_heads, int head_dim, int max_seq, int seq_len, float* out);

/* Greedy selection.  rule 0 = dense sampler (hearth-sampler lib.rs:26-40 penalty
 * over past tokens, then max_by: LAST max index); rule 1 = qwen35 inline argmax
 * (qwen35.rs:1735-1745: FIRST max, no penalty).  Replaces GpuCompute::argmax_f32
 * (lib.rs:338).  Result written to *out_index (device). */
int hh_argmax(hh_ctx* ctx, const float* logits, int64_t n, const uint32_t* past, int64_t n_past,
              float repeat_pen, int rule, uint32_t* out_index);

/* ---- model ---- */
typedef struct {
  int arch;               /* 0 = dense Qwen3/Llama (mod.rs), 1 = qwen35 hybrid (qwen35.rs) */
  int d_model, n_layers, n_heads, n_kv_heads, head_dim, d_ffn, vocab;
  float eps, rope_theta;
  int rope_dim;           /* 0 = head_dim */
  int max_seq;
  int wtype;              /* HH_Q1_0 / HH_Q1_0_G128 / HH_Q2_0 / HH_PQ2_0 / HH_PTQ1_0 */
  int head_type;          /* token_embd / output: HH_Q8_0 */
  int qk_norm;
  int full_attn_interval; /* qwen35: layer i is full attention iff (i+1)%interval==0 */
  int ssm_n_k_heads, ssm_n_v_heads, ssm_head_dim, ssm_conv_kernel;
  int attn_out_gate;      /* qwen35 full attention: attn_q emits [q_h | gate_h] */
  int kv_type;            /* HH_F32 (0): f32 cache (KVStorage::F32, the default); HH_Q8_0: Q8_0 rows
                             (KVStorage::Q8_0, kvcache.rs:41-57, written by write_kv :92-113, read
                             through the dequantized rows as attention_q8_0, ops.rs:946-1030) */
  int had_block;          /* qwen35 Hadamard fold (prism.hadamard.block_size, qwen35.rs:532-610):
                             0 = unfolded; else a power of two dividing every folded width */
  int had_flags;          /* HH_HAD_LATENT_EMBD: token_embd rows get R^-1 after the lookup
                             (inverse_weight_names holds token_embd.weight); HH_HAD_TIED_OUTPUT:
                             no output.weight, the head is token_embd (tied_output, version 2) */
} hh_model_config;
enum { HH_HAD_LATENT_EMBD = 1, HH_HAD_TIED_OUTPUT = 2 };

/* Allocates every weight (native GGUF block layout, uploaded once), the KV
 * cache (f32 [layer][kv_head][max_seq][hd], or the same rows as Q8_0 blocks in a device-internal
 * 64-row interleaved layout; kvcache.rs:11-57), the recurrent state
 * and the step buffers.  Replaces LlamaModel::load's GPU branch (mod.rs:238-282,
 * model/gpu.rs:8-50). */
int hh_model_create(hh_ctx* ctx, const hh_model_config* cfg, hh_model** out);
int hh_model_destroy(hh_model* m);
/* Upload one tensor by GGUF name; bytes are the tensor's native row-major blocks
 * (TensorEntry::row_data, tensor.rs:57-79).  ne0 = n_cols, ne1 = n_rows. */
int hh_model_upload_tensor(hh_model* m, const char* name, int ggml_type, int64_t ne0, int64_t ne1,
                           const void* host_bytes, size_t nbytes);
/* Copy a tensor's device bytes back to host (checks, CPU baselines). */
int hh_model_download_tensor(hh_model* m, const char* name, void* host_bytes, size_t nbytes);
/* Enumerate tensors: name, type, shape and byte size. */
int hh_model_tensor_count(hh_model* m);
int hh_model_tensor_info(hh_model* m, int index, const char** name, int* ggml_type, int64_t* ne0,
                         int64_t* ne1, size_t* nbytes);
/* Sign vector of one fold width (prism.hadamard.sign_widths / sign_values;
 * the `had_signs` map of qwen35.rs:561-586, looked up by matmul width in
 * signs_for, :843-845).  A folded width with no sign vector gets no sign pass,
 * as signs_for() == None.  Widths the model does not fold are accepted and
 * ignored.  Values must be +1 or -1. */
int hh_model_set_hadamard_signs(hh_model* m, int width, const float* signs);

/* Copy the recurrent state of the gdn_index-th Gated-DeltaNet layer to host:
 * [n_v][hd][hd] f32 (GdnState::layer_slice, qwen35.rs:242-261). */
int hh_model_download_state(hh_model* m, int gdn_index, float* host, size_t n_floats);

/* Fill every tensor on the device from the seeded generator (synthetic weights). */
int hh_model_synthesize(hh_model* m, uint64_t seed);
/* Reset KV + recurrent state (fresh session). */
int hh_model_reset(hh_model* m);
/* Pre-fill positions [0, n_pos) of every attention layer's KV cache with the
 * seeded N(0,1) values rounded to fp16. */
int hh_model_prefill_kv_synthetic(hh_model* m, uint64_t seed, int n_pos);
/* Cancel flag polled before each step (mod.rs:461). */
int hh_model_set_cancel(hh_model* m, int cancel);

/* One decode step, mod.rs:451-860 / qwen35.rs:1028-1236: token at pos.  If
 * logits_host != NULL the vocab logits are copied back; if argmax_host != NULL
 * the greedy choice (rule per arch, repetition penalty repeat_pen over the
 * session's past tokens for the dense rule) is returned. */
int hh_model_forward(hh_model* m, uint32_t token, int pos, float* logits_host,
                     uint32_t* argmax_host);

/* Token loop (mod.rs:2718-3012 / qwen35.rs:1654-1804): feed n_prompt tokens from
 * start_pos, then n_gen greedy tokens, all on the device (one HIP graph per step,
 * no host round trip per token).  out_tokens (host) receives n_gen ids;
 * last_logits_host (optional) the logits after the final step. */
int hh_model_generate(hh_model* m, const uint32_t* prompt, int n_prompt, int start_pos, int n_gen,
                      float repeat_pen, uint32_t* out_tokens, float* last_logits_host);

/* Batched prefill (LlamaModel::forward_batch, mod.rs:899-1221): runs
 * tokens[0..n) at positions start_pos.. through every layer with the int8-MFMA
 * GEMM (hh_gemm_q8) and writes their K/V; computes no logits (the reference
 * computes only the last token's, mod.rs:1201-1218: feed that token to
 * hh_model_forward).  On qwen35 hybrids the GDN layers run their per-token
 * prep in parallel and the recurrence in token order; the reference has no
 * batched hybrid path (qwen35.rs:1693-1700 feeds prompts token by token).  Each
 * layer's arithmetic restates the decode step's, so the KV cache and recurrent
 * state equal the ones token-by-token decoding leaves.  hh_model_generate uses
 * it for all prompt tokens but the last.  A Q8_0 KV cache is quantized on
 * write exactly as the decode step writes it. */
int hh_model_prefill(hh_model* m, const uint32_t* tokens, int n, int start_pos);

/* Device time (ms) of the last prefill: hh_model_prefill, or the prompt phase of
 * hh_model_generate (batched prefill plus the last prompt token's step, which
 * yields the first generated token). */
int hh_model_last_prefill_ms(hh_model* m, double* ms);

/* Timing of the last hh_model_generate call, device clock (hipEvents): total ms
 * over the generated-token steps only (prefill excluded). */
int hh_model_last_decode_ms(hh_model* m, double* ms);

/* Average device time (hipEvents on the model's stream) of each stage of the
 * step for one layer, launched `iters` times back to back: out_ms[0..6] =
 * embed, input projection, attention/GDN, output projection, gate+up, down,
 * LM head + greedy selection.  The counterpart of the reference's per-section
 * ForwardTimers (mod.rs:480-857); it perturbs the hidden state, so call it
 * outside a generation. */
int hh_model_time_stages(hh_model* m, int layer, int iters, double* out_ms, int n_out);

/* Measurement, no counterpart in the reference: the read-only HBM rate (GB/s) of
 * reps passes over a fresh nbytes buffer (a multiple of 64 MiB), each lane
 * keeping 8 16-byte loads in flight.  The ceiling a decode step, which is
 * almost all reads, is measured against beside the published 8 TB/s. */
int hh_read_bandwidth(hh_ctx* ctx, size_t nbytes, int reps, double* gbps);

/* ---- GGUF files ----
 * A GGUF v2/v3 file, memory-mapped and parsed: header, metadata and tensor table
 * (hearth-gguf GgufFile::open, gguf.rs:138-218; tensor byte sizes from the
 * GgmlDType block table, ggml.rs:57-171).  Errors: HH_ERR_INVALID (bad magic,
 * unsupported version, truncated file -- GgufError, gguf.rs:12-27),
 * HH_ERR_DTYPE (unknown dtype id), HH_ERR_NOT_FOUND (missing file or key). */
typedef struct hh_gguf hh_gguf;
int hh_gguf_open(const char* path, hh_gguf** out);
int hh_gguf_close(hh_gguf* g);
int hh_gguf_header(hh_gguf* g, uint32_t* version, uint64_t* data_offset, uint64_t* alignment);
int hh_gguf_tensor_count(hh_gguf* g);
/* shape4[d] = ne_d (1 past n_dims); offset is relative to the data section
 * (TensorInfo, tensor.rs:1-24). */
int hh_gguf_tensor_info(hh_gguf* g, int index, const char** name, int* ggml_type, int* n_dims, int64_t* shape4,
                        uint64_t* offset, uint64_t* nbytes);
/* Host pointer to a tensor's bytes inside the mapping (GgufFile::tensor_data, gguf.rs:220-224). */
int hh_gguf_tensor_data(hh_gguf* g, int index, const void** data);
/* Metadata getters with MetaValue::as_u32 / as_f32 / as_str / as_array semantics (meta.rs:26-64). */
int hh_gguf_meta_u32(hh_gguf* g, const char* key, uint32_t* out);
int hh_gguf_meta_f32(hh_gguf* g, const char* key, float* out);
int hh_gguf_meta_str(hh_gguf* g, const char* key, const char** out);
int hh_gguf_meta_array_len(hh_gguf* g, const char* key, uint64_t* out);
/* The decode model's configuration: ModelConfig::from_gguf (config.rs:57-217,
 * arch key prefixes :288-307), head_dim from the Q (dense, mod.rs:156-167) or
 * K projection (qwen35.rs:475-488), the qwen35 GDN geometry (qwen35.rs:490-528)
 * and the KV context cap (kv_budget.rs:19-58: 1.25 GiB of f32 KV, at most 4096
 * tokens for dense models).  ctx_cap_override > 0 replaces that cap
 * (HEARTH_CTX_CAP).  Weight formats come from the tensors: wtype from
 * blk.0.ffn_gate.weight, head_type from token_embd.weight. */
int hh_gguf_model_config(hh_gguf* g, int ctx_cap_override, hh_model_config* cfg);
/* LlamaModel::load / qwen35::load for the device (mod.rs:103-150, model/gpu.rs:8-50):
 * open, derive the configuration, create the model and upload every tensor from
 * the mapping in its native blocks.  A missing output.weight is the tied head
 * (mod.rs:360-364): token_embd.weight is uploaded in its place.  F16 norm/GDN
 * vectors are widened to the f32 the decode path keeps. */
int hh_model_load_gguf(hh_ctx* ctx, const char* path, int ctx_cap_override, hh_model** out);

#ifdef __cplusplus
}
#endif
#endif
