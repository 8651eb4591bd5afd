/*
 * hearth_oracle.h — CPU restatement of Hearth's batch-1 decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * library in hearth_amd/ and the "port" CPU baseline timed by bench.py.  It is
 * never linked into, loaded by, or called from the product path.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the Hearth repository root).
 */
#ifndef HEARTH_ORACLE_H
#define HEARTH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids, crates/hearth-gguf/src/ggml.rs:49-53, :96-100 */
enum { HO_F32 = 0, HO_F16 = 1, HO_Q8_0 = 8, HO_Q1_0 = 41, HO_Q2_0 = 42, HO_Q1_0_G128 = 43,
       HO_PQ2_0 = 142, HO_PTQ1_0 = 143 };

/* ---- scalar conversions (half 2.7.1 f16::from_f32 / to_f32 semantics) ---- */
uint16_t ho_f32_to_f16(float x);
float ho_f16_to_f32(uint16_t h);

/* exp / log shared with the device kernels (definition in hearth_oracle.c) */
float ho_exp(float x);
float ho_log(float x);

/* ---- block formats ---- */
size_t ho_row_bytes(int type, int64_t n_cols);
void ho_quantize_q8_0(const float* x, int64_t n, uint8_t* out);          /* q8_0.rs:20-51 */
int ho_dequantize(int type, const uint8_t* w, int64_t n, float* out);    /* quant lib.rs:169-239 */
/* PTQ1_0 (type 143): 128 weights in 28 bytes, qs[24] at 5 trits/byte (a 16-byte
 * then an 8-byte stage, slot-major), qh[2] at 4 trits/byte, f16 d last
 * (ptq1_0.rs:1-13).  Trit n of byte b is ((b*3^n mod 256)*3) >> 8. */
void ho_quantize_ptq1_0(const float* x, int64_t n, uint8_t* out);        /* ptq1_0.rs:604-643 */
void ho_ptq1_0_pack_codes(const int* code, uint16_t f16_scale, uint8_t* out); /* one block from codes 0/1/2 */

/* ---- dot kernels: DotFn = fn(w, a_q8, n) -> f32 (pool.rs:6) ---- */
float ho_dot_q2_0_q8_0(const uint8_t* w, const uint8_t* a, int64_t n);   /* q2_0.rs:537-574 */
float ho_dot_q1_0_q8_0(const uint8_t* w, const uint8_t* a, int64_t n);   /* q1_0g128.rs:1113-1152 */
float ho_dot_q8_0_q8_0(const uint8_t* w, const uint8_t* a, int64_t n);   /* q8_0.rs:154-171 */
float ho_dot_ptq1_0_q8_0(const uint8_t* w, const uint8_t* a, int64_t n); /* ptq1_0.rs:555-602 */
float ho_dot_q2_0_q8_0_avx2(const uint8_t* w, const uint8_t* a, int64_t n); /* q2_0.rs:308-392 */
float ho_dot_q1_0_q8_0_avx2(const uint8_t* w, const uint8_t* a, int64_t n); /* q1_0g128.rs:255-377 */
int ho_have_avx2(void);

/* Row-parallel GEMV, pool.rs:510-566 partitioning (contiguous ceil(N/T) rows per
 * worker).  arm: 0 = scalar reference semantics, 1 = the AVX2 arm the reference
 * dispatches on AVX2 hosts (falls back to scalar when the host lacks AVX2). */
int ho_gemv(int type, const uint8_t* w, int64_t n_rows, int64_t n_cols, const uint8_t* a_q8,
            float* y, int n_threads, int arm);

/* ---- f32 ops (crates/hearth-llm/src/ops.rs) ---- */
void ho_rms_norm(const float* x, const float* w, float eps, int64_t n, float* out); /* :8-35 */
void ho_rope_table(int max_seq, int rope_dim, float theta, float* table);         /* :78-138 */
void ho_rope_apply(const float* table, int max_seq, int rope_dim, float* x, int pos); /* :140-164 */
void ho_silu(float* x, int64_t n);                                                /* :240-253 */
void ho_softmax(float* x, int64_t n);                                             /* :308-351 */
void ho_attention(const float* q, const float* k, const float* v, int seq_len, int head_dim,
                  float* out, float* scratch);                                    /* :353-406 */
/* The same attention in the device's grouping (split chunks of ho_attn_chunk
 * positions, the kernels' butterflies and trees), for the tests. */
int ho_attn_chunk(int seq_len, int head_dim, int n_kv_heads);
void ho_attention_dev(const float* q, const float* k, const float* v, int seq_len, int head_dim, int n_kv_heads,
                      float* out);

/* ---- Hadamard fold (qwen35.rs:51-118) ---- */
void ho_wht(float* x, int64_t n);                         /* walsh_hadamard_in_place :51-68 */
void ho_hadamard_rotate(float* x, int64_t n, const float* signs, int block);   /* :75-88  R = D.H */
void ho_hadamard_unrotate(float* x, int64_t n, const float* signs, int block); /* :98-110 R^-1 = H.D */

/* ---- greedy selection ---- */
/* hearth-sampler lib.rs:26-40 + :156-175 (repetition penalty, then LAST max on ties) */
uint32_t ho_sample_greedy_dense(float* logits, int64_t n, const uint32_t* past, int64_t n_past,
                                float repeat_pen);
/* qwen35.rs:1735-1745 (strict >, FIRST max on ties, no penalty) */
uint32_t ho_argmax_first(const float* logits, int64_t n);

/* ---- seeded synthetic data (shared definition with the device generator) ---- */
uint64_t ho_name_key(uint64_t seed, const char* name);
int32_t ho_synth_int(uint64_t key, uint64_t idx);   /* Irwin-Hall(4) of u16, zero mean */
float ho_synth_scale(float std);                    /* float multiplier for N(0,std) */
void ho_synth_tensor(int type, uint64_t seed, const char* name, int64_t rows, int64_t cols,
                     float std, float mean, void* out, int n_threads);
uint32_t ho_synth_token(uint64_t seed, int64_t i, uint32_t vocab);

/* ---- model ---- */
typedef struct {
  int arch;            /* 0 = dense Qwen3/Llama, 1 = qwen35 hybrid */
  int d_model, n_layers, n_heads, n_kv_heads, head_dim, d_ffn, vocab;
  float eps, rope_theta;
  int rope_dim;        /* rotated dims per head (0 = head_dim) */
  int max_seq;
  int wtype;           /* layer weight type: HO_Q1_0 / HO_Q2_0 / HO_PQ2_0 / HO_Q8_0 */
  int head_type;       /* token_embd / output type (HO_Q8_0) */
  int qk_norm;         /* per-head q/k RMSNorm present */
  /* qwen35 hybrid geometry */
  int full_attn_interval; /* layer i is full attention iff (i+1) % interval == 0 */
  int ssm_n_k_heads, ssm_n_v_heads, ssm_head_dim, ssm_conv_kernel;
  int attn_out_gate;   /* full-attention layers emit [q|gate] per head */
  int kv_type;         /* HO_F32 or HO_Q8_0 (KVStorage, kvcache.rs:6-9) */
  /* qwen35 Hadamard fold (prism.hadamard.*, qwen35.rs:532-610): block size (0 =
   * none) and flags: 1 = token_embd is latent (R^-1 after lookup),
   * 2 = tied output (the head is token_embd; output.weight absent) */
  int had_block, had_flags;
} ho_config;

typedef struct ho_model ho_model;

ho_model* ho_model_new(const ho_config* cfg);
void ho_model_free(ho_model* m);
/* Host storage for a named tensor (GGUF naming); returns NULL if unknown. */
void* ho_model_tensor(ho_model* m, const char* name, size_t* nbytes, int* type,
                      int64_t* rows, int64_t* cols);
int ho_model_tensor_count(const ho_model* m);
const char* ho_model_tensor_name(const ho_model* m, int i);
/* Fill every tensor from the seeded generator. */
void ho_model_synth(ho_model* m, uint64_t seed, int n_threads);
/* Reset KV (and recurrent) state to empty. */
void ho_model_reset(ho_model* m);
/* Write one position of the f32 KV cache for a layer (prefilled-cache configs). */
int ho_model_kv_prefill_synth(ho_model* m, uint64_t seed, int n_pos);
void ho_model_set_threads(ho_model* m, int n_threads, int arm);
/* fp32 association order of the reductions: 0 = the reference's (ops.rs loops,
 * default), 1 = the HIP kernels' (butterfly / split-sequence), for bit-level
 * comparison with the device.  Same mathematics either way. */
void ho_model_set_order(ho_model* m, int order);
/* One decode step (mod.rs:451-860 dense / qwen35.rs:1028-1236 hybrid). */
int ho_forward(ho_model* m, uint32_t token, int pos, float* logits);
/* Token loop: prompt token-by-token, then n_gen greedy tokens. */
int ho_generate(ho_model* m, const uint32_t* prompt, int n_prompt, int start_pos, int n_gen,
                float repeat_pen, uint32_t* out_tokens, float* last_logits);
/* Sign vector of a fold width (prism.hadamard.sign_widths/_values); widths
 * without one get no sign pass (signs_for() == None, qwen35.rs:843-845). */
int ho_model_set_signs(ho_model* m, int width, const float* signs);
/* Debug taps: copy of the hidden state after the last forward. */
const float* ho_model_hidden(const ho_model* m);

#ifdef __cplusplus
}
#endif
#endif
