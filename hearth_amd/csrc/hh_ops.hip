// hh_ops.hip — non-GEMV operators of the decode step for gfx950:
// Q8_0 quantize / dequantize, RMSNorm, RoPE, embedding lookup, GQA decode
// attention with fused head-norm + RoPE + KV write + Q8_0 output, greedy
// argmax, and the seeded synthetic-data generators.
#include "hh_kernels.h"

namespace {

// ---------------------------------------------------------------------------
// q8_0.rs:20-51 quantize_into (bit-exact): one 32-lane group per block.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_quantize(const float* __restrict__ x, int64_t n,
                                                  uint8_t* __restrict__ out) {
  int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  int64_t b = gid >> 5;
  int lane = threadIdx.x & 31;
  int64_t nb = (n + 31) / 32;
  if (b >= nb) return;   // whole 32-lane groups exit together
  int64_t idx = b * 32 + lane;
  float v = idx < n ? x[idx] : 0.0f;
  float am = group_max<32>(fabsf(v));
  float sc = q8_scale(am);
  int q = idx < n ? q8_round(v, sc) : 0;
  uint8_t* o = out + b * 34;
  o[2 + lane] = (uint8_t)(int8_t)q;
  if (lane == 0) {
    uint32_t h = f2h(sc);
    o[0] = (uint8_t)(h & 0xff);
    o[1] = (uint8_t)(h >> 8);
  }
}

// quant lib.rs:169-239 dequantize for the path's types (bit-exact).
__global__ void k_dequant(int type, const uint8_t* __restrict__ w, int64_t n, float* __restrict__ out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float v = 0.0f;
  if (type == 8) {                                   // q8_0.rs:4-18
    const uint8_t* blk = w + (i / 32) * 34;
    v = h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8)) * (float)(int8_t)blk[2 + (i % 32)];
  } else if (type == 42 || type == 142) {            // q2_0.rs:66-84, pq2_0.rs:32-50
    const uint8_t* blk = w + (i / 128) * 34;
    int e = (int)(i % 128);
    int code = (blk[2 + e / 4] >> (2 * (e % 4))) & 3;
    v = (float)(code - 1) * h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
  } else if (type == 41 || type == 43) {             // q1_0g128.rs:75-98
    const uint8_t* blk = w + (i / 128) * 18;
    int e = (int)(i % 128);
    int bit = (blk[2 + e / 8] >> (e % 8)) & 1;
    v = (float)(bit ? 1 : -1) * h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
  } else if (type == 1) {
    const uint8_t* p = w + i * 2;
    v = h2f((uint32_t)p[0] | ((uint32_t)p[1] << 8));
  } else {
    v = ((const float*)w)[i];
  }
  out[i] = v;
}

// ops.rs:8-35 rms_norm, one workgroup per row.
__global__ __launch_bounds__(256) void k_rmsnorm(const float* __restrict__ x, const float* __restrict__ w,
                                                 float eps, int64_t n, float* __restrict__ out) {
  const float* xr = x + (int64_t)blockIdx.x * n;
  float* orow = out + (int64_t)blockIdx.x * n;
  __shared__ float red[4];
  float ss = 0.0f;
  for (int64_t i = threadIdx.x; i < n; i += 256) ss += xr[i] * xr[i];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = (red[0] + red[1]) + (red[2] + red[3]);
  float inv = 1.0f / sqrtf(tot / (float)n + eps);
  for (int64_t i = threadIdx.x; i < n; i += 256) orow[i] = xr[i] * inv * w[i];
}

// ops.rs:140-164 RopeCache::apply on every head.
__global__ void k_rope(float* x, int n_heads, int hd, int rope_dim, const float* __restrict__ table,
                       int max_seq, int pos) {
  int half = rope_dim / 2;
  int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_heads * half) return;
  int h = t / half, i = t % half;
  const float* base = table + (size_t)(pos % max_seq) * half * 2;
  float s = base[i], c = base[half + i];
  float* xh = x + (size_t)h * hd;
  float x0 = xh[i], x1 = xh[i + half];
  xh[i] = x0 * c - x1 * s;
  xh[i + half] = x0 * s + x1 * c;
}

// mod.rs:483-504: hidden = dequantize(token_embd row), token from the step state.
__global__ __launch_bounds__(256) void k_embed(int type, const uint8_t* __restrict__ table, int d,
                                               const StepState* __restrict__ st, float* __restrict__ hidden) {
  int tok = st->token;
  for (int i = threadIdx.x; i < d; i += 256) {
    float v;
    if (type == 8) {
      const uint8_t* blk = table + (size_t)tok * (d / 32) * 34 + (size_t)(i / 32) * 34;
      v = h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8)) * (float)(int8_t)blk[2 + (i % 32)];
    } else if (type == 42 || type == 142) {
      const uint8_t* blk = table + (size_t)tok * (d / 128) * 34 + (size_t)(i / 128) * 34;
      int e = i % 128;
      int code = (blk[2 + e / 4] >> (2 * (e % 4))) & 3;
      v = (float)(code - 1) * h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    } else {
      const uint8_t* blk = table + (size_t)tok * (d / 128) * 18 + (size_t)(i / 128) * 18;
      int e = i % 128;
      int bit = (blk[2 + e / 8] >> (e % 8)) & 1;
      v = (float)(bit ? 1 : -1) * h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    }
    hidden[i] = v;
  }
}

// ---------------------------------------------------------------------------
// GQA decode attention (ops.rs:353-406 per q-head, mod.rs:687-704 head map
// kvh = qh / (n_heads/n_kv); qwen35.rs:1495-1640 with the q|gate split and
// sigmoid gate).  Split over the sequence: workgroup (s, kvh) owns positions
// [s*C, s*C+C) for the G query heads of kv head kvh, with C*hd = 8192 so a
// chunk of K and of V is 32 KB each, staged through LDS.  Prep (per-head
// RMSNorm mod.rs:551-578, RoPE :582-593, KV write :596-605) is fused: every
// workgroup normalises its q heads; the one holding `pos` also writes K/V.
// The last workgroup of a kv head (device counter) merges the splits
// (max-rescaled sums), applies the qwen35 gate, and emits the packed Q8_0
// input of attn_output.
// ---------------------------------------------------------------------------
HH_DEV void head_norm_rope(float* v, int hd, const float* nw, float eps, const float* rope, int rope_dim,
                           int max_seq, int pos, int lane, float* tmp_pair) {
  // v: LDS vector of hd floats, processed by one wave
  if (nw) {
    float ss = 0.0f;
    for (int d = lane; d < hd; d += 64) ss += v[d] * v[d];
    ss = wave_sum(ss);
    float inv = 1.0f / sqrtf(ss / (float)hd + eps);
    for (int d = lane; d < hd; d += 64) v[d] = v[d] * inv * nw[d];
  }
  if (rope) {
    int half = rope_dim / 2;
    const float* base = rope + (size_t)(pos % max_seq) * half * 2;
    float r0[4], r1[4];
    int cnt = 0;
    for (int i = lane; i < half; i += 64, ++cnt) {
      float s = base[i], c = base[half + i];
      float x0 = v[i], x1 = v[i + half];
      r0[cnt] = x0 * c - x1 * s;
      r1[cnt] = x0 * s + x1 * c;
    }
    cnt = 0;
    for (int i = lane; i < half; i += 64, ++cnt) {
      v[i] = r0[cnt];
      v[i + half] = r1[cnt];
    }
  }
  (void)tmp_pair;
}

__global__ __launch_bounds__(256) void k_attn(AttnArgs a) {
  extern __shared__ __align__(16) float sm[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int s = blockIdx.x, kvh = blockIdx.y;
  const int hd = a.hd, G = a.n_heads / a.n_kv, C = a.chunk;
  int seq, pos;
  bool prep;
  if (a.fixed_seq > 0) {
    seq = a.fixed_seq; pos = -1; prep = false;
  } else {
    pos = a.state->pos; seq = pos + 1; prep = true;
  }
  const int n_active = (seq + C - 1) / C;
  if (s >= n_active) return;
  const int p0 = s * C, np = min(C, seq - p0);
  const bool has_new = prep && pos >= p0 && pos < p0 + np;
  const int KS = hd + 4;
  float* qs = sm;                 // G*hd
  float* Ks = qs + G * hd;        // C*KS
  float* Vs = Ks + C * KS;        // C*hd
  float* sc = Vs + C * hd;        // G*C
  float* kn = sc + G * C;         // hd
  float* vn = kn + hd;            // hd
  float* ml = vn + hd;            // 2*G
  float* wts = ml + 2 * G + 8;    // G * max_splits (combine)
  const size_t hstride = (size_t)a.max_seq * hd;
  const float* kg = a.k_cache + (size_t)kvh * hstride;
  const float* vg = a.v_cache + (size_t)kvh * hstride;

  // 1. issue this chunk's K/V loads (C*hd == 8192 floats each: 8 float4 per lane)
  float4 kr[8], vr[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int f = (i * 256 + tid) * 4;
    int row = f / hd, col = f % hd;
    if (row < np && p0 + row != pos) {
      kr[i] = *(const float4*)(kg + (size_t)(p0 + row) * hd + col);
      vr[i] = *(const float4*)(vg + (size_t)(p0 + row) * hd + col);
    }
  }
  // 2. q heads (and the new k/v) : raw -> LDS, norm + rope by one wave per head
  for (int h = 0; h < G; ++h) {
    int qh = kvh * G + h;
    const float* src = a.qkv + (a.gated ? (size_t)qh * 2 * hd : (size_t)qh * hd);
    for (int d = tid; d < hd; d += 256) qs[h * hd + d] = src[d];
  }
  if (has_new) {
    const float* ksrc = a.qkv + a.q_stride_heads + (size_t)kvh * hd;
    const float* vsrc = a.qkv + a.q_stride_heads + (size_t)a.n_kv * hd + (size_t)kvh * hd;
    for (int d = tid; d < hd; d += 256) { kn[d] = ksrc[d]; vn[d] = vsrc[d]; }
  }
  __syncthreads();
  if (prep) {
    for (int h = wid; h < G; h += 4)
      head_norm_rope(qs + h * hd, hd, a.q_norm, a.eps, a.rope, a.rope_dim, a.max_seq, pos, lane, nullptr);
    if (has_new && wid == (G % 4)) {
      head_norm_rope(kn, hd, a.k_norm, a.eps, a.rope, a.rope_dim, a.max_seq, pos, lane, nullptr);
    }
  }
  __syncthreads();
  if (has_new) {   // kvcache.rs:92-113 write_kv
    float* kdst = a.k_cache + (size_t)kvh * hstride + (size_t)pos * hd;
    float* vdst = a.v_cache + (size_t)kvh * hstride + (size_t)pos * hd;
    for (int d = tid; d < hd; d += 256) { kdst[d] = kn[d]; vdst[d] = vn[d]; }
  }
  // 3. chunk into LDS
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int f = (i * 256 + tid) * 4;
    int row = f / hd, col = f % hd;
    if (row < np) {
      float4 k4 = kr[i], v4 = vr[i];
      if (p0 + row == pos) {
        k4 = make_float4(kn[col], kn[col + 1], kn[col + 2], kn[col + 3]);
        v4 = make_float4(vn[col], vn[col + 1], vn[col + 2], vn[col + 3]);
      }
      *(float4*)(Ks + row * KS + col) = k4;
      *(float4*)(Vs + row * hd + col) = v4;
    }
  }
  __syncthreads();
  // 4. scores (ops.rs:362-374): dot * 1/sqrt(hd)
  const float inv_sqrt = 1.0f / sqrtf((float)hd);
  for (int idx = tid; idx < G * C; idx += 256) {
    int h = idx / C, j = idx % C;
    float sc_v = -INFINITY;
    if (j < np) {
      const float4* kq = (const float4*)(Ks + j * KS);
      const float4* qq = (const float4*)(qs + h * hd);
      float acc = 0.0f;
      for (int d4 = 0; d4 < hd / 4; ++d4) {
        float4 k4 = kq[d4], q4 = qq[d4];
        acc = fmaf(q4.x, k4.x, acc);
        acc = fmaf(q4.y, k4.y, acc);
        acc = fmaf(q4.z, k4.z, acc);
        acc = fmaf(q4.w, k4.w, acc);
      }
      sc_v = acc * inv_sqrt;
    }
    sc[idx] = sc_v;
  }
  __syncthreads();
  // 5. per-head local softmax statistics (C <= 64)
  for (int h = wid; h < G; h += 4) {
    float v = lane < C ? sc[h * C + lane] : -INFINITY;
    float m = wave_max(v);
    float e = (lane < np) ? hx_exp(v - m) : 0.0f;
    float l = wave_sum(e);
    if (lane < C) sc[h * C + lane] = e;
    if (lane == 0) { ml[2 * h] = m; ml[2 * h + 1] = l; }
  }
  __syncthreads();
  // 6. o = sum_j e_j v_j
  const size_t pbase = ((size_t)kvh * a.max_splits + s) * G;
  for (int idx = tid; idx < G * hd; idx += 256) {
    int h = idx / hd, d = idx % hd;
    float acc = 0.0f;
    for (int j = 0; j < np; ++j) acc = fmaf(sc[h * C + j], Vs[j * hd + d], acc);
    a.part_o[(pbase + h) * hd + d] = acc;
  }
  if (tid < G) {
    a.part_ml[(pbase + tid) * 2] = ml[2 * tid];
    a.part_ml[(pbase + tid) * 2 + 1] = ml[2 * tid + 1];
  }
  // 7. last workgroup of this kv head merges the splits
  __shared__ int is_last;
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    is_last = (atomicAdd(a.counters + kvh, 1) == n_active - 1);
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  for (int h = wid; h < G; h += 4) {
    const size_t hb = (size_t)kvh * a.max_splits * G + h;   // + s'*G
    float M = -INFINITY;
    for (int t = lane; t < n_active; t += 64) M = fmaxf(M, a.part_ml[(hb + (size_t)t * G) * 2]);
    M = wave_max(M);
    float L = 0.0f;
    for (int t = lane; t < n_active; t += 64) {
      float e = hx_exp(a.part_ml[(hb + (size_t)t * G) * 2] - M);
      wts[h * a.max_splits + t] = e;
      L += e * a.part_ml[(hb + (size_t)t * G) * 2 + 1];
    }
    L = wave_sum(L);
    float invL = 1.0f / L;
    int qh = kvh * G + h;
    // o[d] = sum_t w_t o_t[d] in split order; the partials of 16 splits are
    // fetched together so the loop waits on one round trip per batch
    const size_t tstride = (size_t)G * hd;
    for (int d0 = 0; d0 < hd; d0 += 64) {
      int d = d0 + lane;
      float o = 0.0f;
      const float* pb = a.part_o + hb * hd + d;
      for (int t0 = 0; t0 < n_active; t0 += 16) {
        float pv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) pv[i] = (t0 + i < n_active) ? pb[(size_t)(t0 + i) * tstride] : 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (t0 + i < n_active) o = fmaf(wts[h * a.max_splits + t0 + i], pv[i], o);
      }
      o = o * invL;
      if (a.gated) {   // qwen35.rs:1627-1629 attn_out /= 1 + exp(-gate)
        float g = a.qkv[(size_t)qh * 2 * hd + hd + d];
        o = o / (1.0f + hx_exp(-g));
      }
      if (a.out_f32) a.out_f32[(size_t)qh * hd + d] = o;
      if (a.act_out) {
        float am = group_max<32>(fabsf(o));
        float scq = q8_scale(am);
        int q = q8_round(o, scq);
        int qsum = group_sum_i<32>(q);
        int e = qh * hd + d;
        int K = a.n_heads * hd;
        a.act_out[perm_pos(a.act_fmt, e)] = (uint8_t)(int8_t)q;
        if ((lane & 31) == 0) {
          ((float*)(a.act_out + K))[e >> 5] = h2f(f2h(scq));
          ((int*)(a.act_out + K + (K / 32) * 4))[e >> 5] = qsum;
        }
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    a.counters[kvh] = 0;
    __threadfence();
  }
}

// ---------------------------------------------------------------------------
// Greedy selection over a logits vector (standalone operator).
// ---------------------------------------------------------------------------
HH_DEV bool better(int rule, float v2, int i2, float v1, int i1) {
  return rule == 0 ? (v2 > v1 || (v2 == v1 && i2 > i1)) : (v2 > v1 || (v2 == v1 && i2 < i1));
}

__global__ __launch_bounds__(256) void k_argmax(const float* __restrict__ logits, int64_t n,
                                                const int* __restrict__ counts, float pen, int rule,
                                                float* part_val, int* part_idx, int* counter, uint32_t* out) {
  __shared__ float sv[256];
  __shared__ int si[256];
  __shared__ int is_last;
  const int tid = threadIdx.x;
  const bool do_pen = rule == 0 && counts && !(fabsf(pen - 1.0f) < 1e-6f);
  float bv = -INFINITY;
  int bi = rule == 0 ? -1 : 0x7fffffff;
  for (int64_t i = (int64_t)blockIdx.x * 256 + tid; i < n; i += (int64_t)gridDim.x * 256) {
    float v = logits[i];
    if (do_pen) {
      int c = counts[i];
      for (int k = 0; k < c; ++k) v = (v > 0.0f) ? v / pen : v * pen;
    }
    if (v == v && better(rule, v, (int)i, bv, bi)) { bv = v; bi = (int)i; }
  }
  sv[tid] = bv; si[tid] = bi;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o && better(rule, sv[tid + o], si[tid + o], sv[tid], si[tid])) { sv[tid] = sv[tid + o]; si[tid] = si[tid + o]; }
    __syncthreads();
  }
  if (tid == 0) {
    part_val[blockIdx.x] = sv[0];
    part_idx[blockIdx.x] = si[0];
    __threadfence();
    is_last = atomicAdd(counter, 1) == (int)gridDim.x - 1;
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  bv = -INFINITY; bi = rule == 0 ? -1 : 0x7fffffff;
  for (int b = tid; b < (int)gridDim.x; b += 256) {
    float v = part_val[b]; int i = part_idx[b];
    if (better(rule, v, i, bv, bi)) { bv = v; bi = i; }
  }
  sv[tid] = bv; si[tid] = bi;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o && better(rule, sv[tid + o], si[tid + o], sv[tid], si[tid])) { sv[tid] = sv[tid + o]; si[tid] = si[tid + o]; }
    __syncthreads();
  }
  if (tid == 0) {
    *out = (uint32_t)(si[0] < 0 ? 0 : si[0]);
    *counter = 0;
  }
}

__global__ void k_count_tokens(const uint32_t* past, int64_t n, int* counts) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) atomicAdd(counts + past[i], 1);
}

__global__ void k_fill_i32(int* p, int64_t n, int v) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------
// Seeded synthetic tensors (same definition as the CPU checker in tests).
// ---------------------------------------------------------------------------
__global__ void k_synth_f32(uint64_t key, int64_t n, float c, float mean, float* out) {
#pragma clang fp contract(off)
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float t = __fmul_rn((float)synth_int(key, (uint64_t)i), c);
  out[i] = __fadd_rn(t, mean);
}

__global__ void k_synth_q8(uint64_t key, int64_t nblocks, float c, uint8_t* out) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  float v[32];
  float am = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    v[j] = __fmul_rn((float)synth_int(key, (uint64_t)(b * 32 + j)), c);
    float a = fabsf(v[j]);
    if (a > am) am = a;
  }
  float sc = q8_scale(am);
  uint32_t h = f2h(sc);
  uint8_t* o = out + b * 34;
  o[0] = (uint8_t)(h & 0xff);
  o[1] = (uint8_t)(h >> 8);
#pragma unroll
  for (int j = 0; j < 32; ++j) o[2 + j] = (uint8_t)(int8_t)q8_round(v[j], sc);
}

// Q1_0 / Q2_0 from the integers: absmean scale S*c/128, sign bit (I >= 0), or
// ternary code (256|I| >= S -> +-1, else 0).
__global__ void k_synth_bits(int is_q1, uint64_t key, int64_t nblocks, float cq, uint8_t* out) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  int32_t iv[128];
  int64_t S = 0;
  for (int j = 0; j < 128; ++j) {
    iv[j] = synth_int(key, (uint64_t)(b * 128 + j));
    S += iv[j] < 0 ? -(int64_t)iv[j] : iv[j];
  }
  float scale = __fmul_rn((float)S, cq);
  uint32_t h = f2h(scale);
  int bb = is_q1 ? 18 : 34;
  uint8_t* o = out + b * bb;
  o[0] = (uint8_t)(h & 0xff);
  o[1] = (uint8_t)(h >> 8);
  if (is_q1) {
    for (int k = 0; k < 16; ++k) {
      uint32_t byte = 0;
      for (int j = 0; j < 8; ++j) byte |= (iv[k * 8 + j] >= 0 ? 1u : 0u) << j;
      o[2 + k] = (uint8_t)byte;
    }
  } else {
    for (int k = 0; k < 32; ++k) {
      uint32_t byte = 0;
      for (int j = 0; j < 4; ++j) {
        int32_t x = iv[k * 4 + j];
        int64_t ax = x < 0 ? -(int64_t)x : x;
        int code = 1;
        if (S > 0 && 256 * ax >= S) code = x > 0 ? 2 : 0;
        byte |= (uint32_t)code << (2 * j);
      }
      o[2 + k] = (uint8_t)byte;
    }
  }
}

// KV prefill: value = f16(I * (1/sd)), index ((p * n_kv) + h) * hd + j.
__global__ void k_kv_synth(uint64_t key, int n_pos, int n_kv, int hd, int max_seq, float cs, float* cache) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t total = (int64_t)n_pos * n_kv * hd;
  if (i >= total) return;
  int j = (int)(i % hd);
  int64_t r = i / hd;
  int h = (int)(r % n_kv);
  int p = (int)(r / n_kv);
  float v = h2f(f2h(__fmul_rn((float)synth_int(key, (uint64_t)i), cs)));
  cache[((size_t)h * max_seq + p) * hd + j] = v;
}

inline int ok() { return hipGetLastError() == hipSuccess ? 0 : 1; }
inline unsigned nblk(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }

}  // namespace

int hh_quantize_launch(const float* x, int64_t n, uint8_t* out, hipStream_t s) {
  int64_t nb = (n + 31) / 32;
  if (nb == 0) return 0;
  hipLaunchKernelGGL(k_quantize, dim3(nblk(nb * 32, 256)), dim3(256), 0, s, x, n, out);
  return ok();
}

int hh_dequant_launch(int type, const void* w, int64_t n, float* out, hipStream_t s) {
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_dequant, dim3(nblk(n, 256)), dim3(256), 0, s, type, (const uint8_t*)w, n, out);
  return ok();
}

int hh_rmsnorm_launch(const float* x, const float* w, float eps, int64_t rows, int64_t n, float* out,
                      hipStream_t s) {
  if (rows == 0) return 0;
  hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)rows), dim3(256), 0, s, x, w, eps, n, out);
  return ok();
}

int hh_rope_launch(float* x, int n_heads, int hd, int rope_dim, const float* table, int max_seq, int pos,
                   hipStream_t s) {
  int n = n_heads * (rope_dim / 2);
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_rope, dim3(nblk(n, 256)), dim3(256), 0, s, x, n_heads, hd, rope_dim, table, max_seq, pos);
  return ok();
}

int hh_embed_launch(int type, const uint8_t* table, int d, const StepState* st, float* hidden, hipStream_t s) {
  hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), 0, s, type, table, d, st, hidden);
  return ok();
}

int hh_attn_launch(const AttnArgs& a, hipStream_t s) {
  int G = a.n_heads / a.n_kv;
  size_t floats = (size_t)G * a.hd + (size_t)a.chunk * (a.hd + 4) + (size_t)a.chunk * a.hd + (size_t)G * a.chunk +
                  2 * (size_t)a.hd + 2 * G + 8 + (size_t)G * a.max_splits;
  if (a.hd != 128 && a.hd != 256) return 1;
  hipLaunchKernelGGL(k_attn, dim3(a.max_splits, a.n_kv), dim3(256), floats * 4, s, a);
  return ok();
}

int hh_argmax_launch(const float* logits, int64_t n, const int* counts, float pen, int rule, float* part_val,
                     int* part_idx, int* counter, uint32_t* out, hipStream_t s) {
  int nb = (int)std::min<int64_t>(1024, (n + 255) / 256);
  if (nb < 1) nb = 1;
  hipLaunchKernelGGL(k_argmax, dim3(nb), dim3(256), 0, s, logits, n, counts, pen, rule, part_val, part_idx,
                     counter, out);
  return ok();
}

int hh_count_tokens_launch(const uint32_t* past, int64_t n_past, int* counts, hipStream_t s) {
  if (n_past == 0) return 0;
  hipLaunchKernelGGL(k_count_tokens, dim3(nblk(n_past, 256)), dim3(256), 0, s, past, n_past, counts);
  return ok();
}

int hh_fill_i32_launch(int* p, int64_t n, int v, hipStream_t s) {
  if (n == 0) return 0;
  hipLaunchKernelGGL(k_fill_i32, dim3(nblk(n, 256)), dim3(256), 0, s, p, n, v);
  return ok();
}

int hh_synth_launch(int type, uint64_t key, int64_t rows, int64_t cols, float c, float cq, float mean, void* out,
                    hipStream_t s) {
  int64_t n = rows * cols;
  if (n == 0) return 0;
  if (type == 0) {
    hipLaunchKernelGGL(k_synth_f32, dim3(nblk(n, 256)), dim3(256), 0, s, key, n, c, mean, (float*)out);
  } else if (type == 8) {
    hipLaunchKernelGGL(k_synth_q8, dim3(nblk(n / 32, 256)), dim3(256), 0, s, key, n / 32, c, (uint8_t*)out);
  } else if (type == 41 || type == 43 || type == 42 || type == 142) {
    int is_q1 = (type == 41 || type == 43);
    hipLaunchKernelGGL(k_synth_bits, dim3(nblk(n / 128, 128)), dim3(128), 0, s, is_q1, key, n / 128, cq,
                       (uint8_t*)out);
  } else {
    return 1;
  }
  return ok();
}

int hh_kv_synth_launch(uint64_t key, int n_pos, int n_kv, int hd, int max_seq, float cs, float* cache,
                       hipStream_t s) {
  int64_t total = (int64_t)n_pos * n_kv * hd;
  if (total == 0) return 0;
  hipLaunchKernelGGL(k_kv_synth, dim3(nblk(total, 256)), dim3(256), 0, s, key, n_pos, n_kv, hd, max_seq, cs, cache);
  return ok();
}
