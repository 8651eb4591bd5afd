// hh_ops.hip — non-GEMV operators of the decode step for gfx950:
// Q8_0 quantize / dequantize, RMSNorm, RoPE, embedding lookup, GQA decode
// attention with fused head-norm + RoPE + KV write + Q8_0 output, greedy
// argmax, and the seeded synthetic-data generators.
#include "hh_kernels.h"

#include <type_traits>

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
  int q = idx < n ? q8_round_r(v, sc, q8_rcp(sc)) : 0;
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
  } else if (type == 143) {                          // ptq1_0.rs:72-110
    const uint8_t* blk = w + (i / 128) * 28;
    const int e = (int)(i % 128);
    int byte, n;
    if (e < 80) { byte = e & 15; n = e >> 4; }
    else if (e < 120) { byte = 16 + ((e - 80) & 7); n = (e - 80) >> 3; }
    else { byte = 24 + ((e - 120) & 1); n = (e - 120) >> 1; }
    const uint32_t p3[5] = {1, 3, 9, 27, 81};
    const int t = (int)(((((uint32_t)blk[byte] * p3[n]) & 0xffu) * 3u) >> 8);
    v = (float)(t - 1) * h2f((uint32_t)blk[26] | ((uint32_t)blk[27] << 8));
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

// hidden = dequantize(token_embd row), token from the step state.
__global__ __launch_bounds__(256) void k_embed(int type, const uint8_t* __restrict__ table, int d,
                                               const StepState* __restrict__ st, float* __restrict__ hidden,
                                               const float* __restrict__ signs, int had_block) {
  extern __shared__ __align__(16) float ebuf[];
  embed_row<256>(type, table, d, st->token, hidden, signs, had_block, ebuf);
}

// ---------------------------------------------------------------------------
// GQA decode attention (ops.rs:353-406 per q-head, mod.rs:687-704 head map
// kvh = qh / (n_heads/n_kv); qwen35.rs:1495-1640 with the q|gate split and
// sigmoid gate).  Split over the sequence: workgroup (s, kvh) owns positions
// [s*C, s*C+C) for the G query heads of kv head kvh, with C*hd = 8192 so a
// chunk of K and of V is 32 KB each (f32), held in registers.  Prep (per-head
// RMSNorm mod.rs:551-578, RoPE :582-593, KV write :596-605) is fused: every
// workgroup normalises its q heads; the one holding `pos` also writes K/V.
// A second kernel merges the splits (max-rescaled sums), applies the qwen35
// gate, and emits the packed Q8_0 input of attn_output.
// ---------------------------------------------------------------------------
// A lane's float4 column slice x[4c .. 4c+3] of one head (c < LPR = HD/4;
// every LPR-lane group holds the whole head).  Per-head RMSNorm
// (mod.rs:551-578): ss_c = ((x0^2 + x1^2) + x2^2) + x3^2, summed over the
// group by an ascending butterfly; out = (x * inv) * w.  NeoX RoPE on the
// first rope_dim dims (ops.rs:140-164): the partner element i +- rope_dim/2
// sits rope_dim/8 lanes away.
template <int LPR>
HH_DEV float4 slice_norm(float4 x, float4 w, float eps) {
  float ss = x.x * x.x + x.y * x.y;
  ss = ss + x.z * x.z;
  ss = ss + x.w * x.w;
  ss = group_sum<LPR>(ss);
  const float inv = 1.0f / sqrtf(ss / (float)(4 * LPR) + eps);
  return make_float4(x.x * inv * w.x, x.y * inv * w.y, x.z * inv * w.z, x.w * inv * w.w);
}

// The RoPE table row of a lane's slice (rotation index c4 mod half): sin and
// cos as stored.  slice_rope rotates the first half as x0 cos - x1 sin and the
// second as x1 cos + x0 sin (= x0 sin + x1 cos: IEEE addition commutes), the
// products and roundings of ops.rs's form, bit for bit.
HH_DEV const float* rope_sin_ptr(const float* rope, int pos, int max_seq, int rope_dim, int c4) {
  const int half = rope_dim / 2, ib = c4 < half ? c4 : c4 - half;
  return rope + (size_t)(pos % max_seq) * half * 2 + ib;   // cos at + half
}
HH_DEV void rope_row(const float* rope, int pos, int max_seq, int rope_dim, int c4, float4& sn, float4& cs) {
  const float* ps = rope_sin_ptr(rope, pos, max_seq, rope_dim, c4);
  sn = *(const float4*)ps;
  cs = *(const float4*)(ps + rope_dim / 2);
}
// One reduce-scatter level at offset O in {16, 32}: lanes below the offset bit
// keep lo and receive the partner's lo, lanes above keep hi and receive the
// partner's hi, and every lane returns keep + received.  The VALU swaps
// (v_permlane16/32_swap(lo, hi)) hand each lane exactly that pair, so the sum
// of the two results is keep + received (IEEE addition commutes).
template <int O> HH_DEV float swap_pair_sum(float lo, float hi) {
  static_assert(O == 16 || O == 32, "offset");
  const unsigned a = __float_as_uint(lo), b = __float_as_uint(hi);
  if constexpr (O == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// sn/cs from rope_row; lanes with 4c >= rope_dim keep x.
HH_DEV float4 slice_rope(float4 x, float4 sn, float4 cs, int c4, int rope_dim) {
  const int half = rope_dim / 2, X = half / 4;
  float4 y;   // partner slice (all lanes exchange; the wave stays converged)
  if (X == 8) {   // rope_dim 64 (uniform branch)
    y.x = xor_lane<8>(x.x); y.y = xor_lane<8>(x.y); y.z = xor_lane<8>(x.z); y.w = xor_lane<8>(x.w);
  } else if (X == 16) {   // rope_dim 128
    y.x = xor_lane<16>(x.x); y.y = xor_lane<16>(x.y); y.z = xor_lane<16>(x.z); y.w = xor_lane<16>(x.w);
  } else {
    y.x = __shfl_xor(x.x, X, 64); y.y = __shfl_xor(x.y, X, 64);
    y.z = __shfl_xor(x.z, X, 64); y.w = __shfl_xor(x.w, X, 64);
  }
  const float4 r = c4 < half ? make_float4(x.x * cs.x - y.x * sn.x, x.y * cs.y - y.y * sn.y,
                                           x.z * cs.z - y.z * sn.z, x.w * cs.w - y.w * sn.w)
                              : make_float4(x.x * cs.x + y.x * sn.x, x.y * cs.y + y.y * sn.y,
                                           x.z * cs.z + y.z * sn.z, x.w * cs.w + y.w * sn.w);
  return c4 < rope_dim ? r : x;
}

// Butterfly sum of NV values held by each lane of an aligned LPR-lane group,
// done as a reduce-scatter: at offset O every lane keeps one half of its
// values and adds the partner's copy of that half.  Each kept value equals
// the all-lanes butterfly x_l + x_(l^O) at that level, so the result for
// value k is the butterfly sum with offsets LPR/2, ..., 1.  On return lane l
// holds value k = (l % LPR) >> log2(LPR / NV).
// Lanes hand over their values in a lane-dependent register order: register
// r of lane l holds value r ^ rs_perm<NV, LPR / 2>(l).  At each level below
// offset 16 every lane then keeps registers [0, N/2) and sends [N/2, N): a
// lane whose offset bit is set holds the upper half in the lower registers,
// and its partner's upper registers hold that same half, so each kept sum is
// the same pair of values, added in the same order, with no per-lane select.
// (The permlane swaps of the offsets 16 and 32 pair registers r and r + N/2
// across the lanes themselves.)
template <int N, int O> HH_DEV int rs_perm(int lane) {
  if constexpr (N > 1) return ((O < 16 && (lane & O)) ? N / 2 : 0) ^ rs_perm<N / 2, O / 2>(lane);
  else return 0;
}
template <int N, int O> struct ReduceScatter {
  static HH_DEV float run(float* v) {
    if constexpr (N > 1) {
      static_assert(O > 0, "more values than lanes");
#pragma unroll
      for (int k = 0; k < N / 2; ++k) {
        if constexpr (O >= 16) v[k] = swap_pair_sum<O>(v[k], v[k + N / 2]);
        else v[k] = v[k] + xor_lane<O>(v[k + N / 2]);
      }
      return ReduceScatter<N / 2, O / 2>::run(v);
    } else {
      float x = v[0];
      if constexpr (O >= 32) x += xor_lane<32>(x);
      if constexpr (O >= 16) x += xor_lane<16>(x);
      if constexpr (O >= 8) x += xor_lane<8>(x);
      if constexpr (O >= 4) x += xor_lane<4>(x);
      if constexpr (O >= 2) x += xor_lane<2>(x);
      if constexpr (O >= 1) x += xor_lane<1>(x);
      return x;
    }
  }
};

// The same butterfly sum with values in the natural register order: lanes
// whose offset bit is set keep the upper half, chosen per lane.  The decode
// split uses it: its one pass is latency-bound, and the permuted order's
// extra K addressing and q swaps cost more there than the selects.
template <int N, int O> struct ReduceScatterSel {
  static HH_DEV float run(float* v, int lane) {
    if constexpr (N > 1) {
      static_assert(O > 0, "more values than lanes");
      const bool up = (lane & O) != 0;
#pragma unroll
      for (int k = 0; k < N / 2; ++k) {
        if constexpr (O >= 16) {
          v[k] = swap_pair_sum<O>(v[k], v[k + N / 2]);
        } else {
          const float send = up ? v[k] : v[k + N / 2];
          const float keep = up ? v[k + N / 2] : v[k];
          v[k] = keep + xor_lane<O>(send);
        }
      }
      return ReduceScatterSel<N / 2, O / 2>::run(v, lane);
    } else {
      float x = v[0];
      if constexpr (O >= 32) x += xor_lane<32>(x);
      if constexpr (O >= 16) x += xor_lane<16>(x);
      if constexpr (O >= 8) x += xor_lane<8>(x);
      if constexpr (O >= 4) x += xor_lane<4>(x);
      if constexpr (O >= 2) x += xor_lane<2>(x);
      if constexpr (O >= 1) x += xor_lane<1>(x);
      return x;
    }
  }
};

// Split kernel: workgroup (s, kvh) owns positions [s*C, s*C + C) of kv head
// kvh (C = attn_chunk_for: 8192/hd or twice that) for its G query heads,
// with ATTN_NT lanes.  Thread t
// holds one float4 column slice (c = t % LPR) of rows j = i*RPI + t/LPR,
// i < NR, of K and V in registers, so the chunk is read from HBM exactly
// once and never staged through LDS.
//  * score(h, j) = (butterfly over the LPR lanes of the row of the 4-term
//    fma chain q.k) * 1/sqrt(hd)
//  * e = exp(score - m), m and l = sum e by a 64-lane butterfly
//  * o(h, d): per row group `sub` an fma chain over i; hd 128: the two row
//    groups of a wave are added; then the NW wave values by pairwise_tree.
// Writes the unnormalised partial o and (m, l) of every (split, head).
constexpr int ATTN_NT = 512;

// ((v0 + v1) + (v2 + v3)) + ... over N = 2^k values.
template <int N> HH_DEV float pairwise_tree(float* t) {
#pragma unroll
  for (int w = N; w > 1; w >>= 1)
#pragma unroll
    for (int i = 0; i < w / 2; ++i) t[i] = t[2 * i] + t[2 * i + 1];
  return t[0];
}

// Zeros that stand in for K/V rows a split workgroup does not hold, so that
// its loads need no branch (never written).
__device__ __align__(32) float attn_zero_row[8];   // also a zero StepState stand-in (state_lanes)

// Q8_0 KV rows (KV8): the [n_kv][max_seq] rows of hd values (max_seq a
// multiple of 64) are stored in 64-row blocks of 68*hd bytes, the block's int8
// values then its f16 block scales (hd/32 per row), laid out for the attention
// split's lanes: in a block, row j = i*RPI + sub (RPI = 512 / (hd/4) rows per pass of a
// 512-lane workgroup) keeps its 4-byte slice c (elements 4c .. 4c+3) at
// ((sub*(hd/4) + c)*NRB + i)*4, NRB = 64/RPI, and its scale of block cb at
// f16 index (sub*(hd/32) + cb)*NRB + i after the block's values.  A lane (sub, c) then finds the slices of its
// rows i, i+1, .. side by side: 4 rows in one 16-byte load, their scales in
// one 8-byte load.  A slice's value is its 4 int8 times the block's f16 scale,
// exactly the f32 value attention_q8_0 (ops.rs:946-1030) multiplies.
HH_DEV float4 kv_dequant4(uint32_t v, float s) {
  return make_float4((float)(int8_t)(v & 0xff) * s, (float)(int8_t)((v >> 8) & 0xff) * s,
                     (float)(int8_t)((v >> 16) & 0xff) * s, (float)(int8_t)(v >> 24) * s);
}
struct KvQ8 {
  int8_t* q;
  uint16_t* d;
  HH_DEV KvQ8(float* cache, int /*n_kv*/, int /*max_seq*/, int hd) : q((int8_t*)cache), d((uint16_t*)cache) {}
  // A 64-row block holds its 64*hd int8 values, then their 64*hd/32 f16 scales
  // (68*hd bytes); inside a block the values of 4 rows that one lane reads
  // together sit side by side.  Byte offset of row `row`'s slice c
  // (row = kvh*max_seq + p):
  static HH_DEV size_t qoff(size_t row, int hd, int c) {
    const int R = 512 / (hd / 4), nrb = 64 / R, j = (int)(row & 63);
    return (row >> 6) * 68 * (size_t)hd + ((size_t)((j % R) * (hd / 4) + c) * nrb + j / R) * 4;
  }
  // f16 index (from the cache base) of row `row`'s scale of 32-block cb
  static HH_DEV size_t doff(size_t row, int hd, int cb) {
    const int R = 512 / (hd / 4), nrb = 64 / R, j = (int)(row & 63);
    return (row >> 6) * 34 * (size_t)hd + 32 * (size_t)hd + (size_t)((j % R) * (hd / 32) + cb) * nrb + j / R;
  }
  HH_DEV float4 load(size_t row, int hd, int c) const {   // lane slice c of one row
    return kv_dequant4(*(const uint32_t*)(q + qoff(row, hd, c)), h2f(d[doff(row, hd, c >> 3)]));
  }
  // the slices c of rows row, row + RPI, row + 2 RPI, row + 3 RPI (row's block
  // position a multiple of 4 passes): 16 bytes and four scales, or zeros
  // from attn_zero_row when !ok
  HH_DEV void load4(size_t row, int hd, int c, bool ok, uint4& v, uint2& sc) const {
    v = *(ok ? (const uint4*)(q + qoff(row, hd, c)) : (const uint4*)attn_zero_row);
    sc = *(ok ? (const uint2*)(d + doff(row, hd, c >> 3)) : (const uint2*)attn_zero_row);
  }
};

// write_kv for a Q8_0 cache (kvcache.rs:104-108, quantize_q8_0_block :274-303):
// the 8 lanes of a 32-value block share max|x|; returns the dequantized slice
// that every later reader sees.  `write`: this lane stores its 4 bytes (and
// lane 0 of the block the scale).
HH_DEV float4 kv_q8_store(float4 x, const KvQ8& kv, size_t row, int hd, int c, bool write) {
  const float vv[4] = {x.x, x.y, x.z, x.w};
  float am = fmaxf(fmaxf(fabsf(vv[0]), fabsf(vv[1])), fmaxf(fabsf(vv[2]), fabsf(vv[3])));
  am = group_max<8>(am);
  const float sc = q8_scale(am), rc = q8_rcp(sc);
  const uint32_t h = f2h(sc);
  const float d = h2f(h);
  uint32_t word = 0;
  float out[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = q8_round_r(vv[i], sc, rc);
    word |= ((uint32_t)q & 0xffu) << (8 * i);
    out[i] = (float)q * d;
  }
  if (write) {
    *(uint32_t*)(kv.q + KvQ8::qoff(row, hd, c)) = word;
    if ((c & 7) == 0) kv.d[KvQ8::doff(row, hd, c >> 3)] = (uint16_t)h;
  }
  return make_float4(out[0], out[1], out[2], out[3]);
}

// GT: the GQA group size n_heads / n_kv when it is one of the instantiated
// values (the per-head loops then have exact trip counts), 0 = read at run time.
// The split body for chunks of C positions (attn_chunk_for).
template <int HD, int NTA, bool KV8, int GT, int C>
HH_DEV void attn_split_body(const AttnArgs& a, int G, int seq, int pos, bool prep) {
  constexpr int LPR = HD / 4, RPI = NTA / LPR, NR = C / RPI, NW = NTA / 64;
  static_assert(NR * RPI == C && NR >= 1 && C <= 128, "geometry");
  extern __shared__ __align__(16) float sm[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int n_active = (seq + C - 1) / C;
  // workgroup -> (chunk s, kv head): the last (partial) chunk of every kv head
  // first, then the other chunks chunk-major; the grid's spare workgroups exit.
  // A launch with more workgroups than CUs places the last ones beside
  // another workgroup, where they run late; this puts the light chunk first
  // and leaves the late places to whole chunks (8B at 2k context: the
  // attention stage 13.2 -> 12.9 us in a timing build).
  int s, kvh;
  {
    const int L = blockIdx.x, nk = a.n_kv;
    if (L < nk) {
      s = n_active - 1;
      kvh = L;
    } else {
      s = (L - nk) / nk;
      kvh = L - nk - s * nk;
      if (s >= n_active - 1) return;
    }
  }
  const int p0 = s * C, np = min(C, seq - p0);
  const bool has_new = prep && pos >= p0 && pos < p0 + np;
  const int sub = tid / LPR, c = tid % LPR;
  float* sc = sm;                 // G*C
  float* ml = sc + G * C;         // 2*G (+pad)
  float* red = ml + ((2 * G + 4 + 3) & ~3);   // NW waves * 4 heads * HD (16-byte aligned)
  const size_t hstride = (size_t)a.max_seq * HD;
  const float* kg = a.k_cache + (size_t)kvh * hstride + 4 * c;
  const float* vg = a.v_cache + (size_t)kvh * hstride + 4 * c;
  const KvQ8 kq(a.k_cache, a.n_kv, a.max_seq, HD), vq(a.v_cache, a.n_kv, a.max_seq, HD);
  const size_t row0 = (size_t)kvh * a.max_seq;

  // 1. the small loads first (vector loads return in issue order): this
  // lane's slice of every q head and of the new k/v, the norm weights and the
  // RoPE row.  Like the K/V loads below they are unconditional (absent ones
  // read the zero row), so no wait on them can land before the K/V issue.
  constexpr int GMAX = GT > 0 ? GT : 8;
  const float* z = attn_zero_row;
  float4 q4[(GMAX + 3) & ~3];
#pragma unroll
  for (int h = 0; h < ((GMAX + 3) & ~3); ++h) {
    q4[h] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (h < G) {
      const int qh = kvh * G + h;
      q4[h] = *(const float4*)(a.qkv + (a.gated ? (size_t)qh * 2 * HD : (size_t)qh * HD) + 4 * c);
    }
  }
  const float* kv_new = a.qkv + a.q_stride_heads + (size_t)kvh * HD + 4 * c;
  const float4 kn_raw = *(const float4*)(has_new ? kv_new : z);
  const float4 vn_raw = *(const float4*)(has_new ? kv_new + (size_t)a.n_kv * HD : z);
  const float4 nq4 = *(const float4*)(prep && a.q_norm ? a.q_norm + 4 * c : z);
  const float4 nk4 = *(const float4*)(prep && a.k_norm ? a.k_norm + 4 * c : z);
  const bool has_rope = prep && a.rope && 4 * c < a.rope_dim;
  const float* ps = has_rope ? rope_sin_ptr(a.rope, pos, a.max_seq, a.rope_dim, 4 * c) : z;
  const float4 sn4 = *(const float4*)ps;
  const float4 cs4 = *(const float4*)(has_rope ? ps + a.rope_dim / 2 : z);
  float4 kn4 = kn_raw, vn4 = vn_raw;
  __builtin_amdgcn_sched_barrier(0);   // keep these loads ahead of the K/V stream

  // 2. this chunk's K/V.  The loads are unconditional: a row the chunk does
  // not hold (past the end, or the new position, filled in below) reads the
  // zero row instead.  A load under a branch leaves the compiler no exact
  // count of loads in flight, and its conservative wait would hold step 3's q
  // prep until every K/V row had landed.
  float4 kr[NR], vr[NR];
  // Q8_0 rows stay as loaded (four rows per 16-byte load, the blocked layout of
  // KvQ8) until their first use: K before the scores, V before o.  Dequantizing
  // here would wait for the whole stream before the q prep below.
  uint4 kw[NR / 4], vw[NR / 4];
  uint2 ks[NR / 4], vs[NR / 4];
  static_assert(NR % 4 == 0, "four rows per load");
  if constexpr (KV8) {
    // a group's 64-row block lies in the cache when the group starts below max_seq
#pragma unroll
    for (int g = 0; g < NR / 4; ++g)
      kq.load4(row0 + p0 + 4 * g * RPI + sub, HD, c, p0 + 4 * g * RPI < a.max_seq, kw[g], ks[g]);
#pragma unroll
    for (int g = 0; g < NR / 4; ++g)
      vq.load4(row0 + p0 + 4 * g * RPI + sub, HD, c, p0 + 4 * g * RPI < a.max_seq, vw[g], vs[g]);
  } else {
    // every K row before the V rows: loads return in issue order, so the scores
    // need not wait for V
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int j = i * RPI + sub;
      const bool held = j < np && p0 + j != pos;
      kr[i] = *(held ? (const float4*)(kg + (size_t)(p0 + j) * HD) : (const float4*)attn_zero_row);
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int j = i * RPI + sub;
      const bool held = j < np && p0 + j != pos;
      vr[i] = *(held ? (const float4*)(vg + (size_t)(p0 + j) * HD) : (const float4*)attn_zero_row);
    }
  }
  // 3. q heads and the new k: per-head norm + rope on the lane's slice
  if (prep) {
#pragma unroll
    for (int h = 0; h < GMAX; ++h) {
      if (h < G) {
        if (a.q_norm) q4[h] = slice_norm<LPR>(q4[h], nq4, a.eps);
        if (a.rope) q4[h] = slice_rope(q4[h], sn4, cs4, 4 * c, a.rope_dim);
      }
    }
    if (has_new) {   // uniform over the workgroup
      if (a.k_norm) kn4 = slice_norm<LPR>(kn4, nk4, a.eps);
      if (a.rope) kn4 = slice_rope(kn4, sn4, cs4, 4 * c, a.rope_dim);
      // kvcache.rs:92-113 write_kv, then the row joins this chunk
      if constexpr (KV8) {
        kn4 = kv_q8_store(kn4, kq, row0 + pos, HD, c, sub == 0);
        vn4 = kv_q8_store(vn4, vq, row0 + pos, HD, c, sub == 0);
      } else if (sub == 0) {
        *(float4*)(a.k_cache + (size_t)kvh * hstride + (size_t)pos * HD + 4 * c) = kn4;
        *(float4*)(a.v_cache + (size_t)kvh * hstride + (size_t)pos * HD + 4 * c) = vn4;
      }
      if constexpr (!KV8) {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
          if (p0 + i * RPI + sub == pos) { kr[i] = kn4; vr[i] = vn4; }
        }
      }
    }
  }
  // row i of the lane from its load group (rows absent from the chunk, and the
  // new position, are zero; the new row is then put in from registers)
  auto unpack = [&](const uint4* w, const uint2* sc, float4* r, float4 nw) {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int j = i * RPI + sub, g = i / 4, t = i % 4;
      const bool held = j < np && p0 + j != pos;
      const uint32_t b = t == 0 ? w[g].x : t == 1 ? w[g].y : t == 2 ? w[g].z : w[g].w;
      const uint32_t d = ((t < 2 ? sc[g].x : sc[g].y) >> (16 * (t & 1))) & 0xffffu;
      r[i] = held ? kv_dequant4(b, h2f(d)) : make_float4(0.f, 0.f, 0.f, 0.f);
      if (has_new && p0 + j == pos) r[i] = nw;
    }
  };
  if constexpr (KV8) unpack(kw, ks, kr, kn4);
  // 4. scores (ops.rs:362-374), four heads per pass
  const float inv_sqrt = 1.0f / sqrtf((float)HD);
  constexpr int NV = 4 * NR;                          // values per lane per pass
  constexpr int KSH = (LPR == 64 ? 6 : 5) - (NV == 32 ? 5 : NV == 16 ? 4 : 3);   // log2(LPR / NV)
#pragma unroll
  for (int hg = 0; hg < GMAX; hg += 4) {
    if (hg >= G) break;
    float v[NV];
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      const float4 qq = q4[hg + hh];
#pragma unroll
      for (int i = 0; i < NR; ++i) {
        float p = qq.x * kr[i].x;
        p = fmaf(qq.y, kr[i].y, p);
        p = fmaf(qq.z, kr[i].z, p);
        p = fmaf(qq.w, kr[i].w, p);
        v[hh * NR + i] = p;
      }
    }
    const float r = ReduceScatterSel<NV, LPR / 2>::run(v, lane);
    const int k = (lane & (LPR - 1)) >> KSH;
    const int h = hg + k / NR, j = (k % NR) * RPI + sub;
    if (h < G && (lane & ((1 << KSH) - 1)) == 0) sc[h * C + j] = (j < np) ? r * inv_sqrt : -INFINITY;
  }
  __syncthreads();
  // 5. per-head softmax statistics over the chunk (C = 128: two positions per
  // lane, added before the butterfly)
  for (int h = wid; h < G; h += NW) {
    if constexpr (C <= 64) {
      float x = lane < C ? sc[h * C + lane] : -INFINITY;
      float m = wave_max_nonan(x);
      float e = (lane < np) ? hx_exp(x - m) : 0.0f;
      float l = wave_sum(e);
      if (lane < C) sc[h * C + lane] = e;
      if (lane == 0) { ml[2 * h] = m; ml[2 * h + 1] = l; }
    } else {
      const float x0 = sc[h * C + lane], x1 = sc[h * C + 64 + lane];
      const float m = wave_max_nonan(fmaxf(x0, x1));
      const float e0 = (lane < np) ? hx_exp(x0 - m) : 0.0f;
      const float e1 = (64 + lane < np) ? hx_exp(x1 - m) : 0.0f;
      const float l = wave_sum(e0 + e1);
      sc[h * C + lane] = e0;
      sc[h * C + 64 + lane] = e1;
      if (lane == 0) { ml[2 * h] = m; ml[2 * h + 1] = l; }
    }
  }
  __syncthreads();
  if constexpr (KV8) unpack(vw, vs, vr, vn4);
  // 6. o = sum_j e_j v_j
  const size_t pbase = ((size_t)kvh * a.max_splits + s) * G;
  for (int hg = 0; hg < G; hg += 4) {
    float acc[16];
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
      if (hg + hh < G) {
        const float* eh = sc + (hg + hh) * C + sub;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
          const float e = eh[i * RPI];
          o0 = fmaf(e, vr[i].x, o0);
          o1 = fmaf(e, vr[i].y, o1);
          o2 = fmaf(e, vr[i].z, o2);
          o3 = fmaf(e, vr[i].w, o3);
        }
      }
      acc[hh * 4 + 0] = o0; acc[hh * 4 + 1] = o1; acc[hh * 4 + 2] = o2; acc[hh * 4 + 3] = o3;
    }
    if constexpr (LPR == 32) {
      // the two row groups of this wave: lanes < 32 keep heads 0-1, others 2-3
      const bool up = (lane & 32) != 0;
      float xs[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) xs[k] = swap_pair_sum<32>(acc[k], acc[k + 8]);
      // values kk = k (+ 8 on the upper half) go to row wid*4 + kk/4, column
      // 4c + kk%4: two 16-byte writes per lane (scalar writes at a 4-dword
      // lane stride would conflict 4 ways)
#pragma unroll
      for (int g = 0; g < 2; ++g)
        *(float4*)(red + (wid * 4 + g + (up ? 2 : 0)) * HD + 4 * c) =
            make_float4(xs[4 * g], xs[4 * g + 1], xs[4 * g + 2], xs[4 * g + 3]);
    } else {
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(float4*)(red + (wid * 4 + g) * HD + 4 * c) = make_float4(acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]);
    }
    __syncthreads();
    for (int idx = tid; idx < 4 * HD; idx += NTA) {
      const int h = hg + idx / HD;
      if (h < G) {
        float t[NW];
#pragma unroll
        for (int w = 0; w < NW; ++w) t[w] = red[w * 4 * HD + idx];
        a.part_o[(pbase + h) * HD + (idx % HD)] = pairwise_tree<NW>(t);
      }
    }
    __syncthreads();
  }
  if (tid < G) {
    a.part_ml[(pbase + tid) * 2] = ml[2 * tid];
    a.part_ml[(pbase + tid) * 2 + 1] = ml[2 * tid + 1];
  }
}

template <int HD, int NTA, bool KV8, int GT>
__global__ __launch_bounds__(NTA) void k_attn_split(AttnArgs a) {
  const int G = GT > 0 ? GT : a.n_heads / a.n_kv;
  int seq, pos;
  bool prep;
  if (a.fixed_seq > 0) {
    seq = a.fixed_seq; pos = -1; prep = false;
  } else {
    pos = a.state->pos; seq = pos + 1; prep = true;
  }
  if (attn_chunk_for(seq, HD, a.n_kv) == 8192 / HD) attn_split_body<HD, NTA, KV8, GT, 8192 / HD>(a, G, seq, pos, prep);
  else attn_split_body<HD, NTA, KV8, GT, 16384 / HD>(a, G, seq, pos, prep);
}

// Merge kernel: workgroup (qh, 64-column slice).  M = max m_t, w_t =
// exp(m_t - M), L = sum w_t l_t (lane-strided over t, then a butterfly);
// wave g sums the splits t = g (mod 4) as an fma chain in increasing t, and
// o = ((P0 + P1) + (P2 + P3)) / L.  Applies the qwen35 output gate and emits
// the f32 row and/or the packed Q8_0 input of attn_output.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_merge(AttnArgs a) {
  extern __shared__ __align__(16) float wm[];
  float* wts = wm;                         // max_splits
  float* pw = wm + a.max_splits;           // 4 x 64
  float* sL = pw + 256;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int G = a.n_heads / a.n_kv;
  // workgroup id -> (kv head, query head in the group, 64-column slice), kv
  // head fastest: with round-robin dispatch the merge of kv head k runs on the
  // XCD whose split workgroups wrote its partials (split ids also put the kv
  // head fastest)
  const int kvh = (int)blockIdx.x % a.n_kv, rest = (int)blockIdx.x / a.n_kv;
  const int h = rest % G, qh = kvh * G + h, d = (rest / G) * 64 + lane;
  // The step position is a vector load among the others (a scalar load's
  // wait would also cover the kernel arguments, putting its round trip ahead
  // of every load below); the loads of the first 64 splits clamp to the grid,
  // not to the active splits, so no address waits for it.
  const int sv = state_lanes(a.state ? (const void*)a.state : (const void*)attn_zero_row);
  const size_t hb = (size_t)kvh * a.max_splits * G + h;
  const size_t tstride = (size_t)G * HD;
  const float* pb = a.part_o + hb * HD + d;
  // Loads in the order their consumers need them, all issued before any
  // wait: wave 0's (m, l) pairs of splits lane (its M/L pass), the gate (the
  // last step, wave 0), then every wave's 16 partials.  The partial loads are
  // unconditional (splits past the end re-read the last; the fma below skips
  // them): under a branch, a load leaves the compiler no exact count of loads
  // in flight, and its wait would cover every load issued before it.
  float2 ml0 = make_float2(-INFINITY, 0.0f);
  float g = 0.0f;
  if (wid == 0) {
    ml0 = *(const float2*)(a.part_ml + (hb + (size_t)min(lane, a.max_splits - 1) * G) * 2);
    if (a.gated) g = a.qkv[(size_t)qh * 2 * HD + HD + d];
  }
  float pv[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int t = min(wid + 4 * i, a.max_splits - 1);
    pv[i] = pb[(size_t)t * tstride];
  }
  const int seq = a.fixed_seq > 0 ? a.fixed_seq : __builtin_amdgcn_readfirstlane(sv) + 1;
  const int C = attn_chunk_for(seq, HD, a.n_kv);
  const int n_active = (seq + C - 1) / C;
  if (wid == 0) {
    float M = lane < n_active ? ml0.x : -INFINITY;
    for (int t = lane + 64; t < n_active; t += 64) M = fmaxf(M, a.part_ml[(hb + (size_t)t * G) * 2]);
    M = wave_max(M);
    float L = 0.0f;
    if (lane < n_active) {
      const float e = hx_exp(ml0.x - M);
      wts[lane] = e;
      L += e * ml0.y;
    }
    for (int t = lane + 64; t < n_active; t += 64) {
      float e = hx_exp(a.part_ml[(hb + (size_t)t * G) * 2] - M);
      wts[t] = e;
      L += e * a.part_ml[(hb + (size_t)t * G) * 2 + 1];
    }
    L = wave_sum(L);
    if (lane == 0) *sL = L;
  }
  __syncthreads();
  float P = 0.0f;
  for (int t0 = 0; t0 < n_active; t0 += 64) {
    if (t0 > 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int t = min(t0 + wid + 4 * i, n_active - 1);
        pv[i] = pb[(size_t)t * tstride];
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = t0 + wid + 4 * i;
      if (t < n_active) P = fmaf(wts[t], pv[i], P);
    }
  }
  pw[wid * 64 + lane] = P;
  __syncthreads();
  if (wid != 0) return;
  float o = (pw[lane] + pw[64 + lane]) + (pw[128 + lane] + pw[192 + lane]);
  o = o * (1.0f / *sL);
  if (a.gated) o = o / (1.0f + hx_exp(-g));   // qwen35.rs:1627-1629 attn_out /= 1 + exp(-gate)
  if (a.out_f32) a.out_f32[(size_t)qh * HD + d] = o;
  if (a.act_out) {
    float am = group_max<32>(fabsf(o));
    float scq = q8_scale(am);
    int q = q8_round_r(o, scq, q8_rcp(scq));
    int qsum = group_sum_i<32>(q);
    int e = qh * HD + d;
    int K = a.n_heads * HD;
    a.act_out[perm_pos(a.act_fmt, e)] = (uint8_t)(int8_t)q;
    if ((lane & 31) == 0) {
      ((float*)(a.act_out + K))[e >> 5] = h2f(f2h(scq));
      ((int*)(a.act_out + K + (K / 32) * 4))[e >> 5] = qsum;
    }
  }
}

// ---------------------------------------------------------------------------
// Batched prefill (forward_batch, mod.rs:899-1221) pieces.  Each restates, per
// token row, the arithmetic of the decode step's fused kernels, so a prompt
// prefilled here leaves the same KV cache and residual stream as one fed token
// by token.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_embed_rows(int type, const uint8_t* __restrict__ table, int d,
                                                    const uint32_t* __restrict__ toks, float* __restrict__ H,
                                                    const float* __restrict__ signs, int had_block) {
  extern __shared__ __align__(16) float ebuf[];
  const int s = blockIdx.x;
  embed_row<256>(type, table, d, (int)toks[s], H + (size_t)s * d, signs, had_block, ebuf);
}

// The fold of a matmul input row (qwen35.rs:914-941) then Q8_0 into the GEMM's
// split layout, for row s = blockIdx.x: optional rms_norm(x, w) first (the
// k_norm_q8_rows arithmetic), optional GDN grouped head order
// (qwen35.rs:1452-1478), signs, the WHT per had_block chunk, then per 32-block
// the Q8_0 of the rotated values.  buf: K floats of LDS.
__global__ __launch_bounds__(256) void k_rot_q8_rows(const float* __restrict__ X, const float* __restrict__ w,
                                                     float eps, int K, const float* __restrict__ signs, int had_block,
                                                     int perm_nk, int perm_rep, int8_t* __restrict__ xq,
                                                     float* __restrict__ xd) {
  extern __shared__ __align__(16) float rbuf[];
  __shared__ float red16[16];
  const int s = blockIdx.x, tid = threadIdx.x;
  const float* x = X + (size_t)s * K;
  float inv = 1.0f;
  if (w) inv = 1.0f / sqrtf(block_sumsq_f4(x, K, red16) / (float)K + eps);   // ops.rs:22-23
  for (int e = tid * 4; e < K; e += 1024) {
    const float4 xv = *(const float4*)(x + e);
    float v[4] = {xv.x, xv.y, xv.z, xv.w};
    if (w) {
      const float4 wv = *(const float4*)(w + e);
      v[0] = v[0] * inv * wv.x; v[1] = v[1] * inv * wv.y; v[2] = v[2] * inv * wv.z; v[3] = v[3] * inv * wv.w;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = perm_rep > 1 ? grouped_pos(e + i, 128, perm_nk, perm_rep) : e + i;
      rbuf[d] = v[i] * signs[d];
    }
  }
  lds_wht<256>(rbuf, K, had_block);
  for (int e = tid * 4; e < K; e += 1024) {
    const float4 t = *(const float4*)(rbuf + e);
    float vv[4] = {t.x, t.y, t.z, t.w};
    float am = fmaxf(fmaxf(fabsf(vv[0]), fabsf(vv[1])), fmaxf(fabsf(vv[2]), fabsf(vv[3])));
    am = group_max<8>(am);
    const float sc = q8_scale(am), rc = q8_rcp(sc);
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) word |= ((uint32_t)q8_round_r(vv[i], sc, rc) & 0xffu) << (8 * i);
    *(uint32_t*)(xq + (size_t)s * K + e) = word;
    if ((tid & 7) == 0) xd[(size_t)s * (K / 32) + (e >> 5)] = h2f(f2h(sc));
  }
}

// rms_norm(x_s, w) then Q8_0 of row s = blockIdx.x into the GEMM's split
// layout (int8 xq[s][K], f32 block scales xd[s][K/32]): the GEMV prologue's
// arithmetic (block_sumsq_f4 order, (x * inv) * w, per-block scale from the max
// of |v|, reciprocal rounding with the exact tie fallback).
__global__ __launch_bounds__(256) void k_norm_q8_rows(const float* __restrict__ X, const float* __restrict__ w,
                                                      float eps, int K, int8_t* __restrict__ xq, float* __restrict__ xd) {
  __shared__ float red16[16];
  const int s = blockIdx.x, tid = threadIdx.x;
  const float* x = X + (size_t)s * K;
  const float tot = block_sumsq_f4(x, K, red16);
  const float inv = 1.0f / sqrtf(tot / (float)K + eps);   // ops.rs:22-23
  for (int e = tid * 4; e < K; e += 1024) {
    const float4 xv = *(const float4*)(x + e), wv = *(const float4*)(w + e);
    float vv[4] = {xv.x * inv * wv.x, xv.y * inv * wv.y, xv.z * inv * wv.z, xv.w * inv * wv.w};
    float am = fmaxf(fmaxf(fabsf(vv[0]), fabsf(vv[1])), fmaxf(fabsf(vv[2]), fabsf(vv[3])));
    am = group_max<8>(am);
    const float sc = q8_scale(am), rc = q8_rcp(sc);
    uint32_t word = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) word |= ((uint32_t)q8_round_r(vv[i], sc, rc) & 0xffu) << (8 * i);
    *(uint32_t*)(xq + (size_t)s * K + e) = word;
    if ((tid & 7) == 0) xd[(size_t)s * (K / 32) + (e >> 5)] = h2f(f2h(sc));
  }
}

// The residual add then k_norm_q8_rows of the same rows, one pass: H = H + T
// (k_add_rows' add) is kept in registers, written back, and normalized from
// there.  Lane tid holds elements (tid + 256 i) * 4, which are both
// block_sumsq_f4's slots (slot j sums i = j, j + 4, ... in that order) and
// k_norm_q8_rows' quantization slices, so every sum and rounding is theirs.
__global__ __launch_bounds__(256) void k_add_norm_q8_rows(float* __restrict__ H, const float* __restrict__ T,
                                                          const float* __restrict__ w, float eps, int K,
                                                          int8_t* __restrict__ xq, float* __restrict__ xd) {
  __shared__ float red16[16];
  const int s = blockIdx.x, tid = threadIdx.x;
  float* h = H + (size_t)s * K;
  const float* t = T + (size_t)s * K;
  const int NI = K / 1024;   // <= 8
  float4 v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i < NI) {
      const int e = (tid + 256 * i) * 4;
      const float4 a = *(const float4*)(h + e), b = *(const float4*)(t + e);
      v[i] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);   // mod.rs:718-720, :776-778
      *(float4*)(h + e) = v[i];
    }
  }
  float ss[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    ss[j] = 0.0f;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      if (j + 4 * c < NI) {
        const float4 x = v[j + 4 * c];
        ss[j] += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) ss[j] = wave_sum(ss[j]);
  if ((tid & 63) == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) red16[(tid >> 6) + 4 * j] = ss[j];
  }
  __syncthreads();
  const float tot = tree16(red16);
  const float inv = 1.0f / sqrtf(tot / (float)K + eps);   // ops.rs:22-23
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i < NI) {
      const int e = (tid + 256 * i) * 4;
      const float4 xv = v[i], wv = *(const float4*)(w + e);
      float vv[4] = {xv.x * inv * wv.x, xv.y * inv * wv.y, xv.z * inv * wv.z, xv.w * inv * wv.w};
      float am = fmaxf(fmaxf(fabsf(vv[0]), fabsf(vv[1])), fmaxf(fabsf(vv[2]), fabsf(vv[3])));
      am = group_max<8>(am);
      const float sc = q8_scale(am), rc = q8_rcp(sc);
      uint32_t word = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) word |= ((uint32_t)q8_round_r(vv[k], sc, rc) & 0xffu) << (8 * k);
      *(uint32_t*)(xq + (size_t)s * K + e) = word;
      if ((tid & 7) == 0) xd[(size_t)s * (K / 32) + (e >> 5)] = h2f(f2h(sc));
    }
  }
}

// silu(g) * u of the [gate; up] rows of token s, then Q8_0 into the split
// layout: the SILU epilogue's arithmetic (ops.rs:240-253, q8_0.rs:20-51), on
// float4 slices (F % 1024 == 0): lane l of pass p takes elements
// 4(256p + l) .. +3, so a Q8_0 block is 8 lanes and its max a group max over
// them (exact: max does not depend on the order); four passes' loads are
// issued together.
__global__ __launch_bounds__(256) void k_silu_q8_rows4(const float* __restrict__ GU, int F, int8_t* __restrict__ xq,
                                                       float* __restrict__ xd, float* __restrict__ yf) {
  const int s = blockIdx.x, tid = threadIdx.x;
  const float* g = GU + (size_t)s * 2 * F;
  const int np = F / 1024;
#pragma unroll 4
  for (int p = 0; p < np; ++p) {
    const int i = 4 * (256 * p + tid);
    const float4 gv4 = *(const float4*)(g + i), uv4 = *(const float4*)(g + F + i);
    const float gv[4] = {gv4.x, gv4.y, gv4.z, gv4.w}, uv[4] = {uv4.x, uv4.y, uv4.z, uv4.w};
    float h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float sg = gv[k] / (1.0f + hx_exp(-gv[k]));
      h[k] = sg * uv[k];
    }
    if (yf) {   // folded model: rotated and quantized by k_rot_q8_rows
      *(float4*)(yf + (size_t)s * F + i) = make_float4(h[0], h[1], h[2], h[3]);
      continue;
    }
    float am = fmaxf(fmaxf(fabsf(h[0]), fabsf(h[1])), fmaxf(fabsf(h[2]), fabsf(h[3])));
    am = group_max<8>(am);
    const float sc = q8_scale(am), rc = q8_rcp(sc);
    uint32_t word = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) word |= ((uint32_t)q8_round_r(h[k], sc, rc) & 0xffu) << (8 * k);
    *(uint32_t*)(xq + (size_t)s * F + i) = word;
    if ((tid & 7) == 0) xd[(size_t)s * (F / 32) + (i >> 5)] = h2f(f2h(sc));
  }
}

__global__ void k_add_rows(float* __restrict__ H, const float* __restrict__ T, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) H[i] = H[i] + T[i];   // mod.rs:718-720, :776-778
}

// Per token s (blockIdx.x) and kv head (blockIdx.y): the G query heads' and
// the key's per-head RMSNorm + RoPE on float4 slices of LPR lanes (the split
// kernel's slice_norm / slice_rope), K and V written at pos0 + s, the
// rotated q kept for the attention pass.  One LPR-lane group per head.
template <int HD, bool KV8>
__global__ __launch_bounds__(512) void k_prefill_qk(const float* __restrict__ QKV, int n_in, int n_heads, int n_kv,
                                                    const float* __restrict__ q_norm, const float* __restrict__ k_norm,
                                                    float eps, const float* __restrict__ rope, int rope_dim,
                                                    int max_seq, int pos0, int gated, float* __restrict__ k_cache,
                                                    float* __restrict__ v_cache, float* __restrict__ QB) {
  constexpr int LPR = HD / 4;
  const int s = blockIdx.x, kvh = blockIdx.y, G = n_heads / n_kv;
  const int grp = threadIdx.x / LPR, c = threadIdx.x % LPR;
  const int pos = pos0 + s;
  const float* row = QKV + (size_t)s * n_in;
  if (grp > G) return;   // whole LPR-lane groups
  const bool is_k = grp == G;
  const int qh = kvh * G + grp;
  // qwen35 gated attention interleaves [q_h | gate_h] per head (qwen35.rs:1552-1559)
  const size_t qs = gated ? 2 * HD : HD, kv0 = (size_t)n_heads * qs;
  float4 x = is_k ? *(const float4*)(row + kv0 + (size_t)kvh * HD + 4 * c)
                  : *(const float4*)(row + (size_t)qh * qs + 4 * c);
  const float* nw = is_k ? k_norm : q_norm;
  if (nw) x = slice_norm<LPR>(x, *(const float4*)(nw + 4 * c), eps);
  if (rope) {
    float4 sn = make_float4(0.f, 0.f, 0.f, 0.f), cs = sn;
    if (4 * c < rope_dim) rope_row(rope, pos, max_seq, rope_dim, 4 * c, sn, cs);
    x = slice_rope(x, sn, cs, 4 * c, rope_dim);
  }
  if (is_k) {
    const float4 v = *(const float4*)(row + kv0 + (size_t)n_kv * HD + (size_t)kvh * HD + 4 * c);
    if constexpr (KV8) {   // quantized on write exactly as the decode step's kv_q8_store
      const size_t r = (size_t)kvh * max_seq + pos;
      kv_q8_store(x, KvQ8(k_cache, n_kv, max_seq, HD), r, HD, c, true);
      kv_q8_store(v, KvQ8(v_cache, n_kv, max_seq, HD), r, HD, c, true);
    } else {
      const size_t off = ((size_t)kvh * max_seq + pos) * HD + 4 * c;
      *(float4*)(k_cache + off) = x;
      *(float4*)(v_cache + off) = v;
    }
  } else {
    *(float4*)(QB + (size_t)s * n_heads * HD + (size_t)qh * HD + 4 * c) = x;
  }
}

// Prefill attention, split pass: workgroup (chunk c, kv head, token tile)
// holds K/V rows of chunk c in registers exactly as k_attn_split does and
// runs the decode arithmetic (scores, chunk softmax, P.V and their reduction
// order) once per token of the tile whose position reaches the chunk, NTOK
// tokens per pass.  GMAX bounds the query heads per kv head (registers).
// Partials: PO[((sl*n_kv + kvh)*n_chunks + c)*G + h][HD], PML likewise x2.
template <int HD, int NTA, bool KV8, int GMAX, int NTOK, int GT, int C>
__global__ __launch_bounds__(NTA) void k_attn_prefill_split(const float* __restrict__ QB, const float* __restrict__ k_cache,
                                                            const float* __restrict__ v_cache, int n_heads, int n_kv,
                                                            int max_seq, int pos0, int S, int t0, int TT, int n_chunks,
                                                            float* __restrict__ PO, float* __restrict__ PML) {
  constexpr int LPR = HD / 4, RPI = NTA / LPR, NR = C / RPI, NW = NTA / 64;
  extern __shared__ __align__(16) float sm[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int c = blockIdx.x, kvh = blockIdx.y, G = GT > 0 ? GT : n_heads / n_kv;
  const int sl0 = blockIdx.z * TT, sl1 = min(sl0 + TT, S - t0);   // tile-launch-relative tokens
  const int p0 = c * C;
  const int np_max = min(C, pos0 + t0 + sl1 - p0);
  if (sl0 >= sl1 || np_max <= 0) return;
  const int sub = tid / LPR, cc = tid % LPR;
  float* sc = sm;                          // NTOK * G * C
  float* ml = sc + NTOK * G * C;           // NTOK * 2 * G (+pad)
  float* red = ml + ((NTOK * 2 * G + 4 + 3) & ~3);   // NTOK * NW waves * 4 heads * HD (16-byte aligned)
  const size_t hstride = (size_t)max_seq * HD;
  const float* kg = k_cache + (size_t)kvh * hstride + 4 * cc;
  const float* vg = v_cache + (size_t)kvh * hstride + 4 * cc;
  // K rows and q heads in the reduce-scatter's register order
  // (ReduceScatter): K register i holds row (i ^ pi) * RPI + sub, q register
  // h of a group of four head (h ^ ph); V rows stay in order (the P.V chain
  // runs over i).  The q rows arrive normalized and rotated, so no step here
  // needs the lanes of a row on one head.
  constexpr int NV = 4 * NR;
  const int rsp = rs_perm<NV, LPR / 2>(lane), pi = rsp % NR, ph = rsp / NR;
  float4 kr[NR], vr[NR];
  // every K row before the V rows (the scores need only K)
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int jk = (i ^ pi) * RPI + sub;
    kr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (KV8) {
      const size_t r = (size_t)kvh * max_seq + p0;
      if (jk < np_max) kr[i] = KvQ8(const_cast<float*>(k_cache), n_kv, max_seq, HD).load(r + jk, HD, cc);
    } else {
      if (jk < np_max) kr[i] = *(const float4*)(kg + (size_t)(p0 + jk) * HD);
    }
  }
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int j = i * RPI + sub;
    vr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (KV8) {
      const size_t r = (size_t)kvh * max_seq + p0;
      if (j < np_max) vr[i] = KvQ8(const_cast<float*>(v_cache), n_kv, max_seq, HD).load(r + j, HD, cc);
    } else {
      if (j < np_max) vr[i] = *(const float4*)(vg + (size_t)(p0 + j) * HD);
    }
  }
  const float inv_sqrt = 1.0f / sqrtf((float)HD);
  constexpr int KSH = (LPR == 64 ? 6 : 5) - (NV == 32 ? 5 : NV == 16 ? 4 : 3);
  // NTOK tokens per pass (each with the decode arithmetic of one token): their
  // softmax rows spread over all waves and they share the barriers.  Tokens
  // before the first whose position reaches the chunk skip it.
  const int sl_first = max(sl0, p0 - pos0 - t0);
  for (int sl = sl_first; sl < sl1; sl += NTOK) {
    const int nt = min(NTOK, sl1 - sl);
#pragma unroll
    for (int u = 0; u < NTOK; ++u) {
      if (u >= nt) break;   // uniform
      const int s = t0 + sl + u, np = min(C, pos0 + s + 1 - p0);
      float4 q4[GMAX];
#pragma unroll
      for (int h = 0; h < GMAX; ++h) {
        q4[h] = make_float4(0.f, 0.f, 0.f, 0.f);
        if ((h & ~3) < G) {
          const int hs = (h & ~3) | ((h & 3) ^ ph);
          const float* qp = QB + (size_t)s * n_heads * HD + (size_t)(kvh * G + hs) * HD + 4 * cc;
          q4[h] = *(const float4*)(hs < G ? qp : attn_zero_row);
        }
      }
      float* scu = sc + u * G * C;
#pragma unroll
      for (int hg = 0; hg < GMAX; hg += 4) {
        if (hg >= G) break;
        float v[NV];
#pragma unroll
        for (int hh = 0; hh < 4; ++hh) {
          const float4 qq = hg + hh < GMAX ? q4[hg + hh] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
          for (int i = 0; i < NR; ++i) {
            float pp = qq.x * kr[i].x;
            pp = fmaf(qq.y, kr[i].y, pp);
            pp = fmaf(qq.z, kr[i].z, pp);
            pp = fmaf(qq.w, kr[i].w, pp);
            v[hh * NR + i] = pp;
          }
        }
        const float r = ReduceScatter<NV, LPR / 2>::run(v);
        const int k = (lane & (LPR - 1)) >> KSH;
        const int h = hg + k / NR, j = (k % NR) * RPI + sub;
        if (h < G && (lane & ((1 << KSH) - 1)) == 0) scu[h * C + j] = (j < np) ? r * inv_sqrt : -INFINITY;
      }
    }
    __syncthreads();
    for (int pr = wid; pr < nt * G; pr += NW) {
      const int u = pr / G, h = pr % G;
      const int np = min(C, pos0 + t0 + sl + u + 1 - p0);
      float* row = sc + (u * G + h) * C;
      if constexpr (C <= 64) {
        float x = lane < C ? row[lane] : -INFINITY;
        float m = wave_max_nonan(x);
        float e = (lane < np) ? hx_exp(x - m) : 0.0f;
        float l = wave_sum(e);
        if (lane < C) row[lane] = e;
        if (lane == 0) { ml[(u * G + h) * 2] = m; ml[(u * G + h) * 2 + 1] = l; }
      } else {   // C = 128, as the decode split
        const float x0 = row[lane], x1 = row[64 + lane];
        const float m = wave_max_nonan(fmaxf(x0, x1));
        const float e0 = (lane < np) ? hx_exp(x0 - m) : 0.0f;
        const float e1 = (64 + lane < np) ? hx_exp(x1 - m) : 0.0f;
        const float l = wave_sum(e0 + e1);
        row[lane] = e0;
        row[64 + lane] = e1;
        if (lane == 0) { ml[(u * G + h) * 2] = m; ml[(u * G + h) * 2 + 1] = l; }
      }
    }
    __syncthreads();
    for (int hg = 0; hg < G; hg += 4) {
#pragma unroll
      for (int u = 0; u < NTOK; ++u) {
        if (u >= nt) break;
        float acc[16];
#pragma unroll
        for (int hh = 0; hh < 4; ++hh) {
          float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
          if (hg + hh < G) {
            const float* eh = sc + (u * G + hg + hh) * C + sub;
#pragma unroll
            for (int i = 0; i < NR; ++i) {
              const float e = eh[i * RPI];
              o0 = fmaf(e, vr[i].x, o0);
              o1 = fmaf(e, vr[i].y, o1);
              o2 = fmaf(e, vr[i].z, o2);
              o3 = fmaf(e, vr[i].w, o3);
            }
          }
          acc[hh * 4 + 0] = o0; acc[hh * 4 + 1] = o1; acc[hh * 4 + 2] = o2; acc[hh * 4 + 3] = o3;
        }
        float* redu = red + u * NW * 4 * HD;
        if constexpr (LPR == 32) {
          const bool up = (lane & 32) != 0;
          float xs[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) xs[k] = swap_pair_sum<32>(acc[k], acc[k + 8]);
#pragma unroll
          for (int g = 0; g < 2; ++g)   // two 16-byte writes per lane, as the decode split
            *(float4*)(redu + (wid * 4 + g + (up ? 2 : 0)) * HD + 4 * cc) =
                make_float4(xs[4 * g], xs[4 * g + 1], xs[4 * g + 2], xs[4 * g + 3]);
        } else {
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *(float4*)(redu + (wid * 4 + g) * HD + 4 * cc) =
                make_float4(acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]);
        }
      }
      __syncthreads();
      if constexpr (4 * HD == NTA) {
        // lane tid owns value r4 = tid of every token u: its partial sits at
        // a fixed offset from token u's block, one token stride apart
        const int h = hg + tid / HD;
        if (h < G) {
          const size_t tok = (size_t)n_kv * n_chunks * G * HD;
          float* dst = PO + (((size_t)sl * n_kv + kvh) * n_chunks + c) * G * HD + (size_t)hg * HD + tid;
          for (int u = 0; u < nt; ++u) {
            const float* redu = red + u * NW * 4 * HD;
            float t[NW];
#pragma unroll
            for (int w = 0; w < NW; ++w) t[w] = redu[w * 4 * HD + tid];
            dst[u * tok] = pairwise_tree<NW>(t);
          }
        }
      } else {
        for (int idx = tid; idx < nt * 4 * HD; idx += NTA) {
          const int u = idx / (4 * HD), r4 = idx % (4 * HD);
          const int h = hg + r4 / HD;
          if (h < G) {
            const float* redu = red + u * NW * 4 * HD;
            float t[NW];
#pragma unroll
            for (int w = 0; w < NW; ++w) t[w] = redu[w * 4 * HD + r4];
            const size_t pbase = ((size_t)((sl + u) * n_kv + kvh) * n_chunks + c) * G;
            PO[(pbase + h) * HD + (r4 % HD)] = pairwise_tree<NW>(t);
          }
        }
      }
      __syncthreads();
    }
    if (tid < nt * G) {
      const int u = tid / G, h = tid % G;
      const size_t pbase = ((size_t)((sl + u) * n_kv + kvh) * n_chunks + c) * G;
      PML[(pbase + h) * 2] = ml[(u * G + h) * 2];
      PML[(pbase + h) * 2 + 1] = ml[(u * G + h) * 2 + 1];
    }
  }
}

// Prefill attention, merge pass: k_attn_merge's arithmetic for token t0 + sl,
// one wave per (token, query head): pair blockIdx.x * 4 + wave = sl * n_heads
// + qh.  Lane l holds columns CPL*l .. CPL*l + CPL-1 (CPL = HD / 64) and runs
// the four split chains of k_attn_merge's four waves itself (chain g: splits
// t = g (mod 4), fma in increasing t), then ((P0 + P1) + (P2 + P3)) / L.  M and
// L are k_attn_merge's wave-0 pass.  Writes the Q8_0 row of attn_output's
// input in the GEMM's split layout.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_prefill_merge(const float* __restrict__ PO, const float* __restrict__ PML,
                                                            int n_heads, int n_kv, int n_chunks, int C, int pos0, int t0,
                                                            int n, const float* __restrict__ gate, int gate_row,
                                                            int8_t* __restrict__ yq, float* __restrict__ yd,
                                                            float* __restrict__ yf) {
  constexpr int CPL = HD / 64;
  extern __shared__ __align__(16) float wm[];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  float* wts = wm + wid * n_chunks;        // this wave's split weights
  const int pair = blockIdx.x * 4 + wid;
  const bool live = pair < n * n_heads;    // uniform per wave
  const int sl = live ? pair / n_heads : 0, qh = pair % n_heads;
  const int G = n_heads / n_kv, kvh = qh / G, h = qh % G;
  const int s = t0 + sl, seq = pos0 + s + 1;
  const int n_active = live ? (seq + C - 1) / C : 0;
  const size_t hb = (size_t)(sl * n_kv + kvh) * n_chunks * G + h;
  const size_t tstride = (size_t)G * HD;
  const int d0 = CPL * lane;
  const float* pb = PO + hb * HD + d0;
  float M = -INFINITY;
  for (int t = lane; t < n_active; t += 64) M = fmaxf(M, PML[(hb + (size_t)t * G) * 2]);
  M = wave_max(M);
  float L = 0.0f;
  for (int t = lane; t < n_active; t += 64) {
    float e = hx_exp(PML[(hb + (size_t)t * G) * 2] - M);
    wts[t] = e;
    L += e * PML[(hb + (size_t)t * G) * 2 + 1];
  }
  L = wave_sum(L);
  __syncthreads();
  float P[4][CPL];
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int k = 0; k < CPL; ++k) P[g][k] = 0.0f;
  for (int tb = 0; tb < n_active; tb += 16) {
    float pv[16][CPL];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float* src = pb + (size_t)min(tb + i, n_active - 1) * tstride;
      if constexpr (CPL == 2) {
        const float2 v = *(const float2*)src;
        pv[i][0] = v.x; pv[i][1] = v.y;
      } else {
        const float4 v = *(const float4*)src;
        pv[i][0] = v.x; pv[i][1] = v.y; pv[i][2] = v.z; pv[i][3] = v.w;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = tb + i;
      if (t < n_active) {
        const float w = wts[t];
#pragma unroll
        for (int k = 0; k < CPL; ++k) P[i & 3][k] = fmaf(w, pv[i][k], P[i & 3][k]);
      }
    }
  }
  if (!live) return;
  const float rl = 1.0f / L;
  float o[CPL], gv[CPL];
  if (gate) {
    const float* gp = gate + (size_t)s * gate_row + (size_t)qh * 2 * HD + HD + d0;
#pragma unroll
    for (int k = 0; k < CPL; ++k) gv[k] = gp[k];
  }
#pragma unroll
  for (int k = 0; k < CPL; ++k) {
    o[k] = (P[0][k] + P[1][k]) + (P[2][k] + P[3][k]);
    o[k] = o[k] * rl;
    if (gate) o[k] = o[k] / (1.0f + hx_exp(-gv[k]));   // qwen35.rs:1627-1629, as k_attn_merge
  }
  if (yf) {   // folded model: rotated and quantized by k_rot_q8_rows
#pragma unroll
    for (int k = 0; k < CPL; ++k) yf[(size_t)s * n_heads * HD + qh * HD + d0 + k] = o[k];
    return;
  }
  // one Q8_0 block = 32 columns = 32 / CPL lanes
  float am = fabsf(o[0]);
#pragma unroll
  for (int k = 1; k < CPL; ++k) am = fmaxf(am, fabsf(o[k]));
  am = group_max<32 / CPL>(am);
  const float scq = q8_scale(am), rc = q8_rcp(scq);
  const int e = qh * HD + d0, K = n_heads * HD;
  uint32_t word = 0;
#pragma unroll
  for (int k = 0; k < CPL; ++k) word |= ((uint32_t)q8_round_r(o[k], scq, rc) & 0xffu) << (8 * k);
  if constexpr (CPL == 2) *(uint16_t*)(yq + (size_t)s * K + e) = (uint16_t)word;
  else *(uint32_t*)(yq + (size_t)s * K + e) = word;
  if ((lane & (32 / CPL - 1)) == 0) yd[(size_t)s * (K / 32) + (e >> 5)] = h2f(f2h(scq));
}

// ---------------------------------------------------------------------------
// Prefill attention on fp32 MFMA (opt-in, HH_PREFILL_ATTN=mfma): the causal
// attention of a whole prompt as a flash-style pass per (token tile, kv head),
// for the batched prefill only.  It regroups the fp32 sums (16x16x4 MFMA
// products, an online softmax over 32-position chunks, exp2 of prescaled
// scores), so it matches the split/merge path (and token-by-token decode) to
// fp32 rounding, not bit for bit; that path stays the default.
//
// Workgroup = W = G*T waves, T = max(1, 8 / G) token tiles of 16 (4 to 8
// waves); wave w handles query head kvh*G + w % G for tokens s0 + 16 (w / G)
// + 0..15, so a staged chunk serves up to 8 query rows per position.  The 1-D
// grid runs the kv heads fastest: with the round-robin dispatch over the 8
// XCDs, one kv head's workgroups share an XCD and its L2 (n_kv dividing 8).
// The workgroup stages each 32-position chunk of its kv head's K and V in LDS
// (dequantized when the cache holds Q8_0 rows).  Per chunk and wave:
//   S^T (positions x queries) = K Q^T: A = K rows, B = Q^T held in registers,
//     dims permuted within 16-dim blocks (lane group g takes dims 16j + 4g + m
//     in step m) on both operands, so each step still sums matching dims;
//   online softmax per query column (each lane owns one query);
//   O^T (dims x queries) += V^T P^T: P^T stays in the C registers of S^T, read
//     in step r as position 4g + r of the lane's group, with A = V[4g + r][dim].
// Then O / L, the qwen35 sigmoid gate, and the Q8_0 row of attn_output's input
// in the GEMM's split layout (or the f32 row for a folded model).
template <int HD, bool KV8>
__global__ __launch_bounds__(512) void k_attn_prefill_mfma(const float* __restrict__ QB, const float* __restrict__ k_cache,
                                                           const float* __restrict__ v_cache, int n_heads, int n_kv,
                                                           int max_seq, int pos0, int t0, int n,
                                                           const float* __restrict__ gate, int gate_row,
                                                           int8_t* __restrict__ yq, float* __restrict__ yd,
                                                           float* __restrict__ yf) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  // chunk positions (64 measured the same at head_dim 128), LDS row stride,
  // dim blocks, 16-position tiles
  constexpr int CHK = 32, RS = HD + 4, NJ = HD / 16, NQT = CHK / 16;
  __shared__ __align__(16) float Ks[CHK * RS];
  __shared__ __align__(16) float Vs[CHK * RS];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6, nth = blockDim.x;
  const int mi = lane & 15, g = lane >> 4;
  const int G = n_heads / n_kv, T = G >= 8 ? 1 : 8 / G;
  const int kvh = (int)blockIdx.x % n_kv, h = wid % G, qh = kvh * G + h;
  const int tile0 = t0 + ((int)blockIdx.x / n_kv) * 16 * T;   // first token of the workgroup
  const int last = min(t0 + n, tile0 + 16 * T) - 1;           // its last valid token
  const int sq_raw = tile0 + 16 * (wid / G) + mi;
  const bool qvalid = sq_raw < t0 + n;
  const int sq = min(sq_raw, t0 + n - 1);                     // out-of-range lanes compute a valid row
  const int pq = pos0 + sq;
  // q prescaled by log2(e) / sqrt(HD): the scores come out in base-2 units
  const float qs = 1.4426950408889634f / sqrtf((float)HD);
  f32x4 q4[NJ];
  {
    const float* qp = QB + ((size_t)sq * n_heads + qh) * HD + 4 * g;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float4 v = *(const float4*)(qp + 16 * j);
      q4[j] = (f32x4){v.x * qs, v.y * qs, v.z * qs, v.w * qs};
    }
  }
  f32x4 o[NJ];
#pragma unroll
  for (int t = 0; t < NJ; ++t) o[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;
  const int p_last = pos0 + last;
  const int n_chunks = p_last / CHK + 1;
  const KvQ8 kq(const_cast<float*>(k_cache), n_kv, max_seq, HD), vq(const_cast<float*>(v_cache), n_kv, max_seq, HD);
  const size_t row0 = (size_t)kvh * max_seq;
  for (int c = 0; c < n_chunks; ++c) {
    const int pbase = c * CHK;
    __syncthreads();   // every wave is done with the previous chunk
    for (int i = tid; i < CHK * HD / 4; i += nth) {
      const int r = i / (HD / 4), cc = i % (HD / 4);
      const int p = min(pbase + r, p_last);   // rows past the last position: any valid row (masked below)
      float4 kv, vv;
      if constexpr (KV8) {
        kv = kq.load(row0 + p, HD, cc);
        vv = vq.load(row0 + p, HD, cc);
      } else {
        kv = *(const float4*)(k_cache + (row0 + p) * HD + 4 * cc);
        vv = *(const float4*)(v_cache + (row0 + p) * HD + 4 * cc);
      }
      *(float4*)(Ks + r * RS + 4 * cc) = kv;
      *(float4*)(Vs + r * RS + 4 * cc) = vv;
    }
    __syncthreads();
    // S^T for the chunk's 16-position tiles
    f32x4 sc[NQT];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      const float* kr = Ks + (16 * qt + mi) * RS + 4 * g;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const float4 k4 = *(const float4*)(kr + 16 * j);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.x, q4[j][0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.y, q4[j][1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.z, q4[j][2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.w, q4[j][3], acc, 0, 0, 0);
      }
      sc[qt] = acc;
    }
    // causal mask and the chunk's maximum per query
    float cmax = -INFINITY;
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p = pbase + 16 * qt + 4 * g + r;
        if (p > pq) sc[qt][r] = -INFINITY;
        cmax = fmaxf(cmax, sc[qt][r]);
      }
    cmax = fmaxf(cmax, xor_lane<16>(cmax));
    cmax = fmaxf(cmax, xor_lane<32>(cmax));
    const float m_new = fmaxf(m_run, cmax);   // position 0 is in chunk 0: finite from the start
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float psum = 0.0f;
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[qt][r] = __builtin_amdgcn_exp2f(sc[qt][r] - m_new);
        psum += sc[qt][r];
      }
    psum += xor_lane<16>(psum);
    psum += xor_lane<32>(psum);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < NJ; ++t) o[t] *= alpha;
    // O^T += V^T P^T
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float* vr = Vs + (16 * qt + 4 * g + r) * RS + mi;
#pragma unroll
        for (int t = 0; t < NJ; ++t)
          o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[16 * t], sc[qt][r], o[t], 0, 0, 0);
      }
  }
  // lane holds dims 16 t + 4 g + r of token sq
  const float rl = 1.0f / l_run;
  const int K = n_heads * HD;
#pragma unroll
  for (int t = 0; t < NJ; ++t) {
    o[t] *= rl;
    if (gate) {   // qwen35.rs:1627-1629: attn_out /= 1 + exp(-gate)
      const float4 gv = *(const float4*)(gate + (size_t)sq * gate_row + (size_t)qh * 2 * HD + HD + 16 * t + 4 * g);
      const float gg[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) o[t][r] = o[t][r] / (1.0f + hx_exp(-gg[r]));
    }
  }
  if (yf) {
    if (qvalid)
#pragma unroll
      for (int t = 0; t < NJ; ++t)
        *(float4*)(yf + (size_t)sq * K + qh * HD + 16 * t + 4 * g) = make_float4(o[t][0], o[t][1], o[t][2], o[t][3]);
    return;
  }
#pragma unroll
  for (int b = 0; b < NJ / 2; ++b) {   // Q8_0 block b = dims 32 b .. 32 b + 31 = tiles 2b, 2b + 1
    float am = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) am = fmaxf(am, fabsf(o[2 * b + u][r]));
    am = fmaxf(am, xor_lane<16>(am));
    am = fmaxf(am, xor_lane<32>(am));
    const float scq = q8_scale(am), rc = q8_rcp(scq);
    if (qvalid) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        uint32_t word = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) word |= ((uint32_t)q8_round_r(o[2 * b + u][r], scq, rc) & 0xffu) << (8 * r);
        *(uint32_t*)(yq + (size_t)sq * K + qh * HD + 16 * (2 * b + u) + 4 * g) = word;
      }
      if (g == 0) yd[(size_t)sq * (K / 32) + (qh * HD) / 32 + b] = h2f(f2h(scq));
    }
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

// Measurement: stream n16 16-byte words, 8 loads in flight per lane, and keep
// nothing (the store needs a sum no launch produces: `never` is -1).  Its rate
// is the read-only HBM ceiling the decode step's streams are judged against.
__global__ __launch_bounds__(1024) void k_read_probe(const uint4* __restrict__ p, int64_t n16, int* sink, int never) {
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 7 * stride < n16; i += 8 * stride) {
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[i + u * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].w;
  }
  if (acc == 0x12345678u && (int)threadIdx.x == never) *sink = (int)acc;
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
// mode 0: Q2_0 codes, 1: Q1_0 sign bits, 2: the Q2_0 codes packed as PTQ1_0
// (ptq1_0.rs:604-643 packing), so a PTQ1_0 model holds the Q2_0 weights.
__global__ void k_synth_bits(int mode, uint64_t key, int64_t nblocks, float cq, uint8_t* out) {
  const int is_q1 = mode == 1;
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
  if (mode == 2) {
    auto code = [&](int e) -> uint32_t {
      int32_t x = iv[e];
      int64_t ax = x < 0 ? -(int64_t)x : x;
      return (S > 0 && 256 * ax >= S) ? (x > 0 ? 2u : 0u) : 1u;
    };
    uint8_t* o = out + b * 28;
    for (int m = 0; m < 24; ++m) {
      uint32_t q = 0;
      for (int n = 0; n < 5; ++n) q = q * 3u + code(m < 16 ? 16 * n + m : 80 + 8 * n + (m - 16));
      o[m] = (uint8_t)((q * 256u + 242u) / 243u);
    }
    for (int hh = 0; hh < 2; ++hh) {
      uint32_t q = 0;
      for (int n = 0; n < 4; ++n) q = q * 3u + code(120 + hh + 2 * n);
      o[24 + hh] = (uint8_t)((q * 3u * 256u + 242u) / 243u);
    }
    o[26] = (uint8_t)(h & 0xff);
    o[27] = (uint8_t)(h >> 8);
    return;
  }
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

// Same values, stored as Q8_0 rows (one thread per 32-value block).
__global__ void k_kv_synth_q8(uint64_t key, int n_pos, int n_kv, int hd, int max_seq, float cs, float* cache) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int nb = hd / 32;
  if (b >= (int64_t)n_pos * n_kv * nb) return;
  const int blk = (int)(b % nb);
  const int64_t r = b / nb;
  const int h = (int)(r % n_kv), p = (int)(r / n_kv);
  float v[32], am = 0.0f;
  for (int j = 0; j < 32; ++j) {
    const int64_t i = r * hd + blk * 32 + j;   // the f32 generator's index ((p*n_kv)+h)*hd + j
    v[j] = h2f(f2h(__fmul_rn((float)synth_int(key, (uint64_t)i), cs)));
    am = fmaxf(am, fabsf(v[j]));
  }
  const float sc = q8_scale(am), rc = q8_rcp(sc);
  const size_t row = (size_t)h * max_seq + p;
  const KvQ8 kv(cache, n_kv, max_seq, hd);
  for (int j = 0; j < 32; ++j) kv.q[KvQ8::qoff(row, hd, blk * 8 + j / 4) + j % 4] = (int8_t)q8_round_r(v[j], sc, rc);
  kv.d[KvQ8::doff(row, hd, blk)] = (uint16_t)f2h(sc);
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

int hh_embed_launch(int type, const uint8_t* table, int d, const StepState* st, float* hidden,
                    const float* signs, int had_block, hipStream_t s) {
  if (had_block > 0 && (d % had_block || !signs)) return 1;
  hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), had_block > 0 ? (size_t)d * 4 : 0, s, type, table, d, st, hidden,
                     signs, had_block);
  return ok();
}

int hh_attn_launch(const AttnArgs& a, hipStream_t s) {
  const int G = a.n_heads / a.n_kv;
  if (a.hd != 128 && a.hd != 256) return 1;
  if (a.chunk != 8192 / a.hd || a.n_kv * G != a.n_heads || G > 8) return 1;
  const size_t split_lds = 4 * ((size_t)G * 2 * a.chunk + 2 * G + 8 + (ATTN_NT / 64) * 4 * (size_t)a.hd);   // wide chunks
  const size_t merge_lds = 4 * ((size_t)a.max_splits + 256 + 4);
  const dim3 g(a.max_splits * a.n_kv), b(ATTN_NT);
  auto split = [&](auto hd_c, auto kv8_c) {
    constexpr int HD = decltype(hd_c)::value;
    constexpr bool KV8 = decltype(kv8_c)::value;
    switch (G) {
      case 1: hipLaunchKernelGGL((k_attn_split<HD, ATTN_NT, KV8, 1>), g, b, split_lds, s, a); break;
      case 2: hipLaunchKernelGGL((k_attn_split<HD, ATTN_NT, KV8, 2>), g, b, split_lds, s, a); break;
      case 4: hipLaunchKernelGGL((k_attn_split<HD, ATTN_NT, KV8, 4>), g, b, split_lds, s, a); break;
      case 6: hipLaunchKernelGGL((k_attn_split<HD, ATTN_NT, KV8, 6>), g, b, split_lds, s, a); break;
      case 8: hipLaunchKernelGGL((k_attn_split<HD, ATTN_NT, KV8, 8>), g, b, split_lds, s, a); break;
      default: hipLaunchKernelGGL((k_attn_split<HD, ATTN_NT, KV8, 0>), g, b, split_lds, s, a); break;
    }
  };
  using T128 = std::integral_constant<int, 128>;
  using T256 = std::integral_constant<int, 256>;
  if (a.hd == 128) {
    if (a.kv_q8) split(T128{}, std::true_type{});
    else split(T128{}, std::false_type{});
    hipLaunchKernelGGL(k_attn_merge<128>, dim3(a.n_heads * 2), dim3(256), merge_lds, s, a);
  } else {
    if (a.kv_q8) split(T256{}, std::true_type{});
    else split(T256{}, std::false_type{});
    hipLaunchKernelGGL(k_attn_merge<256>, dim3(a.n_heads * 4), dim3(256), merge_lds, s, a);
  }
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
  } else if (type == 41 || type == 43 || type == 42 || type == 142 || type == 143) {
    int mode = (type == 41 || type == 43) ? 1 : type == 143 ? 2 : 0;
    hipLaunchKernelGGL(k_synth_bits, dim3(nblk(n / 128, 128)), dim3(128), 0, s, mode, key, n / 128, cq,
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

int hh_kv_synth_q8_launch(uint64_t key, int n_pos, int n_kv, int hd, int max_seq, float cs, float* cache,
                          hipStream_t s) {
  int64_t total = (int64_t)n_pos * n_kv * (hd / 32);
  if (total == 0) return 0;
  hipLaunchKernelGGL(k_kv_synth_q8, dim3(nblk(total, 64)), dim3(64), 0, s, key, n_pos, n_kv, hd, max_seq, cs,
                     cache);
  return ok();
}

int hh_embed_rows_launch(int type, const uint8_t* table, int d, const uint32_t* toks, int S, float* H,
                         const float* signs, int had_block, hipStream_t s) {
  if (had_block > 0 && (d % had_block || !signs)) return 1;
  hipLaunchKernelGGL(k_embed_rows, dim3(S), dim3(256), had_block > 0 ? (size_t)d * 4 : 0, s, type, table, d, toks, H,
                     signs, had_block);
  return ok();
}

int hh_rot_q8_rows_launch(const float* X, const float* w, float eps, int K, int S, const float* signs, int had_block,
                          int perm_nk, int perm_rep, int8_t* xq, float* xd, hipStream_t s) {
  if (K % 1024 != 0 || !signs || had_block < 2 || (had_block & (had_block - 1)) || K % had_block) return 1;
  if (perm_rep > 1 && K != perm_nk * perm_rep * 128) return 1;
  hipLaunchKernelGGL(k_rot_q8_rows, dim3(S), dim3(256), (size_t)K * 4, s, X, w, eps, K, signs, had_block, perm_nk,
                     perm_rep, xq, xd);
  return ok();
}

int hh_norm_q8_rows_launch(const float* X, const float* w, float eps, int K, int S, int8_t* xq, float* xd,
                           hipStream_t s) {
  if (K % 1024 != 0) return 1;
  hipLaunchKernelGGL(k_norm_q8_rows, dim3(S), dim3(256), 0, s, X, w, eps, K, xq, xd);
  return ok();
}

int hh_silu_q8_rows_launch(const float* GU, int F, int S, int8_t* xq, float* xd, float* yf, hipStream_t s) {
  if (F % 1024 != 0) return 1;   // models hold d_ffn to multiples of 1024
  hipLaunchKernelGGL(k_silu_q8_rows4, dim3(S), dim3(256), 0, s, GU, F, xq, xd, yf);
  return ok();
}

int hh_add_norm_q8_rows_launch(float* H, const float* T, const float* w, float eps, int K, int S, int8_t* xq,
                               float* xd, hipStream_t s) {
  if (K % 1024 != 0 || K > 8192) return 1;
  hipLaunchKernelGGL(k_add_norm_q8_rows, dim3(S), dim3(256), 0, s, H, T, w, eps, K, xq, xd);
  return ok();
}

int hh_add_rows_launch(float* H, const float* T, int64_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_add_rows, dim3(nblk(n, 256)), dim3(256), 0, s, H, T, n);
  return ok();
}

int hh_prefill_qk_launch(int hd, const float* QKV, int n_in, int n_heads, int n_kv, const float* q_norm,
                         const float* k_norm, float eps, const float* rope, int rope_dim, int max_seq, int pos0, int S,
                         int gated, int kv_q8, float* k_cache, float* v_cache, float* QB, hipStream_t s) {
  const int G = n_heads / n_kv;
  const dim3 g(S, n_kv), b(512);
#define HH_PQK(HDV, KV)                                                                                          \
  hipLaunchKernelGGL((k_prefill_qk<HDV, KV>), g, b, 0, s, QKV, n_in, n_heads, n_kv, q_norm, k_norm, eps, rope, \
                     rope_dim, max_seq, pos0, gated, k_cache, v_cache, QB)
  if (hd == 128 && G + 1 <= 512 / 32) {
    if (kv_q8) HH_PQK(128, true); else HH_PQK(128, false);
  } else if (hd == 256 && G + 1 <= 512 / 64) {
    if (kv_q8) HH_PQK(256, true); else HH_PQK(256, false);
  } else {
    return 1;
  }
#undef HH_PQK
  return ok();
}

// Attention for tokens [t0, t0 + n) of a prefill; PO/PML hold n tokens'
// partials at a stride of n_chunks narrow chunks.  Each token uses the chunk
// width the decode step uses at its sequence length (attn_chunk_for): the
// tokens below the width's threshold and those past it go as two passes.
int hh_prefill_attn_launch(int hd, const float* QB, const float* k_cache, const float* v_cache, int n_heads, int n_kv,
                           int max_seq, int pos0, int t0, int n, int n_chunks, float* PO, float* PML,
                           const float* gate, int gate_row, int kv_q8, int8_t* yq, float* yd, float* yf,
                           hipStream_t s) {
  // tokens per split pass: 4 at head_dim 128, 1 at 256 (measured on the 8B and
  // 9B/27B shapes; more tokens per pass cost occupancy at 256)
  const int NTOK = hd == 128 ? 4 : 1;
  const int G = n_heads / n_kv, TT = 16;
  if (G > 8 || n_kv * G != n_heads || (hd != 128 && hd != 256)) return 1;
  const int cn = 8192 / hd;
  // token t (sequence length pos0 + t + 1) takes the wide chunk past seq_wide
  const int seq_wide = cn * (256 / n_kv);
  const int tw = std::min(t0 + n, std::max(t0, seq_wide - pos0));
  auto pass = [&](int ta, int na, int C) -> int {
    if (na <= 0) return 0;
    // the grid's chunk count: the caller's stride for the narrow pass (its XCD
    // spread), for the wide one the chunks it reaches rounded up to 3 mod 8 the
    // same way; workgroups past a token tile's last chunk exit
    int nc = n_chunks;
    if (C != cn) {
      nc = (pos0 + ta + na + C - 1) / C;
      nc += (3 - nc % 8 + 8) % 8;
    }
    const size_t split_lds = 4 * (NTOK * ((size_t)G * C + 2 * G + (ATTN_NT / 64) * 4 * (size_t)hd) + 8);
    const size_t merge_lds = 4 * (4 * (size_t)n_chunks);
    dim3 g1(nc, n_kv, (na + TT - 1) / TT), g2((na * n_heads + 3) / 4);
#define HH_PSPLIT(HDV, KV, GM, GTV, CV)                                                                           \
  hipLaunchKernelGGL((k_attn_prefill_split<HDV, ATTN_NT, KV, GM, HDV == 128 ? 4 : 1, GTV, CV>), g1, dim3(ATTN_NT), \
                     split_lds, s, QB, k_cache, v_cache, n_heads, n_kv, max_seq, pos0, ta + na, ta, TT, n_chunks, PO, \
                     PML)
    // group sizes 4 and 8 get exact trip counts (GT), others read G at run time
#define HH_PSPLIT_G(HDV, KV, CV)                                      \
  do {                                                                \
    if (G == 4) HH_PSPLIT(HDV, KV, 4, 4, CV);                         \
    else if (G < 4) HH_PSPLIT(HDV, KV, 4, 0, CV);                     \
    else if (G == 8) HH_PSPLIT(HDV, KV, 8, 8, CV);                    \
    else HH_PSPLIT(HDV, KV, 8, 0, CV);                                \
  } while (0)
#define HH_PSPLIT_C(HDV, KV)                                          \
  do {                                                                \
    if (C == 8192 / HDV) HH_PSPLIT_G(HDV, KV, 8192 / HDV);            \
    else HH_PSPLIT_G(HDV, KV, 16384 / HDV);                           \
  } while (0)
    if (hd == 128) {
      if (kv_q8) HH_PSPLIT_C(128, true); else HH_PSPLIT_C(128, false);
      hipLaunchKernelGGL(k_attn_prefill_merge<128>, g2, dim3(256), merge_lds, s, PO, PML, n_heads, n_kv, n_chunks, C,
                         pos0, ta, na, gate, gate_row, yq, yd, yf);
    } else {
      if (kv_q8) HH_PSPLIT_C(256, true); else HH_PSPLIT_C(256, false);
      hipLaunchKernelGGL(k_attn_prefill_merge<256>, g2, dim3(256), merge_lds, s, PO, PML, n_heads, n_kv, n_chunks, C,
                         pos0, ta, na, gate, gate_row, yq, yd, yf);
    }
#undef HH_PSPLIT_C
#undef HH_PSPLIT_G
#undef HH_PSPLIT
    return hipGetLastError() == hipSuccess ? 0 : 1;
  };
  if (pass(t0, tw - t0, cn)) return 1;
  return pass(tw, t0 + n - tw, 2 * cn);
}

// The whole prompt's attention on fp32 MFMA (k_attn_prefill_mfma): tokens
// [t0, t0 + n) at positions pos0 + t0 ..; no partials.
int hh_prefill_attn_mfma_launch(int hd, const float* QB, const float* k_cache, const float* v_cache, int n_heads,
                                int n_kv, int max_seq, int pos0, int t0, int n, const float* gate, int gate_row,
                                int kv_q8, int8_t* yq, float* yd, float* yf, hipStream_t s) {
  const int G = n_heads / n_kv;
  if (G < 1 || G > 8 || n_kv * G != n_heads || n <= 0) return 1;
  const int T = G >= 8 ? 1 : 8 / G;
  dim3 grid(((n + 16 * T - 1) / (16 * T)) * n_kv), block(64 * G * T);
#define HH_PMFMA(HDV, KV) \
  hipLaunchKernelGGL((k_attn_prefill_mfma<HDV, KV>), grid, block, 0, s, QB, k_cache, v_cache, n_heads, n_kv, max_seq, \
                     pos0, t0, n, gate, gate_row, yq, yd, yf)
  if (hd == 128) {
    if (kv_q8) HH_PMFMA(128, true); else HH_PMFMA(128, false);
  } else if (hd == 256) {
    if (kv_q8) HH_PMFMA(256, true); else HH_PMFMA(256, false);
  } else {
    return 1;
  }
#undef HH_PMFMA
  return ok();
}


int hh_read_probe_launch(const void* p, int64_t nbytes, int* sink, hipStream_t s) {
  hipLaunchKernelGGL(k_read_probe, dim3(512), dim3(1024), 0, s, (const uint4*)p, nbytes / 16, sink, -1);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
