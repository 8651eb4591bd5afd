// hh_gdn.hip — Gated-DeltaNet decode step for the qwen35 hybrids (gfx950).
//
// Restates qwen35.rs:1239-1492 (gdn_layer, no Hadamard fold):
//   conv window prepare/push + depthwise conv (k taps) + silu   :1294-1303, :1820-1829, :264-315
//   per-head L2 norm of q and k, 1/sqrt(sum x^2 + eps)          :1332-1347
//   g = softplus(alpha + dt_bias) * ssm_a ; beta = sigmoid(b)    :1359-1363, :1809-1815
//   alpha/beta = dense f32 [n_v x d] matvec of the normed input  :1285-1291, :1015-1025
//   per v-head h, k-group h % n_k:                               :1371-1404
//     dot_j = sum_i S[i][j] k[i]  (state before decay)
//     S[i][j] = S[i][j]*exp(g) + k[i] * beta*(v_j - dot_j)
//     o_j = sum_i S[i][j] q[i] / sqrt(hd)
//   gated RMSNorm: rms_norm(o_h, ssm_norm) * silu(z)             :1427-1439
// The fp32 state [n_v][hd][hd] stays resident in HBM; it is read and written
// once per token.
//
// Kernel 1 (prep): workgroups [0, conv_dim/256) do conv + silu (+ L2 norm for
//   the q/k channels, 2 heads of 128 per workgroup); then one workgroup per
//   v-head computes its alpha/beta from rms_norm(hidden, attn_norm).
// Kernel 2 (recurrence): one workgroup per v-head updates the head's state,
//   then applies the gated norm and writes the packed Q8_0 input of ssm_out.
#include "hh_kernels.h"

namespace {

HH_DEV float softplus_f(float x) { return x > 20.0f ? x : hx_log(1.0f + hx_exp(x)); }

// N wave sums at once, as a reduce-scatter with ascending offsets: at offset
// O a lane keeps one half of its values (the upper half where its offset bit
// is set) and adds the partner's copy; once one value is left the remaining
// offsets are a plain butterfly.  Each value's additions pair the same lane
// groups as wave_sum's, so lane l returns wave_sum of value
// k = sum_i bit_i(l) * N / 2^(i+1) (N = 8: 4 b0 + 2 b1 + b2).
template <int N, int O = 1> HH_DEV float rs_asc(float* v, int lane) {
  if constexpr (N > 1) {
    const bool up = (lane & O) != 0;
#pragma unroll
    for (int k = 0; k < N / 2; ++k) {
      const float send = up ? v[k] : v[k + N / 2];
      const float keep = up ? v[k + N / 2] : v[k];
      v[k] = keep + xor_lane<O>(send);
    }
    return rs_asc<N / 2, 2 * O>(v, lane);
  } else {
    float x = v[0];
    if constexpr (O <= 1) x += xor_lane<1>(x);
    if constexpr (O <= 2) x += xor_lane<2>(x);
    if constexpr (O <= 4) x += xor_lane<4>(x);
    if constexpr (O <= 8) x += xor_lane<8>(x);
    if constexpr (O <= 16) x += xor_lane<16>(x);
    if constexpr (O <= 32) x += xor_lane<32>(x);
    return x;
  }
}

// Token s = blockIdx.y of a batched prefill: conv + silu + L2 norm of every
// channel (g / beta per v-head: k_gdn_ab_rows).  The window's earlier inputs
// come from the projection rows of tokens s-1, s-2, ... and, before the first
// token, from conv buffer pos0 & 1, which k_gdn_conv_advance moves on
// afterwards.
__global__ __launch_bounds__(256) void k_gdn_prep_rows(GdnArgs a) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int kdim = a.n_k * a.hd, vdim = a.n_v * a.hd, conv_dim = 2 * kdim + vdim;
  const int s = blockIdx.y;
  __shared__ float red[16];
  const int ch = blockIdx.x * 256 + tid;
  const int K = a.kernel;
  float win[8];
  const float* cs = a.conv_state + (size_t)(a.pos0 & 1) * conv_dim * (K - 1) + (size_t)ch * (K - 1);
  for (int t = 0; t < K - 1; ++t) {
    const int u = s - (K - 1) + t;   // token of window slot t
    win[t] = u >= 0 ? a.proj[(size_t)u * a.row_in + ch] : cs[s + t];
  }
  win[K - 1] = a.proj[(size_t)s * a.row_in + ch];
  const float* w = a.conv_w + (size_t)ch * K;
  float acc = 0.0f;
  for (int t = 0; t < K; ++t) acc += w[t] * win[t];
  float y = acc / (1.0f + hx_exp(-acc));             // silu
  if (ch < 2 * kdim) {
    // L2 norm over the 128-channel head this lane belongs to (2 waves per head)
    float ss = wave_sum(y * y);
    if (lane == 0) red[wid] = ss;
    __syncthreads();
    int hw = wid & ~1;
    float tot = red[hw] + red[hw + 1];
    float inv = 1.0f / sqrtf(tot + a.eps);
    a.qk[(size_t)s * 2 * kdim + ch] = y * inv;
  } else {
    a.vconv[(size_t)s * vdim + ch - 2 * kdim] = y;
  }
}

// rs_asc's value index of lane l: k = sum_i bit_i(l) * N / 2^(i+1)
template <int N> HH_DEV int rs_asc_index(int lane) {
  int k = 0;
#pragma unroll
  for (int i = 0, w = N / 2; w >= 1; ++i, w >>= 1) k += ((lane >> i) & 1) * w;
  return k;
}

// alpha/beta of v-head h = blockIdx.x for tokens 4 blockIdx.y .. +3
// (matvec_dense :1015-1025 on rms_norm(hidden, attn_norm)).  Lane t holds the
// float4s at 4(t + 256j) + 4096c (the block_sumsq_f4 slots) of each token's
// hidden row, attn_norm and both weight rows; the weight rows and attn_norm
// are read once for the four tokens.  Order (the input projection's, k_gemv's
// alpha/beta epilogue): slot t + 256j sums its products over c, then element,
// ascending; the 64 slots of each (wave, j) by butterfly into W[wave + 4j];
// tree16(W).  The butterflies of all four tokens run as one reduce-scatter
// per phase (rs_asc: the same pairs as wave_sum's), so each phase has one
// barrier.
template <int NC>   // float4 columns per slot: d <= 4096 NC
__global__ __launch_bounds__(256) void k_gdn_ab_rows(GdnArgs a) {
  constexpr int TB = 4;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int h = blockIdx.x, s0 = blockIdx.y * TB, d = a.d, S = a.S;
  const float* wa = a.w_alpha + (size_t)h * d;
  const float* wb = a.w_beta + (size_t)h * d;
  __shared__ float red_s[TB][16], red_a[TB][16], red_b[TB][16];
  float4 hx[TB][4][NC], hw[4][NC], va[4][NC], vb[4][NC];
#pragma unroll
  for (int u = 0; u < TB; ++u) {
    const size_t su = (size_t)min(s0 + u, S - 1);
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 4 * (tid + 256 * j) + 4096 * c;
        hx[u][j][c] = e < d ? *(const float4*)(a.hidden + su * d + e) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
  }
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * (tid + 256 * j) + 4096 * c;
      hw[j][c] = va[j][c] = vb[j][c] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (e < d) {
        hw[j][c] = *(const float4*)(a.attn_norm + e);
        va[j][c] = *(const float4*)(wa + e);
        vb[j][c] = *(const float4*)(wb + e);
      }
    }
  // sums of squares in block_sumsq_f4's order, value u*4 + j
  float ss[TB * 4];
#pragma unroll
  for (int u = 0; u < TB; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float q = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c)
        if (4 * (tid + 256 * j) + 4096 * c < d)
          q += hx[u][j][c].x * hx[u][j][c].x + hx[u][j][c].y * hx[u][j][c].y + hx[u][j][c].z * hx[u][j][c].z +
               hx[u][j][c].w * hx[u][j][c].w;
      ss[u * 4 + j] = q;
    }
  {
    const float x = rs_asc<TB * 4>(ss, lane);
    if (lane < TB * 4) {
      const int k = rs_asc_index<TB * 4>(lane);
      red_s[k / 4][wid + 4 * (k % 4)] = x;
    }
  }
  __syncthreads();
  // alpha / beta slot sums, value u*8 + j (alpha) and u*8 + 4 + j (beta)
  float v[TB * 8];
#pragma unroll
  for (int u = 0; u < TB; ++u) {
    const float inv = 1.0f / sqrtf(tree16(red_s[u]) / (float)d + a.eps);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float sa = 0.0f, sb = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (4 * (tid + 256 * j) + 4096 * c >= d) continue;
        const float x[4] = {hx[u][j][c].x * inv * hw[j][c].x, hx[u][j][c].y * inv * hw[j][c].y,
                            hx[u][j][c].z * inv * hw[j][c].z, hx[u][j][c].w * inv * hw[j][c].w};
        const float ua[4] = {va[j][c].x, va[j][c].y, va[j][c].z, va[j][c].w};
        const float ub[4] = {vb[j][c].x, vb[j][c].y, vb[j][c].z, vb[j][c].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sa = sa + ua[i] * x[i];
          sb = sb + ub[i] * x[i];
        }
      }
      v[u * 8 + j] = sa;
      v[u * 8 + 4 + j] = sb;
    }
  }
  {
    const float x = rs_asc<TB * 8>(v, lane);
    if (lane < TB * 8) {
      const int k = rs_asc_index<TB * 8>(lane), u = k / 8, r = k % 8;
      if (r < 4) red_a[u][wid + 4 * r] = x;
      else red_b[u][wid + 4 * (r - 4)] = x;
    }
  }
  __syncthreads();
  if (tid < TB && s0 + tid < S) {
    const int s = s0 + tid;
    const float A = tree16(red_a[tid]);
    const float B = tree16(red_b[tid]);
    const float gg = softplus_f(A + a.dt_bias[h]) * a.ssm_a[h];
    a.ab[(size_t)s * 2 * a.n_v + h] = gg;
    a.ab[(size_t)s * 2 * a.n_v + a.n_v + h] = 1.0f / (1.0f + hx_exp(-B));
    // the decay once per (token, head) rather than in each of the 512 recurrence lanes
    a.dec_rows[(size_t)s * a.n_v + h] = hx_exp(gg);
  }
}

// The decode step of one GDN layer: one 1024-lane workgroup per v-head h.
// Lanes 0..383 first run the causal conv + silu of the head's channels (the
// q and k channels of its k-group, then its own v channels; window from conv
// buffer pos & 1, the shifted window written to buffer (pos + 1) & 1 by the
// channel's owner: k-group channels by head h < n_k, v channels by h) and the
// L2 norms of q and k (two wave sums per 128-channel head, as k_gdn_prep_rows).
// g and beta come from the input projection's raw alpha / beta dots.  Then
// lane = (column slice jb, row chunk ic, column jj): column j = 32 jb + jj,
// rows 16 ic .. 16 ic + 15.  The column dots sum the 8 row-chunk partials in
// chunk order.  The gated norm of the head's 128 outputs runs in wave 0 from LDS.
template <int KT>   // the conv kernel length, or 0: read at run time (<= 8)
__global__ __launch_bounds__(1024) void k_gdn_step(GdnArgs a) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  constexpr int hd = 128;
  constexpr int KM = KT > 0 ? KT : 8;
  const int h = blockIdx.x;
  const int jj = tid & 31, ic = (tid >> 5) & 7, jb = tid >> 8;
  const int j = jb * 32 + jj;
  const int kg = h % a.n_k;
  const int kdim = a.n_k * hd, conv_dim = 2 * kdim + a.n_v * hd, K = KT > 0 ? KT : a.kernel;
  float* S = a.state + (size_t)h * hd * hd;
  __shared__ float part[4][8][33];
  __shared__ float kv_s[2][hd];
  __shared__ float v_s[hd];
  __shared__ float o_s[hd];
  __shared__ float red[4];
  // 1. the small loads first, unconditional (lanes 384.. read channel 0's
  // window; the tail's gate and norm weight are read by every wave): vector
  // loads return in issue order, and a load under a branch leaves the
  // compiler no exact count of loads in flight, so either would make the
  // conv chain wait for the state stream below.
  const bool conv_lane = tid < 3 * hd;
  const int ct = conv_lane ? tid : 0;
  const int ch = ct < hd ? kg * hd + ct : ct < 2 * hd ? kdim + kg * hd + (ct - hd) : 2 * kdim + h * hd + (ct - 2 * hd);
  // both conv buffers' windows: which one holds this step's is the step
  // position's parity, a load of its own that the addresses then need not wait for
  const size_t buf = (size_t)conv_dim * (K - 1);
  const float* cs0 = a.conv_state + (size_t)ch * (K - 1);
  const float* w = a.conv_w + (size_t)ch * K;
  float win0[KM], win1[KM], wc[KM];
#pragma unroll
  for (int t = 0; t < KM; ++t) {
    win0[t] = 0.0f;
    win1[t] = 0.0f;
    wc[t] = 0.0f;
    if (t < K - 1) {
      win0[t] = cs0[t];
      win1[t] = cs0[buf + t];
    }
  }
  const float xin = a.proj[ch];
#pragma unroll
  for (int t = 0; t < KM; ++t)
    if (t < K) wc[t] = w[t];
  const float zg[2] = {a.z[(size_t)h * hd + lane], a.z[(size_t)h * hd + 64 + lane]};
  const float nw[2] = {a.ssm_norm[lane], a.ssm_norm[64 + lane]};
  const float alpha = a.ab_raw[h], braw = a.ab_raw[a.n_v + h], dtb = a.dt_bias[h], sa = a.ssm_a[h];
  __builtin_amdgcn_sched_barrier(0);
  // 2. the head's state, column j, rows 16 ic .. 16 ic + 15
  float sreg[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) sreg[r] = S[(size_t)(ic * 16 + r) * hd + j];
  float y = 0.0f;
  const int pos = a.st->pos;
  if (conv_lane) {   // conv + silu (qwen35.rs:1294-1303, :1820-1829)
    float win[KM];
#pragma unroll
    for (int t = 0; t < KM; ++t) win[t] = (t == K - 1) ? xin : (pos & 1) ? win1[t] : win0[t];
    if (tid >= 2 * hd || h < a.n_k) {
      float* cd = a.conv_state + (size_t)((pos + 1) & 1) * buf + (size_t)ch * (K - 1);
#pragma unroll
      for (int t = 0; t < KM - 1; ++t)
        if (t < K - 1) cd[t] = win[t + 1];
    }
    float acc = 0.0f;
#pragma unroll
    for (int t = 0; t < KM; ++t)
      if (t < K) acc += wc[t] * win[t];
    y = acc / (1.0f + hx_exp(-acc));
    if (tid < 2 * hd) {
      const float ss = wave_sum(y * y);
      if (lane == 0) red[wid] = ss;
    } else {
      v_s[tid - 2 * hd] = y;
    }
  }
  // g = softplus(alpha + dt_bias) * ssm_a, beta = sigmoid(b) (qwen35.rs:1359-1363)
  const float decay = hx_exp(softplus_f(alpha + dtb) * sa);
  const float b = 1.0f / (1.0f + hx_exp(-braw));
  __syncthreads();
  if (tid < 2 * hd) {   // L2 norm of the q (lanes 0..127) and k (128..255) heads
    const int hw = wid & ~1;
    const float inv = 1.0f / sqrtf((red[hw] + red[hw + 1]) + a.eps);
    kv_s[tid < hd ? 1 : 0][tid & (hd - 1)] = y * inv;
  }
  __syncthreads();
  const float vj = v_s[j];
  float dp = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) dp += sreg[r] * kv_s[0][ic * 16 + r];
  part[jb][ic][jj] = dp;
  __syncthreads();
  float dot = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) dot += part[jb][c][jj];
  const float bd = b * (vj - dot);
  float op = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float sn = sreg[r] * decay + kv_s[0][ic * 16 + r] * bd;
    S[(size_t)(ic * 16 + r) * hd + j] = sn;
    op += sn * kv_s[1][ic * 16 + r];
  }
  __syncthreads();
  part[jb][ic][jj] = op;
  __syncthreads();
  if (ic == 0) {
    float o = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) o += part[jb][c][jj];
    o_s[j] = o * (1.0f / sqrtf((float)hd));
  }
  __syncthreads();
  if (tid >= 64) return;
  // gated RMSNorm + Q8_0 of the head's outputs (qwen35.rs:1425-1439)
  const float v0 = o_s[lane], v1 = o_s[64 + lane];
  const float ss = wave_sum(v0 * v0 + v1 * v1);
  const float inv = 1.0f / sqrtf(ss / (float)hd + a.eps);
  const float vals[2] = {v0, v1};
  const int Kv = a.n_v * hd;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int dd = k * 64 + lane;
    const float nv = vals[k] * inv * nw[k];
    const float z = zg[k];
    const float o = nv * (z / (1.0f + hx_exp(-z)));
    if (a.out_f32) {   // folded model: ssm_out's prologue permutes, rotates and quantizes
      a.out_f32[h * hd + dd] = o;
      continue;
    }
    const float am = group_max<32>(fabsf(o));
    const float sc = q8_scale(am);
    const int q = q8_round_r(o, sc, q8_rcp(sc));
    const int qs = group_sum_i<32>(q);
    const int e = h * hd + dd;
    a.act_out[perm_pos(a.act_fmt, e)] = (uint8_t)(int8_t)q;
    if ((lane & 31) == 0) {
      ((float*)(a.act_out + Kv))[e >> 5] = h2f(f2h(sc));
      ((int*)(a.act_out + Kv + (Kv / 32) * 4))[e >> 5] = qs;
    }
  }
}

// Batched prefill: conv_state after S tokens holds the last K-1 inputs.
__global__ __launch_bounds__(256) void k_gdn_conv_advance(GdnArgs a) {
  const int kdim = a.n_k * a.hd, conv_dim = 2 * kdim + a.n_v * a.hd;
  const int ch = blockIdx.x * 256 + threadIdx.x;
  if (ch >= conv_dim) return;
  const int K = a.kernel, S = a.S;
  const size_t buf = (size_t)conv_dim * (K - 1);
  const float* cs = a.conv_state + (size_t)(a.pos0 & 1) * buf + (size_t)ch * (K - 1);
  float* cd = a.conv_state + (size_t)((a.pos0 + S) & 1) * buf + (size_t)ch * (K - 1);
  float nw[7];
  for (int t = 0; t < K - 1; ++t) {
    const int u = S - (K - 1) + t;
    nw[t] = u >= 0 ? a.proj[(size_t)u * a.row_in + ch] : cs[S + t];
  }
  for (int t = 0; t < K - 1; ++t) cd[t] = nw[t];
}

// Batched prefill recurrence.  A head's state columns evolve independently,
// so workgroup (h, jb) owns columns 32 jb .. 32 jb + 31 of head h, 8 per wave,
// and runs k_gdn_step's per-token arithmetic for tokens 0 .. S-1 in order with
// the state in registers: lane (column jj, row chunk ic) of a wave keeps rows
// 16 ic .. 16 ic + 15 of column j, its column's 8 chunks in 8 adjacent lanes.
// The column dots add the 8 chunk partials in chunk order, exactly as the
// decode kernel does through LDS, here with in-row lane shifts (no barrier per
// token).  o (before the gated norm) goes to o_rows[s][v_dim].  Inputs are
// staged per block of TB tokens: the next block's k/q, v, g and beta are
// loaded into registers while the current block runs.
constexpr int REC_TB = 8;
HH_DEV float sum8_in_order(float p) {   // lanes 8g: ((((0 + p0) + p1) + ...) + p7) of lanes 8g .. 8g+7
  float s = 0.0f;
  s += p;
  s += dpp_from_lane_plus<1>(p);
  s += dpp_from_lane_plus<2>(p);
  s += dpp_from_lane_plus<3>(p);
  s += dpp_from_lane_plus<4>(p);
  s += dpp_from_lane_plus<5>(p);
  s += dpp_from_lane_plus<6>(p);
  s += dpp_from_lane_plus<7>(p);
  return s;
}
HH_DEV float from_group_base8(float v) {   // every lane <- lane (lane & ~7)
  // quad broadcast of lane 4q, then banks 1 and 3 of each row (lanes 4-7,
  // 12-15) take lane - 4: two DPP moves, no LDS round trip
  const int q = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x00, 0xF, 0xF, false);
  return __int_as_float(__builtin_amdgcn_update_dpp(q, q, 0x114, 0xF, 0xA, false));
}
__global__ __launch_bounds__(256) void k_gdn_rec_rows(GdnArgs a) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  constexpr int hd = 128, TB = REC_TB;
  const int h = blockIdx.x >> 2, jb = blockIdx.x & 3;
  const int ic = lane & 7, jj = lane >> 3;
  const int j = jb * 32 + wid * 8 + jj;
  const int kg = h % a.n_k;
  const int kdim = a.n_k * hd, vdim = a.n_v * hd, S = a.S;
  float* St = a.state + (size_t)h * hd * hd;
  __shared__ float kvb[2][TB][2 * hd];   // per token: k[0..127], q[128..255]
  float sreg[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) sreg[r] = St[(size_t)(ic * 16 + r) * hd + j];
  // staging lane tid < 128 carries k[tid], lanes 128.. carry q[tid - 128]
  const float* kq0 = a.qk + (size_t)kg * hd + (tid & (hd - 1)) + (tid < hd ? kdim : 0);
  const float* v0 = a.vconv + (size_t)h * hd + j;
  float nkq[TB], nv[TB], ng[TB], nb[TB];
  auto load_block = [&](int blk) {
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      const size_t sl = (size_t)min(blk * TB + t, S - 1);   // unconditional loads
      nkq[t] = kq0[sl * 2 * kdim];
      nv[t] = v0[sl * vdim];
      ng[t] = a.dec_rows[sl * a.n_v + h];
      nb[t] = a.ab[sl * 2 * a.n_v + a.n_v + h];
    }
  };
  load_block(0);
  float cv[TB], cg[TB], cb[TB];
  const float inv_hd = 1.0f / sqrtf((float)hd);
  const int n_blk = (S + TB - 1) / TB;
  for (int blk = 0; blk < n_blk; ++blk) {
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      kvb[blk & 1][t][tid] = nkq[t];
      cv[t] = nv[t];
      cg[t] = ng[t];
      cb[t] = nb[t];
    }
    if (blk + 1 < n_blk) load_block(blk + 1);
    __syncthreads();   // the other buffer was last read a whole block ago
    // the block's outputs are stored after its tokens, so token t's output
    // chain can overlap token t + 1's dot chain
    const int nt = min(TB, S - blk * TB);
    float ob[TB], dec[TB];
#pragma unroll
    for (int t = 0; t < TB; ++t) dec[t] = cg[t];   // exp(g), from k_gdn_prep_rows
    // token t's k and q slices sit in registers, token t + 1's are read from
    // LDS while token t computes (the LDS round trip is off the state chain)
    float kc[16], qc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      kc[r] = kvb[blk & 1][0][ic * 16 + r];
      qc[r] = kvb[blk & 1][0][hd + ic * 16 + r];
    }
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      if (t >= nt) break;   // uniform
      float kn[16], qn[16];
      if (t + 1 < TB) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          kn[r] = kvb[blk & 1][t + 1][ic * 16 + r];
          qn[r] = kvb[blk & 1][t + 1][hd + ic * 16 + r];
        }
      }
      float dp = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) dp += sreg[r] * kc[r];
      const float dot = from_group_base8(sum8_in_order(dp));
      const float bd = cb[t] * (cv[t] - dot);
      float op = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sreg[r] = sreg[r] * dec[t] + kc[r] * bd;
        op += sreg[r] * qc[r];
      }
      ob[t] = sum8_in_order(op);
      if (t + 1 < TB) {
#pragma unroll
        for (int r = 0; r < 16; ++r) { kc[r] = kn[r]; qc[r] = qn[r]; }
      }
    }
    if (ic == 0) {
#pragma unroll
      for (int t = 0; t < TB; ++t)
        if (t < nt) a.o_rows[(size_t)(blk * TB + t) * vdim + (size_t)h * hd + j] = ob[t] * inv_hd;
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) St[(size_t)(ic * 16 + r) * hd + j] = sreg[r];
}

// Gated RMSNorm + Q8_0 of o_rows (k_gdn_step's tail per token and head), into
// the GEMM's split activation layout xq[S][v_dim], xd[S][v_dim/32].
// Workgroup (s, 4 heads), one wave per head.
__global__ __launch_bounds__(256) void k_gdn_gated_rows(GdnArgs a) {
  constexpr int hd = 128;
  const int lane = threadIdx.x & 63;
  const int s = blockIdx.y, h = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (h >= a.n_v) return;
  const int kdim = a.n_k * hd, vdim = a.n_v * hd;
  const float* o = a.o_rows + (size_t)s * vdim + (size_t)h * hd;
  const float* z = a.proj + (size_t)s * a.row_in + 2 * kdim + vdim + (size_t)h * hd;
  const float v0 = o[lane], v1 = o[64 + lane];
  const float ss = wave_sum(v0 * v0 + v1 * v1);
  const float inv = 1.0f / sqrtf(ss / (float)hd + a.eps);
  const float vals[2] = {v0, v1};
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int dd = k * 64 + lane;
    const float nv = vals[k] * inv * a.ssm_norm[dd];
    const float zz = z[dd];
    const float y = nv * (zz / (1.0f + hx_exp(-zz)));
    if (a.y_rows) {   // folded model: k_rot_q8_rows permutes, rotates and quantizes
      a.y_rows[(size_t)s * vdim + h * hd + dd] = y;
      continue;
    }
    const float am = group_max<32>(fabsf(y));
    const float sc = q8_scale(am);
    const int q = q8_round_r(y, sc, q8_rcp(sc));
    const int e = h * hd + dd;
    a.xq[(size_t)s * vdim + e] = (int8_t)q;
    if ((lane & 31) == 0) a.xd[(size_t)s * (vdim / 32) + (e >> 5)] = h2f(f2h(sc));
  }
}

}  // namespace

int hh_gdn_launch(const GdnArgs& a, hipStream_t s) {
  const int kdim = a.n_k * a.hd, vdim = a.n_v * a.hd, conv_dim = 2 * kdim + vdim;
  if (conv_dim % 256 || a.hd != 128 || a.kernel > 8) return 1;
  int n_conv_wg = conv_dim / 256;
  if (a.d % 1024 || a.d > 8192) return 1;
  if (!a.ab_raw || !a.st || a.n_v % a.n_k) return 1;
  (void)n_conv_wg;
  if (a.kernel == 4) hipLaunchKernelGGL(k_gdn_step<4>, dim3(a.n_v), dim3(1024), 0, s, a);
  else hipLaunchKernelGGL(k_gdn_step<0>, dim3(a.n_v), dim3(1024), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

// Batched prefill of one GDN layer over a.S tokens (the proj rows already hold
// the in_proj outputs): prep per token, conv window advance, recurrence,
// gated norm rows.
int hh_gdn_rows_launch(const GdnArgs& a, float* chunk_scratch, hipStream_t s) {
  const int kdim = a.n_k * a.hd, vdim = a.n_v * a.hd, conv_dim = 2 * kdim + vdim;
  if (conv_dim % 256 || a.hd != 128 || a.kernel > 8 || a.kernel < 2) return 1;
  if (a.d % 1024 || a.d > 8192 || a.S <= 0 || a.S > 65535) return 1;
  const int n_conv_wg = conv_dim / 256;
  hipLaunchKernelGGL(k_gdn_prep_rows, dim3(n_conv_wg, a.S), dim3(256), 0, s, a);
  if (hipGetLastError() != hipSuccess) return 1;
  const dim3 gab(a.n_v, (a.S + 3) / 4);
  if (a.d <= 4096) hipLaunchKernelGGL(k_gdn_ab_rows<1>, gab, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(k_gdn_ab_rows<2>, gab, dim3(256), 0, s, a);
  if (hipGetLastError() != hipSuccess) return 1;
  hipLaunchKernelGGL(k_gdn_conv_advance, dim3(n_conv_wg), dim3(256), 0, s, a);
  if (hipGetLastError() != hipSuccess) return 1;
  if (chunk_scratch) {   // chunked recurrence (hh_gdn_chunk.hip): fp32-rounding parity
    if (hh_gdn_chunked_rec_launch(a, chunk_scratch, s)) return 1;
  } else {
    hipLaunchKernelGGL(k_gdn_rec_rows, dim3(a.n_v * 4), dim3(256), 0, s, a);
    if (hipGetLastError() != hipSuccess) return 1;
  }
  hipLaunchKernelGGL(k_gdn_gated_rows, dim3((a.n_v + 3) / 4, a.S), dim3(256), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
