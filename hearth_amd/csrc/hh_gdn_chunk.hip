// hh_gdn_chunk.hip — chunked Gated-DeltaNet recurrence for the batched hybrid
// prefill (gfx950, fp32 MFMA).  An alternative to k_gdn_rec_rows, selected per
// model (HH_GDN_CHUNKED=1); the sequential kernel stays the default because it
// reproduces the token-by-token decode bit for bit.
//
// The reference's delta rule (qwen35.rs:1371-1404), per v-head and token t:
//   u_t = beta_t (v_t - S_{t-1}^T k_t)        (dot on the undecayed state)
//   S_t = a_t S_{t-1} + k_t u_t^T,  a_t = exp(g_t)
//   o_t = S_t^T q_t / sqrt(hd)
// For a chunk of C tokens starting from state S_0, with G_t = g_0 + ... + g_t
// (G_{-1} = 0):
//   S_t = e^{G_t} S_0 + sum_{s<=t} e^{G_t - G_s} k_s u_s^T
//   (I + A) U = B,  A[t][s] = beta_t e^{G_{t-1} - G_s} (k_t . k_s)  (s < t)
//                   B[t]    = beta_t (v_t - e^{G_{t-1}} S_0^T k_t)
//   o_t = (e^{G_t} S_0^T q_t + sum_{s<=t} e^{G_t - G_s} (q_t . k_s) u_s) / sqrt(hd)
//   S_C = e^{G_{C-1}} S_0 + sum_s e^{G_{C-1} - G_s} k_s u_s^T
// Every exponent is <= 0 (g = softplus(.) * ssm_a with ssm_a < 0 on trained
// and synthetic models), so no factor overflows.  The sums are regrouped, so
// the result matches the sequential rule to fp32 rounding, not bit for bit.
//
// Kernel 1 (k_gdn_chunk_prep, one workgroup per (chunk, head), independent):
//   G, T = (I + A)^-1 (16 x 16 diagonal blocks by forward substitution, the
//   off-diagonal blocks as T_ij = -T_ii sum_k A_ik T_kj), M[t][s] = e^{G_t - G_s} (q_t . k_s).
// Kernel 2 (k_gdn_chunk_scan, one workgroup per (head, 16 state columns),
//   chunks in order): K S, B, U = T B, outputs, state update, with the 16-column
//   state block in LDS and the next chunk's operands loading into registers.
//   The matrix products run on v_mfma_f32_16x16x4_f32.
// Measured (2048-token prompts, one MI355X): 9B hybrid prefill 110.0 -> 92.8 ms,
// 27B 319.4 -> 284.7 ms against the sequential recurrence.
#include "hh_kernels.h"

namespace {

constexpr int CH = 64;        // tokens per chunk
constexpr int HD = 128;       // head dim (k and v)
constexpr int CNT = 256;      // lanes per workgroup (4 waves)

typedef float f32x4 __attribute__((ext_vector_type(4)));

// One 16x16 output tile over K = 4 * nsteps: D += A(m, k) B(k, n), lane l
// supplies A(l % 16, 4 s + l / 16) and B(4 s + l / 16, l % 16); D[4 (l / 16) + r][l % 16]
// lands in acc[r].
template <typename FA, typename FB>
HH_DEV f32x4 mfma_tile(f32x4 acc, int nsteps, FA fa, FB fb) {
  const int l = threadIdx.x & 63, mi = l & 15, kk = l >> 4;
  for (int s = 0; s < nsteps; ++s) {
    const int k = 4 * s + kk;
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa(mi, k), fb(k, mi), acc, 0, 0, 0);
  }
  return acc;
}

// Per (chunk c = blockIdx.x, head h = blockIdx.y): T and M (CH x CH) and G (CH)
// into scratch [h][c][2 CH CH + CH].
__global__ __launch_bounds__(CNT) void k_gdn_chunk_prep(GdnArgs a, float* __restrict__ scr, int n_chunks) {
  // K and Q of the chunk; once the Gram tiles are in registers the same LDS
  // holds A (over K) and T (over Q)
  __shared__ float bufK[CH][HD + 1], bufQ[CH][HD + 1];
  __shared__ float Gs[CH], Bt[CH];
  __shared__ float Xs[4][16][17];
  float(*Am)[CH + 1] = (float(*)[CH + 1])&bufK[0][0];
  float(*Tm)[CH + 1] = (float(*)[CH + 1])&bufQ[0][0];
  const int tid = threadIdx.x, wid = tid >> 6, l = tid & 63;
  const int c = blockIdx.x, h = blockIdx.y;
  const int kg = h % a.n_k, kdim = a.n_k * HD, S = a.S;
  const int t0 = c * CH, n = min(CH, S - t0);
  for (int e = tid; e < CH * HD; e += CNT) {
    const int t = e / HD, i = e % HD;
    const bool in = t < n;
    const float* row = a.qk + (size_t)(t0 + (in ? t : 0)) * 2 * kdim + (size_t)kg * HD + i;
    bufQ[t][i] = in ? row[0] : 0.0f;
    bufK[t][i] = in ? row[kdim] : 0.0f;
  }
  if (tid < CH) {
    const bool in = tid < n;
    const size_t r = (size_t)(t0 + (in ? tid : 0)) * 2 * a.n_v;
    Gs[tid] = in ? a.ab[r + h] : 0.0f;          // g_t (padded tokens: no decay)
    Bt[tid] = in ? a.ab[r + a.n_v + h] : 0.0f;  // beta_t (padded tokens: no update)
  }
  __syncthreads();
  if (tid == 0) {   // inclusive prefix sum of g in token order
    float acc = 0.0f;
    for (int t = 0; t < CH; ++t) { acc += Gs[t]; Gs[t] = acc; }
  }
  // K K^T and Q K^T tiles (t-block tt >> 2, s-block tt & 3), 4 per wave, in registers
  f32x4 kk[4], qk[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int tt = wid * 4 + q, tb = (tt >> 2) * 16, sb = (tt & 3) * 16;
    kk[q] = (f32x4){0.f, 0.f, 0.f, 0.f};
    qk[q] = kk[q];
    if (sb <= tb) {
      kk[q] = mfma_tile(kk[q], HD / 4, [&](int m, int k) { return bufK[tb + m][k]; },
                        [&](int k, int nn) { return bufK[sb + nn][k]; });
      qk[q] = mfma_tile(qk[q], HD / 4, [&](int m, int k) { return bufQ[tb + m][k]; },
                        [&](int k, int nn) { return bufK[sb + nn][k]; });
    }
  }
  __syncthreads();   // K and Q are no longer read
  float* out = scr + ((size_t)h * n_chunks + c) * (2 * CH * CH + CH);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int tt = wid * 4 + q, tb = (tt >> 2) * 16, sb = (tt & 3) * 16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = tb + 4 * (l >> 4) + r, s = sb + (l & 15);
      const float gt1 = t > 0 ? Gs[t - 1] : 0.0f;
      Am[t][s] = s < t ? Bt[t] * hx_exp(gt1 - Gs[s]) * kk[q][r] : 0.0f;
      out[CH * CH + t * CH + s] = s <= t ? hx_exp(Gs[t] - Gs[s]) * qk[q][r] : 0.0f;   // M
    }
  }
  if (tid < CH) out[2 * CH * CH + tid] = Gs[tid];
  for (int e = tid; e < CH * CH; e += CNT) Tm[e / CH][e % CH] = 0.0f;
  __syncthreads();
  // T = (I + A)^-1 (unit lower triangular) by 16 x 16 blocks.  Diagonal block b
  // (wave b, lanes 0..15 = columns): T[t][s] = -sum_{r=s}^{t-1} A[t][r] T[r][s].
  {
    const int b0 = 16 * wid, sc = l & 15;
    float tc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) tc[r] = r == sc ? 1.0f : 0.0f;
#pragma unroll
    for (int t = 1; t < 16; ++t) {
      float p = 0.0f;
#pragma unroll
      for (int r = 0; r < t; ++r)
        if (r >= sc) p += Am[b0 + t][b0 + r] * tc[r];
      if (sc < t) tc[t] = -p;
    }
    if (l < 16) {
#pragma unroll
      for (int r = 0; r < 16; ++r) Tm[b0 + r][b0 + sc] = tc[r];
    }
  }
  __syncthreads();
  // off-diagonal blocks, block row i after block row i - 1:
  // T_ij = -T_ii (sum_{k=j}^{i-1} A_ik T_kj)
  for (int i = 1; i < 4; ++i) {
    const int j = wid;
    if (j < i) {
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      for (int k = j; k < i; ++k)
        x = mfma_tile(x, 4, [&](int m, int kk2) { return Am[16 * i + m][16 * k + kk2]; },
                      [&](int kk2, int nn) { return Tm[16 * k + kk2][16 * j + nn]; });
#pragma unroll
      for (int r = 0; r < 4; ++r) Xs[j][4 * (l >> 4) + r][l & 15] = x[r];
      f32x4 y = {0.f, 0.f, 0.f, 0.f};
      y = mfma_tile(y, 4, [&](int m, int kk2) { return Tm[16 * i + m][16 * i + kk2]; },
                    [&](int kk2, int nn) { return Xs[j][kk2][nn]; });
#pragma unroll
      for (int r = 0; r < 4; ++r) Tm[16 * i + 4 * (l >> 4) + r][16 * j + (l & 15)] = -y[r];
    }
    __syncthreads();
  }
  for (int e = tid; e < CH * CH; e += CNT) out[e] = Tm[e / CH][e % CH];
}

// Per (head h = blockIdx.x / (HD / NC), column block jb): the chunks in order,
// the NC-column state block in LDS.  Wave w owns token rows 16w .. 16w+15.
// The next chunk's K, Q, T, M and v are loaded into registers while the
// current chunk computes.
template <int NC>
__global__ __launch_bounds__(CNT) void k_gdn_chunk_scan(GdnArgs a, const float* __restrict__ scr, int n_chunks) {
  constexpr int NCT = NC / 16;                     // column tiles
  constexpr int PKQ = CH * HD / CNT;               // K (and Q) floats per lane
  constexpr int PTM = CH * CH / CNT;               // T (and M) floats per lane
  constexpr int PV = (CH * NC + CNT - 1) / CNT;    // v floats per lane
  extern __shared__ __align__(16) float sm[];
  float(*Ks)[HD + 1] = (float(*)[HD + 1])sm;
  float(*Qs)[HD + 1] = (float(*)[HD + 1])(sm + CH * (HD + 1));
  float(*Tm)[CH + 1] = (float(*)[CH + 1])(sm + 2 * CH * (HD + 1));
  float(*Mm)[CH + 1] = (float(*)[CH + 1])(sm + 2 * CH * (HD + 1) + CH * (CH + 1));
  float(*Sb)[NC + 1] = (float(*)[NC + 1])(sm + 2 * CH * (HD + 1) + 2 * CH * (CH + 1));   // HD x NC state
  float(*Ub)[NC + 1] = Sb + HD;                                 // CH x NC: B, then U
  float(*Vb)[NC + 1] = Ub + CH;                                 // CH x NC
  float* Gs = (float*)(Vb + CH);
  float* Bt = Gs + CH;
  float* Ws = Bt + CH;                                          // e^{G_last - G_s}
  const int tid = threadIdx.x, wid = tid >> 6, l = tid & 63;
  constexpr int WPH = HD / NC;
  const int h = blockIdx.x / WPH, j0 = (blockIdx.x % WPH) * NC;
  const int kg = h % a.n_k, kdim = a.n_k * HD, vdim = a.n_v * HD, S = a.S;
  float* St = a.state + (size_t)h * HD * HD;
  for (int e = tid; e < HD * NC; e += CNT) Sb[e / NC][e % NC] = St[(size_t)(e / NC) * HD + j0 + e % NC];
  const float inv_hd = 1.0f / sqrtf((float)HD);
  float rk[PKQ], rq[PKQ], rt[PTM], rm[PTM], rv[PV], rg = 0.0f, rb = 0.0f;
  auto fetch = [&](int c) {   // chunk c's operands into registers
    const int t0 = c * CH, n = min(CH, S - t0);
    const float* in = scr + ((size_t)h * n_chunks + c) * (2 * CH * CH + CH);
#pragma unroll
    for (int q = 0; q < PKQ; ++q) {
      const int e = tid + CNT * q, t = e / HD, i = e % HD;
      const float* row = a.qk + (size_t)(t0 + min(t, n - 1)) * 2 * kdim + (size_t)kg * HD + i;
      rq[q] = t < n ? row[0] : 0.0f;
      rk[q] = t < n ? row[kdim] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < PTM; ++q) {
      rt[q] = in[tid + CNT * q];
      rm[q] = in[CH * CH + tid + CNT * q];
    }
#pragma unroll
    for (int q = 0; q < PV; ++q) {
      const int e = tid + CNT * q, t = e / NC, j = e % NC;
      rv[q] = (e < CH * NC && t < n) ? a.vconv[(size_t)(t0 + t) * vdim + (size_t)h * HD + j0 + j] : 0.0f;
    }
    if (tid < CH) {
      rg = in[2 * CH * CH + tid];
      rb = tid < n ? a.ab[(size_t)(t0 + tid) * 2 * a.n_v + a.n_v + h] : 0.0f;
    }
  };
  fetch(0);
  for (int c = 0; c < n_chunks; ++c) {
    const int t0 = c * CH, n = min(CH, S - t0);
    __syncthreads();   // the previous chunk's readers are done
#pragma unroll
    for (int q = 0; q < PKQ; ++q) {
      const int e = tid + CNT * q;
      Ks[e / HD][e % HD] = rk[q];
      Qs[e / HD][e % HD] = rq[q];
    }
#pragma unroll
    for (int q = 0; q < PTM; ++q) {
      const int e = tid + CNT * q;
      Tm[e / CH][e % CH] = rt[q];
      Mm[e / CH][e % CH] = rm[q];
    }
#pragma unroll
    for (int q = 0; q < PV; ++q) {
      const int e = tid + CNT * q;
      if (e < CH * NC) Vb[e / NC][e % NC] = rv[q];
    }
    if (tid < CH) { Gs[tid] = rg; Bt[tid] = rb; }
    __syncthreads();
    if (c + 1 < n_chunks) fetch(c + 1);
    if (tid < CH) Ws[tid] = hx_exp(Gs[CH - 1] - Gs[tid]);
    const int tb = 16 * wid;
    f32x4 ks[NCT], qs[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      ks[ct] = (f32x4){0.f, 0.f, 0.f, 0.f};
      qs[ct] = ks[ct];
      ks[ct] = mfma_tile(ks[ct], HD / 4, [&](int m, int k) { return Ks[tb + m][k]; },
                         [&](int k, int nn) { return Sb[k][16 * ct + nn]; });
      qs[ct] = mfma_tile(qs[ct], HD / 4, [&](int m, int k) { return Qs[tb + m][k]; },
                         [&](int k, int nn) { return Sb[k][16 * ct + nn]; });
    }
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) {   // B[t] = beta_t (v_t - e^{G_{t-1}} (S_0^T k_t))
        const int t = tb + 4 * (l >> 4) + r, j = 16 * ct + (l & 15);
        const float gt1 = t > 0 ? Gs[t - 1] : 0.0f;
        Ub[t][j] = Bt[t] * (Vb[t][j] - hx_exp(gt1) * ks[ct][r]);
      }
    __syncthreads();
    f32x4 u[NCT];   // U = T B (rows of wave w need s < 16w + 16)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      u[ct] = (f32x4){0.f, 0.f, 0.f, 0.f};
      u[ct] = mfma_tile(u[ct], (tb + 16) / 4, [&](int m, int k) { return Tm[tb + m][k]; },
                        [&](int k, int nn) { return Ub[k][16 * ct + nn]; });
    }
    __syncthreads();   // every wave has read B
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) Ub[tb + 4 * (l >> 4) + r][16 * ct + (l & 15)] = u[ct][r];
    __syncthreads();
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {   // o_t = (e^{G_t} S_0^T q_t + sum_{s<=t} M[t][s] u_s) / sqrt(hd)
      f32x4 o = {0.f, 0.f, 0.f, 0.f};
      o = mfma_tile(o, (tb + 16) / 4, [&](int m, int k) { return Mm[tb + m][k]; },
                    [&](int k, int nn) { return Ub[k][16 * ct + nn]; });
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = tb + 4 * (l >> 4) + r, j = 16 * ct + (l & 15);
        if (t < n)
          a.o_rows[(size_t)(t0 + t) * vdim + (size_t)h * HD + j0 + j] = (hx_exp(Gs[t]) * qs[ct][r] + o[r]) * inv_hd;
      }
    }
    // S <- e^{G_last} S + sum_s e^{G_last - G_s} k_s u_s^T: key-row tiles 2w, 2w+1
    f32x4 sn[2][NCT];
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const int ib = 32 * wid + 16 * q;
        sn[q][ct] = (f32x4){0.f, 0.f, 0.f, 0.f};
        sn[q][ct] = mfma_tile(sn[q][ct], CH / 4, [&](int m, int k) { return Ks[k][ib + m] * Ws[k]; },
                              [&](int k, int nn) { return Ub[k][16 * ct + nn]; });
      }
    const float dl = hx_exp(Gs[CH - 1]);
    __syncthreads();   // every wave has read S
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 32 * wid + 16 * q + 4 * (l >> 4) + r, j = 16 * ct + (l & 15);
          Sb[i][j] = dl * Sb[i][j] + sn[q][ct][r];
        }
  }
  __syncthreads();
  for (int e = tid; e < HD * NC; e += CNT) St[(size_t)(e / NC) * HD + j0 + e % NC] = Sb[e / NC][e % NC];
}

}  // namespace

size_t hh_gdn_chunk_scratch_bytes(int n_v, int S) {
  const int n_chunks = (S + CH - 1) / CH;
  return sizeof(float) * (size_t)n_v * n_chunks * (2 * CH * CH + CH);
}

// The recurrence of hh_gdn_rows_launch in chunked form: a.qk, a.vconv, a.ab
// prepared per token; writes a.o_rows and advances a.state.
int hh_gdn_chunked_rec_launch(const GdnArgs& a, float* scratch, hipStream_t s) {
  if (a.hd != HD || a.S <= 0) return 1;
  const int n_chunks = (a.S + CH - 1) / CH;
  hipLaunchKernelGGL(k_gdn_chunk_prep, dim3(n_chunks, a.n_v), dim3(CNT), 0, s, a, scratch, n_chunks);
  if (hipGetLastError() != hipSuccess) return 1;
  // 16 state columns per scan workgroup (8 per head, 256 workgroups): measured
  // faster than 32 columns on the 9B and 27B prefills (92.8 / 96.3 ms)
  constexpr int NC = 16;
  const size_t lds =
      sizeof(float) * ((size_t)2 * CH * (HD + 1) + 2 * CH * (CH + 1) + (HD + 2 * CH) * (NC + 1) + 3 * CH);
  hipLaunchKernelGGL(k_gdn_chunk_scan<NC>, dim3(a.n_v * (HD / NC)), dim3(CNT), lds, s, a, scratch, n_chunks);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
