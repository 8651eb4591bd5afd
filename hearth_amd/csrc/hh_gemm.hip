// hh_gemm.hip — batched (prefill) quantized GEMM on int8 MFMA for gfx950.
//
// Semantics: out[s*n + r] = dot_fn(w + r*row_bytes, x + s*q8_stride, K) for
// every token s < seq_len and row r < n: par_dot_rows_batched with DotFn /
// DotFn2 (pool.rs:40-80, :568-618; matmul.rs:580-674), whose paired kernels
// are bit-identical to the single-token dot (q2_0.rs:936-986).  Here too:
// every 32-element sub-block dot is an exact int32 from
// v_mfma_i32_16x16x32_i8, and the fp32 combine follows the scalar kernels
// (q2_0.rs:537-574, q1_0g128.rs:1113-1152, q8_0.rs:154-171):
//   Q2/Q1: block_acc = (((0 + i0*da0) + i1*da1) + i2*da2) + i3*da3;
//          sum += block_acc * dw          (128-weight blocks, 4 sub-blocks)
//   Q8:    sum += ((float)i * dw) * da     (32-weight blocks)
// so each output equals the decode GEMV's bit for bit.
//
// Tiling: a 512-lane workgroup owns 128 tokens x TN rows (64 or 96); wave w
// owns tokens [16w, 16w+16) and all TN rows as TN/16 16x16 MFMA tiles.  Per
// 128-column step the workgroup stages the activation bytes and scales of its
// 128 tokens and the weight blocks of its TN rows in LDS, the weight codes widened to
// int8 (code - 1, or +-1 per sign bit) once as they are stored
// (double-buffered: the next step's global loads are issued before this
// step's MFMAs).  Activations come split (int8 rows + f32 block scales), so
// staging is plain 16-byte copies; the standard Q8_0 layout of the operator
// entry point is split by k_q8_split first.  Operand layouts (checked on the device): A lane l = row l%16,
// k = 8*(l/16) .. +8; B lane l = column l%16, same k; C lane l = column l%16,
// rows 4*(l/16) .. +4.
#include "hh_kernels.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int NTG = 512;       // lanes per workgroup (8 waves, two per SIMD)
constexpr int TM = 128;        // tokens per workgroup
// rows per workgroup: TN (a template argument) = 64, or 96 for the large-N
// launches of the non-Q8 formats (96 rows hold 6 MFMA tiles per wave within
// the 256 registers of two waves per SIMD; Q8_0 would spill)
constexpr int KS = 128;        // columns per step
// LDS bytes per token / weight row: 34 dwords (= 2 mod 32 banks), so the 16
// rows of an MFMA operand read (8 bytes per lane) fall on distinct bank pairs;
// rows are 8-byte aligned, so tile stores are 8 bytes wide.
constexpr int AROW = KS + 8;

// Activations arrive split: xq = int8 [seq][K], xd = f32 [seq][K/32] (the
// Q8_0 scale of each 32-block).  Per step a lane copies two 16-byte pieces of
// the 128 x 128 int8 tile and one scale; weight roles are wave-uniform.
template <int TN> struct Stage {
  int8_t a[TM * AROW];     // activations, int8
  int8_t w[TN * AROW];     // weights widened to int8 (code - 1, or +-1)
  float da[4 * TM];        // activation scale per (sub-block, token)
  float dw[TN * 4];        // weight scale per row (Q2/Q1: [0]; Q8: per sub-block)
  float nmd[TM];           // -GEMM_MAGIC * d_a of sub-block 0, per token
};

// Sub-block 0 of each block starts its MFMA from GEMM_MAGIC_BITS, so the int32
// result c = MAGIC_BITS + i reads as the float GEMM_MAGIC + i exactly (|i| <
// 2^22), and fma(c, d_a, -GEMM_MAGIC * d_a) is i * d_a exactly (both terms and
// the result fit f32's 24 bits): the block accumulator's first term, as
// fma((float)i, d_a, 0) gives it, without the int -> float convert.
constexpr float GEMM_MAGIC = 12582912.0f;   // 1.5 * 2^23
constexpr int GEMM_MAGIC_BITS = 0x4B400000;

// Q2_0 codes (8 per u16, LSB first) -> 8 int8 (code - 1): spread the four
// 2-bit fields of a byte to byte lanes, then (c + 0x7f) ^ 0x80 per lane.
HH_DEV uint32_t q2_spread4(uint32_t y) {
  uint32_t z = (y | (y << 6) | (y << 12) | (y << 18)) & 0x03030303u;
  return (z + 0x7f7f7f7fu) ^ 0x80808080u;
}
// Q1_0 sign bits (4 in y, LSB first) -> 4 int8 (+1 / -1): bit j to byte lane
// j, then (2b + 0x7f) ^ 0x80 per lane (0 -> 0xff, 1 -> 0x01, no carries).
HH_DEV uint32_t q1_spread4(uint32_t y) {
  uint32_t z = (y | (y << 7) | (y << 14) | (y << 21)) & 0x01010101u;
  return ((z << 1) + 0x7f7f7f7fu) ^ 0x80808080u;
}

// PTQ1_0 block (ptq1_0.rs:1-13) as 7 dwords: qs[24] (5 trits per byte; bytes
// 0..15 -> elements 16n + m, 16..23 -> 80 + 8n + (m-16)), then qh[2] (4 trits,
// elements 120 + 2n + h) and the f16 scale.  Trit n of byte b is
// ((b*3^n mod 256)*3) >> 8, walked on two 16-bit lanes per dword.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
HH_DEV uint32_t pt_step(u16x2& lo, u16x2& hi) {   // the next slot's trits of 4 bytes, as bytes
  const u16x2 three = {3, 3}, eight = {8, 8};
  const u16x2 ql = lo * three, qh = hi * three;
  const uint32_t t = __builtin_bit_cast(uint32_t, (u16x2)(ql >> eight)) |
                     (__builtin_bit_cast(uint32_t, (u16x2)(qh >> eight)) << 8);
  lo = __builtin_bit_cast(u16x2, __builtin_bit_cast(uint32_t, ql) & 0x00ff00ffu);
  hi = __builtin_bit_cast(u16x2, __builtin_bit_cast(uint32_t, qh) & 0x00ff00ffu);
  return t;
}
HH_DEV uint32_t trit_to_i8x4(uint32_t t) { return (t + 0x7f7f7f7fu) ^ 0x80808080u; }   // t - 1 per byte

template <int FMT> HH_DEV constexpr int w_code_units() {
  return FMT == FMT_Q2 ? 16 : FMT == FMT_Q1 ? 8 : FMT == FMT_PT ? 7 : 64;
}
template <int FMT> HH_DEV constexpr int w_block_bytes() { return FMT == FMT_Q1 ? 18 : FMT == FMT_PT ? 28 : 34; }
template <int FMT> HH_DEV constexpr int w_scale_off() { return FMT == FMT_PT ? 26 : 0; }
template <int FMT, int TN> HH_DEV constexpr int w_regs() { return (TN * w_code_units<FMT>() + NTG - 1) / NTG; }
template <int FMT> HH_DEV constexpr int w_scales() { return FMT == FMT_Q8 ? 4 : 1; }   // per row per step

template <int FMT, int TN> struct Regs {
  uint4 a[2];
  float ad;
  uint32_t w[w_regs<FMT, TN>()];
  uint32_t ws;
};

template <int FMT, int TN>
HH_DEV void stage_load(Regs<FMT, TN>& R, const uint8_t* __restrict__ w, const int8_t* __restrict__ xq,
                       const float* __restrict__ xd, int n, int seq, int K, int r0, int s0, int kb) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = tid + NTG * i, t = idx >> 3, piece = idx & 7;
    const int sidx = min(s0 + t, seq - 1);
    R.a[i] = *(const uint4*)(xq + (size_t)sidx * K + (size_t)kb * KS + 16 * piece);
  }
  {
    const int t = tid >> 2, sub = tid & 3;
    const int sidx = min(s0 + t, seq - 1);
    R.ad = xd[(size_t)sidx * (K / 32) + kb * 4 + sub];
  }
  constexpr int CU = w_code_units<FMT>();
  const size_t row_bytes = (size_t)K / (FMT == FMT_Q8 ? 32 : 128) * w_block_bytes<FMT>();
  const size_t step_bytes = FMT == FMT_Q8 ? 136 : w_block_bytes<FMT>();
#pragma unroll
  for (int i = 0; i < w_regs<FMT, TN>(); ++i) {
    const int idx = min(tid + NTG * i, TN * CU - 1);
    const int rr = idx / CU, u = idx % CU, r = min(r0 + rr, n - 1);
    const uint8_t* base = w + (size_t)r * row_bytes + (size_t)kb * step_bytes;
    if constexpr (FMT == FMT_Q8) R.w[i] = *(const uint16_t*)(base + (u / 16) * 34 + 2 + 2 * (u % 16));
    else if constexpr (FMT == FMT_PT) R.w[i] = *(const uint32_t*)(base + 4 * u);
    else R.w[i] = *(const uint16_t*)(base + 2 + 2 * u);
  }
  if (tid < TN * w_scales<FMT>()) {   // waves 0 (Q2/Q1) or 0-3 (Q8): uniform
    const int rr = tid / w_scales<FMT>(), b = tid % w_scales<FMT>(), r = min(r0 + rr, n - 1);
    R.ws = *(const uint16_t*)(w + (size_t)r * row_bytes + (size_t)kb * step_bytes + 34 * b + w_scale_off<FMT>());
  }
}

template <int FMT, int TN>
HH_DEV void stage_store(Stage<TN>& st, const Regs<FMT, TN>& R) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int idx = tid + NTG * i, t = idx >> 3, piece = idx & 7;
    uint2* dst = (uint2*)(st.a + t * AROW + 16 * piece);
    dst[0] = make_uint2(R.a[i].x, R.a[i].y);
    dst[1] = make_uint2(R.a[i].z, R.a[i].w);
  }
  st.da[(tid & 3) * TM + (tid >> 2)] = R.ad;        // loaded as (t = tid / 4, sub = tid % 4)
  if ((tid & 3) == 0) st.nmd[tid >> 2] = -GEMM_MAGIC * R.ad;
  constexpr int CU = w_code_units<FMT>();
#pragma unroll
  for (int i = 0; i < w_regs<FMT, TN>(); ++i) {
    const int idx = tid + NTG * i;
    if (idx < TN * CU) {   // TN = 64: Q2 1024, Q1 512, Q8 4096, PTQ1_0 448 (lanes 448.. idle)
      const int rr = idx / CU, u = idx % CU;
      const uint32_t v = R.w[i];
      if constexpr (FMT == FMT_Q2) {
        *(uint2*)(st.w + rr * AROW + 8 * u) = make_uint2(q2_spread4(v & 0xffu), q2_spread4(v >> 8));
      } else if constexpr (FMT == FMT_PT) {
        int8_t* wr = st.w + rr * AROW;
        if (u < 6) {   // qs dword: stage A (u < 4) or stage B
          u16x2 lo = __builtin_bit_cast(u16x2, v & 0x00ff00ffu), hi = __builtin_bit_cast(u16x2, (v >> 8) & 0x00ff00ffu);
#pragma unroll
          for (int n = 0; n < 5; ++n) {
            const int e = u < 4 ? 16 * n + 4 * u : 80 + 8 * n + 4 * (u - 4);
            *(uint32_t*)(wr + e) = trit_to_i8x4(pt_step(lo, hi));
          }
        } else {       // qh bytes 24, 25 -> elements 120 + 2n + h
          u16x2 p = __builtin_bit_cast(u16x2, (v & 0xffu) | ((v << 8) & 0x00ff0000u));
          const u16x2 three = {3, 3}, eight = {8, 8};
          uint32_t t[4];
#pragma unroll
          for (int n = 0; n < 4; ++n) {
            const u16x2 q = p * three;
            t[n] = __builtin_bit_cast(uint32_t, (u16x2)(q >> eight));
            p = __builtin_bit_cast(u16x2, __builtin_bit_cast(uint32_t, q) & 0x00ff00ffu);
          }
          *(uint32_t*)(wr + 120) = trit_to_i8x4(__builtin_amdgcn_perm(t[1], t[0], 0x06040200u));
          *(uint32_t*)(wr + 124) = trit_to_i8x4(__builtin_amdgcn_perm(t[3], t[2], 0x06040200u));
        }
      } else if constexpr (FMT == FMT_Q1) {
        uint2* dst = (uint2*)(st.w + rr * AROW + 16 * u);
        dst[0] = make_uint2(q1_spread4(v & 0xfu), q1_spread4((v >> 4) & 0xfu));
        dst[1] = make_uint2(q1_spread4((v >> 8) & 0xfu), q1_spread4((v >> 12) & 0xfu));
      } else {
        *(uint16_t*)(st.w + rr * AROW + 32 * (u / 16) + 2 * (u % 16)) = (uint16_t)v;
      }
    }
  }
  if (tid < TN * w_scales<FMT>()) {
    const int rr = tid / w_scales<FMT>(), b = tid % w_scales<FMT>();
    st.dw[rr * 4 + b] = h2f(R.ws);
  }
}

template <int FMT, int TN>
__global__ __launch_bounds__(NTG) void k_gemm(const uint8_t* __restrict__ w, const int8_t* __restrict__ xq,
                                              const float* __restrict__ xd, float* __restrict__ out, int n, int K,
                                              int seq) {
#pragma clang fp contract(off)
  __shared__ Stage<TN> st[2];
  constexpr int NTT = TN / 16;   // MFMA tiles per wave
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int r0 = blockIdx.x * TN, s0 = blockIdx.y * TM;
  const int nsteps = K / KS;
  float sum[NTT][4], bacc[NTT][4];
#pragma unroll
  for (int t = 0; t < NTT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) { sum[t][r] = 0.0f; bacc[t][r] = 0.0f; }

  // Two register sets: at the end of step kb, step kb + 1 (loaded two steps
  // earlier) is written to the free LDS buffer and the global loads of step
  // kb + 3 are issued into the register set just freed, so every load has two
  // steps' compute to land.
  Regs<FMT, TN> R0, R1;
  stage_load<FMT, TN>(R0, w, xq, xd, n, seq, K, r0, s0, 0);
  if (nsteps > 1) stage_load<FMT, TN>(R1, w, xq, xd, n, seq, K, r0, s0, 1);
  stage_store<FMT, TN>(st[0], R0);
  if (nsteps > 2) stage_load<FMT, TN>(R0, w, xq, xd, n, seq, K, r0, s0, 2);
  __syncthreads();
  const int arow = 16 * wid + (lane & 15);   // A operand token (within the tile)
  const int kg = 8 * (lane >> 4);            // k offset within a sub-block
  const int tok0 = 16 * wid + 4 * (lane >> 4);
  auto step = [&](int kb, Regs<FMT, TN>& Rn) {   // Rn holds step kb + 1
    const Stage<TN>& S = st[kb & 1];
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
      const long a = *(const long*)(S.a + arow * AROW + sub * 32 + kg);
      const float4 da4 = *(const float4*)(S.da + sub * TM + tok0);
      const float da[4] = {da4.x, da4.y, da4.z, da4.w};
      float nm[4] = {0.f, 0.f, 0.f, 0.f};
      if (FMT != FMT_Q8 && sub == 0) {
        const float4 n4 = *(const float4*)(S.nmd + tok0);
        nm[0] = n4.x; nm[1] = n4.y; nm[2] = n4.z; nm[3] = n4.w;
      }
#pragma unroll
      for (int t = 0; t < NTT; ++t) {
        const int col = 16 * t + (lane & 15);
        const long b = *(const long*)(S.w + col * AROW + sub * 32 + kg);
        if constexpr (FMT != FMT_Q8) {
          if (sub == 0) {   // compile-time after unrolling
            const v4i cm = {GEMM_MAGIC_BITS, GEMM_MAGIC_BITS, GEMM_MAGIC_BITS, GEMM_MAGIC_BITS};
            const v4i c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, cm, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) bacc[t][r] = fmaf(__int_as_float(c[r]), da[r], nm[r]);
            continue;
          }
        }
        v4i c = {0, 0, 0, 0};
        c = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
        if constexpr (FMT == FMT_Q8) {
          const float dw = S.dw[col * 4 + sub];
#pragma unroll
          for (int r = 0; r < 4; ++r) sum[t][r] += ((float)c[r] * dw) * da[r];
        } else {
          // exact product: |c| <= 32 * 128 * 2 = 2^13 and da is an f16 value
          // (<= 11 significant bits), so c * da fits f32's 24 bits and the
          // fma equals bacc + (float)c * da rounded once, as the scalar order
#pragma unroll
          for (int r = 0; r < 4; ++r) bacc[t][r] = fmaf((float)c[r], da[r], bacc[t][r]);
        }
      }
    }
    if constexpr (FMT != FMT_Q8) {
#pragma unroll
      for (int t = 0; t < NTT; ++t) {
        const float dw = S.dw[(16 * t + (lane & 15)) * 4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sum[t][r] += bacc[t][r] * dw;
          bacc[t][r] = 0.0f;
        }
      }
    }
    if (kb + 1 < nsteps) stage_store<FMT, TN>(st[(kb + 1) & 1], Rn);
    if (kb + 3 < nsteps) stage_load<FMT, TN>(Rn, w, xq, xd, n, seq, K, r0, s0, kb + 3);
    __syncthreads();
  };
  for (int kb = 0; kb < nsteps; kb += 2) {
    step(kb, R1);
    if (kb + 1 < nsteps) step(kb + 1, R0);
  }
#pragma unroll
  for (int t = 0; t < NTT; ++t) {
    const int r = r0 + 16 * t + (lane & 15);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int s = s0 + tok0 + q;
      if (r < n && s < seq) out[(size_t)s * n + r] = sum[t][q];
    }
  }
}

// Standard Q8_0 rows -> split layout (int8 [seq][K], f32 scales [seq][K/32]).
__global__ void k_q8_split(const uint8_t* __restrict__ x, int64_t nblocks, int8_t* __restrict__ xq,
                           float* __restrict__ xd) {
  const int64_t b = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  const int l = threadIdx.x & 31;
  if (b >= nblocks) return;
  const uint8_t* blk = x + b * 34;
  xq[b * 32 + l] = (int8_t)blk[2 + l];
  if (l == 0) xd[b] = h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
}

}  // namespace

int hh_gemm_launch(int fmt, const uint8_t* w, int n, int K, const int8_t* xq, const float* xd, int seq, float* out,
                   hipStream_t s) {
  if (K % KS != 0 || n <= 0 || seq <= 0) return 1;
  // 96-row tiles where they still give >= 1024 workgroups (8B / 27B FFN
  // gate+up: +6-7%); 64 otherwise (96 made the 27B down, N = 5120, 7% slower)
  const long tiles96 = (long)((n + 95) / 96) * ((seq + TM - 1) / TM);
  const bool wide = fmt != FMT_Q8 && tiles96 >= 1024;
  const int TNv = wide ? 96 : 64;
  dim3 grid((n + TNv - 1) / TNv, (seq + TM - 1) / TM);
#define HH_GEMM(F, T) hipLaunchKernelGGL((k_gemm<F, T>), grid, dim3(NTG), 0, s, w, xq, xd, out, n, K, seq)
  switch (fmt) {
    case FMT_Q2: if (wide) HH_GEMM(FMT_Q2, 96); else HH_GEMM(FMT_Q2, 64); break;
    case FMT_Q1: if (wide) HH_GEMM(FMT_Q1, 96); else HH_GEMM(FMT_Q1, 64); break;
    case FMT_Q8: HH_GEMM(FMT_Q8, 64); break;
    case FMT_PT: if (wide) HH_GEMM(FMT_PT, 96); else HH_GEMM(FMT_PT, 64); break;
    default: return 1;
  }
#undef HH_GEMM
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

int hh_q8_split_launch(const uint8_t* x, int64_t nblocks, int8_t* xq, float* xd, hipStream_t s) {
  if (nblocks <= 0) return 0;
  hipLaunchKernelGGL(k_q8_split, dim3((unsigned)((nblocks + 7) / 8)), dim3(256), 0, s, x, nblocks, xq, xd);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}
