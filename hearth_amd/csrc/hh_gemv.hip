// hh_gemv.hip — quantized GEMV on packed Q8_0 activations for gfx950.
//
// Semantics: y[r] = dot_fn(w + r*row_bytes, x_q8, K), dot_fn one of
//   dot_q2_0_q8_0_ptr   (q2_0.rs:537-574 scalar semantics, :308-392 shipped arm)
//   dot_q1_0g128_q8_0_ptr (q1_0g128.rs:1113-1152)
//   dot_q8_0_q8_0_ptr   (q8_0.rs:154-171)
// over the rows par_dot_rows distributes across CPU workers (pool.rs:510-566).
// Each 32-element sub-block dot is an exact int32; the fp32 combination
// (sub-block * d_a, block * d_w) follows the scalar kernels, with the per-row
// sum split over units and added in a fixed order (deterministic run to run).
//
// Mapping: a workgroup (256 lanes) owns a row range; its units (2 blocks each)
// are taken by consecutive lanes, so each wave load instruction covers one
// contiguous 4352-byte (Q2/Q8) or 2304-byte (Q1) stretch of HBM.  Weight loads
// for the first batch are issued before the activation prologue and every
// later batch is double-buffered in VGPRs, so the prologue (RMSNorm + Q8_0
// quantization, or a copy) overlaps the first HBM round trip.
//
// Prologues:  PRO_PACKED  packed activation from global (written by a producer
//             PRO_RMSNORM rms_norm(x, w) then Q8_0 (ops.rs:442-487 rms_norm_q8
//                         semantics with ops.rs:8-35 operation order)
//             PRO_STDQ8   standard Q8_0 blocks (the DotFn activation format)
// Epilogues:  EPI_STORE   y[r] = sum
//             EPI_ADD     y[r] += sum (the residual adds of mod.rs:718-720, :776-778)
//             EPI_SILU    gate/up pair -> silu(g)*u -> packed Q8_0 (ops.rs:273-306)
//             EPI_LOGITS  logits, repetition penalty, greedy argmax (sampler lib.rs:26-40,
//                         :167-175; qwen35.rs:1735-1745), device step-state advance
#include "hh_kernels.h"

namespace {

enum { PRO_PACKED = 0, PRO_RMSNORM = 1, PRO_STDQ8 = 2, PRO_NORMROT = 3, PRO_F32ROT = 4, PRO_RMSNORM_ALL = 5 };
enum { EPI_STORE = 0, EPI_ADD = 1, EPI_SILU = 2, EPI_LOGITS = 3 };


HH_DEV int sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

// ---- unit dot products: w = unit dwords, aq/ad/as = the unit's activation ----
// Each returns the two per-block products p[blk] = block_acc * w_scale with the
// scalar kernels' exact fp32 operation order (separate multiply and add, no
// contraction): block_acc = (((0 + s0*d0) + s1*d1) + s2*d2) + s3*d3.  The row
// sum then adds the products in block order, so a row equals the scalar
// DotFn bit for bit.
// Q2: the activation chunk of 16 elements is staged as four nibble words
// [hi even | hi odd | lo even | lo odd]: a = 16 (a >> 4) + (a & 15) exactly, nibble n
// of an even (odd) word belongs to element 2n (2n + 1).  The 16 codes of a weight
// dword D (code m at bits 2m) then need only two masks: D & 0x33333333 holds the
// even codes as nibbles, (D >> 2) & 0x33333333 the odd ones, and
// sum code * a = 16 sdot8(codes, hi) + udot8(codes, lo).
constexpr uint32_t M4 = 0x33333333u;
constexpr uint32_t M8 = 0x11111111u;
HH_DEV void unit_q2(const uint32_t (&w)[17], const int8_t* aq, const float* ad, const int* as, float (&pr)[2]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    uint32_t c[8];
    float dw;
    if (blk == 0) {
      dw = h2f(w[0]);
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = __builtin_amdgcn_alignbit(w[i + 1], w[i], 16);
    } else {
      dw = h2f(w[8] >> 16);
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = w[9 + i];
    }
    float bacc = 0.0f;
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
      const i32x4* A = (const i32x4*)(aq + blk * 128 + sub * 32);
      i32x4 a0 = A[0], a1 = A[1];
      const uint32_t D0 = c[2 * sub], D1 = c[2 * sub + 1];
      const uint32_t e0 = D0 & M4, o0 = (D0 >> 2) & M4, e1 = D1 & M4, o1 = (D1 >> 2) & M4;
      int hi = 0;
      hi = __builtin_amdgcn_sdot8((int)e0, a0.x, hi, false);
      hi = __builtin_amdgcn_sdot8((int)o0, a0.y, hi, false);
      hi = __builtin_amdgcn_sdot8((int)e1, a1.x, hi, false);
      hi = __builtin_amdgcn_sdot8((int)o1, a1.y, hi, false);
      // the unsigned chain starts at -sum(a) (mod 2^32, exact once added to
      // 16 hi): sum (code-1)*a = sum code*a - sum a
      uint32_t lo = (uint32_t)(-as[blk * 4 + sub]);
      lo = __builtin_amdgcn_udot8(e0, (uint32_t)a0.z, lo, false);
      lo = __builtin_amdgcn_udot8(o0, (uint32_t)a0.w, lo, false);
      lo = __builtin_amdgcn_udot8(e1, (uint32_t)a1.z, lo, false);
      lo = __builtin_amdgcn_udot8(o1, (uint32_t)a1.w, lo, false);
      const int s = hi * 16 + (int)lo;
      // block_acc += dot * a_scale: |dot| < 2^13 and a_scale is an f16 value,
      // so the product is exact in f32 and the fma rounds once, as the
      // separate multiply and add do
      bacc = fmaf((float)s, ad[blk * 4 + sub], bacc);
    }
    pr[blk] = bacc * dw;                      // sum += block_acc * w_scale
  }
}

HH_DEV void unit_q1(const uint32_t (&w)[9], const int8_t* aq, const float* ad, const int* as, float (&pr)[2]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    uint32_t c[4];
    float dw;
    if (blk == 0) {
      dw = h2f(w[0]);
#pragma unroll
      for (int i = 0; i < 4; ++i) c[i] = __builtin_amdgcn_alignbit(w[i + 1], w[i], 16);
    } else {
      dw = h2f(w[4] >> 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) c[i] = w[5 + i];
    }
    float bacc = 0.0f;
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
      // activation chunk: hi words H0..H3, lo words L0..L3; nibble n of word k is
      // element 4n + k, as bit 4n + k of (D >> k) & 0x11111111
      const i32x4* A = (const i32x4*)(aq + blk * 128 + sub * 32);
      i32x4 a0 = A[0], a1 = A[1];
      const uint32_t D = c[sub];
      const uint32_t p0 = D & M8, p1 = (D >> 1) & M8, p2 = (D >> 2) & M8, p3 = (D >> 3) & M8;
      int hi = 0;
      hi = __builtin_amdgcn_sdot8((int)p0, a0.x, hi, false);
      hi = __builtin_amdgcn_sdot8((int)p1, a0.y, hi, false);
      hi = __builtin_amdgcn_sdot8((int)p2, a0.z, hi, false);
      hi = __builtin_amdgcn_sdot8((int)p3, a0.w, hi, false);
      uint32_t lo = 0;
      lo = __builtin_amdgcn_udot8(p0, (uint32_t)a1.x, lo, false);
      lo = __builtin_amdgcn_udot8(p1, (uint32_t)a1.y, lo, false);
      lo = __builtin_amdgcn_udot8(p2, (uint32_t)a1.z, lo, false);
      lo = __builtin_amdgcn_udot8(p3, (uint32_t)a1.w, lo, false);
      int s = hi * 16 + (int)lo;
      s = 2 * s - as[blk * 4 + sub];          // sum (+-1)*a = 2*sum bit*a - sum a
      bacc = fmaf((float)s, ad[blk * 4 + sub], bacc);   // exact product (|s| < 2^12), one rounding
    }
    pr[blk] = bacc * dw;
  }
}

HH_DEV void unit_q8(const uint32_t (&w)[17], const int8_t* aq, const float* ad, const int* /*as*/, float (&pr)[2]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    uint32_t c[8];
    float dw;
    if (blk == 0) {
      dw = h2f(w[0]);
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = __builtin_amdgcn_alignbit(w[i + 1], w[i], 16);
    } else {
      dw = h2f(w[8] >> 16);
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = w[9 + i];
    }
    const i32x4* A = (const i32x4*)(aq + blk * 32);
    i32x4 a0 = A[0], a1 = A[1];
    int s = 0;
    s = sdot4(c[0], a0.x, s); s = sdot4(c[1], a0.y, s); s = sdot4(c[2], a0.z, s); s = sdot4(c[3], a0.w, s);
    s = sdot4(c[4], a1.x, s); s = sdot4(c[5], a1.y, s); s = sdot4(c[6], a1.z, s); s = sdot4(c[7], a1.w, s);
    pr[blk] = (float)s * dw * ad[blk];        // sumf += sumi as f32 * d0 * d1
  }
}

// PTQ1_0 (ptq1_0.rs:1-13): a block is qs[24] at 5 trits per byte (bytes 0..15
// give elements 16n + m, bytes 16..23 elements 80 + 8n + (m-16)), qh[2] at 4
// trits per byte (elements 120 + 2n + h), then the f16 scale.  Trit n of byte b
// is ((b*3^n mod 256)*3) >> 8.  Every workgroup tabulates the 256 byte values
// once in LDS (pt_lut: trits 0..3 as int8 (trit - 1) in .x, trit 4 in .y's low
// byte); a qs dword then takes four table reads and a 4x4 byte transpose
// (v_perm) to give, per trit index n, the four bytes' (trit - 1) values in
// element order, ready for v_dot4 against the activations.
__shared__ uint2 pt_lut[256];

HH_DEV uint2 pt_lut_entry(uint32_t b) {
  uint32_t p = b, t[5];
#pragma unroll
  for (int n = 0; n < 5; ++n) {
    const uint32_t q = 3u * p;
    t[n] = q >> 8;
    p = q & 0xffu;
  }
  uint32_t x = 0;
#pragma unroll
  for (int n = 0; n < 4; ++n) x |= ((t[n] - 1u) & 0xffu) << (8 * n);
  return make_uint2(x, (t[4] - 1u) & 0xffu);
}

// The five slots of a qs dword: out[n] = byte n of each of the four bytes'
// table entries (byte m of out[n] from byte m of the dword).
HH_DEV void pt_slots(uint32_t q, uint32_t (&out)[5]) {
  const uint2 L0 = pt_lut[q & 0xffu], L1 = pt_lut[(q >> 8) & 0xffu], L2 = pt_lut[(q >> 16) & 0xffu],
              L3 = pt_lut[q >> 24];
  // perm(a, b, sel): selector 0..3 picks b's bytes, 4..7 a's
  const uint32_t p01l = __builtin_amdgcn_perm(L1.x, L0.x, 0x05010400u);   // [L0.b0, L1.b0, L0.b1, L1.b1]
  const uint32_t p01h = __builtin_amdgcn_perm(L1.x, L0.x, 0x07030602u);   // [L0.b2, L1.b2, L0.b3, L1.b3]
  const uint32_t p23l = __builtin_amdgcn_perm(L3.x, L2.x, 0x05010400u);
  const uint32_t p23h = __builtin_amdgcn_perm(L3.x, L2.x, 0x07030602u);
  out[0] = __builtin_amdgcn_perm(p23l, p01l, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(p23l, p01l, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(p23h, p01h, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(p23h, p01h, 0x07060302u);
  const uint32_t y01 = __builtin_amdgcn_perm(L1.y, L0.y, 0x0c0c0400u);   // [L0.y0, L1.y0, 0, 0]
  const uint32_t y23 = __builtin_amdgcn_perm(L3.y, L2.y, 0x04000c0cu);   // [0, 0, L2.y0, L3.y0]
  out[4] = y01 | y23;
}

// One PTQ1_0 block (dwords w[0..6]) against its 128 activations: per
// sub-block the int dot sum((trit - 1) * a), then the scalar kernel's fp32
// combine (ptq1_0.rs:587-599), as unit_q2.
HH_DEV float block_pt(const uint32_t* w, const int8_t* aq, const float* ad, const int* /*as*/) {
#pragma clang fp contract(off)
  const int* A = (const int*)aq;   // 32 activation dwords of the block
  int s[4] = {0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 4; ++j) {   // stage A: slot n -> elements 16n + 4j .. +3
    uint32_t sl[5];
    pt_slots(w[j], sl);
#pragma unroll
    for (int n = 0; n < 5; ++n) s[n >> 1] = sdot4(sl[n], (uint32_t)A[4 * n + j], s[n >> 1]);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {   // stage B: slot n -> elements 80 + 8n + 4j .. +3
    uint32_t sl[5];
    pt_slots(w[4 + j], sl);
#pragma unroll
    for (int n = 0; n < 5; ++n) {
      const int sub = n < 2 ? 2 : 3;
      s[sub] = sdot4(sl[n], (uint32_t)A[20 + 2 * n + j], s[sub]);
    }
  }
  {   // qh: bytes 24, 25 -> elements 120 + 2n + h
    const uint32_t W = w[6];
    const uint32_t Q0 = pt_lut[W & 0xffu].x, Q1 = pt_lut[(W >> 8) & 0xffu].x;
    s[3] = sdot4(__builtin_amdgcn_perm(Q1, Q0, 0x05010400u), (uint32_t)A[30], s[3]);   // n = 0, 1
    s[3] = sdot4(__builtin_amdgcn_perm(Q1, Q0, 0x07030602u), (uint32_t)A[31], s[3]);   // n = 2, 3
  }
  float bacc = 0.0f;
#pragma unroll
  for (int sub = 0; sub < 4; ++sub) bacc = fmaf((float)s[sub], ad[sub], bacc);   // exact product, one rounding
  return bacc * h2f(w[6] >> 16);
}

HH_DEV void unit_pt(const uint32_t (&w)[14], const int8_t* aq, const float* ad, const int* as, float (&pr)[2]) {
  pr[0] = block_pt(w, aq, ad, as);
  pr[1] = block_pt(w + 7, aq + 128, ad + 4, as + 4);
}

// Plain loads: on gfx950 the non-temporal variant of this stream measured
// ~4.0 TB/s against ~6.2 TB/s for ordinary loads of the same 68-byte units.
template <int FMT> HH_DEV void load_unit(uint32_t (&w)[UnitT<FMT>::DW], const uint8_t* p) {
  const u32x4_a4* v = (const u32x4_a4*)p;
  if constexpr (FMT == FMT_PT) {
    u32x4_a4 a = v[0], b = v[1], c = v[2];
    u32x2_a4 d = *(const u32x2_a4*)(p + 48);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    w[8] = c.x; w[9] = c.y; w[10] = c.z; w[11] = c.w;
    w[12] = d.x; w[13] = d.y;
  } else if constexpr (FMT == FMT_Q1) {
    u32x4_a4 a = v[0], b = v[1];
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    w[8] = *(const uint32_t*)(p + 32);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4_a4 a = v[i];
      w[4 * i] = a.x; w[4 * i + 1] = a.y; w[4 * i + 2] = a.z; w[4 * i + 3] = a.w;
    }
    w[16] = *(const uint32_t*)(p + 64);
  }
}

template <int FMT> HH_DEV void unit_dot(const uint32_t (&w)[UnitT<FMT>::DW], const int8_t* aq,
                                        const float* ad, const int* as, float (&pr)[2]) {
  if constexpr (FMT == FMT_Q2) unit_q2(w, aq, ad, as, pr);
  else if constexpr (FMT == FMT_Q1) unit_q1(w, aq, ad, as, pr);
  else if constexpr (FMT == FMT_PT) unit_pt(w, aq, ad, as, pr);
  else unit_q8(w, aq, ad, as, pr);
}

// ---------------------------------------------------------------------------
// Activation staging.  Each prologue has an issue half (global loads into
// registers) and a store half (registers -> LDS).  The issue half runs before
// any weight load: vector loads retire in order, so an activation load issued
// after the weight loads would wait for them.
//
// LDS layout: aq = int8 activations, unit t at t*qstride; ds = per unit
// [d_0 .. d_{SUBS-1}, s_0 .. s_{SUBS-1}] padded to DSS words (conflict-free
// 128-bit reads by consecutive units); part = block products transposed.
// ---------------------------------------------------------------------------
template <int FMT> HH_DEV constexpr int dss() { return FMT == FMT_Q8 ? 8 : 20; }

template <int FMT> HH_DEV void put_ds(float* ds, int blk32, float d, int s) {
  constexpr int SUBS = UnitT<FMT>::SUBS;
  int t = blk32 / SUBS, sub = blk32 - t * SUBS;
  ds[t * dss<FMT>() + sub] = d;
  ((int*)ds)[t * dss<FMT>() + SUBS + sub] = s;
}

// Stage the int8 activations of elements e .. e+3 (e % 4 == 0, bytes of w in
// element order) into the workgroup's LDS copy; lanes with in == false write
// nothing.  Q2: byte q = (e % 16) / 4 of each nibble word of the chunk
// (elements e, e+2 are the even pair, e+1, e+3 the odd pair).  Q1: lanes t and
// t ^ 1 hold elements e and e ^ 4 of one 32-element chunk (the whole wave
// calls this); after a lane swap the lane of e % 8 == 0 writes byte (e % 32) / 8
// of the four hi words, its partner that byte of the four lo words.  Other
// formats: one byte per element at lds_qpos.
template <int FMT> HH_DEV void put4(int8_t* aq, int e, uint32_t w, bool in) {
  if constexpr (FMT == FMT_Q1) {
    const uint32_t o = (uint32_t)bfly_xchg<1>((int)w);
    if (!in) return;
    const bool first = (e & 4) == 0;
    const uint32_t a = first ? w : o, b = first ? o : w;   // elements 8B + k, 8B + 4 + k
    uint8_t* ch = (uint8_t*)aq + (e >> 8) * 272 + (e & 224) + (first ? 0 : 16) + ((e & 31) >> 3);
    const int sh = first ? 4 : 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) ch[4 * k] = (uint8_t)(((a >> (8 * k + sh)) & 0x0Fu) | (((b >> (8 * k + sh)) & 0x0Fu) << 4));
    return;
  }
  if (!in) return;
  if constexpr (FMT == FMT_Q2) {
    uint8_t* ch = (uint8_t*)aq + (e >> 8) * 272 + (e & 240);
    const int q = (e & 15) >> 2;
    ch[q] = (uint8_t)(((w >> 4) & 0x0Fu) | ((w >> 16) & 0xF0u));        // hi even
    ch[4 + q] = (uint8_t)(((w >> 12) & 0x0Fu) | ((w >> 24) & 0xF0u));   // hi odd
    ch[8 + q] = (uint8_t)((w & 0x0Fu) | ((w >> 12) & 0xF0u));           // lo even
    ch[12 + q] = (uint8_t)(((w >> 8) & 0x0Fu) | ((w >> 20) & 0xF0u));   // lo odd
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) aq[lds_qpos(FMT, e + i)] = (int8_t)(w >> (8 * i));
  }
}

// A GEMV workgroup is NT = 1024 lanes (16 waves, one workgroup per CU at
// the decode shapes): the activation prologue is the same for every
// workgroup, so the fewer workgroups share a CU, the less of it each CU
// repeats, and 16 waves hide its instruction latencies.
constexpr int NT = 1024;

// The RMSNorm prologue runs in the first NORM_L lanes (waves 0-7).  When it
// reduces the sum of squares itself, that sum is complete before any wave
// issues a weight load: the activation read then meets an idle memory system
// instead of queueing behind the whole chip's weight stream (measured on the
// 8B gate+up: 13.3 -> 12.2 us).  When the producer handed over the sum's tree
// nodes (GemvArgs::sq_in) nothing is reduced and the weights go out at once.
// Eight staging waves rather than four: with the hand-off the quantization is
// the prologue's critical path (9B GDN in_proj 7.65 -> 6.75 us, 8B gate+up
// 10.3 -> 10.2 us).  The packed prologue (a plain copy) is staged by every
// lane and overlaps the weight loads.
constexpr int NORM_L = 512;
constexpr int PK_L = NT;

// PRO_RMSNORM: rms_norm(x, w) then Q8_0, in lanes t < NORM_L.  Slot s
// (s < 1024) owns the float4s at 4s + 4096c (c < NORM_CH); lane t runs slots
// t + NORM_L*j (j < NJ).  Sum of squares in the order of block_sumsq_f4:
// slot s sums its float4s in c order as ss + (((x0^2 + x1^2) + x2^2) + x3^2),
// slots 64w .. 64w+63 reduce by butterfly into W_w, the total is tree16(W).
// Words per row of the GEMV block-product buffer: 2P products rounded up to a
// multiple of 8, plus 4.
__host__ __device__ inline int gemv_part_stride(int P) { return ((2 * P + 7) & ~7) + 4; }

constexpr int NORM_CH = 2;   // K <= 8192
template <int NL> struct NormRegsT {
  static constexpr int NJ = 1024 / NL;
  float4 x[NJ][NORM_CH], w[NJ][NORM_CH];
  float4 sq;               // p.sq_in: tree nodes 4l .. 4l + 3 (lane l of the wave)
  float* nbuf = nullptr;   // non-null: the f32 normed vector is also kept here (LDS)
};

template <int NL> HH_DEV void norm_issue(const GemvArgs& p, NormRegsT<NL>& r) {
  constexpr int NJ = NormRegsT<NL>::NJ;
  const int tid = threadIdx.x;
  if (tid >= NL) return;
  if (p.sq_in) r.sq = *(const float4*)(p.sq_in + 4 * min(tid & 63, (p.K >> 6) - 1));   // K / 16 nodes
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int c = 0; c < NORM_CH; ++c) {
      const int e = (tid + NL * j) * 4 + 4096 * c;
      if (e < p.K) {
        r.x[j][c] = *(const float4*)(p.x + e);
        r.w[j][c] = *(const float4*)(p.norm_w + e);
      }
    }
}

template <int NL> HH_DEV void norm_partial(const GemvArgs& p, const NormRegsT<NL>& r, float* red) {
  constexpr int NJ = NormRegsT<NL>::NJ;
  const int tid = threadIdx.x;
  if (tid >= NL) return;
  float ss[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    ss[j] = 0.0f;
#pragma unroll
    for (int c = 0; c < NORM_CH; ++c)
      if ((tid + NL * j) * 4 + 4096 * c < p.K)
        ss[j] += r.x[j][c].x * r.x[j][c].x + r.x[j][c].y * r.x[j][c].y + r.x[j][c].z * r.x[j][c].z +
                 r.x[j][c].w * r.x[j][c].w;
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) ss[j] = wave_sum(ss[j]);
  if ((tid & 63) == 0) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) red[(tid >> 6) + (NL / 64) * j] = ss[j];
  }
}

// The sum of squares from the producer's tree nodes, in this wave alone: lane
// l adds nodes 4l .. 4l+3 pairwise, then the wave's butterfly.  Node b covers
// slots 4b .. 4b+3, so lane l's value is the tree node over slots 16l .. 16l+15
// and the butterfly completes the same pairwise tree over the 1024 slots that
// wave_sum + tree16 form (K <= 4096: one float4 per slot; nodes past K / 16
// are zero, as those slots are).
template <int NL> HH_DEV float norm_total_sq(const GemvArgs& p, const NormRegsT<NL>& r) {
  const bool has = 4 * (threadIdx.x & 63) < (p.K >> 4);
  const float v = has ? (r.sq.x + r.sq.y) + (r.sq.z + r.sq.w) : 0.0f;
  return wave_sum(v);
}

template <int FMT, int NL>
HH_DEV void norm_finish(const GemvArgs& p, const NormRegsT<NL>& r, int8_t* aq, float* ds, const float* red) {
  constexpr int NJ = NormRegsT<NL>::NJ;
  const int tid = threadIdx.x;
  if (tid >= NL) return;
  const int K = p.K;
  const float tot = p.sq_in ? norm_total_sq<NL>(p, r) : tree16(red);
  const float inv = 1.0f / sqrtf(tot / (float)K + p.eps);   // ops.rs:22-23
#pragma unroll
  for (int c = 0; c < NORM_CH; ++c) {
    if (c > 0 && 4096 * c >= K) break;   // uniform: whole chunk absent
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int e = (tid + NL * j) * 4 + 4096 * c;
      if (4096 * c + NL * j * 4 >= K) break;   // uniform
      const bool in = e < K;
      float vv[4] = {r.x[j][c].x * inv * r.w[j][c].x, r.x[j][c].y * inv * r.w[j][c].y,   // ops.rs:29 (x * inv) * w
                     r.x[j][c].z * inv * r.w[j][c].z, r.x[j][c].w * inv * r.w[j][c].w};
      if (r.nbuf && in) *(float4*)(r.nbuf + e) = make_float4(vv[0], vv[1], vv[2], vv[3]);
      float am = fmaxf(fmaxf(fabsf(vv[0]), fabsf(vv[1])), fmaxf(fabsf(vv[2]), fabsf(vv[3])));
      am = group_max<8>(am);
      const float sc = q8_scale(am), rc = q8_rcp(sc);
      int qs = 0;
      uint32_t word = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int q = q8_round_r(vv[i], sc, rc);
        qs += q;
        word |= ((uint32_t)q & 0xffu) << (8 * i);
      }
      qs = group_sum_i<8>(qs);
      put4<FMT>(aq, e, word, in);
      if (in && (tid & 7) == 0) put_ds<FMT>(ds, e >> 5, h2f(f2h(sc)), qs);
    }
  }
}

template <int FMT, int NL>
HH_DEV void norm_store(const GemvArgs& p, const NormRegsT<NL>& r, int8_t* aq, float* ds, float* red) {
  if (!p.sq_in) {   // uniform
    norm_partial<NL>(p, r, red);
    __syncthreads();
  }
  norm_finish<FMT, NL>(p, r, aq, ds, red);
}

// PRO_PACKED: packed activation [q K][d K/32][s K/32] from a producer kernel,
// staged by lanes t < PK_L.
constexpr int PK_Q = 32768 / 16 / PK_L;   // 16-byte chunks per lane: K <= 32768
constexpr int PK_D = 1024 / PK_L;
struct PackedRegs { i32x4 q[PK_Q]; float d[PK_D]; int s[PK_D]; };

HH_DEV void packed_issue(const GemvArgs& p, PackedRegs& r) {
  const int tid = threadIdx.x, K = p.K;
  if (tid >= PK_L) return;
#pragma unroll
  for (int i = 0; i < PK_Q; ++i) {
    int c = tid + PK_L * i;
    if (c < K / 16) r.q[i] = *(const i32x4*)(p.act + c * 16);
  }
#pragma unroll
  for (int i = 0; i < PK_D; ++i) {
    int b = tid + PK_L * i;
    if (b < K / 32) {
      r.d[i] = ((const float*)(p.act + K))[b];
      r.s[i] = ((const int*)(p.act + K + (K / 32) * 4))[b];
    }
  }
}

template <int FMT> HH_DEV void packed_store(const GemvArgs& p, const PackedRegs& r, int8_t* aq, float* ds) {
  const int tid = threadIdx.x, K = p.K;
  if (tid >= PK_L) return;
  constexpr int EL = UnitT<FMT>::EL;
#pragma unroll
  for (int i = 0; i < PK_Q; ++i) {
    int c = tid + PK_L * i;
    i32x4 v = r.q[i];
    if constexpr (FMT == FMT_Q1) {
      // a 32-element chunk is the 16-byte pieces of lanes t (dwords 0-3) and t ^ 1
      // (dwords 4-7); dword j holds elements j, j+8, j+16, j+24 (element 8i+j at byte
      // 4j+i).  Hi word k pairs dwords k and 4+k: the even lane writes the hi words,
      // the odd lane the lo words, each at its own 16 bytes.
      const uint32_t o0 = bfly_xchg<1>(v.x), o1 = bfly_xchg<1>(v.y), o2 = bfly_xchg<1>(v.z), o3 = bfly_xchg<1>(v.w);
      const bool first = (c & 1) == 0;
      const uint32_t m = 0x0F0F0F0Fu;
      const uint32_t lo_[4] = {first ? (uint32_t)v.x : o0, first ? (uint32_t)v.y : o1, first ? (uint32_t)v.z : o2,
                               first ? (uint32_t)v.w : o3};
      const uint32_t hi_[4] = {first ? o0 : (uint32_t)v.x, first ? o1 : (uint32_t)v.y, first ? o2 : (uint32_t)v.z,
                               first ? o3 : (uint32_t)v.w};
      uint32_t r4[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        r4[k] = first ? (((lo_[k] >> 4) & m) | (hi_[k] & ~m)) : ((lo_[k] & m) | ((hi_[k] << 4) & ~m));
      v.x = (int)r4[0]; v.y = (int)r4[1]; v.z = (int)r4[2]; v.w = (int)r4[3];
    }
    if (c < K / 16) {
      int e = c * 16;
      if constexpr (FMT == FMT_Q2) {
        // packed chunk: dword k holds elements k, k+4, k+8, k+12 (element 4i+k at byte
        // 4k+i), so byte j of the even words pairs dwords 0 and 2, of the odd words 1 and 3
        const uint32_t d0 = v.x, d1 = v.y, d2 = v.z, d3 = v.w, m = 0x0F0F0F0Fu;
        v.x = (int)(((d0 >> 4) & m) | (d2 & ~m));
        v.y = (int)(((d1 >> 4) & m) | (d3 & ~m));
        v.z = (int)((d0 & m) | ((d2 << 4) & ~m));
        v.w = (int)((d1 & m) | ((d3 << 4) & ~m));
      }
      *(i32x4*)(aq + (e / EL) * qstride<FMT>() + (e % EL)) = v;
    }
  }
#pragma unroll
  for (int i = 0; i < PK_D; ++i) {
    int b = tid + PK_L * i;
    if (b < K / 32) put_ds<FMT>(ds, b, r.d[i], r.s[i]);
  }
}

// PRO_STDQ8: standard Q8_0 blocks (DotFn activation format), K <= 20480.
constexpr int SQ_C = 5;
struct StdRegs { uint32_t q[SQ_C]; uint32_t d[SQ_C]; };

HH_DEV void std_issue(const GemvArgs& p, StdRegs& r) {
  const int tid = threadIdx.x, K = p.K;
#pragma unroll
  for (int c = 0; c < SQ_C; ++c) {
    int e = tid * 4 + c * 4 * NT;
    if (e < K) {
      const uint8_t* blk = p.act + (size_t)(e >> 5) * 34;
      const uint16_t* q16 = (const uint16_t*)(blk + 2 + (e & 31));
      r.q[c] = (uint32_t)q16[0] | ((uint32_t)q16[1] << 16);
      r.d[c] = *(const uint16_t*)blk;
    }
  }
}

template <int FMT> HH_DEV void std_store(const GemvArgs& p, const StdRegs& r, int8_t* aq, float* ds) {
  const int tid = threadIdx.x, K = p.K;
#pragma unroll
  for (int c = 0; c < SQ_C; ++c) {
    int e = tid * 4 + c * 4 * NT;
    if (c > 0 && c * 4 * NT >= K) break;   // uniform
    int qs = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) qs += (int)(int8_t)((r.q[c] >> (8 * i)) & 0xffu);
    qs = group_sum_i<8>(qs);
    put4<FMT>(aq, e, r.q[c], e < K);
    if (e < K && (tid & 7) == 0) put_ds<FMT>(ds, e >> 5, h2f(r.d[c]), qs);
  }
}

// PRO_NORMROT / PRO_F32ROT: the prologues of a Hadamard-folded matmul
// (qwen35.rs:914-941, `mm(.., had = true)`): the f32 input (rms_norm(x, w), or
// x itself, optionally moved to the GDN grouped head order of qwen35.rs:1452-1478)
// times the signs goes to an LDS buffer, the WHT runs per had_block chunk
// (lds_wht), and the rotated vector is quantized like norm_finish.  Lane t
// (of NT) owns the float4s at 4t + 4096c; the sum of squares has the
// block_sumsq_f4 order (slot t, c ascending; wave sums; tree16), as the
// unfolded RMSNorm prologue.  K <= ROT_C * 4096.
constexpr int ROT_C = 5;
template <int FMT, bool NORM> struct RotStage {
  float4 x[ROT_C], w[ROT_C];
  float* buf;   // K floats of LDS, free once the activation is staged
  float* nbuf = nullptr;   // non-null: the unrotated f32 vector is also kept here (LDS)
  HH_DEV void issue(const GemvArgs& p) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int c = 0; c < ROT_C; ++c) {
      const int e = 4 * tid + 4096 * c;
      if (e < p.K) {
        x[c] = *(const float4*)(p.x + e);
        if constexpr (NORM) w[c] = *(const float4*)(p.norm_w + e);
      }
    }
  }
  HH_DEV void store(const GemvArgs& p, int8_t* aq, float* ds, float* red) {
    const int tid = threadIdx.x, K = p.K;
    float inv = 1.0f;
    if constexpr (NORM) {
      float ss = 0.0f;
#pragma unroll
      for (int c = 0; c < ROT_C; ++c)
        if (4 * tid + 4096 * c < K) ss += x[c].x * x[c].x + x[c].y * x[c].y + x[c].z * x[c].z + x[c].w * x[c].w;
      ss = wave_sum(ss);
      if ((tid & 63) == 0) red[tid >> 6] = ss;
      __syncthreads();
      inv = 1.0f / sqrtf(tree16(red) / (float)K + p.eps);   // ops.rs:22-23
    }
    const bool perm = p.perm_rep > 1;
#pragma unroll
    for (int c = 0; c < ROT_C; ++c) {
      const int e = 4 * tid + 4096 * c;
      if (e < K) {
        float v[4] = {x[c].x, x[c].y, x[c].z, x[c].w};
        if constexpr (NORM) {
          v[0] = v[0] * inv * w[c].x; v[1] = v[1] * inv * w[c].y;   // ops.rs:29 (x * inv) * w
          v[2] = v[2] * inv * w[c].z; v[3] = v[3] * inv * w[c].w;
        }
        if (nbuf) *(float4*)(nbuf + e) = make_float4(v[0], v[1], v[2], v[3]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = perm ? grouped_pos(e + i, 128, p.perm_nk, p.perm_rep) : e + i;
          buf[d] = v[i] * p.signs[d];
        }
      }
    }
    lds_wht<NT>(buf, K, p.had_block);
#pragma unroll
    for (int c = 0; c < ROT_C; ++c) {
      if (4096 * c >= K) break;   // uniform
      const int e = 4 * tid + 4096 * c;
      const bool in = e < K;
      float vv[4] = {0.f, 0.f, 0.f, 0.f};
      if (in) {
        const float4 t = *(const float4*)(buf + e);
        vv[0] = t.x; vv[1] = t.y; vv[2] = t.z; vv[3] = t.w;
      }
      float am = fmaxf(fmaxf(fabsf(vv[0]), fabsf(vv[1])), fmaxf(fabsf(vv[2]), fabsf(vv[3])));
      am = group_max<8>(am);
      const float sc = q8_scale(am), rc = q8_rcp(sc);
      int qs = 0;
      uint32_t word = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = q8_round_r(vv[i], sc, rc);
        qs += q;
        word |= ((uint32_t)q & 0xffu) << (8 * i);
      }
      qs = group_sum_i<8>(qs);
      put4<FMT>(aq, e, word, in);
      if (in && (tid & 7) == 0) put_ds<FMT>(ds, e >> 5, h2f(f2h(sc)), qs);
    }
  }
};

template <int FMT, int PRO> struct ActStage;
template <int FMT> struct ActStage<FMT, PRO_NORMROT> : RotStage<FMT, true> {
  HH_DEV const float* r_nbuf() const { return this->nbuf; }
};
template <int FMT> struct ActStage<FMT, PRO_F32ROT> : RotStage<FMT, false> {};
template <int FMT> struct ActStage<FMT, PRO_RMSNORM> {
  NormRegsT<NORM_L> r;
  HH_DEV const float* r_nbuf() const { return r.nbuf; }
  HH_DEV void issue(const GemvArgs& p) { norm_issue<NORM_L>(p, r); }
  HH_DEV void store(const GemvArgs& p, int8_t* aq, float* ds, float* red) { norm_store<FMT, NORM_L>(p, r, aq, ds, red); }
  // Without p.sq_in: the lane's part of the sum of squares, which waits for its
  // activation loads, so the kernel's barrier after it holds every weight load
  // until the activation has landed.  With p.sq_in nothing waits here and the
  // weights stream at once (8B gate+up 10.98 -> 10.24 us, 9B GDN in_proj 7.97
  // -> 7.63 us against the in-kernel reduction).
  HH_DEV void part1(const GemvArgs& p, int8_t*, float*, float* red) {
    if (!p.sq_in) norm_partial<NORM_L>(p, r, red);
  }
  HH_DEV void part2(const GemvArgs& p, int8_t* aq, float* ds, float* red) { norm_finish<FMT, NORM_L>(p, r, aq, ds, red); }
};
// PRO_RMSNORM_ALL: the same arithmetic in all NT lanes (lane t holds slot t),
// staged like the packed prologue: its loads are issued before the weights
// and the weights stream while every lane quantizes its four values.
template <int FMT> struct ActStage<FMT, PRO_RMSNORM_ALL> {
  NormRegsT<NT> r;
  HH_DEV const float* r_nbuf() const { return r.nbuf; }
  HH_DEV void issue(const GemvArgs& p) { norm_issue<NT>(p, r); }
  HH_DEV void store(const GemvArgs& p, int8_t* aq, float* ds, float* red) { norm_store<FMT, NT>(p, r, aq, ds, red); }
};
template <int FMT> struct ActStage<FMT, PRO_PACKED> {
  PackedRegs r;
  HH_DEV void issue(const GemvArgs& p) { packed_issue(p, r); }
  HH_DEV void store(const GemvArgs& p, int8_t* aq, float* ds, float*) { packed_store<FMT>(p, r, aq, ds); }
};
template <int FMT> struct ActStage<FMT, PRO_STDQ8> {
  StdRegs r;
  HH_DEV void issue(const GemvArgs& p) { std_issue(p, r); }
  HH_DEV void store(const GemvArgs& p, int8_t* aq, float* ds, float*) { std_store<FMT>(p, r, aq, ds); }
};

// NU = 1, 2, 4: every lane holds at most NU units, all loaded at once before
// the prologue (one batch).  NU = 0: larger workgroups stream batches of
// DEPTH units per lane, double-buffered in VGPRs.  Every weight load is
// unconditional (lanes past the last unit re-read it): a load under a branch
// makes the compiler count it as possibly absent, and the wait for an earlier
// load then also waits for the weight loads issued after it.
template <int FMT, int PRO, int EPI, int NU>
__global__ __launch_bounds__(NT) void k_gemv(GemvArgs p) {
  constexpr int DW = UnitT<FMT>::DW;
  constexpr int UB = UnitT<FMT>::BYTES;
  constexpr int DEPTH = NU > 0 ? NU : 2;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int K = p.K;
  const int P = p.P;

  if constexpr (EPI == EPI_LOGITS) {
    // Prompt tokens other than the last need no logits (forward_batch computes
    // only the last token's, mod.rs:1201-1218); k_head_final advances the state.
    const StepState* st = p.state;
    if (st->step + 1 < st->n_prompt) return;
  }

  // rows owned by this workgroup.  EPI_SILU: the gate rows come in blocks
  // of 32 (one Q8_0 block of the output); workgroup g takes blocks g, g + G,
  // ... (G = grid size), all its gate rows first, then the matching up rows.
  int rows_total, r0 = 0, nbw = 0;
  if constexpr (EPI == EPI_SILU) {
    const int nblk = p.half_rows / 32;
    nbw = (nblk - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    rows_total = 64 * nbw;
  } else {
    r0 = blockIdx.x * p.rows_per_wg;
    rows_total = min(p.rows_per_wg, p.n_rows - r0);
  }
  const int U = rows_total * P;

  // LDS carve-up
  const int nunits_act = K / UnitT<FMT>::EL;
  int8_t* aq = (int8_t*)smem;
  float* ds = (float*)(smem + nunits_act * qstride<FMT>());
  // Block products by row: part[row * RSJ + j] for product j = 2*unit + blk,
  // RSJ = 4 (mod 8) words, so the row-sum pass (one lane per row, 16-byte
  // reads) puts each 8 lanes' reads on distinct banks; they follow rowsum and
  // the prologue buffers (below).  The rotating prologues keep them
  // transposed, part[j * RS + row] with RS = rows + 1, ahead of the wave
  // partials: there the by-row form costs the compiler 12-48 more bytes of
  // spills per lane.
  constexpr bool PART_T = PRO == PRO_NORMROT || PRO == PRO_F32ROT;
  const int NPR = 2 * P;
  const int RSJ = gemv_part_stride(P);
  const int RS = rows_total + 1;
  float* part = ds + nunits_act * dss<FMT>();
  float* red = PART_T ? part + 2 * P * RS : part;   // 16 wave partials
  float* rowsum = red + 16;

  auto unit_addr = [&](int lu) -> const uint8_t* {
    int rl = lu / P, t = lu - rl * P;
    int grow;
    if constexpr (EPI == EPI_SILU) {
      const int gl = rl < 32 * nbw ? rl : rl - 32 * nbw;   // local gate row
      grow = ((int)blockIdx.x + (gl >> 5) * (int)gridDim.x) * 32 + (gl & 31);
      if (rl >= 32 * nbw) grow += p.half_rows;
    } else {
      grow = r0 + rl;
    }
    return p.w + ((size_t)grow * P + t) * UB;
  };

  // With the RMSNorm prologue, lanes 0..NORM_L-1 stage the activation before
  // issuing weights; they take the last units of each batch (none at all when
  // the workgroup holds fewer than NT - NORM_L units).  Products are indexed by
  // unit, so the mapping does not change any sum.
  // GDN input projection: this workgroup's alpha/beta row (qwen35.rs:1285-1291)
  constexpr bool AB_OK = (PRO == PRO_RMSNORM || PRO == PRO_RMSNORM_ALL || PRO == PRO_NORMROT) && EPI == EPI_STORE;
  const bool ab = AB_OK && p.ab_out && (int)blockIdx.x < p.ab_rows;   // uniform
  __shared__ float abred[16];
  float4 abw[2];
  const int lt = PRO == PRO_RMSNORM ? ((tid + NORM_L) & (NT - 1)) : tid;
  const int NI = (U + NT - 1) / NT;
  const int NB = (NI + DEPTH - 1) / DEPTH;
  uint32_t wa[DEPTH][DW], wb[NU > 0 ? 1 : DEPTH][DW];

  auto load_batch = [&](uint32_t (&wr)[DEPTH][DW], int b) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      int lu = min((b * DEPTH + d) * NT + lt, U - 1);
      load_unit<FMT>(wr[d], unit_addr(lu));
    }
    if constexpr (AB_OK) {   // behind the first batch: waited for in the epilogue only
      if (ab && b == 0) {
        const int row = blockIdx.x;
        const float* wrow = row < p.ab_n ? p.ab_wa + (size_t)row * K : p.ab_wb + (size_t)(row - p.ab_n) * K;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const int e = 4 * tid + 4096 * c;
          abw[c] = e < K ? *(const float4*)(wrow + e) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
  };
  auto comp_batch = [&](const uint32_t (&wr)[DEPTH][DW], int b) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      int lu = (b * DEPTH + d) * NT + lt;
      if (lu < U) {
        int rl = lu / P, t = lu - rl * P;
        float pr[2];
        const float* ud = ds + t * dss<FMT>();
        unit_dot<FMT>(wr[d], aq + t * qstride<FMT>(), ud, (const int*)(ud + UnitT<FMT>::SUBS), pr);
        if constexpr (PART_T) {
          part[(2 * t) * RS + rl] = pr[0];
          part[(2 * t + 1) * RS + rl] = pr[1];
        } else {
          *(float2*)(part + rl * RSJ + 2 * t) = make_float2(pr[0], pr[1]);
        }
      }
    }
  };

  ActStage<FMT, PRO> act;
  float* lds_tail = (float*)(((uintptr_t)(rowsum + rows_total) + 15) & ~(uintptr_t)15);   // 16-byte aligned
  if constexpr (PRO == PRO_NORMROT || PRO == PRO_F32ROT) {   // K floats after rowsum
    act.buf = lds_tail;
    lds_tail += K;
  }
  if constexpr (AB_OK) {
    if (ab) {
      if constexpr (PRO == PRO_RMSNORM || PRO == PRO_RMSNORM_ALL) act.r.nbuf = lds_tail;
      else act.nbuf = lds_tail;
      lds_tail += K;
    }
  }
  if constexpr (!PART_T) part = lds_tail;
  act.issue(p);                      // activation first (in-order retirement)
  // the residual of this lane's row (EPI_ADD), read now rather than after the
  // row sums, where its round trip would be the kernel's last step
  // (unconditional: lanes past the rows re-read the last)
  float yres = 0.0f;
  if constexpr (EPI == EPI_ADD) yres = p.y[r0 + min(tid, rows_total - 1)];
  if constexpr (FMT == FMT_PT) {     // read only after the prologue's barrier
    if (tid < 256) pt_lut[tid] = pt_lut_entry(tid);
  }
  if constexpr (NU > 0 && PRO == PRO_RMSNORM) {
    // The NORM_L staging lanes stage the activation and raise `ready`; every
    // wave computes as soon as `ready` is complete and its own weights have
    // arrived.  No barrier
    // separates the weight loads from the dot products: a CU's weight stream
    // retires in issue order while the waves that issued first already compute.
    __shared__ int ready;
    if (tid == 0) ready = 0;
    act.part1(p, aq, ds, red);       // waits for this lane's activation loads
    __syncthreads();                 // sum of squares complete, `ready` cleared
    if (tid < NORM_L) {
      act.part2(p, aq, ds, red);
      if ((tid & 63) == 0) __hip_atomic_fetch_add(&ready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    load_batch(wa, 0);               // the whole share of this lane
    for (int it = 0; __hip_atomic_load(&ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < NORM_L / 64 &&
                     it < (1 << 22); ++it)
      __builtin_amdgcn_s_sleep(1);
    comp_batch(wa, 0);
  } else if constexpr (NU > 0) {
    load_batch(wa, 0);               // the whole share of this lane
    act.store(p, aq, ds, red);
    __syncthreads();
    comp_batch(wa, 0);
  } else {
    load_batch(wa, 0);
    load_batch(wb, 1);
    act.store(p, aq, ds, red);
    __syncthreads();
    int b = 0;
    for (; b + 2 < NB; b += 2) {
      comp_batch(wa, b);
      load_batch(wa, b + 2);
      comp_batch(wb, b + 1);
      load_batch(wb, b + 3);
    }
    comp_batch(wa, b);
    if (b + 1 < NB) comp_batch(wb, b + 1);
  }
  if constexpr (AB_OK) {
    // alpha/beta dot (matvec_dense, qwen35.rs:1015-1025) in 1024 slots: slot t
    // sums w * x over its float4s at 4t + 4096c (c, then element, ascending);
    // each wave's 64 slots by butterfly into abred; tree16 of abred after the
    // row sums.  Run here, its wave sums share the barrier below.
    if (ab) {
      const float* nb = act.r_nbuf();
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int e = 4 * tid + 4096 * c;
        if (e < K) {
          const float4 x = *(const float4*)(nb + e);
          acc = acc + abw[c].x * x.x;
          acc = acc + abw[c].y * x.y;
          acc = acc + abw[c].z * x.z;
          acc = acc + abw[c].w * x.w;
        }
      }
      acc = wave_sum(acc);
      if ((tid & 63) == 0) abred[tid >> 6] = acc;
    }
  }
  __syncthreads();

  // per-row sums over the block products in block order (the scalar loop);
  // by row: up to 32 products per LDS round trip (16-byte reads); transposed:
  // 16; the additions stay sequential
  for (int r = tid; r < rows_total; r += NT) {
    float s = 0.0f;
    int j = 0;
    if constexpr (PART_T) {
      for (; j + 16 <= NPR; j += 16) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = part[(j + i) * RS + r];
#pragma unroll
        for (int i = 0; i < 16; ++i) s += v[i];
      }
      for (; j < NPR; ++j) s += part[j * RS + r];
    } else {
      const float* pr = part + r * RSJ;
      for (; j + 32 <= NPR; j += 32) {
        float4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = ((const float4*)(pr + j))[i];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          s += v[i].x;
          s += v[i].y;
          s += v[i].z;
          s += v[i].w;
        }
      }
      for (; j + 16 <= NPR; j += 16) {
        float4 v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = ((const float4*)(pr + j))[i];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s += v[i].x;
          s += v[i].y;
          s += v[i].z;
          s += v[i].w;
        }
      }
      for (; j + 4 <= NPR; j += 4) {
        const float4 v = *(const float4*)(pr + j);
        s += v.x;
        s += v.y;
        s += v.z;
        s += v.w;
      }
      for (; j < NPR; ++j) s += pr[j];
    }
    rowsum[r] = s;
  }
  // EPI_STORE / EPI_ADD read rowsum[r] in the lane that wrote it (and the
  // alpha/beta wave sums were written before the barrier above): no barrier
  if constexpr (EPI != EPI_STORE && EPI != EPI_ADD) __syncthreads();

  if constexpr (EPI == EPI_STORE || EPI == EPI_ADD) {
    for (int r = tid; r < rows_total; r += NT) {
      if constexpr (EPI == EPI_STORE) p.y[r0 + r] = rowsum[r];
      else p.y[r0 + r] = (r == tid ? yres : p.y[r0 + r]) + rowsum[r];
    }
    if constexpr (EPI == EPI_ADD) {
      if (p.sq_out) {   // uniform; the launcher checks rows_per_wg % 16 == 0
        // the RMSNorm tree over the rows just written, whole wave active:
        // s (lane 4t) = ((v0 + v1) + v2) + v3, node (lane 16k) = (s0 + s1) + (s2 + s3)
        const float yv = tid < rows_total ? yres + rowsum[tid] : 0.0f;
        const float v = yv * yv;
        float t = v + dpp_from_lane_plus<1>(v);
        t = t + dpp_from_lane_plus<2>(v);
        t = t + dpp_from_lane_plus<3>(v);
        const float h = t + dpp_from_lane_plus<4>(t);
        const float node = h + dpp_from_lane_plus<8>(h);
        if (tid < rows_total && (tid & 15) == 0) p.sq_out[(r0 + tid) >> 4] = node;
      }
    }
    if constexpr (AB_OK) {
      if (ab && tid == 0) p.ab_out[blockIdx.x] = tree16(abred);   // wave sums written before the row sums
    }
  } else if constexpr (EPI == EPI_SILU) {
    // ops.rs:240-253 silu then mul_elem (mod.rs:758-763), then Q8_0 (q8_0.rs:20-51)
    const int R2 = 32 * nbw;
    for (int i0 = 0; i0 < R2; i0 += NT) {
      int i = i0 + tid;
      float h = 0.0f;
      if (i < R2) {
        float g = rowsum[i];
        float sg = g / (1.0f + hx_exp(-g));
        h = sg * rowsum[R2 + i];
      }
      float am = group_max<32>(fabsf(h));
      float sc = q8_scale(am);
      int q = q8_round_r(h, sc, q8_rcp(sc));
      int qs = group_sum_i<32>(q);
      if (p.y) {   // folded model: the next matmul rotates the f32 vector first
        if (i < R2) p.y[((int)blockIdx.x + (i >> 5) * (int)gridDim.x) * 32 + (i & 31)] = h;
        continue;
      }
      if (i < R2) {
        int e = ((int)blockIdx.x + (i >> 5) * (int)gridDim.x) * 32 + (i & 31);
        p.act_out[perm_pos(p.act_out_fmt, e)] = (uint8_t)(int8_t)q;
        if ((i & 31) == 0) {
          float* od = (float*)(p.act_out + p.act_out_k);
          int* os = (int*)(p.act_out + p.act_out_k + (p.act_out_k / 32) * 4);
          od[e >> 5] = h2f(f2h(sc));
          os[e >> 5] = qs;
        }
      }
    }
  } else if constexpr (EPI == EPI_LOGITS) {
    const StepState* st = p.state;
    const int rule = p.rule;
    const float pen = st->pen;
    const bool do_pen = !(fabsf(pen - 1.0f) < 1e-6f);
    float bv = -INFINITY;
    int bi = (rule == 0) ? -1 : 0x7fffffff;
    for (int r = tid; r < rows_total; r += NT) {
      float v = rowsum[r];
      int gr = r0 + r;
      if (p.y) p.y[gr] = v;
      if (rule == 0 && do_pen) {
        int c = p.counts[gr];
        for (int k = 0; k < c; ++k) v = (v > 0.0f) ? v / pen : v * pen;   // lib.rs:26-40
      }
      bool better = (rule == 0) ? (v > bv || (v == bv && gr > bi)) : (v > bv || (v == bv && gr < bi));
      if (v != v) better = false;
      if (better) { bv = v; bi = gr; }
    }
    // workgroup reduction
    __shared__ float sv[NT];
    __shared__ int si[NT];
    sv[tid] = bv;
    si[tid] = bi;
    __syncthreads();
    for (int o = NT / 2; o > 0; o >>= 1) {
      if (tid < o) {
        float v2 = sv[tid + o];
        int i2 = si[tid + o];
        float v1 = sv[tid];
        int i1 = si[tid];
        bool take = (rule == 0) ? (v2 > v1 || (v2 == v1 && i2 > i1)) : (v2 > v1 || (v2 == v1 && i2 < i1));
        if (take) { sv[tid] = v2; si[tid] = i2; }
      }
      __syncthreads();
    }
    if (tid == 0) {
      p.part_val[blockIdx.x] = sv[0];
      p.part_idx[blockIdx.x] = si[0];
    }
  }
}


// Greedy selection over the per-workgroup (value, index) partials of the
// EPI_LOGITS head, with the same tie rule, then the step-state advance:
// record the token, count it into the penalty history, move to the next
// position.  For a prompt token other than the last the head computed
// nothing and the state advances to the next prompt token.
// The next step's embedding (mod.rs:483-504), written here so that the next
// decode step needs no embedding kernel: all lanes, once the token is known.
HH_DEV void head_final_embed(const GemvArgs& p, int tok, float* ebuf) {
  if (!p.emb_out) return;   // uniform
  embed_row<1024>(p.emb_type, p.emb_table, p.emb_d, tok, p.emb_out, p.emb_signs, p.emb_had, ebuf);
}

__global__ __launch_bounds__(1024) void k_head_final(GemvArgs p, int n_part) {
  extern __shared__ __align__(16) float ebuf[];   // emb_d floats for a latent table
  __shared__ float sv[1024];
  __shared__ int si[1024];
  __shared__ int step0, prompt_only, next_tok, advanced;
  StepState* st = p.state;
  const int tid = threadIdx.x;
  const int rule = p.rule;
  if (tid == 0) {
    step0 = st->step;
    prompt_only = (st->step + 1 < st->n_prompt);
    next_tok = st->token;
    advanced = 0;
  }
  __syncthreads();
  const int s = step0;
  if (prompt_only) {
    if (tid == 0) {
      next_tok = (int)p.prompt[s + 1];
      st->token = next_tok;
      st->pos = st->pos + 1;
      st->step = s + 1;
    }
    __syncthreads();
    head_final_embed(p, next_tok, ebuf);
    return;
  }
  float v1 = -INFINITY;
  int i1 = (rule == 0) ? -1 : 0x7fffffff;
  for (int b = tid; b < n_part; b += 1024) {
    float v2 = p.part_val[b];
    int i2 = p.part_idx[b];
    bool take = (rule == 0) ? (v2 > v1 || (v2 == v1 && i2 > i1)) : (v2 > v1 || (v2 == v1 && i2 < i1));
    if (take) { v1 = v2; i1 = i2; }
  }
  sv[tid] = v1;
  si[tid] = i1;
  __syncthreads();
  for (int o = 512; o > 0; o >>= 1) {
    if (tid < o) {
      float v2 = sv[tid + o];
      int i2 = si[tid + o];
      float va = sv[tid];
      int ia = si[tid];
      bool take = (rule == 0) ? (v2 > va || (v2 == va && i2 > ia)) : (v2 > va || (v2 == va && i2 < ia));
      if (take) { sv[tid] = v2; si[tid] = i2; }
    }
    __syncthreads();
  }
  if (tid == 0) {
    int tok = si[0];
    if (tok < 0 || tok >= p.n_rows) tok = 0;
    st->argmax = tok;
    if (st->update) {
      int gen = s + 1 - st->n_prompt;           // index of this generated token
      if (gen >= 0 && gen < p.max_out) p.out_tokens[gen] = (uint32_t)tok;
      p.counts[tok] += 1;                        // past_tokens.push(token)
      st->token = tok;
      st->pos = st->pos + 1;
      st->step = s + 1;
      next_tok = tok;
      advanced = 1;
    }
  }
  __syncthreads();
  if (advanced) head_final_embed(p, next_tok, ebuf);   // uniform
}


// LM head (EPI_LOGITS): output_norm + Q8_0 of the hidden state, then every
// vocab row's dot, the repetition penalty and the argmax partials
// (sampler lib.rs:26-40, :167-175; qwen35.rs:1735-1745).  One workgroup per
// CU stages the activation once; then each wave streams whole rows on its
// own (rows gw, gw + W, ... for global wave gw of W), double-buffered in
// VGPRs, with no further workgroup barrier.  Lane l holds the row's units
// l + 64u (u < U); the row value is q_l = sum_u (p_2t + p_2t+1) over its
// units' block products, then an ascending butterfly over the 64 lanes.
template <int FMT, int U, int PRO>
__global__ __launch_bounds__(NT) void k_head(GemvArgs p) {
  constexpr int DW = UnitT<FMT>::DW;
  constexpr int UB = UnitT<FMT>::BYTES;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int K = p.K, P = p.P, n = p.n_rows;
  const int nunits_act = K / UnitT<FMT>::EL;
  int8_t* aq = (int8_t*)smem;
  float* ds = (float*)(smem + nunits_act * qstride<FMT>());
  float* red = ds + nunits_act * dss<FMT>();     // 16
  float* bvs = red + 16;                         // 16 wave bests
  int* bis = (int*)(bvs + 16);

  const int gw = blockIdx.x * (NT / 64) + wv, W = gridDim.x * (NT / 64);
  // a row's repetition count is loaded with its weights (every lane, one
  // address): loaded later, its wait would also wait for the next row's units
  const int* cnt_src = p.counts ? p.counts : (const int*)p.w;
  auto load_row = [&](uint32_t (&wr)[U][DW], int& cnt, int r) {
    r = min(r, n - 1);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = min(lane + 64 * u, P - 1);
      load_unit<FMT>(wr[u], p.w + ((size_t)r * P + t) * UB);
    }
    cnt = cnt_src[p.counts ? r : 0];
  };
  const int rule = p.rule;
  float pen = 1.0f;        // StepState::pen, taken once the first loads are out
  bool do_pen = false;
  float bv = -INFINITY;
  int bi = (rule == 0) ? -1 : 0x7fffffff;
  auto row = [&](const uint32_t (&wr)[U][DW], int cnt, int r) {
    float q = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = lane + 64 * u;
      if (t < P) {
        float pr[2];
        const float* ud = ds + t * dss<FMT>();
        unit_dot<FMT>(wr[u], aq + t * qstride<FMT>(), ud, (const int*)(ud + UnitT<FMT>::SUBS), pr);
        q = q + (pr[0] + pr[1]);
      }
    }
    float v = group_sum<64>(q);
    if (lane == 0) {
      if (p.y) p.y[r] = v;
      if (do_pen) {
        for (int k = 0; k < cnt; ++k) v = (v > 0.0f) ? v / pen : v * pen;   // lib.rs:26-40
      }
      bool better = (rule == 0) ? (v > bv || (v == bv && r > bi)) : (v > bv || (v == bv && r < bi));
      if (v != v) better = false;
      if (better) { bv = v; bi = r; }
    }
  };

  ActStage<FMT, PRO> act;
  if constexpr (PRO == PRO_NORMROT) act.buf = (float*)(bis + 16);   // K floats after the wave bests
  act.issue(p);
  uint32_t wa[U][DW], wb[U][DW];
  int ca, cb;
  load_row(wa, ca, gw);
  // the step state, read behind the first row: the loop waits for that row anyway
  const int sv = state_lanes(p.state);
  act.store(p, aq, ds, red);
  __syncthreads();
  // StepState::step + 1 < n_prompt: k_head_final advances the prompt, no rows
  const int n_eff = __builtin_amdgcn_readlane(sv, 1) + 1 < __builtin_amdgcn_readlane(sv, 3) ? 0 : n;
  pen = __int_as_float(__builtin_amdgcn_readlane(sv, 7));
  do_pen = rule == 0 && !(fabsf(pen - 1.0f) < 1e-6f);
  for (int r = gw; r < n_eff; r += 2 * W) {
    load_row(wb, cb, r + W);
    row(wa, ca, r);
    load_row(wa, ca, r + 2 * W);
    if (r + W < n_eff) row(wb, cb, r + W);
  }
  if (lane == 0) { bvs[wv] = bv; bis[wv] = bi; }
  __syncthreads();
  if (tid == 0) {
    float v1 = bvs[0];
    int i1 = bis[0];
    for (int w = 1; w < NT / 64; ++w) {
      const float v2 = bvs[w];
      const int i2 = bis[w];
      const bool take = (rule == 0) ? (v2 > v1 || (v2 == v1 && i2 > i1)) : (v2 > v1 || (v2 == v1 && i2 < i1));
      if (take) { v1 = v2; i1 = i2; }
    }
    p.part_val[blockIdx.x] = v1;
    p.part_idx[blockIdx.x] = i1;
  }
}

template <int FMT>
int launch_head(GemvArgs a, hipStream_t s, int* n_wg_out) {
  const int n_wg = std::max(1, std::min(256, (a.n_rows + NT / 64 - 1) / (NT / 64)));
  const int nunits = a.K / UnitT<FMT>::EL;
  const bool rot = a.had_block > 0;
  const size_t lds = (size_t)nunits * (UnitT<FMT>::EL + 16) + (size_t)nunits * (FMT == FMT_Q8 ? 8 : 20) * 4 + 48 * 4 +
                     (rot ? (size_t)a.K * 4 : 0);
  if (rot && (a.K > ROT_C * 4096 || !a.signs)) return 1;
  if (a.P <= 64) {
    if (rot) hipLaunchKernelGGL((k_head<FMT, 1, PRO_NORMROT>), dim3(n_wg), dim3(NT), lds, s, a);
    else hipLaunchKernelGGL((k_head<FMT, 1, PRO_RMSNORM>), dim3(n_wg), dim3(NT), lds, s, a);
  } else if (a.P <= 128) {
    if (rot) hipLaunchKernelGGL((k_head<FMT, 2, PRO_NORMROT>), dim3(n_wg), dim3(NT), lds, s, a);
    else hipLaunchKernelGGL((k_head<FMT, 2, PRO_RMSNORM>), dim3(n_wg), dim3(NT), lds, s, a);
  } else {
    return 1;
  }
  *n_wg_out = n_wg;
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

template <int FMT, int PRO, int EPI, int NU>
int launch_t(const GemvArgs& a, int n_wg, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL((k_gemv<FMT, PRO, EPI, NU>), dim3(n_wg), dim3(NT), lds, s, a);
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

template <int FMT, int PRO, int EPI>
int launch_u(const GemvArgs& a, int nu, int n_wg, size_t lds, hipStream_t s) {
  switch (nu) {
    case 1: return launch_t<FMT, PRO, EPI, 1>(a, n_wg, lds, s);
    case 2: return launch_t<FMT, PRO, EPI, 2>(a, n_wg, lds, s);
    case 4: return launch_t<FMT, PRO, EPI, 4>(a, n_wg, lds, s);
    default: return launch_t<FMT, PRO, EPI, 0>(a, n_wg, lds, s);
  }
}

// Prologue/epilogue pairs of the decode step (and the STDQ8 operator).
template <int FMT>
int launch_p(const GemvArgs& a, int pro, int epi, int nu, int n_wg, size_t lds, hipStream_t s) {
  switch (pro) {
    case PRO_PACKED:
      if (a.K > PK_Q * 16 * PK_L) return 1;
      if (epi == EPI_ADD) return launch_u<FMT, PRO_PACKED, EPI_ADD>(a, nu, n_wg, lds, s);
      if (epi == EPI_STORE) return launch_u<FMT, PRO_PACKED, EPI_STORE>(a, nu, n_wg, lds, s);
      return 1;
    case PRO_STDQ8:
      if (a.K > SQ_C * 4 * NT) return 1;
      if (epi == EPI_STORE) return launch_u<FMT, PRO_STDQ8, EPI_STORE>(a, nu, n_wg, lds, s);
      return 1;
    case PRO_RMSNORM:
      if (a.K % 1024 != 0 || a.K > NORM_CH * 4096) return 1;
      if (epi == EPI_STORE) return launch_u<FMT, PRO_RMSNORM, EPI_STORE>(a, nu, n_wg, lds, s);
      if (epi == EPI_SILU) return launch_u<FMT, PRO_RMSNORM, EPI_SILU>(a, nu, n_wg, lds, s);
      return 1;
    case PRO_RMSNORM_ALL:
      if (a.K % 1024 != 0 || a.K > NORM_CH * 4096) return 1;
      if (epi == EPI_STORE) return launch_u<FMT, PRO_RMSNORM_ALL, EPI_STORE>(a, nu, n_wg, lds, s);
      if (epi == EPI_SILU) return launch_u<FMT, PRO_RMSNORM_ALL, EPI_SILU>(a, nu, n_wg, lds, s);
      return 1;
    case PRO_NORMROT:
      if (epi == EPI_STORE) return launch_u<FMT, PRO_NORMROT, EPI_STORE>(a, nu, n_wg, lds, s);
      if (epi == EPI_SILU) return launch_u<FMT, PRO_NORMROT, EPI_SILU>(a, nu, n_wg, lds, s);
      return 1;
    case PRO_F32ROT:
      if (epi == EPI_ADD) return launch_u<FMT, PRO_F32ROT, EPI_ADD>(a, nu, n_wg, lds, s);
      return 1;
  }
  return 1;
}

}  // namespace

int hh_fmt_of(int ggml_type) {
  switch (ggml_type) {
    case 8: return FMT_Q8;
    case 41: case 43: return FMT_Q1;
    case 42: case 142: return FMT_Q2;
    case 143: return FMT_PT;
  }
  return -1;
}

int hh_unit_el(int fmt) { return fmt == FMT_Q8 ? 64 : 256; }

// LDS bytes for a launch and the workgroup count.
size_t hh_gemv_lds(int fmt, int K, int rows_total_per_wg) {
  int el = hh_unit_el(fmt);
  int P = K / el;
  size_t qb = (size_t)(K / el) * (el + 16);
  size_t dsb = (size_t)(K / el) * (fmt == FMT_Q8 ? 8 : 20) * 4;
  // block products: by row (gemv_part_stride) or transposed (rows + 1 per product)
  const size_t pw = std::max((size_t)rows_total_per_wg * gemv_part_stride(P), (size_t)(rows_total_per_wg + 1) * 2 * P);
  size_t b = qb + dsb + 16 * 4 + (size_t)rows_total_per_wg * 4 + 16 + pw * 4;
  return (b + 15) & ~(size_t)15;
}

// EPI_SILU workgroups for nblk 32-row gate blocks.  Past two blocks per
// workgroup every workgroup takes the same count: 27B (544 blocks) on 182
// workgroups of 3 instead of 256 of 2 or 3, gate+up 17.01 -> 16.57 us, step
// 3.331 -> 3.315 ms.  Two or fewer stay on up to 256 workgroups (8B and 9B,
// 384 blocks: even shares measured the same).
static int silu_grid(int nblk) {
  if (nblk <= 512) return std::min(nblk, 256);
  const int per = (nblk + 255) / 256;
  return (nblk + per - 1) / per;
}

int hh_gemv_launch(int fmt, int pro, int epi, GemvArgs a, hipStream_t s) {
  int el = hh_unit_el(fmt);
  if (a.K % el != 0) return 1;
  if (a.sq_in && (pro != PRO_RMSNORM || a.K % 64 != 0 || a.K > 4096)) return 1;
  if (a.sq_out && (epi != EPI_ADD || a.rows_per_wg % 16 != 0 || a.rows_per_wg > NT || a.n_rows % 16 != 0)) return 1;
  a.P = a.K / el;
  int n_wg, rows_total;
  const bool rot = pro == PRO_NORMROT || pro == PRO_F32ROT;
  if (rot) {   // folded prologue: whole fold chunks, K <= ROT_C * 4096
    if (!a.signs || a.had_block < 2 || (a.had_block & (a.had_block - 1)) || a.K % a.had_block || a.K % 1024 ||
        a.K > ROT_C * 4096)
      return 1;
    if (pro == PRO_F32ROT && a.perm_rep > 1 && a.K != a.perm_nk * a.perm_rep * 128) return 1;
  }
  if (epi == EPI_LOGITS) {   // persistent row-streaming head + finalize
    if (a.K % 1024 != 0 || a.K > NORM_CH * 4096) return 1;
    if (pro != PRO_RMSNORM && pro != PRO_NORMROT) return 1;
    if (pro == PRO_RMSNORM) a.had_block = 0;
    int rc = 1;
    switch (fmt) {
      case FMT_Q2: rc = launch_head<FMT_Q2>(a, s, &n_wg); break;
      case FMT_Q1: rc = launch_head<FMT_Q1>(a, s, &n_wg); break;
      case FMT_Q8: rc = launch_head<FMT_Q8>(a, s, &n_wg); break;
    }
    if (rc) return rc;
    hipLaunchKernelGGL(k_head_final, dim3(1), dim3(1024), a.emb_out && a.emb_had > 0 ? (size_t)a.emb_d * 4 : 0, s, a, n_wg);
    return hipGetLastError() == hipSuccess ? 0 : 1;
  }
  if (epi == EPI_SILU) {
    if (a.half_rows % 32 != 0) return 1;
    const int nblk = a.half_rows / 32;
    n_wg = silu_grid(nblk);
    rows_total = 64 * ((nblk + n_wg - 1) / n_wg);   // the largest share
  } else {
    n_wg = (a.n_rows + a.rows_per_wg - 1) / a.rows_per_wg;
    rows_total = a.rows_per_wg;
  }
  size_t lds = hh_gemv_lds(fmt, a.K, rows_total);
  if (rot) lds += (size_t)a.K * 4 + 16;   // the rotation buffer after rowsum
  if (a.ab_out) {   // the normed vector kept for the alpha/beta rows
    if (epi != EPI_STORE || (pro != PRO_RMSNORM && pro != PRO_RMSNORM_ALL && pro != PRO_NORMROT) || a.K > 8192 ||
        a.ab_rows > n_wg ||
        a.ab_rows != 2 * a.ab_n)
      return 1;
    lds += (size_t)a.K * 4 + (rot ? 0 : 16);
  }
  if (pro == PRO_RMSNORM && epi == EPI_STORE) {
    // A workgroup with at most 32 KB of weights runs the RMSNorm prologue in all
    // lanes with its weights issued behind the activation (8B in_proj 7.13 ->
    // 6.55 us); larger shares keep the staging waves and the `ready` hand-off
    // (9B GDN in_proj, 52 KB: 7.96 -> 8.33 us the other way).
    const int ub = fmt == FMT_Q1 ? UnitT<FMT_Q1>::BYTES : fmt == FMT_PT ? UnitT<FMT_PT>::BYTES : UnitT<FMT_Q2>::BYTES;
    if ((size_t)rows_total * a.P * ub <= 32768) pro = PRO_RMSNORM_ALL;
  }
  const int ni = (rows_total * a.P + NT - 1) / NT;   // units per lane
  const int nu = ni <= 1 ? 1 : ni <= 2 ? 2 : ni <= 4 ? 4 : 0;
  int rc = 1;
  switch (fmt) {
    case FMT_Q2: rc = launch_p<FMT_Q2>(a, pro, epi, nu, n_wg, lds, s); break;
    case FMT_Q1: rc = launch_p<FMT_Q1>(a, pro, epi, nu, n_wg, lds, s); break;
    case FMT_PT: rc = launch_p<FMT_PT>(a, pro, epi, nu, n_wg, lds, s); break;
    case FMT_Q8: rc = launch_p<FMT_Q8>(a, pro, epi, nu, n_wg, lds, s); break;
  }
  if (rc == 0 && epi == EPI_LOGITS) {
    hipLaunchKernelGGL(k_head_final, dim3(1), dim3(1024), a.emb_out && a.emb_had > 0 ? (size_t)a.emb_d * 4 : 0, s, a, n_wg);
    rc = hipGetLastError() == hipSuccess ? 0 : 1;
  }
  return rc;
}

int hh_gemv_grid(int epi, const GemvArgs& a) {
  if (epi == EPI_SILU) return silu_grid(a.half_rows / 32);
  return (a.n_rows + a.rows_per_wg - 1) / a.rows_per_wg;
}
