// hh_device.h — device-side helpers shared by the gfx950 kernels.
//
// Formats (crates/hearth-gguf/src/ggml.rs:49-53, :105-171):
//   Q8_0 : 32 el / 34 B  [f16 d][32 x i8]                    (q8_0.rs:4-51)
//   Q1_0 : 128 el / 18 B [f16 d][16 B sign bits, LSB first]  (q1_0g128.rs:75-98)
//   Q2_0 : 128 el / 34 B [f16 d][32 B 2-bit codes, LSB first, w = code-1] (q2_0.rs:66-84)
//
// Weights stay in that native layout in HBM.  A GEMV lane works on a "unit" of
// whole blocks whose byte size is a multiple of 4 (so one dword-aligned 68- or
// 36-byte load feeds it): Q2_0 2 blocks (256 el, 68 B), Q1_0 2 blocks (256 el,
// 36 B), Q8_0 2 blocks (64 el, 68 B).  Rows are contiguous, so a matrix is a flat
// array of units and consecutive lanes read consecutive units.
//
// Activations enter the GEMV as a "packed" Q8_0 vector: the same int8 values and
// f16 scales as Q8_0 (bit-exact with q8_0.rs:20-51), stored as
//   q[K] int8, permuted within 16/32-element chunks to match the weight format's
//        bit-extraction order (so one AND + one v_dot4 handles 4 elements),
//   d[K/32] f32 (the f16 scale widened), s[K/32] int32 (sum of q per block; lets
//        the unsigned 2-bit codes stand in for code-1 and bits for +-1).
#pragma once
#include <cstddef>
#include <hip/hip_runtime.h>
#include <stdint.h>

#define HH_DEV __device__ __forceinline__

enum : int { FMT_Q8 = 0, FMT_Q1 = 1, FMT_Q2 = 2, FMT_PT = 3 };

typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

template <int FMT> struct UnitT;
template <> struct UnitT<FMT_Q2> { static constexpr int EL = 256, DW = 17, BYTES = 68, SUBS = 8; };
template <> struct UnitT<FMT_Q1> { static constexpr int EL = 256, DW = 9, BYTES = 36, SUBS = 8; };
template <> struct UnitT<FMT_Q8> { static constexpr int EL = 64, DW = 17, BYTES = 68, SUBS = 2; };
template <> struct UnitT<FMT_PT> { static constexpr int EL = 256, DW = 14, BYTES = 56, SUBS = 8; };

// LDS stride of one unit's int8 activations (16 B pad spreads units over banks).
template <int FMT> HH_DEV constexpr int qstride() { return UnitT<FMT>::EL + 16; }

HH_DEV float h2f(uint32_t h16) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(h16 & 0xffffu)); }

// f32 -> f16 bits, round to nearest even (half 2.7.1 f16::from_f32), written
// with integer operations.  A plain (_Float16) cast is not used because the
// compiler may fold fptrunc(a * b) into a mixed-precision multiply that rounds
// the exact product to f16 once, which differs from rounding the f32 product
// when that product sits exactly on an f16 tie.
HH_DEV uint32_t f2h(float xf) {
  uint32_t x = __float_as_uint(xf);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) return sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u);
  int half_exp = (int)exp - 127 + 15;
  if (half_exp >= 0x1f) return sign | 0x7c00u;
  if (half_exp <= 0) {
    if (14 - half_exp > 24) return sign;
    man |= 0x800000u;
    uint32_t shift = (uint32_t)(14 - half_exp);
    uint32_t half_man = man >> shift;
    uint32_t round_bit = 1u << (shift - 1);
    if ((man & round_bit) && (man & (3u * round_bit - 1u))) half_man++;
    return sign | half_man;
  }
  uint32_t r = sign | ((uint32_t)half_exp << 10);
  r += man >> 13;
  if ((man & 0x1000u) && (man & 0x2fffu)) r++;
  return r;
}

// exp and log used by every transcendental of the path (softmax, silu,
// sigmoid, softplus, the GDN decay).  Cody & Waite range reduction
// x = n ln2 + r (ln2 split in a 16-bit-exact high part and a low part), then the
// Taylor series of e^r to degree 7 (|r| <= ln2/2: truncation < 2^-27) and a
// two-step power-of-two scale (inputs below -87.33, whose results would be
// subnormal, give 0); log via m = 2^-e x in [sqrt(1/2), sqrt(2)),
// s = (m-1)/(m+1), log m = 2 atanh(s) (odd series to s^13).  Every step is an
// IEEE single operation with explicit fmaf, so the CPU checker evaluates the
// identical function bit for bit.  Accuracy ~1-2 ulp (tested against libm).
HH_DEV float hx_exp(float x_in) {
  // branch-free: the range cases are selected at the end, the polynomial runs
  // on the clamped argument (equal to x_in whenever its result is kept)
  const float x = fminf(fmaxf(x_in, -87.33f), 88.72f);
  float n = rintf(x * 1.44269504088896341f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.428606765330187e-06f, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  int n1 = ni / 2, n2 = ni - n1;
  float r_ = p * __uint_as_float((uint32_t)(127 + n1) << 23) * __uint_as_float((uint32_t)(127 + n2) << 23);
  r_ = x_in > 88.72f ? __uint_as_float(0x7f800000u) : r_;
  r_ = x_in < -87.33f ? 0.0f : r_;   // results below the normal range are flushed (both sides)
  return x_in != x_in ? x_in : r_;
}
HH_DEV float hx_log(float x) {
  if (!(x > 0.0f)) return x == 0.0f ? __uint_as_float(0xff800000u) : __uint_as_float(0x7fc00000u);
  if (x == __uint_as_float(0x7f800000u)) return x;
  uint32_t b = __float_as_uint(x);
  int e;
  if ((b >> 23) == 0) {  // subnormal: scale up by 2^23
    x = x * 8388608.0f;
    b = __float_as_uint(x);
    e = (int)(b >> 23) - 127 - 23;
  } else {
    e = (int)(b >> 23) - 127;
  }
  float m = __uint_as_float((b & 0x7fffffu) | 0x3f800000u);
  if (m > 1.41421356f) { m = m * 0.5f; e += 1; }
  float s = (m - 1.0f) / (m + 1.0f);
  float s2 = s * s;
  float p = 1.0f / 13.0f;
  p = fmaf(p, s2, 1.0f / 11.0f);
  p = fmaf(p, s2, 1.0f / 9.0f);
  p = fmaf(p, s2, 1.0f / 7.0f);
  p = fmaf(p, s2, 1.0f / 5.0f);
  p = fmaf(p, s2, 1.0f / 3.0f);
  p = fmaf(p, s2, 1.0f);
  float lm = (2.0f * s) * p;
  float fe = (float)e;
  return fmaf(fe, 0.693145751953125f, fmaf(fe, 1.428606765330187e-06f, lm));
}

// Position of element e (within the vector) in the permuted int8 array of a
// packed activation (the hand-off between kernels):
//   Q2: chunk of 16; element 4i+k -> k*4+i     (the bytes of (D >> 2k) & 0x03030303)
//   Q1: chunk of 32; element 8i+j -> j*4+i     (the bytes of (D >> j)  & 0x01010101)
//   PTQ1_0 and Q8_0: natural order (a PTQ1_0 slot covers consecutive elements)
// The GEMV stages Q2 and Q1 chunks in LDS as nibble words instead (put4 and
// packed_store in hh_gemv.hip); the grouping above makes that a few bit operations.
HH_DEV int perm_pos(int fmt, int e) {
  if (fmt == FMT_Q2) { int r = e & 15; return (e & ~15) | ((r & 3) << 2) | (r >> 2); }
  if (fmt == FMT_Q1) { int r = e & 31; return (e & ~31) | ((r & 7) << 2) | (r >> 3); }
  return e;
}
// Same, with the per-unit LDS padding applied.
HH_DEV int lds_qpos(int fmt, int e) {
  int p = perm_pos(fmt, e);
  if (fmt == FMT_Q8) return (p >> 6) * 80 + (p & 63);
  return (p >> 8) * 272 + (p & 255);
}

// Q8_0 quantization of one value given the block's f32 scale (q8_0.rs:44):
// (x / scale).round().clamp(-128, 127) as i8 ; NaN -> 0 as Rust's `as` does.
HH_DEV int q8_round(float x, float scale) {
  float v = roundf(x / scale);
  v = fminf(fmaxf(v, -128.0f), 127.0f);
  return (v != v) ? 0 : (int)v;
}
// q8_round with the block's reciprocal scale from v_rcp_f32 (<= 1 ulp):
// t = x * rcp is within 2^-15.3 of the correctly rounded x / scale for
// |x / scale| <= 127.5, so unless t lies within 2^-14 of a half-integer both
// round to the same integer.  Near a tie, and for non-finite t, the exact
// division decides.
HH_DEV int q8_round_r(float x, float scale, float rcp) {
  const float t = x * rcp;
  const float d = fabsf(fabsf(t - truncf(t)) - 0.5f);
  if (!(d >= 0x1p-14f)) return q8_round(x, scale);
  return (int)fminf(fmaxf(roundf(t), -128.0f), 127.0f);
}
HH_DEV float q8_rcp(float scale) { return __builtin_amdgcn_rcpf(scale); }
// q8_0.rs:35: scale = max_abs == 0 ? 1 : max_abs / 127.
HH_DEV float q8_scale(float amax) { return amax == 0.0f ? 1.0f : amax / 127.0f; }

// ---- wave helpers (wave64) ----
// Butterfly reductions run with ascending offsets 1, 2, 4, ..., 32.  Before
// the step at offset O every aligned group of O lanes holds one value, so the
// partner across bit O can be read with cheap lane permutes instead of LDS
// permutes: 1 and 2 are exact xor (DPP quad_perm), 4 and 8 mirror the 8- and
// 16-lane rows (DPP row_half_mirror / row_mirror: the mirrored lane lies in
// the partner group), 16 is a ds_swizzle xor within 32 lanes, and 32 reads
// lanes 0 and 32.  Callers keep the whole wave active.
template <int O> HH_DEV int bfly_xchg(int v) {
  if constexpr (O == 1) return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
  else if constexpr (O == 2) return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
  else if constexpr (O == 4) return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
  else if constexpr (O == 8) return __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
  else if constexpr (O == 16) return __builtin_amdgcn_ds_swizzle(v, 0x401F);
  else {
    static_assert(O == 32, "offset");
    int lo = __builtin_amdgcn_readlane(v, 0), hi = __builtin_amdgcn_readlane(v, 32);
    return (__lane_id() < 32) ? hi : lo;
  }
}
template <int O> HH_DEV float bfly_xchg(float v) { return __int_as_float(bfly_xchg<O>(__float_as_int(v))); }

// The value of lane (l ^ O), O a power of two: DPP within a 16-lane row for
// O <= 8 (quad_perm for 1 and 2, row_ror:8 for 8, row_shl:4 / row_shr:4 by the
// lane's bit 2 for 4), an LDS permute beyond.  The whole wave must be active.
template <int O> HH_DEV float xor_lane(float v) {
  const int x = __float_as_int(v);
  if constexpr (O == 1) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
  else if constexpr (O == 2) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
  else if constexpr (O == 4) {
    // banks 0 and 2 of each row (lane bit 2 clear) read lane + 4, then banks
    // 1 and 3 read lane - 4 over the first result
    const int up = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xF, 0x5, false);
    return __int_as_float(__builtin_amdgcn_update_dpp(up, x, 0x114, 0xF, 0xA, false));
  } else if constexpr (O == 8) return __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));
  else if constexpr (O == 16) {   // v_permlane16_swap(x, x): {rows 0,0,2,2 of x; rows 1,1,3,3 of x}
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
  } else {                        // O == 32: v_permlane32_swap(x, x): {low half twice; high half twice}
    static_assert(O == 32, "offset");
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
  }
}

// Reductions over aligned groups of W lanes (W power of two <= 64); every
// lane of a group ends with the group's value.
template <int W> HH_DEV float group_sum(float v) {
  if constexpr (W > 1) v = v + bfly_xchg<1>(v);
  if constexpr (W > 2) v = v + bfly_xchg<2>(v);
  if constexpr (W > 4) v = v + bfly_xchg<4>(v);
  if constexpr (W > 8) v = v + bfly_xchg<8>(v);
  if constexpr (W > 16) v = v + bfly_xchg<16>(v);
  if constexpr (W > 32) v = v + bfly_xchg<32>(v);
  return v;
}
template <int W> HH_DEV float group_max(float v) {
  if constexpr (W > 1) v = fmaxf(v, bfly_xchg<1>(v));
  if constexpr (W > 2) v = fmaxf(v, bfly_xchg<2>(v));
  if constexpr (W > 4) v = fmaxf(v, bfly_xchg<4>(v));
  if constexpr (W > 8) v = fmaxf(v, bfly_xchg<8>(v));
  if constexpr (W > 16) v = fmaxf(v, bfly_xchg<16>(v));
  if constexpr (W > 32) v = fmaxf(v, bfly_xchg<32>(v));
  return v;
}
template <int W> HH_DEV int group_sum_i(int v) {
  if constexpr (W > 1) v += bfly_xchg<1>(v);
  if constexpr (W > 2) v += bfly_xchg<2>(v);
  if constexpr (W > 4) v += bfly_xchg<4>(v);
  if constexpr (W > 8) v += bfly_xchg<8>(v);
  if constexpr (W > 16) v += bfly_xchg<16>(v);
  if constexpr (W > 32) v += bfly_xchg<32>(v);
  return v;
}
HH_DEV float wave_sum(float v) { return group_sum<64>(v); }
// lane i <- lane i + K within its 16-lane row (DPP row_shl); lanes whose
// source falls outside the row get 0
template <int K> HH_DEV float dpp_from_lane_plus(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 | K, 0xF, 0xF, false));
}
HH_DEV float wave_max(float v) { return group_max<64>(v); }
// wave_max for values that hold no NaN (softmax scores, -inf allowed): a
// plain v_max_f32 per level, where fmaxf (and the med3 form, which the
// compiler folds back into it) also quiets both operands first.
HH_DEV float vmax_nonan(float a, float b) {
  float r;
  asm("v_max_f32_e32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
HH_DEV float wave_max_nonan(float v) {
  v = vmax_nonan(v, bfly_xchg<1>(v));
  v = vmax_nonan(v, bfly_xchg<2>(v));
  v = vmax_nonan(v, bfly_xchg<4>(v));
  v = vmax_nonan(v, bfly_xchg<8>(v));
  v = vmax_nonan(v, bfly_xchg<16>(v));
  v = vmax_nonan(v, bfly_xchg<32>(v));
  return v;
}

// Pairwise tree over 16 values (the wave sums of a 1024-slot reduction).
HH_DEV float tree16(const float* v) {
  float a0 = (v[0] + v[1]) + (v[2] + v[3]), a1 = (v[4] + v[5]) + (v[6] + v[7]);
  float a2 = (v[8] + v[9]) + (v[10] + v[11]), a3 = (v[12] + v[13]) + (v[14] + v[15]);
  return (a0 + a1) + (a2 + a3);
}

// Sum of squares of a K-vector (K % 1024 == 0) in the fixed order every
// full-width RMSNorm of the path uses: 1024 slots, slot t summing the float4s
// x[4t + 4096c .. +3] in c order as ss + (((x0^2 + x1^2) + x2^2) + x3^2);
// slots 64w .. 64w+63 reduce by wave_sum into W_w; the total is tree16(W).
// A 256-lane workgroup runs slots t, t+256, t+512, t+768 in lane t.
// red16: 16 floats of LDS.
HH_DEV float block_sumsq_f4(const float* __restrict__ x, int K, float* red16) {
  const int tid = threadIdx.x;
  float ss[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    ss[j] = 0.0f;
    for (int e = (tid + 256 * j) * 4; e < K; e += 4096) {
      float4 v = *(const float4*)(x + e);
      ss[j] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) ss[j] = wave_sum(ss[j]);
  if ((tid & 63) == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) red16[(tid >> 6) + 4 * j] = ss[j];
  }
  __syncthreads();
  return tree16(red16);
}

// ---- Hadamard fold (qwen35.rs:51-118) ----
// Normalized Sylvester Walsh-Hadamard transform of every `blk`-element chunk
// of x[K] (K % blk == 0) in LDS, by all NTH lanes of the workgroup:
// butterflies h = 1, 2, 4, ..., blk/2 with x[i] = a + b, x[i + h] = a - b for
// every i with bit h clear, then x *= 1/sqrt(blk).  Each output is the same
// sequence of IEEE additions as the reference's in-place loop, so the result
// is bit-identical.  Starts and ends with a workgroup barrier.
template <int NTH> HH_DEV void lds_wht(float* x, int K, int blk) {
  const int tid = threadIdx.x;
  for (int h = 1; h < blk; h <<= 1) {
    __syncthreads();
    for (int p = tid; p < K / 2; p += NTH) {
      const int i = ((p & ~(h - 1)) << 1) | (p & (h - 1));
      const float a = x[i], b = x[i + h];
      x[i] = a + b;
      x[i + h] = a - b;
    }
  }
  __syncthreads();
  const float sc = 1.0f / sqrtf((float)blk);
  for (int i = tid; i < K; i += NTH) x[i] = x[i] * sc;
  __syncthreads();
}

// mod.rs:483-504: element i of the dequantized token_embd row of token tok.
HH_DEV float embed_value(int type, const uint8_t* __restrict__ table, int d, int tok, int i) {
  if (type == 8) {
    const uint8_t* blk = table + (size_t)tok * (d / 32) * 34 + (size_t)(i / 32) * 34;
    return h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8)) * (float)(int8_t)blk[2 + (i % 32)];
  } else if (type == 42 || type == 142) {
    const uint8_t* blk = table + (size_t)tok * (d / 128) * 34 + (size_t)(i / 128) * 34;
    int e = i % 128;
    int code = (blk[2 + e / 4] >> (2 * (e % 4))) & 3;
    return (float)(code - 1) * h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
  }
  const uint8_t* blk = table + (size_t)tok * (d / 128) * 18 + (size_t)(i / 128) * 18;
  int e = i % 128;
  int bit = (blk[2 + e / 8] >> (e % 8)) & 1;
  return (float)(bit ? 1 : -1) * h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
}

// A latent (Hadamard-folded) embedding row gets R^-1 = H D after the lookup
// (qwen35.rs:1054-1066, hadamard_unrotate :98-110): the WHT per had_block chunk,
// then the sign pass.  buf: d floats of LDS.
// NTH: the workgroup's lane count (all lanes call this; the latent path has barriers).
template <int NTH>
HH_DEV void embed_row(int type, const uint8_t* __restrict__ table, int d, int tok, float* __restrict__ out,
                      const float* __restrict__ signs, int had_block, float* buf) {
  if (had_block <= 0) {
    for (int i = threadIdx.x; i < d; i += NTH) out[i] = embed_value(type, table, d, tok, i);
    return;
  }
  for (int i = threadIdx.x; i < d; i += NTH) buf[i] = embed_value(type, table, d, tok, i);
  lds_wht<NTH>(buf, d, had_block);
  for (int i = threadIdx.x; i < d; i += NTH) out[i] = buf[i] * signs[i];
}

// Slot of element e of a GDN head-major vector in the grouped order the
// ssm_out fold was computed in (qwen35.rs:1452-1478): head h = r * nk + kg
// moves to head slot kg * rep + r.
HH_DEV int grouped_pos(int e, int hd, int nk, int rep) {
  const int h = e / hd;
  return ((h % nk) * rep + h / nk) * hd + (e - h * hd);
}

// ---- counter-based seeded generator (shared definition with the CPU checker) ----
HH_DEV uint64_t mix64(uint64_t x) {
  x ^= x >> 30;
  x *= 0xbf58476d1ce4e5b9ull;
  x ^= x >> 27;
  x *= 0x94d049bb133111ebull;
  x ^= x >> 31;
  return x;
}
HH_DEV int32_t synth_int(uint64_t key, uint64_t idx) {
  uint64_t h = mix64(key + idx * 0x9e3779b97f4a7c15ull);
  int32_t s = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) + (int32_t)((h >> 32) & 0xffff) +
              (int32_t)(h >> 48);
  return s - 131070;
}

// Device-side step state: the token loop runs without host round trips.
// The 8 ints of the step state, lane l holding int l & 7: one vector load.
// Its fields are taken with readlane where used.  A scalar load of the state
// would be waited for together with the kernel-argument loads that the first
// vector loads' addresses need (scalar loads return out of order, so that wait
// is lgkmcnt(0)), putting the state's round trip ahead of them.
HH_DEV int state_lanes(const void* st) { return ((const int*)st)[threadIdx.x & 7]; }

// Positions per attention split (one workgroup per chunk and kv head): 8192 /
// hd, or twice that once the chunks of all kv heads at that width would
// outnumber MI355X's 256 CUs.  Past that count the last workgroups share a CU
// with another and finish late, and wider chunks take fewer barriers per
// position; below it the narrow chunk keeps more workgroups busy.  8B decode
// step, narrow only -> this rule: 1k context 1.387 -> 1.391 ms, 2k 1.497 ->
// 1.490, 4k 1.679 -> 1.616, 8k 2.007 -> 1.886.
__host__ __device__ inline int attn_chunk_for(int seq, int hd, int n_kv) {
  const int c = 8192 / hd;
  return (long long)((seq + c - 1) / c) * n_kv > 256 ? 2 * c : c;
}

struct StepState {
  int pos;        // position of the token being fed
  int step;       // steps executed in this session
  int token;      // token being fed
  int n_prompt;   // prompt length (steps < n_prompt-1 take the next prompt token)
  int update;     // 1: record argmax + repetition counts (generate), 0: forward only
  int argmax;     // last greedy choice
  int cancel;     // host-set cancel flag
  float pen;      // repetition penalty for the dense greedy rule
};
static_assert(sizeof(StepState) == 32 && offsetof(StepState, step) == 4 && offsetof(StepState, n_prompt) == 12 &&
                  offsetof(StepState, pen) == 28,
              "state_lanes readers take ints 1, 3 and 7");
