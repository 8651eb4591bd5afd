/*
 * hearth_oracle.c — CPU restatement of Hearth's batch-1 decode path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP library and the
 * "port" CPU baseline.  The product (hearth_amd/) never links or calls it.
 *
 * Compiled with -ffp-contract=off so that every a*b+c below is two roundings,
 * as in the reference's scalar Rust code; the places where the reference uses
 * an explicit fused multiply-add (wide::f32x8::mul_add, _mm256_fmadd_ps) call
 * fmaf() here.
 *
 * Citations are "file:line" in the Hearth repository.
 *
 * Parity pins (what checks each function, besides the GPU comparison):
 *   ho_f32_to_f16       numpy float16 (IEEE RNE) over ~10^6 values + specials
 *   ho_quantize_q8_0    hand-computed known answers (zero block -> 0x3C00,
 *                       max 127 -> scale 1.0), q8_0.rs:177-212 tests, numpy
 *   ho_dequantize       q2_0.rs:738-766, pq2_0.rs:79-93, q2_0.rs:913-934,
 *                       q1_0g128.rs:1459-1502 known answers
 *   dots                brute-force dequant-then-dot, generator fixtures of
 *                       q2_0.rs:939-986 / q1_0g128.rs:1504-1551
 *   rms_norm/rope/...   invariants (unit RMS, norm-preserving rotation, softmax
 *                       sums to 1) and tiny brute force in numpy
 *   forward/generate    composition of the above; token-level parity unpinned
 *                       against the Rust binary (no rustc in this image)
 */
#include "hearth_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* f16 <-> f32 (half 2.7.1 semantics: IEEE binary16, round-to-nearest-even)  */
/* ------------------------------------------------------------------------- */

uint16_t ho_f32_to_f16(float xf) {
  uint32_t x;
  memcpy(&x, &xf, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) {
    if (man) return (uint16_t)(sign | 0x7e00u | (man >> 13));
    return (uint16_t)(sign | 0x7c00u);
  }
  int half_exp = (int)exp - 127 + 15;
  if (half_exp >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (half_exp <= 0) {
    if (14 - half_exp > 24) return (uint16_t)sign;
    man |= 0x800000u;
    uint32_t shift = (uint32_t)(14 - half_exp);
    uint32_t half_man = man >> shift;
    uint32_t round_bit = 1u << (shift - 1);
    if ((man & round_bit) && (man & (3u * round_bit - 1u))) half_man++;
    return (uint16_t)(sign | half_man);
  }
  uint32_t half_man = man >> 13;
  uint32_t round_bit = 0x1000u;
  uint32_t r = sign | ((uint32_t)half_exp << 10);
  r += half_man;
  if ((man & round_bit) && (man & (3u * round_bit - 1u))) r++;
  return (uint16_t)r;
}

float ho_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t man = (uint32_t)h & 0x3ffu;
  uint32_t out;
  if (exp == 0) {
    if (man == 0) {
      out = sign;
    } else {
      int e = -1;
      do { e++; man <<= 1; } while ((man & 0x400u) == 0);
      out = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
    }
  } else if (exp == 0x1f) {
    out = sign | 0x7f800000u | (man << 13);
  } else {
    out = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}

/* exp / log shared with the device kernels (hearth_amd/csrc/hh_device.h):
 * Cody & Waite reduction x = n ln2 + r with ln2 = 0.693145751953125 +
 * 1.428606765330187e-06, Taylor series of e^r to degree 7, power-of-two scale
 * in two steps; log m (m in [sqrt(1/2), sqrt(2))) = 2 atanh((m-1)/(m+1)) to the
 * s^13 term.  The reference's own exp is wide::f32x8::exp (a polynomial in the
 * `wide` crate, used by ops.rs:246/:284/:331) and Rust f32::exp/ln elsewhere;
 * neither is reproducible bit for bit here (parity unpinned at the ulp level),
 * so both implementations of this path evaluate this one function. */
float ho_exp(float x) {
  if (x != x) return x;
  if (x > 88.72f) return INFINITY;
  if (x < -87.33f) return 0.0f;
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
  uint32_t b1 = (uint32_t)(127 + n1) << 23, b2 = (uint32_t)(127 + n2) << 23;
  float f1, f2;
  memcpy(&f1, &b1, 4);
  memcpy(&f2, &b2, 4);
  return p * f1 * f2;
}

float ho_log(float x) {
  if (!(x > 0.0f)) return x == 0.0f ? -INFINITY : NAN;
  if (isinf(x)) return x;
  uint32_t b;
  memcpy(&b, &x, 4);
  int e;
  if ((b >> 23) == 0) {
    x = x * 8388608.0f;
    memcpy(&b, &x, 4);
    e = (int)(b >> 23) - 127 - 23;
  } else {
    e = (int)(b >> 23) - 127;
  }
  uint32_t mb = (b & 0x7fffffu) | 0x3f800000u;
  float m;
  memcpy(&m, &mb, 4);
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

/* ho_f16_to_f32 of every half, tabulated once (the dots read a scale per block) */
static float f16tab[65536];
__attribute__((constructor)) static void init_f16tab(void) {
  for (uint32_t h = 0; h < 65536; h++) f16tab[h] = ho_f16_to_f32((uint16_t)h);
}
static inline float rd_f16(const uint8_t* p) { return f16tab[p[0] | (p[1] << 8)]; }

/* ------------------------------------------------------------------------- */
/* formats                                                                   */
/* ------------------------------------------------------------------------- */

/* ggml.rs:105-171: block sizes and bytes. */
size_t ho_row_bytes(int type, int64_t n) {
  switch (type) {
    case HO_F32: return (size_t)n * 4;
    case HO_F16: return (size_t)n * 2;
    case HO_Q8_0: return (size_t)(n / 32) * 34;
    case HO_Q1_0:
    case HO_Q1_0_G128: return (size_t)(n / 128) * 18;
    case HO_Q2_0:
    case HO_PQ2_0: return (size_t)(n / 128) * 34;
    case HO_PTQ1_0: return (size_t)(n / 128) * 28;
    default: return 0;
  }
}

/* Rust `f32 as i8` after clamp(-128,127): saturating, NaN -> 0. */
static inline int8_t sat_i8(float v) {
  if (v != v) return 0;
  return (int8_t)(int)v;
}

/* q8_0.rs:20-51 quantize_into. */
void ho_quantize_q8_0(const float* src, int64_t n, uint8_t* dst) {
  int64_t blocks = (n + 31) / 32;
  for (int64_t b = 0; b < blocks; b++) {
    int64_t start = b * 32;
    float max_abs = 0.0f;
    for (int i = 0; i < 32; i++) {
      int64_t idx = start + i;
      if (idx < n) {
        float v = fabsf(src[idx]);
        if (v > max_abs) max_abs = v;
      }
    }
    float scale = (max_abs == 0.0f) ? 1.0f : max_abs / 127.0f;
    uint16_t h = ho_f32_to_f16(scale);
    uint8_t* o = dst + b * 34;
    o[0] = (uint8_t)(h & 0xff);
    o[1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; i++) {
      int64_t idx = start + i;
      int8_t q = 0;
      if (idx < n) {
        float v = roundf(src[idx] / scale);
        if (v < -128.0f) v = -128.0f;
        if (v > 127.0f) v = 127.0f;
        q = sat_i8(v);
      }
      o[2 + i] = (uint8_t)q;
    }
  }
}

/* PTQ1_0 (ptq1_0.rs:1-13, :72-110).  Trit n of a packed byte: the byte is
 * ceil(256*Q/243) for Q = sum t_k 3^(4-k), and b*3^n mod 256 keeps the fraction
 * Q*3^n/243 mod 1 to within the rounding, so ((b*3^n mod 256)*3) >> 8 is t_n. */
static inline int ptq_trit(unsigned b, int n) {
  static const unsigned p3[5] = {1, 3, 9, 27, 81};
  return (int)((((b * p3[n]) & 0xffu) * 3u) >> 8);
}
/* Position in the block of element (stage byte m, slot n) and of qh trits:
 * stage A = bytes 0..15 -> 16n + m; stage B = bytes 16..23 -> 80 + 8n + (m-16);
 * qh byte h (0,1), slot n < 4 -> 120 + 2n + h. */
static void ptq_block_trits(const uint8_t* blk, int8_t* t /* 128 weights in {-1,0,1} */) {
  for (int m = 0; m < 24; m++)
    for (int n = 0; n < 5; n++) {
      int e = m < 16 ? 16 * n + m : 80 + 8 * n + (m - 16);
      t[e] = (int8_t)(ptq_trit(blk[m], n) - 1);
    }
  for (int h = 0; h < 2; h++)
    for (int n = 0; n < 4; n++) t[120 + 2 * n + h] = (int8_t)(ptq_trit(blk[24 + h], n) - 1);
}

/* ptq1_0.rs:604-643 quantize (ternary round of x/amax, base-3 pack, ceil to the
 * 256/243 grid; the qh byte carries 4 trits and a trailing zero). */
void ho_quantize_ptq1_0(const float* src, int64_t n, uint8_t* dst) {
  int64_t blocks = n / 128;
  for (int64_t b = 0; b < blocks; b++) {
    const float* x = src + b * 128;
    float amax = 0.0f;
    for (int i = 0; i < 128; i++) amax = fmaxf(amax, fabsf(x[i]));
    float d = amax, id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t* o = dst + b * 28;
    memset(o, 0, 28);
    uint16_t h = ho_f32_to_f16(d);
    o[26] = (uint8_t)(h & 0xff);
    o[27] = (uint8_t)(h >> 8);
    for (int m = 0; m < 24; m++) {
      unsigned q = 0;
      for (int nn = 0; nn < 5; nn++) {
        int e = m < 16 ? 16 * nn + m : 80 + 8 * nn + (m - 16);
        int xi = (int)roundf(x[e] * id) + 1;
        q = (q * 3u + (unsigned)xi) & 0xffu;
      }
      o[m] = (uint8_t)((q * 256u + 242u) / 243u);
    }
    for (int hh = 0; hh < 2; hh++) {
      unsigned q = 0;
      for (int mm = 0; mm < 4; mm++) {
        int xi = (int)roundf(x[120 + hh + 2 * mm] * id) + 1;
        q = (q * 3u + (unsigned)xi) & 0xffu;
      }
      q = (q * 3u) & 0xffu;
      o[24 + hh] = (uint8_t)((q * 256u + 242u) / 243u);
    }
  }
}

/* q8_0.rs:4-18, q2_0.rs:66-84 (pq2_0.rs:32-50 same bytes), q1_0g128.rs:75-98. */
int ho_dequantize(int type, const uint8_t* w, int64_t n, float* out) {
  switch (type) {
    case HO_F32: memcpy(out, w, (size_t)n * 4); return 0;
    case HO_F16:
      for (int64_t i = 0; i < n; i++) out[i] = rd_f16(w + 2 * i);
      return 0;
    case HO_Q8_0:
      for (int64_t i = 0; i < n; i++) {
        const uint8_t* blk = w + (i / 32) * 34;
        out[i] = rd_f16(blk) * (float)(int8_t)blk[2 + (i % 32)];
      }
      return 0;
    case HO_Q2_0:
    case HO_PQ2_0:
      for (int64_t i = 0; i < n; i++) {
        const uint8_t* blk = w + (i / 128) * 34;
        int e = (int)(i % 128);
        int code = (blk[2 + e / 4] >> (2 * (e % 4))) & 3;
        out[i] = (float)(code - 1) * rd_f16(blk);
      }
      return 0;
    case HO_Q1_0:
    case HO_Q1_0_G128:
      for (int64_t i = 0; i < n; i++) {
        const uint8_t* blk = w + (i / 128) * 18;
        int e = (int)(i % 128);
        int bit = (blk[2 + e / 8] >> (e % 8)) & 1;
        out[i] = (float)(bit ? 1 : -1) * rd_f16(blk);
      }
      return 0;
    case HO_PTQ1_0:   /* ptq1_0.rs:72-110 */
      for (int64_t b = 0; b < n / 128; b++) {
        int8_t t[128];
        const uint8_t* blk = w + b * 28;
        ptq_block_trits(blk, t);
        float d = rd_f16(blk + 26);
        for (int e = 0; e < 128; e++) out[b * 128 + e] = (float)t[e] * d;
      }
      return 0;
    default: return 1;
  }
}

/* ------------------------------------------------------------------------- */
/* dot kernels                                                               */
/* ------------------------------------------------------------------------- */

/* Exact int32 sub-block dots (32 elements) for the scalar-order kernels below.
 * The integer sum is exact in any order, so it is computed with AVX2 byte
 * multiply-adds from per-byte expansion tables; only the fp32 combine above it
 * has to follow the reference's order.  q2lut[b] = the four 2-bit codes of byte
 * b as bytes (LSB first); q1lut[b] = the eight bits of b as 0/1 bytes. */
static uint32_t q2lut[256];
static uint64_t q1lut[256];
__attribute__((constructor)) static void init_luts(void) {
  for (int b = 0; b < 256; b++) {
    uint32_t v = 0;
    for (int k = 0; k < 4; k++) v |= (uint32_t)((b >> (2 * k)) & 3) << (8 * k);
    q2lut[b] = v;
    uint64_t u = 0;
    for (int k = 0; k < 8; k++) u |= (uint64_t)((b >> k) & 1) << (8 * k);
    q1lut[b] = u;
  }
}
static inline int32_t hsum_i32x8(__m256i v) {
  __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
  s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
  return _mm_cvtsi128_si32(s);
}
/* The four exact sub-block dots of one 128-element block at once (the integer
 * sums do not depend on the order): out[s] = sum (code - 1) * a over sub-block
 * s, codes widened through the byte tables by a gather, the four 8-lane
 * partial vectors reduced together by horizontal adds. */
static inline void block_reduce4(const __m256i* v, int32_t* out) {
  __m256i h01 = _mm256_hadd_epi32(v[0], v[1]);
  __m256i h23 = _mm256_hadd_epi32(v[2], v[3]);
  __m256i h = _mm256_hadd_epi32(h01, h23);
  _mm_storeu_si128((__m128i*)out, _mm_add_epi32(_mm256_castsi256_si128(h), _mm256_extracti128_si256(h, 1)));
}
static inline __m256i sub_partial(__m256i u, const uint8_t* ab) {
  const __m256i ones8 = _mm256_set1_epi8(1), ones16 = _mm256_set1_epi16(1);
  __m256i av = _mm256_loadu_si256((const __m256i*)(ab + 2));
  return _mm256_sub_epi32(_mm256_madd_epi16(_mm256_maddubs_epi16(u, av), ones16),
                          _mm256_madd_epi16(_mm256_maddubs_epi16(ones8, av), ones16));
}
static inline void block_dots_q2(const uint8_t* qs, const uint8_t* ab, int32_t* out) {
  __m256i v[4];
  for (int sub = 0; sub < 4; sub++) {
    __m256i idx = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)(qs + 8 * sub)));
    v[sub] = sub_partial(_mm256_i32gather_epi32((const int*)q2lut, idx, 4), ab + sub * 34);
  }
  block_reduce4(v, out);
}
static inline void block_dots_q1(const uint8_t* bits, const uint8_t* ab, int32_t* out) {
  __m256i v[4];
  for (int sub = 0; sub < 4; sub++) {
    __m128i idx = _mm_cvtepu8_epi32(_mm_cvtsi32_si128(*(const int*)(bits + 4 * sub)));
    __m256i u = _mm256_i32gather_epi64((const long long*)q1lut, idx, 8);
    v[sub] = sub_partial(_mm256_add_epi8(u, u), ab + sub * 34);
  }
  block_reduce4(v, out);
}

/* q2_0.rs:537-574 scalar Q2_0 x Q8_0. */
float ho_dot_q2_0_q8_0(const uint8_t* w, const uint8_t* a, int64_t n) {
  int64_t blocks = n / 128;
  float sum = 0.0f;
  for (int64_t b = 0; b < blocks; b++) {
    const uint8_t* wb = w + b * 34;
    float w_scale = rd_f16(wb);
    const uint8_t* qs = wb + 2;
    float block_acc = 0.0f;
    int32_t dots[4];
    block_dots_q2(qs, a + b * 4 * 34, dots);   /* sum (code - 1) * a per sub-block, exact */
    for (int sub = 0; sub < 4; sub++) {
      float a_scale = rd_f16(a + (b * 4 + sub) * 34);
      block_acc += (float)dots[sub] * a_scale;
    }
    sum += block_acc * w_scale;
  }
  return sum;
}

/* ptq1_0.rs:555-602 scalar PTQ1_0 x Q8_0: per 32-element sub-block an exact
 * int dot, block_acc += dot * d_a, sum += block_acc * d (the Q2_0 structure). */
float ho_dot_ptq1_0_q8_0(const uint8_t* w, const uint8_t* a, int64_t n) {
  int64_t blocks = n / 128;
  float sum = 0.0f;
  for (int64_t b = 0; b < blocks; b++) {
    const uint8_t* wb = w + b * 28;
    int8_t t[128];
    ptq_block_trits(wb, t);
    float block_acc = 0.0f;
    for (int sub = 0; sub < 4; sub++) {
      const uint8_t* ab = a + (b * 4 + sub) * 34;
      float a_scale = rd_f16(ab);
      const int8_t* av = (const int8_t*)(ab + 2);
      int32_t dot = 0;
      for (int i = 0; i < 32; i++) dot += (int32_t)t[sub * 32 + i] * (int32_t)av[i];
      block_acc += (float)dot * a_scale;
    }
    sum += block_acc * rd_f16(wb + 26);
  }
  return sum;
}

/* q1_0g128.rs:1113-1152 scalar Q1_0_G128 x Q8_0. */
float ho_dot_q1_0_q8_0(const uint8_t* w, const uint8_t* a, int64_t n) {
  int64_t blocks = n / 128;
  float sum = 0.0f;
  for (int64_t b = 0; b < blocks; b++) {
    const uint8_t* wb = w + b * 18;
    float w_scale = rd_f16(wb);
    const uint8_t* bits = wb + 2;
    float block_acc = 0.0f;
    int32_t dots[4];
    block_dots_q1(bits, a + b * 4 * 34, dots);   /* sum (bit ? 1 : -1) * a per sub-block, exact */
    for (int sub = 0; sub < 4; sub++) {
      float a_scale = rd_f16(a + (b * 4 + sub) * 34);
      block_acc += (float)dots[sub] * a_scale;
    }
    sum += block_acc * w_scale;
  }
  return sum;
}

/* q8_0.rs:154-171 Q8_0 x Q8_0. */
float ho_dot_q8_0_q8_0(const uint8_t* w, const uint8_t* a, int64_t n) {
  int64_t blocks = n / 32;
  float sumf = 0.0f;
  for (int64_t b = 0; b < blocks; b++) {
    float d0 = rd_f16(w + b * 34);
    float d1 = rd_f16(a + b * 34);
    const int8_t* wv = (const int8_t*)(w + b * 34 + 2);
    const int8_t* av = (const int8_t*)(a + b * 34 + 2);
    /* exact int32 sum of the 32 products (int8 widened to int16, then madd) */
    __m256i w0 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)wv));
    __m256i w1 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(wv + 16)));
    __m256i a0 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)av));
    __m256i a1 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(av + 16)));
    int32_t sumi = hsum_i32x8(_mm256_add_epi32(_mm256_madd_epi16(w0, a0), _mm256_madd_epi16(w1, a1)));
    sumf += (float)sumi * d0 * d1;
  }
  return sumf;
}

int ho_have_avx2(void) {
  __builtin_cpu_init();
  return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

__attribute__((target("avx2,fma,f16c"))) static float hsum8(__m256 v) {
  __m128 lo = _mm256_castps256_ps128(v);
  __m128 hi = _mm256_extractf128_ps(v, 1);
  __m128 s = _mm_add_ps(lo, hi);
  s = _mm_add_ps(s, _mm_movehl_ps(s, s));
  s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
  return _mm_cvtss_f32(s);
}

/* The i16 code table of q2_0.rs:26-40 (Q2V_I16): code byte -> 4 x (code-1). */
static int16_t g_q2v_i16[256][4];
static void init_q2v(void) {
  static int done = 0;
  if (done) return;
  for (int b = 0; b < 256; b++)
    for (int j = 0; j < 4; j++) g_q2v_i16[b][j] = (int16_t)(((b >> (2 * j)) & 3) - 1);
  done = 1;
}

/* q2_0.rs:308-392: AVX2 LUT arm (the arm Hearth dispatches on AVX2 hosts). */
__attribute__((target("avx2,fma,f16c")))
float ho_dot_q2_0_q8_0_avx2(const uint8_t* w, const uint8_t* a, int64_t n) {
  init_q2v();
  int64_t blocks = n / 128;
  __m256 acc_global = _mm256_setzero_ps();
  for (int64_t b = 0; b < blocks; b++) {
    const uint8_t* wb = w + b * 34;
    __m256 w_scale = _mm256_set1_ps(rd_f16(wb));
    const uint8_t* qs = wb + 2;
    __m256 acc_block = _mm256_setzero_ps();
    for (int sub = 0; sub < 4; sub++) {
      const uint8_t* ab = a + (b * 4 + sub) * 34;
      __m256 a_scale = _mm256_set1_ps(rd_f16(ab));
      const uint8_t* av = ab + 2;
      const uint8_t* qsub = qs + sub * 8;
      __m256i acc = _mm256_setzero_si256();
      for (int half = 0; half < 2; half++) {
        __m256i a16 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i*)(av + 16 * half)));
        int16_t wbuf[16];
        for (int k = 0; k < 4; k++) memcpy(wbuf + 4 * k, g_q2v_i16[qsub[4 * half + k]], 8);
        __m256i s = _mm256_loadu_si256((const __m256i*)wbuf);
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(a16, s));
      }
      acc_block = _mm256_fmadd_ps(a_scale, _mm256_cvtepi32_ps(acc), acc_block);
    }
    acc_global = _mm256_fmadd_ps(w_scale, acc_block, acc_global);
  }
  return hsum8(acc_global);
}

/* q1_0g128.rs:255-377: AVX2 shuffle arm (sign expansion + maddubs). */
__attribute__((target("avx2,fma,f16c")))
float ho_dot_q1_0_q8_0_avx2(const uint8_t* w, const uint8_t* a, int64_t n) {
  int64_t blocks = n / 128;
  const __m256i ones_8 = _mm256_set1_epi8(1);
  const __m256i ones_16 = _mm256_set1_epi16(1);
  const __m256i zero = _mm256_setzero_si256();
  const __m256i byte_shuf = _mm256_setr_epi8(0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 1, 1, 1, 2, 2,
                                             2, 2, 2, 2, 2, 2, 3, 3, 3, 3, 3, 3, 3, 3);
  const __m256i bit_masks = _mm256_setr_epi8(1, 2, 4, 8, 16, 32, 64, -128, 1, 2, 4, 8, 16, 32, 64,
                                             -128, 1, 2, 4, 8, 16, 32, 64, -128, 1, 2, 4, 8, 16,
                                             32, 64, -128);
  __m256 acc = _mm256_setzero_ps();
  for (int64_t b = 0; b < blocks; b++) {
    const uint8_t* wb = w + b * 18;
    float w_scale = rd_f16(wb);
    __m256 acc_block = _mm256_setzero_ps();
    for (int k = 0; k < 4; k++) {
      uint32_t qsk;
      memcpy(&qsk, wb + 2 + 4 * k, 4);
      const uint8_t* ab = a + (b * 4 + k) * 34;
      float a_scale = rd_f16(ab);
      __m256i qy = _mm256_loadu_si256((const __m256i*)(ab + 2));
      __m256i sm = _mm256_cmpeq_epi8(
          _mm256_and_si256(_mm256_shuffle_epi8(_mm256_set1_epi32((int)qsk), byte_shuf), bit_masks),
          zero);
      __m256i sy = _mm256_sub_epi8(_mm256_xor_si256(qy, sm), sm);
      __m256i s32 = _mm256_madd_epi16(_mm256_maddubs_epi16(ones_8, sy), ones_16);
      acc_block = _mm256_fmadd_ps(_mm256_set1_ps(a_scale), _mm256_cvtepi32_ps(s32), acc_block);
    }
    acc = _mm256_fmadd_ps(_mm256_set1_ps(w_scale), acc_block, acc);
  }
  return hsum8(acc);
}

typedef float (*dot_fn)(const uint8_t*, const uint8_t*, int64_t);

static dot_fn pick_dot(int type, int arm) {
  int avx = arm && ho_have_avx2();
  switch (type) {
    case HO_Q2_0:
    case HO_PQ2_0: return avx ? ho_dot_q2_0_q8_0_avx2 : ho_dot_q2_0_q8_0;
    case HO_Q1_0:
    case HO_Q1_0_G128: return avx ? ho_dot_q1_0_q8_0_avx2 : ho_dot_q1_0_q8_0;
    case HO_Q8_0: return ho_dot_q8_0_q8_0;
    case HO_PTQ1_0: return ho_dot_ptq1_0_q8_0;
    default: return NULL;
  }
}

/* pool.rs:510-566 par_dot_rows: worker i owns rows [i*chunk, min(N,(i+1)*chunk)),
 * chunk = ceil(N/T) (pool.rs:321-323). */
int ho_gemv(int type, const uint8_t* w, int64_t n_rows, int64_t n_cols, const uint8_t* a,
            float* y, int n_threads, int arm) {
  dot_fn f = pick_dot(type, arm);
  if (!f) return 1;
  size_t rb = ho_row_bytes(type, n_cols);
  if (n_threads < 1) n_threads = 1;
  int64_t chunk = (n_rows + n_threads - 1) / n_threads;
#pragma omp parallel for num_threads(n_threads) schedule(static, 1)
  for (int t = 0; t < n_threads; t++) {
    int64_t r0 = (int64_t)t * chunk, r1 = r0 + chunk;
    if (r1 > n_rows) r1 = n_rows;
    for (int64_t r = r0; r < r1; r++) y[r] = f(w + (size_t)r * rb, a, n_cols);
  }
  return 0;
}

/* ------------------------------------------------------------------------- */
/* f32 ops (ops.rs)                                                          */
/* ------------------------------------------------------------------------- */

/* wide::f32x8::reduce_add lane order: ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)). */
static float reduce8(const float* l) {
  float s0 = l[0] + l[4], s1 = l[1] + l[5], s2 = l[2] + l[6], s3 = l[3] + l[7];
  float t0 = s0 + s2, t1 = s1 + s3;
  return t0 + t1;
}

/* ops.rs:8-35 rms_norm: 8-lane FMA sum of squares, out = (x * inv) * w. */
void ho_rms_norm(const float* x, const float* w, float eps, int64_t n, float* out) {
  float lanes[8] = {0};
  int64_t chunks = n / 8, rem = n % 8;
  for (int64_t i = 0; i < chunks; i++)
    for (int l = 0; l < 8; l++) lanes[l] = fmaf(x[i * 8 + l], x[i * 8 + l], lanes[l]);
  float sum_sq = 0.0f + reduce8(lanes);
  for (int64_t i = n - rem; i < n; i++) sum_sq += x[i] * x[i];
  float rms = sqrtf(sum_sq / (float)n + eps);
  float inv = 1.0f / rms;
  for (int64_t i = 0; i < chunks * 8; i++) out[i] = x[i] * inv * w[i];
  for (int64_t i = n - rem; i < n; i++) out[i] = w[i] * x[i] * inv;
}

/* ops.rs:78-138 RopeCache::new (no scaling): table[pos][0..half) = sin,
 * table[pos][half..2half) = cos, freq = pos * inv_freq[i]. */
void ho_rope_table(int max_seq, int rope_dim, float theta, float* table) {
  int half = rope_dim / 2;
  float* inv_freq = (float*)malloc(sizeof(float) * (size_t)half);
  for (int i = 0; i < half; i++)
    inv_freq[i] = 1.0f / powf(theta, 2.0f * (float)i / (float)rope_dim);
  for (int pos = 0; pos < max_seq; pos++) {
    for (int i = 0; i < half; i++) {
      float freq = (float)pos * 1.0f * inv_freq[i];
      float* base = table + (size_t)pos * half * 2;
      base[i] = sinf(freq);
      base[half + i] = cosf(freq);
    }
  }
  free(inv_freq);
}

/* ops.rs:140-164 RopeCache::apply: NeoX halves. */
void ho_rope_apply(const float* table, int max_seq, int rope_dim, float* x, int pos) {
  int half = rope_dim / 2;
  const float* base = table + (size_t)(pos % max_seq) * half * 2;
  for (int i = 0; i < half; i++) {
    float s = base[i], c = base[half + i];
    float x0 = x[i], x1 = x[i + half];
    x[i] = x0 * c - x1 * s;
    x[i + half] = x0 * s + x1 * c;
  }
}

/* ops.rs:240-253 silu. */
void ho_silu(float* x, int64_t n) {
  for (int64_t i = 0; i < n; i++) x[i] = x[i] / (1.0f + ho_exp(-x[i]));
}

/* ops.rs:308-351 softmax. */
void ho_softmax(float* x, int64_t n) {
  if (n == 0) return;
  int64_t chunks = n / 8, rem = n % 8;
  float vmax[8];
  for (int l = 0; l < 8; l++) vmax[l] = -INFINITY;
  for (int64_t i = 0; i < chunks; i++)
    for (int l = 0; l < 8; l++) vmax[l] = x[i * 8 + l] > vmax[l] ? x[i * 8 + l] : vmax[l];
  float max_val = vmax[0];
  for (int l = 1; l < 8; l++) max_val = fmaxf(max_val, vmax[l]);
  for (int64_t i = n - rem; i < n; i++) max_val = fmaxf(max_val, x[i]);
  float lanes[8] = {0};
  for (int64_t i = 0; i < chunks; i++)
    for (int l = 0; l < 8; l++) {
      float e = ho_exp(x[i * 8 + l] - max_val);
      lanes[l] = fmaf(e, 1.0f, lanes[l]);
      x[i * 8 + l] = e;
    }
  float sum = reduce8(lanes);
  for (int64_t i = n - rem; i < n; i++) {
    x[i] = ho_exp(x[i] - max_val);
    sum += x[i];
  }
  if (sum > 0.0f) {
    float inv = 1.0f / sum;
    for (int64_t i = 0; i < chunks * 8; i++) x[i] = x[i] * inv;
    for (int64_t i = n - rem; i < n; i++) x[i] /= sum;
  }
}

/* ops.rs:353-406 attention for one query head over [seq_len][head_dim] K/V. */
void ho_attention(const float* q, const float* k, const float* v, int seq_len, int hd, float* out,
                  float* scratch) {
  int chunks = hd / 8, rem = hd % 8;
  float inv_sqrt_hd = 1.0f / sqrtf((float)hd);
  for (int p = 0; p < seq_len; p++) {
    const float* kr = k + (size_t)p * hd;
    float lanes[8] = {0};
    for (int i = 0; i < chunks; i++)
      for (int l = 0; l < 8; l++) lanes[l] = fmaf(q[i * 8 + l], kr[i * 8 + l], lanes[l]);
    float score = reduce8(lanes);
    for (int i = hd - rem; i < hd; i++) score += q[i] * kr[i];
    scratch[p] = score * inv_sqrt_hd;
  }
  ho_softmax(scratch, seq_len);
  for (int d = 0; d < chunks * 8; d++) {
    float acc = 0.0f;
    for (int p = 0; p < seq_len; p++) acc = fmaf(v[(size_t)p * hd + d], scratch[p], acc);
    out[d] = acc;
  }
  for (int d = hd - rem; d < hd; d++) {
    float acc = 0.0f;
    for (int p = 0; p < seq_len; p++) acc += scratch[p] * v[(size_t)p * hd + d];
    out[d] = acc;
  }
}

/* ------------------------------------------------------------------------- */
/* Hadamard fold                                                             */
/* ------------------------------------------------------------------------- */

/* qwen35.rs:51-68: normalized Sylvester WHT, butterflies h = 1, 2, 4, ... with
 * x[i] = a + b, x[i|h] = a - b for every i with bit h clear, then x *= 1/sqrt(n). */
void ho_wht(float* x, int64_t n) {
  const float s = 1.0f / sqrtf((float)n);
  for (int64_t h = 1; h < n; h <<= 1)
    for (int64_t i = 0; i < n; i++)
      if (!(i & h)) {
        float a = x[i], b = x[i | h];
        x[i] = a + b;
        x[i | h] = a - b;
      }
  for (int64_t i = 0; i < n; i++) x[i] *= s;
}

/* qwen35.rs:75-88: sign pass (when present), then the WHT per block. */
void ho_hadamard_rotate(float* x, int64_t n, const float* signs, int block) {
  if (signs)
    for (int64_t i = 0; i < n; i++) x[i] *= signs[i];
  for (int64_t o = 0; o + block <= n; o += block) ho_wht(x + o, block);
}

/* qwen35.rs:98-110: WHT per block first, then the sign pass. */
void ho_hadamard_unrotate(float* x, int64_t n, const float* signs, int block) {
  for (int64_t o = 0; o + block <= n; o += block) ho_wht(x + o, block);
  if (signs)
    for (int64_t i = 0; i < n; i++) x[i] *= signs[i];
}

/* ------------------------------------------------------------------------- */
/* greedy selection                                                          */
/* ------------------------------------------------------------------------- */

/* hearth-sampler lib.rs:26-40 apply_repetition_penalty, then :167-175 greedy
 * max_by(partial_cmp): on equal values max_by keeps the LATER element. */
uint32_t ho_sample_greedy_dense(float* logits, int64_t n, const uint32_t* past, int64_t n_past,
                                float pen) {
  if (!(fabsf(pen - 1.0f) < 1e-6f)) {
    for (int64_t t = 0; t < n_past; t++) {
      uint32_t idx = past[t];
      if ((int64_t)idx < n) {
        if (logits[idx] > 0.0f) logits[idx] /= pen;
        else logits[idx] *= pen;
      }
    }
  }
  int64_t best = 0;
  for (int64_t i = 1; i < n; i++)
    if (!(logits[i] < logits[best])) best = i; /* >= : ties go to the later index */
  return (uint32_t)best;
}

/* qwen35.rs:1735-1745: strict > scan from -inf. */
uint32_t ho_argmax_first(const float* logits, int64_t n) {
  int64_t best = 0;
  float bv = -INFINITY;
  for (int64_t i = 0; i < n; i++)
    if (logits[i] > bv) { bv = logits[i]; best = i; }
  return (uint32_t)best;
}

/* ------------------------------------------------------------------------- */
/* seeded synthetic data                                                     */
/* ------------------------------------------------------------------------- */
/* Definition shared with the device generator (hearth_amd/csrc): a counter-
 * based SplitMix64 stream per tensor; each element is the sum of four 16-bit
 * uniforms minus its mean (Irwin-Hall(4), sd 37837.23), i.e. an integer whose
 * distribution approximates N(0, sd^2).  Quantized tensors are built from the
 * integers directly, so their bytes are an exact integer function of the seed
 * (absmean scale for Q1_0/Q2_0, as in BitNet-style ternary export). */

static inline uint64_t mix64(uint64_t x) {
  x ^= x >> 30;
  x *= 0xbf58476d1ce4e5b9ull;
  x ^= x >> 27;
  x *= 0x94d049bb133111ebull;
  x ^= x >> 31;
  return x;
}

uint64_t ho_name_key(uint64_t seed, const char* name) {
  uint64_t h = 0xcbf29ce484222325ull; /* FNV-1a 64 */
  for (const unsigned char* p = (const unsigned char*)name; *p; p++) {
    h ^= *p;
    h *= 0x100000001b3ull;
  }
  return mix64(seed ^ mix64(h));
}

int32_t ho_synth_int(uint64_t key, uint64_t idx) {
  uint64_t h = mix64(key + idx * 0x9e3779b97f4a7c15ull);
  int32_t s = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) +
              (int32_t)((h >> 32) & 0xffff) + (int32_t)(h >> 48);
  return s - 131070;
}

float ho_synth_scale(float std) { return std / 37837.227f; }

uint32_t ho_synth_token(uint64_t seed, int64_t i, uint32_t vocab) {
  uint64_t key = ho_name_key(seed, "prompt");
  return (uint32_t)(mix64(key + (uint64_t)i * 0x9e3779b97f4a7c15ull) % vocab);
}

/* Packs 128 ternary codes (0/1/2 = weight -1/0/+1) and an f16 scale into one
 * PTQ1_0 block, as ho_quantize_ptq1_0 packs rounded values. */
void ho_ptq1_0_pack_codes(const int* code, uint16_t h, uint8_t* o) {
  memset(o, 0, 28);
  o[26] = (uint8_t)(h & 0xff);
  o[27] = (uint8_t)(h >> 8);
  for (int m = 0; m < 24; m++) {
    unsigned q = 0;
    for (int nn = 0; nn < 5; nn++) q = q * 3u + (unsigned)code[m < 16 ? 16 * nn + m : 80 + 8 * nn + (m - 16)];
    o[m] = (uint8_t)((q * 256u + 242u) / 243u);
  }
  for (int hh = 0; hh < 2; hh++) {
    unsigned q = 0;
    for (int mm = 0; mm < 4; mm++) q = q * 3u + (unsigned)code[120 + hh + 2 * mm];
    q *= 3u;
    o[24 + hh] = (uint8_t)((q * 256u + 242u) / 243u);
  }
}

void ho_synth_tensor(int type, uint64_t seed, const char* name, int64_t rows, int64_t cols,
                     float std, float mean, void* out, int n_threads) {
  uint64_t key = ho_name_key(seed, name);
  float c = ho_synth_scale(std);
  size_t rb = ho_row_bytes(type, cols);
  if (n_threads < 1) n_threads = 1;
#pragma omp parallel for num_threads(n_threads) schedule(static)
  for (int64_t r = 0; r < rows; r++) {
    uint64_t base = (uint64_t)r * (uint64_t)cols;
    if (type == HO_F32) {
      float* o = (float*)out + r * cols;
      for (int64_t j = 0; j < cols; j++) {
        float t = (float)ho_synth_int(key, base + j) * c;
        o[j] = t + mean;
      }
    } else if (type == HO_Q8_0) {
      uint8_t* o = (uint8_t*)out + (size_t)r * rb;
      float tmp[32];
      for (int64_t b = 0; b < cols / 32; b++) {
        for (int j = 0; j < 32; j++) tmp[j] = (float)ho_synth_int(key, base + b * 32 + j) * c;
        ho_quantize_q8_0(tmp, 32, o + b * 34);
      }
    } else if (type == HO_PTQ1_0) {
      /* the Q2_0 generator's ternary codes and scale, packed as PTQ1_0: the two
       * formats then hold the same weights */
      uint8_t* o = (uint8_t*)out + (size_t)r * rb;
      for (int64_t b = 0; b < cols / 128; b++) {
        int32_t iv[128];
        int64_t S = 0;
        for (int j = 0; j < 128; j++) {
          iv[j] = ho_synth_int(key, base + b * 128 + j);
          S += iv[j] < 0 ? -(int64_t)iv[j] : iv[j];
        }
        float scale = (float)S * (c / 128.0f);
        int code[128];
        for (int j = 0; j < 128; j++) {
          int64_t a = iv[j] < 0 ? -(int64_t)iv[j] : iv[j];
          code[j] = 1;
          if (S > 0 && 256 * a >= S) code[j] = iv[j] > 0 ? 2 : 0;
        }
        ho_ptq1_0_pack_codes(code, ho_f32_to_f16(scale), o + b * 28);
      }
    } else if (type == HO_Q1_0 || type == HO_Q1_0_G128 || type == HO_Q2_0 || type == HO_PQ2_0) {
      int is_q1 = (type == HO_Q1_0 || type == HO_Q1_0_G128);
      int bb = is_q1 ? 18 : 34;
      uint8_t* o = (uint8_t*)out + (size_t)r * rb;
      int32_t iv[128];
      float cq = c / 128.0f;
      for (int64_t b = 0; b < cols / 128; b++) {
        int64_t S = 0;
        for (int j = 0; j < 128; j++) {
          iv[j] = ho_synth_int(key, base + b * 128 + j);
          S += iv[j] < 0 ? -(int64_t)iv[j] : iv[j];
        }
        float scale = (float)S * cq;
        uint16_t h = ho_f32_to_f16(scale);
        uint8_t* blk = o + b * bb;
        blk[0] = (uint8_t)(h & 0xff);
        blk[1] = (uint8_t)(h >> 8);
        memset(blk + 2, 0, (size_t)(bb - 2));
        for (int j = 0; j < 128; j++) {
          if (is_q1) {
            if (iv[j] >= 0) blk[2 + j / 8] |= (uint8_t)(1u << (j % 8));
          } else {
            int64_t a = iv[j] < 0 ? -(int64_t)iv[j] : iv[j];
            int code = 1;
            if (S > 0 && 256 * a >= S) code = iv[j] > 0 ? 2 : 0;
            blk[2 + j / 4] |= (uint8_t)(code << (2 * (j % 4)));
          }
        }
      }
    }
  }
}


/* ------------------------------------------------------------------------- */
/* device association order (ORDER_DEVICE)                                   */
/* ------------------------------------------------------------------------- */
/* The same mathematics as the reference-order functions above, with the fp32
 * additions grouped as the HIP kernels group them, so the two implementations
 * can be compared bit for bit.  Wave reductions are butterflies over 64 lanes
 * (lane i adds lane i^o for o = 1..32); the vector sum of squares is 1024
 * slot-strided float4 partials, per-wave butterflies, then a 16-way pairwise
 * tree. */

static float bfly64(const float* v) {
  /* the device's wave_sum: butterfly with ascending offsets 1, 2, ..., 32 */
  float a[64], b[64];
  memcpy(a, v, sizeof a);
  for (int o = 1; o < 64; o <<= 1) {
    for (int i = 0; i < 64; i++) b[i] = a[i] + a[i ^ o];
    memcpy(a, b, sizeof a);
  }
  return a[0];
}

static float tree16f(const float* w) {
  /* 16-way pairwise tree: ((w0 + w1) + (w2 + w3)) + ..., then the four quads pairwise */
  float a0 = (w[0] + w[1]) + (w[2] + w[3]), a1 = (w[4] + w[5]) + (w[6] + w[7]);
  float a2 = (w[8] + w[9]) + (w[10] + w[11]), a3 = (w[12] + w[13]) + (w[14] + w[15]);
  return (a0 + a1) + (a2 + a3);
}

static float dev_sumsq_block(const float* x, int64_t K) {
  /* 1024 slots: slot t sums the float4s at 4t + 4096c in c order; slots
   * 64w..64w+63 butterfly into W_w; the 16 W_w add as a pairwise tree. */
  float lanes[1024], w[16];
  for (int t = 0; t < 1024; t++) {
    float ss = 0.0f;
    for (int64_t e = 4 * t; e < K; e += 4096) {
      float q = x[e] * x[e] + x[e + 1] * x[e + 1];
      q = q + x[e + 2] * x[e + 2];
      q = q + x[e + 3] * x[e + 3];
      ss = ss + q;
    }
    lanes[t] = ss;
  }
  for (int k = 0; k < 16; k++) w[k] = bfly64(lanes + 64 * k);
  return tree16f(w);
}

static void dev_rms_norm_block(const float* x, const float* w, float eps, int64_t K, float* out) {
  float inv = 1.0f / sqrtf(dev_sumsq_block(x, K) / (float)K + eps);
  for (int64_t i = 0; i < K; i++) out[i] = x[i] * inv * w[i];
}

static float dev_sumsq_wave(const float* x, int n) {
  float lanes[64];
  for (int l = 0; l < 64; l++) {
    float ss = 0.0f;
    for (int d = l; d < n; d += 64) ss = ss + x[d] * x[d];
    lanes[l] = ss;
  }
  return bfly64(lanes);
}

static void dev_rms_norm_wave(const float* x, const float* w, float eps, int n, float* out) {
  float inv = 1.0f / sqrtf(dev_sumsq_wave(x, n) / (float)n + eps);
  for (int i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

/* Attention head RMSNorm as the split kernel computes it on hd/4 lanes, each
 * holding a float4 slice: ss_c = ((x0^2 + x1^2) + x2^2) + x3^2, then an
 * ascending butterfly over the hd/4 lanes. */
static void dev_rms_norm_slices(const float* x, const float* w, float eps, int n, float* out) {
  float a[64], b[64];
  const int L = n / 4;
  for (int c = 0; c < L; c++) {
    float q = x[4 * c] * x[4 * c] + x[4 * c + 1] * x[4 * c + 1];
    q = q + x[4 * c + 2] * x[4 * c + 2];
    a[c] = q + x[4 * c + 3] * x[4 * c + 3];
  }
  for (int o = 1; o < L; o <<= 1) {
    for (int i = 0; i < L; i++) b[i] = a[i] + a[i ^ o];
    memcpy(a, b, sizeof(float) * (size_t)L);
  }
  float inv = 1.0f / sqrtf(a[0] / (float)n + eps);
  for (int i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

/* Split-sequence attention for one query head: chunks of C = 8192/hd positions,
 * per chunk max / exp / butterfly sum / sequential fma of p*v, then the chunks
 * merged with exp(m_s - M) weights. */
/* Butterfly sum over n lanes (n a power of two <= 64), offsets n/2 .. 1. */
static float bfly_n(const float* v, int n) {
  float a[64], b[64];
  memcpy(a, v, sizeof(float) * (size_t)n);
  for (int o = n / 2; o > 0; o >>= 1) {
    for (int i = 0; i < n; i++) b[i] = a[i] + a[i ^ o];
    memcpy(a, b, sizeof(float) * (size_t)n);
  }
  return a[0];
}

/* Lanes per workgroup of the device's attention split kernel (ATTN_NT). */
#define DEV_ATTN_NT 512

/* CUs of the device whose split geometry the device order follows (MI355X). */
#define DEV_ATTN_CUS 256

/* Positions per split: 8192/hd, or twice that once the (chunk, kv head) pairs
 * at that width outnumber the device's CUs. */
static int dev_attn_chunk(int seq, int hd, int n_kv) {
  int c = 8192 / hd;
  return (int64_t)((seq + c - 1) / c) * n_kv > DEV_ATTN_CUS ? 2 * c : c;
}

/* Split-sequence attention in the device's grouping: chunks of C positions
 * (dev_attn_chunk); a score is the butterfly over hd/4 column slices of a
 * 4-term fma chain; a chunk's softmax sum is the 64-lane butterfly of its e
 * values (C = 128: of e_l + e_{64+l}); the chunk's o is summed per row group
 * (rows i*RPI + sub) as an fma chain over i and the groups are combined
 * pairwise; splits merge with w_t = exp(m_t - M) as four strided fma chains
 * added pairwise.  The reference computes the same softmax-weighted sum in
 * one pass (ops.rs:353-406). */
static void dev_attention(const float* q, const float* k, const float* v, int seq, int hd, int n_kv, float* out) {
  const int C = dev_attn_chunk(seq, hd, n_kv), LPR = hd / 4, RPI = DEV_ATTN_NT / LPR, NR = C / RPI,
            NW = DEV_ATTN_NT / 64;
  const int ns = (seq + C - 1) / C;
  float inv_sqrt = 1.0f / sqrtf((float)hd);
  float* ms = (float*)malloc(sizeof(float) * (size_t)ns * (hd + 3));
  float* ls = ms + ns;
  float* wts = ls + ns;
  float* os = wts + ns;
  for (int s = 0; s < ns; s++) {
    int p0 = s * C, np = seq - p0 < C ? seq - p0 : C;
    float sc[128], e[128], parts[64], lanes[64];
    for (int l = 0; l < 128; l++) sc[l] = -INFINITY;
    for (int j = 0; j < np; j++) {
      const float* kr = k + (size_t)(p0 + j) * hd;
      for (int c = 0; c < LPR; c++) {
        float p = q[4 * c] * kr[4 * c];
        p = fmaf(q[4 * c + 1], kr[4 * c + 1], p);
        p = fmaf(q[4 * c + 2], kr[4 * c + 2], p);
        p = fmaf(q[4 * c + 3], kr[4 * c + 3], p);
        parts[c] = p;
      }
      sc[j] = bfly_n(parts, LPR) * inv_sqrt;
    }
    float m = -INFINITY;
    for (int l = 0; l < 128; l++) m = fmaxf(m, sc[l]);
    for (int l = 0; l < 128; l++) e[l] = l < np ? ho_exp(sc[l] - m) : 0.0f;
    ms[s] = m;
    for (int l = 0; l < 64; l++) lanes[l] = C > 64 ? e[l] + e[64 + l] : e[l];
    ls[s] = bfly64(lanes);
    for (int d = 0; d < hd; d++) {
      float A[64] = {0}, X[32];
      for (int sub = 0; sub < RPI; sub++) {
        float acc = 0.0f;
        for (int i = 0; i < NR; i++) {
          int j = i * RPI + sub;
          if (j < np) acc = fmaf(e[j], v[(size_t)(p0 + j) * hd + d], acc);
        }
        A[sub] = acc;
      }
      for (int w = 0; w < NW; w++) X[w] = (LPR == 32) ? A[2 * w] + A[2 * w + 1] : A[w];
      for (int w = NW; w > 1; w >>= 1)
        for (int i = 0; i < w / 2; i++) X[i] = X[2 * i] + X[2 * i + 1];
      os[(size_t)s * hd + d] = X[0];
    }
  }
  float M = -INFINITY;
  for (int s = 0; s < ns; s++) M = fmaxf(M, ms[s]);
  float lanes[64];
  for (int l = 0; l < 64; l++) {
    float L = 0.0f;
    for (int t = l; t < ns; t += 64) {
      float w = ho_exp(ms[t] - M);
      wts[t] = w;
      L = L + w * ls[t];
    }
    lanes[l] = L;
  }
  float invL = 1.0f / bfly64(lanes);
  for (int d = 0; d < hd; d++) {
    float P[4];
    for (int g = 0; g < 4; g++) {
      P[g] = 0.0f;
      for (int t = g; t < ns; t += 4) P[g] = fmaf(wts[t], os[(size_t)t * hd + d], P[g]);
    }
    out[d] = ((P[0] + P[1]) + (P[2] + P[3])) * invL;
  }
  free(ms);
}

/* The device-order attention of one query head (test entry point) and its
 * chunk width. */
int ho_attn_chunk(int seq, int hd, int n_kv) { return dev_attn_chunk(seq, hd, n_kv); }
void ho_attention_dev(const float* q, const float* k, const float* v, int seq, int hd, int n_kv, float* out) {
  dev_attention(q, k, v, seq, hd, n_kv, out);
}

/* ------------------------------------------------------------------------- */
/* model                                                                     */
/* ------------------------------------------------------------------------- */

typedef struct {
  char name[64];
  int type;
  int64_t rows, cols;
  float std, mean;
  size_t nbytes;
  uint8_t* data;
} tensor_t;

typedef struct {
  tensor_t *attn_norm, *attn_q, *attn_k, *attn_v, *attn_output, *attn_q_norm, *attn_k_norm,
      *ffn_norm, *ffn_gate, *ffn_up, *ffn_down, *post_norm;
  tensor_t *attn_qkv, *attn_gate, *ssm_conv1d, *ssm_dt, *ssm_a, *ssm_alpha, *ssm_beta, *ssm_norm,
      *ssm_out;
  int is_gdn, attn_idx;
} layer_t;

struct ho_model {
  ho_config cfg;
  int n_tensors;
  tensor_t* tensors;
  layer_t* layers;
  tensor_t *token_embd, *output, *output_norm;
  float* rope;
  int rope_dim;
  /* caches */
  int n_attn_layers;
  float *k_cache, *v_cache; /* [attn_layer][kv_head][max_seq][hd] */
  int* cur_len;             /* per attn layer */
  float* gdn_state;         /* [layer][v_head][hd][hd] */
  float* conv_state;        /* [layer][kernel-1][conv_dim] stored [ch][k-1] */
  /* scratch */
  float *hidden, *normed, *q, *k, *v, *attn_out, *gate, *up, *tmp, *scores, *logits_tmp, *big;
  uint8_t* q8;
  int n_threads, arm;
  int order; /* 0 = reference association order, 1 = device order */
  /* Hadamard fold: sign vectors by width (qwen35.rs:843-845), rotation scratch */
  int n_signs, sign_w[8];
  float* signs[8];
  float* rot;
  /* Q8_0 activation trace (diagnostics, ho_model_q8_trace): mode 1 appends
   * every matmul input's Q8_0 bytes to trace, mode 2 uses the recorded bytes
   * in place of its own and counts the bytes that differ */
  int trace_mode;
  uint8_t* trace;
  size_t trace_cap, trace_pos;
  int64_t trace_diff, trace_acts_diff;
};

static tensor_t* add_tensor(ho_model* m, const char* name, int type, int64_t rows, int64_t cols,
                            float std, float mean) {
  tensor_t* t = &m->tensors[m->n_tensors++];
  snprintf(t->name, sizeof t->name, "%s", name);
  t->type = type;
  t->rows = rows;
  t->cols = cols;
  t->std = std;
  t->mean = mean;
  t->nbytes = ho_row_bytes(type, cols) * (size_t)rows;
  t->data = (uint8_t*)malloc(t->nbytes ? t->nbytes : 1);
  return t;
}

static tensor_t* addf(ho_model* m, const char* fmt, int layer, int type, int64_t rows,
                      int64_t cols, float std, float mean) {
  char name[64];
  snprintf(name, sizeof name, fmt, layer);
  return add_tensor(m, name, type, rows, cols, std, mean);
}

static void* xcalloc(size_t n, size_t s) {
  void* p = calloc(n ? n : 1, s);
  if (!p) {
    fprintf(stderr, "oracle: out of memory (%zu bytes)\n", n * s);
    abort();
  }
  return p;
}

ho_model* ho_model_new(const ho_config* cfg) {
  ho_model* m = (ho_model*)xcalloc(1, sizeof(ho_model));
  m->cfg = *cfg;
  const ho_config* c = &m->cfg;
  int L = c->n_layers, d = c->d_model, hd = c->head_dim;
  int nq = c->n_heads * hd, nkv = c->n_kv_heads * hd;
  m->tensors = (tensor_t*)xcalloc((size_t)(L * 24 + 8), sizeof(tensor_t));
  m->layers = (layer_t*)xcalloc((size_t)L, sizeof(layer_t));
  m->token_embd = add_tensor(m, "token_embd.weight", c->head_type, c->vocab, d, 0.02f, 0.0f);
  /* tied output (prism.hadamard.tied_output): the latent token_embd is the head */
  m->output = (c->arch == 1 && (c->had_flags & 2)) ? m->token_embd
                                                   : add_tensor(m, "output.weight", c->head_type, c->vocab, d, 0.02f, 0.0f);
  m->output_norm = add_tensor(m, "output_norm.weight", HO_F32, 1, d, 0.02f, 1.0f);
  int wt = c->wtype;
  int kdim = c->ssm_n_k_heads * c->ssm_head_dim, vdim = c->ssm_n_v_heads * c->ssm_head_dim;
  int conv_dim = 2 * kdim + vdim;
  m->n_attn_layers = 0;
  for (int i = 0; i < L; i++) {
    layer_t* ly = &m->layers[i];
    ly->is_gdn = (c->arch == 1) && ((i + 1) % c->full_attn_interval != 0);
    ly->attn_norm = addf(m, "blk.%d.attn_norm.weight", i, HO_F32, 1, d, 0.02f, 1.0f);
    if (c->arch == 1)
      ly->post_norm = addf(m, "blk.%d.post_attention_norm.weight", i, HO_F32, 1, d, 0.02f, 1.0f);
    else
      ly->ffn_norm = addf(m, "blk.%d.ffn_norm.weight", i, HO_F32, 1, d, 0.02f, 1.0f);
    if (ly->is_gdn) {
      ly->attn_qkv = addf(m, "blk.%d.attn_qkv.weight", i, wt, conv_dim, d, 0.02f, 0.0f);
      ly->attn_gate = addf(m, "blk.%d.attn_gate.weight", i, wt, vdim, d, 0.02f, 0.0f);
      ly->ssm_conv1d = addf(m, "blk.%d.ssm_conv1d.weight", i, HO_F32, conv_dim, c->ssm_conv_kernel,
                            0.3f, 0.0f);
      ly->ssm_dt = addf(m, "blk.%d.ssm_dt.bias", i, HO_F32, 1, c->ssm_n_v_heads, 0.5f, 0.0f);
      ly->ssm_a = addf(m, "blk.%d.ssm_a", i, HO_F32, 1, c->ssm_n_v_heads, 0.1f, -1.0f);
      ly->ssm_alpha =
          addf(m, "blk.%d.ssm_alpha.weight", i, HO_F32, c->ssm_n_v_heads, d, 0.02f, 0.0f);
      ly->ssm_beta = addf(m, "blk.%d.ssm_beta.weight", i, HO_F32, c->ssm_n_v_heads, d, 0.02f, 0.0f);
      ly->ssm_norm = addf(m, "blk.%d.ssm_norm.weight", i, HO_F32, 1, c->ssm_head_dim, 0.02f, 1.0f);
      ly->ssm_out = addf(m, "blk.%d.ssm_out.weight", i, wt, d, vdim, 0.02f, 0.0f);
    } else {
      int qrows = c->attn_out_gate ? 2 * nq : nq;
      ly->attn_idx = m->n_attn_layers++;
      ly->attn_q = addf(m, "blk.%d.attn_q.weight", i, wt, qrows, d, 0.02f, 0.0f);
      ly->attn_k = addf(m, "blk.%d.attn_k.weight", i, wt, nkv, d, 0.02f, 0.0f);
      ly->attn_v = addf(m, "blk.%d.attn_v.weight", i, wt, nkv, d, 0.02f, 0.0f);
      ly->attn_output = addf(m, "blk.%d.attn_output.weight", i, wt, d, nq, 0.02f, 0.0f);
      if (c->qk_norm) {
        ly->attn_q_norm = addf(m, "blk.%d.attn_q_norm.weight", i, HO_F32, 1, hd, 0.02f, 1.0f);
        ly->attn_k_norm = addf(m, "blk.%d.attn_k_norm.weight", i, HO_F32, 1, hd, 0.02f, 1.0f);
      }
    }
    ly->ffn_gate = addf(m, "blk.%d.ffn_gate.weight", i, wt, c->d_ffn, d, 0.02f, 0.0f);
    ly->ffn_up = addf(m, "blk.%d.ffn_up.weight", i, wt, c->d_ffn, d, 0.02f, 0.0f);
    ly->ffn_down = addf(m, "blk.%d.ffn_down.weight", i, wt, d, c->d_ffn, 0.02f, 0.0f);
  }
  m->rope_dim = c->rope_dim > 0 ? c->rope_dim : c->head_dim;
  m->rope = (float*)xcalloc((size_t)c->max_seq * (size_t)m->rope_dim, sizeof(float));
  ho_rope_table(c->max_seq, m->rope_dim, c->rope_theta, m->rope);
  size_t kv = (size_t)m->n_attn_layers * c->n_kv_heads * (size_t)c->max_seq * hd;
  m->k_cache = (float*)xcalloc(kv, sizeof(float));
  m->v_cache = (float*)xcalloc(kv, sizeof(float));
  m->cur_len = (int*)xcalloc((size_t)m->n_attn_layers + 1, sizeof(int));
  if (c->arch == 1) {
    m->gdn_state = (float*)xcalloc(
        (size_t)L * c->ssm_n_v_heads * (size_t)c->ssm_head_dim * c->ssm_head_dim, sizeof(float));
    m->conv_state =
        (float*)xcalloc((size_t)L * (c->ssm_conv_kernel - 1) * (size_t)conv_dim, sizeof(float));
  }
  size_t wide = (size_t)d;
  if ((size_t)c->d_ffn > wide) wide = c->d_ffn;
  if ((size_t)(2 * nq) > wide) wide = 2 * nq;
  if ((size_t)conv_dim > wide) wide = conv_dim;
  m->hidden = (float*)xcalloc(wide, sizeof(float));
  m->normed = (float*)xcalloc(wide, sizeof(float));
  m->q = (float*)xcalloc(wide, sizeof(float));
  m->k = (float*)xcalloc(wide, sizeof(float));
  m->v = (float*)xcalloc(wide, sizeof(float));
  m->attn_out = (float*)xcalloc(wide, sizeof(float));
  m->gate = (float*)xcalloc(wide, sizeof(float));
  m->up = (float*)xcalloc(wide, sizeof(float));
  m->tmp = (float*)xcalloc(wide, sizeof(float));
  m->big = (float*)xcalloc(wide * 4, sizeof(float));
  m->scores = (float*)xcalloc((size_t)c->max_seq + 8, sizeof(float));
  m->q8 = (uint8_t*)xcalloc(wide / 32 * 34 + 64, 1);
  m->rot = (float*)xcalloc(wide, sizeof(float));
  m->n_threads = 1;
  m->arm = 0;
  return m;
}

void ho_model_free(ho_model* m) {
  if (!m) return;
  for (int i = 0; i < m->n_tensors; i++) free(m->tensors[i].data);
  free(m->tensors);
  free(m->layers);
  free(m->rope);
  free(m->k_cache);
  free(m->v_cache);
  free(m->cur_len);
  free(m->gdn_state);
  free(m->conv_state);
  free(m->hidden); free(m->normed); free(m->q); free(m->k); free(m->v); free(m->attn_out);
  free(m->gate); free(m->up); free(m->tmp); free(m->big); free(m->scores); free(m->q8);
  free(m->rot);
  for (int i = 0; i < m->n_signs; i++) free(m->signs[i]);
  free(m);
}

int ho_model_tensor_count(const ho_model* m) { return m->n_tensors; }
const char* ho_model_tensor_name(const ho_model* m, int i) {
  return (i >= 0 && i < m->n_tensors) ? m->tensors[i].name : NULL;
}

void* ho_model_tensor(ho_model* m, const char* name, size_t* nbytes, int* type, int64_t* rows,
                      int64_t* cols) {
  for (int i = 0; i < m->n_tensors; i++) {
    tensor_t* t = &m->tensors[i];
    if (strcmp(t->name, name) == 0) {
      if (nbytes) *nbytes = t->nbytes;
      if (type) *type = t->type;
      if (rows) *rows = t->rows;
      if (cols) *cols = t->cols;
      return t->data;
    }
  }
  return NULL;
}

void ho_model_synth(ho_model* m, uint64_t seed, int n_threads) {
  for (int i = 0; i < m->n_tensors; i++) {
    tensor_t* t = &m->tensors[i];
    ho_synth_tensor(t->type, seed, t->name, t->rows, t->cols, t->std, t->mean, t->data, n_threads);
  }
}

void ho_model_reset(ho_model* m) {
  const ho_config* c = &m->cfg;
  size_t kv = (size_t)m->n_attn_layers * c->n_kv_heads * (size_t)c->max_seq * c->head_dim;
  memset(m->k_cache, 0, kv * 4);
  memset(m->v_cache, 0, kv * 4);
  memset(m->cur_len, 0, sizeof(int) * (size_t)(m->n_attn_layers + 1));
  if (c->arch == 1) {
    int kdim = c->ssm_n_k_heads * c->ssm_head_dim, vdim = c->ssm_n_v_heads * c->ssm_head_dim;
    memset(m->gdn_state, 0,
           sizeof(float) * (size_t)c->n_layers * c->ssm_n_v_heads * c->ssm_head_dim *
               c->ssm_head_dim);
    memset(m->conv_state, 0,
           sizeof(float) * (size_t)c->n_layers * (c->ssm_conv_kernel - 1) * (2 * kdim + vdim));
  }
}

/* KVStorage::Q8_0 (kvcache.rs:41-57): write_kv quantizes the row into Q8_0
 * blocks (:92-113, quantize_q8_0_block :274-303) and every reader dequantizes
 * it (:287-317, attention_q8_0 ops.rs:946-1030: the int8 times the f16 scale,
 * exact in f32).  Holding dequant(quant(row)) in f32 is therefore the same
 * cache as seen by attention. */
static void kv_store_row(const ho_config* c, float* dst, const float* src, int hd) {
  if (c->kv_type != HO_Q8_0) {
    memcpy(dst, src, sizeof(float) * hd);
    return;
  }
  uint8_t blk[34 * 16];
  ho_quantize_q8_0(src, hd, blk);
  ho_dequantize(HO_Q8_0, blk, hd, dst);
}

/* KV prefill with N(0,1) values rounded to fp16 (stored exactly in f32):
 * value(layer l, kv head h, pos p, dim j) = f16(I * (1/sd)) with stream
 * "blk.<l>.kv_k" / "blk.<l>.kv_v", index ((p * n_kv) + h) * hd + j. */
int ho_model_kv_prefill_synth(ho_model* m, uint64_t seed, int n_pos) {
  const ho_config* c = &m->cfg;
  if (n_pos > c->max_seq) return 1;
  float cs = ho_synth_scale(1.0f);
  int hd = c->head_dim;
  for (int li = 0; li < c->n_layers; li++) {
    layer_t* ly = &m->layers[li];
    if (ly->is_gdn) continue;
    char nk[64], nv[64];
    snprintf(nk, sizeof nk, "blk.%d.kv_k", li);
    snprintf(nv, sizeof nv, "blk.%d.kv_v", li);
    uint64_t kk = ho_name_key(seed, nk), kvk = ho_name_key(seed, nv);
    for (int h = 0; h < c->n_kv_heads; h++) {
      float* kb = m->k_cache + ((size_t)ly->attn_idx * c->n_kv_heads + h) * (size_t)c->max_seq * hd;
      float* vb = m->v_cache + ((size_t)ly->attn_idx * c->n_kv_heads + h) * (size_t)c->max_seq * hd;
      for (int p = 0; p < n_pos; p++) {
        for (int j = 0; j < hd; j++) {
          uint64_t idx = ((uint64_t)p * c->n_kv_heads + h) * hd + j;
          kb[(size_t)p * hd + j] = ho_f16_to_f32(ho_f32_to_f16((float)ho_synth_int(kk, idx) * cs));
          vb[(size_t)p * hd + j] = ho_f16_to_f32(ho_f32_to_f16((float)ho_synth_int(kvk, idx) * cs));
        }
        kv_store_row(c, kb + (size_t)p * hd, kb + (size_t)p * hd, hd);
        kv_store_row(c, vb + (size_t)p * hd, vb + (size_t)p * hd, hd);
      }
    }
    m->cur_len[ly->attn_idx] = n_pos;
  }
  return 0;
}

void ho_model_set_order(ho_model* m, int order) { m->order = order; }

/* full-width RMSNorm / per-head RMSNorm / attention in the model's order */
static void norm_d(const ho_model* m, const float* x, const float* w, int64_t n, float* out) {
  if (m->order) dev_rms_norm_block(x, w, m->cfg.eps, n, out);
  else ho_rms_norm(x, w, m->cfg.eps, n, out);
}
static void norm_head(const ho_model* m, const float* x, const float* w, int n, float* out) {
  if (m->order) dev_rms_norm_wave(x, w, m->cfg.eps, n, out);
  else ho_rms_norm(x, w, m->cfg.eps, n, out);
}
static void norm_head_attn(const ho_model* m, const float* x, const float* w, int n, float* out) {
  if (m->order) dev_rms_norm_slices(x, w, m->cfg.eps, n, out);
  else ho_rms_norm(x, w, m->cfg.eps, n, out);
}

void ho_model_set_threads(ho_model* m, int n_threads, int arm) {
  m->n_threads = n_threads < 1 ? 1 : n_threads;
  m->arm = arm;
}

const float* ho_model_hidden(const ho_model* m) { return m->hidden; }

/* Work buffers left by the last forward (the last layer's values), for
 * diagnostics: 0 hidden, 1 normed, 2 q, 3 k, 4 v, 5 attn_out, 6 gate (after
 * silu), 7 up, 8 tmp (last projection output), 9 big (silu(gate)*up). */
const float* ho_model_buffer(const ho_model* m, int which) {
  const float* b[10] = {m->hidden, m->normed, m->q, m->k, m->v, m->attn_out, m->gate, m->up, m->tmp, m->big};
  return which >= 0 && which < 10 ? b[which] : NULL;
}

static const float* signs_for(const ho_model* m, int width) {
  for (int i = 0; i < m->n_signs; i++)
    if (m->sign_w[i] == width) return m->signs[i];
  return NULL;
}

int ho_model_set_signs(ho_model* m, int width, const float* signs) {
  for (int i = 0; i < m->n_signs; i++)
    if (m->sign_w[i] == width) { memcpy(m->signs[i], signs, sizeof(float) * (size_t)width); return 0; }
  if (m->n_signs == 8 || width <= 0) return 1;
  m->sign_w[m->n_signs] = width;
  m->signs[m->n_signs] = (float*)xcalloc((size_t)width, sizeof(float));
  memcpy(m->signs[m->n_signs], signs, sizeof(float) * (size_t)width);
  m->n_signs++;
  return 0;
}

/* The activation a matmul quantizes: x itself, or on a folded qwen35 model its
 * rotation R x (qwen35.rs:914-941, `mm(.., had = true)`; every hybrid matmul
 * input is folded). */
static const float* fold_input(ho_model* m, const float* x, int64_t n) {
  if (m->cfg.arch != 1 || m->cfg.had_block <= 0) return x;
  memcpy(m->rot, x, sizeof(float) * (size_t)n);
  ho_hadamard_rotate(m->rot, n, signs_for(m, (int)n), m->cfg.had_block);
  return m->rot;
}

/* quantize_act (q8_0.rs:20-51) of a matmul input into m->q8, with the trace */
static void quant_act(ho_model* m, const float* x, int64_t n) {
  ho_quantize_q8_0(x, n, m->q8);
  const size_t nb = (size_t)(n / 32) * 34;
  if (m->trace_mode == 0 || m->trace_pos + nb > m->trace_cap) return;
  uint8_t* t = m->trace + m->trace_pos;
  if (m->trace_mode == 1) {
    memcpy(t, m->q8, nb);
  } else {
    int64_t d = 0;
    for (size_t i = 0; i < nb; i++) d += t[i] != m->q8[i];
    m->trace_diff += d;
    m->trace_acts_diff += d > 0;
    memcpy(m->q8, t, nb);
  }
  m->trace_pos += nb;
}

/* Diagnostics: mode 0 off; 1 record every matmul input's Q8_0 bytes into buf
 * (cap bytes); 2 replay them: each matmul then reads the recorded bytes
 * instead of its own quantization.  Resets the cursor and the counters. */
void ho_model_q8_trace(ho_model* m, int mode, uint8_t* buf, size_t cap) {
  m->trace_mode = mode;
  m->trace = buf;
  m->trace_cap = cap;
  m->trace_pos = 0;
  m->trace_diff = m->trace_acts_diff = 0;
}

/* bytes used so far; out[0] = replayed bytes that differed from the model's
 * own quantization, out[1] = matmul inputs with at least one such byte */
size_t ho_model_q8_trace_stats(const ho_model* m, int64_t* out) {
  if (out) { out[0] = m->trace_diff; out[1] = m->trace_acts_diff; }
  return m->trace_pos;
}

/* matmul.rs:50-378 for the quantized dtypes: quantize_act + par_dot_rows. */
static void mm(ho_model* m, const tensor_t* w, const float* x, float* out) {
  quant_act(m, fold_input(m, x, w->cols), w->cols);
  ho_gemv(w->type, w->data, w->rows, w->cols, m->q8, out, m->n_threads, m->arm);
}

/* The device's LM-head row value: lane l (of 64) holds the units t = l + 64u
 * (two blocks each, u increasing) and sums q = q + (p_2t + p_2t+1) of their
 * scalar block products; the lanes combine by bfly64. */
static void dev_head_gemv(int type, const uint8_t* w, int64_t rows, int64_t K, const uint8_t* a, float* out,
                          int threads) {
  const int el = (type == 8) ? 32 : 128;
  const size_t bb = ho_row_bytes(type, el), abb = (size_t)(el / 32) * 34, rb = ho_row_bytes(type, K);
  const int64_t P = K / (2 * el);
  float (*dot)(const uint8_t*, const uint8_t*, int64_t) =
      type == 8 ? ho_dot_q8_0_q8_0 : (type == 41 || type == 43) ? ho_dot_q1_0_q8_0 : ho_dot_q2_0_q8_0;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t r = 0; r < rows; r++) {
    const uint8_t* wr = w + (size_t)r * rb;
    float lanes[64];
    for (int l = 0; l < 64; l++) {
      float q = 0.0f;
      for (int64_t t = l; t < P; t += 64) {
        float p0 = dot(wr + (size_t)(2 * t) * bb, a + (size_t)(2 * t) * abb, el);
        float p1 = dot(wr + (size_t)(2 * t + 1) * bb, a + (size_t)(2 * t + 1) * abb, el);
        q = q + (p0 + p1);
      }
      lanes[l] = q;
    }
    out[r] = bfly64(lanes);
  }
}

/* LM head in the model's order. */
static void head_mm(ho_model* m, const float* x, float* logits) {
  if (!logits) return; /* a prompt token whose logits nobody reads */
  const tensor_t* w = m->output;
  quant_act(m, fold_input(m, x, w->cols), w->cols);
  if (m->order) dev_head_gemv(w->type, w->data, w->rows, w->cols, m->q8, logits, m->n_threads);
  else ho_gemv(w->type, w->data, w->rows, w->cols, m->q8, logits, m->n_threads, m->arm);
}

/* qwen35.rs:1809-1815 */
static float softplus(float x) { return x > 20.0f ? x : ho_log(1.0f + ho_exp(x)); }

/* mod.rs:451-860 (dense decode step) */
static int forward_dense(ho_model* m, uint32_t token, int pos, float* logits) {
  const ho_config* c = &m->cfg;
  int d = c->d_model, hd = c->head_dim, nh = c->n_heads, nkvh = c->n_kv_heads;
  int nq = nh * hd;
  if ((int64_t)token >= m->token_embd->rows || pos >= c->max_seq) return 3;
  memset(m->hidden, 0, sizeof(float) * (size_t)d);
  ho_dequantize(m->token_embd->type, m->token_embd->data + ho_row_bytes(m->token_embd->type, d) * token,
                d, m->hidden);
  for (int li = 0; li < c->n_layers; li++) {
    layer_t* ly = &m->layers[li];
    norm_d(m, m->hidden, (const float*)ly->attn_norm->data, d, m->normed);
    mm(m, ly->attn_q, m->normed, m->q);
    mm(m, ly->attn_k, m->normed, m->k);
    mm(m, ly->attn_v, m->normed, m->v);
    if (ly->attn_q_norm) {
      for (int h = 0; h < nh; h++) {
        memcpy(m->tmp, m->q + h * hd, sizeof(float) * hd);
        norm_head_attn(m, m->tmp, (const float*)ly->attn_q_norm->data, hd, m->q + h * hd);
      }
    }
    if (ly->attn_k_norm) {
      for (int h = 0; h < nkvh; h++) {
        memcpy(m->tmp, m->k + h * hd, sizeof(float) * hd);
        norm_head_attn(m, m->tmp, (const float*)ly->attn_k_norm->data, hd, m->k + h * hd);
      }
    }
    for (int h = 0; h < nh; h++) ho_rope_apply(m->rope, c->max_seq, m->rope_dim, m->q + h * hd, pos);
    for (int h = 0; h < nkvh; h++) ho_rope_apply(m->rope, c->max_seq, m->rope_dim, m->k + h * hd, pos);
    int ai = ly->attn_idx;
    size_t head_stride = (size_t)c->max_seq * hd;
    float* kbase = m->k_cache + (size_t)ai * nkvh * head_stride;
    float* vbase = m->v_cache + (size_t)ai * nkvh * head_stride;
    for (int h = 0; h < nkvh; h++) { /* kvcache.rs:92-113 */
      kv_store_row(c, kbase + h * head_stride + (size_t)pos * hd, m->k + h * hd, hd);
      kv_store_row(c, vbase + h * head_stride + (size_t)pos * hd, m->v + h * hd, hd);
    }
    int seq_len = m->cur_len[ai] + 1; /* mod.rs:474: current_len before this write + 1 */
    if (pos + 1 > m->cur_len[ai]) m->cur_len[ai] = pos + 1;
    int rep = nh / nkvh;
    for (int qh = 0; qh < nh; qh++) {
      int kvh = qh / rep;
      if (m->order)
        dev_attention(m->q + qh * hd, kbase + kvh * head_stride, vbase + kvh * head_stride, seq_len, hd, nkvh,
                      m->attn_out + qh * hd);
      else
        ho_attention(m->q + qh * hd, kbase + kvh * head_stride, vbase + kvh * head_stride, seq_len, hd,
                     m->attn_out + qh * hd, m->scores);
    }
    mm(m, ly->attn_output, m->attn_out, m->tmp);
    for (int i = 0; i < d; i++) m->hidden[i] += m->tmp[i];
    norm_d(m, m->hidden, (const float*)ly->ffn_norm->data, d, m->normed);
    mm(m, ly->ffn_gate, m->normed, m->gate);
    mm(m, ly->ffn_up, m->normed, m->up);
    ho_silu(m->gate, c->d_ffn);
    for (int i = 0; i < c->d_ffn; i++) m->big[i] = m->gate[i] * m->up[i];
    mm(m, ly->ffn_down, m->big, m->tmp);
    for (int i = 0; i < d; i++) m->hidden[i] += m->tmp[i];
  }
  norm_d(m, m->hidden, (const float*)m->output_norm->data, d, m->normed);
  head_mm(m, m->normed, logits);
  (void)nq;
  return 0;
}

/* qwen35.rs:1239-1492 gdn_layer. Writes the branch output
 * into m->attn_out[0..d). */
static void gdn_layer(ho_model* m, int li, layer_t* ly) {
  const ho_config* c = &m->cfg;
  int d = c->d_model, hd = c->ssm_head_dim, nk = c->ssm_n_k_heads, nv = c->ssm_n_v_heads;
  int kdim = nk * hd, vdim = nv * hd, conv_dim = 2 * kdim + vdim, K = c->ssm_conv_kernel;
  float* qkv = m->big;              /* conv_dim */
  float* z = m->gate;               /* vdim */
  float* conv_out = m->big + conv_dim; /* conv_dim */
  float* oh = m->big + 2 * (size_t)conv_dim; /* vdim */
  float abuf[256], bbuf[256], gdec[256], beta[256];
  mm(m, ly->attn_qkv, m->normed, qkv);
  mm(m, ly->attn_gate, m->normed, z);
  /* :1015-1025 matvec_dense for alpha/beta */
  for (int r = 0; r < nv; r++) {
    const float* wa = (const float*)ly->ssm_alpha->data + (size_t)r * d;
    const float* wb = (const float*)ly->ssm_beta->data + (size_t)r * d;
    if (m->order) {   /* the input projection's epilogue: 1024 slots, slot t sums the float4s
                         at 4t + 4096c (c, then element, ascending); slots 64w..64w+63
                         butterfly into W_w; the 16 W_w add as a pairwise tree */
      float la[1024], lb[1024], wa16[16], wb16[16];
      for (int t = 0; t < 1024; t++) {
        float a = 0.0f, b = 0.0f;
        for (int e0 = 4 * t; e0 < d; e0 += 4096)
          for (int i = 0; i < 4; i++) {
            a = a + wa[e0 + i] * m->normed[e0 + i];
            b = b + wb[e0 + i] * m->normed[e0 + i];
          }
        la[t] = a;
        lb[t] = b;
      }
      for (int w = 0; w < 16; w++) { wa16[w] = bfly64(la + 64 * w); wb16[w] = bfly64(lb + 64 * w); }
      abuf[r] = tree16f(wa16);
      bbuf[r] = tree16f(wb16);
      continue;
    }
    float acc = 0.0f, accb = 0.0f;
    for (int j = 0; j < d; j++) { acc += wa[j] * m->normed[j]; accb += wb[j] * m->normed[j]; }
    abuf[r] = acc;
    bbuf[r] = accb;
  }
  /* ConvState prepare/push (:264-315) + depthwise_conv (:1820-1829) + silu */
  float* cs = m->conv_state + (size_t)li * (K - 1) * conv_dim;
  const float* cw = (const float*)ly->ssm_conv1d->data;
  for (int ch = 0; ch < conv_dim; ch++) {
    float win[8];
    for (int t = 0; t < K - 1; t++) win[t] = cs[(size_t)ch * (K - 1) + t];
    win[K - 1] = qkv[ch];
    for (int t = 0; t < K - 1; t++) cs[(size_t)ch * (K - 1) + t] = win[t + 1];
    float acc = 0.0f;
    for (int t = 0; t < K; t++) acc += cw[(size_t)ch * K + t] * win[t];
    conv_out[ch] = acc;
  }
  ho_silu(conv_out, conv_dim);
  /* l2 norm of q and k heads (:1332-1347) */
  float* qn = m->tmp;  /* 2*kdim fits in `wide` */
  memcpy(qn, conv_out, sizeof(float) * 2 * (size_t)kdim);
  for (int h = 0; h < 2 * nk; h++) {
    float ss = 0.0f;
    if (m->order) {   /* two 64-lane butterflies, then their sum */
      float la[64], lb[64];
      for (int l = 0; l < 64; l++) {
        la[l] = qn[h * hd + l] * qn[h * hd + l];
        lb[l] = qn[h * hd + 64 + l] * qn[h * hd + 64 + l];
      }
      ss = bfly64(la) + bfly64(lb);
    } else
    for (int j = 0; j < hd; j++) ss += qn[h * hd + j] * qn[h * hd + j];
    float inv = 1.0f / sqrtf(ss + c->eps);
    for (int j = 0; j < hd; j++) qn[h * hd + j] *= inv;
  }
  const float* kn = qn + kdim;
  const float* vconv = conv_out + 2 * kdim;
  const float* dtb = (const float*)ly->ssm_dt->data;
  const float* sa = (const float*)ly->ssm_a->data;
  for (int h = 0; h < nv; h++) {
    gdec[h] = softplus(abuf[h] + dtb[h]) * sa[h];
    beta[h] = 1.0f / (1.0f + ho_exp(-bbuf[h]));
  }
  float scale_q = 1.0f / sqrtf((float)hd);
  float* state = m->gdn_state + (size_t)li * nv * hd * hd;
  for (int h = 0; h < nv; h++) { /* :1371-1404 */
    int kg = h % nk;
    float decay = ho_exp(gdec[h]);
    float b = beta[h];
    float* S = state + (size_t)h * hd * hd;
    const float* kk = kn + kg * hd;
    const float* qq = qn + kg * hd;
    if (m->order) {   /* 8 row-chunks of 16, each summed sequentially, chunks in order */
      for (int j = 0; j < hd; j++) {
        float dp[8], dot = 0.0f;
        for (int c = 0; c < 8; c++) {
          float a = 0.0f;
          for (int r = 0; r < 16; r++) a = a + S[(size_t)(c * 16 + r) * hd + j] * kk[c * 16 + r];
          dp[c] = a;
        }
        for (int c = 0; c < 8; c++) dot = dot + dp[c];
        float bd = b * (vconv[h * hd + j] - dot);
        float o = 0.0f, op[8];
        for (int c = 0; c < 8; c++) {
          float a = 0.0f;
          for (int r = 0; r < 16; r++) {
            size_t ix = (size_t)(c * 16 + r) * hd + j;
            float sn = S[ix] * decay + kk[c * 16 + r] * bd;
            S[ix] = sn;
            a = a + sn * qq[c * 16 + r];
          }
          op[c] = a;
        }
        for (int c = 0; c < 8; c++) o = o + op[c];
        m->attn_out[h * hd + j] = o * scale_q;
      }
      continue;
    }
    for (int j = 0; j < hd; j++) {
      float dot = 0.0f;
      for (int i = 0; i < hd; i++) dot += S[(size_t)i * hd + j] * kk[i];
      float bd = b * (vconv[h * hd + j] - dot);
      for (int i = 0; i < hd; i++) S[(size_t)i * hd + j] = S[(size_t)i * hd + j] * decay + kk[i] * bd;
    }
    for (int j = 0; j < hd; j++) {
      float acc = 0.0f;
      for (int i = 0; i < hd; i++) acc += S[(size_t)i * hd + j] * qq[i];
      m->attn_out[h * hd + j] = acc * scale_q;
    }
  }
  /* gated RMSNorm (:1427-1439) */
  for (int h = 0; h < nv; h++)
    norm_head(m, m->attn_out + h * hd, (const float*)ly->ssm_norm->data, hd, oh + h * hd);
  ho_silu(z, vdim);
  for (int i = 0; i < vdim; i++) oh[i] *= z[i];
  if (c->had_block > 0 && nv / nk > 1) {
    /* :1452-1478: the fold of ssm_out was computed in grouped head order
     * [hd, rep, nk]: head h = r*nk + kg moves to slot kg*rep + r first */
    int rep = nv / nk;
    float* perm = m->up;
    for (int h = 0; h < nv; h++)
      memcpy(perm + (size_t)((h % nk) * rep + h / nk) * hd, oh + (size_t)h * hd, sizeof(float) * hd);
    memcpy(oh, perm, sizeof(float) * vdim);
  }
  mm(m, ly->ssm_out, oh, m->attn_out);
}

/* qwen35.rs:1495-1640 attn_layer (gated full attention). Output in m->attn_out[0..d). */
static void attn_layer_q35(ho_model* m, int pos, layer_t* ly) {
  const ho_config* c = &m->cfg;
  int hd = c->head_dim, nh = c->n_heads, nkvh = c->n_kv_heads, nq = nh * hd;
  float* qg = m->big; /* 2*nq */
  float* gate = m->gate;
  mm(m, ly->attn_q, m->normed, qg);
  mm(m, ly->attn_k, m->normed, m->k);
  mm(m, ly->attn_v, m->normed, m->v);
  for (int h = 0; h < nh; h++) {
    memcpy(gate + h * hd, qg + (size_t)h * 2 * hd + hd, sizeof(float) * hd);
    memmove(m->q + h * hd, qg + (size_t)h * 2 * hd, sizeof(float) * hd);
  }
  for (int h = 0; h < nh; h++) {
    norm_head_attn(m, m->q + h * hd, (const float*)ly->attn_q_norm->data, hd, m->tmp);
    memcpy(m->q + h * hd, m->tmp, sizeof(float) * hd);
  }
  for (int h = 0; h < nkvh; h++) {
    norm_head_attn(m, m->k + h * hd, (const float*)ly->attn_k_norm->data, hd, m->tmp);
    memcpy(m->k + h * hd, m->tmp, sizeof(float) * hd);
  }
  for (int h = 0; h < nh; h++) ho_rope_apply(m->rope, c->max_seq, m->rope_dim, m->q + h * hd, pos);
  for (int h = 0; h < nkvh; h++) ho_rope_apply(m->rope, c->max_seq, m->rope_dim, m->k + h * hd, pos);
  int ai = ly->attn_idx;
  size_t hs = (size_t)c->max_seq * hd;
  float* kb = m->k_cache + (size_t)ai * nkvh * hs;
  float* vb = m->v_cache + (size_t)ai * nkvh * hs;
  for (int h = 0; h < nkvh; h++) {
    kv_store_row(c, kb + h * hs + (size_t)pos * hd, m->k + h * hd, hd);
    kv_store_row(c, vb + h * hs + (size_t)pos * hd, m->v + h * hd, hd);
  }
  if (pos + 1 > m->cur_len[ai]) m->cur_len[ai] = pos + 1;
  int seq_len = m->cur_len[ai];
  int rep = nh / nkvh;
  float scale = 1.0f / sqrtf((float)hd);
  for (int qh = 0; qh < nh; qh++) { /* :1599-1624 scalar loops */
    int kvh = qh / rep;
    const float* qq = m->q + qh * hd;
    if (m->order) {
      dev_attention(qq, kb + kvh * hs, vb + kvh * hs, seq_len, hd, nkvh, m->attn_out + qh * hd);
      continue;
    }
    for (int t = 0; t < seq_len; t++) {
      const float* kr = kb + kvh * hs + (size_t)t * hd;
      float acc = 0.0f;
      for (int i = 0; i < hd; i++) acc += qq[i] * kr[i];
      m->scores[t] = acc * scale;
    }
    ho_softmax(m->scores, seq_len);
    for (int i = 0; i < hd; i++) {
      float acc = 0.0f;
      for (int t = 0; t < seq_len; t++) acc += m->scores[t] * vb[kvh * hs + (size_t)t * hd + i];
      m->attn_out[qh * hd + i] = acc;
    }
  }
  for (int i = 0; i < nq; i++) m->attn_out[i] /= 1.0f + ho_exp(-gate[i]);
  memcpy(m->up, m->attn_out, sizeof(float) * nq);
  mm(m, ly->attn_output, m->up, m->attn_out);
}

/* qwen35.rs:1028-1236 forward, with the Hadamard fold when had_block > 0. */
static int forward_hybrid(ho_model* m, uint32_t token, int pos, float* logits) {
  const ho_config* c = &m->cfg;
  int d = c->d_model;
  if ((int64_t)token >= m->token_embd->rows || pos >= c->max_seq) return 3;
  ho_dequantize(m->token_embd->type, m->token_embd->data + ho_row_bytes(m->token_embd->type, d) * token,
                d, m->hidden);
  /* :1054-1066: a latent table's rows are stored folded by R; the lookup applies R^-1 */
  if (c->had_block > 0 && (c->had_flags & 1)) ho_hadamard_unrotate(m->hidden, d, signs_for(m, d), c->had_block);
  for (int li = 0; li < c->n_layers; li++) {
    layer_t* ly = &m->layers[li];
    norm_d(m, m->hidden, (const float*)ly->attn_norm->data, d, m->normed);
    if (ly->is_gdn) gdn_layer(m, li, ly);
    else attn_layer_q35(m, pos, ly);
    for (int i = 0; i < d; i++) m->hidden[i] += m->attn_out[i];
    norm_d(m, m->hidden, (const float*)ly->post_norm->data, d, m->normed);
    mm(m, ly->ffn_gate, m->normed, m->gate);
    mm(m, ly->ffn_up, m->normed, m->up);
    ho_silu(m->gate, c->d_ffn);
    for (int i = 0; i < c->d_ffn; i++) m->gate[i] *= m->up[i];
    mm(m, ly->ffn_down, m->gate, m->attn_out);
    for (int i = 0; i < d; i++) m->hidden[i] += m->attn_out[i];
  }
  norm_d(m, m->hidden, (const float*)m->output_norm->data, d, m->normed);
  head_mm(m, m->normed, logits);
  return 0;
}

int ho_forward(ho_model* m, uint32_t token, int pos, float* logits) {
  return m->cfg.arch == 1 ? forward_hybrid(m, token, pos, logits)
                          : forward_dense(m, token, pos, logits);
}

/* mod.rs:2718-3012 (dense) / qwen35.rs:1654-1804 (hybrid) token loop, greedy,
 * prompt fed token-by-token from start_pos. */
int ho_generate(ho_model* m, const uint32_t* prompt, int n_prompt, int start_pos, int n_gen,
                float pen, uint32_t* out_tokens, float* last_logits) {
  const ho_config* c = &m->cfg;
  float* logits = (float*)xcalloc((size_t)c->vocab, sizeof(float));
  float* sample_buf = (float*)xcalloc((size_t)c->vocab, sizeof(float));
  uint32_t* past = (uint32_t*)xcalloc((size_t)n_gen + 2, sizeof(uint32_t));
  int n_past = 0, rc = 0;
  for (int i = 0; i < n_prompt; i++) {
    rc = ho_forward(m, prompt[i], start_pos + i, i + 1 < n_prompt ? NULL : logits);
    if (rc) goto done;
  }
  past[n_past++] = prompt[n_prompt - 1];
  for (int g = 0; g < n_gen; g++) {
    int pos = start_pos + n_prompt + g;
    uint32_t tok;
    if (c->arch == 1) tok = ho_argmax_first(logits, c->vocab);
    else {
      memcpy(sample_buf, logits, sizeof(float) * (size_t)c->vocab); /* sample_buf copy */
      tok = ho_sample_greedy_dense(sample_buf, c->vocab, past, n_past, pen);
    }
    out_tokens[g] = tok;
    past[n_past++] = tok;
    if (g + 1 < n_gen || last_logits) {
      rc = ho_forward(m, tok, pos, logits);
      if (rc) goto done;
    }
  }
  if (last_logits) memcpy(last_logits, logits, sizeof(float) * (size_t)c->vocab);
done:
  free(logits);
  free(sample_buf);
  free(past);
  return rc;
}
