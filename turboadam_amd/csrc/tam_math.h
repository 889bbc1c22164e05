// tam_math.h -- single-source (host + gfx950 device) arithmetic for the
// TurboAdam packed-state step.
//
// Everything here is built from IEEE-754 basic operations only (+, -, *, /,
// sqrt, fma, conversions, integer ops), compiled with -ffp-contract=off, so a
// function returns the same bits on the host and on the GPU.  Contents:
//   * Philox4x32-10 counter-based generator (Salmon et al., SC'11) and the
//     24-bit uniform drawn from one output word;
//   * fp32 -> fp16 / bf16 round-to-nearest-even;
//   * tam_logf / tam_expf: correctly rounded fp32 log and exp.  A fast fp64
//     evaluation (table + short polynomial, relative error < 2^-50) is
//     accepted when a rounding test proves the fp32 result; otherwise a
//     double-double evaluation (error < 2^-100) decides.  The reference CPU
//     path evaluates these with MKL (turboadam/quantize.py:256, :275); the
//     correctly rounded value is what both the oracle and the GPU compute.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tam_tables.h"

#define TAM_HD __host__ __device__ __forceinline__

// ---------------------------------------------------------------------------
// bit casts
// ---------------------------------------------------------------------------
TAM_HD uint32_t tam_f2u(float x) { return __builtin_bit_cast(uint32_t, x); }
TAM_HD float tam_u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
TAM_HD uint64_t tam_d2u(double x) { return __builtin_bit_cast(uint64_t, x); }
TAM_HD double tam_u2d(uint64_t u) { return __builtin_bit_cast(double, u); }
TAM_HD bool tam_isnan(float x) { return x != x; }
TAM_HD float tam_inf() { return tam_u2f(0x7f800000u); }
TAM_HD float tam_qnan() { return tam_u2f(0x7fc00000u); }

// ---------------------------------------------------------------------------
// Philox4x32-10
// ---------------------------------------------------------------------------
#define TAM_PHILOX_M0 0xD2511F53u
#define TAM_PHILOX_M1 0xCD9E8D57u
#define TAM_PHILOX_W0 0x9E3779B9u
#define TAM_PHILOX_W1 0xBB67AE85u

struct TamU4 {
  uint32_t x, y, z, w;
};

// fma(a, b, k) for a constant k that is not an inline operand: on the device
// one v_fma_f64 reading k from an SGPR pair (the compiler would copy k into
// the accumulator of a v_fmac_f64 first, a 64-bit move per use).  Same result.
TAM_HD double tam_fma_k(double a, double b, double k) {
#if defined(__HIP_DEVICE_COMPILE__)
  double r;
  asm("v_fma_f64 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(k));
  return r;
#else
  return __builtin_fma(a, b, k);
#endif
}

// a ^ b ^ c in one gfx950 three-input bitwise instruction (truth table 0x96).
TAM_HD uint32_t tam_xor3(uint32_t a, uint32_t b, uint32_t c) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
#else
  return a ^ b ^ c;
#endif
}

TAM_HD TamU4 tam_philox4x32_10(TamU4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += TAM_PHILOX_W0;
      k1 += TAM_PHILOX_W1;
    }
    const uint64_t p0 = (uint64_t)TAM_PHILOX_M0 * c.x;
    const uint64_t p1 = (uint64_t)TAM_PHILOX_M1 * c.z;
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    TamU4 n;
    n.x = tam_xor3(hi1, c.y, k0);
    n.y = lo1;
    n.z = tam_xor3(hi0, c.w, k1);
    n.w = lo0;
    c = n;
  }
  return c;
}

// Stochastic-rounding draws of tensor `tid` at optimizer step `step`.  The
// elements of the tensor's zero-padded block layout go in groups of 16
// consecutive ones, e = 16t + k; group t takes the 384 bits of three
// Philox4x32-10 blocks with counters (3t + j, tid, step, (3t + j) >> 32),
// j = 0, 1, 2, key (seed_lo, seed_hi), read as the little-endian words
// w0..w11.  Element k's draw is the 24-bit integer whose high 16 bits are
// bits [16k, 16k+16) (half k % 2 of word k / 2: the first two blocks) and
// whose low 8 bits are bits [256 + 8k, 256 + 8k + 8) (byte k of the third
// block): uniform = that integer * 2^-24 (exact).  Every output bit is used.
// The high parts of elements 8h .. 8h + 7 are block 3t + h alone, which is
// all that the certified fast path of the re-quantisation reads.
TAM_HD TamU4 tam_philox_block(uint64_t ctr, uint32_t tid, uint32_t step, uint32_t seed_lo, uint32_t seed_hi) {
  TamU4 c;
  c.x = (uint32_t)ctr;
  c.y = tid;
  c.z = step;
  c.w = (uint32_t)(ctr >> 32);
  return tam_philox4x32_10(c, seed_lo, seed_hi);
}

// The 24-bit draw of element 2i + o (o = 0 or 1) of a half-group: high 16
// bits from half o of word a (word i of the half's first block), low 8 bits
// the low byte of lo8.
TAM_HD uint32_t tam_draw24(uint32_t a, uint32_t o, uint32_t lo8) {
  return ((o ? (a >> 16) : (a & 0xffffu)) << 8) | (lo8 & 0xffu);
}

// The draws of the 8 consecutive elements e0 .. e0+7 (e0 a multiple of 8) of
// group t = e0/16, half h = (e0/8) % 2: high parts from block 3t + h, low
// bytes 8h .. 8h+7 of block 3t + 2 (its words 2h and 2h + 1).
TAM_HD void tam_draws8(uint64_t e0, uint32_t tid, uint32_t step, uint32_t seed_lo, uint32_t seed_hi,
                       uint32_t* r) {
  const uint32_t h = (uint32_t)(e0 >> 3) & 1u;
  const uint64_t c0 = 3u * (e0 >> 4);
  const TamU4 a = tam_philox_block(c0 + h, tid, step, seed_lo, seed_hi);
  const TamU4 c = tam_philox_block(c0 + 2u, tid, step, seed_lo, seed_hi);
  const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
  const uint32_t c0w = h ? c.z : c.x, c1w = h ? c.w : c.y;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = tam_draw24(aw[j >> 1], (uint32_t)j & 1u, (j < 4 ? c0w : c1w) >> (8 * (j & 3)));
}

// Uniform of a 24-bit draw.
TAM_HD float tam_u24f(uint32_t d) { return (float)d * 0x1p-24f; }

// ---------------------------------------------------------------------------
// fp16 / bf16 rounding (round to nearest, ties to even)
// ---------------------------------------------------------------------------
TAM_HD uint16_t tam_f32_to_f16(float x) {
  _Float16 h = (_Float16)x;
  return __builtin_bit_cast(uint16_t, h);
}
TAM_HD float tam_f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
TAM_HD uint16_t tam_f32_to_bf16(float x) {
  const uint32_t u = tam_f2u(x);
  if (tam_isnan(x)) return (uint16_t)0x7fc0u;
  const uint32_t r = u + 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(r >> 16);
}
TAM_HD float tam_bf16_to_f32(uint16_t b) { return tam_u2f((uint32_t)b << 16); }
// Hardware round-to-nearest-even to bf16 (v_cvt_pk_bf16_f32 on gfx950).  Equal
// to tam_f32_to_bf16 for every non-NaN input; callers pass no NaN.
TAM_HD uint16_t tam_f32_to_bf16_rne(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }

// ---------------------------------------------------------------------------
// double-double helpers (slow paths)
// ---------------------------------------------------------------------------
struct TamDD {
  double hi, lo;
};
TAM_HD TamDD tam_two_sum(double a, double b) {
  TamDD r;
  r.hi = a + b;
  const double bb = r.hi - a;
  r.lo = (a - (r.hi - bb)) + (b - bb);
  return r;
}
TAM_HD TamDD tam_fast_two_sum(double a, double b) {  // |a| >= |b|
  TamDD r;
  r.hi = a + b;
  r.lo = b - (r.hi - a);
  return r;
}
TAM_HD TamDD tam_dd_add(TamDD a, TamDD b) {
  TamDD s = tam_two_sum(a.hi, b.hi);
  TamDD t = tam_two_sum(a.lo, b.lo);
  s.lo += t.hi;
  s = tam_fast_two_sum(s.hi, s.lo);
  s.lo += t.lo;
  return tam_fast_two_sum(s.hi, s.lo);
}
TAM_HD TamDD tam_dd_mul_d(TamDD a, double b) {
  TamDD p;
  p.hi = a.hi * b;
  p.lo = __builtin_fma(a.hi, b, -p.hi);
  p.lo = __builtin_fma(a.lo, b, p.lo);
  return tam_fast_two_sum(p.hi, p.lo);
}
TAM_HD TamDD tam_dd_mul(TamDD a, TamDD b) {
  TamDD p;
  p.hi = a.hi * b.hi;
  p.lo = __builtin_fma(a.hi, b.hi, -p.hi);
  p.lo = __builtin_fma(a.hi, b.lo, p.lo);
  p.lo = __builtin_fma(a.lo, b.hi, p.lo);
  return tam_fast_two_sum(p.hi, p.lo);
}

// One fp32 step away from f in the direction of +inf (up=true) or -inf.
TAM_HD float tam_next_float(float f, bool up) {
  uint32_t u = tam_f2u(f);
  if ((u & 0x7fffffffu) == 0) return up ? tam_u2f(1u) : tam_u2f(0x80000001u);
  const bool neg = (u >> 31) != 0;
  if (up != neg) u += 1; else u -= 1;
  return tam_u2f(u);
}

// Correctly rounded fp32 value of the double-double hi + lo (|lo| <= ulp(hi)/2).
TAM_HD float tam_dd_to_f32(TamDD v) {
  float f = (float)v.hi;
  const double diff = v.hi - (double)f;
  if (diff != 0.0 && v.lo != 0.0) {
    const float fn = tam_next_float(f, diff > 0.0);
    const double mid = ((double)f + (double)fn) * 0.5;
    if (v.hi == mid && ((diff > 0.0) == (v.lo > 0.0))) f = fn;
  }
  return f;
}

// ---------------------------------------------------------------------------
// tables (device copy in __constant__, host copy in a static array)
// ---------------------------------------------------------------------------
static __constant__ TamLogEntry tam_log_tab_d[129] = TAM_LOG_TABLE_INIT;
static const TamLogEntry tam_log_tab_h[129] = TAM_LOG_TABLE_INIT;
static __constant__ TamLogDD tam_logdd_tab_d[129] = TAM_LOGDD_TABLE_INIT;
static const TamLogDD tam_logdd_tab_h[129] = TAM_LOGDD_TABLE_INIT;
static __constant__ TamDD tam_exp_tab_d[64] = TAM_EXP_TABLE_INIT;
static const TamDD tam_exp_tab_h[64] = TAM_EXP_TABLE_INIT;
static __constant__ TamDD tam_invk_d[17] = TAM_INVK_INIT;
static const TamDD tam_invk_h[17] = TAM_INVK_INIT;
static __constant__ TamDD tam_invfact_d[17] = TAM_INVFACT_INIT;
static const TamDD tam_invfact_h[17] = TAM_INVFACT_INIT;

TAM_HD TamLogEntry tam_log_entry(int j) {
#if __HIP_DEVICE_COMPILE__
  return tam_log_tab_d[j];
#else
  return tam_log_tab_h[j];
#endif
}
TAM_HD TamLogDD tam_logdd_entry(int j) {
#if __HIP_DEVICE_COMPILE__
  return tam_logdd_tab_d[j];
#else
  return tam_logdd_tab_h[j];
#endif
}
TAM_HD TamDD tam_exp_entry(int j) {
#if __HIP_DEVICE_COMPILE__
  return tam_exp_tab_d[j];
#else
  return tam_exp_tab_h[j];
#endif
}
TAM_HD TamDD tam_invk(int k) {
#if __HIP_DEVICE_COMPILE__
  return tam_invk_d[k];
#else
  return tam_invk_h[k];
#endif
}
TAM_HD TamDD tam_invfact(int k) {
#if __HIP_DEVICE_COMPILE__
  return tam_invfact_d[k];
#else
  return tam_invfact_h[k];
#endif
}

// ---------------------------------------------------------------------------
// log
// ---------------------------------------------------------------------------
// Slow path: log(x) = e*ln2 + T_j + log1p(r) in double-double, r exact.
__host__ __device__ __attribute__((noinline)) inline float tam_logf_slow(int e, int j, double r) {
  // log1p(r) = sum_{k>=1} (-1)^(k+1) r^k / k, |r| <= 2^-8, 14 terms.
  TamDD p = tam_invk(14);
  p.hi = -p.hi;
  p.lo = -p.lo;
  for (int k = 13; k >= 1; --k) {
    p = tam_dd_mul_d(p, r);
    TamDD c = tam_invk(k);
    if ((k & 1) == 0) {
      c.hi = -c.hi;
      c.lo = -c.lo;
    }
    p = tam_dd_add(p, c);
  }
  p = tam_dd_mul_d(p, r);
  const double de = (double)e;
  TamDD l2;
  l2.hi = de * TAM_LN2_HI;  // exact: ln2_hi has 45 bits, |e| < 2^8
  l2.lo = 0.0;
  TamDD l2lo = tam_two_sum(de * TAM_LN2_LO, de * TAM_LN2_LO2);
  l2 = tam_dd_add(l2, l2lo);
  const TamLogDD t = tam_logdd_entry(j);
  TamDD tj;
  tj.hi = t.t_hi;
  tj.lo = t.t_lo;
  TamDD y = tam_dd_add(tam_dd_add(l2, tj), p);
  return tam_dd_to_f32(y);
}

// Correctly rounded logf for every fp32 input (log(+0) = -inf, negative -> NaN).
// `tab(j)` returns entry j of the 129-entry table (a kernel may pass a copy
// held in LDS); tam_logf below reads the constant-memory copy.
template <typename Tab>
TAM_HD float tam_logf_with(float x, Tab tab) {
  uint32_t u = tam_f2u(x);
  if (u >= 0x7f800000u || u == 0u) {
    if (u == 0x7f800000u) return x;                   // +inf
    if ((u & 0x7fffffffu) > 0x7f800000u) return x;    // NaN
    if ((u & 0x7fffffffu) == 0u) return -tam_inf();   // +-0
    return tam_qnan();                                // negative
  }
  int e = 0;
  if (u < 0x00800000u) {  // subnormal: scale by 2^25 (exact)
    x = x * 0x1p25f;
    u = tam_f2u(x);
    e = -25;
  }
  e += (int)(u >> 23) - 127;
  const uint32_t mant = u & 0x7fffffu;
  const int j = (int)((mant + (1u << 15)) >> 16);  // round(128*(m-1)), 0..128
  const double m = (double)tam_u2f(mant | 0x3f800000u);
  const TamLogEntry t = tab(j);
  const double r = __builtin_fma(m, (double)t.c, -1.0);  // exact, |r| <= 2^-8
  // log1p(r) ~ r + r^2 * (-1/2 + r/3 - r^2/4 + r^3/5 - r^4/6)
  double q = __builtin_fma(r, -0x1.5555555555555p-3, 0x1.999999999999ap-3);
  q = __builtin_fma(r, q, -0.25);
  q = tam_fma_k(r, q, 0x1.5555555555555p-2);
  q = __builtin_fma(r, q, -0.5);
  const double p = __builtin_fma(r * r, q, r);
  const double de = (double)e;
  const double s = __builtin_fma(de, TAM_LN2_HI, t.t_hi);
  const double lo = __builtin_fma(de, TAM_LN2_LO, (double)t.t_lo) + p;
  const double y = s + lo;
  const double err = (__builtin_fabs(s) + __builtin_fabs(lo)) * 0x1p-49;
  const float a = (float)(y - err);
  const float b = (float)(y + err);
  if (a == b) return a;
  return tam_logf_slow(e, j, r);
}

TAM_HD float tam_logf(float x) {
  return tam_logf_with(x, [](int j) { return tam_log_entry(j); });
}

// ---------------------------------------------------------------------------
// exp
// ---------------------------------------------------------------------------
TAM_HD double tam_pow2i(int E) {  // 2^E for -1022 <= E <= 1023
  return tam_u2d((uint64_t)(E + 1023) << 52);
}

__host__ __device__ __attribute__((noinline)) inline float tam_expf_slow(double x, double kd) {
  // r = x - k*ln2/64 as a double-double
  const double rh = __builtin_fma(-kd, TAM_LN2_64_HI, x);  // exact
  TamDD r = tam_two_sum(rh, -kd * TAM_LN2_64_LO);
  TamDD c2;
  c2.hi = __builtin_fma(-kd, TAM_LN2_64_LO, kd * TAM_LN2_64_LO);  // error of -kd*lo
  c2.lo = -kd * TAM_LN2_64_LO2;
  r = tam_dd_add(r, c2);
  // e^r - 1 = sum_{k=1}^{13} r^k / k!   (|r| <= 0.0055)
  TamDD p = tam_invfact(13);
  for (int k = 12; k >= 1; --k) {
    p = tam_dd_mul(p, r);
    p = tam_dd_add(p, tam_invfact(k));
  }
  p = tam_dd_mul(p, r);
  const int k = (int)kd;
  const int jj = k & 63;
  const int E = k >> 6;
  const TamDD t = tam_exp_entry(jj);
  TamDD y = tam_dd_add(t, tam_dd_mul(t, p));
  const double sc = tam_pow2i(E);
  y.hi *= sc;
  y.lo *= sc;
  return tam_dd_to_f32(y);
}

// Correctly rounded expf for every fp32 input.  `tab(j)` returns entry j of the
// 64-entry table of 2^(j/64) as double-doubles.
template <typename Tab>
TAM_HD float tam_expf_with(float xf, Tab tab) {
  if (tam_isnan(xf)) return xf;
  if (xf > 89.0f) return tam_inf();
  if (xf < -104.0f) return 0.0f;
  const double x = (double)xf;
  const double kd = __builtin_rint(x * TAM_INV_LN2_64);
  const double rh = __builtin_fma(-kd, TAM_LN2_64_HI, x);  // exact
  const double r = rh + (-kd * TAM_LN2_64_LO);
  // e^r - 1 ~ r + r^2 * (1/2 + r/6 + r^2/24 + r^3/120 + r^4/720)
  double q = __builtin_fma(r, 0x1.6c16c16c16c17p-10, 0x1.1111111111111p-7);
  q = tam_fma_k(r, q, 0x1.5555555555555p-5);
  q = tam_fma_k(r, q, 0x1.5555555555555p-3);
  q = __builtin_fma(r, q, 0.5);
  const double em1 = __builtin_fma(r * r, q, r);
  const int k = (int)kd;
  const TamDD t = tab(k & 63);
  const double y = t.hi + __builtin_fma(t.hi, em1, t.lo);
  const double z = y * tam_pow2i(k >> 6);
  const double err = z * 0x1p-49;
  const float a = (float)(z - err);
  const float b = (float)(z + err);
  if (a == b) return a;
  return tam_expf_slow(x, kd);
}

TAM_HD float tam_expf(float xf) {
  return tam_expf_with(xf, [](int j) { return tam_exp_entry(j); });
}
