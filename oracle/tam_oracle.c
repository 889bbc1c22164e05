/* tam_oracle.c -- TEST INFRASTRUCTURE ONLY.  Never linked into, loaded by or
 * called from the turboadam_amd product path; only tests/, the smoke check
 * and bench.py's cpu_baseline leg use it, as the checker.
 *
 * A scalar CPU restatement of the reference TurboAdam step
 * (davidkny22/turboadam, src/turboadam), one parameter tensor at a time, in
 * "exact mode": the reference's library-defined operations are fixed to
 *   - exp / log: correctly rounded fp32 (evaluated as (float)expl / (float)logl,
 *     64-bit-significand x87 arithmetic),
 *   - dot products and block L2 norms: per 8 consecutive elements an fp32
 *     pairwise tree of the products (first level fused, fma(x0, y0,
 *     fl(x1*y1))), widened to fp64; a balanced fp64 pairwise tree over the 16
 *     partials of a 128-element block, then over the blocks zero-padded to a
 *     power of two; rounded to fp32 once (norms: fp64 sqrt, then rounded),
 *   - sqrt: correctly rounded,
 * and every other operation is the fp32 operation torch performs, in the
 * reference's order (fma exactly where torch fuses: Tensor.add_(alpha=) and
 * addcmul_).  Stochastic-rounding uniforms: Philox4x32-10 (its own
 * implementation here): elements in groups of 16, group t = e/16 taking the
 * 384 bits of the blocks with counters (3t + j, tensor_id, step, (3t+j)>>32),
 * j = 0..2, key seed, little endian; element 16t + k takes the 24-bit
 * integer whose high 16 bits are bits [16k, 16k+16) (blocks 3t and 3t + 1)
 * and whose low 8 bits are bits [256 + 8k, 256 + 8k + 8) (block 3t + 2),
 * u = that integer * 2^-24.  Compiled with -ffp-contract=off.
 * Loops over independent blocks or elements run under OpenMP; each iteration
 * writes its own outputs and every reduction runs in its fixed order after
 * the loop, so results do not depend on the thread count.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "tam_oracle.h"

#define OR_BS 128

/* ---------------------------------------------------------------- bits */
static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* ---------------------------------------------------------------- philox */
/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11). */
void or_philox4x32_10(const uint32_t ctr[4], uint32_t k0, uint32_t k1, uint32_t out[4]) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
  for (int r = 0; r < 10; ++r) {
    uint64_t a = (uint64_t)0xD2511F53u * c0;
    uint64_t b = (uint64_t)0xCD9E8D57u * c2;
    uint32_t n0 = (uint32_t)(b >> 32) ^ c1 ^ k0;
    uint32_t n1 = (uint32_t)b;
    uint32_t n2 = (uint32_t)(a >> 32) ^ c3 ^ k1;
    uint32_t n3 = (uint32_t)a;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* The 384 bits of draw group t: the Philox blocks with counters (3t + j,
 * tid, step, (3t + j) >> 32), j = 0, 1, 2, as little-endian bytes. */
static void or_group_bytes(uint64_t t, uint32_t tid, uint32_t step, uint64_t seed, uint8_t bytes[48]) {
  for (int j = 0; j < 3; ++j) {
    uint64_t c = 3 * t + (uint64_t)j;
    uint32_t ctr[4] = {(uint32_t)c, tid, step, (uint32_t)(c >> 32)};
    uint32_t w[4];
    or_philox4x32_10(ctr, (uint32_t)seed, (uint32_t)(seed >> 32), w);
    for (int i = 0; i < 4; ++i)
      for (int b = 0; b < 4; ++b) bytes[16 * j + 4 * i + b] = (uint8_t)(w[i] >> (8 * b));
  }
}

/* The 16 stochastic-rounding uniforms of draw group t (elements 16t ..
 * 16t+15): element 16t + k takes the 24-bit integer with high 16 bits from
 * bits [16k, 16k + 16) of the group (bytes 2k, 2k + 1) and low 8 bits from
 * bits [256 + 8k, 256 + 8k + 8) (byte 32 + k), times 2^-24.  The high parts
 * come from the first two blocks alone. */
static void or_group_uniforms(uint64_t t, uint32_t tid, uint32_t step, uint64_t seed, float* u16) {
  uint8_t bytes[48];
  or_group_bytes(t, tid, step, seed, bytes);
  for (int k = 0; k < 16; ++k) {
    uint32_t d = ((uint32_t)bytes[2 * k] << 8) | ((uint32_t)bytes[2 * k + 1] << 16) | (uint32_t)bytes[32 + k];
    u16[k] = (float)d * (1.0f / 16777216.0f);
  }
}

/* Uniforms of the synthetic test inputs (oracle/inputs.py): the same group
 * bits, element 16t + k taking the 24-bit integer at bits [24k, 24k + 24). */
void or_input_uniforms(uint32_t tid, uint32_t step, uint64_t seed, uint64_t count, float* out) {
  uint8_t bytes[48];
  for (uint64_t t = 0; t * 16 < count; ++t) {
    or_group_bytes(t, tid, step, seed, bytes);
    for (int k = 0; k < 16 && t * 16 + (uint64_t)k < count; ++k) {
      uint32_t d = (uint32_t)bytes[3 * k] | ((uint32_t)bytes[3 * k + 1] << 8) | ((uint32_t)bytes[3 * k + 2] << 16);
      out[t * 16 + (uint64_t)k] = (float)d * (1.0f / 16777216.0f);
    }
  }
}

static float or_uniform(uint64_t e, uint32_t tid, uint32_t step, uint64_t seed) {
  float u16[16];
  or_group_uniforms(e >> 4, tid, step, seed, u16);
  return u16[e & 15];
}

void or_philox_uniforms(uint32_t tid, uint32_t step, uint64_t seed, uint64_t count, float* out) {
  float u16[16];
  for (uint64_t t = 0; t * 16 < count; ++t) {
    or_group_uniforms(t, tid, step, seed, u16);
    for (int k = 0; k < 16 && t * 16 + (uint64_t)k < count; ++k) out[t * 16 + (uint64_t)k] = u16[k];
  }
}

/* ------------------------------------------------------ fp16 / bf16 RNE */
uint16_t or_f32_to_f16(float x) {
  uint32_t u = f2u(x);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) { /* inf / nan */
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    return (uint16_t)(sign | 0x7c00u);
  }
  int e = (int)(a >> 23) - 127;
  uint32_t mant = (a & 0x7fffffu) | 0x800000u; /* 24-bit significand (normal) */
  if (a < 0x00800000u) return (uint16_t)sign;  /* fp32 subnormal -> +-0 in fp16 */
  if (e > 15) return (uint16_t)(sign | 0x7c00u);
  int shift;                                   /* bits to drop from the 24-bit significand */
  uint32_t hexp;
  if (e >= -14) { shift = 13; hexp = (uint32_t)(e + 15); }
  else { shift = 13 + (-14 - e); hexp = 0; }
  if (shift > 24) return (uint16_t)sign;       /* below half of the smallest subnormal */
  uint32_t q = mant >> shift;
  uint32_t rem = mant & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1;
  uint32_t h;
  if (hexp == 0) h = q;                        /* subnormal (q may carry into the normal range) */
  else h = (hexp << 10) + (q - 0x400u);        /* q in [0x400, 0x800]; carry bumps the exponent */
  if (h >= 0x7c00u) h = 0x7c00u;
  return (uint16_t)(sign | h);
}

float or_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
  if (e == 0) { float v = (float)m * (1.0f / 16777216.0f); return sign ? -v : v; } /* m * 2^-24 */
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t or_f32_to_bf16(float x) {
  if (x != x) return 0x7fc0u;
  uint32_t u = f2u(x);
  uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}
float or_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* ------------------------------------------------------ exact transcendentals */
float or_logf(float x) {
  if (x != x) return x;
  if (x < 0.0f) return u2f(0x7fc00000u);
  if (x == 0.0f) return -INFINITY;
  if (isinf(x)) return x;
  return (float)logl((long double)x);
}
float or_expf(float x) {
  if (x != x) return x;
  if (x > 100.0f) return INFINITY;
  if (x < -110.0f) return 0.0f;
  return (float)expl((long double)x);
}

/* ------------------------------------------------------ pairwise fp64 sums */
static double pairwise(const double* x, uint64_t n) { /* n is a power of two */
  if (n == 1) return x[0];
  return pairwise(x, n / 2) + pairwise(x + n / 2, n / 2);
}

/* Balanced pairwise sum of x[0..n) zero-padded to the next power of two. */
double or_pairwise_sum(const double* x, uint64_t n) {
  uint64_t P = 1;
  while (P < n) P <<= 1;
  double* buf = (double*)calloc(P, sizeof(double));
  memcpy(buf, x, n * sizeof(double));
  double s = pairwise(buf, P);
  free(buf);
  return s;
}

/* ------------------------------------------------------ element access */
static float ld(const void* p, int dtype, uint64_t i) {
  if (dtype == 0) return ((const float*)p)[i];
  uint16_t h = ((const uint16_t*)p)[i];
  return dtype == 1 ? or_bf16_to_f32(h) : or_f16_to_f32(h);
}
static float round_p(float x, int dtype) {
  if (dtype == 0) return x;
  if (dtype == 1) return or_bf16_to_f32(or_f32_to_bf16(x));
  return or_f16_to_f32(or_f32_to_f16(x));
}
static void st(void* p, int dtype, uint64_t i, float v) {
  if (dtype == 0) ((float*)p)[i] = v;
  else if (dtype == 1) ((uint16_t*)p)[i] = or_f32_to_bf16(v);
  else ((uint16_t*)p)[i] = or_f32_to_f16(v);
}

/* ------------------------------------------------------ CoState pieces */
/* decode_blocks, reference costate.py:261-324 (m_hat = alpha*g + scale*sign). */
void or_decode_blocks(const uint8_t* labels, const uint8_t* signs, const float* norms, const uint16_t* amp,
                      float alpha, const float* g, uint64_t n, float q, float* m_hat) {
#pragma omp parallel for schedule(static)
  for (uint64_t i = 0; i < n; ++i) {
    uint64_t b = i / OR_BS;
    float s = 0.0f;
    if (labels[b] == 1) s = norms[b] / q;           /* :306, :313 */
    else if (labels[b] == 2) s = or_f16_to_f32(amp[b]); /* :314 */
    uint32_t bit = (signs[i >> 3] >> (7 - (i & 7))) & 1u; /* :203-209 */
    float sgn = 1.0f - 2.0f * (float)bit;
    float d = s * sgn;                              /* :317-319 */
    float ag = alpha * g[i];
    m_hat[i] = ag + d;                              /* :323 */
  }
}

/* fp32 partial of the 8 products x[i]*y[i], i in [i0, i0 + 8) (0 past n):
 * p_k = fma(x_2k, y_2k, fl(x_2k+1 * y_2k+1)), then fl(fl(p0 + p1) + fl(p2 + p3)). */
static float lane8(const float* x, const float* y, uint64_t n, uint64_t i0) {
  float a[8], b[8], p[4];
  for (int k = 0; k < 8; ++k) {
    uint64_t i = i0 + (uint64_t)k;
    a[k] = i < n ? x[i] : 0.0f;
    b[k] = i < n ? y[i] : 0.0f;
  }
  for (int k = 0; k < 4; ++k) {
    float t = a[2 * k + 1] * b[2 * k + 1];
    p[k] = fmaf(a[2 * k], b[2 * k], t);
  }
  float s01 = p[0] + p[1], s23 = p[2] + p[3];
  return s01 + s23;
}

/* Sum over block b of x*y: fp64 pairwise over its 16 lane partials. */
static double block_dot(const float* x, const float* y, uint64_t n, uint64_t b) {
  double l[OR_BS / 8];
  for (int j = 0; j < OR_BS / 8; ++j) l[j] = (double)lane8(x, y, n, b * OR_BS + 8u * (uint64_t)j);
  return pairwise(l, OR_BS / 8);
}

/* decompose, reference costate.py:22-43. */
float or_decompose(const float* m, const float* g, uint64_t n, float* delta) {
  uint64_t nb = (n + OR_BS - 1) / OR_BS;
  double* bgg = (double*)malloc(nb * sizeof(double));
  double* bmg = (double*)malloc(nb * sizeof(double));
#pragma omp parallel for schedule(static)
  for (uint64_t b = 0; b < nb; ++b) {
    bgg[b] = block_dot(g, g, n, b);
    bmg[b] = block_dot(m, g, n, b);
  }
  float gg = (float)(or_pairwise_sum(bgg, nb) + 0.0);
  float mg = (float)(or_pairwise_sum(bmg, nb) + 0.0);
  free(bgg);
  free(bmg);
  float alpha = gg > 0.0f ? mg / gg : 0.0f;        /* :39-41 */
#pragma omp parallel for schedule(static)
  for (uint64_t i = 0; i < n; ++i) {
    float ag = alpha * g[i];
    delta[i] = m[i] - ag;                          /* :42 */
  }
  return alpha;
}

/* L2 norm of block b of x (zero padded): the block's sum of squares as in
 * block_dot, fp64 sqrt, rounded once. */
static float block_norm(const float* x, uint64_t n, uint64_t b) {
  return (float)sqrt(block_dot(x, x, n, b));
}

/* compute_block_ratios, reference costate.py:51-86. */
void or_block_ratios(const float* delta, const float* m, uint64_t n, float* ratios) {
  uint64_t nb = (n + OR_BS - 1) / OR_BS;
#pragma omp parallel for schedule(static)
  for (uint64_t b = 0; b < nb; ++b) {
    float dn = block_norm(delta, n, b);
    float mn = block_norm(m, n, b);
    ratios[b] = mn == 0.0f ? 0.0f : dn / mn;       /* :81-84 */
  }
}

static int cmp_u32(const void* a, const void* b) {
  uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
  return x < y ? -1 : (x > y ? 1 : 0);
}

/* compute_thresholds, reference costate.py:94-118 (ratios are >= +0 or NaN,
 * so the fp32 bit patterns sort like torch.sort with NaN last). */
void or_thresholds(const float* ratios, uint64_t nb, uint64_t k_lo, uint64_t k_hi, float* tau0, float* tau1) {
  uint32_t* s = (uint32_t*)malloc(nb * sizeof(uint32_t));
  for (uint64_t i = 0; i < nb; ++i) s[i] = f2u(ratios[i]);
  qsort(s, nb, sizeof(uint32_t), cmp_u32);
  *tau0 = u2f(s[k_lo]);
  *tau1 = u2f(s[k_hi]);
  free(s);
}

/* classify_blocks, reference costate.py:126-149. */
void or_classify(const float* ratios, uint64_t nb, float tau0, float tau1, uint8_t* labels) {
  for (uint64_t b = 0; b < nb; ++b) {
    uint8_t l = 0;
    if (ratios[b] >= tau0) l = 1;
    if (ratios[b] >= tau1) l = 2;
    labels[b] = l;
  }
}

/* encode_blocks, reference costate.py:213-258 (+ _pack_signs :157-182). */
void or_encode(const float* delta, uint64_t n, float q, uint8_t* signs, float* norms, uint16_t* amp) {
  uint64_t nb = (n + OR_BS - 1) / OR_BS;
#pragma omp parallel for schedule(static)
  for (uint64_t b = 0; b < nb; ++b) {
    float nd = block_norm(delta, n, b);
    norms[b] = nd;
    amp[b] = or_f32_to_f16(nd / q);
  }
  uint64_t nbytes = (n + 7) / 8;
#pragma omp parallel for schedule(static)
  for (uint64_t j = 0; j < nbytes; ++j) {
    uint32_t byte = 0;
    for (int k = 0; k < 8; ++k) {
      uint64_t i = j * 8 + k;
      uint32_t bit = (i < n && delta[i] < 0.0f) ? 1u : 0u;
      byte |= bit << (7 - k);
    }
    signs[j] = (uint8_t)byte;
  }
}

/* CoStateManager.update, reference costate.py:367-464 (no error feedback).
 * State arrays are updated in place; *alpha is alpha_{t-1} on entry and
 * alpha_t on exit.  m_out receives m_t. */
/* With error feedback (ef, costate.py:409-437) the residual is added to g in
 * the EMA (decompose keeps g); after encoding, ef_error = delta - decode(new
 * encoding, alpha = 0) becomes the residual (has_ef == 0, its first step) or
 * enters its EMA: r = fl(beta1*r) + fl((1-beta1)*ef_error). */
void or_costate_update_ef(const float* g, uint64_t n, float beta1, float one_minus_beta1, float q,
                          uint64_t k_lo, uint64_t k_hi, int has_state, uint8_t* labels, uint8_t* signs,
                          float* norms, uint16_t* amp, float* alpha, int ef, int has_ef, float* ef_residual,
                          float* m_out) {
  uint64_t nb = (n + OR_BS - 1) / OR_BS;
  float* m_hat = (float*)calloc(n, sizeof(float));
  if (has_state) or_decode_blocks(labels, signs, norms, amp, *alpha, g, n, q, m_hat);
#pragma omp parallel for schedule(static)
  for (uint64_t i = 0; i < n; ++i) {
    float gc = (ef && has_ef) ? g[i] + ef_residual[i] : g[i];  /* :410-413 */
    float a = beta1 * m_hat[i];
    float b = one_minus_beta1 * gc;
    m_out[i] = a + b;                              /* :416 */
  }
  float* delta = (float*)malloc(n * sizeof(float));
  float* ratios = (float*)malloc(nb * sizeof(float));
  float al = or_decompose(m_out, g, n, delta);
  or_block_ratios(delta, m_out, n, ratios);
  float t0, t1;
  or_thresholds(ratios, nb, k_lo, k_hi, &t0, &t1);
  or_classify(ratios, nb, t0, t1, labels);
  or_encode(delta, n, q, signs, norms, amp);
  *alpha = al;
  if (ef) {                                        /* :428-437 */
    or_decode_blocks(labels, signs, norms, amp, 0.0f, g, n, q, m_hat);
#pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < n; ++i) {
      float e = delta[i] - m_hat[i];
      if (has_ef) {
        float a = beta1 * ef_residual[i];
        float b = one_minus_beta1 * e;
        ef_residual[i] = a + b;
      } else {
        ef_residual[i] = e;
      }
    }
  }
  free(m_hat);
  free(delta);
  free(ratios);
}

void or_costate_update(const float* g, uint64_t n, float beta1, float one_minus_beta1, float q,
                       uint64_t k_lo, uint64_t k_hi, int has_state, uint8_t* labels, uint8_t* signs,
                       float* norms, uint16_t* amp, float* alpha, float* m_out) {
  or_costate_update_ef(g, n, beta1, one_minus_beta1, q, k_lo, k_hi, has_state, labels, signs, norms, amp, alpha,
                       0, 0, NULL, m_out);
}

/* fused_v_update, reference quantize.py:222-299.  idx (N_pad) and scales
 * (2*nb f16) updated in place; v_out receives v (n).  The draw of element i is
 * the one of element e_base + i (a block-aligned slice of a larger parameter
 * draws as that parameter does). */
static void or_fused_v_update_at(uint8_t* idx, uint16_t* scales, const float* g, uint64_t n, int bits,
                                 float beta2, float one_minus_beta2, uint32_t tid, uint32_t step, uint64_t seed,
                                 uint64_t e_base, float* v_out) {
  uint64_t nb = (n + OR_BS - 1) / OR_BS;
  float nbk = (float)(1u << bits);
#pragma omp parallel for schedule(static)
  for (uint64_t b = 0; b < nb; ++b) {
    float vb[OR_BS], lg[OR_BS];
    float lmin = or_f16_to_f32(scales[2 * b]);
    float lmax = or_f16_to_f32(scales[2 * b + 1]);
    float span = lmax - lmin;                      /* :253-255 */
    float nmin = INFINITY, nmax = -INFINITY;
    int nan_seen = 0;
    float nan_val = 0.0f;
    for (int j = 0; j < OR_BS; ++j) {
      uint64_t i = b * OR_BS + j;
      float t = ((float)idx[i] + 0.5f) / nbk;      /* :256 */
      float lv = lmin + t * span;
      float vo = or_expf(lv);
      float g2 = i < n ? g[i] * g[i] : 0.0f;       /* :259-267 */
      float vb1 = vo * beta2;
      vb[j] = fmaf(one_minus_beta2, g2, vb1);      /* :270 add_(alpha=) is fused */
      float c = vb[j] < 1e-38f ? 1e-38f : vb[j];   /* :275 clamp(min=1e-38) */
      lg[j] = or_logf(c);
      if (i < n) {                                 /* :276-280, NaN propagates */
        if (lg[j] != lg[j]) { if (!nan_seen) { nan_seen = 1; nan_val = lg[j]; } }
        else {
          if (lg[j] < nmin) nmin = lg[j];
          if (lg[j] > nmax) nmax = lg[j];
        }
      }
    }
    if (nan_seen) { nmin = nan_val; nmax = nan_val; }
    scales[2 * b] = or_f32_to_f16(nmin);           /* :281 */
    scales[2 * b + 1] = or_f32_to_f16(nmax);
    float sp = nmax - nmin;
    if (sp < 1e-10f) sp = 1e-10f;                  /* :283 clamp(min=1e-10) */
    float ub[OR_BS];                               /* the block's draws (8 groups of 16) */
    for (int t = 0; t < OR_BS / 16; ++t)
      or_group_uniforms((e_base + b * OR_BS) / 16 + (uint64_t)t, tid, step, seed, ub + 16 * t);
    for (int j = 0; j < OR_BS; ++j) {
      uint64_t i = b * OR_BS + j;
      float c = ((lg[j] - nmin) / sp) * nbk;       /* :284-285 */
      float f = floorf(c);
      float fr = c - f;
      float u = ub[j];
      float r = f + (u < fr ? 1.0f : 0.0f);        /* :288-294 */
      if (r < 0.0f) r = 0.0f;
      if (r > nbk - 1.0f) r = nbk - 1.0f;
      idx[i] = (r != r) ? 0 : (uint8_t)r;
      if (i < n) v_out[i] = vb[j];
    }
  }
}

void or_fused_v_update(uint8_t* idx, uint16_t* scales, const float* g, uint64_t n, int bits, float beta2,
                       float one_minus_beta2, uint32_t tid, uint32_t step, uint64_t seed, float* v_out) {
  or_fused_v_update_at(idx, scales, g, n, bits, beta2, one_minus_beta2, tid, step, seed, 0, v_out);
}

/* dequantize_logscale_nbits, reference quantize.py:183-214 (and decompress_v,
 * oneq.py:51-67): out[i] = exp(lmin + ((idx + 0.5) / 2^bits) * span) for the
 * first n values, each operation rounded to fp32 in the reference's order
 * (the division by 2^bits is exact), exp correctly rounded. */
void or_dequantize(const uint8_t* idx, const uint16_t* scales, uint64_t n, int bits, float* out) {
  float nbk = (float)(1u << bits);
#pragma omp parallel for schedule(static)
  for (uint64_t i = 0; i < n; ++i) {
    uint64_t b = i / OR_BS;
    float lmin = or_f16_to_f32(scales[2 * b]);
    float lmax = or_f16_to_f32(scales[2 * b + 1]);
    float span = lmax - lmin;
    float t = ((float)idx[i] + 0.5f) / nbk;
    float lv = lmin + t * span;
    out[i] = or_expf(lv);
  }
}

/* quantize_logscale_nbits, reference quantize.py:126-180, on v already padded
 * to whole blocks (npad a multiple of 128).  Min / max run over every value
 * of the block (NaN propagates); stochastic != 0 draws u as the step does. */
void or_quantize_logscale(const float* v, uint64_t npad, int bits, int stochastic, uint32_t tid, uint32_t step,
                          uint64_t seed, uint8_t* idx, uint16_t* scales) {
  uint64_t nb = npad / OR_BS;
  float nbk = (float)(1u << bits);
  float top = (float)((double)(1u << bits) - 0.001);  /* clamp(0, n_buckets - 0.001), :179 */
#pragma omp parallel for schedule(static)
  for (uint64_t b = 0; b < nb; ++b) {
    float lg[OR_BS];
    float lmin = INFINITY, lmax = -INFINITY;
    int nan_seen = 0;
    for (int j = 0; j < OR_BS; ++j) {
      float x = v[b * OR_BS + j];
      float c = x < 1e-38f ? 1e-38f : x;              /* clamp(min=1e-38), :155 */
      lg[j] = or_logf(c);
      if (lg[j] != lg[j]) nan_seen = 1;
      else {
        if (lg[j] < lmin) lmin = lg[j];
        if (lg[j] > lmax) lmax = lg[j];
      }
    }
    if (nan_seen) lmin = lmax = NAN;                   /* min / max propagate NaN, :157-158 */
    scales[2 * b] = or_f32_to_f16(lmin);               /* :159 */
    scales[2 * b + 1] = or_f32_to_f16(lmax);
    float sp = lmax - lmin;
    if (sp < 1e-10f) sp = 1e-10f;                      /* :161 */
    for (int j = 0; j < OR_BS; ++j) {
      uint64_t i = b * OR_BS + j;
      float c = ((lg[j] - lmin) / sp) * nbk;           /* :162-163 */
      float q;
      if (stochastic) {                                /* :165-175 */
        float f = floorf(c);
        float u = or_uniform(i, tid, step, seed);
        q = f + (u < c - f ? 1.0f : 0.0f);
        if (q < 0.0f) q = 0.0f;
        if (q > nbk - 1.0f) q = nbk - 1.0f;
      } else {                                         /* :177-178 */
        q = c < 0.0f ? 0.0f : c;
        if (q > top) q = top;
      }
      idx[i] = (q != q) ? 0 : (uint8_t)q;
    }
  }
}

/* ------------------------------------------------------ one parameter's step */
/* OrTensor and the OR_FLAG_* values: tam_oracle.h */

/* TurboAdam._full_step_kernel body for one parameter, reference
 * optimizer.py:97-170 (the caller increments the step counter and supplies
 * the fp32 scalars). */
void or_step_tensor(OrTensor* t, uint64_t seed) {
  uint64_t n = t->n;
  float* g = (float*)malloc(n * sizeof(float));
  float* p = (float*)malloc(n * sizeof(float));
  float* m = (float*)malloc(n * sizeof(float));
  float* v = (float*)malloc(n * sizeof(float));
#pragma omp parallel for schedule(static)
  for (uint64_t i = 0; i < n; ++i) {
    g[i] = ld(t->grad, (int)t->dtype, i);
    p[i] = ld(t->param, (int)t->dtype, i);
  }
  if (t->flags & OR_FLAG_WD)                        /* :106-107 */
#pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < n; ++i) p[i] = round_p(p[i] * t->c_wd, (int)t->dtype);
  if (t->flags & OR_FLAG_COSTATE) {                 /* :110-111 */
    or_costate_update_ef(g, n, t->beta1, t->one_minus_beta1, t->sqrt_block, t->k_lo, t->k_hi,
                         (t->flags & OR_FLAG_HAS_STATE) != 0, t->labels, t->signs, t->norms, t->amp, t->alpha,
                         (t->flags & OR_FLAG_EF) != 0, (t->flags & OR_FLAG_HAS_EF) != 0, t->ef_residual, m);
  } else {                                          /* :113-114 */
#pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < n; ++i) {
      float a = t->exp_avg[i] * t->beta1;
      t->exp_avg[i] = fmaf(t->one_minus_beta1, g[i], a);
      m[i] = t->exp_avg[i];
    }
  }
  if (t->flags & OR_FLAG_COMPRESS_V) {              /* :121-163 */
    or_fused_v_update_at(t->v_idx, t->v_scales, g, n, (int)t->v_bits, t->beta2, t->one_minus_beta2, t->tensor_id,
                         t->step, seed, (uint64_t)t->block0 * OR_BS, v);
  } else {                                          /* :165-167 */
#pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < n; ++i) {
      float a = t->exp_avg_sq[i] * t->beta2;
      float b = t->one_minus_beta2 * g[i];
      t->exp_avg_sq[i] = fmaf(b, g[i], a);
      v[i] = t->exp_avg_sq[i];
    }
  }
#pragma omp parallel for schedule(static)
  for (uint64_t i = 0; i < n; ++i) {
    float vq = v[i] / t->bias_correction2;          /* :163 */
    float den = sqrtf(vq) + t->eps;
    float d2 = den * t->bias_correction1;           /* :170 */
    float num = t->neg_lr * m[i];
    float upd = num / d2;
    p[i] = p[i] + upd;
    st(t->param, (int)t->dtype, i, p[i]);
  }
  free(g);
  free(p);
  free(m);
  free(v);
}

size_t or_struct_size(void) { return sizeof(OrTensor); }
