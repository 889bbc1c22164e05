// tam_step.hip -- gfx950 kernels and C-ABI entry points of the TurboAdam
// packed-state optimizer step.
//
// Work layout.  A block is 128 consecutive elements of one tensor (the
// reference's quantisation / CoState block, utils.py:18).  A tile is 16
// consecutive blocks (2048 elements) of one tensor, aligned on 16-block
// boundaries inside the tensor.  A 256-thread workgroup processes one tile
// at a time: thread t owns elements [8t, 8t+8) of the tile, so the 16 lanes
// t = 16k..16k+15 of one wave64 own block k of the tile.  Tiles of all
// tensors are numbered consecutively (tensor i owns tiles
// [tile0_i, tile0_i + ntiles_i)) and persistent workgroups stride over them,
// so one launch covers the whole parameter list.
//
// Per step (tam_multi_tensor_step):
//   K1 tam_k1_main    every tile: CoState decode + EMA (or fp32 exp_avg EMA),
//                     1Q decode + EMA + stochastic re-quantisation (or fp32
//                     exp_avg_sq), denominator, decoupled weight decay,
//                     parameter update; per-tile fp64 partials of g.g, m.g.
//   K2 tam_k_alpha    one workgroup per CoState tensor: alpha = m.g / g.g.
//   K3 tam_k2_encode  CoState tiles: recompute m, delta = m - alpha*g, sign
//                     bits, block norms, fp16 amplitudes, block ratios.
//   K4 tam_k3_select  one workgroup per CoState tensor: radix selection of the
//                     two order statistics, labels, alpha write-back.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/turboadam_amd.h"
#include "tam_math.h"

#define TAM_WG 256
#define TAM_EPL 8
#define TAM_BPT 16  // blocks per tile
#define TAM_TILE_ELEMS (TAM_BPT * TAM_BLOCK_SIZE)
#define TAM_SEL_WG 1024

// ---------------------------------------------------------------------------
// error reporting
// ---------------------------------------------------------------------------
static thread_local char tam_err_buf[512];

static int tam_fail(int code, const char* fmt, const char* a = "", long b = 0) {
  snprintf(tam_err_buf, sizeof(tam_err_buf), fmt, a, b);
  return code;
}

#define TAM_HIP_CHECK(expr)                                                   \
  do {                                                                        \
    hipError_t e_ = (expr);                                                   \
    if (e_ != hipSuccess)                                                     \
      return tam_fail(TAM_E_HIP, "HIP error in %s: code %ld", #expr, (long)e_); \
  } while (0)

// ---------------------------------------------------------------------------
// element loads / stores (8 consecutive elements per lane)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float tam_load_scalar(const void* base, uint32_t dtype, uint64_t i) {
  if (dtype == TAM_DTYPE_F32) return ((const float*)base)[i];
  const uint16_t h = ((const uint16_t*)base)[i];
  return dtype == TAM_DTYPE_BF16 ? tam_bf16_to_f32(h) : tam_f16_to_f32(h);
}

__device__ __forceinline__ void tam_unpack8_16(uint4 w, uint32_t dtype, float* out) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint16_t lo = (uint16_t)(ws[k] & 0xffffu), hi = (uint16_t)(ws[k] >> 16);
    if (dtype == TAM_DTYPE_BF16) {
      out[2 * k] = tam_bf16_to_f32(lo);
      out[2 * k + 1] = tam_bf16_to_f32(hi);
    } else {
      out[2 * k] = tam_f16_to_f32(lo);
      out[2 * k + 1] = tam_f16_to_f32(hi);
    }
  }
}

// Loads elements [e0, e0+8) (zero beyond n).
__device__ __forceinline__ void tam_load8(const void* base, uint32_t dtype, uint64_t e0, uint64_t n,
                                          bool vec_ok, float* out) {
  if (vec_ok && e0 + TAM_EPL <= n) {
    if (dtype == TAM_DTYPE_F32) {
      const float4* p = (const float4*)((const float*)base + e0);
      const float4 a = p[0], b = p[1];
      out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
      out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
    } else {
      const uint4 w = *(const uint4*)((const uint16_t*)base + e0);
      tam_unpack8_16(w, dtype, out);
    }
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) out[i] = (e0 + i < n) ? tam_load_scalar(base, dtype, e0 + i) : 0.0f;
  }
}

__device__ __forceinline__ uint16_t tam_round16(float x, uint32_t dtype) {
  return dtype == TAM_DTYPE_BF16 ? tam_f32_to_bf16(x) : tam_f32_to_f16(x);
}

// Rounds a value to the parameter dtype and back (R_p).
__device__ __forceinline__ float tam_round_p(float x, uint32_t dtype) {
  if (dtype == TAM_DTYPE_F32) return x;
  if (dtype == TAM_DTYPE_BF16) return tam_bf16_to_f32(tam_f32_to_bf16(x));
  return tam_f16_to_f32(tam_f32_to_f16(x));
}

__device__ __forceinline__ void tam_store8(void* base, uint32_t dtype, uint64_t e0, uint64_t n, bool vec_ok,
                                           const float* v) {
  if (vec_ok && e0 + TAM_EPL <= n) {
    if (dtype == TAM_DTYPE_F32) {
      float4* p = (float4*)((float*)base + e0);
      p[0] = make_float4(v[0], v[1], v[2], v[3]);
      p[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      uint32_t w[4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        w[k] = (uint32_t)tam_round16(v[2 * k], dtype) | ((uint32_t)tam_round16(v[2 * k + 1], dtype) << 16);
      *(uint4*)((uint16_t*)base + e0) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      if (e0 + i < n) {
        if (dtype == TAM_DTYPE_F32) ((float*)base)[e0 + i] = v[i];
        else ((uint16_t*)base)[e0 + i] = tam_round16(v[i], dtype);
      }
    }
  }
}

// fp32 loads/stores of state arrays that may have a ragged end.
__device__ __forceinline__ void tam_load8_f32(const float* base, uint64_t e0, uint64_t n, float* out) {
  tam_load8(base, TAM_DTYPE_F32, e0, n, true, out);
}
__device__ __forceinline__ void tam_store8_f32(float* base, uint64_t e0, uint64_t n, const float* v) {
  tam_store8(base, TAM_DTYPE_F32, e0, n, true, v);
}

// ---------------------------------------------------------------------------
// reductions over the 16 lanes of a block (one DPP row)
// ---------------------------------------------------------------------------
// gfx9 DPP controls: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror
// (lane i <-> 7-i within each half row), row_mirror (lane i <-> 15-i).
#define TAM_DPP_XOR1 0xB1
#define TAM_DPP_XOR2 0x4E
#define TAM_DPP_HALF_MIRROR 0x141
#define TAM_DPP_MIRROR 0x140

template <int CTRL>
__device__ __forceinline__ uint32_t tam_dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float tam_dppf(float v) {
  return tam_u2f(tam_dpp<CTRL>(tam_f2u(v)));
}
template <int CTRL>
__device__ __forceinline__ double tam_dppd(double v) {
  const uint64_t u = tam_d2u(v);
  const uint32_t lo = tam_dpp<CTRL>((uint32_t)u), hi = tam_dpp<CTRL>((uint32_t)(u >> 32));
  return tam_u2d(((uint64_t)hi << 32) | lo);
}

// Balanced pairwise sum of 8 values (adjacent pairing).
__device__ __forceinline__ double tam_pair8(const double* x) {
  return ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
}

// Sum over the 16 lanes of a block with adjacent pairing.  After the two quad
// steps every lane of a quad holds the same value, so the mirrors pair quad 0
// with quad 1 and half 0 with half 1 exactly as a balanced tree does (and
// a + b == b + a), and every lane ends with the same value.
__device__ __forceinline__ double tam_block_sum(double v) {
  v = v + tam_dppd<TAM_DPP_XOR1>(v);
  v = v + tam_dppd<TAM_DPP_XOR2>(v);
  v = v + tam_dppd<TAM_DPP_HALF_MIRROR>(v);
  v = v + tam_dppd<TAM_DPP_MIRROR>(v);
  return v;
}
__device__ __forceinline__ float tam_block_fmin(float v) {  // IEEE minNum; NaN tracked separately
  v = __builtin_fminf(v, tam_dppf<TAM_DPP_XOR1>(v));
  v = __builtin_fminf(v, tam_dppf<TAM_DPP_XOR2>(v));
  v = __builtin_fminf(v, tam_dppf<TAM_DPP_HALF_MIRROR>(v));
  v = __builtin_fminf(v, tam_dppf<TAM_DPP_MIRROR>(v));
  return v;
}
__device__ __forceinline__ float tam_block_fmax(float v) {
  v = __builtin_fmaxf(v, tam_dppf<TAM_DPP_XOR1>(v));
  v = __builtin_fmaxf(v, tam_dppf<TAM_DPP_XOR2>(v));
  v = __builtin_fmaxf(v, tam_dppf<TAM_DPP_HALF_MIRROR>(v));
  v = __builtin_fmaxf(v, tam_dppf<TAM_DPP_MIRROR>(v));
  return v;
}
__device__ __forceinline__ uint32_t tam_block_or(uint32_t v) {
  v |= tam_dpp<TAM_DPP_XOR1>(v);
  v |= tam_dpp<TAM_DPP_XOR2>(v);
  v |= tam_dpp<TAM_DPP_HALF_MIRROR>(v);
  v |= tam_dpp<TAM_DPP_MIRROR>(v);
  return v;
}

// ---------------------------------------------------------------------------
// shared per-element pieces (identical in pass 1 and pass 2 so both see the same m)
// ---------------------------------------------------------------------------
// CoState first moment of elements e0..e0+7 (reference costate.py:398-416):
//   m_hat = has_state ? fl(fl(alpha*g) + s_b*sgn) : 0,  m = fl(fl(b1*m_hat) + fl(ob1*g))
__device__ __forceinline__ void tam_costate_m(const TamTensor& d, uint32_t b, uint64_t e0, float alpha_prev,
                                              const float* g, float* m) {
  const bool has = (d.flags & TAM_FLAG_HAS_STATE) != 0;
  float s = 0.0f;
  uint32_t byte = 0;
  if (has) {
    const uint32_t label = d.labels[b];
    if (label == 1u) s = d.norms[b] / d.sqrt_block;  // costate.py:306 (true division)
    else if (label == 2u) s = tam_f16_to_f32(d.amp[b]);
    if (e0 < d.n) byte = d.signs[e0 >> 3];
  }
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) {
    float mh = 0.0f;
    if (has) {
      const float sd = ((byte >> (7 - i)) & 1u) ? -s : s;  // s * (1 - 2*bit), costate.py:207-209, :317-319
      mh = alpha_prev * g[i] + sd;
    }
    m[i] = d.beta1 * mh + d.one_minus_beta1 * g[i];
  }
}

// Block of a tile and element offset of this thread.
struct TamLane {
  uint32_t bl;   // block within the tile (0..15)
  uint32_t l16;  // lane within the block (0..15)
};

__device__ __forceinline__ TamLane tam_lane() {
  TamLane L;
  L.bl = threadIdx.x >> 4;
  L.l16 = threadIdx.x & 15u;
  return L;
}

// Tensor owning global tile `tile` (binary search over tile0).
__device__ __forceinline__ int tam_find_tensor(const TamTensor* __restrict__ T, int nT, uint32_t tile) {
  int lo = 0, hi = nT - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (T[mid].tile0 <= tile) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// 1Q second moment of one lane's 8 elements (reference quantize.py:222-299)
// ---------------------------------------------------------------------------
// Index of an element: with c = fl(fl(l - lmin)/sp) * 2^bits and u its
// uniform, the reference computes floor(c) + (u < c - floor(c)) clamped to
// [0, 2^bits - 1]; for real c and u in [0,1) that equals ceil(c - u).  The fast
// path evaluates c from the hardware log2 (v_log_f32, whose error against the
// correctly rounded ln is below 2^-21 |ln| for every normal input -- checked
// exhaustively on gfx950) and accepts ceil(c~ - u) only when the whole error
// interval [c~ - u - B, c~ - u + B] lies between the same integers (or clamps
// to the same end); otherwise the element takes the exact path (correctly
// rounded log and division).  lmin and lmax are the correctly rounded logs of
// the block's smallest and largest v (log is monotone, so they equal the min
// and max of the per-element logs).
__device__ __forceinline__ void tam_vpath(const TamTensor& d, uint32_t b, bool bvalid, uint64_t e0,
                                          const TamLane& L, const float* g, float* v, float (*lut)[64],
                                          uint32_t seed_lo, uint32_t seed_hi) {
  const uint32_t bits = d.v_bits;
  const uint32_t nbk = 1u << bits;
  const float fnb = (float)nbk;
  const float inv_nbk = 1.0f / fnb;  // exact power of two
  float lmin0 = 0.0f, span0 = 0.0f;
  uint32_t iw0 = 0, iw1 = 0;
  if (bvalid) {
    const uint32_t sc = ((const uint32_t*)d.v_scales)[b];
    lmin0 = tam_f16_to_f32((uint16_t)(sc & 0xffffu));
    span0 = tam_f16_to_f32((uint16_t)(sc >> 16)) - lmin0;  // quantize.py:253-255
    const uint2 iw = *(const uint2*)(d.v_idx + e0);
    iw0 = iw.x;
    iw1 = iw.y;
  }
  // decode (quantize.py:256): per-block table of the 2^bits values
  float vo[TAM_EPL];
  if (nbk <= 64u) {
    if (bvalid) {
      for (uint32_t k = L.l16; k < nbk; k += 16u) lut[L.bl][k] = tam_expf(lmin0 + ((float)k + 0.5f) * inv_nbk * span0);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      const uint32_t idx = ((i < 4 ? iw0 : iw1) >> (8 * (i & 3))) & 0xffu;
      vo[i] = bvalid ? lut[L.bl][idx & 63u] : 0.0f;
    }
    __syncthreads();
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      const uint32_t idx = ((i < 4 ? iw0 : iw1) >> (8 * (i & 3))) & 0xffu;
      vo[i] = tam_expf(lmin0 + ((float)idx + 0.5f) * inv_nbk * span0);
    }
  }
  // EMA (quantize.py:259-270) and the clamp of :275
  float vc[TAM_EPL];
  float vmn = tam_inf(), vmx = -tam_inf();
  uint32_t nan_seen = 0;
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) {
    const bool valid = e0 + i < d.n;
    const float g2 = valid ? g[i] * g[i] : 0.0f;
    v[i] = __builtin_fmaf(d.one_minus_beta2, g2, vo[i] * d.beta2);
    vc[i] = v[i] < 1e-38f ? 1e-38f : v[i];
    if (valid && bvalid) {
      nan_seen |= tam_isnan(vc[i]) ? 1u : 0u;
      vmn = __builtin_fminf(vmn, vc[i]);
      vmx = __builtin_fmaxf(vmx, vc[i]);
    }
  }
  vmn = tam_block_fmin(vmn);
  vmx = tam_block_fmax(vmx);
  nan_seen = tam_block_or(nan_seen);
  // correctly rounded logs of the extremes: even lanes log(vmin), odd lanes log(vmax)
  const float lx = tam_logf((L.l16 & 1u) ? vmx : vmn);
  const float ly = tam_dppf<TAM_DPP_XOR1>(lx);
  float lmn = (L.l16 & 1u) ? ly : lx;
  float lmx = (L.l16 & 1u) ? lx : ly;
  if (nan_seen) lmn = lmx = tam_qnan();  // torch.min / torch.max propagate NaN
  if (!bvalid) return;
  float sp = lmx - lmn;  // quantize.py:283
  sp = sp < 1e-10f ? 1e-10f : sp;
  if (L.l16 == 0) {
    ((uint32_t*)d.v_scales)[b] = (uint32_t)tam_f32_to_f16(lmn) | ((uint32_t)tam_f32_to_f16(lmx) << 16);
  }
  // certified stochastic rounding
  const double dnb = (double)nbk;
  const double inv_sp = 1.0 / (double)sp;
  const double K = 0x1.62e42fefa39efp-1 * dnb * inv_sp;  // c~ = log2(v) * K + C
  const double C = -(double)lmn * dnb * inv_sp;
  const double K2 = K * (0x1p-21 + 0x1p-50);
  const double Cerr = __builtin_fabs(C) * 0x1p-50 + 0x1p-40;
  const uint64_t quad0 = e0 >> 2;
  const TamU4 r0 = tam_philox_quad(quad0, d.tensor_id, d.step, seed_lo, seed_hi);
  const TamU4 r1 = tam_philox_quad(quad0 + 1, d.tensor_id, d.step, seed_lo, seed_hi);
  const uint32_t rw[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
  uint32_t qb[TAM_EPL];
  uint32_t amb = 0;
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) {
    const double ud = (double)(rw[i] >> 8) * 0x1p-24;
    double q = 0.0;
    bool ok = false;
    if (vc[i] >= 0x1p-126f) {  // normal input (false for NaN)
      const double l2 = (double)__builtin_amdgcn_logf(vc[i]);
      const double ct = __builtin_fma(l2, K, C);
      const double dd = ct - ud;
      const double B = __builtin_fma(__builtin_fabs(l2), K2, __builtin_fma(__builtin_fabs(ct), 0x1p-22, Cerr));
      const double ql = __builtin_ceil(dd - B);
      ok = ql >= dd + B;  // no integer in (dd - B, dd + B): ceil is the same over the interval
      q = ql;
    }
    amb |= ok ? 0u : (1u << i);
    const int qi = (int)q;
    qb[i] = (uint32_t)(qi < 0 ? 0 : (qi > (int)(nbk - 1) ? (int)(nbk - 1) : qi));
  }
  if (amb) {
    // exact path: the reference's own sequence with correctly rounded log and division
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      if (amb & (1u << i)) {
        const float l = tam_logf(vc[i]);
        const float c = ((l - lmn) / sp) * fnb;  // quantize.py:284-285
        const float f = __builtin_floorf(c);
        const float fr = c - f;
        const float u = (float)(rw[i] >> 8) * 0x1p-24f;
        float q = f + (u < fr ? 1.0f : 0.0f);  // quantize.py:288-294
        q = q < 0.0f ? 0.0f : q;
        q = q > fnb - 1.0f ? fnb - 1.0f : q;
        qb[i] = tam_isnan(q) ? 0u : (uint32_t)q;
      }
    }
  }
  const uint32_t ow0 = qb[0] | (qb[1] << 8) | (qb[2] << 16) | (qb[3] << 24);
  const uint32_t ow1 = qb[4] | (qb[5] << 8) | (qb[6] << 16) | (qb[7] << 24);
  *(uint2*)(d.v_idx + e0) = make_uint2(ow0, ow1);
}

// ---------------------------------------------------------------------------
// parameter update (reference optimizer.py:106-107, :163, :170)
// ---------------------------------------------------------------------------
// Exact sequence: q1 = fl(v/bc2), s = fl(sqrt(q1)), den = fl(s + eps),
// t2 = fl(den*bc1), a = fl(-lr*m), upd = fl(a/t2), p = R_p(fl(p + upd)).
// fp32 parameters: q1 comes from the fp64 reciprocal of bc2 when a rounding
// test proves the fp32 rounding, else from the division.  bf16 / fp16
// parameters: a fast sequence with the hardware rsq / rcp gives u~ with
// |u~ - upd| <= 2^-19 |u~| + 2^-148 (the exact sequence's six roundings and
// the fast sequence's five are each 2^-24 relative, both hardware seeds are
// within 2^-23 -- checked exhaustively on gfx950).  With s~ = fl(p + u~),
// fl(p + upd) lies within E = 2^-19 |u~| + 2^-22 |s~| + 2^-148 of s~, so
// R_p(fl(p + upd)) is accepted when R_p(fl(s~ - E)) == R_p(fl(s~ + E)) (R_p and
// fl are monotone); otherwise the exact sequence runs.  The result of a
// 16-bit parameter is returned as its bit pattern in pb.
__device__ __forceinline__ void tam_update(const TamTensor& d, uint32_t dtype, float* p, const float* m,
                                           const float* v, uint16_t* pb) {
  const bool wd = (d.flags & TAM_FLAG_WD) != 0;
  if (dtype == TAM_DTYPE_F32) {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      const double y = (double)v[i] * d.inv_bc2;
      const double e = __builtin_fabs(y) * 0x1p-51;
      float q1 = (float)(y - e);
      if (!(q1 == (float)(y + e))) q1 = v[i] / d.bias_correction2;
      const float den = __builtin_sqrtf(q1) + d.eps;
      const float pv = wd ? p[i] * d.c_wd : p[i];
      p[i] = pv + (d.neg_lr * m[i]) / (den * d.bias_correction1);
    }
    return;
  }
  const bool bf = dtype == TAM_DTYPE_BF16;
  uint32_t amb = 0;
  float pw[TAM_EPL];
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) {
    pw[i] = wd ? tam_round_p(p[i] * d.c_wd, dtype) : p[i];
    const float q = v[i] * d.inv_bc2_f32;
    const float s = q * __builtin_amdgcn_rsqf(q);
    const float t2 = (s + d.eps) * d.bias_correction1;
    const float a = d.neg_lr * m[i];
    const float u = a * __builtin_amdgcn_rcpf(t2);
    const float st = pw[i] + u;
    const float E = __builtin_fmaf(__builtin_fabsf(u), 0x1p-19f, __builtin_fmaf(__builtin_fabsf(st), 0x1p-22f, 0x1p-148f));
    const float lo = st - E, hi = st + E;
    // finite, normal hardware inputs and outputs; NaN fails every comparison
    const bool ok0 = (q >= 0x1p-126f) && (t2 < 0x1p125f) && (__builtin_fabsf(st) < 0x1p126f);
    const float lc = ok0 ? lo : 0.0f, hc = ok0 ? hi : 1.0f;
    const uint16_t rl = bf ? tam_f32_to_bf16_rne(lc) : tam_f32_to_f16(lc);
    const uint16_t rh = bf ? tam_f32_to_bf16_rne(hc) : tam_f32_to_f16(hc);
    const bool ok = ok0 && rl == rh;
    pb[i] = rl;
    amb |= ok ? 0u : (1u << i);
  }
  if (amb) {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      if (amb & (1u << i)) {
        const float den = __builtin_sqrtf(v[i] / d.bias_correction2) + d.eps;
        pb[i] = tam_round16(pw[i] + (d.neg_lr * m[i]) / (den * d.bias_correction1), dtype);
      }
    }
  }
}

// Stores 8 16-bit parameter patterns (elements [e0, e0+8), none beyond n).
__device__ __forceinline__ void tam_store8_bits(void* base, uint64_t e0, uint64_t n, bool vec_ok, const uint16_t* b) {
  if (vec_ok && e0 + TAM_EPL <= n) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = (uint32_t)b[2 * k] | ((uint32_t)b[2 * k + 1] << 16);
    *(uint4*)((uint16_t*)base + e0) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i)
      if (e0 + i < n) ((uint16_t*)base)[e0 + i] = b[i];
  }
}

// ---------------------------------------------------------------------------
// K1: the fused pass over every tile
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(TAM_WG) void tam_k1_main(const TamTensor* __restrict__ T, int nT,
                                                      uint32_t total_tiles, uint32_t seed_lo,
                                                      uint32_t seed_hi, double2* __restrict__ partials) {
  __shared__ float lut[TAM_BPT][64];
  __shared__ double2 wred[TAM_WG / 64];
  const TamLane L = tam_lane();
  int ti = tam_find_tensor(T, nT, blockIdx.x);
  for (uint32_t tile = blockIdx.x; tile < total_tiles; tile += gridDim.x) {
    while (tile >= T[ti].tile0 + T[ti].ntiles) ++ti;
    const TamTensor& d = T[ti];
    const uint32_t b = (tile - d.tile0) * TAM_BPT + L.bl;  // block within the tensor
    const bool bvalid = b < d.nb;
    const uint64_t e0 = (uint64_t)b * TAM_BLOCK_SIZE + L.l16 * TAM_EPL;
    const uint32_t dtype = d.dtype;
    const bool costate = (d.flags & TAM_FLAG_COSTATE) != 0;
    const bool vec_p = (((uintptr_t)d.param | (uintptr_t)d.grad) & 15u) == 0;

    float g[TAM_EPL], p[TAM_EPL], m[TAM_EPL], v[TAM_EPL];
    if (bvalid) {
      tam_load8(d.grad, dtype, e0, d.n, vec_p, g);
      tam_load8(d.param, dtype, e0, d.n, vec_p, p);
    } else {
#pragma unroll
      for (int i = 0; i < TAM_EPL; ++i) g[i] = p[i] = m[i] = v[i] = 0.0f;
    }

    // ---- first moment ---------------------------------------------------
    if (costate) {
      const float alpha_prev = (d.flags & TAM_FLAG_HAS_STATE) ? *d.alpha : 0.0f;
      if (bvalid) tam_costate_m(d, b, e0, alpha_prev, g, m);
      double gg[TAM_EPL], mg[TAM_EPL];
#pragma unroll
      for (int i = 0; i < TAM_EPL; ++i) {
        const bool ok = bvalid && (e0 + i < d.n);
        gg[i] = ok ? (double)g[i] * (double)g[i] : 0.0;
        mg[i] = ok ? (double)m[i] * (double)g[i] : 0.0;
      }
      double sgg = tam_block_sum(tam_pair8(gg));
      double smg = tam_block_sum(tam_pair8(mg));
      // blocks of one wave: adjacent pairs, then pairs of pairs
      sgg = sgg + __shfl_xor(sgg, 16);
      smg = smg + __shfl_xor(smg, 16);
      sgg = sgg + __shfl_xor(sgg, 32);
      smg = smg + __shfl_xor(smg, 32);
      if ((threadIdx.x & 63u) == 0) wred[threadIdx.x >> 6] = make_double2(sgg, smg);
      __syncthreads();
      if (threadIdx.x == 0) {
        const double a = (wred[0].x + wred[1].x) + (wred[2].x + wred[3].x);
        const double c = (wred[0].y + wred[1].y) + (wred[2].y + wred[3].y);
        partials[tile] = make_double2(a, c);
      }
      __syncthreads();  // wred is rewritten by the next tile
    } else if (bvalid) {
      // fp32 exp_avg (optimizer.py:113): m = fma(1-b1, g, fl(m*b1))
      float ea[TAM_EPL];
      tam_load8_f32(d.exp_avg, e0, d.n, ea);
#pragma unroll
      for (int i = 0; i < TAM_EPL; ++i) m[i] = __builtin_fmaf(d.one_minus_beta1, g[i], ea[i] * d.beta1);
      tam_store8_f32(d.exp_avg, e0, d.n, m);
    }

    // ---- second moment --------------------------------------------------
    if (d.flags & TAM_FLAG_COMPRESS_V) {
      tam_vpath(d, b, bvalid, e0, L, g, v, lut, seed_lo, seed_hi);
    } else if (bvalid) {
      // fp32 exp_avg_sq (optimizer.py:166): v = fma(fl((1-b2)*g), g, fl(v*b2))
      float es[TAM_EPL];
      tam_load8_f32(d.exp_avg_sq, e0, d.n, es);
#pragma unroll
      for (int i = 0; i < TAM_EPL; ++i) v[i] = __builtin_fmaf(d.one_minus_beta2 * g[i], g[i], es[i] * d.beta2);
      tam_store8_f32(d.exp_avg_sq, e0, d.n, v);
    }

    // ---- parameter update -----------------------------------------------
    if (bvalid) {
      uint16_t pb[TAM_EPL];
      tam_update(d, dtype, p, m, v, pb);
      if (dtype == TAM_DTYPE_F32) tam_store8(d.param, dtype, e0, d.n, vec_p, p);
      else tam_store8_bits(d.param, e0, d.n, vec_p, pb);
    }
  }
}

// ---------------------------------------------------------------------------
// K2: alpha of every CoState tensor (costate.py:37-41)
// ---------------------------------------------------------------------------
// Balanced pairwise sum of x[0..count) zero-padded to a power of two, by one
// 256-thread workgroup.  Aligned chunks of 2048 values are summed in LDS; the
// chunk sums (a power of two of them, at most 2048) are summed the same way.
__device__ double2 tam_wg_pairwise2(const double2* __restrict__ x, uint32_t count, double2* sh,
                                    double2* chunks) {
  uint32_t P = 1;
  while (P < count) P <<= 1;
  const uint32_t CH = TAM_WG * 8;
  const uint32_t nchunks = P > CH ? P / CH : 1;
  const uint32_t lim = P > CH ? CH : P;
  const uint32_t tid = threadIdx.x;
  for (uint32_t c = 0; c < nchunks; ++c) {
    double a[8], q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t local = tid * 8 + i;
      const uint32_t k = c * CH + local;
      const double2 v = (local < lim && k < count) ? x[k] : make_double2(0.0, 0.0);
      a[i] = v.x;
      q[i] = v.y;
    }
    sh[tid] = make_double2(tam_pair8(a), tam_pair8(q));
    __syncthreads();
    for (uint32_t w = TAM_WG / 2; w >= 1; w >>= 1) {
      double2 s = make_double2(0.0, 0.0);
      if (tid < w) {
        const double2 l = sh[2 * tid], r = sh[2 * tid + 1];
        s = make_double2(l.x + r.x, l.y + r.y);
      }
      __syncthreads();
      if (tid < w) sh[tid] = s;
      __syncthreads();
    }
    if (tid == 0) chunks[c] = sh[0];
    __syncthreads();
  }
  for (uint32_t w = nchunks / 2; w >= 1; w >>= 1) {  // w <= 1024: at most 4 pairs per thread
    double2 s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = tid + j * TAM_WG;
      if (i < w) {
        const double2 l = chunks[2 * i], r = chunks[2 * i + 1];
        s[j] = make_double2(l.x + r.x, l.y + r.y);
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = tid + j * TAM_WG;
      if (i < w) chunks[i] = s[j];
    }
    __syncthreads();
  }
  return chunks[0];
}

__global__ __launch_bounds__(TAM_WG) void tam_k_alpha(const TamTensor* __restrict__ T,
                                                      const double2* __restrict__ partials,
                                                      float* __restrict__ alpha_new) {
  __shared__ double2 sh[TAM_WG];
  __shared__ double2 chunks[2048];
  const TamTensor& d = T[blockIdx.x];
  if (!(d.flags & TAM_FLAG_COSTATE)) return;
  const double2 s = tam_wg_pairwise2(partials + d.tile0, d.ntiles, sh, chunks);
  if (threadIdx.x == 0) {
    // dot products round to fp32 once; +0.0 makes an exact-zero sum +0
    const float gg = (float)(s.x + 0.0);
    const float mg = (float)(s.y + 0.0);
    alpha_new[blockIdx.x] = gg > 0.0f ? mg / gg : 0.0f;
  }
}

// ---------------------------------------------------------------------------
// K3: CoState encode (costate.py:419-425, :213-258) and block ratios (:51-86)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(TAM_WG) void tam_k2_encode(const TamTensor* __restrict__ T, int nT,
                                                        uint32_t total_tiles,
                                                        const float* __restrict__ alpha_new,
                                                        float* __restrict__ ratios) {
  const TamLane L = tam_lane();
  int ti = tam_find_tensor(T, nT, blockIdx.x);
  for (uint32_t tile = blockIdx.x; tile < total_tiles; tile += gridDim.x) {
    while (tile >= T[ti].tile0 + T[ti].ntiles) ++ti;
    const TamTensor& d = T[ti];
    if (!(d.flags & TAM_FLAG_COSTATE)) continue;  // uniform over the workgroup
    const uint32_t b = (tile - d.tile0) * TAM_BPT + L.bl;
    const bool bvalid = b < d.nb;
    const uint64_t e0 = (uint64_t)b * TAM_BLOCK_SIZE + L.l16 * TAM_EPL;
    const bool vec_g = ((uintptr_t)d.grad & 15u) == 0;
    float g[TAM_EPL], m[TAM_EPL];
    double dd[TAM_EPL], mm[TAM_EPL];
    uint32_t sbyte = 0;
    if (bvalid) {
      tam_load8(d.grad, d.dtype, e0, d.n, vec_g, g);
      const float alpha_prev = (d.flags & TAM_FLAG_HAS_STATE) ? *d.alpha : 0.0f;
      tam_costate_m(d, b, e0, alpha_prev, g, m);
      const float a = alpha_new[ti];
#pragma unroll
      for (int i = 0; i < TAM_EPL; ++i) {
        const bool ok = e0 + i < d.n;
        const float delta = ok ? m[i] - a * g[i] : 0.0f;  // costate.py:42
        dd[i] = (double)delta * (double)delta;
        mm[i] = ok ? (double)m[i] * (double)m[i] : 0.0;
        sbyte |= (delta < 0.0f ? 1u : 0u) << (7 - i);  // costate.py:170-181
      }
    } else {
#pragma unroll
      for (int i = 0; i < TAM_EPL; ++i) dd[i] = mm[i] = 0.0;
    }
    const double sd = tam_block_sum(tam_pair8(dd));
    const double sm = tam_block_sum(tam_pair8(mm));
    if (bvalid) {
      if (e0 < d.n) d.signs[e0 >> 3] = (uint8_t)sbyte;
      if (L.l16 == 0) {
        const float nd = (float)__builtin_sqrt(sd);
        const float nm = (float)__builtin_sqrt(sm);
        d.norms[b] = nd;                                   // costate.py:241
        d.amp[b] = tam_f32_to_f16(nd / d.sqrt_block);     // costate.py:248
        ratios[d.ratio_off + b] = nm == 0.0f ? 0.0f : nd / nm;  // costate.py:81-84
      }
    }
  }
}

// ---------------------------------------------------------------------------
// K4: order statistics of the ratios (costate.py:114-118), labels
// (costate.py:146-148), alpha write-back (costate.py:443-454)
// ---------------------------------------------------------------------------
// Ratios are >= +0 or NaN, so their fp32 bit patterns order like torch.sort
// (NaN last).  The selection is an MSD radix select on those patterns: a
// min/max pass finds the bits all keys share, then 11-bit digits below the
// highest differing bit are histogrammed in LDS (keys of similar magnitude
// spread over the bins instead of piling into a few), at most three passes.

// Exclusive prefix sum over the 1024 threads of the workgroup.
__device__ uint32_t tam_wg_excl_scan(uint32_t v, uint32_t* wsum) {
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  uint32_t inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t t = __shfl_up(inc, off);
    if (lane >= (uint32_t)off) inc += t;
  }
  if (lane == 63u) wsum[w] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t acc = 0;
    for (int i = 0; i < TAM_SEL_WG / 64; ++i) {
      const uint32_t t = wsum[i];
      wsum[i] = acc;
      acc += t;
    }
  }
  __syncthreads();
  const uint32_t r = wsum[w] + inc - v;
  __syncthreads();
  return r;
}

__device__ uint32_t tam_wg_reduce_u32(uint32_t v, bool is_max, uint32_t* wsum) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t t = __shfl_xor(v, off);
    v = is_max ? (t > v ? t : v) : (t < v ? t : v);
  }
  if ((threadIdx.x & 63u) == 0) wsum[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t r = wsum[0];
  for (int i = 1; i < TAM_SEL_WG / 64; ++i) r = is_max ? (wsum[i] > r ? wsum[i] : r) : (wsum[i] < r ? wsum[i] : r);
  __syncthreads();
  return r;
}

// Visits every key of a tensor: 16 keys per thread in flight (four uint4
// loads), then the < 4 trailing keys.  `keys` is 16-byte aligned.
template <typename F>
__device__ __forceinline__ void tam_for_keys(const uint32_t* __restrict__ keys, uint32_t nb, F&& f) {
  const uint4* k4 = (const uint4*)keys;
  const uint32_t n4 = nb >> 2;
  const uint32_t stride = TAM_SEL_WG;
  uint32_t i = threadIdx.x;
  for (; i + 3 * stride < n4; i += 4 * stride) {
    const uint4 a = k4[i], b = k4[i + stride], c = k4[i + 2 * stride], e = k4[i + 3 * stride];
    f(a.x); f(a.y); f(a.z); f(a.w);
    f(b.x); f(b.y); f(b.z); f(b.w);
    f(c.x); f(c.y); f(c.z); f(c.w);
    f(e.x); f(e.y); f(e.z); f(e.w);
  }
  for (; i < n4; i += stride) {
    const uint4 a = k4[i];
    f(a.x); f(a.y); f(a.z); f(a.w);
  }
  const uint32_t t = (n4 << 2) + threadIdx.x;
  if (t < nb) f(keys[t]);
}

__global__ __launch_bounds__(TAM_SEL_WG) void tam_k3_select(const TamTensor* __restrict__ T,
                                                            const float* __restrict__ alpha_new,
                                                            const float* __restrict__ ratios) {
  __shared__ uint32_t hist[2][2048];
  __shared__ uint32_t wsum[TAM_SEL_WG / 64];
  __shared__ uint32_t sel_prefix[2], sel_k[2];
  const TamTensor& d = T[blockIdx.x];
  if (!(d.flags & TAM_FLAG_COSTATE)) return;
  const uint32_t nb = d.nb;
  const uint32_t* keys = (const uint32_t*)(ratios + d.ratio_off);
  const uint32_t tid = threadIdx.x;
  uint32_t kmin = 0xffffffffu, kmax = 0u;
  tam_for_keys(keys, nb, [&](uint32_t k) {
    kmin = k < kmin ? k : kmin;
    kmax = k > kmax ? k : kmax;
  });
  kmin = tam_wg_reduce_u32(kmin, false, wsum);
  kmax = tam_wg_reduce_u32(kmax, true, wsum);
  if (tid == 0) {
    sel_prefix[0] = sel_prefix[1] = kmin;  // bits above the highest differing bit
    sel_k[0] = d.k_lo;
    sel_k[1] = d.k_hi;
  }
  __syncthreads();
  const uint32_t diff = kmin ^ kmax;
  int top = diff ? 31 - __builtin_clz(diff) : -1;  // highest differing bit
  uint32_t mask = top >= 31 ? 0u : (0xffffffffu << (top + 1));
  if (top >= 0 && tid == 0) sel_prefix[0] = sel_prefix[1] = kmin & mask;
  __syncthreads();
  while (top >= 0) {
    const int sh = top >= 10 ? top - 10 : 0;
    const uint32_t dmask = (1u << (top - sh + 1)) - 1u;
    for (uint32_t i = tid; i < 2048; i += TAM_SEL_WG) hist[0][i] = hist[1][i] = 0;
    __syncthreads();
    const uint32_t p0 = sel_prefix[0], p1 = sel_prefix[1];
    const bool same = p0 == p1;
    tam_for_keys(keys, nb, [&](uint32_t key) {
      const uint32_t dg = (key >> sh) & dmask;
      const uint32_t km = key & mask;
      if (km == p0) atomicAdd(&hist[0][dg], 1u);
      if (!same && km == p1) atomicAdd(&hist[1][dg], 1u);
    });
    __syncthreads();
    for (int t = 0; t < 2; ++t) {
      const int src = same ? 0 : t;
      const uint32_t h0 = hist[src][2 * tid], h1 = hist[src][2 * tid + 1];
      const uint32_t pre = tam_wg_excl_scan(h0 + h1, wsum);
      const uint32_t k = sel_k[t];
      __syncthreads();
      if (k >= pre && k < pre + h0 + h1) {
        const bool first = k < pre + h0;
        const uint32_t digit = 2 * tid + (first ? 0u : 1u);
        sel_k[t] = k - (first ? pre : pre + h0);
        sel_prefix[t] |= digit << sh;
      }
      __syncthreads();
    }
    mask |= dmask << sh;
    top = sh - 1;
  }
  const float tau0 = tam_u2f(sel_prefix[0]);
  const float tau1 = tam_u2f(sel_prefix[1]);
  const float* r = ratios + d.ratio_off;
  for (uint32_t i = tid; i < nb; i += TAM_SEL_WG) {
    const float x = r[i];
    d.labels[i] = x >= tau1 ? (uint8_t)2 : (x >= tau0 ? (uint8_t)1 : (uint8_t)0);
  }
  if (tid == 0) *d.alpha = alpha_new[blockIdx.x];
}

// ---------------------------------------------------------------------------
// utility kernels
// ---------------------------------------------------------------------------
__global__ void tam_k_v_dequantize(const uint8_t* __restrict__ idx, const uint16_t* __restrict__ scales,
                                   uint64_t n, uint32_t bits, float* __restrict__ out) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint64_t b = i / TAM_BLOCK_SIZE;
  const float lmin = tam_f16_to_f32(scales[2 * b]);
  const float lmax = tam_f16_to_f32(scales[2 * b + 1]);
  const float span = lmax - lmin;
  const float inv_nbk = 1.0f / (float)(1u << bits);
  out[i] = tam_expf(lmin + ((float)idx[i] + 0.5f) * inv_nbk * span);
}

__global__ void tam_k_philox_uniforms(uint32_t tid, uint32_t step, uint32_t seed_lo, uint32_t seed_hi,
                                      uint64_t count, float* __restrict__ out) {
  const uint64_t q = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q * 4 >= count) return;
  const TamU4 r = tam_philox_quad(q, tid, step, seed_lo, seed_hi);
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
  for (int k = 0; k < 4; ++k)
    if (q * 4 + k < count) out[q * 4 + k] = tam_u01(w[k]);
}

__global__ void tam_k_math_eval(int fn, const float* __restrict__ in, float* __restrict__ out, uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float x = in[i];
  float y;
  switch (fn) {
    case 0: y = tam_logf(x); break;
    case 1: y = tam_expf(x); break;
    case 2: y = tam_f16_to_f32(tam_f32_to_f16(x)); break;
    case 3: y = tam_bf16_to_f32(tam_f32_to_bf16(x)); break;
    case 4: y = __builtin_sqrtf(x); break;
    case 5: y = tam_bf16_to_f32(tam_f32_to_bf16_rne(x)); break;
    default: y = x; break;
  }
  out[i] = y;
}

// ---------------------------------------------------------------------------
// host entry points
// ---------------------------------------------------------------------------
static int tam_device_cus(void) {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cus[dev] = v;
  }
  return cus[dev];
}

static uint64_t tam_align_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

extern "C" {

int tam_abi_version(void) { return TAM_ABI_VERSION; }

size_t tam_struct_size(int which) {
  if (which == 0) return sizeof(TamTensor);
  if (which == 1) return sizeof(TamStepInfo);
  return 0;
}

const char* tam_last_error(void) { return tam_err_buf; }

int tam_prepare(TamTensor* tensors, int n_tensors, TamStepInfo* info) {
  tam_err_buf[0] = 0;
  if (!info || n_tensors < 0 || (n_tensors > 0 && !tensors)) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  uint64_t tiles = 0, ratio_blocks = 0;
  uint32_t ncs = 0;
  for (int i = 0; i < n_tensors; ++i) {
    TamTensor& t = tensors[i];
    if (t.n == 0) return tam_fail(TAM_E_INVALID, "%stensor %ld has no elements", "", i);
    if (t.dtype > TAM_DTYPE_F16) return tam_fail(TAM_E_INVALID, "%stensor %ld: unknown dtype", "", i);
    if (!t.param || !t.grad) return tam_fail(TAM_E_INVALID, "%stensor %ld: null param/grad", "", i);
    const uint64_t nb = (t.n + TAM_BLOCK_SIZE - 1) / TAM_BLOCK_SIZE;
    if (nb > (1ull << 31)) return tam_fail(TAM_E_INVALID, "%stensor %ld too large", "", i);
    const uint64_t nt = (nb + TAM_BPT - 1) / TAM_BPT;
    if (nt > (1ull << 22)) return tam_fail(TAM_E_INVALID, "%stensor %ld too large", "", i);
    if (t.flags & TAM_FLAG_COMPRESS_V) {
      if (!(t.v_bits == 2 || t.v_bits == 3 || t.v_bits == 4 || t.v_bits == 6 || t.v_bits == 8))
        return tam_fail(TAM_E_INVALID, "%stensor %ld: v_bits must be 2, 3, 4, 6 or 8", "", i);
      if (!t.v_idx || !t.v_scales) return tam_fail(TAM_E_INVALID, "%stensor %ld: null v state", "", i);
      if (((uintptr_t)t.v_idx & 7u) || ((uintptr_t)t.v_scales & 3u))
        return tam_fail(TAM_E_INVALID, "%stensor %ld: misaligned v state", "", i);
    } else if (!t.exp_avg_sq || ((uintptr_t)t.exp_avg_sq & 15u)) {
      return tam_fail(TAM_E_INVALID, "%stensor %ld: exp_avg_sq null or misaligned", "", i);
    }
    if (t.flags & TAM_FLAG_COSTATE) {
      if (!t.signs || !t.labels || !t.norms || !t.amp || !t.alpha)
        return tam_fail(TAM_E_INVALID, "%stensor %ld: null CoState state", "", i);
      if (t.k_lo >= nb || t.k_hi >= nb) return tam_fail(TAM_E_INVALID, "%stensor %ld: rank out of range", "", i);
      t.ratio_off = ratio_blocks;
      ratio_blocks += (nb + 3) & ~3ull;  // 16-byte aligned per tensor
      ++ncs;
    } else if (!t.exp_avg || ((uintptr_t)t.exp_avg & 15u)) {
      return tam_fail(TAM_E_INVALID, "%stensor %ld: exp_avg null or misaligned", "", i);
    }
    t.nb = (uint32_t)nb;
    t.ntiles = (uint32_t)nt;
    t.tile0 = (uint32_t)tiles;
    tiles += nt;
    if (tiles > 0xffffffffull) return tam_fail(TAM_E_INVALID, "%stoo many tiles", "", 0);
  }
  memset(info, 0, sizeof(*info));
  info->n_tensors = n_tensors;
  info->total_tiles = (uint32_t)tiles;
  info->n_costate = ncs;
  info->ratio_blocks = ratio_blocks;
  uint64_t off = 0;
  info->off_partials = off;
  off = tam_align_up(off + tiles * sizeof(double2), 256);
  info->off_alpha = off;
  off = tam_align_up(off + (uint64_t)n_tensors * sizeof(float), 256);
  info->off_ratios = off;
  off = tam_align_up(off + ratio_blocks * sizeof(float), 256);
  info->ws_bytes = off;
  return TAM_OK;
}

static int tam_launch_pass(int pass, const TamTensor* d_tensors, const TamStepInfo* info, uint64_t seed,
                           void* workspace, size_t ws_bytes, hipStream_t s) {
  if (!info || (info->n_tensors > 0 && !d_tensors)) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (pass < 0 || pass > 3) return tam_fail(TAM_E_INVALID, "%sunknown pass %ld", "", pass);
  if (info->n_tensors == 0 || info->total_tiles == 0) return TAM_OK;
  if (!workspace || ws_bytes < info->ws_bytes)
    return tam_fail(TAM_E_WORKSPACE, "%sworkspace too small: need %ld bytes", "", (long)info->ws_bytes);
  if (pass > 0 && info->n_costate == 0) return TAM_OK;
  char* ws = (char*)workspace;
  double2* partials = (double2*)(ws + info->off_partials);
  float* alpha_new = (float*)(ws + info->off_alpha);
  float* ratios = (float*)(ws + info->off_ratios);
  const int cus = tam_device_cus();
  const uint32_t grid = info->total_tiles < (uint32_t)(cus * 8) ? info->total_tiles : (uint32_t)(cus * 8);
  switch (pass) {
    case 0:
      hipLaunchKernelGGL(tam_k1_main, dim3(grid), dim3(TAM_WG), 0, s, d_tensors, info->n_tensors,
                         info->total_tiles, (uint32_t)seed, (uint32_t)(seed >> 32), partials);
      break;
    case 1:
      hipLaunchKernelGGL(tam_k_alpha, dim3(info->n_tensors), dim3(TAM_WG), 0, s, d_tensors, partials, alpha_new);
      break;
    case 2:
      hipLaunchKernelGGL(tam_k2_encode, dim3(grid), dim3(TAM_WG), 0, s, d_tensors, info->n_tensors,
                         info->total_tiles, alpha_new, ratios);
      break;
    default:
      hipLaunchKernelGGL(tam_k3_select, dim3(info->n_tensors), dim3(TAM_SEL_WG), 0, s, d_tensors, alpha_new,
                         ratios);
      break;
  }
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

int tam_step_pass(int pass, const TamTensor* d_tensors, const TamStepInfo* info, uint64_t seed, void* workspace,
                  size_t ws_bytes, void* stream) {
  tam_err_buf[0] = 0;
  return tam_launch_pass(pass, d_tensors, info, seed, workspace, ws_bytes, (hipStream_t)stream);
}

int tam_multi_tensor_step(const TamTensor* d_tensors, const TamTensor* h_tensors, const TamStepInfo* info,
                          uint64_t seed, void* workspace, size_t ws_bytes, void* stream) {
  tam_err_buf[0] = 0;
  (void)h_tensors;
  for (int pass = 0; pass < 4; ++pass) {
    const int rc = tam_launch_pass(pass, d_tensors, info, seed, workspace, ws_bytes, (hipStream_t)stream);
    if (rc != TAM_OK) return rc;
  }
  return TAM_OK;
}

int tam_v_dequantize(const uint8_t* v_idx, const uint16_t* v_scales, uint64_t n, uint32_t v_bits, float* out,
                     void* stream) {
  tam_err_buf[0] = 0;
  if (!v_idx || !v_scales || !out) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (!(v_bits == 2 || v_bits == 3 || v_bits == 4 || v_bits == 6 || v_bits == 8))
    return tam_fail(TAM_E_INVALID, "%sv_bits must be 2, 3, 4, 6 or 8", "");
  if (n == 0) return TAM_OK;
  const uint64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(tam_k_v_dequantize, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, v_idx,
                     v_scales, n, v_bits, out);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

int tam_philox_uniforms(uint32_t tensor_id, uint32_t step, uint64_t seed, uint64_t count, float* out,
                        void* stream) {
  tam_err_buf[0] = 0;
  if (!out) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (count == 0) return TAM_OK;
  const uint64_t quads = (count + 3) / 4;
  const uint64_t blocks = (quads + 255) / 256;
  hipLaunchKernelGGL(tam_k_philox_uniforms, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream,
                     tensor_id, step, (uint32_t)seed, (uint32_t)(seed >> 32), count, out);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

int tam_math_eval(int fn, const float* in, float* out, uint64_t n, void* stream) {
  tam_err_buf[0] = 0;
  if (!in || !out) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (fn < 0 || fn > 5) return tam_fail(TAM_E_INVALID, "%sunknown function %ld", "", fn);
  if (n == 0) return TAM_OK;
  const uint64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(tam_k_math_eval, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, fn, in, out, n);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

}  // extern "C"
