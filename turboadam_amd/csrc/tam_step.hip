// tam_step.hip -- gfx950 kernels and C-ABI entry points of the TurboAdam
// packed-state optimizer step.
//
// Work layout.  A block is 128 consecutive elements of one tensor (the
// reference's quantisation / CoState block, utils.py:18).  A tile is 16
// consecutive blocks (2048 elements) of one tensor, aligned on 16-block
// boundaries inside the tensor.  A 256-thread workgroup processes one tile
// at a time: thread t owns elements [8t, 8t+8) of the tile, so the 16 lanes
// t = 16k..16k+15 of one wave64 own block k of the tile and each wave owns a
// quarter tile (4 blocks); the waves never synchronise with each other.
// Tiles of all tensors are numbered consecutively (tensor i owns tiles
// [tile0_i, tile0_i + ntiles_i)) and persistent workgroups stride over them,
// so one launch covers the whole parameter list.
//
// Per step (tam_multi_tensor_step), four passes:
//   pass 0  tam_k1_main_<dtype> (full quarters; one kernel per parameter dtype
//           present) and tam_k1_tail (the other quarters): CoState decode + EMA
//           (or fp32 exp_avg EMA), 1Q decode + EMA + stochastic
//           re-quantisation (or fp32 exp_avg_sq), denominator, decoupled
//           weight decay, parameter update; per-quarter-tile partials of
//           g.g and m.g (fp32 per lane, fp64 across lanes and blocks).
//   pass 1  tam_k_alpha_chunks, tam_k_alpha: alpha = m.g / g.g per CoState
//           tensor (pairwise trees over the partials).
//   pass 2  tam_k2_encode: CoState tiles: recompute m, delta = m - alpha*g,
//           sign bits, block norms, fp16 amplitudes, block ratios.
//   pass 3  tam_k_sel_minmax, tam_k_sel_hist and tam_k_sel_pick (three
//           rounds), tam_k_sel_labels: radix selection of the two order
//           statistics over slices of the ratios, labels, alpha write-back.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <atomic>
#include <stdio.h>
#include <string.h>

#include "../../include/turboadam_amd.h"
#include "tam_math.h"

#define TAM_WG 256
#define TAM_EPL 8
#define TAM_BPT 16  // blocks per tile
#define TAM_TILE_ELEMS (TAM_BPT * TAM_BLOCK_SIZE)

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
// fallback counters (measurement builds only: -DTAM_STATS=1)
// ---------------------------------------------------------------------------
// How often the certified fast paths of pass 0's full units hand elements to
// the exact sequence: lanes (per half unit) whose re-quantisation runs the
// exact path, elements it recomputes, lanes whose 16-bit update runs the exact
// sequence, and pairs it recomputes.  Read with tam_stats_read, which exists
// only in such builds; the product library has neither.
#ifndef TAM_STATS
#define TAM_STATS 0
#endif
enum { TAM_ST_VQ_LANES, TAM_ST_VQ_ELEMS, TAM_ST_UPD_LANES, TAM_ST_UPD_PAIRS, TAM_ST_COUNT };
#if TAM_STATS
__device__ unsigned long long tam_stats[TAM_ST_COUNT];
#define TAM_STAT(i) atomicAdd(&tam_stats[i], 1ull)
#else
#define TAM_STAT(i) ((void)0)
#endif

// ---------------------------------------------------------------------------
// global-memory access
// ---------------------------------------------------------------------------
// Device pointers read from a TamTensor are generic (flat) pointers; casting
// them to the global address space lets the compiler emit global_load /
// global_store, which wait on the vector-memory counter only (flat accesses
// also hold the LDS counter, so every LDS wait would wait on them as well).
#define TAM_GLOBAL __attribute__((address_space(1)))
#define TAM_LDS __attribute__((address_space(3)))
typedef float TamF4 __attribute__((ext_vector_type(4)));
typedef uint32_t TamW4 __attribute__((ext_vector_type(4)));
typedef uint32_t TamW2 __attribute__((ext_vector_type(2)));
typedef double TamD2 __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ TAM_GLOBAL T* tam_g(T* p) {
  return (TAM_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ const TAM_GLOBAL T* tam_g(const T* p) {
  return (const TAM_GLOBAL T*)p;
}

// 16-bit element bits -> fp32 (exact)
template <uint32_t DT>
__device__ __forceinline__ float tam_h2f(uint32_t h) {
  return DT == TAM_DTYPE_BF16 ? tam_u2f(h << 16) : tam_f16_to_f32((uint16_t)h);
}

// Rounds to the parameter dtype (round to nearest even); NaN gives a quiet NaN.
template <uint32_t DT>
__device__ __forceinline__ uint16_t tam_round16_hw(float x) {
  return DT == TAM_DTYPE_BF16 ? tam_f32_to_bf16_rne(x) : tam_f32_to_f16(x);
}

// The 8 16-bit elements of a 16-byte word as fp32 (exact).
template <uint32_t DT>
__device__ __forceinline__ void tam_unpack8(TamW4 w, float* out) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    out[2 * k] = tam_h2f<DT>(ws[k] & 0xffffu);
    out[2 * k + 1] = tam_h2f<DT>(ws[k] >> 16);
  }
}

// Elements [e0, e0+8) of a parameter or gradient.  FULL: all 8 exist and the
// array is 16-byte aligned; otherwise only the first nv exist (the rest read 0).
template <uint32_t DT, bool FULL>
__device__ __forceinline__ void tam_ld8(const void* base, uint64_t e0, uint32_t nv, float* out) {
  if (DT == TAM_DTYPE_F32) {
    const float* b = (const float*)base + e0;
    if (FULL) {
      const TamF4 a = tam_g((const TamF4*)b)[0], c = tam_g((const TamF4*)b)[1];
      out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
      out[4] = c.x; out[5] = c.y; out[6] = c.z; out[7] = c.w;
    } else {
#pragma unroll
      for (int i = 0; i < TAM_EPL; ++i) out[i] = (uint32_t)i < nv ? tam_g(b)[i] : 0.0f;
    }
  } else {
    const uint16_t* b = (const uint16_t*)base + e0;
    if (FULL) {
      tam_unpack8<DT>(tam_g((const TamW4*)b)[0], out);
    } else {
#pragma unroll
      for (int i = 0; i < TAM_EPL; ++i) out[i] = (uint32_t)i < nv ? tam_h2f<DT>(tam_g(b)[i]) : 0.0f;
    }
  }
}

// fp32 state arrays (exp_avg / exp_avg_sq, 16-byte aligned)
template <bool FULL>
__device__ __forceinline__ void tam_ld8_f32(const float* base, uint64_t e0, uint32_t nv, float* out) {
  tam_ld8<TAM_DTYPE_F32, FULL>(base, e0, nv, out);
}
template <bool FULL>
__device__ __forceinline__ void tam_st8_f32(float* base, uint64_t e0, uint32_t nv, const float* v) {
  float* b = base + e0;
  if (FULL) {
    tam_g((TamF4*)b)[0] = TamF4{v[0], v[1], v[2], v[3]};
    tam_g((TamF4*)b)[1] = TamF4{v[4], v[5], v[6], v[7]};
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i)
      if ((uint32_t)i < nv) tam_g(b)[i] = v[i];
  }
}

// 16-bit parameter bit patterns, two per word (element 2k in the low half of
// word k, 2k + 1 in the high half)
template <bool FULL>
__device__ __forceinline__ void tam_st8_bits(void* base, uint64_t e0, uint32_t nv, const uint32_t* pw2) {
  uint16_t* b = (uint16_t*)base + e0;
  if (FULL) {
    tam_g((TamW4*)b)[0] = TamW4{pw2[0], pw2[1], pw2[2], pw2[3]};
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i)
      if ((uint32_t)i < nv) tam_g(b)[i] = (uint16_t)(pw2[i >> 1] >> (16 * (i & 1)));
  }
}

// Rounds a value to a 16-bit parameter dtype (software round to nearest even,
// NaN -> canonical quiet NaN, as torch's conversion).
__device__ __forceinline__ uint16_t tam_round16(float x, uint32_t dtype) {
  return dtype == TAM_DTYPE_BF16 ? tam_f32_to_bf16(x) : tam_f32_to_f16(x);
}

// ---------------------------------------------------------------------------
// reductions over the 16 lanes of a block (one DPP row)
// ---------------------------------------------------------------------------
// gfx9 DPP controls: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror
// (lane i <-> 7-i within each half row), row_mirror (lane i <-> 15-i),
// row_ror:4 and row_ror:8 (lane i reads lane (i - 4) mod 16, (i - 8) mod 16).
#define TAM_DPP_XOR1 0xB1
#define TAM_DPP_XOR2 0x4E
#define TAM_DPP_HALF_MIRROR 0x141
#define TAM_DPP_MIRROR 0x140
#define TAM_DPP_ROR4 0x124
#define TAM_DPP_ROR8 0x128

// Every control used here reads a lane of the same row, so no lane is out of
// range and bound_ctrl (read 0 from an invalid lane) never applies; with it
// set the compiler needs no copy of an `old` value.
template <int CTRL>
__device__ __forceinline__ uint32_t tam_dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
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

// Value of `v` in lane `l` of the wave (uniform result).
__device__ __forceinline__ double tam_readlane_d(double v, int l) {
  const uint64_t u = tam_d2u(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
  return tam_u2d(((uint64_t)hi << 32) | lo);
}

// Balanced pairwise sum of 8 values (adjacent pairing).
__device__ __forceinline__ double tam_pair8(const double* x) {
  return ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
}
// A lane's partial of a dot product or sum of squares (the reduction contract
// of the alpha dots and the block norms): the 8 products a[i]*b[i] of fp32
// values in an fp32 pairwise tree whose first level is fused,
// p_k = fma(a_2k, b_2k, fl(a_2k+1 * b_2k+1)), then fl(fl(p0 + p1) + fl(p2 + p3)).
// The callers widen it to fp64 for the sums across lanes and blocks.
__device__ __forceinline__ float tam_lane_dot(const float* a, const float* b) {
  const float p0 = __builtin_fmaf(a[0], b[0], a[1] * b[1]);
  const float p1 = __builtin_fmaf(a[2], b[2], a[3] * b[3]);
  const float p2 = __builtin_fmaf(a[4], b[4], a[5] * b[5]);
  const float p3 = __builtin_fmaf(a[6], b[6], a[7] * b[7]);
  return (p0 + p1) + (p2 + p3);
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
// x plus its value in the paired row (rows 0/1 and 2/3: v_permlane16_swap) or
// half wave (v_permlane32_swap).  Both operands of the swap are x, so every lane
// receives its partner's x in one of the two results and the sum is the same in
// both partners.  Requires every lane of the wave active.
template <int ROWS>
__device__ __forceinline__ double tam_swap_add(double x) {
  const uint64_t u = tam_d2u(x);
  const uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
  const auto l = ROWS == 1 ? __builtin_amdgcn_permlane16_swap(lo, lo, true, false)
                           : __builtin_amdgcn_permlane32_swap(lo, lo, true, false);
  const auto h = ROWS == 1 ? __builtin_amdgcn_permlane16_swap(hi, hi, true, false)
                           : __builtin_amdgcn_permlane32_swap(hi, hi, true, false);
  return tam_u2d(((uint64_t)h[0] << 32) | l[0]) + tam_u2d(((uint64_t)h[1] << 32) | l[1]);
}

// Per-block sums of a and b with the tree of tam_block_sum, in one reduction:
// after the first step even lanes carry partial sums of a and odd lanes of b
// (quad steps pair lanes of equal parity); row_ror:4 then pairs lanes 0-3
// with 4-7 and row_ror:8 pairs 0-7 with 8-15.  The sum of a is valid in lanes
// 12 and 14 of each row, the sum of b in lanes 13 and 15.
__device__ __forceinline__ double tam_row_sum2(double a, double b, bool odd) {
  double x = (odd ? b : a) + tam_dppd<TAM_DPP_XOR1>(odd ? a : b);
  x = x + tam_dppd<TAM_DPP_XOR2>(x);
  x = x + tam_dppd<TAM_DPP_ROR4>(x);
  return x + tam_dppd<TAM_DPP_ROR8>(x);
}

// Sums of a and b over a wave's 4 blocks: tam_row_sum2 per block, then
// (b0 + b1) + (b2 + b3) through the swaps (blocks 0/1 and 2/3, then the two
// halves).  Returns the sum of a in lane 12 and the sum of b in lane 13.
// Requires every lane active.
__device__ __forceinline__ double tam_quarter_sum2(double a, double b, uint32_t lane) {
  double x = tam_row_sum2(a, b, (lane & 1u) != 0);
  x = tam_swap_add<1>(x);
  return tam_swap_add<2>(x);
}

// Minimum / maximum over the block of unsigned keys (bit patterns of
// positive floats order like the floats).
__device__ __forceinline__ uint32_t tam_block_umin(uint32_t v) {
  v = __builtin_elementwise_min(v, tam_dpp<TAM_DPP_XOR1>(v));
  v = __builtin_elementwise_min(v, tam_dpp<TAM_DPP_XOR2>(v));
  v = __builtin_elementwise_min(v, tam_dpp<TAM_DPP_HALF_MIRROR>(v));
  v = __builtin_elementwise_min(v, tam_dpp<TAM_DPP_MIRROR>(v));
  return v;
}
__device__ __forceinline__ uint32_t tam_block_umax(uint32_t v) {
  v = __builtin_elementwise_max(v, tam_dpp<TAM_DPP_XOR1>(v));
  v = __builtin_elementwise_max(v, tam_dpp<TAM_DPP_XOR2>(v));
  v = __builtin_elementwise_max(v, tam_dpp<TAM_DPP_HALF_MIRROR>(v));
  v = __builtin_elementwise_max(v, tam_dpp<TAM_DPP_MIRROR>(v));
  return v;
}
__device__ __forceinline__ uint32_t tam_block_or(uint32_t v) {
  v |= tam_dpp<TAM_DPP_XOR1>(v);
  v |= tam_dpp<TAM_DPP_XOR2>(v);
  v |= tam_dpp<TAM_DPP_HALF_MIRROR>(v);
  v |= tam_dpp<TAM_DPP_MIRROR>(v);
  return v;
}

// Compiler-only barrier: memory accesses are not moved across it (no
// instruction is emitted).  Placed after a quarter's loads so that none of them
// is sunk below the first use of another (each would then wait on its own).
__device__ __forceinline__ void tam_compiler_fence() { asm volatile("" ::: "memory"); }

// Value barrier: the compiler treats x as rewritten here, so no computation on
// x moves above this point.  Pinning every loaded value after a fence keeps the
// compiler from interleaving arithmetic on early loads with the issue of later
// ones (each such use would wait on its load before the later loads issue).
__device__ __forceinline__ void tam_pin(uint32_t& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void tam_pin(float& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void tam_pin(TamW4& x) { asm volatile("" : "+v"(x)); }

// Instruction choices the compiler would not make by itself.  On gfx950 a
// shift or v_and_or_b32 issues at half the rate of v_add_u32 or of a
// v_bitop3_b32 whose operands are all VGPRs (a uniform constant would go to an
// SGPR, and back-to-back reads of one SGPR also halve the rate).
// A constant held in a VGPR.
__device__ __forceinline__ uint32_t tam_vconst(uint32_t k) {
  uint32_t r;
  asm("v_mov_b32 %0, %1" : "=v"(r) : "i"(k));
  return r;
}
// x + x (the compiler would emit the shift x << 1).
__device__ __forceinline__ uint32_t tam_dbl(uint32_t x) {
  uint32_t r;
  asm("v_add_u32 %0, %1, %1" : "=v"(r) : "v"(x));
  return r;
}
// A uniform value copied to a VGPR.
__device__ __forceinline__ uint32_t tam_vcopy(uint32_t x) {
  uint32_t r;
  asm("v_mov_b32 %0, %1" : "=v"(r) : "s"(x));
  return r;
}
// (x & m) | y in one v_bitop3_b32 (truth table over x, m, y: 0xF0 & 0xCC | 0xAA).
__device__ __forceinline__ uint32_t tam_and_or(uint32_t x, uint32_t m, uint32_t y) {
  return __builtin_amdgcn_bitop3_b32(x, m, y, 0xEA);
}

// Orders this wave's LDS accesses before and after the call (LDS operations of
// one wave execute in order, so no s_barrier is needed between lanes of a wave).
__device__ __forceinline__ void tam_wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------
// one wave's share of a tile
// ---------------------------------------------------------------------------
// A wave owns 4 consecutive blocks (512 elements) of a tile: lane l holds
// elements [8*(l%16), 8*(l%16)+8) of block 4*wq + l/16 of its tensor, where wq
// is the wave's quarter-tile index within the tensor.  `full` quarters lie
// entirely inside the tensor (and its arrays are 16-byte aligned): no
// per-element bounds.  Other quarters check every element against n.
struct TamWave {
  uint32_t lane;  // 0..63
  uint32_t l16;   // lane within the block
  uint32_t b;     // block within the tensor
  uint64_t e0;    // first element of the lane
  uint32_t nv;    // elements of the lane inside the tensor (0..8)
  bool bvalid;    // block b exists (b < nb)
};

__device__ __forceinline__ TamWave tam_wave(const TamTensor& d, uint32_t wq, uint32_t lane, bool full) {
  TamWave W;
  W.lane = lane;
  W.l16 = lane & 15u;
  W.b = wq * 4u + (lane >> 4);
  W.e0 = (uint64_t)W.b * TAM_BLOCK_SIZE + W.l16 * TAM_EPL;
  if (full) {
    W.nv = TAM_EPL;
    W.bvalid = true;
  } else {
    const uint64_t n = d.n;
    W.nv = W.e0 >= n ? 0u : (n - W.e0 >= TAM_EPL ? (uint32_t)TAM_EPL : (uint32_t)(n - W.e0));
    W.bvalid = W.b < d.nb;
  }
  return W;
}

// CoState first moment of the lane's 8 elements (reference costate.py:398-416):
//   m_hat = has_state ? fl(fl(alpha*g) + s_b*sgn) : 0,  m = fl(fl(b1*m_hat) + fl(ob1*g))
// with s_b = norm_b / sqrt(128) for phase blocks (costate.py:306, true
// division), the fp16 amplitude for amplitude blocks, 0 for null blocks.
// The CoState state of the lane's block (label, norm, amplitude) and its sign
// byte, loaded before any of it is used (no load waits on the label).
struct TamCsIn {
  uint32_t label, amp, byte;
  float nrm;
};
// Error feedback: the new encoding of a tensor is staged in the workspace
// (passes 2 and 3) until pass 4 has used the previous one.  Layout as
// tam_ef_stage_bytes: norms f32[nb], amplitudes f16[nb], labels u8[nb], sign
// bytes u8[ceil(n/8)].
struct TamStage {
  float* norms;
  uint16_t* amp;
  uint8_t* labels;
  uint8_t* signs;
};
__device__ __forceinline__ TamStage tam_stage(const TamTensor& d, char* ws) {
  char* b = ws + d.ef_off;
  TamStage st;
  st.norms = (float*)b;
  st.amp = (uint16_t*)(b + 4ull * d.nb);
  st.labels = (uint8_t*)(b + 6ull * d.nb);
  st.signs = (uint8_t*)(b + 7ull * d.nb);
  return st;
}

// The gradient of the EMA term of an error-feedback tensor: g + residual once
// a residual exists (costate.py:410-413), else g.
template <bool FULL>
__device__ __forceinline__ void tam_ef_grad(const TamTensor& d, const TamWave& W, const float* g, float* ge) {
  if (d.flags & TAM_FLAG_HAS_EF) {
    float r[TAM_EPL];
    tam_ld8_f32<FULL>(d.ef_residual, W.e0, W.nv, r);
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) ge[i] = g[i] + r[i];
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) ge[i] = g[i];
  }
}

template <bool FULL>
__device__ __forceinline__ TamCsIn tam_cs_load(const TamTensor& d, const TamWave& W) {
  TamCsIn c = {0u, 0u, 0u, 0.0f};
  if ((d.flags & TAM_FLAG_HAS_STATE) && (FULL || W.bvalid)) {
    c.label = tam_g(d.labels)[W.b];
    c.nrm = tam_g(d.norms)[W.b];
    c.amp = tam_g(d.amp)[W.b];
    if (FULL || W.nv > 0) c.byte = tam_g(d.signs)[W.e0 >> 3];
  }
  return c;
}

// fl(x / fl(sqrt(128))) (costate.py:306, true division) as the fp64 product of
// x and the correctly rounded fp64 reciprocal of fl(sqrt(128)): its error is
// below 2^-52 relative, while a quotient of two 24-bit significands never lies
// within 2^-49 of an fp32 rounding boundary, so the fp32 rounding of the
// product is the correctly rounded quotient for every fp32 x (also checked
// exhaustively on the host).
#define TAM_SQRT_BLOCK_F 0x1.6a09e6p+3f
__device__ __forceinline__ float tam_div_sqrt_block(float x) {
  return (float)((double)x * (1.0 / (double)TAM_SQRT_BLOCK_F));
}

// ge is the gradient of the EMA term: g, or g + the error-feedback residual
// (costate.py:410-416; the decode keeps g).
// The decoded EMA of 8 elements from their block's |s| (bit pattern) and sign
// byte.  s * (1 - 2*bit), costate.py:207-209, :317-319: s has a clear sign bit
// (a norm or an fp16 amplitude), so the bit becomes the sign of s; element i's
// bit (bit 7 - i of the byte) reaches bit 31 of sh after i doublings.
template <bool VMASK>
__device__ __forceinline__ void tam_cs_decode_m(const TamTensor& d, uint32_t sabs, uint32_t byte, float alpha_prev,
                                                const float* g, const float* ge, float* m) {
  const uint32_t sign_bit = VMASK ? tam_vconst(0x80000000u) : 0x80000000u;
  uint32_t sh = byte << 24;
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) {
    const float sd = tam_u2f(tam_and_or(sh, sign_bit, sabs));
    sh = tam_dbl(sh);
    const float mh = alpha_prev * g[i] + sd;
    m[i] = d.beta1 * mh + d.one_minus_beta1 * ge[i];
  }
}
// |s| of a valid block (bit pattern): the norm over sqrt(128) for label 1, the
// fp16 amplitude for label 2, else 0; both candidates are evaluated and
// selected without a branch.
__device__ __forceinline__ uint32_t tam_cs_sabs(const TamCsIn& cs) {
  const float sph = tam_div_sqrt_block(cs.nrm), af = tam_f16_to_f32((uint16_t)cs.amp);
  return tam_f2u(cs.label == 1u ? sph : (cs.label == 2u ? af : 0.0f)) & 0x7fffffffu;
}

// VMASK: the sign mask is held in a VGPR and the block scale is selected
// without a branch (false where the kernel has no register to spare: the mask
// then comes from an SGPR and the scale from a branch).
template <bool FULL, bool VMASK = true>
__device__ __forceinline__ void tam_costate_m(const TamTensor& d, const TamWave& W, const TamCsIn& cs,
                                              float alpha_prev, const float* g, const float* ge, float* m) {
  const bool has = (d.flags & TAM_FLAG_HAS_STATE) != 0;  // uniform over the launch
  if (has) {
    const uint32_t byte = cs.byte;
    float s = 0.0f;
    if constexpr (VMASK) {
      s = (FULL || W.bvalid) ? tam_u2f(tam_cs_sabs(cs)) : 0.0f;
    } else if (FULL || W.bvalid) {
      const float sph = tam_div_sqrt_block(cs.nrm);
      s = cs.label == 1u ? sph : (cs.label == 2u ? tam_f16_to_f32((uint16_t)cs.amp) : 0.0f);
    }
    tam_cs_decode_m<VMASK>(d, tam_f2u(s) & 0x7fffffffu, byte, alpha_prev, g, ge, m);
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) m[i] = d.beta1 * 0.0f + d.one_minus_beta1 * ge[i];
  }
}

// 1Q second moment of the lane's 8 elements (reference quantize.py:222-299).
//
// Decode (quantize.py:256): the 2^bits values exp(lmin + ((k+0.5)/2^bits)*span)
// of a block are computed once per block: for 2^bits <= 16 lane k of the block
// computes value k and elements fetch theirs with ds_bpermute; for 64 levels
// through a per-wave LDS table; 8-bit indices evaluate per element.
//
// Index of an element: with c = fl(fl(l - lmin)/sp) * 2^bits and u its
// uniform, the reference computes floor(c) + (u < c - floor(c)) clamped to
// [0, 2^bits - 1]; for real c and u in [0,1) that equals ceil(c - u).  The fast
// path evaluates c~ = log2(v)*K + C in fp32 (K = ln2*2^bits/sp, C =
// -lmin*2^bits/sp) from the hardware log2 (v_log_f32, whose error against the
// correctly rounded ln is below 2^-21 |ln| for every normal input -- checked
// exhaustively on gfx950) and bounds |(c - u) - d| <= B for d = fl(c~ - u):
//   B = |log2 v| K 2^-20 + |c~| 2^-21 + |C| 2^-21 + 2^-22
// (hardware log error, the two fp32 roundings of c, the errors of K and C, the
// fma and the subtraction, each with margin).  ceil(d) is accepted when
// [d - B, d + B] lies in (q - 1, q], q = ceil(d): with r = q - d (exact by
// Sterbenz, or at least 1/2 when q = 1), r >= B and 1 - r > B (1 - r is
// exact for r >= 1/2 and above 1/2 otherwise).  The clamp to [0, 2^bits - 1]
// then gives the reference's index.  Otherwise the element takes the exact
// path (correctly rounded log and division).  lmin and lmax are the correctly rounded logs of
// the block's smallest and largest v (log is monotone, so they equal the min
// and max of the per-element logs).
// The 1Q state of the lane: its block's fp16 (log_min, log_max) pair and its 8 indices.
struct TamVIn {
  uint32_t sc, iw0, iw1;
};
template <bool FULL>
__device__ __forceinline__ TamVIn tam_v_load(const TamTensor& d, const TamWave& W) {
  TamVIn r = {0u, 0u, 0u};
  if (FULL || W.bvalid) {
    r.sc = tam_g((const uint32_t*)d.v_scales)[W.b];
    const TamW2 iw = tam_g((const TamW2*)(d.v_idx + W.e0))[0];
    r.iw0 = iw.x;
    r.iw1 = iw.y;
  }
  return r;
}

// LDS copies of the log / exp tables (the correctly rounded log and exp of a
// block read them at LDS latency instead of a dependent global load).
struct TamLdsTabs {
  TamLogEntry log[129];
  TamDD exp[64];
};
__device__ __forceinline__ void tam_lds_tabs_fill(TamLdsTabs* t) {
  for (uint32_t i = threadIdx.x; i < 129u; i += blockDim.x) t->log[i] = tam_log_tab_d[i];
  for (uint32_t i = threadIdx.x; i < 64u; i += blockDim.x) t->exp[i] = tam_exp_tab_d[i];
  __syncthreads();
}
__device__ __forceinline__ float tam_logf_lds(float x, const TamLdsTabs* t) {
  return tam_logf_with(x, [t](int j) { return t->log[j]; });
}
__device__ __forceinline__ float tam_expf_lds(float x, const TamLdsTabs* t) {
  return tam_expf_with(x, [t](int j) { return t->exp[j]; });
}

// Block extremes of v (valid elements only).  When v >= +0 or NaN (0 <= beta2
// <= 1): kmn / kmx are the bit patterns of the smallest and largest v before
// the clamp, and nan_seen is 1 when a v is NaN.  Otherwise (v may be
// negative): kmn / kmx are the extremes of the clamped v, and nan_seen has bit
// 1 set (no bound on the unclamped v; the update takes its exact sequence).
struct TamVExt {
  uint32_t kmn, kmx, nan_seen;
};
#define TAM_VEXT_NAN 1u
#define TAM_VEXT_CLAMPED 2u
#define TAM_BITS_1EM38 0x006ce3eeu  // f32(1e-38) (subnormal)

// First half: decode, EMA, clamp, block extremes.  The parameter update runs
// between the halves (it needs v, not the new indices), so that p, m and v are
// no longer live during the re-quantisation.
template <bool FULL>
__device__ __forceinline__ TamVExt tam_vpath_a(const TamTensor& d, const TamWave& W, const TamVIn& vin,
                                               const float* g, float* v, float* vc, float* lutw,
                                               const TamLdsTabs* tabs) {
  const uint32_t bits = d.v_bits;
  const uint32_t nbk = 1u << bits;
  const float fnb = (float)nbk;
  const float inv_nbk = 1.0f / fnb;  // exact power of two
  const bool bvalid = FULL || W.bvalid;
  const float lmin0 = tam_f16_to_f32((uint16_t)(vin.sc & 0xffffu));
  const float span0 = tam_f16_to_f32((uint16_t)(vin.sc >> 16)) - lmin0;  // quantize.py:253-255
  const uint32_t iw0 = vin.iw0, iw1 = vin.iw1;
  uint32_t idx[TAM_EPL];
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) idx[i] = ((i < 4 ? iw0 : iw1) >> (8 * (i & 3))) & 0xffu;
  float vo[TAM_EPL];
  if (nbk <= 16u) {
    // every lane of the wave takes part in the permutes
    const uint32_t k = W.l16 & (nbk - 1u);
    const float val = tam_expf_lds(lmin0 + ((float)k + 0.5f) * inv_nbk * span0, tabs);
    const uint32_t row = W.lane & 48u;
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      const int src = (int)((row + (idx[i] & (nbk - 1u))) << 2);
      const float x = tam_u2f((uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)tam_f2u(val)));
      vo[i] = bvalid ? x : 0.0f;
    }
  } else if (nbk == 64u) {
    float* tab = lutw + (W.lane >> 4) * 64u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t k = W.l16 + 16u * (uint32_t)j;
      tab[k] = tam_expf_lds(lmin0 + ((float)k + 0.5f) * inv_nbk * span0, tabs);
    }
    tam_wave_lds_sync();
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) vo[i] = bvalid ? tab[idx[i] & 63u] : 0.0f;
    tam_wave_lds_sync();  // the next tile rewrites the table
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) vo[i] = tam_expf_lds(lmin0 + ((float)idx[i] + 0.5f) * inv_nbk * span0, tabs);
  }
  // EMA (quantize.py:259-270) and the clamp of :275.
  TamVExt x;
  if (d.beta2 >= 0.0f && d.one_minus_beta2 >= 0.0f) {  // uniform
    // v >= +0 or NaN.  The extremes are taken on the bit patterns of v with
    // the sign bit cleared: -0 orders as +0 and a NaN of either sign orders
    // above +inf.  The clamp commutes with min and max, so vpath_b clamps the
    // extremes; vc = max(v, 1e-38) equals the clamp except for a NaN, whose
    // block is re-quantised from its NaN extremes whatever vc holds.
    uint32_t xmn = 0xffffffffu, xmx = 0u;
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      const bool valid = FULL || (uint32_t)i < W.nv;
      const float g2 = valid ? g[i] * g[i] : 0.0f;
      v[i] = __builtin_fmaf(d.one_minus_beta2, g2, vo[i] * d.beta2);
      vc[i] = __builtin_fmaxf(v[i], 1e-38f);
      const uint32_t k = tam_f2u(v[i]) & 0x7fffffffu;
      if (valid && bvalid) {
        xmn = __builtin_elementwise_min(xmn, k);
        xmx = __builtin_elementwise_max(xmx, k);
      }
    }
    x.kmn = tam_block_umin(xmn);
    x.kmx = tam_block_umax(xmx);
    x.nan_seen = x.kmx > 0x7f800000u ? TAM_VEXT_NAN : 0u;
  } else {
    // v may be negative: extremes of the clamped v, NaN tested per element
    uint32_t kmn = 0x7f800000u, kmx = 0u;
    uint32_t nan_seen = 0;
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      const bool valid = FULL || (uint32_t)i < W.nv;
      const float g2 = valid ? g[i] * g[i] : 0.0f;
      v[i] = __builtin_fmaf(d.one_minus_beta2, g2, vo[i] * d.beta2);
      vc[i] = v[i] < 1e-38f ? 1e-38f : v[i];
      if (valid && bvalid) {
        nan_seen |= tam_isnan(vc[i]) ? 1u : 0u;
        kmn = __builtin_elementwise_min(kmn, tam_f2u(vc[i]));
        kmx = __builtin_elementwise_max(kmx, tam_f2u(vc[i]));
      }
    }
    x.kmn = tam_block_umin(kmn);
    x.kmx = tam_block_umax(kmx);
    x.nan_seen = (tam_block_or(nan_seen) ? TAM_VEXT_NAN : 0u) | TAM_VEXT_CLAMPED;
  }
  return x;
}

// Extremes of |v| over the lane's valid elements (an fp32 second moment): a
// negative q gives a NaN in the fast update and fails its own test, so
// magnitudes bound the range test.
template <bool FULL>
__device__ __forceinline__ TamVExt tam_lane_extremes(const float* v, uint32_t nv) {
  uint32_t xmn = 0xffffffffu, xmx = 0u;
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) {
    if (FULL || (uint32_t)i < nv) {
      xmn = __builtin_elementwise_min(xmn, tam_f2u(v[i]) & 0x7fffffffu);
      xmx = __builtin_elementwise_max(xmx, tam_f2u(v[i]) & 0x7fffffffu);
    }
  }
  TamVExt x;
  x.kmn = xmn;
  x.kmx = xmx;
  x.nan_seen = x.kmx > 0x7f800000u ? TAM_VEXT_NAN : 0u;
  return x;
}

// Whether q = fl(v * f32(1/bc2)) is a positive normal for every v of the
// block (the certified 16-bit update's input range): q is monotone in v, so
// the block's smallest and largest v decide.  False when the extremes bound
// only the clamped v or a v is NaN.
__device__ __forceinline__ bool tam_q_in_range(const TamTensor& d, const TamVExt& x) {
  return x.nan_seen == 0u && tam_u2f(x.kmn) * d.inv_bc2_f32 >= 0x1p-126f &&
         tam_u2f(x.kmx) * d.inv_bc2_f32 <= 0x1.fffffep127f;
}

// Second half: logs of the extremes, scales, stochastic re-quantisation.
template <bool FULL>
__device__ __forceinline__ void tam_vpath_b(const TamTensor& d, const TamWave& W, const float* vc, TamVExt x,
                                            const TamLdsTabs* tabs, uint32_t seed_lo, uint32_t seed_hi) {
  const uint32_t nbk = 1u << d.v_bits;
  const float fnb = (float)nbk;
  const bool bvalid = FULL || W.bvalid;
  // extremes of the clamped v (quantize.py:275-280)
  const uint32_t kmn = __builtin_elementwise_max(x.kmn, TAM_BITS_1EM38);
  const uint32_t kmx = __builtin_elementwise_max(x.kmx, TAM_BITS_1EM38);
  const bool nan_seen = (x.nan_seen & TAM_VEXT_NAN) != 0u;
  // correctly rounded logs of the extremes: even lanes log(vmin), odd lanes log(vmax)
  const float lx = tam_logf_lds(tam_u2f((W.l16 & 1u) ? kmx : kmn), tabs);
  const float ly = tam_dppf<TAM_DPP_XOR1>(lx);
  float lmn = (W.l16 & 1u) ? ly : lx;
  float lmx = (W.l16 & 1u) ? lx : ly;
  if (nan_seen) lmn = lmx = tam_qnan();  // torch.min / torch.max propagate NaN
  if (!bvalid) return;
  float sp = lmx - lmn;  // quantize.py:283
  sp = sp < 1e-10f ? 1e-10f : sp;
  if (W.l16 == 0) {
    tam_g((uint32_t*)d.v_scales)[W.b] = (uint32_t)tam_f32_to_f16(lmn) | ((uint32_t)tam_f32_to_f16(lmx) << 16);
  }
  // certified stochastic rounding.  K and C from the hardware reciprocal of
  // sp (within 2^-23): K within 2^-22 of ln2*2^bits/sp, C within 2^-22.4 of
  // -lmin*2^bits/sp.  Partial blocks (c~ = K log2 v + C, per element) take
  // |log2 v| K 2^-20 and |C| 2^-21 into their bound; full blocks use K with
  // the ratio form below.
  const float rsp = __builtin_amdgcn_rcpf(sp);
  const float K = (0x1.62e430p-1f * fnb) * rsp;
  const float C = (-lmn * fnb) * rsp;
  const float KB = K * 0x1p-20f;
  const float CB = __builtin_fmaf(__builtin_fabsf(C), 0x1p-21f, 0x1p-22f);
  // the lane's 8 draws (24-bit integers)
  uint32_t rw[TAM_EPL];
  tam_draws8(W.e0, d.tensor_id, d.step, seed_lo, seed_hi, rw);
  // indices go straight into their bytes (v_cvt_pk_u8_f32 of an integral
  // value in [0, 255]); partial blocks accept per element (lane masks)
  uint32_t ow[2] = {0u, 0u};
  bool okv[TAM_EPL];
  bool all_ok = true;
  // Full blocks: every element lies in [vmin, vmax] (normal, no NaN checked
  // once here), so one bound B serves the block.  With F = 2^bits the exact
  // path's index is ceil(c - u), c = F fl(fl(l - lmin)/sp), l = fl(ln v).  The
  // fast path takes c~ = K log2(t) from the hardware log2 of t = fl(v rcp(vmin)),
  // which lies within 2^-22 of [1, vmax/vmin]: the hardware log's error is
  // relative to log2 t <= (lmax - lmin)/ln2 rather than to |log2 v|, so the
  // bound stays small when a block's log span sp is small (as 1Q's repeated
  // re-quantisation makes it).  |c~ - c| is within:
  //   F 2^-24 (Lm + |lmin|)/sp   the roundings of l and of lmin to fp32
  //                              (Lm = max(|lmin|, |lmax|) bounds |l|);
  //   F 2^-22 / sp               rcp(vmin) (2^-23.3) and the product (2^-24);
  //   F 2^-21                    the hardware log2 (2^-21 relative; measured 2^-22.6);
  //   F 2^-20                    the exact path's roundings of l - lmin and of
  //                              the division, and K's (ln2 in fp32, rcp(sp));
  //   (F + 2) 2^-21              the fma roundings of values up to F + 3/2,
  // all times 1 + 2^-16 for the fp32 evaluation of the bound.  When B < 1/4,
  // |c~| <= F + 1 (c lies in [0, F]).  The fast path evaluates d = fl(c~ + 1/2 - u)
  // and q = rndne(d), which is ceil(c - u) when d lies farther than B from every
  // half-integer; t = d - q is exact.  A lane is accepted when max |t| < H =
  // 1/2 - (B + 2^-22); otherwise its elements are tested one by one in the exact
  // path below.  Blocks with sp > 64 or vmax >= 2^100 (t or rcp(vmin) out of
  // range) take the exact path.
  float H = -1.0f, rmin = 0.0f;
  if (FULL) {
    rmin = __builtin_amdgcn_rcpf(tam_u2f(kmn));
    const float Lm = __builtin_fmaxf(__builtin_fabsf(lmn), __builtin_fabsf(lmx));
    const float per_sp = __builtin_fmaf(Lm + __builtin_fabsf(lmn), 0x1p-24f, 0x1p-22f);
    const float flat = __builtin_fmaf(fnb, 0x1p-21f + 0x1p-20f, (fnb + 2.0f) * 0x1p-21f);
    const float Bb = __builtin_fmaf(fnb * rsp, per_sp, flat) * (1.0f + 0x1p-16f);
    const bool blk_ok = (tam_u2f(kmn) >= 0x1p-126f) && (tam_u2f(kmx) < 0x1p100f) && !nan_seen && (sp <= 64.0f) &&
                        (Bb < 0.25f);
    H = blk_ok ? 0.5f - (Bb + 0x1p-22f) : -1.0f;
    float tmax = 0.0f;
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      const float l2 = __builtin_amdgcn_logf(vc[i] * rmin);
      const float ct = __builtin_fmaf(l2, K, 0.5f);
      const float dd = __builtin_fmaf(-(float)rw[i], 0x1p-24f, ct);  // fl(ct - u), u exact
      const float q = __builtin_rintf(dd);
      tmax = __builtin_fmaxf(tmax, __builtin_fabsf(dd - q));
      // the exact path overwrites rejected elements
      ow[i >> 2] = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_amdgcn_fmed3f(q, 0.0f, fnb - 1.0f), i & 3, ow[i >> 2]);
    }
    all_ok = tmax < H;  // false for a NaN bound (then H = -1)
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      const float l2 = __builtin_amdgcn_logf(vc[i]);
      const float ct = __builtin_fmaf(l2, K, C);
      const float dd = __builtin_fmaf(-(float)rw[i], 0x1p-24f, ct);  // fl(ct - u), u exact
      const float B = __builtin_fmaf(__builtin_fabsf(l2), KB, __builtin_fmaf(__builtin_fabsf(ct), 0x1p-21f, CB));
      const float q = __builtin_ceilf(dd);
      const float r = q - dd;
      okv[i] = (vc[i] >= 0x1p-126f) && (r >= B) && (1.0f - r > B);  // false for NaN
      all_ok &= okv[i];
      ow[i >> 2] = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_amdgcn_fmed3f(q, 0.0f, fnb - 1.0f), i & 3, ow[i >> 2]);
    }
  }
  if (!all_ok) {
    // exact path: the reference's own sequence with correctly rounded log and division
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      if (FULL) {  // the element's own test, as in the lane's
        const float dd = __builtin_fmaf(-(float)rw[i], 0x1p-24f,
                                        __builtin_fmaf(__builtin_amdgcn_logf(vc[i] * rmin), K, 0.5f));
        okv[i] = __builtin_fabsf(dd - __builtin_rintf(dd)) < H;
      }
      if (!okv[i]) {
        const float l = tam_logf_lds(vc[i], tabs);
        const float c = ((l - lmn) / sp) * fnb;  // quantize.py:284-285
        const float f = __builtin_floorf(c);
        const float fr = c - f;
        const float u = (float)rw[i] * 0x1p-24f;
        float q = f + (u < fr ? 1.0f : 0.0f);  // quantize.py:288-294
        q = q < 0.0f ? 0.0f : q;
        q = q > fnb - 1.0f ? fnb - 1.0f : q;
        const uint32_t qi = tam_isnan(q) ? 0u : (uint32_t)q;
        const uint32_t sh = 8u * (uint32_t)(i & 3);
        ow[i >> 2] = (ow[i >> 2] & ~(0xffu << sh)) | (qi << sh);
      }
    }
  }
  tam_g((TamW2*)(d.v_idx + W.e0))[0] = TamW2{ow[0], ow[1]};
}

// ---------------------------------------------------------------------------
// parameter update (reference optimizer.py:106-107, :163, :170)
// ---------------------------------------------------------------------------
// Exact sequence: q1 = fl(v/bc2), s = fl(sqrt(q1)), den = fl(s + eps),
// t2 = fl(den*bc1), a = fl(-lr*m), upd = fl(a/t2), p = R_p(fl(p + upd)).
// fp32 parameters: q1 comes from the fp64 reciprocal of bc2 when a rounding
// test proves the fp32 rounding, else from the division.
//
// bf16 / fp16 parameters: a fast sequence u~ = fl(fl(c*m) * r) with
// r = rcp(fl(s~ + eps)), s~ = sqrt(q) (v_sqrt_f32), q = fl(v * fl(1/bc2)),
// c = fl(-lr/bc1).  In the model fl(x) = x(1 + d) + e (|d| <= 2^-24,
// |e| <= 2^-150 and e != 0 only below 2^-126), with q a positive normal and
// 0 <= eps < 2^124 (so 2^-63 <= den < 2^125 and r is a normal):
//  * relative parts: the exact sequence's six roundings, the fast
//    sequence's six and the two hardware results (v_sqrt_f32 within
//    2^-23.36 and v_rcp_f32 within 2^-23 on normal inputs -- each checked
//    exhaustively on gfx950), 16 units of 2^-24, inside 2^-19;
//  * absolute parts: e of fl(-lr*m) divided by t2 (at most
//    2^-150 r/bc1 (1 + 2^-21)), e of c*m times r, and e of upd and u~, below
//    2^-147 r/bc1 + 2^-149.
// So |u~ - upd| <= 2^-19 |u~| + 2^-147 r/bc1 + 2^-149, and when |u~| < 2^126
// (upd then finite), fl(p + upd) lies within 2^-19 |u~| + 2^-22 |s| +
// 2^-147 r/bc1 + 2^-148 of s = fl(p + u~).  On a lane the test below accepts,
// q >= 2^-126 and eps >= 0, so r <= min(1/eps, 2^63) (1 + 2^-21): the last two
// terms are below the per-tensor constant k_abs (tam_abs_term), and
//   E = 2^-19 |u~| + 2^-22 |s| + k_abs
// bounds the distance; the kernels use the larger 2^-19 max|u~| + 2^-22 |s|
// + k_abs, max over the lane's elements.  R_p and fl are monotone (overflow included), so
// R_p(fl(p + upd)) is accepted when R_p(fl(s - E)) == R_p(fl(s + E)) and s is
// not a NaN (an infinite s makes fl(s - E) a NaN, which fails the equality).
// Elements go in pairs: one packed conversion rounds both fl(s - E), another
// both fl(s + E), and the pair is accepted when the two words agree; the fma
// product of the pair's s values, accumulated per lane, stays finite only
// when no s is a NaN (an overflow of it only rejects more).  q_ok tells that
// every q of the block is a positive normal (tam_q_in_range); |u~| < 2^126 is
// tested per lane.  A lane that fails either, and a pair that fails its own
// test, takes the exact sequence.  The results of a 16-bit parameter are
// returned as bit patterns, two per word (element 2k in the low half of pw2[k]).
typedef float TamF2 __attribute__((ext_vector_type(2)));
typedef __bf16 TamBf2 __attribute__((ext_vector_type(2)));
typedef _Float16 TamH2 __attribute__((ext_vector_type(2)));
// k_abs of the certified 16-bit update: 2^-147/bc1 * min(1/eps, 2^63) *
// (1 + 2^-20) + 2^-148, evaluated in fp64 and rounded up to fp32 (host and
// device prologue compute it the same way).
__host__ __device__ inline float tam_abs_term(float bc1, float eps) {
  const double ie = eps > 0.0f ? 1.0 / (double)eps : 0x1p63;
  const double x = 0x1p-147 / (double)bc1 * (ie < 0x1p63 ? ie : 0x1p63) * (1.0 + 0x1p-20) + 0x1p-148;
  float c = (float)x;
  if ((double)c < x) c = tam_next_float(c, true);
  return c;
}
// x and y rounded to the 16-bit dtype (round to nearest even) in one packed
// conversion: x in the low half, y in the high half
template <uint32_t DT>
__device__ __forceinline__ uint32_t tam_pack16(float x, float y) {
  if (DT == TAM_DTYPE_BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector((TamF2){x, y}, TamBf2));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((TamF2){x, y}, TamH2));
}
template <uint32_t DT>
__device__ __forceinline__ void tam_update(const TamTensor& d, float* p, const float* m, const float* v,
                                           uint32_t* pw2, bool q_ok) {
  const bool wd = (d.flags & TAM_FLAG_WD) != 0;
  if (DT == TAM_DTYPE_F32) {
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
  float pw[TAM_EPL];
  // weight decay rounds to the parameter dtype (p.mul_ on a 16-bit tensor)
  if (wd && DT == TAM_DTYPE_BF16) {
    // converting (0, x) puts bf16(x) in the high half over a zero low half:
    // the word is bf16(x) as fp32, with no shift or mask
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i)
      pw[i] = tam_u2f(__builtin_bit_cast(uint32_t, __builtin_convertvector((TamF2){0.0f, p[i] * d.c_wd}, TamBf2)));
  } else if (wd) {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) pw[i] = tam_h2f<DT>(tam_round16_hw<DT>(p[i] * d.c_wd));
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) pw[i] = p[i];
  }
  // c_lr = fl(-lr / bc1), from tam_prepare (one more rounding in the fast
  // sequence, inside the 2^-19 bound)
  const float c_lr = d.c_lr, k_abs = d.k_abs;
  // per-pair acceptance as lane masks
  bool okp[TAM_EPL / 2];
  bool all_ok = true;
  float umax = 0.0f, nacc = 0.0f;
  float st[TAM_EPL];
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) {
    const float q = v[i] * d.inv_bc2_f32;
    const float s = __builtin_amdgcn_sqrtf(q);
    const float r = __builtin_amdgcn_rcpf(s + d.eps);
    const float u = (c_lr * m[i]) * r;
    st[i] = pw[i] + u;
    umax = __builtin_fmaxf(umax, __builtin_fabsf(u));  // a NaN u makes st NaN
  }
  // 2^-19 |u| + k_abs of every element of the lane is at most this one term
  // (E only grows: the test can only reject more)
  const float eu = __builtin_fmaf(umax, 0x1p-19f, k_abs);
#pragma unroll
  for (int k = 0; k < TAM_EPL / 2; ++k) {
    const float s0 = st[2 * k], s1 = st[2 * k + 1];
    const float e0 = __builtin_fmaf(__builtin_fabsf(s0), 0x1p-22f, eu);
    const float e1 = __builtin_fmaf(__builtin_fabsf(s1), 0x1p-22f, eu);
    nacc = __builtin_fmaf(s0, s1, nacc);
    const uint32_t lo = tam_pack16<DT>(s0 - e0, s1 - e1);
    const uint32_t hi = tam_pack16<DT>(s0 + e0, s1 + e1);
    pw2[k] = lo;
    okp[k] = lo == hi;
    all_ok &= okp[k];
  }
  // eps is uniform: 0 <= eps < 2^124 (no cancellation in s + eps; den < 2^125)
  const bool lane_ok = q_ok && umax < 0x1p126f && __builtin_fabsf(nacc) < __builtin_inff() && d.eps >= 0.0f &&
                       d.eps < 0x1p124f;
  if (!(lane_ok && all_ok)) {
    TAM_STAT(TAM_ST_UPD_LANES);
#pragma unroll
    for (int k = 0; k < TAM_EPL / 2; ++k) {
      if (!(lane_ok && okp[k])) {
        TAM_STAT(TAM_ST_UPD_PAIRS);
        uint32_t w = 0u;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int i = 2 * k + j;
          const float den = __builtin_sqrtf(v[i] / d.bias_correction2) + d.eps;
          w |= (uint32_t)tam_round16(pw[i] + (d.neg_lr * m[i]) / (den * d.bias_correction1), DT) << (16 * j);
        }
        pw2[k] = w;
      }
    }
  }
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

// Position of workgroup b among the G workgroups of a tile loop.  Workgroups
// are dispatched to the 8 XCDs in turn (b % 8); with TAM_XCD_TILES the
// workgroups of one XCD take consecutive positions, so the tiles one round of
// the loop gives an XCD are consecutive and the small per-block arrays'
// 128-byte lines are written whole within one L2 (a line written in parts
// from two XCDs reaches memory as two partial writes, each a
// read-modify-write).  A permutation of 0 .. G-1 when G is a multiple of 8.
#ifndef TAM_XCD_TILES
#define TAM_XCD_TILES 1
#endif
__device__ __forceinline__ uint32_t tam_tile_slot(uint32_t b, uint32_t G) {
  if (!TAM_XCD_TILES || (G & 7u)) return b;
  return (b & 7u) * (G >> 3) + (b >> 3);
}

// The tensor holding `tile`, given that tensor ti or a later one holds it
// (persistent workgroups visit their tiles in increasing order).  A grid
// stride spans a few large tensors but can span hundreds of small ones, so a
// few steps forward come first and a binary search over the rest after: each
// step is a dependent load of a descriptor.
__device__ __forceinline__ int tam_advance_tensor(const TamTensor* __restrict__ T, int nT, int ti, uint32_t tile) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const TamTensor& d = T[__builtin_amdgcn_readfirstlane(ti)];
    if (tile < d.tile0 + d.ntiles) return ti;
    ++ti;  // a later tensor holds the tile, so ti + 1 < nT
  }
  int lo = ti, hi = nT - 1;  // the last tensor starting at or before the tile
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (T[__builtin_amdgcn_readfirstlane(mid)].tile0 <= tile) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Whether a wave's quarter of tile `wq` lies inside the tensor with aligned arrays.
__device__ __forceinline__ bool tam_quarter_full(const TamTensor& d, uint32_t wq) {
  const bool aligned = (((uintptr_t)d.param | (uintptr_t)d.grad) & 15u) == 0;
  return aligned && (uint64_t)(wq + 1u) * (4u * TAM_BLOCK_SIZE) <= d.n;
}

// ---------------------------------------------------------------------------
// Device-side step scalars (TAM_FLAG_DEVICE_STEP; a step captured in a graph)
// ---------------------------------------------------------------------------
// One workgroup.  First every DEVICE_STEP descriptor gets the fields the host
// fills otherwise, from the counters as they stand before this step: the step
// number (Philox counter word), the bias corrections of the group's step
// (reference optimizer.py:172-188, from the host-built table), 1/bc2 in fp64
// and fp32, -lr/bc1, and HAS_STATE / HAS_EF once the tensor has been updated;
// after a barrier the counters advance.  The divisions are the correctly
// rounded ones tam_prepare and the host perform.  When *found_inf is nonzero
// (a GradScaler skip) the descriptors get TAM_FLAG_SKIP instead, every later
// launch of the step returns at once, and the counters stay.
__global__ __launch_bounds__(1024) void tam_k_device_step(TamTensor* __restrict__ T, int nT) {
  for (int i = threadIdx.x; i < nT; i += blockDim.x) {
    TamTensor& d = T[i];
    if (!(d.flags & TAM_FLAG_DEVICE_STEP)) continue;
    const bool skip = d.found_inf != nullptr && *d.found_inf != 0.0f;
    const uint32_t own = *d.step_dev;
    const uint32_t t = *d.bc_step + 1u;
    const uint32_t k = (t < d.bc_len ? t : d.bc_len) - 1u;
    const float bc1 = d.bc_table[2u * k], bc2 = d.bc_table[2u * k + 1u];
    d.step = own + 1u;
    d.bias_correction1 = bc1;
    d.bias_correction2 = bc2;
    d.inv_bc2 = 1.0 / (double)bc2;
    d.inv_bc2_f32 = (float)d.inv_bc2;
    d.c_lr = d.neg_lr / bc1;
    d.k_abs = tam_abs_term(bc1, d.eps);
    uint32_t f = d.flags & ~(TAM_FLAG_HAS_STATE | TAM_FLAG_HAS_EF);
    if (own > 0u) {
      if (f & TAM_FLAG_COSTATE) f |= TAM_FLAG_HAS_STATE;
      if (f & TAM_FLAG_EF) f |= TAM_FLAG_HAS_EF;
    }
    d.flags = f | (skip ? TAM_FLAG_SKIP : 0u);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nT; i += blockDim.x) {
    const TamTensor& d = T[i];
    if ((d.flags & (TAM_FLAG_DEVICE_STEP | TAM_FLAG_SKIP)) == TAM_FLAG_DEVICE_STEP) *d.step_dev = d.step;
  }
}

// A step skipped on the device (TAM_FLAG_SKIP; found_inf is given for every
// descriptor or for none, so descriptor 0 decides for the whole step).
__device__ __forceinline__ bool tam_step_skipped(const TamTensor* __restrict__ T) {
  return (T[0].flags & TAM_FLAG_SKIP) != 0u;
}

// ---------------------------------------------------------------------------
// Pass 0: the fused update
// ---------------------------------------------------------------------------
// Per quarter tile: loads, first moment (CoState or fp32), second moment (1Q or
// fp32), update, store; for CoState tensors the fp64 partial sums of g.g and
// m.g over the quarter's 4 blocks (pairwise: blocks, then pairs of blocks).
template <uint32_t DT, bool FULL, bool EF = false>
__device__ __forceinline__ void tam_k1_quarter(const TamTensor& d, uint32_t wq, uint32_t lane, float* lutw,
                                               const TamLdsTabs* tabs, uint32_t seed_lo, uint32_t seed_hi,
                                               double2* __restrict__ part) {
  const TamWave W = tam_wave(d, wq, lane, FULL);
  const bool costate = (d.flags & TAM_FLAG_COSTATE) != 0;
  const bool compress_v = (d.flags & TAM_FLAG_COMPRESS_V) != 0;
  float g[TAM_EPL], p[TAM_EPL], m[TAM_EPL], v[TAM_EPL];
  // every load of the quarter is issued before any result is used
  if (FULL || W.bvalid) {
    tam_ld8<DT, FULL>(d.grad, W.e0, W.nv, g);
    tam_ld8<DT, FULL>(d.param, W.e0, W.nv, p);
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) g[i] = p[i] = 0.0f;
  }
  const TamCsIn cs = costate ? tam_cs_load<FULL>(d, W) : TamCsIn{0u, 0u, 0u, 0.0f};
  const TamVIn vin = compress_v ? tam_v_load<FULL>(d, W) : TamVIn{0u, 0u, 0u};
  const float alpha_prev = (costate && (d.flags & TAM_FLAG_HAS_STATE)) ? tam_g(d.alpha)[0] : 0.0f;
  tam_compiler_fence();
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) m[i] = v[i] = 0.0f;

  // ---- first moment ---------------------------------------------------
  if (costate) {
    if (EF) {  // error feedback: the EMA takes g + residual (costate.py:410-416)
      float ge[TAM_EPL];
      tam_ef_grad<FULL>(d, W, g, ge);
      if (FULL || W.bvalid) tam_costate_m<FULL>(d, W, cs, alpha_prev, g, ge, m);
    } else if (FULL || W.bvalid) {
      tam_costate_m<FULL>(d, W, cs, alpha_prev, g, g, m);
    }
    float gz[TAM_EPL], mz[TAM_EPL];
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      const bool ok = FULL || (W.bvalid && (uint32_t)i < W.nv);
      gz[i] = ok ? g[i] : 0.0f;
      mz[i] = ok ? m[i] : 0.0f;
    }
    // lane partials in fp32, then in fp64 per block and over the wave's 4
    // blocks (block k in lanes 16k..16k+15): adjacent pairs, then the two
    // pairs; lane 12 stores g.g, lane 13 m.g
    const double t = tam_quarter_sum2((double)tam_lane_dot(gz, gz), (double)tam_lane_dot(mz, gz), lane);
    if (lane - 12u < 2u) tam_g((double*)part)[lane - 12u] = t;
  } else if (FULL || W.bvalid) {
    // fp32 exp_avg (optimizer.py:113): m = fma(1-b1, g, fl(m*b1))
    float ea[TAM_EPL];
    tam_ld8_f32<FULL>(d.exp_avg, W.e0, W.nv, ea);
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) m[i] = __builtin_fmaf(d.one_minus_beta1, g[i], ea[i] * d.beta1);
    tam_st8_f32<FULL>(d.exp_avg, W.e0, W.nv, m);
  }

  // ---- second moment --------------------------------------------------
  float vc[TAM_EPL];
  TamVExt vx = {0u, 0u, 0u};
  if (compress_v) {
    vx = tam_vpath_a<FULL>(d, W, vin, g, v, vc, lutw, tabs);
  } else if (FULL || W.bvalid) {
    // fp32 exp_avg_sq (optimizer.py:166): v = fma(fl((1-b2)*g), g, fl(v*b2))
    float es[TAM_EPL];
    tam_ld8_f32<FULL>(d.exp_avg_sq, W.e0, W.nv, es);
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) v[i] = __builtin_fmaf(d.one_minus_beta2 * g[i], g[i], es[i] * d.beta2);
    tam_st8_f32<FULL>(d.exp_avg_sq, W.e0, W.nv, v);
  }

  // ---- parameter update -----------------------------------------------
  if (FULL || W.bvalid) {
    uint32_t pw2[TAM_EPL / 2];
    bool q_ok = false;
    if (DT != TAM_DTYPE_F32) q_ok = tam_q_in_range(d, compress_v ? vx : tam_lane_extremes<FULL>(v, W.nv));
    tam_update<DT>(d, p, m, v, pw2, q_ok);
    if (DT == TAM_DTYPE_F32) tam_st8_f32<FULL>((float*)d.param, W.e0, W.nv, p);
    else tam_st8_bits<FULL>(d.param, W.e0, W.nv, pw2);
  }

  // ---- re-quantisation of v -------------------------------------------
  if (compress_v) tam_vpath_b<FULL>(d, W, vc, vx, tabs, seed_lo, seed_hi);
}

// ---------------------------------------------------------------------------
// Pass 0 over full units: 16 elements per lane
// ---------------------------------------------------------------------------
// A unit is 8 consecutive blocks (1024 elements: quarters 2u and 2u + 1) of
// one tensor, processed by one wave: lane l owns elements [16(l%8), 16(l%8)+16)
// of block 8u + l/8, so the 8 lanes of each DPP half-row hold one block.  The
// arithmetic is the quarter path's, element for element; what is done once per
// block and lane -- the correctly rounded logs of the block extremes, the
// rounding bounds, the cross-lane reductions, the addressing -- is shared by 16
// elements of a lane instead of 8, and loads and stores move 32 bytes per lane
// and array.  The unit's two quarter partials go to their quarters' slots.
#define TAM_EPU 16   // elements per lane in a unit
#define TAM_K1U_WG 128  // threads of a (virtual) main pass-0 workgroup: two waves, one unit each per tile
// Virtual workgroups per hardware workgroup of the main pass-0 kernels: each
// pair of waves strides over the tiles as a workgroup of its own
#ifndef TAM_K1_VWG
#define TAM_K1_VWG 1
#endif
#define TAM_K1_BLOCK (TAM_K1U_WG * TAM_K1_VWG)

// Minimum / maximum / or over the 8 lanes of a half-row (one block).
__device__ __forceinline__ uint32_t tam_half_umin(uint32_t v) {
  v = __builtin_elementwise_min(v, tam_dpp<TAM_DPP_XOR1>(v));
  v = __builtin_elementwise_min(v, tam_dpp<TAM_DPP_XOR2>(v));
  return __builtin_elementwise_min(v, tam_dpp<TAM_DPP_HALF_MIRROR>(v));
}
__device__ __forceinline__ uint32_t tam_half_umax(uint32_t v) {
  v = __builtin_elementwise_max(v, tam_dpp<TAM_DPP_XOR1>(v));
  v = __builtin_elementwise_max(v, tam_dpp<TAM_DPP_XOR2>(v));
  return __builtin_elementwise_max(v, tam_dpp<TAM_DPP_HALF_MIRROR>(v));
}
__device__ __forceinline__ uint32_t tam_half_or(uint32_t v) {
  v |= tam_dpp<TAM_DPP_XOR1>(v);
  v |= tam_dpp<TAM_DPP_XOR2>(v);
  return v | tam_dpp<TAM_DPP_HALF_MIRROR>(v);
}

// Sums of a and b over each block (8 lanes, each holding the fp64 sum of its
// two 8-element partials), then over the unit's two quarters, (b0 + b1) +
// (b2 + b3) and (b4 + b5) + (b6 + b7): the pairwise tree of the quarter path.
// After the first step even lanes carry partial sums of a and odd lanes of b
// (every later step pairs lanes an even distance apart); row_ror:4 completes
// each block in lanes 4..7 of its half-row, row_ror:8 pairs the two blocks of
// a row in lanes 4..7 and 12..15, and the swap pairs rows 0/1 and 2/3.  The
// sums of a are valid in lanes 12 (quarter 0) and 44 (quarter 1), of b in
// lanes 13 and 45.  Requires every lane active.
__device__ __forceinline__ double tam_unit_sum2(double a, double b, uint32_t lane) {
  const bool odd = (lane & 1u) != 0;
  double x = (odd ? b : a) + tam_dppd<TAM_DPP_XOR1>(odd ? a : b);
  x = x + tam_dppd<TAM_DPP_XOR2>(x);
  x = x + tam_dppd<TAM_DPP_ROR4>(x);
  x = x + tam_dppd<TAM_DPP_ROR8>(x);
  return tam_swap_add<1>(x);
}

// Whether unit u lies inside the tensor with aligned arrays.
__device__ __forceinline__ bool tam_unit_full(const TamTensor& d, uint32_t u) {
  const bool aligned = (((uintptr_t)d.param | (uintptr_t)d.grad) & 15u) == 0;
  return aligned && (uint64_t)(u + 1u) * (8u * TAM_BLOCK_SIZE) <= d.n;
}

// 1Q decode (quantize.py:252-256), EMA (:259-270) and block extremes of a
// lane's 16 elements; as tam_vpath_a for a full quarter.  The 2^bits decode
// levels of a block are evaluated once: for at most 8 levels lane k of the
// block evaluates level k and elements fetch theirs with ds_bpermute; for 16
// and 64 levels the block's 8 lanes fill its row of a per-wave LDS table; 8-bit
// indices evaluate per element.
__device__ __forceinline__ TamVExt tam_vunit_a(const TamTensor& d, uint32_t lane, uint32_t sc, TamW4 iw,
                                               const float* g, float* v, float* lutw, const TamLdsTabs* tabs) {
  const uint32_t nbk = 1u << d.v_bits;
  const float inv_nbk = 1.0f / (float)nbk;  // exact power of two
  const float lmin0 = tam_f16_to_f32((uint16_t)(sc & 0xffffu));
  const float span0 = tam_f16_to_f32((uint16_t)(sc >> 16)) - lmin0;  // quantize.py:253-255
  const uint32_t ws[4] = {iw.x, iw.y, iw.z, iw.w};
  uint32_t idx[TAM_EPU];
#pragma unroll
  for (int i = 0; i < TAM_EPU; ++i) idx[i] = (ws[i >> 2] >> (8 * (i & 3))) & 0xffu;
  const uint32_t l8 = lane & 7u;
  float vo[TAM_EPU];
  if (nbk <= 8u) {
    // every lane of the wave takes part in the permutes
    const uint32_t k = l8 & (nbk - 1u);
    const float val = tam_expf_lds(lmin0 + ((float)k + 0.5f) * inv_nbk * span0, tabs);
    const uint32_t row = lane & ~7u;
#pragma unroll
    for (int i = 0; i < TAM_EPU; ++i) {
      const int src = (int)((row + (idx[i] & (nbk - 1u))) << 2);
      vo[i] = tam_u2f((uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)tam_f2u(val)));
    }
  } else if (nbk <= 64u) {
    float* tab = lutw + (lane >> 3) * 64u;
    for (uint32_t k = l8; k < nbk; k += 8u) tab[k] = tam_expf_lds(lmin0 + ((float)k + 0.5f) * inv_nbk * span0, tabs);
    tam_wave_lds_sync();
    // LDS byte address of element i's level: the row (256 bytes, 256-byte
    // aligned) or'ed with 4 * index, the index word shifted so that index i
    // lands at bit 2 and masked to 4 * (2^bits - 1)
    const uint32_t base = (uint32_t)(uintptr_t)(TAM_LDS float*)tab, vmask = tam_vcopy(4u * (nbk - 1u));
#pragma unroll
    for (int i = 0; i < TAM_EPU; ++i) {
      const uint32_t w = ws[i >> 2], sh = 8u * (uint32_t)(i & 3);
      const uint32_t a = tam_and_or(sh == 0u ? w << 2 : w >> (sh - 2u), vmask, base);
      vo[i] = *(const TAM_LDS float*)(uintptr_t)a;
    }
    tam_wave_lds_sync();  // the next unit rewrites the table
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPU; ++i) vo[i] = tam_expf_lds(lmin0 + ((float)idx[i] + 0.5f) * inv_nbk * span0, tabs);
  }
  TamVExt x;
  if (d.beta2 >= 0.0f && d.one_minus_beta2 >= 0.0f) {  // uniform: v >= +0 or NaN (see tam_vpath_a)
    // v is never -0 here (vo >= +0 from the levels, g*g >= +0, and an fma
    // whose addends are +0 and -0 gives +0), so its bit pattern orders as
    // the value; a NaN of either sign lies above +inf
    uint32_t xmn = 0xffffffffu, xmx = 0u;
#pragma unroll
    for (int i = 0; i < TAM_EPU; ++i) {
      v[i] = __builtin_fmaf(d.one_minus_beta2, g[i] * g[i], vo[i] * d.beta2);
      const uint32_t k = tam_f2u(v[i]);
      xmn = __builtin_elementwise_min(xmn, k);
      xmx = __builtin_elementwise_max(xmx, k);
    }
    x.kmn = tam_half_umin(xmn);
    x.kmx = tam_half_umax(xmx);
    x.nan_seen = x.kmx > 0x7f800000u ? TAM_VEXT_NAN : 0u;
  } else {
    // v may be negative: extremes of the clamped v, NaN tested per element
    uint32_t kmn = 0x7f800000u, kmx = 0u, nan_seen = 0u;
#pragma unroll
    for (int i = 0; i < TAM_EPU; ++i) {
      v[i] = __builtin_fmaf(d.one_minus_beta2, g[i] * g[i], vo[i] * d.beta2);
      const float vc = v[i] < 1e-38f ? 1e-38f : v[i];
      nan_seen |= tam_isnan(vc) ? 1u : 0u;
      kmn = __builtin_elementwise_min(kmn, tam_f2u(vc));
      kmx = __builtin_elementwise_max(kmx, tam_f2u(vc));
    }
    x.kmn = tam_half_umin(kmn);
    x.kmx = tam_half_umax(kmx);
    x.nan_seen = (tam_half_or(nan_seen) ? TAM_VEXT_NAN : 0u) | TAM_VEXT_CLAMPED;
  }
  return x;
}

// Logs of the block extremes, scales, certified stochastic re-quantisation of
// a lane's 16 elements; as tam_vpath_b for a full quarter (same bound, same
// fast path, same exact fallback).  Every v of a block that passes the block
// test lies in [vmin, vmax] with vmin >= 2^-126, where the clamp to 1e-38
// (quantize.py:275) leaves it unchanged, so the fast path reads v itself; the
// exact path clamps.
__device__ __forceinline__ void tam_vunit_b(const TamTensor& d, uint32_t lane, uint32_t b, uint64_t e0,
                                            const float* v, TamVExt x, const TamLdsTabs* tabs, uint32_t seed_lo,
                                            uint32_t seed_hi) {
  const float fnb = (float)(1u << d.v_bits);
  const uint32_t l8 = lane & 7u;
  const uint32_t kmn = __builtin_elementwise_max(x.kmn, TAM_BITS_1EM38);
  const uint32_t kmx = __builtin_elementwise_max(x.kmx, TAM_BITS_1EM38);
  const bool nan_seen = (x.nan_seen & TAM_VEXT_NAN) != 0u;
  // correctly rounded logs of the extremes: even lanes log(vmin), odd lanes log(vmax)
  const float lx = tam_logf_lds(tam_u2f((l8 & 1u) ? kmx : kmn), tabs);
  const float ly = tam_dppf<TAM_DPP_XOR1>(lx);
  float lmn = (l8 & 1u) ? ly : lx;
  float lmx = (l8 & 1u) ? lx : ly;
  if (nan_seen) lmn = lmx = tam_qnan();  // torch.min / torch.max propagate NaN
  float sp = lmx - lmn;  // quantize.py:283
  sp = sp < 1e-10f ? 1e-10f : sp;
  if (l8 == 0u)
    tam_g((uint32_t*)d.v_scales)[b] = (uint32_t)tam_f32_to_f16(lmn) | ((uint32_t)tam_f32_to_f16(lmx) << 16);
  const float rsp = __builtin_amdgcn_rcpf(sp);
  const float K = (0x1.62e430p-1f * fnb) * rsp;
  // the block bound of tam_vpath_b (full blocks)
  const float rmin = __builtin_amdgcn_rcpf(tam_u2f(kmn));
  const float Lm = __builtin_fmaxf(__builtin_fabsf(lmn), __builtin_fabsf(lmx));
  const float per_sp = __builtin_fmaf(Lm + __builtin_fabsf(lmn), 0x1p-24f, 0x1p-22f);
  const float flat = __builtin_fmaf(fnb, 0x1p-21f + 0x1p-20f, (fnb + 2.0f) * 0x1p-21f);
  const float Bb = __builtin_fmaf(fnb * rsp, per_sp, flat) * (1.0f + 0x1p-16f);
  const bool blk_ok = (tam_u2f(kmn) >= 0x1p-126f) && (tam_u2f(kmx) < 0x1p100f) && !nan_seen && (sp <= 64.0f) &&
                      (Bb < 0.25f);
  // The fast path subtracts u' = hi 2^-16 + 2^-17 from c~ + 1, hi the high 16
  // bits of the draw: |u - u'| <= 2^-17.  The quarter path's bound plus 2^-17
  // covers that, plus 2^-21 the rounding of the larger c~ + 1.
  const float H = blk_ok ? 0.5f - (Bb + (0x1p-17f + 0x1p-21f)) : -1.0f;
  const uint32_t byte_lsb = d.v_bits < 8u ? 0x01010101u : 0u;  // uniform
  const uint32_t m16 = tam_vconst(0x7fff80u), one = tam_vconst(0x3f800040u);  // 1 + 2^-17
  // the lane's 16 elements are one group of draws (tam_draws8): half h of 8
  // takes its high parts from block 3t + h; the low bytes (block 3t + 2) are
  // computed only where the exact path runs
  const uint64_t c0 = 3u * (e0 >> 4);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const float* vh = v + TAM_EPL * h;
    const TamU4 a = tam_philox_block(c0 + (uint32_t)h, d.tensor_id, d.step, seed_lo, seed_hi);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
    // draw i as the fp32 1 + u': the high 16 bits of the draw (half i % 2 of
    // word i / 2) at mantissa bits 7..22 over 1 + 2^-17
    const auto draw1 = [&](int i) -> float {
      const uint32_t x = w[i >> 1];
      return tam_u2f(tam_and_or((i & 1) ? x >> 9 : __builtin_amdgcn_alignbit(x, x, 25), m16, one));
    };
    uint32_t ow[2] = {0u, 0u};
    float tmax = 0.0f;
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      const float l2 = __builtin_amdgcn_logf(vh[i] * rmin);
      const float dd = __builtin_fmaf(l2, K, 1.5f) - draw1(i);  // fl(fl(c~ + 1) - (1 + u'))
      const float q = __builtin_rintf(dd);
      tmax = __builtin_fmaxf(tmax, __builtin_fabsf(dd - q));
      // v_cvt_pk_u8_f32 saturates to [0, 255]; the exact path overwrites rejected elements
      ow[i >> 2] = __builtin_amdgcn_cvt_pk_u8_f32(q, i & 3, ow[i >> 2]);
    }
    // An accepted q lies in [0, 2^bits] (q = -1 or 2^bits + 1 would put d half
    // a unit from q), so the clamp to 2^bits - 1 moves only the byte 2^bits:
    // each byte loses its bit `bits` (no borrow crosses a byte; with 8 bits the
    // saturation has clamped)
    ow[0] -= (ow[0] >> d.v_bits) & byte_lsb;
    ow[1] -= (ow[1] >> d.v_bits) & byte_lsb;
    if (!(tmax < H)) {  // false for a NaN bound (then H = -1)
      TAM_STAT(TAM_ST_VQ_LANES);
      // exact path: the reference's own sequence with correctly rounded log
      // and division, and the whole 24-bit draws
      const TamU4 c = tam_philox_block(c0 + 2u, d.tensor_id, d.step, seed_lo, seed_hi);
      const uint32_t lo0 = h ? c.z : c.x, lo1 = h ? c.w : c.y;
      uint32_t rw[TAM_EPL];
#pragma unroll
      for (int i = 0; i < TAM_EPL; ++i) rw[i] = tam_draw24(w[i >> 1], (uint32_t)i & 1u, (i < 4 ? lo0 : lo1) >> (8 * (i & 3)));
#pragma unroll
      for (int i = 0; i < TAM_EPL; ++i) {
        const float dd = __builtin_fmaf(__builtin_amdgcn_logf(vh[i] * rmin), K, 1.5f) - draw1(i);
        if (!(__builtin_fabsf(dd - __builtin_rintf(dd)) < H)) {
          TAM_STAT(TAM_ST_VQ_ELEMS);
          const float vc = vh[i] < 1e-38f ? 1e-38f : vh[i];  // quantize.py:275
          const float l = tam_logf_lds(vc, tabs);
          const float c = ((l - lmn) / sp) * fnb;  // quantize.py:284-285
          const float f = __builtin_floorf(c);
          const float fr = c - f;
          const float u = (float)rw[i] * 0x1p-24f;
          float q = f + (u < fr ? 1.0f : 0.0f);  // quantize.py:288-294
          q = q < 0.0f ? 0.0f : q;
          q = q > fnb - 1.0f ? fnb - 1.0f : q;
          const uint32_t qi = tam_isnan(q) ? 0u : (uint32_t)q;
          const uint32_t sh = 8u * (uint32_t)(i & 3);
          ow[i >> 2] = (ow[i >> 2] & ~(0xffu << sh)) | (qi << sh);
        }
      }
    }
    tam_g((TamW2*)(d.v_idx + e0 + TAM_EPL * h))[0] = TamW2{ow[0], ow[1]};
  }
}

// One wave's unit: loads, first moment (CoState or fp32), second moment (1Q or
// fp32), update, store; for CoState tensors the partial sums of g.g and m.g of
// the unit's two quarters (part: quarter 2u's {g.g, m.g}, then 2u + 1's).
// Every load of the unit (but an fp32 parameter's) is issued first and its
// value pinned, so the unit waits on memory once.
template <uint32_t DT>
__device__ __forceinline__ void tam_k1_unit(const TamTensor& d, uint32_t u, uint32_t lane, float* lutw,
                                            const TamLdsTabs* tabs, uint32_t seed_lo, uint32_t seed_hi,
                                            double* __restrict__ part) {
  constexpr int NW = DT == TAM_DTYPE_F32 ? 4 : 2;  // 16-byte words per lane of a parameter-dtype array
  const uint32_t l8 = lane & 7u;
  const uint32_t b = u * 8u + (lane >> 3);
  const uint64_t e0 = (uint64_t)b * TAM_BLOCK_SIZE + l8 * TAM_EPU;
  const bool costate = (d.flags & TAM_FLAG_COSTATE) != 0;
  const bool compress_v = (d.flags & TAM_FLAG_COMPRESS_V) != 0;
  const bool has_state = costate && (d.flags & TAM_FLAG_HAS_STATE);
  const uint64_t off = e0 * (DT == TAM_DTYPE_F32 ? 4u : 2u);
  TamW4 gw[NW], pw[NW];
#pragma unroll
  for (int k = 0; k < NW; ++k) gw[k] = tam_g((const TamW4*)((const char*)d.grad + off))[k];
  // an fp32 parameter (16 registers) is loaded just before the update: held
  // from here it would make the kernel spill at 4 waves per SIMD
  if constexpr (DT != TAM_DTYPE_F32) {
#pragma unroll
    for (int k = 0; k < NW; ++k) pw[k] = tam_g((const TamW4*)((const char*)d.param + off))[k];
  }
  uint32_t label = 0u, amp = 0u, sbytes = 0u;  // sbytes: sign bytes of elements e0..e0+7 (low) and e0+8..e0+15
  float nrm = 0.0f, alpha_prev = 0.0f;
  if (has_state) {
    label = tam_g(d.labels)[b];
    nrm = tam_g(d.norms)[b];
    amp = tam_g(d.amp)[b];
    sbytes = tam_g((const uint16_t*)(d.signs + (e0 >> 3)))[0];
    alpha_prev = tam_g(d.alpha)[0];
  }
  uint32_t sc = 0u;
  TamW4 iw = {0u, 0u, 0u, 0u};
  if (compress_v) {
    sc = tam_g((const uint32_t*)d.v_scales)[b];
    iw = tam_g((const TamW4*)(d.v_idx + e0))[0];
  }
  tam_compiler_fence();
#pragma unroll
  for (int k = 0; k < NW; ++k) {
    tam_pin(gw[k]);
    if constexpr (DT != TAM_DTYPE_F32) tam_pin(pw[k]);
  }
  tam_pin(label);
  tam_pin(nrm);
  tam_pin(amp);
  tam_pin(sbytes);
  tam_pin(alpha_prev);
  tam_pin(sc);
  tam_pin(iw);
  float g[TAM_EPU], p[TAM_EPU], m[TAM_EPU], v[TAM_EPU];
  if constexpr (DT == TAM_DTYPE_F32) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const TamF4 gk = __builtin_bit_cast(TamF4, gw[k]);
      g[4 * k] = gk.x; g[4 * k + 1] = gk.y; g[4 * k + 2] = gk.z; g[4 * k + 3] = gk.w;
    }
  } else {
    tam_unpack8<DT>(gw[0], g);
    tam_unpack8<DT>(gw[1], g + TAM_EPL);
    tam_unpack8<DT>(pw[0], p);
    tam_unpack8<DT>(pw[1], p + TAM_EPL);
  }
  const TamCsIn cs = {label, amp, 0u, nrm};

  // ---- first moment ---------------------------------------------------
  if (costate) {
    if (has_state) {
      const uint32_t sabs = tam_cs_sabs(cs);  // shared by the lane's two sign bytes
      tam_cs_decode_m<true>(d, sabs, sbytes & 0xffu, alpha_prev, g, g, m);
      tam_cs_decode_m<true>(d, sabs, sbytes >> 8, alpha_prev, g + TAM_EPL, g + TAM_EPL, m + TAM_EPL);
    } else {
#pragma unroll
      for (int i = 0; i < TAM_EPU; ++i) m[i] = d.beta1 * 0.0f + d.one_minus_beta1 * g[i];
    }
    // lane partials in fp32, their fp64 sum, then per block and quarter in fp64
    const double t = tam_unit_sum2((double)tam_lane_dot(g, g) + (double)tam_lane_dot(g + TAM_EPL, g + TAM_EPL),
                                   (double)tam_lane_dot(m, g) + (double)tam_lane_dot(m + TAM_EPL, g + TAM_EPL),
                                   lane);
    if ((lane & 31u) - 12u < 2u) tam_g(part)[(lane >> 5) * 2u + (lane & 1u)] = t;
  } else {
    // fp32 exp_avg (optimizer.py:113): m = fma(1-b1, g, fl(m*b1))
    // (fp32 moments are loaded here, not with the unit's other loads: their
    // registers would otherwise count against every unit of the kernel)
    float ea[TAM_EPU];
    tam_ld8_f32<true>(d.exp_avg, e0, TAM_EPL, ea);
    tam_ld8_f32<true>(d.exp_avg, e0 + TAM_EPL, TAM_EPL, ea + TAM_EPL);
#pragma unroll
    for (int i = 0; i < TAM_EPU; ++i) m[i] = __builtin_fmaf(d.one_minus_beta1, g[i], ea[i] * d.beta1);
    tam_st8_f32<true>(d.exp_avg, e0, TAM_EPL, m);
    tam_st8_f32<true>(d.exp_avg, e0 + TAM_EPL, TAM_EPL, m + TAM_EPL);
  }

  // ---- second moment --------------------------------------------------
  TamVExt vx = {0u, 0u, 0u};
  if (compress_v) {
    vx = tam_vunit_a(d, lane, sc, iw, g, v, lutw, tabs);
  } else {
    // fp32 exp_avg_sq (optimizer.py:166): v = fma(fl((1-b2)*g), g, fl(v*b2))
    float es[TAM_EPU];
    tam_ld8_f32<true>(d.exp_avg_sq, e0, TAM_EPL, es);
    tam_ld8_f32<true>(d.exp_avg_sq, e0 + TAM_EPL, TAM_EPL, es + TAM_EPL);
#pragma unroll
    for (int i = 0; i < TAM_EPU; ++i) v[i] = __builtin_fmaf(d.one_minus_beta2 * g[i], g[i], es[i] * d.beta2);
    tam_st8_f32<true>(d.exp_avg_sq, e0, TAM_EPL, v);
    tam_st8_f32<true>(d.exp_avg_sq, e0 + TAM_EPL, TAM_EPL, v + TAM_EPL);
  }

  // ---- parameter update -----------------------------------------------
  {
    if constexpr (DT == TAM_DTYPE_F32) {
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        const TamF4 pk = __builtin_bit_cast(TamF4, tam_g((const TamW4*)((const char*)d.param + off))[k]);
        p[4 * k] = pk.x; p[4 * k + 1] = pk.y; p[4 * k + 2] = pk.z; p[4 * k + 3] = pk.w;
      }
    }
    uint32_t pw2[TAM_EPU / 2];
    bool q_ok = false;
    if (DT != TAM_DTYPE_F32) {
      TamVExt e = vx;
      if (!compress_v) {
        const TamVExt e1 = tam_lane_extremes<true>(v, TAM_EPL), e2 = tam_lane_extremes<true>(v + TAM_EPL, TAM_EPL);
        e.kmn = __builtin_elementwise_min(e1.kmn, e2.kmn);
        e.kmx = __builtin_elementwise_max(e1.kmx, e2.kmx);
        e.nan_seen = e1.nan_seen | e2.nan_seen;
      }
      q_ok = tam_q_in_range(d, e);
    }
    tam_update<DT>(d, p, m, v, pw2, q_ok);
    tam_update<DT>(d, p + TAM_EPL, m + TAM_EPL, v + TAM_EPL, pw2 + TAM_EPL / 2, q_ok);
    if (DT == TAM_DTYPE_F32) {
      tam_st8_f32<true>((float*)d.param, e0, TAM_EPL, p);
      tam_st8_f32<true>((float*)d.param, e0 + TAM_EPL, TAM_EPL, p + TAM_EPL);
    } else {
      tam_st8_bits<true>(d.param, e0, TAM_EPL, pw2);
      tam_st8_bits<true>(d.param, e0 + TAM_EPL, TAM_EPL, pw2 + TAM_EPL / 2);
    }
  }

  // ---- re-quantisation of v -------------------------------------------
  if (compress_v) tam_vunit_b(d, lane, b, e0, v, vx, tabs, seed_lo, seed_hi);
}

// Full units (inside the tensor, aligned arrays) of one parameter dtype:
// persistent workgroups of two waves stride over the tiles; wave w takes unit
// 2(tile - tile0) + w of the tile's tensor (quarters 4(tile - tile0) + 2w and
// + 2w + 1), and the waves never synchronise with each other.  One kernel per
// dtype holds only that dtype's code, so each gets its own register budget.
template <uint32_t DT>
__device__ __forceinline__ void tam_k1_full_body(const TamTensor* __restrict__ T, int nT, uint32_t total_tiles,
                                                 uint32_t seed_lo, uint32_t seed_hi,
                                                 double2* __restrict__ partials) {
  if (tam_step_skipped(T)) return;
  // rows of 64 levels, 256-byte aligned (tam_vunit_a forms addresses by or)
  __shared__ __attribute__((aligned(256))) float lut[TAM_K1_BLOCK / 64][8 * 64];
  __shared__ TamLdsTabs tabs;
  tam_lds_tabs_fill(&tabs);
  const uint32_t hw_wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;
  const uint32_t wave = hw_wave & 1u;  // within the virtual workgroup
  const uint32_t stride = gridDim.x * TAM_K1_VWG;
  float* lutw = lut[hw_wave];
  // tensor by tensor: the descriptor is read once per tensor, then the wave
  // takes its units of the tensor in grid strides
  uint32_t tile = tam_tile_slot(blockIdx.x, gridDim.x) * TAM_K1_VWG + (hw_wave >> 1);
  int ti = tam_find_tensor(T, nT, tile < total_tiles ? tile : total_tiles - 1u);
  while (tile < total_tiles) {
    ti = tam_advance_tensor(T, nT, ti, tile);
    const TamTensor& d = T[ti];
    const uint32_t end = d.tile0 + d.ntiles;  // the tensor's tiles end here
    if (d.dtype == DT && !(d.flags & TAM_FLAG_EF)) {  // uniform; EF: tam_k1_ef
      // units u < nfull are full (inside the tensor, aligned arrays); the
      // rest are tam_k1_tail's, and u grows with the tile
      const bool aligned = (((uintptr_t)d.param | (uintptr_t)d.grad) & 15u) == 0;
      const uint64_t nfull = aligned ? d.n / (8u * TAM_BLOCK_SIZE) : 0u;
      for (; tile < end; tile += stride) {
        const uint32_t u = (tile - d.tile0) * 2u + wave;  // unit within the tensor
        if (u >= nfull) break;
        double* part = (double*)(partials + (uint64_t)tile * 4u + 2u * wave);
        tam_k1_unit<DT>(d, u, lane, lutw, &tabs, seed_lo, seed_hi, part);
      }
    }
    while (tile < end) tile += stride;  // this workgroup's first tile past the tensor
  }
}

#define TAM_K1_FULL_KERNEL(NAME, DT, WAVES)                                                                     \
  __global__ __launch_bounds__(TAM_K1_BLOCK) __attribute__((amdgpu_waves_per_eu(WAVES, WAVES))) void NAME(    \
      const TamTensor* __restrict__ T, int nT, uint32_t total_tiles, uint32_t seed_lo, uint32_t seed_hi,      \
      double2* __restrict__ partials) {                                                                       \
    tam_k1_full_body<DT>(T, nT, total_tiles, seed_lo, seed_hi, partials);                                     \
  }
#ifndef TAM_K1_WAVES_BF16
#define TAM_K1_WAVES_BF16 4
#endif
#ifndef TAM_K1_WAVES_F16
#define TAM_K1_WAVES_F16 4
#endif
#ifndef TAM_K1_WAVES_F32
#define TAM_K1_WAVES_F32 4
#endif
TAM_K1_FULL_KERNEL(tam_k1_main_bf16, TAM_DTYPE_BF16, TAM_K1_WAVES_BF16)
TAM_K1_FULL_KERNEL(tam_k1_main_f16, TAM_DTYPE_F16, TAM_K1_WAVES_F16)
TAM_K1_FULL_KERNEL(tam_k1_main_f32, TAM_DTYPE_F32, TAM_K1_WAVES_F32)

// ---------------------------------------------------------------------------
// Selection state of a CoState tensor (workspace), set afresh every step by
// pass 0's tail kernel
// ---------------------------------------------------------------------------
struct TamSel {
  uint32_t kmin, kmax;  // key range (tam_k_sel_minmax)
  uint32_t prefix[2];   // bits fixed so far of the k_lo-th and k_hi-th smallest ratio
  uint32_t k[2];        // rank within the ratios sharing that prefix
  uint32_t mask;        // bits fixed so far
  int32_t top;          // highest bit not yet fixed (-1: done; 32: no round run yet)
};

// Every thread of one workgroup: tensor d's selection state before the key
// range is known and its cleared histogram (4096 counts).
__device__ __forceinline__ void tam_sel_reset_wg(const TamTensor& d, TamSel* __restrict__ sel,
                                                 uint32_t* __restrict__ hist) {
  for (uint32_t i = threadIdx.x; i < 4096u; i += blockDim.x) tam_g(hist)[i] = 0u;
  if (threadIdx.x == 0) {
    TamSel z;
    z.kmin = 0xffffffffu;
    z.kmax = 0u;
    z.prefix[0] = z.prefix[1] = 0u;
    z.k[0] = d.k_lo;
    z.k[1] = d.k_hi;
    z.mask = 0u;
    z.top = 32;
    *sel = z;
  }
}

// The quarters outside full units: the last (at most five) quarters of each
// tensor, or every quarter of a tensor whose parameter or gradient is not
// 16-byte aligned.  An aligned tensor has one workgroup; an unaligned one has
// one per TAM_TAIL_TILES tiles (tam_prepare: tail0, tail_wgs), so a large
// unaligned tensor spreads over the GPU.  Wave w takes every fourth quarter of
// the workgroup's range.
__device__ __forceinline__ int tam_tail_tensor(const TamTensor* __restrict__ T, int nT, uint32_t wg) {
  int lo = 0, hi = nT - 1;  // the last tensor whose first tail workgroup is at or before wg
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (T[mid].tail0 <= wg) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__global__ __launch_bounds__(TAM_WG) void tam_k1_tail(const TamTensor* __restrict__ T, int nT, uint32_t seed_lo,
                                                      uint32_t seed_hi, double2* __restrict__ partials,
                                                      TamSel* __restrict__ sel, uint32_t* __restrict__ hist) {
  if (tam_step_skipped(T)) return;
  const int ti = tam_tail_tensor(T, nT, blockIdx.x);
  const TamTensor& d = T[ti];
  // the tensor's first tail workgroup sets its selection state
  if ((d.flags & TAM_FLAG_COSTATE) && blockIdx.x == d.tail0)
    tam_sel_reset_wg(d, sel + ti, hist + (uint64_t)ti * 4096u);
  if (d.flags & TAM_FLAG_EF) return;  // the whole workgroup: tam_k1_ef covers the tensor
  __shared__ float lut[TAM_WG / 64][4 * 64];
  __shared__ TamLdsTabs tabs;
  tam_lds_tabs_fill(&tabs);
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  const bool aligned = (((uintptr_t)d.param | (uintptr_t)d.grad) & 15u) == 0;
  const uint32_t nq = d.ntiles * 4u;
  uint32_t first, last;
  if (aligned) {  // full units precede: tam_k1_main_<dtype> takes them
    first = 2u * (uint32_t)(d.n / (8u * TAM_BLOCK_SIZE));
    last = nq;
  } else {
    const uint32_t local = blockIdx.x - d.tail0;
    first = local * (4u * TAM_TAIL_TILES);
    last = first + 4u * TAM_TAIL_TILES < nq ? first + 4u * TAM_TAIL_TILES : nq;
  }
  for (uint32_t wq = first + wave; wq < last; wq += 4u) {
    double2* part = partials + (uint64_t)d.tile0 * 4u + wq;
    switch (d.dtype) {
      case TAM_DTYPE_BF16:
        tam_k1_quarter<TAM_DTYPE_BF16, false>(d, wq, lane, lut[wave], &tabs, seed_lo, seed_hi, part);
        break;
      case TAM_DTYPE_F16:
        tam_k1_quarter<TAM_DTYPE_F16, false>(d, wq, lane, lut[wave], &tabs, seed_lo, seed_hi, part);
        break;
      default:
        tam_k1_quarter<TAM_DTYPE_F32, false>(d, wq, lane, lut[wave], &tabs, seed_lo, seed_hi, part);
        break;
    }
  }
}

// Every quarter of the tensors with error feedback (full or not, any dtype):
// persistent workgroups stride over the tiles as the main kernels do.
__global__ __launch_bounds__(TAM_WG) void tam_k1_ef(const TamTensor* __restrict__ T, int nT, uint32_t total_tiles,
                                                    uint32_t seed_lo, uint32_t seed_hi,
                                                    double2* __restrict__ partials) {
  if (tam_step_skipped(T)) return;
  __shared__ float lut[TAM_WG / 64][4 * 64];
  __shared__ TamLdsTabs tabs;
  tam_lds_tabs_fill(&tabs);
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  int ti = tam_find_tensor(T, nT, blockIdx.x);
  for (uint32_t tile = blockIdx.x; tile < total_tiles; tile += gridDim.x) {
    ti = tam_advance_tensor(T, nT, ti, tile);
    const TamTensor& d = T[ti];
    if (!(d.flags & TAM_FLAG_EF)) continue;  // uniform over the workgroup
    const uint32_t wq = (tile - d.tile0) * 4u + wave;
    double2* part = partials + (uint64_t)tile * 4u + wave;
    const bool full = tam_quarter_full(d, wq);
    switch (d.dtype) {
      case TAM_DTYPE_BF16:
        if (full) tam_k1_quarter<TAM_DTYPE_BF16, true, true>(d, wq, lane, lut[wave], &tabs, seed_lo, seed_hi, part);
        else tam_k1_quarter<TAM_DTYPE_BF16, false, true>(d, wq, lane, lut[wave], &tabs, seed_lo, seed_hi, part);
        break;
      case TAM_DTYPE_F16:
        if (full) tam_k1_quarter<TAM_DTYPE_F16, true, true>(d, wq, lane, lut[wave], &tabs, seed_lo, seed_hi, part);
        else tam_k1_quarter<TAM_DTYPE_F16, false, true>(d, wq, lane, lut[wave], &tabs, seed_lo, seed_hi, part);
        break;
      default:
        if (full) tam_k1_quarter<TAM_DTYPE_F32, true, true>(d, wq, lane, lut[wave], &tabs, seed_lo, seed_hi, part);
        else tam_k1_quarter<TAM_DTYPE_F32, false, true>(d, wq, lane, lut[wave], &tabs, seed_lo, seed_hi, part);
        break;
    }
  }
}

// ---------------------------------------------------------------------------
// Pass 1: alpha of every CoState tensor (costate.py:37-41)
// ---------------------------------------------------------------------------
// The dot products are balanced pairwise sums over the tensor's quarter-tile
// partials zero-padded to a power of two P.  The padded array is cut into
// aligned chunks of 8192 (one chunk of P when P <= 8192); chunk sums are
// subtrees of the same tree.  tam_k_alpha_chunks sums every chunk of every
// tensor (one workgroup per chunk: 32 consecutive values per thread, then a
// tree in LDS); tam_k_alpha sums each tensor's chunk sums (at most 2048, a
// power of two) and forms alpha.  Zero padding does not change the sum:
// x + 0 == x, and +0.0 added to the result settles the sign of an exact zero.
#define TAM_PAIR_PER_THREAD 32
#define TAM_CHUNK (TAM_WG * TAM_PAIR_PER_THREAD)

__device__ __forceinline__ uint32_t tam_pow2_at_least(uint32_t x) {
  uint32_t p = 1;
  while (p < x) p <<= 1;
  return p;
}
// Chunks of a tensor's padded partial array (0 for tensors without CoState).
__host__ __device__ __forceinline__ uint32_t tam_alpha_chunks(uint32_t flags, uint32_t ntiles) {
  if (!(flags & TAM_FLAG_COSTATE)) return 0;
  uint32_t p = 1;
  while (p < ntiles * 4u) p <<= 1;
  return p > TAM_CHUNK ? p / TAM_CHUNK : 1u;
}

// Pairwise sum of sh[0..n) (n a power of two, n <= 2 * TAM_WG) in place; every
// thread of the workgroup calls it.  Returns sh[0].
__device__ double2 tam_wg_tree(double2* sh, uint32_t n) {
  const uint32_t tid = threadIdx.x;
  for (uint32_t w = n / 2; w >= 1; w >>= 1) {
    double2 s = make_double2(0.0, 0.0);
    if (tid < w) {
      const double2 l = sh[2 * tid], r = sh[2 * tid + 1];
      s = make_double2(l.x + r.x, l.y + r.y);
    }
    __syncthreads();
    if (tid < w) sh[tid] = s;
    __syncthreads();
  }
  return sh[0];
}

__global__ __launch_bounds__(TAM_WG) void tam_k_alpha_chunks(const TamTensor* __restrict__ T, int nT,
                                                             const double2* __restrict__ partials,
                                                             double2* __restrict__ chunk_sums) {
  if (tam_step_skipped(T)) return;
  __shared__ double2 sh[TAM_WG];
  const uint32_t c = blockIdx.x;
  // tensor owning chunk c: the first whose chunk range ends after c
  int lo = 0, hi = nT - 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (T[mid].chunk0 + tam_alpha_chunks(T[mid].flags, T[mid].ntiles) > c) hi = mid; else lo = mid + 1;
  }
  const TamTensor& d = T[lo];
  const uint32_t count = d.ntiles * 4u;                 // quarter-tile partials of the tensor
  const uint32_t P = tam_pow2_at_least(count);
  const uint32_t lim = P > TAM_CHUNK ? TAM_CHUNK : P;   // leaves of this chunk's subtree
  const uint32_t base = (c - d.chunk0) * TAM_CHUNK;
  const double2* x = partials + (uint64_t)d.tile0 * 4u;
  const uint32_t tid = threadIdx.x;
  double sa[4], sq[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    double a[8], q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t local = tid * TAM_PAIR_PER_THREAD + h * 8 + i;
      const uint32_t k = base + local;
      const double2 v = (local < lim && k < count) ? x[k] : make_double2(0.0, 0.0);
      a[i] = v.x;
      q[i] = v.y;
    }
    sa[h] = tam_pair8(a);
    sq[h] = tam_pair8(q);
  }
  sh[tid] = make_double2((sa[0] + sa[1]) + (sa[2] + sa[3]), (sq[0] + sq[1]) + (sq[2] + sq[3]));
  __syncthreads();
  const double2 r = tam_wg_tree(sh, TAM_WG);
  if (tid == 0) chunk_sums[c] = r;
}

__global__ __launch_bounds__(TAM_WG) void tam_k_alpha(const TamTensor* __restrict__ T,
                                                      const double2* __restrict__ chunk_sums,
                                                      float* __restrict__ alpha_new) {
  if (tam_step_skipped(T)) return;
  __shared__ double2 sh[2048];
  const TamTensor& d = T[blockIdx.x];
  const uint32_t nch = tam_alpha_chunks(d.flags, d.ntiles);
  if (nch == 0) return;
  for (uint32_t i = threadIdx.x; i < nch; i += TAM_WG) sh[i] = chunk_sums[d.chunk0 + i];
  __syncthreads();
  // nch is a power of two <= 2048: fold it to at most 2 * TAM_WG with pairwise steps first
  uint32_t n = nch;
  while (n > 2 * TAM_WG) {
    const uint32_t w = n / 2;
    double2 s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = threadIdx.x + j * TAM_WG;
      if (i < w) s[j] = make_double2(sh[2 * i].x + sh[2 * i + 1].x, sh[2 * i].y + sh[2 * i + 1].y);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t i = threadIdx.x + j * TAM_WG;
      if (i < w) sh[i] = s[j];
    }
    __syncthreads();
    n = w;
  }
  const double2 s = tam_wg_tree(sh, n);
  if (threadIdx.x == 0) {
    // dot products round to fp32 once; +0.0 makes an exact-zero sum +0
    const float gg = (float)(s.x + 0.0);
    const float mg = (float)(s.y + 0.0);
    alpha_new[blockIdx.x] = gg > 0.0f ? mg / gg : 0.0f;
  }
}

// ---------------------------------------------------------------------------
// Pass 2: CoState encode (costate.py:419-425, :213-258) and block ratios (:51-86)
// ---------------------------------------------------------------------------
// With error feedback the EMA takes g + residual and the encoding goes to the
// tensor's staging area (pass 4 still needs the previous one).
// A pass-2 quarter (16 lanes per block, 8 elements per lane), its inputs loaded in place.
#define TAM_CONST __attribute__((address_space(4)))
template <uint32_t DT, bool FULL>
__device__ __forceinline__ void tam_k2_quarter(const TamTensor& d, uint32_t wq, uint32_t lane, float a,
                                               float* __restrict__ ratios, char* __restrict__ ws) {
  const TamWave W = tam_wave(d, wq, lane, FULL);
  const bool ef = (d.flags & TAM_FLAG_EF) != 0;  // uniform
  float dl[TAM_EPL], md[TAM_EPL];
  uint32_t sbyte = 0;
  if (FULL || W.bvalid) {
    float g[TAM_EPL], ge[TAM_EPL], m[TAM_EPL];
    tam_ld8<DT, FULL>(d.grad, W.e0, W.nv, g);
    const TamCsIn cs = tam_cs_load<FULL>(d, W);
    // a scalar load (alpha is not written in this pass): no vector-memory
    // wait covers the next quarter's loads
    const float alpha_prev = (d.flags & TAM_FLAG_HAS_STATE) ? *(const TAM_CONST float*)d.alpha : 0.0f;
    if (ef) {
      tam_ef_grad<FULL>(d, W, g, ge);
    } else {
#pragma unroll
      for (int i = 0; i < TAM_EPL; ++i) ge[i] = g[i];
    }
    tam_compiler_fence();
    tam_costate_m<FULL, false>(d, W, cs, alpha_prev, g, ge, m);
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      const bool ok = FULL || (uint32_t)i < W.nv;
      const float delta = ok ? m[i] - a * g[i] : 0.0f;  // costate.py:42
      dl[i] = delta;
      md[i] = ok ? m[i] : 0.0f;
      sbyte = 2u * sbyte + (delta < 0.0f ? 1u : 0u);  // element 8j+i is bit 7-i, costate.py:170-181
    }
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) dl[i] = md[i] = 0.0f;
  }
  // Block sums of squares: fp32 lane partials, then the fp64 tree of
  // tam_block_sum: the sum of delta^2 in lane 12 of the block's row, of m^2 in
  // lane 13.  Each lane of a pair evaluates one square root and one division:
  // lane 12 the residual norm and the amplitude, lane 13 the norm of m and the
  // ratio.
  const bool odd = (W.l16 & 1u) != 0;
  const float nx =
      (float)__builtin_sqrt(tam_row_sum2((double)tam_lane_dot(dl, dl), (double)tam_lane_dot(md, md), odd));
  const float ny = tam_dppf<TAM_DPP_XOR1>(nx);
  const float nd = odd ? ny : nx;  // costate.py:241
  const float nm = odd ? nx : ny;
  const float qv = nd / (odd ? nm : d.sqrt_block);  // costate.py:248 / :81-84
  if (FULL || W.bvalid) {
    uint8_t* signs = d.signs;
    float* norms = d.norms;
    uint16_t* amp = d.amp;
    if (ef) {
      const TamStage st = tam_stage(d, ws);
      signs = st.signs;
      norms = st.norms;
      amp = st.amp;
    }
    if (FULL || W.nv > 0) tam_g(signs)[W.e0 >> 3] = (uint8_t)sbyte;
    if (W.l16 == 12u) {
      tam_g(norms)[W.b] = nd;
      tam_g(amp)[W.b] = tam_f32_to_f16(qv);
    } else if (W.l16 == 13u) {
      tam_g(ratios)[d.ratio_off + W.b] = nm == 0.0f ? 0.0f : qv;
    }
  }
}

// A pass-2 quarter of any kind, its inputs loaded in place.
__device__ __forceinline__ void tam_k2_any(const TamTensor& d, uint32_t wq, uint32_t lane, float a,
                                           float* __restrict__ ratios, char* __restrict__ ws) {
  const bool full = tam_quarter_full(d, wq);
  switch (d.dtype) {
    case TAM_DTYPE_BF16:
      if (full) tam_k2_quarter<TAM_DTYPE_BF16, true>(d, wq, lane, a, ratios, ws);
      else tam_k2_quarter<TAM_DTYPE_BF16, false>(d, wq, lane, a, ratios, ws);
      break;
    case TAM_DTYPE_F16:
      if (full) tam_k2_quarter<TAM_DTYPE_F16, true>(d, wq, lane, a, ratios, ws);
      else tam_k2_quarter<TAM_DTYPE_F16, false>(d, wq, lane, a, ratios, ws);
      break;
    default:
      if (full) tam_k2_quarter<TAM_DTYPE_F32, true>(d, wq, lane, a, ratios, ws);
      else tam_k2_quarter<TAM_DTYPE_F32, false>(d, wq, lane, a, ratios, ws);
      break;
  }
}

// Pass 2 over full units of tensors without error feedback (the common case):
// 16 elements per lane, 8 lanes per block, as pass 0's main kernels.  The
// unit's inputs are loaded one unit ahead of their use: the lane's 16 gradient
// elements (two 16-byte words for a 16-bit tensor, four for fp32), its block's
// CoState state and its two sign bytes.  tam_k2_encode takes the units of
// 16-bit tensors, tam_k2_encode_f32 those of fp32 tensors (when it runs).
template <bool F32>
struct TamK2U {
  TamW4 g[F32 ? 4 : 2];
  TamCsIn cs;  // byte: the sign bytes of elements e0..e0+7 (low) and e0+8..e0+15
};
template <bool F32>
__device__ __forceinline__ bool tam_k2u_prefetchable(const TamTensor& d, uint32_t u) {
  return (d.dtype == TAM_DTYPE_F32) == F32 && !(d.flags & TAM_FLAG_EF) && tam_unit_full(d, u);
}
template <bool F32>
__device__ __forceinline__ TamK2U<F32> tam_k2u_load(const TamTensor& d, uint32_t u, uint32_t lane) {
  const uint32_t b = u * 8u + (lane >> 3);
  const uint64_t e0 = (uint64_t)b * TAM_BLOCK_SIZE + (lane & 7u) * TAM_EPU;
  const TAM_GLOBAL TamW4* gp = tam_g((const TamW4*)((const char*)d.grad + e0 * (F32 ? 4u : 2u)));
  TamK2U<F32> r;
#pragma unroll
  for (int k = 0; k < (F32 ? 4 : 2); ++k) r.g[k] = gp[k];
  r.cs = TamCsIn{0u, 0u, 0u, 0.0f};
  if (d.flags & TAM_FLAG_HAS_STATE) {
    r.cs.label = tam_g(d.labels)[b];
    r.cs.nrm = tam_g(d.norms)[b];
    r.cs.amp = tam_g(d.amp)[b];
    r.cs.byte = tam_g((const uint16_t*)(d.signs + (e0 >> 3)))[0];
  }
  return r;
}

// The CoState encode of a unit (as tam_k2_quarter for full quarters): m
// recomputed bit-identically, delta = m - alpha*g, sign bits, block norms of
// delta and m from fp32 lane partials and an fp64 tree over the block's 8
// lanes (the parity split of tam_unit_sum2: after row_ror:4 the sum of
// delta^2 is in lanes 4 and 6 of the half-row, of m^2 in lanes 5 and 7), the
// fp16 amplitude (lane 4) and the ratio (lane 5).
template <uint32_t DT>
__device__ __forceinline__ void tam_k2_unit(const TamTensor& d, uint32_t u, uint32_t lane, float a,
                                            float* __restrict__ ratios, const TamK2U<DT == TAM_DTYPE_F32>& in) {
  const uint32_t l8 = lane & 7u;
  const uint32_t b = u * 8u + (lane >> 3);
  const uint64_t e0 = (uint64_t)b * TAM_BLOCK_SIZE + l8 * TAM_EPU;
  float g[TAM_EPU], m[TAM_EPU], dl[TAM_EPU];
  if constexpr (DT == TAM_DTYPE_F32) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const TamF4 gk = __builtin_bit_cast(TamF4, in.g[k]);
      g[4 * k] = gk.x; g[4 * k + 1] = gk.y; g[4 * k + 2] = gk.z; g[4 * k + 3] = gk.w;
    }
  } else {
    tam_unpack8<DT>(in.g[0], g);
    tam_unpack8<DT>(in.g[1], g + TAM_EPL);
  }
  // a scalar load (alpha is not written in this pass): no vector-memory wait
  // covers the next unit's loads
  const float alpha_prev = (d.flags & TAM_FLAG_HAS_STATE) ? *(const TAM_CONST float*)d.alpha : 0.0f;
  TamWave W;  // only its bvalid is read (full unit)
  W.bvalid = true;
  TamCsIn c0 = in.cs, c1 = in.cs;
  c0.byte = in.cs.byte & 0xffu;
  c1.byte = in.cs.byte >> 8;
  tam_costate_m<true, false>(d, W, c0, alpha_prev, g, g, m);
  tam_costate_m<true, false>(d, W, c1, alpha_prev, g + TAM_EPL, g + TAM_EPL, m + TAM_EPL);
  uint32_t sb0 = 0u, sb1 = 0u;
#pragma unroll
  for (int i = 0; i < TAM_EPU; ++i) {
    dl[i] = m[i] - a * g[i];  // costate.py:42
    // element 8j+k is bit 7-k of byte j (costate.py:170-181)
    if (i < TAM_EPL) sb0 = 2u * sb0 + (dl[i] < 0.0f ? 1u : 0u);
    else sb1 = 2u * sb1 + (dl[i] < 0.0f ? 1u : 0u);
  }
  const bool odd = (l8 & 1u) != 0;
  const double sd = (double)tam_lane_dot(dl, dl) + (double)tam_lane_dot(dl + TAM_EPL, dl + TAM_EPL);
  const double sm = (double)tam_lane_dot(m, m) + (double)tam_lane_dot(m + TAM_EPL, m + TAM_EPL);
  double x = (odd ? sm : sd) + tam_dppd<TAM_DPP_XOR1>(odd ? sd : sm);
  x = x + tam_dppd<TAM_DPP_XOR2>(x);
  x = x + tam_dppd<TAM_DPP_ROR4>(x);
  const float nx = (float)__builtin_sqrt(x);
  const float ny = tam_dppf<TAM_DPP_XOR1>(nx);
  const float nd = odd ? ny : nx;  // costate.py:241
  const float nm = odd ? nx : ny;
  const float qv = nd / (odd ? nm : d.sqrt_block);  // costate.py:248 / :81-84
  tam_g((uint16_t*)(d.signs + (e0 >> 3)))[0] = (uint16_t)(sb0 | (sb1 << 8));
  if (l8 == 4u) {
    tam_g(d.norms)[b] = nd;
    tam_g(d.amp)[b] = tam_f32_to_f16(qv);
  } else if (l8 == 5u) {
    tam_g(ratios)[d.ratio_off + b] = nm == 0.0f ? 0.0f : qv;
  }
}

// Pass 2 is bound by memory latency rather than by its arithmetic or
// bandwidth, so each wave loads the inputs of its next unit before it computes
// the current one.  Descriptors and the alphas come through scalar loads
// (their indices are wave-uniform): no vector-memory wait then covers the
// loads in flight.  Workgroups of two waves stride over the tiles; wave w takes
// unit 2(tile - tile0) + w.  tam_k2_encode takes the full units of 16-bit
// tensors, tam_k2_encode_f32 those of fp32 tensors (both: without error
// feedback).  The kernel given `quarters` also takes, quarter by quarter
// (tam_k2_any), every other unit of a CoState tensor: error feedback, not
// full, or of the other kernel's dtype when that kernel does not run
// (`other_units` false).
#ifndef TAM_K2_WAVES
#define TAM_K2_WAVES 7
#endif
#ifndef TAM_K2_WAVES_F32
#define TAM_K2_WAVES_F32 6
#endif
template <bool F32>
__device__ __forceinline__ void tam_k2_body(const TamTensor* __restrict__ T, int nT, uint32_t total_tiles,
                                            const float* __restrict__ alpha_new, float* __restrict__ ratios,
                                            char* __restrict__ ws, bool quarters, bool other_units) {
  if (tam_step_skipped(T)) return;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63u;
  const auto desc = [&](int i) -> const TamTensor& { return T[__builtin_amdgcn_readfirstlane(i)]; };
  const auto unit_of = [&](uint32_t tile, int ti) { return (tile - desc(ti).tile0) * 2u + wave; };
  // the next tile at or after `tile` with work for this wave (uniform)
  const auto next = [&](uint32_t& tile, int& ti) -> bool {
    for (; tile < total_tiles; tile += gridDim.x) {
      ti = tam_advance_tensor(T, nT, ti, tile);
      const TamTensor& dd = desc(ti);
      if ((dd.flags & TAM_FLAG_COSTATE) && (quarters || tam_k2u_prefetchable<F32>(dd, unit_of(tile, ti))))
        return true;
    }
    return false;
  };
  uint32_t tile = tam_tile_slot(blockIdx.x, gridDim.x);
  int ti = tam_find_tensor(T, nT, tile < total_tiles ? tile : total_tiles - 1u);
  bool have = next(tile, ti);
  TamK2U<F32> pre = {};
  bool pre_ok = have && tam_k2u_prefetchable<F32>(desc(ti), unit_of(tile, ti));
  if (pre_ok) pre = tam_k2u_load<F32>(desc(ti), unit_of(tile, ti), lane);
  while (have) {
    uint32_t ntile = tile + gridDim.x;
    int nti = ti;
    const bool nhave = next(ntile, nti);
    const TamTensor& d = desc(ti);
    const uint32_t u = unit_of(tile, ti);
    const float a = *(const TAM_CONST float*)(alpha_new + __builtin_amdgcn_readfirstlane(ti));
    TamK2U<F32> npre = {};
    const bool npre_ok = nhave && tam_k2u_prefetchable<F32>(desc(nti), unit_of(ntile, nti));
    if (npre_ok) npre = tam_k2u_load<F32>(desc(nti), unit_of(ntile, nti), lane);
    bool done = pre_ok;
    if constexpr (F32) {
      if (pre_ok) tam_k2_unit<TAM_DTYPE_F32>(d, u, lane, a, ratios, pre);
    } else {
      if (pre_ok && d.dtype == TAM_DTYPE_BF16) tam_k2_unit<TAM_DTYPE_BF16>(d, u, lane, a, ratios, pre);
      else if (pre_ok) tam_k2_unit<TAM_DTYPE_F16>(d, u, lane, a, ratios, pre);
    }
    if (!done && quarters && !(other_units && tam_k2u_prefetchable<!F32>(d, u))) {
      tam_k2_any(d, 2u * u, lane, a, ratios, ws);
      tam_k2_any(d, 2u * u + 1u, lane, a, ratios, ws);
    }
    tile = ntile;
    ti = nti;
    have = nhave;
    pre = npre;
    pre_ok = npre_ok;
  }
}

__global__ __launch_bounds__(TAM_K1U_WG) __attribute__((amdgpu_waves_per_eu(TAM_K2_WAVES, TAM_K2_WAVES))) void
tam_k2_encode(const TamTensor* __restrict__ T, int nT, uint32_t total_tiles, const float* __restrict__ alpha_new,
              float* __restrict__ ratios, char* __restrict__ ws, int quarters, int other_units) {
  tam_k2_body<false>(T, nT, total_tiles, alpha_new, ratios, ws, quarters != 0, other_units != 0);
}

__global__ __launch_bounds__(TAM_K1U_WG) __attribute__((amdgpu_waves_per_eu(TAM_K2_WAVES_F32, TAM_K2_WAVES_F32))) void
tam_k2_encode_f32(const TamTensor* __restrict__ T, int nT, uint32_t total_tiles, const float* __restrict__ alpha_new,
                  float* __restrict__ ratios, char* __restrict__ ws, int quarters, int other_units) {
  tam_k2_body<true>(T, nT, total_tiles, alpha_new, ratios, ws, quarters != 0, other_units != 0);
}

// ---------------------------------------------------------------------------
// Pass 3: order statistics of the ratios (costate.py:114-118), labels
// (costate.py:146-148), alpha write-back (costate.py:443-454)
// ---------------------------------------------------------------------------
// Ratios are >= +0 or NaN, so their fp32 bit patterns order like torch.sort
// (NaN last).  The selection is an MSD radix select on those patterns, spread
// over slices of 8192 keys so that large tensors use many workgroups (the
// state and histogram of each tensor are set by pass 0's tail kernel):
//   tam_k_sel_minmax  per slice: min / max of the keys (atomic min / max per
//                     tensor) -- the bits all keys share need no round, and
//                     the first digit starts at the highest bit that differs,
//                     so keys of similar magnitude spread over its bins
//                     instead of piling into a few (LDS atomics on one bin
//                     serialise);
//   tam_k_sel_hist    per slice, three times: LDS histogram of the next 11-bit
//                     digit below the bits already fixed, for the keys that
//                     match the prefix of each of the two ranks, added into
//                     the tensor's histogram;
//   tam_k_sel_pick    per tensor, after each histogram: prefix sums of the
//                     histogram pick the digit holding each rank; the
//                     histogram is cleared for the next round;
//   tam_k_sel_labels  per slice: labels from the two thresholds; alpha
//                     write-back.
#define TAM_SLICE 8192u

__host__ __device__ __forceinline__ uint32_t tam_sel_slices(uint32_t flags, uint32_t nb) {
  return (flags & TAM_FLAG_COSTATE) ? (nb + TAM_SLICE - 1u) / TAM_SLICE : 0u;
}

// Tensor owning selection slice j: the first whose slice range ends after j.
__device__ __forceinline__ int tam_slice_tensor(const TamTensor* __restrict__ T, int nT, uint32_t j) {
  int lo = 0, hi = nT - 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (T[mid].slice0 + tam_sel_slices(T[mid].flags, T[mid].nb) > j) hi = mid; else lo = mid + 1;
  }
  return lo;
}

// Keys [k0, k1) of a tensor's ratios, visited by the 256 threads of a
// workgroup, 8 keys per thread per round (two 16-byte loads; k0 is a
// multiple of 4 and the ratio array 16-byte aligned).
template <typename F>
__device__ __forceinline__ void tam_slice_keys(const uint32_t* __restrict__ keys, uint32_t k0, uint32_t k1, F&& f) {
  for (uint32_t i = k0 + threadIdx.x * 8u; i < k1; i += TAM_WG * 8u) {
    if (i + 8u <= k1) {
      const TamW4 a = tam_g((const TamW4*)(keys + i))[0], b = tam_g((const TamW4*)(keys + i))[1];
      f(a.x); f(a.y); f(a.z); f(a.w);
      f(b.x); f(b.y); f(b.z); f(b.w);
    } else {
      for (uint32_t j = i; j < k1; ++j) f(tam_g(keys)[j]);
    }
  }
}

// The state a round starts from: before the first round, the bits above the
// highest bit where kmin and kmax differ are shared by every key.
__device__ __forceinline__ TamSel tam_sel_begin(TamSel s) {
  if (s.top == 32) {
    const uint32_t diff = s.kmin ^ s.kmax;
    s.top = diff ? 31 - __builtin_clz(diff) : -1;
    s.mask = s.top >= 31 ? 0u : (0xffffffffu << (s.top + 1));
    s.prefix[0] = s.prefix[1] = s.kmin & s.mask;
  }
  return s;
}

// Digit window below the fixed bits: bits [sh, top].
__device__ __forceinline__ void tam_sel_window(int top, int& sh, uint32_t& dmask) {
  sh = top >= 10 ? top - 10 : 0;
  dmask = (1u << (top - sh + 1)) - 1u;
}

__global__ __launch_bounds__(TAM_WG) void tam_k_sel_minmax(const TamTensor* __restrict__ T, int nT,
                                                           const float* __restrict__ ratios, TamSel* __restrict__ sel) {
  if (tam_step_skipped(T)) return;
  __shared__ uint32_t red[2][TAM_WG / 64];
  const int t = tam_slice_tensor(T, nT, blockIdx.x);
  const TamTensor& d = T[t];
  const uint32_t k0 = (blockIdx.x - d.slice0) * TAM_SLICE;
  const uint32_t k1 = k0 + TAM_SLICE < d.nb ? k0 + TAM_SLICE : d.nb;
  uint32_t kmin = 0xffffffffu, kmax = 0u;
  tam_slice_keys((const uint32_t*)(ratios + d.ratio_off), k0, k1, [&](uint32_t k) {
    kmin = k < kmin ? k : kmin;
    kmax = k > kmax ? k : kmax;
  });
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t a = __shfl_xor(kmin, off), b = __shfl_xor(kmax, off);
    kmin = a < kmin ? a : kmin;
    kmax = b > kmax ? b : kmax;
  }
  if ((threadIdx.x & 63u) == 0) {
    red[0][threadIdx.x >> 6] = kmin;
    red[1][threadIdx.x >> 6] = kmax;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < TAM_WG / 64; ++w) {
      kmin = red[0][w] < kmin ? red[0][w] : kmin;
      kmax = red[1][w] > kmax ? red[1][w] : kmax;
    }
    atomicMin(&sel[t].kmin, kmin);
    atomicMax(&sel[t].kmax, kmax);
  }
}

// Exclusive prefix sum over the TAM_WG threads of the workgroup.
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
  uint32_t before = 0u;
  for (uint32_t i = 0; i < w; ++i) before += wsum[i];
  __syncthreads();  // wsum may be reused once every wave has read it
  return before + inc - v;
}

// One round of the selection (three launches, in order; a tensor whose bits
// are all fixed returns at once).
__global__ __launch_bounds__(TAM_WG) void tam_k_sel_hist(const TamTensor* __restrict__ T, int nT,
                                                         const float* __restrict__ ratios,
                                                         const TamSel* __restrict__ sel, uint32_t* __restrict__ hist) {
  if (tam_step_skipped(T)) return;
  __shared__ uint32_t h[2][2048];
  const int t = tam_slice_tensor(T, nT, blockIdx.x);
  const TamTensor& d = T[t];
  const TamSel st = tam_sel_begin(sel[t]);
  if (st.top < 0) return;  // uniform over the workgroup
  int sh;
  uint32_t dmask;
  tam_sel_window(st.top, sh, dmask);
  for (uint32_t i = threadIdx.x; i < 4096u; i += TAM_WG) (&h[0][0])[i] = 0u;
  __syncthreads();
  const uint32_t p0 = st.prefix[0], p1 = st.prefix[1], mask = st.mask;
  const bool same = p0 == p1;
  const uint32_t k0 = (blockIdx.x - d.slice0) * TAM_SLICE;
  const uint32_t k1 = k0 + TAM_SLICE < d.nb ? k0 + TAM_SLICE : d.nb;
  tam_slice_keys((const uint32_t*)(ratios + d.ratio_off), k0, k1, [&](uint32_t key) {
    const uint32_t dg = (key >> sh) & dmask;
    const uint32_t km = key & mask;
    if (km == p0) atomicAdd(&h[0][dg], 1u);
    if (!same && km == p1) atomicAdd(&h[1][dg], 1u);
  });
  __syncthreads();
  uint32_t* gh = hist + (uint64_t)t * 4096u;
  for (uint32_t i = threadIdx.x; i < 4096u; i += TAM_WG) {
    const uint32_t c = (&h[0][0])[i];
    if (c) atomicAdd(&gh[i], c);
  }
}

// After a round's histogram: the digit holding each of a tensor's two ranks
// (ranks with equal prefixes share the first half of the histogram), the new
// state, and the histogram cleared for the next round.  One workgroup per
// tensor.
__global__ __launch_bounds__(TAM_WG) void tam_k_sel_pick(const TamTensor* __restrict__ T, TamSel* __restrict__ sel,
                                                         uint32_t* __restrict__ hist) {
  if (tam_step_skipped(T)) return;
  if (!(T[blockIdx.x].flags & TAM_FLAG_COSTATE)) return;
  __shared__ uint32_t wsum[TAM_WG / 64];
  __shared__ uint32_t new_prefix[2], new_k[2];
  const TamSel st = tam_sel_begin(sel[blockIdx.x]);
  const uint32_t tid = threadIdx.x;
  if (st.top < 0) {  // every bit fixed (or every key equal): the prefixes are the keys
    if (tid == 0) sel[blockIdx.x] = st;
    return;
  }
  int sh;
  uint32_t dmask;
  tam_sel_window(st.top, sh, dmask);
  uint32_t* gh = hist + (uint64_t)blockIdx.x * 4096u;
  const bool same = st.prefix[0] == st.prefix[1];
  if (tid < 2) {
    new_prefix[tid] = st.prefix[tid];
    new_k[tid] = st.k[tid];
  }
  __syncthreads();
  for (int r = 0; r < 2; ++r) {
    // bins 8 tid .. 8 tid + 7 of rank r's histogram
    const uint32_t* hr = gh + (same ? 0u : (uint32_t)r) * 2048u + 8u * tid;
    const TamW4 a = tam_g((const TamW4*)hr)[0], b = tam_g((const TamW4*)hr)[1];
    const uint32_t c[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t tot = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) tot += c[i];
    uint32_t pre = tam_wg_excl_scan(tot, wsum);
    const uint32_t k = st.k[r];
    if (k >= pre && k - pre < tot) {  // one thread: its bins hold rank k
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (k >= pre && k - pre < c[i]) {
          new_k[r] = k - pre;
          new_prefix[r] = st.prefix[r] | ((8u * tid + (uint32_t)i) << sh);
        }
        pre += c[i];
      }
    }
  }
  __syncthreads();
  for (uint32_t i = tid; i < 4096u; i += TAM_WG) tam_g(gh)[i] = 0u;  // for the next round
  if (tid == 0) {
    TamSel o = st;
    o.prefix[0] = new_prefix[0];
    o.prefix[1] = new_prefix[1];
    o.k[0] = new_k[0];
    o.k[1] = new_k[1];
    o.mask = st.mask | (dmask << sh);
    o.top = sh - 1;
    sel[blockIdx.x] = o;
  }
}

__global__ __launch_bounds__(TAM_WG) void tam_k_sel_labels(const TamTensor* __restrict__ T, int nT,
                                                           const float* __restrict__ alpha_new,
                                                           const float* __restrict__ ratios,
                                                           const TamSel* __restrict__ sel, char* __restrict__ ws,
                                                           float* __restrict__ alpha_old) {
  if (tam_step_skipped(T)) return;
  const int t = tam_slice_tensor(T, nT, blockIdx.x);
  const TamTensor& d = T[t];
  const float tau0 = tam_u2f(sel[t].prefix[0]);
  const float tau1 = tam_u2f(sel[t].prefix[1]);
  const uint32_t k0 = (blockIdx.x - d.slice0) * TAM_SLICE;
  const uint32_t k1 = k0 + TAM_SLICE < d.nb ? k0 + TAM_SLICE : d.nb;
  const float* r = ratios + d.ratio_off;
  const bool ef = (d.flags & TAM_FLAG_EF) != 0;  // error feedback: labels to the staging area
  uint8_t* labels = ef ? tam_stage(d, ws).labels : d.labels;
  for (uint32_t i = k0 + threadIdx.x; i < k1; i += TAM_WG) {
    const float x = tam_g(r)[i];
    tam_g(labels)[i] = x >= tau1 ? (uint8_t)2 : (x >= tau0 ? (uint8_t)1 : (uint8_t)0);
  }
  if (blockIdx.x == d.slice0 && threadIdx.x == 0) {
    if (ef) alpha_old[t] = tam_g(d.alpha)[0];  // pass 4 decodes the previous encoding
    tam_g(d.alpha)[0] = alpha_new[t];
  }
}

// ---------------------------------------------------------------------------
// Pass 4 (tensors with error feedback): costate.py:409-437
// ---------------------------------------------------------------------------
// m is recomputed from the previous encoding exactly as in passes 0 and 2,
// delta = m - alpha*g with the new alpha, and the encoding loss
// ef_error = delta - decode(new encoding, alpha = 0) updates the residual:
// r = ef_error on the tensor's first step, fl(beta1*r) + fl((1-beta1)*ef_error)
// after.  The staged encoding then replaces the previous one.  Each quarter
// reads and writes only its own blocks and sign bytes (the stores follow the
// residual store, which needs every load).
template <uint32_t DT, bool FULL>
__device__ __forceinline__ void tam_k4_quarter(const TamTensor& d, uint32_t wq, uint32_t lane, float a_old,
                                               float a_new, char* __restrict__ ws) {
  const TamWave W = tam_wave(d, wq, lane, FULL);
  if (!(FULL || W.bvalid)) return;  // no cross-lane work below
  const bool has_ef = (d.flags & TAM_FLAG_HAS_EF) != 0;
  const TamStage st = tam_stage(d, ws);
  float g[TAM_EPL], ge[TAM_EPL], m[TAM_EPL], r[TAM_EPL];
  tam_ld8<DT, FULL>(d.grad, W.e0, W.nv, g);
  const TamCsIn cs = tam_cs_load<FULL>(d, W);
  TamCsIn cn;  // the staged new encoding of the lane's block
  cn.label = tam_g(st.labels)[W.b];
  cn.nrm = tam_g(st.norms)[W.b];
  cn.amp = tam_g(st.amp)[W.b];
  cn.byte = (FULL || W.nv > 0) ? tam_g(st.signs)[W.e0 >> 3] : 0u;
  if (has_ef) {
    tam_ld8_f32<FULL>(d.ef_residual, W.e0, W.nv, r);
  } else {
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) r[i] = 0.0f;
  }
  tam_compiler_fence();
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) ge[i] = has_ef ? g[i] + r[i] : g[i];
  tam_costate_m<FULL>(d, W, cs, a_old, g, ge, m);
  const float sph = tam_div_sqrt_block(cn.nrm);
  const float s = cn.label == 1u ? sph : (cn.label == 2u ? tam_f16_to_f32((uint16_t)cn.amp) : 0.0f);
  float rn[TAM_EPL];
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) {
    const float delta = m[i] - a_new * g[i];  // costate.py:42
    const float sd = tam_u2f((tam_f2u(s) & 0x7fffffffu) | ((cn.byte << (24 + i)) & 0x80000000u));
    const float dh = 0.0f * g[i] + sd;        // decode with alpha = 0 (costate.py:428-432)
    const float e = delta - dh;
    rn[i] = has_ef ? d.beta1 * r[i] + d.one_minus_beta1 * e : e;
  }
  tam_st8_f32<FULL>(d.ef_residual, W.e0, W.nv, rn);
  tam_compiler_fence();
  if (W.l16 == 0) {
    tam_g(d.labels)[W.b] = (uint8_t)cn.label;
    tam_g(d.norms)[W.b] = cn.nrm;
    tam_g(d.amp)[W.b] = (uint16_t)cn.amp;
  }
  if (FULL || W.nv > 0) tam_g(d.signs)[W.e0 >> 3] = (uint8_t)cn.byte;
}

__global__ __launch_bounds__(TAM_WG) void tam_k4_ef(const TamTensor* __restrict__ T, int nT, uint32_t total_tiles,
                                                    const float* __restrict__ alpha_new,
                                                    const float* __restrict__ alpha_old, char* __restrict__ ws) {
  if (tam_step_skipped(T)) return;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  int ti = tam_find_tensor(T, nT, blockIdx.x);
  for (uint32_t tile = blockIdx.x; tile < total_tiles; tile += gridDim.x) {
    ti = tam_advance_tensor(T, nT, ti, tile);
    const TamTensor& d = T[ti];
    if (!(d.flags & TAM_FLAG_EF)) continue;  // uniform over the workgroup
    const uint32_t wq = (tile - d.tile0) * 4u + wave;
    const float ao = alpha_old[ti], an = alpha_new[ti];
    const bool full = tam_quarter_full(d, wq);
    switch (d.dtype) {
      case TAM_DTYPE_BF16:
        if (full) tam_k4_quarter<TAM_DTYPE_BF16, true>(d, wq, lane, ao, an, ws);
        else tam_k4_quarter<TAM_DTYPE_BF16, false>(d, wq, lane, ao, an, ws);
        break;
      case TAM_DTYPE_F16:
        if (full) tam_k4_quarter<TAM_DTYPE_F16, true>(d, wq, lane, ao, an, ws);
        else tam_k4_quarter<TAM_DTYPE_F16, false>(d, wq, lane, ao, an, ws);
        break;
      default:
        if (full) tam_k4_quarter<TAM_DTYPE_F32, true>(d, wq, lane, ao, an, ws);
        else tam_k4_quarter<TAM_DTYPE_F32, false>(d, wq, lane, ao, an, ws);
        break;
    }
  }
}

// ---------------------------------------------------------------------------
// standalone helpers (the reference's public functions, one tensor per call)
// ---------------------------------------------------------------------------
// They reuse the step's per-quarter code on a TamTensor built in registers
// (or, for the reductions, one built in the caller's workspace by
// tam_k_make_desc), so their arithmetic is the step's arithmetic.

// Quarter grid for n elements: a 256-thread workgroup covers one tile (four
// quarters); wave w of workgroup t takes quarter 4t + w.
__host__ __device__ __forceinline__ uint32_t tam_tiles_of(uint64_t n) {
  const uint64_t nb = (n + TAM_BLOCK_SIZE - 1) / TAM_BLOCK_SIZE;
  return (uint32_t)((nb + TAM_BPT - 1) / TAM_BPT);
}

__device__ __forceinline__ TamTensor tam_local_desc(uint64_t n) {
  TamTensor d;
  memset(&d, 0, sizeof(d));
  d.n = n;
  d.nb = (uint32_t)((n + TAM_BLOCK_SIZE - 1) / TAM_BLOCK_SIZE);
  d.ntiles = tam_tiles_of(n);
  d.sqrt_block = TAM_SQRT_BLOCK_F;
  return d;
}

// decode_blocks (costate.py:261-324), optionally followed by the EMA of
// CoStateManager.update (costate.py:416): m = fl(b1*m_hat) + fl(ob1*g).
// has_state == 0 gives m_hat = 0 (costate.py:405-407).
__global__ __launch_bounds__(TAM_WG) void tam_k_decode(const uint8_t* __restrict__ labels,
                                                       const uint8_t* __restrict__ signs,
                                                       const float* __restrict__ norms,
                                                       const uint16_t* __restrict__ amp,
                                                       const float* __restrict__ alpha, const void* __restrict__ g,
                                                       uint32_t g_dtype, uint64_t n, int has_state, int ema,
                                                       float beta1, float one_minus_beta1, float* __restrict__ out) {
  TamTensor d = tam_local_desc(n);
  d.labels = (uint8_t*)labels;
  d.signs = (uint8_t*)signs;
  d.norms = (float*)norms;
  d.amp = (uint16_t*)amp;
  d.flags = has_state ? TAM_FLAG_HAS_STATE : 0u;
  d.beta1 = ema ? beta1 : 0.0f;
  d.one_minus_beta1 = ema ? one_minus_beta1 : 0.0f;
  const uint32_t wq = blockIdx.x * 4u + (threadIdx.x >> 6);
  const TamWave W = tam_wave(d, wq, threadIdx.x & 63u, false);
  if (!W.bvalid) return;
  float gv[TAM_EPL], m[TAM_EPL];
  switch (g_dtype) {
    case TAM_DTYPE_BF16: tam_ld8<TAM_DTYPE_BF16, false>(g, W.e0, W.nv, gv); break;
    case TAM_DTYPE_F16: tam_ld8<TAM_DTYPE_F16, false>(g, W.e0, W.nv, gv); break;
    default: tam_ld8<TAM_DTYPE_F32, false>(g, W.e0, W.nv, gv); break;
  }
  const TamCsIn cs = tam_cs_load<false>(d, W);
  const float a = has_state ? alpha[0] : 0.0f;
  if (ema) {
    tam_costate_m<false>(d, W, cs, a, gv, gv, m);
  } else {
    // m_hat alone: fl(alpha*g) + s_b*sign (costate.py:317-323)
    const float sph = tam_div_sqrt_block(cs.nrm);
    const float sb = cs.label == 1u ? sph : (cs.label == 2u ? tam_f16_to_f32((uint16_t)cs.amp) : 0.0f);
#pragma unroll
    for (int i = 0; i < TAM_EPL; ++i) {
      const float sd = tam_u2f((tam_f2u(sb) & 0x7fffffffu) | ((cs.byte << (24 + i)) & 0x80000000u));
      m[i] = has_state ? a * gv[i] + sd : 0.0f;
    }
  }
  tam_st8_f32<false>(out, W.e0, W.nv, m);
}

// Quarter partials of g.g and m.g (fp32 inputs), as pass 1 forms them.
__global__ __launch_bounds__(TAM_WG) void tam_k_dot_quarters(const float* __restrict__ m, const float* __restrict__ g,
                                                             uint64_t n, double2* __restrict__ partials) {
  const TamTensor d = tam_local_desc(n);
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  const uint32_t wq = blockIdx.x * 4u + wave;
  const TamWave W = tam_wave(d, wq, lane, false);
  float mv[TAM_EPL], gv[TAM_EPL];
  tam_ld8<TAM_DTYPE_F32, false>(m, W.e0, W.nv, mv);  // elements past n read 0
  tam_ld8<TAM_DTYPE_F32, false>(g, W.e0, W.nv, gv);
  const double sgg = tam_block_sum((double)tam_lane_dot(gv, gv));
  const double smg = tam_block_sum((double)tam_lane_dot(mv, gv));
  const double tgg = (tam_readlane_d(sgg, 0) + tam_readlane_d(sgg, 16)) +
                     (tam_readlane_d(sgg, 32) + tam_readlane_d(sgg, 48));
  const double tmg = (tam_readlane_d(smg, 0) + tam_readlane_d(smg, 16)) +
                     (tam_readlane_d(smg, 32) + tam_readlane_d(smg, 48));
  if (lane == 0) tam_g((TamD2*)(partials + wq))[0] = TamD2{tgg, tmg};
}

// One CoState descriptor for the alpha and selection kernels.
__global__ void tam_k_make_desc(TamTensor* __restrict__ out, uint64_t n, uint32_t nb, uint32_t k_lo, uint32_t k_hi) {
  TamTensor d = tam_local_desc(n);
  d.nb = nb;
  d.flags = TAM_FLAG_COSTATE;
  d.k_lo = k_lo;
  d.k_hi = k_hi;
  *out = d;
}

// Fresh selection state of the one tensor of desc and its cleared histogram.
__global__ __launch_bounds__(TAM_WG) void tam_k_sel_reset(const TamTensor* __restrict__ desc, TamSel* __restrict__ sel,
                                                          uint32_t* __restrict__ hist) {
  tam_sel_reset_wg(desc[0], sel, hist);
}

// delta = fl(m - fl(alpha*g)) (costate.py:42)
__global__ void tam_k_delta(const float* __restrict__ m, const float* __restrict__ g, uint64_t n,
                            const float* __restrict__ alpha, float* __restrict__ delta) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float a = alpha[0];
  delta[i] = m[i] - a * g[i];
}

// Per-block sum of squares of x (zero padded; fp32 lane partials, fp64
// across the block) in all 16 lanes of the block.
__device__ __forceinline__ double tam_block_sq(const float* x, const TamWave& W) {
  float v[TAM_EPL];
  tam_ld8<TAM_DTYPE_F32, false>(x, W.e0, W.nv, v);
  return tam_block_sum((double)tam_lane_dot(v, v));
}

// compute_block_ratios (costate.py:51-86): r = ||delta_b|| / ||m_b||, 0 where ||m_b|| = 0
__global__ __launch_bounds__(TAM_WG) void tam_k_ratios(const float* __restrict__ delta, const float* __restrict__ m,
                                                       uint64_t n, float* __restrict__ ratios) {
  const TamTensor d = tam_local_desc(n);
  const TamWave W = tam_wave(d, blockIdx.x * 4u + (threadIdx.x >> 6), threadIdx.x & 63u, false);
  const double sd = tam_block_sq(delta, W), sm = tam_block_sq(m, W);
  if (W.bvalid && W.l16 == 0) {
    const float nd = (float)__builtin_sqrt(sd), nm = (float)__builtin_sqrt(sm);
    ratios[W.b] = nm == 0.0f ? 0.0f : nd / nm;
  }
}

// encode_blocks (costate.py:213-258): block norms, fp16 amplitudes, sign bits
__global__ __launch_bounds__(TAM_WG) void tam_k_encode(const float* __restrict__ delta, uint64_t n,
                                                       uint8_t* __restrict__ signs, float* __restrict__ norms,
                                                       uint16_t* __restrict__ amp) {
  const TamTensor d = tam_local_desc(n);
  const TamWave W = tam_wave(d, blockIdx.x * 4u + (threadIdx.x >> 6), threadIdx.x & 63u, false);
  float v[TAM_EPL];
  tam_ld8<TAM_DTYPE_F32, false>(delta, W.e0, W.nv, v);
  uint32_t sbyte = 0;
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i)
    sbyte |= (((uint32_t)i < W.nv && v[i] < 0.0f) ? 1u : 0u) << (7 - i);  // costate.py:170-181
  const double sd = tam_block_sum((double)tam_lane_dot(v, v));
  if (!W.bvalid) return;
  if (W.nv > 0) signs[W.e0 >> 3] = (uint8_t)sbyte;
  if (W.l16 == 0) {
    const float nd = (float)__builtin_sqrt(sd);
    norms[W.b] = nd;
    amp[W.b] = tam_f32_to_f16(tam_div_sqrt_block(nd));
  }
}

// classify_blocks (costate.py:126-149), thresholds read from taus[0], taus[1]
__global__ void tam_k_classify(const float* __restrict__ ratios, uint64_t nb, const float* __restrict__ taus,
                               uint8_t* __restrict__ labels) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nb) return;
  const float x = ratios[i], tau0 = taus[0], tau1 = taus[1];
  labels[i] = x >= tau1 ? (uint8_t)2 : (x >= tau0 ? (uint8_t)1 : (uint8_t)0);
}

// The two thresholds of a finished selection.
__global__ void tam_k_sel_taus(const TamSel* __restrict__ sel, float* __restrict__ taus) {
  taus[0] = tam_u2f(sel[0].prefix[0]);
  taus[1] = tam_u2f(sel[0].prefix[1]);
}

// fused_v_update (quantize.py:222-299) for one tensor: the 1Q half of pass 1
// without the first moment and the parameter update; v (fp32, n values) is
// written out.  idx_out / scales_out may equal idx_in / scales_in.
__global__ __launch_bounds__(TAM_WG) void tam_k_fused_v(const uint8_t* idx_in, const uint16_t* scales_in,
                                                        const void* __restrict__ g, uint32_t g_dtype, uint64_t n,
                                                        uint32_t bits, float beta2, float one_minus_beta2,
                                                        uint32_t tensor_id, uint32_t step, uint32_t seed_lo,
                                                        uint32_t seed_hi, uint8_t* idx_out, uint16_t* scales_out,
                                                        float* __restrict__ v_out) {
  __shared__ float lut[TAM_WG / 64][4 * 64];
  __shared__ TamLdsTabs tabs;
  tam_lds_tabs_fill(&tabs);
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  TamTensor d = tam_local_desc(n);
  d.v_idx = (uint8_t*)idx_in;
  d.v_scales = (uint16_t*)scales_in;
  d.v_bits = bits;
  d.beta2 = beta2;
  d.one_minus_beta2 = one_minus_beta2;
  d.tensor_id = tensor_id;
  d.step = step;
  const TamWave W = tam_wave(d, blockIdx.x * 4u + wave, lane, false);
  float gv[TAM_EPL], v[TAM_EPL], vc[TAM_EPL];
  switch (g_dtype) {
    case TAM_DTYPE_BF16: tam_ld8<TAM_DTYPE_BF16, false>(g, W.e0, W.nv, gv); break;
    case TAM_DTYPE_F16: tam_ld8<TAM_DTYPE_F16, false>(g, W.e0, W.nv, gv); break;
    default: tam_ld8<TAM_DTYPE_F32, false>(g, W.e0, W.nv, gv); break;
  }
  const TamVIn vin = tam_v_load<false>(d, W);
  const TamVExt x = tam_vpath_a<false>(d, W, vin, gv, v, vc, lut[wave], &tabs);
  if (W.bvalid) tam_st8_f32<false>(v_out, W.e0, W.nv, v);
  d.v_idx = idx_out;
  d.v_scales = scales_out;
  tam_vpath_b<false>(d, W, vc, x, &tabs, seed_lo, seed_hi);
}

// quantize_logscale_nbits (quantize.py:126-180) of a padded positive tensor:
// per-block fp16 (log_min, log_max) over all of the block's values, and
// indices trunc(clamp(c, 0, 2^bits - 0.001)) (deterministic) or
// floor(c) + (u < frac(c)) clamped (stochastic, Philox draws as in the step),
// c = fl(fl(log v - log_min) / max(span, 1e-10)) * 2^bits.
__global__ __launch_bounds__(TAM_WG) void tam_k_quantize(const float* __restrict__ v, uint64_t npad, uint32_t bits,
                                                         int stochastic, uint32_t tensor_id, uint32_t step,
                                                         uint32_t seed_lo, uint32_t seed_hi,
                                                         uint8_t* __restrict__ idx, uint16_t* __restrict__ scales) {
  __shared__ TamLdsTabs tabs;
  tam_lds_tabs_fill(&tabs);
  const TamTensor d = tam_local_desc(npad);
  const TamWave W = tam_wave(d, blockIdx.x * 4u + (threadIdx.x >> 6), threadIdx.x & 63u, false);
  const float fnb = (float)(1u << bits);
  float x[TAM_EPL], l[TAM_EPL];
  tam_ld8<TAM_DTYPE_F32, false>(v, W.e0, W.nv, x);
  float lmn = tam_inf(), lmx = -tam_inf();
  uint32_t nan_seen = 0;
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) {
    const float c = x[i] < 1e-38f ? 1e-38f : x[i];  // clamp(min=1e-38), NaN stays
    l[i] = tam_logf_lds(c, &tabs);
    if ((uint32_t)i < W.nv) {
      nan_seen |= tam_isnan(l[i]) ? 1u : 0u;
      lmn = __builtin_fminf(lmn, l[i]);
      lmx = __builtin_fmaxf(lmx, l[i]);
    }
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) {  // block min / max over the 16 lanes (minNum / maxNum; NaN tracked apart)
    const float a = s == 0 ? tam_dppf<TAM_DPP_XOR1>(lmn) : s == 1 ? tam_dppf<TAM_DPP_XOR2>(lmn)
                  : s == 2 ? tam_dppf<TAM_DPP_HALF_MIRROR>(lmn) : tam_dppf<TAM_DPP_MIRROR>(lmn);
    const float b = s == 0 ? tam_dppf<TAM_DPP_XOR1>(lmx) : s == 1 ? tam_dppf<TAM_DPP_XOR2>(lmx)
                  : s == 2 ? tam_dppf<TAM_DPP_HALF_MIRROR>(lmx) : tam_dppf<TAM_DPP_MIRROR>(lmx);
    lmn = __builtin_fminf(lmn, a);
    lmx = __builtin_fmaxf(lmx, b);
  }
  nan_seen = tam_block_or(nan_seen);
  if (nan_seen) lmn = lmx = tam_qnan();
  if (!W.bvalid) return;
  if (W.l16 == 0)
    tam_g((uint32_t*)scales)[W.b] = (uint32_t)tam_f32_to_f16(lmn) | ((uint32_t)tam_f32_to_f16(lmx) << 16);
  float sp = lmx - lmn;
  sp = sp < 1e-10f ? 1e-10f : sp;
  uint32_t rw[TAM_EPL] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  if (stochastic) {
    tam_draws8(W.e0, tensor_id, step, seed_lo, seed_hi, rw);
  }
  const float top = fnb - 0.001f;  // f32(2^bits - 0.001)
#pragma unroll
  for (int i = 0; i < TAM_EPL; ++i) {
    const float c = ((l[i] - lmn) / sp) * fnb;
    float q;
    if (stochastic) {
      const float f = __builtin_floorf(c);
      const float u = (float)rw[i] * 0x1p-24f;
      q = f + (u < c - f ? 1.0f : 0.0f);
      q = q < 0.0f ? 0.0f : q;
      q = q > fnb - 1.0f ? fnb - 1.0f : q;
    } else {
      q = c < 0.0f ? 0.0f : c;
      q = q > top ? top : q;
    }
    if ((uint32_t)i < W.nv) idx[W.e0 + i] = tam_isnan(q) ? (uint8_t)0 : (uint8_t)(uint32_t)q;
  }
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

// One thread per 8 elements (half a group of draws).
__global__ void tam_k_philox_uniforms(uint32_t tid, uint32_t step, uint32_t seed_lo, uint32_t seed_hi,
                                      uint64_t count, float* __restrict__ out) {
  const uint64_t e0 = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8u;
  if (e0 >= count) return;
  uint32_t rw[8];
  tam_draws8(e0, tid, step, seed_lo, seed_hi, rw);
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (e0 + k < count) out[e0 + k] = tam_u24f(rw[k]);
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
    case 6: y = __builtin_amdgcn_sqrtf(x); break;
    case 7: y = __builtin_amdgcn_rcpf(x); break;
    case 8: y = __builtin_amdgcn_logf(x); break;
    default: y = x; break;
  }
  out[i] = y;
}

// ---------------------------------------------------------------------------
// host entry points
// ---------------------------------------------------------------------------
// Per-device launch figures, computed once (threads that race store the same value).
static int tam_device_cus(void) {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cus[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cus[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

static uint64_t tam_align_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

// Bytes of an error-feedback tensor's staged encoding in the workspace:
// norms f32[nb] at 0, amplitudes f16[nb] at 4nb, labels u8[nb] at 6nb, sign
// bytes u8[ceil(n/8)] at 7nb.
static uint64_t tam_ef_stage_bytes(uint64_t n, uint64_t nb) { return 7u * nb + (n + 7) / 8; }

// Whether decoupled weight decay leaves every 16-bit parameter unchanged:
// R_p(fl(x * c)) == x for every bf16 x when 1 - 2^-10 <= c <= 1 (fp16: 1 -
// 2^-13), c = f32(1 - lr * wd) (optimizer.py:106-107 on a 16-bit tensor).
// For x > 0 (x < 0 is symmetric; 0 and inf map to themselves, a NaN stays a
// NaN that the update then propagates): fl is monotone and x is an fp32
// value, so x (1 - d)(1 - 2^-24) - 2^-150 <= fl(x c) <= x with d = 1 - c.
// The predecessor of a normal x is at least x 2^-8 below it for bf16 (2^-11
// for fp16), and R_p returns x for anything above the midpoint x (1 - 2^-9)
// (fp16: x (1 - 2^-12)), which (1 - 2^-10)(1 - 2^-24) x - 2^-150 exceeds.
// Subnormal x = k 2^-133 (bf16, k < 128; fp16 k 2^-24, k < 1024) moves by less
// than k d x-units + 2^-150 < half their spacing.  tests/test_oracle_pins.py
// checks the claim on every 16-bit pattern at the bounds.  The kernels then
// skip the product and its rounding.
static bool tam_wd_keeps_16bit(uint32_t dtype, float c_wd) {
  if (dtype == TAM_DTYPE_BF16) return c_wd <= 1.0f && c_wd >= 1.0f - 0x1p-10f;
  if (dtype == TAM_DTYPE_F16) return c_wd <= 1.0f && c_wd >= 1.0f - 0x1p-13f;
  return false;
}

// Workgroups of a kernel that fit on the device at once (CUs times the
// occupancy its registers and LDS allow), cached per device and kernel.  The
// tile loops launch TAM_GRID_ROUNDS times that many workgroups, pass 2
// TAM_K2_GRID_ROUNDS times.  Measured on MI355X (Llama-shaped bf16 set): pass 0
// is 14% faster with 32 rounds than with one resident round of persistent
// workgroups (8 rounds: 1% slower than 32); pass 2, which loads each quarter
// one ahead, is fastest with 8 rounds (7% faster than 32, 15% than 1).
enum { TAM_KS_K1_BF16, TAM_KS_K1_F16, TAM_KS_K1_F32, TAM_KS_K2, TAM_KS_K2_F32, TAM_KS_K1_EF, TAM_KS_K4_EF,
       TAM_KS_COUNT };
#ifndef TAM_K2_GRID_ROUNDS
#define TAM_K2_GRID_ROUNDS 8
#endif
#ifndef TAM_GRID_ROUNDS
#define TAM_GRID_ROUNDS 32
#endif
static uint32_t tam_resident_grid(int which, const void* kernel, int block) {
  static std::atomic<uint32_t> cache[64][TAM_KS_COUNT];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  uint32_t g = cache[dev][which].load(std::memory_order_relaxed);
  if (g == 0) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, 0) != hipSuccess || per_cu <= 0)
      per_cu = 4;
    g = (uint32_t)(per_cu * tam_device_cus());
    cache[dev][which].store(g, std::memory_order_relaxed);
  }
  return g;
}

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
  uint64_t tiles = 0, ratio_blocks = 0, chunks = 0, slices = 0, ef_bytes = 0, tail_blocks = 0;
  uint32_t dtype_mask = 0;
  uint32_t ncs = 0, nef = 0, ndev = 0;
  for (int i = 0; i < n_tensors; ++i) {
    TamTensor& t = tensors[i];
    if (t.n == 0) return tam_fail(TAM_E_INVALID, "%stensor %ld has no elements", "", i);
    if (t.dtype > TAM_DTYPE_F16) return tam_fail(TAM_E_INVALID, "%stensor %ld: unknown dtype", "", i);
    if (t.sqrt_block != TAM_SQRT_BLOCK_F)
      return tam_fail(TAM_E_INVALID, "%stensor %ld: sqrt_block must be f32(sqrt(128))", "", i);
    if (!t.param || !t.grad) return tam_fail(TAM_E_INVALID, "%stensor %ld: null param/grad", "", i);
    if (t.flags & TAM_FLAG_DEVICE_STEP) {
      if (!t.step_dev || !t.bc_step || !t.bc_table || t.bc_len == 0)
        return tam_fail(TAM_E_INVALID, "%stensor %ld: device step counters or table missing", "", i);
      ++ndev;
    }
    if (t.found_inf != tensors[0].found_inf || (t.found_inf && !(t.flags & TAM_FLAG_DEVICE_STEP)))
      return tam_fail(TAM_E_INVALID, "%stensor %ld: found_inf needs DEVICE_STEP and one pointer for all", "", i);
    t.flags &= ~TAM_FLAG_SKIP;
    const uint64_t nb = (t.n + TAM_BLOCK_SIZE - 1) / TAM_BLOCK_SIZE;
    if (nb > (1ull << 31)) return tam_fail(TAM_E_INVALID, "%stensor %ld too large", "", i);
    const uint64_t nt = (nb + TAM_BPT - 1) / TAM_BPT;
    if (nt > (1ull << 22)) return tam_fail(TAM_E_INVALID, "%stensor %ld too large", "", i);
    if (t.flags & TAM_FLAG_COMPRESS_V) {
      if (!(t.v_bits == 2 || t.v_bits == 3 || t.v_bits == 4 || t.v_bits == 6 || t.v_bits == 8))
        return tam_fail(TAM_E_INVALID, "%stensor %ld: v_bits must be 2, 3, 4, 6 or 8", "", i);
      if (!t.v_idx || !t.v_scales) return tam_fail(TAM_E_INVALID, "%stensor %ld: null v state", "", i);
      // 16-byte index loads and stores of a unit's 16 elements per lane; one
      // 32-bit (lmin, lmax) word per block
      if (((uintptr_t)t.v_idx & 15u) || ((uintptr_t)t.v_scales & 3u))
        return tam_fail(TAM_E_INVALID, "%stensor %ld: misaligned v state", "", i);
    } else if (!t.exp_avg_sq || ((uintptr_t)t.exp_avg_sq & 15u)) {
      return tam_fail(TAM_E_INVALID, "%stensor %ld: exp_avg_sq null or misaligned", "", i);
    }
    if (t.flags & TAM_FLAG_COSTATE) {
      if (!t.signs || !t.labels || !t.norms || !t.amp || !t.alpha)
        return tam_fail(TAM_E_INVALID, "%stensor %ld: null CoState state", "", i);
      // 16-bit sign loads and stores (a lane's 16 elements), f32 norms and
      // alpha, f16 amplitudes
      if (((uintptr_t)t.signs & 1u) || ((uintptr_t)t.norms & 3u) || ((uintptr_t)t.amp & 1u) ||
          ((uintptr_t)t.alpha & 3u))
        return tam_fail(TAM_E_INVALID, "%stensor %ld: misaligned CoState state", "", i);
      if (t.k_lo >= nb || t.k_hi >= nb) return tam_fail(TAM_E_INVALID, "%stensor %ld: rank out of range", "", i);
      t.ratio_off = ratio_blocks;
      ratio_blocks += (nb + 3) & ~3ull;  // 16-byte aligned per tensor
      ++ncs;
      if (t.flags & TAM_FLAG_EF) {
        if (!t.ef_residual || ((uintptr_t)t.ef_residual & 15u))
          return tam_fail(TAM_E_INVALID, "%stensor %ld: ef_residual null or misaligned", "", i);
        t.ef_off = ef_bytes;  // relative until the workspace layout is known
        ef_bytes += tam_align_up(tam_ef_stage_bytes(t.n, nb), 256);
        ++nef;
      }
    } else if (!t.exp_avg || ((uintptr_t)t.exp_avg & 15u)) {
      return tam_fail(TAM_E_INVALID, "%stensor %ld: exp_avg null or misaligned", "", i);
    } else if (t.flags & (TAM_FLAG_EF | TAM_FLAG_HAS_EF)) {
      return tam_fail(TAM_E_INVALID, "%stensor %ld: error feedback needs CoState", "", i);
    }
    if ((t.flags & TAM_FLAG_WD) && tam_wd_keeps_16bit(t.dtype, t.c_wd)) t.flags &= ~TAM_FLAG_WD;
    t.nb = (uint32_t)nb;
    t.ntiles = (uint32_t)nt;
    t.tile0 = (uint32_t)tiles;
    const bool aligned = (((uintptr_t)t.param | (uintptr_t)t.grad) & 15u) == 0;
    t.tail0 = (uint32_t)tail_blocks;
    t.tail_wgs = (aligned || (t.flags & TAM_FLAG_EF)) ? 1u : (uint32_t)((nt + TAM_TAIL_TILES - 1) / TAM_TAIL_TILES);
    tail_blocks += t.tail_wgs;
    if (!(t.flags & TAM_FLAG_EF)) dtype_mask |= 1u << t.dtype;  // pass 0's per-dtype kernels skip EF tensors
    t.chunk0 = (uint32_t)chunks;
    t.slice0 = (uint32_t)slices;
    t.c_lr = t.neg_lr / t.bias_correction1;  // fp32 division, correctly rounded
    t.k_abs = tam_abs_term(t.bias_correction1, t.eps);
    tiles += nt;
    chunks += tam_alpha_chunks(t.flags, t.ntiles);
    slices += tam_sel_slices(t.flags, t.nb);
    // below 2^31, so that a tile index plus a grid stride cannot wrap
    if (tiles > (1ull << 31)) return tam_fail(TAM_E_INVALID, "%stoo many tiles", "", 0);
  }
  memset(info, 0, sizeof(*info));
  info->n_tensors = n_tensors;
  info->tail_blocks = (uint32_t)tail_blocks;
  info->total_tiles = (uint32_t)tiles;
  info->n_costate = ncs;
  info->total_chunks = (uint32_t)chunks;
  info->total_slices = (uint32_t)slices;
  info->dtype_mask = dtype_mask;
  info->ratio_blocks = ratio_blocks;
  uint64_t off = 0;
  info->off_partials = off;
  off = tam_align_up(off + tiles * 4u * sizeof(double2), 256);  // one partial per quarter tile
  info->off_alpha = off;
  off = tam_align_up(off + (uint64_t)n_tensors * sizeof(float), 256);
  info->off_ratios = off;
  off = tam_align_up(off + ratio_blocks * sizeof(float), 256);
  info->off_chunks = off;
  off = tam_align_up(off + chunks * sizeof(double2), 256);
  info->off_sel = off;
  off = tam_align_up(off + (uint64_t)n_tensors * sizeof(TamSel), 256);
  info->off_hist = off;
  off = tam_align_up(off + (uint64_t)n_tensors * 4096u * sizeof(uint32_t), 256);
  info->n_ef = nef;
  info->n_device_step = ndev;
  info->off_ef_alpha = off;
  off = tam_align_up(off + (uint64_t)n_tensors * sizeof(float), 256);
  for (int i = 0; i < n_tensors; ++i)
    if (tensors[i].flags & TAM_FLAG_EF) tensors[i].ef_off += off;
  off += ef_bytes;
  info->ws_bytes = off;
  return TAM_OK;
}

static int tam_launch_pass(int pass, const TamTensor* d_tensors, const TamStepInfo* info, uint64_t seed,
                           void* workspace, size_t ws_bytes, hipStream_t s) {
  if (!info || (info->n_tensors > 0 && !d_tensors)) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (pass < 0 || pass > 4) return tam_fail(TAM_E_INVALID, "%sunknown pass %ld", "", pass);
  if (info->n_tensors == 0 || info->total_tiles == 0) return TAM_OK;
  if (!workspace || ws_bytes < info->ws_bytes)
    return tam_fail(TAM_E_WORKSPACE, "%sworkspace too small: need %ld bytes", "", (long)info->ws_bytes);
  if (pass > 0 && info->n_costate == 0) return TAM_OK;
  if (pass == 4 && info->n_ef == 0) return TAM_OK;
  char* ws = (char*)workspace;
  double2* partials = (double2*)(ws + info->off_partials);
  float* alpha_new = (float*)(ws + info->off_alpha);
  float* ratios = (float*)(ws + info->off_ratios);
  double2* chunk_sums = (double2*)(ws + info->off_chunks);
  TamSel* sel = (TamSel*)(ws + info->off_sel);
  uint32_t* hist = (uint32_t*)(ws + info->off_hist);
  float* alpha_old = (float*)(ws + info->off_ef_alpha);
  // vwg: virtual workgroups (each striding over the tiles on its own) per workgroup
  auto grid_of = [&](int which, const void* kernel, int block = TAM_WG, uint32_t vwg = 1u) {
    const uint32_t rounds = (which == TAM_KS_K2 || which == TAM_KS_K2_F32) ? TAM_K2_GRID_ROUNDS : TAM_GRID_ROUNDS;
    const uint32_t g = tam_resident_grid(which, kernel, block) * rounds;
    const uint32_t need = (info->total_tiles + vwg - 1u) / vwg;
    return need < g ? need : g;
  };
  switch (pass) {
    case 0:
      if (info->n_device_step) {  // the descriptors of DEVICE_STEP tensors are completed on the device
        hipLaunchKernelGGL(tam_k_device_step, dim3(1), dim3(1024), 0, s, (TamTensor*)d_tensors, info->n_tensors);
        TAM_HIP_CHECK(hipGetLastError());
      }
      if (info->dtype_mask & (1u << TAM_DTYPE_BF16))
        hipLaunchKernelGGL(tam_k1_main_bf16,
                           dim3(grid_of(TAM_KS_K1_BF16, (const void*)tam_k1_main_bf16, TAM_K1_BLOCK, TAM_K1_VWG)),
                           dim3(TAM_K1_BLOCK), 0, s, d_tensors, info->n_tensors, info->total_tiles, (uint32_t)seed,
                           (uint32_t)(seed >> 32), partials);
      if (info->dtype_mask & (1u << TAM_DTYPE_F16))
        hipLaunchKernelGGL(tam_k1_main_f16,
                           dim3(grid_of(TAM_KS_K1_F16, (const void*)tam_k1_main_f16, TAM_K1_BLOCK, TAM_K1_VWG)),
                           dim3(TAM_K1_BLOCK), 0, s, d_tensors, info->n_tensors, info->total_tiles, (uint32_t)seed,
                           (uint32_t)(seed >> 32), partials);
      if (info->dtype_mask & (1u << TAM_DTYPE_F32))
        hipLaunchKernelGGL(tam_k1_main_f32,
                           dim3(grid_of(TAM_KS_K1_F32, (const void*)tam_k1_main_f32, TAM_K1_BLOCK, TAM_K1_VWG)),
                           dim3(TAM_K1_BLOCK), 0, s, d_tensors, info->n_tensors, info->total_tiles, (uint32_t)seed,
                           (uint32_t)(seed >> 32), partials);
      if (info->n_ef)
        hipLaunchKernelGGL(tam_k1_ef, dim3(grid_of(TAM_KS_K1_EF, (const void*)tam_k1_ef)), dim3(TAM_WG), 0, s,
                           d_tensors, info->n_tensors, info->total_tiles, (uint32_t)seed, (uint32_t)(seed >> 32),
                           partials);
      TAM_HIP_CHECK(hipGetLastError());
      hipLaunchKernelGGL(tam_k1_tail, dim3(info->tail_blocks), dim3(TAM_WG), 0, s, d_tensors, info->n_tensors,
                         (uint32_t)seed, (uint32_t)(seed >> 32), partials, sel, hist);
      break;
    case 1:
      hipLaunchKernelGGL(tam_k_alpha_chunks, dim3(info->total_chunks), dim3(TAM_WG), 0, s, d_tensors,
                         info->n_tensors, partials, chunk_sums);
      TAM_HIP_CHECK(hipGetLastError());
      hipLaunchKernelGGL(tam_k_alpha, dim3(info->n_tensors), dim3(TAM_WG), 0, s, d_tensors, chunk_sums, alpha_new);
      break;
    case 2: {
      // full units by dtype class; the other units' quarters go to the 16-bit
      // kernel when it runs, else to the fp32 one
      const bool has16 = (info->dtype_mask & ((1u << TAM_DTYPE_BF16) | (1u << TAM_DTYPE_F16))) != 0;
      const bool has32 = (info->dtype_mask & (1u << TAM_DTYPE_F32)) != 0;
      if (has16 || !has32)
        hipLaunchKernelGGL(tam_k2_encode, dim3(grid_of(TAM_KS_K2, (const void*)tam_k2_encode, TAM_K1U_WG)),
                           dim3(TAM_K1U_WG), 0, s, d_tensors, info->n_tensors, info->total_tiles, alpha_new, ratios,
                           ws, 1, has32 ? 1 : 0);
      if (has32) {
        TAM_HIP_CHECK(hipGetLastError());
        hipLaunchKernelGGL(tam_k2_encode_f32,
                           dim3(grid_of(TAM_KS_K2_F32, (const void*)tam_k2_encode_f32, TAM_K1U_WG)),
                           dim3(TAM_K1U_WG), 0, s, d_tensors, info->n_tensors, info->total_tiles, alpha_new, ratios,
                           ws, has16 ? 0 : 1, 0);
      }
      break;
    }
    default:
      // the state and histograms were set by pass 0's tail kernel
      hipLaunchKernelGGL(tam_k_sel_minmax, dim3(info->total_slices), dim3(TAM_WG), 0, s, d_tensors,
                         info->n_tensors, ratios, sel);
      TAM_HIP_CHECK(hipGetLastError());
      for (int r = 0; r < 3; ++r) {  // 11-bit digits: at most three rounds fix all 32 bits
        hipLaunchKernelGGL(tam_k_sel_hist, dim3(info->total_slices), dim3(TAM_WG), 0, s, d_tensors,
                           info->n_tensors, ratios, sel, hist);
        TAM_HIP_CHECK(hipGetLastError());
        hipLaunchKernelGGL(tam_k_sel_pick, dim3(info->n_tensors), dim3(TAM_WG), 0, s, d_tensors, sel, hist);
        TAM_HIP_CHECK(hipGetLastError());
      }
      hipLaunchKernelGGL(tam_k_sel_labels, dim3(info->total_slices), dim3(TAM_WG), 0, s, d_tensors,
                         info->n_tensors, alpha_new, ratios, sel, ws, alpha_old);
      break;
    case 4:
      hipLaunchKernelGGL(tam_k4_ef, dim3(grid_of(TAM_KS_K4_EF, (const void*)tam_k4_ef)), dim3(TAM_WG), 0, s, d_tensors,
                         info->n_tensors, info->total_tiles, alpha_new, alpha_old, ws);
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
  for (int pass = 0; pass < 5; ++pass) {  // pass 4 runs only with error feedback
    const int rc = tam_launch_pass(pass, d_tensors, info, seed, workspace, ws_bytes, (hipStream_t)stream);
    if (rc != TAM_OK) return rc;
  }
  return TAM_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// the step without a caller workspace (tam_multi_tensor_step_static)
// ---------------------------------------------------------------------------
// Its workspace is this file-scope device array: every GPU that loads the
// library holds one copy of TAM_STATIC_SCRATCH_BYTES until the process ends.
// Host code never passes `scratch` itself (in host code the name is only a
// stand-in for the symbol); it passes the device address that
// hipGetSymbolAddress returns for the current device, looked up once per
// device on that device's first call and kept in tam_scratch_dev.  Nothing in
// the array must start at zero: pass 0 writes every partial that pass 1
// reads, pass 2 every ratio that pass 3 reads, and pass 3 resets its own
// selection state and histograms first.  Every call on one GPU uses that
// GPU's one array, so calls that overlap on one GPU (on streams not ordered
// with each other) race.
static __device__ __align__(256) char scratch[TAM_STATIC_SCRATCH_BYTES];

static std::atomic<void*> tam_scratch_dev[64];

// Device address of the current device's copy of `scratch`.
static int tam_scratch_ptr(void** out) {
  int dev = -1;
  TAM_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return tam_fail(TAM_E_UNSUPPORTED, "%sdevice index %ld out of range", "", dev);
  void* p = tam_scratch_dev[dev].load(std::memory_order_acquire);
  if (p == nullptr) {  // threads that race look up and store the same address
    TAM_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (p == nullptr) return tam_fail(TAM_E_HIP, "%sno device address for the static scratch", "");
    tam_scratch_dev[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return TAM_OK;
}

extern "C" {

int tam_multi_tensor_step_static(const TamTensor* d_tensors, const TamTensor* h_tensors, const TamStepInfo* info,
                                 uint64_t seed, void* stream) {
  tam_err_buf[0] = 0;
  (void)h_tensors;
  if (!info) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (info->ws_bytes > TAM_STATIC_SCRATCH_BYTES)
    return tam_fail(TAM_E_WORKSPACE, "%sstep needs %ld bytes of workspace, above the static scratch of 64 MiB "
                    "(use tam_multi_tensor_step with a workspace)", "", (long)info->ws_bytes);
  if (info->n_tensors == 0 || info->total_tiles == 0) return TAM_OK;
  void* ws = nullptr;
  const int rc0 = tam_scratch_ptr(&ws);
  if (rc0 != TAM_OK) return rc0;
  for (int pass = 0; pass < 5; ++pass) {
    const int rc = tam_launch_pass(pass, d_tensors, info, seed, ws, TAM_STATIC_SCRATCH_BYTES, (hipStream_t)stream);
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
  const uint64_t eights = (count + 7) / 8;
  const uint64_t blocks = (eights + 255) / 256;
  hipLaunchKernelGGL(tam_k_philox_uniforms, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream,
                     tensor_id, step, (uint32_t)seed, (uint32_t)(seed >> 32), count, out);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

int tam_math_eval(int fn, const float* in, float* out, uint64_t n, void* stream) {
  tam_err_buf[0] = 0;
  if (!in || !out) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (fn < 0 || fn > 8) return tam_fail(TAM_E_INVALID, "%sunknown function %ld", "", fn);
  if (n == 0) return TAM_OK;
  const uint64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(tam_k_math_eval, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream, fn, in, out, n);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}


// ---------------------------------------------------------------------------
// standalone helpers: host side
// ---------------------------------------------------------------------------
static int tam_check_dtype(uint32_t dt) {
  return dt <= TAM_DTYPE_F16 ? TAM_OK : tam_fail(TAM_E_INVALID, "%sunknown dtype %ld", "", (long)dt);
}

int tam_costate_decode(const uint8_t* labels, const uint8_t* signs, const float* norms, const uint16_t* amp,
                       const float* alpha, const void* g, uint32_t g_dtype, uint64_t n, int has_state, int ema,
                       float beta1, float one_minus_beta1, float* m_out, void* stream) {
  tam_err_buf[0] = 0;
  if (!g || !m_out || (has_state && (!labels || !signs || !norms || !amp || !alpha)))
    return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (((uintptr_t)norms | (uintptr_t)alpha) & 3u || (uintptr_t)amp & 1u)
    return tam_fail(TAM_E_INVALID, "%smisaligned CoState state", "");
  if (tam_check_dtype(g_dtype)) return TAM_E_INVALID;
  if (n == 0) return TAM_OK;
  hipLaunchKernelGGL(tam_k_decode, dim3(tam_tiles_of(n)), dim3(TAM_WG), 0, (hipStream_t)stream, labels, signs, norms,
                     amp, alpha, g, g_dtype, n, has_state, ema, beta1, one_minus_beta1, m_out);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

static uint64_t tam_decompose_layout(uint64_t n, uint64_t* off_part, uint64_t* off_chunks, uint64_t* off_alpha) {
  const uint64_t nt = tam_tiles_of(n);
  const uint32_t nch = tam_alpha_chunks(TAM_FLAG_COSTATE, (uint32_t)nt);
  uint64_t off = tam_align_up(sizeof(TamTensor), 256);
  *off_part = off;
  off = tam_align_up(off + nt * 4u * sizeof(double2), 256);
  *off_chunks = off;
  off = tam_align_up(off + (uint64_t)nch * sizeof(double2), 256);
  *off_alpha = off;
  return tam_align_up(off + sizeof(float), 256);
}

size_t tam_decompose_workspace(uint64_t n) {
  uint64_t a, b, c;
  return (size_t)tam_decompose_layout(n, &a, &b, &c);
}

int tam_decompose(const float* m, const float* g, uint64_t n, float* alpha, float* delta, void* workspace,
                  size_t ws_bytes, void* stream) {
  tam_err_buf[0] = 0;
  if (!m || !g || !alpha || !delta || !workspace) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (n == 0 || (n + TAM_BLOCK_SIZE - 1) / TAM_BLOCK_SIZE > (1ull << 31))
    return tam_fail(TAM_E_INVALID, "%selement count out of range", "");
  uint64_t off_part, off_chunks, off_alpha;
  const uint64_t need = tam_decompose_layout(n, &off_part, &off_chunks, &off_alpha);
  if (ws_bytes < need) return tam_fail(TAM_E_WORKSPACE, "%sworkspace too small: need %ld bytes", "", (long)need);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  TamTensor* desc = (TamTensor*)ws;
  const uint32_t nt = tam_tiles_of(n);
  const uint32_t nb = (uint32_t)((n + TAM_BLOCK_SIZE - 1) / TAM_BLOCK_SIZE);
  hipLaunchKernelGGL(tam_k_make_desc, dim3(1), dim3(1), 0, s, desc, n, nb, 0u, 0u);
  TAM_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(tam_k_dot_quarters, dim3(nt), dim3(TAM_WG), 0, s, m, g, n, (double2*)(ws + off_part));
  TAM_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(tam_k_alpha_chunks, dim3(tam_alpha_chunks(TAM_FLAG_COSTATE, nt)), dim3(TAM_WG), 0, s, desc, 1,
                     (const double2*)(ws + off_part), (double2*)(ws + off_chunks));
  TAM_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(tam_k_alpha, dim3(1), dim3(TAM_WG), 0, s, desc, (const double2*)(ws + off_chunks), alpha);
  TAM_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(tam_k_delta, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, m, g, n, alpha, delta);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

int tam_block_ratios(const float* delta, const float* m, uint64_t n, float* ratios, void* stream) {
  tam_err_buf[0] = 0;
  if (!delta || !m || !ratios) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (n == 0) return TAM_OK;
  hipLaunchKernelGGL(tam_k_ratios, dim3(tam_tiles_of(n)), dim3(TAM_WG), 0, (hipStream_t)stream, delta, m, n, ratios);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

static uint64_t tam_thresholds_layout(uint64_t* off_sel, uint64_t* off_hist) {
  uint64_t off = tam_align_up(sizeof(TamTensor), 256);
  *off_sel = off;
  off = tam_align_up(off + sizeof(TamSel), 256);
  *off_hist = off;
  return tam_align_up(off + 4096u * sizeof(uint32_t), 256);
}

size_t tam_thresholds_workspace(uint64_t nb) {
  (void)nb;
  uint64_t a, b;
  return (size_t)tam_thresholds_layout(&a, &b);
}

int tam_thresholds(const float* ratios, uint64_t nb, uint32_t k_lo, uint32_t k_hi, float* taus, void* workspace,
                   size_t ws_bytes, void* stream) {
  tam_err_buf[0] = 0;
  if (!ratios || !taus || !workspace) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (nb == 0 || nb > (1ull << 31)) return tam_fail(TAM_E_INVALID, "%sblock count out of range", "");
  if (k_lo >= nb || k_hi >= nb) return tam_fail(TAM_E_INVALID, "%srank out of range", "");
  if ((uintptr_t)ratios & 15u) return tam_fail(TAM_E_INVALID, "%sratios must be 16-byte aligned", "");
  uint64_t off_sel, off_hist;
  const uint64_t need = tam_thresholds_layout(&off_sel, &off_hist);
  if (ws_bytes < need) return tam_fail(TAM_E_WORKSPACE, "%sworkspace too small: need %ld bytes", "", (long)need);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  TamTensor* desc = (TamTensor*)ws;
  TamSel* sel = (TamSel*)(ws + off_sel);
  uint32_t* hist = (uint32_t*)(ws + off_hist);
  const uint32_t slices = tam_sel_slices(TAM_FLAG_COSTATE, (uint32_t)nb);
  hipLaunchKernelGGL(tam_k_make_desc, dim3(1), dim3(1), 0, s, desc, nb * TAM_BLOCK_SIZE, (uint32_t)nb, k_lo, k_hi);
  TAM_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(tam_k_sel_reset, dim3(1), dim3(TAM_WG), 0, s, desc, sel, hist);
  TAM_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(tam_k_sel_minmax, dim3(slices), dim3(TAM_WG), 0, s, desc, 1, ratios, sel);
  TAM_HIP_CHECK(hipGetLastError());
  for (int r = 0; r < 3; ++r) {
    hipLaunchKernelGGL(tam_k_sel_hist, dim3(slices), dim3(TAM_WG), 0, s, desc, 1, ratios, sel, hist);
    TAM_HIP_CHECK(hipGetLastError());
    hipLaunchKernelGGL(tam_k_sel_pick, dim3(1), dim3(TAM_WG), 0, s, desc, sel, hist);
    TAM_HIP_CHECK(hipGetLastError());
  }
  hipLaunchKernelGGL(tam_k_sel_taus, dim3(1), dim3(1), 0, s, sel, taus);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

int tam_classify(const float* ratios, uint64_t nb, const float* taus, uint8_t* labels, void* stream) {
  tam_err_buf[0] = 0;
  if (!ratios || !taus || !labels) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (nb == 0) return TAM_OK;
  hipLaunchKernelGGL(tam_k_classify, dim3((uint32_t)((nb + 255) / 256)), dim3(256), 0, (hipStream_t)stream, ratios,
                     nb, taus, labels);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

int tam_costate_encode(const float* delta, uint64_t n, uint8_t* signs, float* norms, uint16_t* amp, void* stream) {
  tam_err_buf[0] = 0;
  if (!delta || !signs || !norms || !amp) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if ((uintptr_t)norms & 3u || (uintptr_t)amp & 1u) return tam_fail(TAM_E_INVALID, "%smisaligned CoState state", "");
  if (n == 0) return TAM_OK;
  hipLaunchKernelGGL(tam_k_encode, dim3(tam_tiles_of(n)), dim3(TAM_WG), 0, (hipStream_t)stream, delta, n, signs,
                     norms, amp);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

int tam_fused_v_update(const uint8_t* idx_in, const uint16_t* scales_in, const void* g, uint32_t g_dtype, uint64_t n,
                       uint32_t v_bits, float beta2, float one_minus_beta2, uint32_t tensor_id, uint32_t step,
                       uint64_t seed, uint8_t* idx_out, uint16_t* scales_out, float* v_out, void* stream) {
  tam_err_buf[0] = 0;
  if (!idx_in || !scales_in || !g || !idx_out || !scales_out || !v_out)
    return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (tam_check_dtype(g_dtype)) return TAM_E_INVALID;
  if (!(v_bits == 2 || v_bits == 3 || v_bits == 4 || v_bits == 6 || v_bits == 8))
    return tam_fail(TAM_E_INVALID, "%sv_bits must be 2, 3, 4, 6 or 8", "");
  if (((uintptr_t)idx_in | (uintptr_t)idx_out) & 7u || ((uintptr_t)scales_in | (uintptr_t)scales_out) & 3u)
    return tam_fail(TAM_E_INVALID, "%smisaligned v state", "");
  if (n == 0) return TAM_OK;
  hipLaunchKernelGGL(tam_k_fused_v, dim3(tam_tiles_of(n)), dim3(TAM_WG), 0, (hipStream_t)stream, idx_in, scales_in, g,
                     g_dtype, n, v_bits, beta2, one_minus_beta2, tensor_id, step, (uint32_t)seed,
                     (uint32_t)(seed >> 32), idx_out, scales_out, v_out);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

int tam_v_quantize(const float* v, uint64_t n_padded, uint32_t v_bits, int stochastic, uint32_t tensor_id,
                   uint32_t step, uint64_t seed, uint8_t* idx, uint16_t* scales, void* stream) {
  tam_err_buf[0] = 0;
  if (!v || !idx || !scales) return tam_fail(TAM_E_INVALID, "%snull argument", "");
  if (n_padded % TAM_BLOCK_SIZE) return tam_fail(TAM_E_INVALID, "%slength must be a multiple of 128", "");
  if (!(v_bits == 2 || v_bits == 3 || v_bits == 4 || v_bits == 6 || v_bits == 8))
    return tam_fail(TAM_E_INVALID, "%sv_bits must be 2, 3, 4, 6 or 8", "");
  if ((uintptr_t)scales & 3u) return tam_fail(TAM_E_INVALID, "%smisaligned scales", "");
  if (n_padded == 0) return TAM_OK;
  hipLaunchKernelGGL(tam_k_quantize, dim3(tam_tiles_of(n_padded)), dim3(TAM_WG), 0, (hipStream_t)stream, v, n_padded,
                     v_bits, stochastic, tensor_id, step, (uint32_t)seed, (uint32_t)(seed >> 32), idx, scales);
  TAM_HIP_CHECK(hipGetLastError());
  return TAM_OK;
}

}  // extern "C"

#if TAM_STATS
extern "C" {
// The fallback counters (TAM_ST_COUNT values) into out; reset them to zero
// when reset != 0.  Synchronous.  Measurement builds only.
int tam_stats_read(uint64_t* out, int reset) {
  unsigned long long h[TAM_ST_COUNT];
  TAM_HIP_CHECK(hipDeviceSynchronize());
  TAM_HIP_CHECK(hipMemcpyFromSymbol(h, HIP_SYMBOL(tam_stats), sizeof(h)));
  for (int i = 0; i < TAM_ST_COUNT; ++i) out[i] = (uint64_t)h[i];
  if (reset) {
    memset(h, 0, sizeof(h));
    TAM_HIP_CHECK(hipMemcpyToSymbol(HIP_SYMBOL(tam_stats), h, sizeof(h)));
  }
  return TAM_OK;
}
}  // extern "C"
#endif
