/* tam_oracle.h -- TEST INFRASTRUCTURE ONLY: the parts of the CPU oracle
 * (tam_oracle.c) that a C or C++ checker links against.  Never included by
 * the turboadam_amd product path. */
#ifndef TAM_ORACLE_H
#define TAM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct OrTensor {
  void* param;
  const void* grad;
  uint8_t* v_idx;
  uint16_t* v_scales;
  float* exp_avg_sq;
  float* exp_avg;
  uint8_t* signs;
  uint8_t* labels;
  float* norms;
  uint16_t* amp;
  float* alpha;
  float* ef_residual; /* EF: f32[n] error-feedback residual (in/out) */
  uint64_t n;
  /* block0: first block of this tensor within the parameter it is a
   * block-aligned slice of (0 for a whole parameter); only the stochastic
   * rounding draws depend on it */
  uint32_t dtype, flags, v_bits, tensor_id, step, k_lo, k_hi, block0;
  float c_wd, beta1, one_minus_beta1, beta2, one_minus_beta2, bias_correction1, bias_correction2, eps,
      neg_lr, sqrt_block;
} OrTensor;

#define OR_FLAG_COSTATE 1u
#define OR_FLAG_COMPRESS_V 2u
#define OR_FLAG_HAS_STATE 4u
#define OR_FLAG_WD 8u
#define OR_FLAG_EF 16u
#define OR_FLAG_HAS_EF 32u

/* One parameter's TurboAdam step on host arrays (the caller advances the step
 * counter and supplies the fp32 scalars and flags). */
void or_step_tensor(OrTensor* t, uint64_t seed);
/* The stochastic-rounding uniforms of (tid, step) for elements 0 .. count-1. */
void or_philox_uniforms(uint32_t tid, uint32_t step, uint64_t seed, uint64_t count, float* out);
uint16_t or_f32_to_bf16(float x);
float or_bf16_to_f32(uint16_t b);

#ifdef __cplusplus
}
#endif

#endif
