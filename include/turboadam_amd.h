/* turboadam_amd.h -- C ABI of the MI355X (gfx950) TurboAdam packed-state step.
 *
 * Plain pointers and sizes only.  Every device pointer is HIP device memory
 * owned by the caller; the library allocates no device memory in any entry
 * point below.  Work is enqueued on the caller's HIP stream (`stream` is a
 * hipStream_t passed as void*; NULL = the legacy default stream) and returns
 * without synchronising.  Return value: 0 on success, otherwise a TAM_E_*
 * code; tam_last_error() gives a message for the calling thread.
 *
 * Arithmetic contract: results equal, bit for bit, the reference CPU path
 * (davidkny22/turboadam, src/turboadam/{optimizer,costate,quantize}.py) with
 * its library-defined operations fixed as follows: exp/log correctly rounded;
 * dot products and block L2 norms: per 8 consecutive elements an fp32 pairwise
 * tree of the products with a fused first level (fma(x0, y0, fl(x1*y1))),
 * widened to fp64, then a balanced fp64 pairwise tree over the 16 partials of
 * a 128-element block and over the blocks zero-padded to a power of two,
 * rounded to fp32 once (norms: fp64 sqrt first); sqrt correctly rounded.
 * Stochastic-rounding draws come from Philox4x32-10, key = seed: element
 * e = 16t + k of the zero-padded block layout takes bits [24k, 24k+24) of the
 * 384-bit little-endian string of the blocks with counters (3t + j,
 * tensor_id, step, (3t + j) >> 32), j = 0, 1, 2; uniform = draw * 2^-24.
 */
#ifndef TURBOADAM_AMD_H
#define TURBOADAM_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TAM_ABI_VERSION 8
#define TAM_BLOCK_SIZE 128 /* elements per quantisation / CoState block */
#define TAM_TAIL_TILES 4   /* tiles per tail workgroup of an unaligned tensor */

/* error codes */
#define TAM_OK 0
#define TAM_E_INVALID 1  /* bad argument: dtype, size, flag, null pointer */
#define TAM_E_WORKSPACE 2 /* workspace too small */
#define TAM_E_HIP 3      /* a HIP runtime call failed */
#define TAM_E_UNSUPPORTED 4

/* TamTensor.dtype */
#define TAM_DTYPE_F32 0
#define TAM_DTYPE_BF16 1
#define TAM_DTYPE_F16 2

/* TamTensor.flags */
#define TAM_FLAG_COSTATE 0x1u    /* m kept as CoState (else fp32 exp_avg)       */
#define TAM_FLAG_COMPRESS_V 0x2u /* v kept as 1Q indices (else fp32 exp_avg_sq) */
#define TAM_FLAG_HAS_STATE 0x4u  /* CoState holds a previous encoding          */
#define TAM_FLAG_WD 0x8u         /* apply decoupled weight decay p *= c_wd     */
#define TAM_FLAG_EF 0x10u        /* COSTATE with error feedback (ef_residual)  */
#define TAM_FLAG_HAS_EF 0x20u    /* EF: ef_residual holds a residual           */
#define TAM_FLAG_DEVICE_STEP 0x40u /* step, bias corrections, HAS_STATE and     */
                                 /* HAS_EF come from device counters (capture) */
#define TAM_FLAG_SKIP 0x80u      /* [derived, device] DEVICE_STEP: *found_inf was */
                                 /* nonzero; every launch of the step returns   */

/* One parameter tensor of one optimizer step.  The caller fills the fields
 * marked [in]; tam_prepare() fills the fields marked [derived].  The array is
 * then copied to device memory and handed to tam_multi_tensor_step().
 *
 * Replaces the per-parameter body of TurboAdam._full_step_kernel
 * (reference src/turboadam/optimizer.py:97-170) and the state it touches
 * (optimizer.py:242-286, costate.py:357-365, oneq.py:41-48). */
typedef struct TamTensor {
  void* param;          /* [in] n elements of dtype, updated in place        */
  const void* grad;     /* [in] n elements of dtype                          */
  uint8_t* v_idx;       /* [in] COMPRESS_V: u8[nb*128] 1Q indices (in/out),  */
                        /*      16-byte aligned                              */
  uint16_t* v_scales;   /* [in] COMPRESS_V: f16[nb*2] (log_min, log_max),    */
                        /*      4-byte aligned                               */
  float* exp_avg_sq;    /* [in] !COMPRESS_V: f32[n] second moment            */
  float* exp_avg;       /* [in] !COSTATE: f32[n] first moment                */
  uint8_t* signs;       /* [in] COSTATE: u8[ceil(n/8)] sign bits, MSB first, */
                        /*      2-byte aligned                               */
  uint8_t* labels;      /* [in] COSTATE: u8[nb] 0 null, 1 phase, 2 amplitude */
  float* norms;         /* [in] COSTATE: f32[nb] residual block L2 norms     */
  uint16_t* amp;        /* [in] COSTATE: f16[nb] amplitude scales            */
                        /*      (norms and alpha 4-byte, amp 2-byte aligned) */
  float* alpha;         /* [in] COSTATE: f32[1] projection alpha (in/out)    */
  uint64_t n;           /* [in] number of elements (>= 1)                    */
  uint32_t dtype;       /* [in] TAM_DTYPE_* of param and grad                */
  uint32_t flags;       /* [in] TAM_FLAG_*                                   */
  uint32_t v_bits;      /* [in] 2, 3, 4, 6 or 8                              */
  uint32_t tensor_id;   /* [in] Philox counter word 1                        */
  uint32_t step;        /* [in] 1-based step number (Philox counter word 2)  */
  uint32_t k_lo, k_hi;  /* [in] COSTATE: ranks of the P_null / P_amp ratios  */
  float inv_bc2_f32;    /* [in] f32(1 / bias_correction2)                    */
  float c_wd;           /* [in] f32(1 - lr*wd)                               */
  float beta1, one_minus_beta1, beta2, one_minus_beta2; /* [in] f32 of the doubles */
  float bias_correction1, bias_correction2;             /* [in] f32(1-beta^step)   */
  float eps, neg_lr;    /* [in] f32(eps), f32(-lr)                           */
  float sqrt_block;     /* [in] f32(sqrt(128)) (the only block size)         */
  uint32_t nb;          /* [derived] ceil(n/128)                             */
  uint32_t tile0;       /* [derived] first tile (16 blocks) of this tensor   */
  uint32_t ntiles;      /* [derived] ceil(nb/16)                             */
  uint32_t chunk0;      /* [derived] COSTATE: first alpha-reduction chunk    */
  uint64_t ratio_off;   /* [derived] COSTATE: offset of its ratios (blocks)  */
  double inv_bc2;       /* [in] 1 / (double)bias_correction2 (correctly rounded) */
  uint32_t slice0;      /* [derived] COSTATE: first selection slice (8192 blocks each) */
  float c_lr;           /* [derived] f32(neg_lr / bias_correction1)          */
  float* ef_residual;   /* [in] EF: f32[n] error-feedback residual (in/out;  */
                        /*      written, not read, without HAS_EF)           */
  uint64_t ef_off;      /* [derived] EF: workspace offset of the staged encoding */
  /* DEVICE_STEP (a step that can be captured in a graph and replayed): the
   * first launch of the step fills step, bias_correction1/2, inv_bc2,
   * inv_bc2_f32, c_lr, k_abs and the HAS_STATE / HAS_EF flags of this descriptor in
   * device memory from the counters below, then increments *step_dev.  The
   * host values of those fields are ignored. */
  uint32_t* step_dev;       /* [in] updates of this tensor so far (device)      */
  const uint32_t* bc_step;  /* [in] counter whose next value indexes bc_table:   */
                            /*      the group's last parameter with state       */
                            /*      (reference optimizer.py:172-188)            */
  const float* bc_table;    /* [in] f32 pairs (1-beta1^t, 1-beta2^t), t = 1..bc_len */
  uint32_t bc_len;          /* [in] pairs in bc_table; later steps use the last */
  float k_abs;              /* [derived] absolute error term of the certified   */
                            /*      16-bit update: 2^-147 / bias_correction1 *  */
                            /*      min(1/eps, 2^63) * (1 + 2^-20) + 2^-148,     */
                            /*      rounded up to f32                           */
  const float* found_inf;   /* [in] DEVICE_STEP, or NULL: the step leaves every */
                            /*      tensor and counter unchanged when           */
                            /*      *found_inf != 0 (a GradScaler skip).  Given */
                            /*      for one descriptor, given for all (the same */
                            /*      pointer): the launches test descriptor 0.   */
  uint32_t tail0;           /* [derived] first workgroup of this tensor in pass 0's */
                            /*      kernel for quarters that are not full        */
  uint32_t tail_wgs;        /* [derived] its workgroups there: 1, or one per    */
                            /*      TAM_TAIL_TILES tiles when param or grad is  */
                            /*      not 16-byte aligned (every quarter is then  */
                            /*      bounds-checked)                             */
} TamTensor;

/* Launch summary and workspace layout, filled by tam_prepare(). */
typedef struct TamStepInfo {
  int32_t n_tensors;
  uint32_t total_tiles;
  uint32_t n_costate;
  uint32_t total_chunks;   /* alpha-reduction chunks (8192 partial sums each) */
  uint32_t total_slices;   /* selection slices (8192 block ratios each) */
  uint32_t dtype_mask;     /* bit TAM_DTYPE_x set when a tensor of that dtype without TAM_FLAG_EF is present */
  uint64_t ratio_blocks;   /* sum of nb over CoState tensors */
  uint64_t off_partials;   /* workspace byte offsets */
  uint64_t off_alpha;
  uint64_t off_ratios;
  uint64_t ws_bytes;       /* required workspace size */
  uint64_t off_chunks;
  uint64_t off_sel;
  uint64_t off_hist;
  uint32_t n_ef;           /* tensors with error feedback (a fifth pass runs) */
  uint32_t n_device_step;  /* DEVICE_STEP tensors (pass 0 starts with their prologue) */
  uint64_t off_ef_alpha;   /* EF: previous alpha of each tensor (f32 per tensor) */
  uint32_t tail_blocks;    /* workgroups of pass 0's kernel for quarters that are not full */
} TamStepInfo;

/* Version of this ABI (TAM_ABI_VERSION). */
int tam_abi_version(void);

/* sizeof(TamTensor) for which == 0, sizeof(TamStepInfo) for which == 1, so a
 * binding can check its struct mirror. */
size_t tam_struct_size(int which);

/* Message for the last failing call on this thread ("" if none). */
const char* tam_last_error(void);

/* Host only (no HIP call): validate `tensors`, fill the [derived] fields and
 * the launch summary.  Replaces the lazy-init bookkeeping of TurboAdam.step
 * (reference optimizer.py:232-286) for one step's tensor list. */
int tam_prepare(TamTensor* tensors, int n_tensors, TamStepInfo* info);

/* One fused optimizer step over every tensor of `d_tensors` (device copy of
 * the array prepared by tam_prepare) in four passes: the fused update
 * (decode, EMA, 1Q re-quantisation, AdamW update, dot partials), alpha,
 * CoState encode + block ratios, selection + classification; a fifth for
 * error feedback.  Replaces TurboAdam._full_step_kernel (reference
 * optimizer.py:88-170) with CoStateManager.update (costate.py:367-464) and
 * fused_v_update (quantize.py:222-299 / triton_kernels.py:105-165) inlined.
 * `workspace` must hold info->ws_bytes bytes of device memory (contents need
 * not be kept between calls).  `h_tensors` is the host array tam_prepare()
 * filled; it is not read.  DEVICE_STEP descriptors are completed in place in
 * d_tensors.  No host synchronisation and no allocation: the call can be
 * captured in a HIP graph (with DEVICE_STEP tensors, each replay is a step). */
int tam_multi_tensor_step(const TamTensor* d_tensors, const TamTensor* h_tensors,
                          const TamStepInfo* info, uint64_t seed, void* workspace,
                          size_t ws_bytes, void* stream);

/* tam_multi_tensor_step for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): the same step with no workspace argument.  No counterpart in
 * the reference.  Its workspace is a static device array of
 * TAM_STATIC_SCRATCH_BYTES that the library holds on every GPU it runs on
 * until the process ends; the call allocates nothing (no hipMalloc, no
 * allocating library routine).  A step whose info->ws_bytes exceeds
 * TAM_STATIC_SCRATCH_BYTES (about 1.07e9 parameters of CoState tensors)
 * returns TAM_E_WORKSPACE without launching anything.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (streams not
 * ordered with each other) race.  The caller still provides d_tensors. */
#define TAM_STATIC_SCRATCH_BYTES (64ull << 20)
int tam_multi_tensor_step_static(const TamTensor* d_tensors, const TamTensor* h_tensors,
                                 const TamStepInfo* info, uint64_t seed, void* stream);

/* One of the passes of tam_multi_tensor_step (same arguments): 0 = the fused
 * update, 1 = alpha, 2 = CoState encode, 3 = selection and labels, 4 = the
 * error-feedback residual and commit of the staged encoding (nothing to do
 * without TAM_FLAG_EF tensors).  Issuing passes 0..4 in order on one stream
 * equals one tam_multi_tensor_step call; callers use it to time the passes one
 * by one.  No counterpart in the reference (its step is not split into passes). */
int tam_step_pass(int pass, const TamTensor* d_tensors, const TamStepInfo* info, uint64_t seed,
                  void* workspace, size_t ws_bytes, void* stream);

/* Decode 1Q indices to fp32 v: out[i] = exp(lmin + ((idx+0.5)/2^bits)*span)
 * for i < n.  Replaces dequantize_logscale_nbits (reference quantize.py:183-214)
 * as used by decompress_v (oneq.py:51-67). */
int tam_v_dequantize(const uint8_t* v_idx, const uint16_t* v_scales, uint64_t n,
                     uint32_t v_bits, float* out, void* stream);

/* Stochastic-rounding uniforms of elements [0, count) of tensor `tensor_id`
 * at `step` (the draws the step consumes).  Replaces the rand_buf refill
 * (reference optimizer.py:131) / torch.rand_like (quantize.py:291). */
int tam_philox_uniforms(uint32_t tensor_id, uint32_t step, uint64_t seed,
                        uint64_t count, float* out, void* stream);

/* ---- standalone helpers: the reference's public functions, one tensor per
 * call, with the step's arithmetic.  Device pointers, caller's stream. ---- */

/* decode_blocks (reference costate.py:261-324): m_out[i] = fl(alpha*g[i]) +
 * s_b*sign_i for n elements (g of g_dtype; alpha a device float).  With
 * ema != 0 the EMA of CoStateManager.update (costate.py:416) follows:
 * m_out = fl(beta1*m_hat) + fl(one_minus_beta1*g); has_state == 0 means
 * m_hat = 0 and the CoState arrays are not read. */
int tam_costate_decode(const uint8_t* labels, const uint8_t* signs, const float* norms, const uint16_t* amp,
                       const float* alpha, const void* g, uint32_t g_dtype, uint64_t n, int has_state, int ema,
                       float beta1, float one_minus_beta1, float* m_out, void* stream);

/* decompose (reference costate.py:22-43): *alpha (device float) = fl(mg)/fl(gg)
 * with the step's dot products (the contract above; 0 when gg == 0), delta =
 * fl(m - fl(alpha*g)).  m, g fp32[n].  Workspace: tam_decompose_workspace(n)
 * bytes of device memory. */
size_t tam_decompose_workspace(uint64_t n);
int tam_decompose(const float* m, const float* g, uint64_t n, float* alpha, float* delta, void* workspace,
                  size_t ws_bytes, void* stream);

/* compute_block_ratios (reference costate.py:51-86): ratios[b] =
 * ||delta_b|| / ||m_b|| (the contract's block norms), 0 where ||m_b|| == 0. */
int tam_block_ratios(const float* delta, const float* m, uint64_t n, float* ratios, void* stream);

/* compute_thresholds (reference costate.py:94-118): taus[0], taus[1] (device
 * floats) = the k_lo-th and k_hi-th smallest ratios (NaN last).  ratios is
 * 16-byte aligned; workspace: tam_thresholds_workspace(nb) bytes. */
size_t tam_thresholds_workspace(uint64_t nb);
int tam_thresholds(const float* ratios, uint64_t nb, uint32_t k_lo, uint32_t k_hi, float* taus, void* workspace,
                   size_t ws_bytes, void* stream);

/* classify_blocks (reference costate.py:126-149) with taus[0], taus[1] on the device. */
int tam_classify(const float* ratios, uint64_t nb, const float* taus, uint8_t* labels, void* stream);

/* encode_blocks (reference costate.py:213-258, _pack_signs :157-182): block
 * norms of delta, fp16 amplitudes norm/f32(sqrt(128)), sign bits (MSB first). */
int tam_costate_encode(const float* delta, uint64_t n, uint8_t* signs, float* norms, uint16_t* amp, void* stream);

/* fused_v_update (reference quantize.py:222-299) for one tensor: decode, EMA,
 * re-quantisation with the step's Philox draws for (tensor_id, step, seed);
 * v_out receives v (fp32, n values).  The outputs may be the inputs. */
int tam_fused_v_update(const uint8_t* idx_in, const uint16_t* scales_in, const void* g, uint32_t g_dtype, uint64_t n,
                       uint32_t v_bits, float beta2, float one_minus_beta2, uint32_t tensor_id, uint32_t step,
                       uint64_t seed, uint8_t* idx_out, uint16_t* scales_out, float* v_out, void* stream);

/* quantize_logscale_nbits (reference quantize.py:126-180) of v (n_padded, a
 * multiple of 128): fp16 (log_min, log_max) per block and indices, rounded
 * down (stochastic == 0) or stochastically with the Philox draws. */
int tam_v_quantize(const float* v, uint64_t n_padded, uint32_t v_bits, int stochastic, uint32_t tensor_id,
                   uint32_t step, uint64_t seed, uint8_t* idx, uint16_t* scales, void* stream);

/* Self-check of the device arithmetic: out[i] = f(in[i]) with f selected by
 * `fn` (0 log, 1 exp, 2 f32->f16->f32, 3 f32->bf16->f32 in software, 4 sqrt,
 * 5 f32->bf16->f32 by the hardware conversion; the raw hardware instructions
 * whose error bounds the certified fast paths assume: 6 v_sqrt_f32,
 * 7 v_rcp_f32, 8 v_log_f32 (log2)).  No counterpart in the reference: it lets
 * a caller confirm the device math equals the host. */
int tam_math_eval(int fn, const float* in, float* out, uint64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TURBOADAM_AMD_H */
