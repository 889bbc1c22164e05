// step_check -- a C-ABI caller of libturboadam_amd with no torch and no Python:
// plain pointers, hipMalloc'd state, tam_prepare + tam_multi_tensor_step, the
// host bookkeeping a binding does per step (bias corrections, ranks, flags).
// Two tensors: a bf16 one with CoState m (70001 elements: a tail block) and an
// fp32 one with fp32 m (3000 elements), both with 4-bit 1Q v and weight decay.
// After every step the parameters and every state array are compared byte for
// byte with the CPU oracle (oracle/tam_oracle.c, linked as the checker).
// Prints "capi: ok" and exits 0 on success; exits 1 on a mismatch or an error.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/turboadam_amd.h"
#include "../../oracle/tam_oracle.h"

#define HIP_OK(x)                                                            \
  do {                                                                       \
    hipError_t e_ = (x);                                                     \
    if (e_ != hipSuccess) {                                                  \
      std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));    \
      std::exit(1);                                                          \
    }                                                                        \
  } while (0)

static float f32(double x) { return (float)x; }

// deterministic N(0,1) draws (64-bit LCG + Box-Muller)
struct Rng {
  uint64_t s;
  double uni() {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return ((s >> 11) + 0.5) * 0x1p-53;
  }
  float normal() { return (float)(std::sqrt(-2.0 * std::log(uni())) * std::cos(6.283185307179586 * uni())); }
};

template <typename T>
static T* dev_copy(const std::vector<T>& h) {
  T* d = nullptr;
  HIP_OK(hipMalloc((void**)&d, h.size() * sizeof(T)));
  HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
  return d;
}

template <typename T>
static std::vector<T> host_copy(const T* d, size_t n) {
  std::vector<T> h(n);
  HIP_OK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
  return h;
}

template <typename T>
static int compare(const char* what, int tensor, int step, const T* dev, const std::vector<T>& want) {
  const std::vector<T> got = host_copy(dev, want.size());
  if (std::memcmp(got.data(), want.data(), want.size() * sizeof(T)) == 0) return 0;
  size_t bad = 0, first = want.size();
  for (size_t i = 0; i < want.size(); ++i)
    if (std::memcmp(&got[i], &want[i], sizeof(T)) != 0) {
      ++bad;
      if (first == want.size()) first = i;
    }
  std::printf("step %d tensor %d: %s differs in %zu of %zu (first at %zu)\n", step, tensor, what, bad, want.size(),
              first);
  return 1;
}

// One tensor: host (oracle) state and device state side by side.
struct Side {
  uint64_t n, nb;
  uint32_t dtype;
  bool costate;
  std::vector<uint16_t> p16;  // bf16 parameter bits
  std::vector<float> p32;     // fp32 parameter
  std::vector<uint8_t> idx, signs, labels;
  std::vector<uint16_t> scales, amp;
  std::vector<float> norms, alpha, exp_avg;
  void* d_param = nullptr;
  uint8_t *d_idx = nullptr, *d_signs = nullptr, *d_labels = nullptr;
  uint16_t *d_scales = nullptr, *d_amp = nullptr;
  float *d_norms = nullptr, *d_alpha = nullptr, *d_exp_avg = nullptr;
};

static const uint16_t kVInitScale = 0xd451;  // f16(ln(f32(1e-30))) = -69.0625: the first-step v state

static void init_side(Side& s, uint64_t n, uint32_t dtype, bool costate, Rng& rng) {
  s.n = n;
  s.nb = (n + TAM_BLOCK_SIZE - 1) / TAM_BLOCK_SIZE;
  s.dtype = dtype;
  s.costate = costate;
  if (dtype == TAM_DTYPE_BF16) {
    s.p16.resize(n);
    for (auto& x : s.p16) x = or_f32_to_bf16(0.02f * rng.normal());
    s.d_param = dev_copy(s.p16);
  } else {
    s.p32.resize(n);
    for (auto& x : s.p32) x = 0.02f * rng.normal();
    s.d_param = dev_copy(s.p32);
  }
  s.idx.assign(s.nb * TAM_BLOCK_SIZE, 0);
  s.scales.assign(s.nb * 2, kVInitScale);
  s.d_idx = dev_copy(s.idx);
  s.d_scales = dev_copy(s.scales);
  if (costate) {
    s.signs.assign((n + 7) / 8, 0);
    s.labels.assign(s.nb, 0);
    s.norms.assign(s.nb, 0.0f);
    s.amp.assign(s.nb, 0);
    s.alpha.assign(1, 0.0f);
    s.d_signs = dev_copy(s.signs);
    s.d_labels = dev_copy(s.labels);
    s.d_norms = dev_copy(s.norms);
    s.d_amp = dev_copy(s.amp);
    s.d_alpha = dev_copy(s.alpha);
  } else {
    s.exp_avg.assign(n, 0.0f);
    s.d_exp_avg = dev_copy(s.exp_avg);
  }
}

int main() {
  const double lr = 1e-3, beta1 = 0.9, beta2 = 0.999, eps = 1e-8, wd = 0.01;
  const double null_pct = 0.10, amp_pct = 0.90;
  const uint32_t v_bits = 4;
  const uint64_t seed = 0x5eed1234abcdull;
  if (tam_abi_version() != TAM_ABI_VERSION || tam_struct_size(0) != sizeof(TamTensor) ||
      tam_struct_size(1) != sizeof(TamStepInfo)) {
    std::printf("ABI mismatch\n");
    return 1;
  }
  Rng rng{42};
  Side sides[2];
  init_side(sides[0], 70001, TAM_DTYPE_BF16, true, rng);
  init_side(sides[1], 3000, TAM_DTYPE_F32, false, rng);
  TamTensor* d_desc = nullptr;
  HIP_OK(hipMalloc((void**)&d_desc, 2 * sizeof(TamTensor)));
  void* ws = nullptr;
  size_t ws_bytes = 0;
  int bad = 0;
  for (int step = 1; step <= 3; ++step) {
    // bias corrections of this step, in double, rounded to fp32 once (reference optimizer.py:172-188)
    const double bc1 = 1.0 - std::pow(beta1, step), bc2 = 1.0 - std::pow(beta2, step);
    TamTensor h[2];
    OrTensor o[2];
    std::vector<uint16_t> g16;
    std::vector<float> g32;
    void* d_grad[2] = {nullptr, nullptr};
    for (int t = 0; t < 2; ++t) {
      Side& s = sides[t];
      // the gradient, on both sides
      if (s.dtype == TAM_DTYPE_BF16) {
        g16.resize(s.n);
        for (auto& x : g16) x = or_f32_to_bf16(1e-3f * rng.normal());
        d_grad[t] = dev_copy(g16);
      } else {
        g32.resize(s.n);
        for (auto& x : g32) x = 1e-3f * rng.normal();
        d_grad[t] = dev_copy(g32);
      }
      std::memset(&h[t], 0, sizeof(TamTensor));
      std::memset(&o[t], 0, sizeof(OrTensor));
      uint32_t flags = TAM_FLAG_COMPRESS_V | TAM_FLAG_WD;
      if (s.costate) flags |= TAM_FLAG_COSTATE | (step > 1 ? TAM_FLAG_HAS_STATE : 0u);
      const uint32_t k_lo = (uint32_t)std::max<int64_t>(0, (int64_t)(null_pct * (double)s.nb) - 1);
      const uint32_t k_hi = (uint32_t)std::min<int64_t>((int64_t)s.nb - 1, (int64_t)(amp_pct * (double)s.nb));
      TamTensor& d = h[t];
      d.param = s.d_param;
      d.grad = d_grad[t];
      d.v_idx = s.d_idx;
      d.v_scales = s.d_scales;
      d.exp_avg = s.d_exp_avg;
      d.signs = s.d_signs;
      d.labels = s.d_labels;
      d.norms = s.d_norms;
      d.amp = s.d_amp;
      d.alpha = s.d_alpha;
      d.n = s.n;
      d.dtype = s.dtype;
      d.flags = flags;
      d.v_bits = v_bits;
      d.tensor_id = (uint32_t)t;
      d.step = (uint32_t)step;
      d.k_lo = s.costate ? k_lo : 0;
      d.k_hi = s.costate ? k_hi : 0;
      d.c_wd = f32(1.0 - lr * wd);
      d.beta1 = f32(beta1);
      d.one_minus_beta1 = f32(1.0 - beta1);
      d.beta2 = f32(beta2);
      d.one_minus_beta2 = f32(1.0 - beta2);
      d.bias_correction1 = f32(bc1);
      d.bias_correction2 = f32(bc2);
      d.inv_bc2 = 1.0 / (double)d.bias_correction2;
      d.inv_bc2_f32 = f32(d.inv_bc2);
      d.eps = f32(eps);
      d.neg_lr = f32(-lr);
      d.sqrt_block = f32(std::sqrt(128.0));
      // the oracle's tensor: the same scalars, host arrays
      OrTensor& r = o[t];
      r.param = s.dtype == TAM_DTYPE_BF16 ? (void*)s.p16.data() : (void*)s.p32.data();
      r.grad = s.dtype == TAM_DTYPE_BF16 ? (const void*)g16.data() : (const void*)g32.data();
      r.v_idx = s.idx.data();
      r.v_scales = s.scales.data();
      r.exp_avg = s.costate ? nullptr : s.exp_avg.data();
      r.signs = s.costate ? s.signs.data() : nullptr;
      r.labels = s.costate ? s.labels.data() : nullptr;
      r.norms = s.costate ? s.norms.data() : nullptr;
      r.amp = s.costate ? s.amp.data() : nullptr;
      r.alpha = s.costate ? s.alpha.data() : nullptr;
      r.n = s.n;
      r.dtype = s.dtype;
      r.flags = flags;  // the OR_FLAG_* values equal the TAM_FLAG_* ones used here
      r.v_bits = v_bits;
      r.tensor_id = (uint32_t)t;
      r.step = (uint32_t)step;
      r.k_lo = d.k_lo;
      r.k_hi = d.k_hi;
      r.c_wd = d.c_wd;
      r.beta1 = d.beta1;
      r.one_minus_beta1 = d.one_minus_beta1;
      r.beta2 = d.beta2;
      r.one_minus_beta2 = d.one_minus_beta2;
      r.bias_correction1 = d.bias_correction1;
      r.bias_correction2 = d.bias_correction2;
      r.eps = d.eps;
      r.neg_lr = d.neg_lr;
      r.sqrt_block = d.sqrt_block;
      or_step_tensor(&r, seed);  // the oracle updates the host copies in place
    }
    TamStepInfo info;
    if (tam_prepare(h, 2, &info) != TAM_OK) {
      std::printf("tam_prepare: %s\n", tam_last_error());
      return 1;
    }
    if (info.ws_bytes > ws_bytes) {
      if (ws) HIP_OK(hipFree(ws));
      HIP_OK(hipMalloc(&ws, info.ws_bytes));
      ws_bytes = info.ws_bytes;
    }
    HIP_OK(hipMemcpy(d_desc, h, 2 * sizeof(TamTensor), hipMemcpyHostToDevice));
    if (tam_multi_tensor_step(d_desc, h, &info, seed, ws, ws_bytes, nullptr) != TAM_OK) {
      std::printf("tam_multi_tensor_step: %s\n", tam_last_error());
      return 1;
    }
    HIP_OK(hipDeviceSynchronize());
    for (int t = 0; t < 2; ++t) {
      Side& s = sides[t];
      if (s.dtype == TAM_DTYPE_BF16)
        bad += compare("param", t, step, (const uint16_t*)s.d_param, s.p16);
      else
        bad += compare("param", t, step, (const float*)s.d_param, s.p32);
      bad += compare("v indices", t, step, s.d_idx, s.idx);
      bad += compare("v scales", t, step, s.d_scales, s.scales);
      if (s.costate) {
        bad += compare("sign bits", t, step, s.d_signs, s.signs);
        bad += compare("labels", t, step, s.d_labels, s.labels);
        bad += compare("block norms", t, step, s.d_norms, s.norms);
        bad += compare("amplitudes", t, step, s.d_amp, s.amp);
        bad += compare("alpha", t, step, s.d_alpha, s.alpha);
      } else {
        bad += compare("exp_avg", t, step, s.d_exp_avg, s.exp_avg);
      }
      HIP_OK(hipFree(d_grad[t]));
    }
    std::printf("capi: step %d checked\n", step);
    std::fflush(stdout);
  }
  if (bad) return 1;
  std::printf("capi: ok\n");
  return 0;
}
