// tam_stream.hip -- streaming kernels that measure the HBM bandwidth a plain
// memory-bound kernel reaches on this device (the practical ceiling that the
// step's kernels are compared against).  Measurement infrastructure for
// bench.py only: not part of the optimizer library or its ABI.
//
// tam_stream_run sweeps the shape of a plain stream of 16-byte words:
//   kind     read / write / copy / 2r1w (c = a + b) / inplace (a = a + b);
//   W        16-byte words in flight per lane (4, 8 or 16): every load of a
//            round is issued before the first use;
//   WG       threads per workgroup (256, 512 or 1024);
//   rounds   grid size, in multiples of the workgroups that hold 32 waves on
//            every CU;
//   nt       nontemporal loads and stores (the data is not kept for reuse);
//   layout   which words a lane takes in a round of grid * WG * W words:
//            0 grid-stride (word k of thread t: k * T + t, so each load
//              instruction of a wave covers 1 KiB),
//            1 wave-contiguous (a wave's W loads cover W KiB in a row),
//            2 lane-contiguous (each lane W consecutive words, as a pass-0
//              lane reads its 32-byte parameter and gradient slices).
//
// tam_stream_pass0 streams the arrays of the step's first pass with its access
// widths, one 1024-element unit (8 blocks of 128) per wave and lane l owning
// 16 elements of block l / 8: a 16-bit parameter and gradient (32 bytes per
// lane, parameter written back), the u8 1Q indices (16 bytes, written back),
// per block the 32-bit scale pair (written back), sign bits (2 bytes per lane),
// label, f32 norm and f16 amplitude, and one 16-byte partial per 512
// elements written.  The arithmetic is a few XORs, so it measures the memory
// side alone.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t TamW4 __attribute__((ext_vector_type(4)));
typedef uint32_t TamW2 __attribute__((ext_vector_type(2)));

enum { TAM_ST_READ = 0, TAM_ST_WRITE = 1, TAM_ST_COPY = 2, TAM_ST_ADD = 3, TAM_ST_INPLACE = 4 };

template <bool NT, typename T>
__device__ __forceinline__ T tam_st_ld(const T* p) {
  return NT ? __builtin_nontemporal_load(p) : *p;
}
template <bool NT, typename T>
__device__ __forceinline__ void tam_st_st(T* p, T v) {
  if (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// Word k of thread t in a round starting at `base` (T threads in the grid).
__device__ __forceinline__ uint64_t tam_st_word(int layout, uint64_t base, uint64_t T, uint64_t t, int k, int W) {
  if (layout == 0) return base + (uint64_t)k * T + t;
  if (layout == 1) return base + (t >> 6) * 64u * (uint64_t)W + (uint64_t)k * 64u + (t & 63u);
  return base + t * (uint64_t)W + (uint64_t)k;
}

// kind READ:    x ^= a[i]; one word per thread written to c at the end
// kind WRITE:   c[i] = pattern
// kind COPY:    c[i] = a[i]
// kind ADD:     c[i] = a[i] + b[i]      (two reads, one write, three streams)
// kind INPLACE: a[i] = a[i] + b[i]      (read-modify-write of a, read of b)
template <int KIND, bool NT, int W, int WG>
__global__ __launch_bounds__(WG) void tam_k_stream(TamW4* a, const TamW4* b, TamW4* c, uint64_t n, int layout) {
  const uint64_t T = (uint64_t)gridDim.x * WG;
  const uint64_t t = (uint64_t)blockIdx.x * WG + threadIdx.x;
  const uint64_t per_round = T * (uint64_t)W;
  TamW4 acc = {0u, 0u, 0u, 0u};
  uint64_t base = 0;
  for (; base + per_round <= n; base += per_round) {
    TamW4 x[W], y[W];
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const uint64_t j = tam_st_word(layout, base, T, t, k, W);
      if (KIND != TAM_ST_WRITE) x[k] = tam_st_ld<NT>(a + j);
      if (KIND == TAM_ST_ADD || KIND == TAM_ST_INPLACE) y[k] = tam_st_ld<NT>(b + j);
    }
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const uint64_t j = tam_st_word(layout, base, T, t, k, W);
      if (KIND == TAM_ST_READ) acc ^= x[k];
      if (KIND == TAM_ST_WRITE) tam_st_st<NT>(c + j, TamW4{(uint32_t)j, 1u, 2u, 3u});
      if (KIND == TAM_ST_COPY) tam_st_st<NT>(c + j, x[k]);
      if (KIND == TAM_ST_ADD) tam_st_st<NT>(c + j, x[k] + y[k]);
      if (KIND == TAM_ST_INPLACE) tam_st_st<NT>(a + j, x[k] + y[k]);
    }
  }
  // the last partial round, word by word (grid-stride)
  for (uint64_t i = base + t; i < n; i += T) {
    if (KIND == TAM_ST_READ) acc ^= tam_st_ld<NT>(a + i);
    if (KIND == TAM_ST_WRITE) tam_st_st<NT>(c + i, TamW4{(uint32_t)i, 1u, 2u, 3u});
    if (KIND == TAM_ST_COPY) tam_st_st<NT>(c + i, tam_st_ld<NT>(a + i));
    if (KIND == TAM_ST_ADD) tam_st_st<NT>(c + i, tam_st_ld<NT>(a + i) + tam_st_ld<NT>(b + i));
    if (KIND == TAM_ST_INPLACE) tam_st_st<NT>(a + i, tam_st_ld<NT>(a + i) + tam_st_ld<NT>(b + i));
  }
  // one word per thread (c holds n words, as every operand)
  if (KIND == TAM_ST_READ && t < n) c[t] = acc;
}

template <int KIND, bool NT, int W>
static void tam_st_launch_wg(int wg, dim3 grid, hipStream_t s, TamW4* a, const TamW4* b, TamW4* c, uint64_t n,
                             int layout) {
  if (wg == 256) hipLaunchKernelGGL((tam_k_stream<KIND, NT, W, 256>), grid, dim3(256), 0, s, a, b, c, n, layout);
  else if (wg == 512) hipLaunchKernelGGL((tam_k_stream<KIND, NT, W, 512>), grid, dim3(512), 0, s, a, b, c, n, layout);
  else hipLaunchKernelGGL((tam_k_stream<KIND, NT, W, 1024>), grid, dim3(1024), 0, s, a, b, c, n, layout);
}

template <int KIND, bool NT>
static void tam_st_launch_w(int w, int wg, dim3 grid, hipStream_t s, TamW4* a, const TamW4* b, TamW4* c, uint64_t n,
                            int layout) {
  if (w == 4) tam_st_launch_wg<KIND, NT, 4>(wg, grid, s, a, b, c, n, layout);
  else if (w == 8) tam_st_launch_wg<KIND, NT, 8>(wg, grid, s, a, b, c, n, layout);
  else tam_st_launch_wg<KIND, NT, 16>(wg, grid, s, a, b, c, n, layout);
}

template <int KIND>
static void tam_st_launch(int nt, int w, int wg, dim3 grid, hipStream_t s, TamW4* a, const TamW4* b, TamW4* c,
                          uint64_t n, int layout) {
  if (nt) tam_st_launch_w<KIND, true>(w, wg, grid, s, a, b, c, n, layout);
  else tam_st_launch_w<KIND, false>(w, wg, grid, s, a, b, c, n, layout);
}

// ---------------------------------------------------------------- pass-0 shape
struct TamP0Arrays {
  uint16_t* param;        // 2 bytes per element, read and written
  const uint16_t* grad;   // 2 bytes per element
  uint8_t* idx;           // 1 byte per element, read and written
  uint32_t* scales;       // 4 bytes per block, read and written
  const uint8_t* signs;   // 1 bit per element
  const uint8_t* labels;  // 1 byte per block
  const float* norms;     // 4 bytes per block
  const uint16_t* amp;    // 2 bytes per block
  TamW4* partials;        // 16 bytes per 512 elements, written
};

template <bool NT, typename T>
__device__ __forceinline__ T tam_p0_ld(const T* p) {
  return tam_st_ld<NT>(p);
}

// LAYOUT 0: lane l owns elements [16 l, 16 l + 16) of the unit (32 bytes of a
// 16-bit array per lane, two adjacent 16-byte loads; 16 index bytes); LAYOUT 1:
// lane l owns elements [8 l, 8 l + 8) and [512 + 8 l, 512 + 8 l + 8) (each 16-byte
// load instruction of a 16-bit array covers 1 KiB in a row; two 8-byte index
// loads, each instruction 512 bytes in a row).  NT: nontemporal loads and
// stores of the parameter, gradient and indices.
template <int WG, int LAYOUT, bool NT>
__global__ __launch_bounds__(WG) void tam_k_stream_pass0(TamP0Arrays A, uint64_t units) {
  extern __shared__ uint32_t pad[];  // occupancy control only
  const uint32_t lane = threadIdx.x & 63u;
  const uint64_t waves = (uint64_t)gridDim.x * (WG / 64);
  for (uint64_t u = (uint64_t)blockIdx.x * (WG / 64) + (threadIdx.x >> 6); u < units; u += waves) {
    if (LAYOUT == 0) {
      const uint64_t e0 = u * 1024u + lane * 16u;
      const uint64_t b = u * 8u + (lane >> 3);
      const TamW4* pp = (const TamW4*)(A.param + e0);
      const TamW4* gp = (const TamW4*)(A.grad + e0);
      TamW4 p0 = tam_p0_ld<NT>(pp), p1 = tam_p0_ld<NT>(pp + 1), g0 = tam_p0_ld<NT>(gp), g1 = tam_p0_ld<NT>(gp + 1);
      TamW4 iw = tam_p0_ld<NT>((const TamW4*)(A.idx + e0));
      uint32_t sc = A.scales[b];
      uint32_t sb = *(const uint16_t*)(A.signs + (e0 >> 3));
      uint32_t lb = A.labels[b];
      uint32_t nb = __float_as_uint(A.norms[b]);
      uint32_t am = A.amp[b];
      const uint32_t mix = sb ^ lb ^ nb ^ am ^ sc;
      p0 ^= g0 ^ mix;
      p1 ^= g1 ^ mix;
      iw ^= mix;
      tam_st_st<NT>((TamW4*)(A.param + e0), p0);
      tam_st_st<NT>((TamW4*)(A.param + e0) + 1, p1);
      tam_st_st<NT>((TamW4*)(A.idx + e0), iw);
      if ((lane & 7u) == 0) A.scales[b] = sc ^ 0x00010001u;
      if ((lane & 31u) == 0) A.partials[u * 2u + (lane >> 5)] = p0 ^ g1;
    } else {
      TamW4 pw[2], gw[2];
      TamW2 iw[2];
      uint32_t sc[2], mix[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const uint64_t e0 = u * 1024u + 512u * k + lane * 8u;
        const uint64_t b = u * 8u + 4u * k + (lane >> 4);
        pw[k] = tam_p0_ld<NT>((const TamW4*)(A.param + e0));
        gw[k] = tam_p0_ld<NT>((const TamW4*)(A.grad + e0));
        iw[k] = tam_p0_ld<NT>((const TamW2*)(A.idx + e0));
        sc[k] = A.scales[b];
        mix[k] = (uint32_t)A.signs[e0 >> 3] ^ A.labels[b] ^ __float_as_uint(A.norms[b]) ^ A.amp[b] ^ sc[k];
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const uint64_t e0 = u * 1024u + 512u * k + lane * 8u;
        const uint64_t b = u * 8u + 4u * k + (lane >> 4);
        tam_st_st<NT>((TamW4*)(A.param + e0), pw[k] ^ gw[k] ^ mix[k]);
        tam_st_st<NT>((TamW2*)(A.idx + e0), iw[k] ^ mix[k]);
        if ((lane & 15u) == 0) A.scales[b] = sc[k] ^ 0x00010001u;
      }
      if ((lane & 31u) == 0) A.partials[u * 2u + (lane >> 5)] = pw[0] ^ gw[1];
    }
  }
  if (threadIdx.x == WG) pad[0] = 0;  // never taken: keeps the dynamic LDS
}

template <int WG>
static void tam_p0_launch(int layout, int nt, dim3 grid, uint32_t lds, hipStream_t s, const TamP0Arrays& A,
                          uint64_t units) {
  if (layout == 0 && !nt) hipLaunchKernelGGL((tam_k_stream_pass0<WG, 0, false>), grid, dim3(WG), lds, s, A, units);
  else if (layout == 0) hipLaunchKernelGGL((tam_k_stream_pass0<WG, 0, true>), grid, dim3(WG), lds, s, A, units);
  else if (!nt) hipLaunchKernelGGL((tam_k_stream_pass0<WG, 1, false>), grid, dim3(WG), lds, s, A, units);
  else hipLaunchKernelGGL((tam_k_stream_pass0<WG, 1, true>), grid, dim3(WG), lds, s, A, units);
}

extern "C" {

static int tam_st_cus(void) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return -1;
  return cus;
}

// One launch over n16 16-byte words of each operand the kind uses (a, b and c
// each hold n16 words).  Grid: `rounds` times the workgroups that fill every CU
// with 32 waves (2048 threads), at most one thread per word; the loop covers
// the rest.  Returns the grid used, or a negative value on an invalid argument
// or a launch error.
long tam_stream_run(int kind, int nt, int words, int wg, int layout, void* a, const void* b, void* c, uint64_t n16,
                    int rounds, void* stream) {
  if (kind < TAM_ST_READ || kind > TAM_ST_INPLACE || n16 == 0 || rounds <= 0) return -1;
  if (!(words == 4 || words == 8 || words == 16) || !(wg == 256 || wg == 512 || wg == 1024)) return -1;
  if (layout < 0 || layout > 2) return -1;
  if (words == 16 && wg == 1024 && kind >= TAM_ST_COPY) return -1;  // needs more registers than 16 waves per CU allow
  const int cus = tam_st_cus();
  if (cus <= 0) return -2;
  const uint64_t want = (uint64_t)cus * (2048u / (uint64_t)wg) * (uint64_t)rounds;
  const uint64_t need = (n16 + wg - 1) / (uint64_t)wg;
  const uint32_t grid = (uint32_t)(want < need ? want : need);
  hipStream_t s = (hipStream_t)stream;
  TamW4* A = (TamW4*)a;
  const TamW4* B = (const TamW4*)b;
  TamW4* C = (TamW4*)c;
  switch (kind) {
    case TAM_ST_READ: tam_st_launch<TAM_ST_READ>(nt, words, wg, dim3(grid), s, A, B, C, n16, layout); break;
    case TAM_ST_WRITE: tam_st_launch<TAM_ST_WRITE>(nt, words, wg, dim3(grid), s, A, B, C, n16, layout); break;
    case TAM_ST_COPY: tam_st_launch<TAM_ST_COPY>(nt, words, wg, dim3(grid), s, A, B, C, n16, layout); break;
    case TAM_ST_ADD: tam_st_launch<TAM_ST_ADD>(nt, words, wg, dim3(grid), s, A, B, C, n16, layout); break;
    default: tam_st_launch<TAM_ST_INPLACE>(nt, words, wg, dim3(grid), s, A, B, C, n16, layout); break;
  }
  if (hipGetLastError() != hipSuccess) return -3;
  return (long)grid;
}

// Bytes of each pass-0-shaped array for `units` units of 1024 elements, in the
// order of TamP0Arrays (the caller allocates them, 256-byte aligned).
void tam_stream_pass0_sizes(uint64_t units, uint64_t* sizes) {
  const uint64_t n = units * 1024u, nb = units * 8u;
  sizes[0] = 2 * n;
  sizes[1] = 2 * n;
  sizes[2] = n;
  sizes[3] = 4 * nb;
  sizes[4] = n / 8;
  sizes[5] = nb;
  sizes[6] = 4 * nb;
  sizes[7] = 2 * nb;
  sizes[8] = 16 * (units * 2u);
}

// One launch of the pass-0-shaped stream: `wgs_per_cu` workgroups of wg
// threads per CU times `rounds` (a persistent grid: each wave strides over the
// units), each workgroup holding lds_bytes of LDS (to cap the waves a CU
// holds, as a kernel's register budget would); layout and nt as
// tam_k_stream_pass0's.  Returns the grid or < 0.
long tam_stream_pass0(void* const* arrays, uint64_t units, int wg, int wgs_per_cu, int rounds, uint32_t lds_bytes,
                      int layout, int nt, void* stream) {
  if (!arrays || units == 0 || !(wg == 128 || wg == 256) || wgs_per_cu <= 0 || rounds <= 0 || lds_bytes > 65536 ||
      layout < 0 || layout > 1)
    return -1;
  for (int i = 0; i < 9; ++i)
    if (!arrays[i] || ((uintptr_t)arrays[i] & 15u)) return -1;
  const int cus = tam_st_cus();
  if (cus <= 0) return -2;
  TamP0Arrays A;
  A.param = (uint16_t*)arrays[0];
  A.grad = (const uint16_t*)arrays[1];
  A.idx = (uint8_t*)arrays[2];
  A.scales = (uint32_t*)arrays[3];
  A.signs = (const uint8_t*)arrays[4];
  A.labels = (const uint8_t*)arrays[5];
  A.norms = (const float*)arrays[6];
  A.amp = (const uint16_t*)arrays[7];
  A.partials = (TamW4*)arrays[8];
  const uint32_t grid = (uint32_t)cus * (uint32_t)wgs_per_cu * (uint32_t)rounds;
  hipStream_t s = (hipStream_t)stream;
  if (wg == 128) tam_p0_launch<128>(layout, nt, dim3(grid), lds_bytes, s, A, units);
  else tam_p0_launch<256>(layout, nt, dim3(grid), lds_bytes, s, A, units);
  if (hipGetLastError() != hipSuccess) return -3;
  return (long)grid;
}

}  // extern "C"
