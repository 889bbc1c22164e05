// tam_stream.hip -- streaming kernels that measure the HBM bandwidth a plain
// memory-bound kernel reaches on this device (the practical ceiling that the
// step's kernels are compared against).  Measurement infrastructure for
// bench.py only: not part of the optimizer library or its ABI.
//
// Each kernel moves 16-byte words with a grid-stride loop, four words in
// flight per thread, optionally with nontemporal loads and stores (the `nt`
// bit: the data is not kept in the caches for reuse).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t TamW4 __attribute__((ext_vector_type(4)));

enum { TAM_ST_READ = 0, TAM_ST_WRITE = 1, TAM_ST_COPY = 2, TAM_ST_ADD = 3, TAM_ST_INPLACE = 4 };

template <bool NT>
__device__ __forceinline__ TamW4 tam_st_ld(const TamW4* p) {
  return NT ? __builtin_nontemporal_load(p) : *p;
}
template <bool NT>
__device__ __forceinline__ void tam_st_st(TamW4* p, TamW4 v) {
  if (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// kind READ:    x ^= a[i]; one word per thread written to c at the end
// kind WRITE:   c[i] = pattern
// kind COPY:    c[i] = a[i]
// kind ADD:     c[i] = a[i] + b[i]      (two reads, one write, three streams)
// kind INPLACE: a[i] = a[i] + b[i]      (read-modify-write of a, read of b)
template <int KIND, bool NT>
__global__ __launch_bounds__(256) void tam_k_stream(TamW4* a, const TamW4* b, TamW4* c, uint64_t n) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  TamW4 acc = {0u, 0u, 0u, 0u};
  for (; i + 3 * stride < n; i += 4 * stride) {
    TamW4 x[4], y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (KIND != TAM_ST_WRITE) x[k] = tam_st_ld<NT>(a + i + k * stride);
      if (KIND == TAM_ST_ADD || KIND == TAM_ST_INPLACE) y[k] = tam_st_ld<NT>(b + i + k * stride);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint64_t j = i + k * stride;
      if (KIND == TAM_ST_READ) acc ^= x[k];
      if (KIND == TAM_ST_WRITE) tam_st_st<NT>(c + j, TamW4{(uint32_t)j, 1u, 2u, 3u});
      if (KIND == TAM_ST_COPY) tam_st_st<NT>(c + j, x[k]);
      if (KIND == TAM_ST_ADD) tam_st_st<NT>(c + j, x[k] + y[k]);
      if (KIND == TAM_ST_INPLACE) tam_st_st<NT>(a + j, x[k] + y[k]);
    }
  }
  for (; i < n; i += stride) {
    if (KIND == TAM_ST_READ) acc ^= tam_st_ld<NT>(a + i);
    if (KIND == TAM_ST_WRITE) tam_st_st<NT>(c + i, TamW4{(uint32_t)i, 1u, 2u, 3u});
    if (KIND == TAM_ST_COPY) tam_st_st<NT>(c + i, tam_st_ld<NT>(a + i));
    if (KIND == TAM_ST_ADD) tam_st_st<NT>(c + i, tam_st_ld<NT>(a + i) + tam_st_ld<NT>(b + i));
    if (KIND == TAM_ST_INPLACE) tam_st_st<NT>(a + i, tam_st_ld<NT>(a + i) + tam_st_ld<NT>(b + i));
  }
  // one word per thread (c holds n words, as every operand)
  if (KIND == TAM_ST_READ) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < n) c[t] = acc;
  }
}

template <int KIND>
static void tam_st_launch(int nt, dim3 grid, hipStream_t s, TamW4* a, const TamW4* b, TamW4* c, uint64_t n) {
  if (nt) hipLaunchKernelGGL((tam_k_stream<KIND, true>), grid, dim3(256), 0, s, a, b, c, n);
  else hipLaunchKernelGGL((tam_k_stream<KIND, false>), grid, dim3(256), 0, s, a, b, c, n);
}

extern "C" {

// One launch over n16 16-byte words of each operand the kind uses (a, b and c
// each hold n16 words).  Grid: 8 workgroups per CU times `rounds`, at most one
// thread per word; the grid-stride loop covers the rest.  Returns the grid
// used, or a negative value on an invalid argument or a launch error.
long tam_stream_run(int kind, int nt, void* a, const void* b, void* c, uint64_t n16, int rounds, void* stream) {
  if (kind < TAM_ST_READ || kind > TAM_ST_INPLACE || n16 == 0 || rounds <= 0) return -1;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return -2;
  const uint64_t want = (uint64_t)cus * 8u * (uint64_t)rounds;  // 8 workgroups of 4 waves per CU
  const uint64_t need = (n16 + 255) / 256;
  const uint32_t grid = (uint32_t)(want < need ? want : need);
  hipStream_t s = (hipStream_t)stream;
  TamW4* A = (TamW4*)a;
  const TamW4* B = (const TamW4*)b;
  TamW4* C = (TamW4*)c;
  switch (kind) {
    case TAM_ST_READ: tam_st_launch<TAM_ST_READ>(nt, dim3(grid), s, A, B, C, n16); break;
    case TAM_ST_WRITE: tam_st_launch<TAM_ST_WRITE>(nt, dim3(grid), s, A, B, C, n16); break;
    case TAM_ST_COPY: tam_st_launch<TAM_ST_COPY>(nt, dim3(grid), s, A, B, C, n16); break;
    case TAM_ST_ADD: tam_st_launch<TAM_ST_ADD>(nt, dim3(grid), s, A, B, C, n16); break;
    default: tam_st_launch<TAM_ST_INPLACE>(nt, dim3(grid), s, A, B, C, n16); break;
  }
  if (hipGetLastError() != hipSuccess) return -3;
  return (long)grid;
}

}  // extern "C"
