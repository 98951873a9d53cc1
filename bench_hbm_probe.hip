// HBM bandwidth probe by traffic mix, for bench.py --hbm-ceiling: not part of
// the quantization library.  `python bench.py --build-probe` compiles it into
// bench_hbm_probe.so beside this file.
//
// Each unit of work reads r 16-byte chunks and writes w 16-byte chunks.
// Chunk j of unit u is at byte 16 (j * units + u) of its buffer, so every
// read stream and every write stream is contiguous across lanes (one 1 KiB
// run per wave instruction).  Stores are non-temporal, loads non-temporal or
// plain (NT); the written value is the XOR of the unit's reads (and of u), so
// nothing is dead code.
// With w = 0 each thread XORs its reads into one word of `sink`.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int R, int W, bool NT>
__global__ __launch_bounds__(256) void hbm_mix_kernel(const u32x4* __restrict__ a, u32x4* __restrict__ b,
                                                      int64_t units, uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units; u += stride) {
    u32x4 x = {(uint32_t)u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < R; ++j) x ^= NT ? __builtin_nontemporal_load(a + (int64_t)j * units + u) : a[(int64_t)j * units + u];
#pragma unroll
    for (int j = 0; j < W; ++j) __builtin_nontemporal_store(x ^ (uint32_t)j, b + (int64_t)j * units + u);
    if (W == 0) acc ^= x;
  }
  if (W == 0) sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

template <int R, int W>
static void launch(const void* a, void* b, int64_t units, uint32_t* sink, int grid, bool nt, hipStream_t st) {
  if (nt)
    hipLaunchKernelGGL((hbm_mix_kernel<R, W, true>), dim3(grid), dim3(256), 0, st, (const u32x4*)a, (u32x4*)b, units,
                       sink);
  else
    hipLaunchKernelGGL((hbm_mix_kernel<R, W, false>), dim3(grid), dim3(256), 0, st, (const u32x4*)a, (u32x4*)b, units,
                       sink);
}

// a: r * units * 16 bytes, b: w * units * 16 bytes, sink: grid * 256 words;
// nt: non-temporal loads (1) or plain loads (0).
// Returns 0, or -1 for an unsupported (r, w).
extern "C" int vqx_probe_hbm_mix_loads(const void* a, void* b, int64_t units, int r, int w, void* sink, int grid,
                                       int nt, hipStream_t st) {
  uint32_t* s = (uint32_t*)sink;
  const bool n = nt != 0;
  if (r == 1 && w == 0) launch<1, 0>(a, b, units, s, grid, n, st);
  else if (r == 0 && w == 1) launch<0, 1>(a, b, units, s, grid, n, st);
  else if (r == 1 && w == 1) launch<1, 1>(a, b, units, s, grid, n, st);
  else if (r == 2 && w == 1) launch<2, 1>(a, b, units, s, grid, n, st);
  else if (r == 4 && w == 1) launch<4, 1>(a, b, units, s, grid, n, st);
  else if (r == 1 && w == 2) launch<1, 2>(a, b, units, s, grid, n, st);
  else if (r == 1 && w == 4) launch<1, 4>(a, b, units, s, grid, n, st);
  else return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// The same with non-temporal loads.
extern "C" int vqx_probe_hbm_mix(const void* a, void* b, int64_t units, int r, int w, void* sink, int grid,
                                 hipStream_t st) {
  return vqx_probe_hbm_mix_loads(a, b, units, r, w, sink, grid, 1, st);
}
