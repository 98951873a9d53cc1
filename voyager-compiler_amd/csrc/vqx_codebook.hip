// Per-channel codebook encode/decode.  Row r of x (a channel) has its own
// sorted codebook cb[r, 0..K-1].  Encode follows the reference's codebook
// table rule (quantization/lcq.py:286-291) applied per row: the input is taken
// at its bf16 value (vmap's cast, ops/quantized.py:107-108), clamped to
// [cb[0], cb[K-1]], and the index of the nearest entry under fp32 |x - c| is
// returned, the lowest index on ties; NaN gives 0.  Decode returns
// float(bf16(cb[r, code])), the table value the reference stores.
#include "vqx_kernels.h"

namespace vqx {

// Exact nearest-entry search in a sorted LDS codebook.  For a sorted codebook
// fl(|v - c_i|) is non-increasing over entries below v and non-decreasing over
// entries above it, so the minimum sits at the bracketing pair; the lowest
// index among equal minima is found by walking left while the rounded
// distance stays equal (almost never more than zero steps).
__device__ __forceinline__ uint32_t nearest_sorted(const float* cb, int K, float v) {
  if (v != v) return 0;
  v = v < cb[0] ? cb[0] : v;
  v = v > cb[K - 1] ? cb[K - 1] : v;
  // lower_bound: first index with cb[i] >= v
  int lo = 0, len = K;
  while (len > 0) {
    int half = len >> 1;
    bool lt = cb[lo + half] < v;
    lo = lt ? lo + half + 1 : lo;
    len = lt ? len - half - 1 : half;
  }
  if (lo == 0) return 0;  // v == cb[0]
  float dl = v - cb[lo - 1];
  float dr = lo < K ? cb[lo] - v : __builtin_huge_valf();
  if (dr < dl) return (uint32_t)lo;
  int i = lo - 1;
  while (i > 0 && v - cb[i - 1] == dl) --i;
  return (uint32_t)i;
}

// One workgroup per row (grid-stride over rows); the row's codebook in LDS;
// each thread encodes 16 consecutive elements per step.
template <typename T>
__global__ __launch_bounds__(256) void cb_encode_kernel(const T* __restrict__ x, int64_t rows, int64_t cols,
                                                        const float* __restrict__ cb, int K,
                                                        uint8_t* __restrict__ codes) {
  extern __shared__ float s_cb[];
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    __syncthreads();
    for (int k = threadIdx.x; k < K; k += blockDim.x) s_cb[k] = cb[r * K + k];
    __syncthreads();
    const T* xr = x + r * cols;
    uint8_t* cr = codes + r * cols;
    int64_t ng = cols / 16;
    for (int64_t g = threadIdx.x; g < ng; g += blockDim.x) {
      float v[16];
      if constexpr (std::is_same<T, float>::value) {
        const f32x4* q = reinterpret_cast<const f32x4*>(xr + g * 16);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          f32x4 a = ld_nt(q + k);
          v[4 * k] = a.x; v[4 * k + 1] = a.y; v[4 * k + 2] = a.z; v[4 * k + 3] = a.w;
        }
      } else {
        const u32x4* q = reinterpret_cast<const u32x4*>(xr + g * 16);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          u32x4 a = ld_nt(q + k);
          uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            v[8 * k + 2 * j] = u2f(w[j] << 16);
            v[8 * k + 2 * j + 1] = u2f(w[j] & 0xFFFF0000u);
          }
        }
      }
      uint32_t c[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) c[j] = nearest_sorted(s_cb, K, bf2f(f2bf(v[j])));
      u32x4 w;
      w.x = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
      w.y = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
      w.z = c[8] | (c[9] << 8) | (c[10] << 16) | (c[11] << 24);
      w.w = c[12] | (c[13] << 8) | (c[14] << 16) | (c[15] << 24);
      st_nt(reinterpret_cast<u32x4*>(cr + g * 16), w);
    }
    for (int64_t i = ng * 16 + threadIdx.x; i < cols; i += blockDim.x) {
      float xv = std::is_same<T, float>::value ? (float)xr[i] : u2f((uint32_t)((const uint16_t*)xr)[i] << 16);
      cr[i] = (uint8_t)nearest_sorted(s_cb, K, bf2f(f2bf(xv)));
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void cb_decode_kernel(const uint8_t* __restrict__ codes, int64_t rows,
                                                        int64_t cols, const float* __restrict__ cb, int K,
                                                        T* __restrict__ out) {
  extern __shared__ float s_cb[];
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    __syncthreads();
    for (int k = threadIdx.x; k < K; k += blockDim.x) s_cb[k] = bf2f(f2bf(cb[r * K + k]));
    __syncthreads();
    const uint8_t* cr = codes + r * cols;
    T* orow = out + r * cols;
    int64_t ng = cols / 16;
    for (int64_t g = threadIdx.x; g < ng; g += blockDim.x) {
      u32x4 w = ld_nt(reinterpret_cast<const u32x4*>(cr + g * 16));
      uint32_t ww[4] = {w.x, w.y, w.z, w.w};
      float v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        uint32_t c = (ww[j >> 2] >> (8 * (j & 3))) & 0xFFu;
        v[j] = s_cb[c < (uint32_t)K ? c : K - 1];
      }
      if constexpr (std::is_same<T, float>::value) {
        f32x4* q = reinterpret_cast<f32x4*>(orow + g * 16);
#pragma unroll
        for (int k = 0; k < 4; ++k) st_nt(q + k, f32x4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]});
      } else {
        u32x4* q = reinterpret_cast<u32x4*>(orow + g * 16);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          u32x4 a;
          a.x = (f2u(v[8 * k]) >> 16) | (f2u(v[8 * k + 1]) & 0xFFFF0000u);
          a.y = (f2u(v[8 * k + 2]) >> 16) | (f2u(v[8 * k + 3]) & 0xFFFF0000u);
          a.z = (f2u(v[8 * k + 4]) >> 16) | (f2u(v[8 * k + 5]) & 0xFFFF0000u);
          a.w = (f2u(v[8 * k + 6]) >> 16) | (f2u(v[8 * k + 7]) & 0xFFFF0000u);
          st_nt(q + k, a);
        }
      }
    }
    for (int64_t i = ng * 16 + threadIdx.x; i < cols; i += blockDim.x) {
      uint32_t c = cr[i];
      float v = s_cb[c < (uint32_t)K ? c : K - 1];
      if constexpr (std::is_same<T, float>::value) orow[i] = v;
      else ((uint16_t*)orow)[i] = (uint16_t)(f2u(v) >> 16);
    }
  }
}

int codebook_encode(const void* x, int dtype, int64_t rows, int64_t cols, const float* cb, int K,
                    uint8_t* codes, hipStream_t st) {
  if (K < 1 || K > 256) return set_error(kErrInvalid, "codebook size %d outside [1,256]", K);
  if (rows < 0 || cols < 0) return set_error(kErrInvalid, "negative shape");
  if (rows == 0 || cols == 0) return kOk;
  if (!aligned(x, 16) || !aligned(codes, 16) || (cols % 16) != 0)
    return set_error(kErrInvalid, "codebook encode needs 16-byte aligned rows (cols %% 16 == 0)");
  unsigned grid = (unsigned)(rows < (int64_t)num_cus() * 8 ? rows : (int64_t)num_cus() * 8);
  size_t lds = sizeof(float) * K;
  if (dtype == kF32)
    hipLaunchKernelGGL((cb_encode_kernel<float>), dim3(grid), dim3(256), lds, st, (const float*)x, rows, cols,
                       cb, K, codes);
  else if (dtype == kBF16)
    hipLaunchKernelGGL((cb_encode_kernel<uint16_t>), dim3(grid), dim3(256), lds, st, (const uint16_t*)x,
                       rows, cols, cb, K, codes);
  else
    return set_error(kErrInvalid, "codebook input dtype %d not supported", dtype);
  return check_launch("codebook_encode");
}

int codebook_decode(const uint8_t* codes, int64_t rows, int64_t cols, const float* cb, int K, void* out,
                    int dtype, hipStream_t st) {
  if (K < 1 || K > 256) return set_error(kErrInvalid, "codebook size %d outside [1,256]", K);
  if (rows < 0 || cols < 0) return set_error(kErrInvalid, "negative shape");
  if (rows == 0 || cols == 0) return kOk;
  if (!aligned(out, 16) || !aligned(codes, 16) || (cols % 16) != 0)
    return set_error(kErrInvalid, "codebook decode needs 16-byte aligned rows (cols %% 16 == 0)");
  unsigned grid = (unsigned)(rows < (int64_t)num_cus() * 8 ? rows : (int64_t)num_cus() * 8);
  size_t lds = sizeof(float) * K;
  if (dtype == kF32)
    hipLaunchKernelGGL((cb_decode_kernel<float>), dim3(grid), dim3(256), lds, st, codes, rows, cols, cb, K,
                       (float*)out);
  else if (dtype == kBF16)
    hipLaunchKernelGGL((cb_decode_kernel<uint16_t>), dim3(grid), dim3(256), lds, st, codes, rows, cols, cb,
                       K, (uint16_t*)out);
  else
    return set_error(kErrInvalid, "codebook output dtype %d not supported", dtype);
  return check_launch("codebook_decode");
}

}  // namespace vqx
