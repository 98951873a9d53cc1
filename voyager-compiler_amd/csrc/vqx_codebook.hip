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

// Monotone 16-bit key of a bf16 pattern: key order = value order (-0 just
// below +0, both compare equal as values), NaN patterns above +Inf.
__device__ __forceinline__ uint32_t bf16_key(uint32_t h) { return (h & 0x8000u) ? (h ^ 0xFFFFu) : (h | 0x8000u); }
__device__ __forceinline__ uint32_t key_bf16(uint32_t k) { return (k & 0x8000u) ? (k & 0x7FFFu) : (k ^ 0xFFFFu); }

// The code of a bf16 value under the row's codebook is non-decreasing in the
// value, so it is the number of decision thresholds at or below its key:
// t[i] = the smallest key whose code exceeds i (i = 0 .. K-2).  With a =
// cb[i] and b the first later entry above a (duplicates of a never win: the
// lowest index does), code(v) > i exactly when fp32 |b - v| < |v - a|, i.e.
// fl(b - v) < fl(v - a), also outside [a, b] (and for the clamped values
// beyond the codebook's ends); that predicate is monotone in v, so t[i] is a
// binary search over the bf16 keys around [a, b].  No later entry above a:
// no threshold (0x10000, above every key).
__device__ uint32_t code_threshold(const float* cb, int K, int i) {
  const float a = cb[i];
  int j = i + 1;
  while (j < K && !(cb[j] > a)) ++j;
  if (j == K) return 0x10000u;
  const float b = cb[j];
  auto closer_to_b = [&](int k) {
    float v = bf2f(key_bf16((uint32_t)k));
    return (b - v) < (v - a);
  };
  // closer_to_b(lo) is false (lo is below a), closer_to_b(hi) true (above b)
  int lo = (int)bf16_key(f2bf(a)) - 2, hi = (int)bf16_key(f2bf(b)) + 2;
  lo = lo < 0x7F ? 0x7F : lo;        // -Inf
  hi = hi > 0xFF80 ? 0xFF80 : hi;    // +Inf
  while (lo + 1 < hi) {
    int mid = (lo + hi) >> 1;
    if (closer_to_b(mid)) hi = mid; else lo = mid;
  }
  return (uint32_t)hi;
}

// Lane-interleaved streaming: a wave's chunk is 64 lanes x 16 consecutive
// elements taken as 4 sub-chunks of 64 x 4, so each load / store instruction
// of the wave covers one contiguous span.
constexpr int kCbChunk = 1024;  // elements per wave chunk

// Per-channel encode: one workgroup per row (grid-stride over rows); the
// row's sorted thresholds (padded with ~0 to a power of two P) in LDS; per
// element the bf16 key and a branch-free search of log2(P) steps.
template <typename T>
__global__ __launch_bounds__(256) void cb_encode_kernel(const T* __restrict__ x, int64_t rows, int64_t cols,
                                                        const float* __restrict__ cb, int K, int P,
                                                        uint8_t* __restrict__ codes) {
  extern __shared__ float s_cb[];               // K fp32 entries, then P uint32 thresholds
  uint32_t* s_t = reinterpret_cast<uint32_t*>(s_cb + K);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    __syncthreads();
    for (int k = threadIdx.x; k < K; k += blockDim.x) s_cb[k] = cb[r * K + k];
    __syncthreads();
    for (int k = threadIdx.x; k < P; k += blockDim.x) s_t[k] = k < K - 1 ? code_threshold(s_cb, K, k) : 0xFFFFFFFFu;
    __syncthreads();
    const T* xr = x + r * cols;
    uint8_t* cr = codes + r * cols;
    auto encode = [&](float v) -> uint32_t {
      uint32_t key = bf16_key(f2bf(v));
      uint32_t pos = 0;
      for (int step = P >> 1; step > 0; step >>= 1) pos += s_t[pos + step - 1] <= key ? step : 0;
      return v != v ? 0u : pos;
    };
    int64_t full = cols / kCbChunk * kCbChunk;
    for (int64_t base = (int64_t)wave * kCbChunk; base < full; base += (int64_t)nwaves * kCbChunk) {
      float v[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t e = base + q * 256 + lane * 4;
        if constexpr (std::is_same<T, float>::value) {
          f32x4 a = ld_nt(reinterpret_cast<const f32x4*>(xr + e));
          v[4 * q] = a.x; v[4 * q + 1] = a.y; v[4 * q + 2] = a.z; v[4 * q + 3] = a.w;
        } else {
          u32x2 a = ld_nt(reinterpret_cast<const u32x2*>(xr + e));
          v[4 * q] = u2f(a.x << 16); v[4 * q + 1] = u2f(a.x & 0xFFFF0000u);
          v[4 * q + 2] = u2f(a.y << 16); v[4 * q + 3] = u2f(a.y & 0xFFFF0000u);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t c0 = encode(v[4 * q]), c1 = encode(v[4 * q + 1]), c2 = encode(v[4 * q + 2]),
                 c3 = encode(v[4 * q + 3]);
        __builtin_nontemporal_store(c0 | (c1 << 8) | (c2 << 16) | (c3 << 24),
                                    reinterpret_cast<uint32_t*>(cr + base + q * 256 + lane * 4));
      }
    }
    for (int64_t i = full + threadIdx.x; i < cols; i += blockDim.x) {
      float xv = std::is_same<T, float>::value ? (float)xr[i] : u2f((uint32_t)((const uint16_t*)xr)[i] << 16);
      cr[i] = (uint8_t)encode(xv);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void cb_decode_kernel(const uint8_t* __restrict__ codes, int64_t rows,
                                                        int64_t cols, const float* __restrict__ cb, int K,
                                                        T* __restrict__ out) {
  extern __shared__ float s_cb[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    __syncthreads();
    for (int k = threadIdx.x; k < K; k += blockDim.x) s_cb[k] = bf2f(f2bf(cb[r * K + k]));
    __syncthreads();
    const uint8_t* cr = codes + r * cols;
    T* orow = out + r * cols;
    auto value = [&](uint32_t c) { return s_cb[c < (uint32_t)K ? c : K - 1]; };
    int64_t full = cols / kCbChunk * kCbChunk;
    for (int64_t base = (int64_t)wave * kCbChunk; base < full; base += (int64_t)nwaves * kCbChunk) {
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) w[q] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(cr + base + q * 256 + lane * 4));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v0 = value(w[q] & 0xFFu), v1 = value((w[q] >> 8) & 0xFFu), v2 = value((w[q] >> 16) & 0xFFu),
              v3 = value(w[q] >> 24);
        const int64_t e = base + q * 256 + lane * 4;
        if constexpr (std::is_same<T, float>::value) {
          st_nt(reinterpret_cast<f32x4*>(orow + e), f32x4{v0, v1, v2, v3});
        } else {
          u32x2 a = {(f2u(v0) >> 16) | (f2u(v1) & 0xFFFF0000u), (f2u(v2) >> 16) | (f2u(v3) & 0xFFFF0000u)};
          st_nt(reinterpret_cast<u32x2*>(orow + e), a);
        }
      }
    }
    for (int64_t i = full + threadIdx.x; i < cols; i += blockDim.x) {
      float v = value(cr[i]);
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
  int P = 1;
  while (P < K) P <<= 1;  // K - 1 thresholds padded to a power of two >= K (codes up to P - 1)
  size_t lds = sizeof(float) * K + sizeof(uint32_t) * P;
  if (dtype == kF32)
    hipLaunchKernelGGL((cb_encode_kernel<float>), dim3(grid), dim3(256), lds, st, (const float*)x, rows, cols,
                       cb, K, P, codes);
  else if (dtype == kBF16)
    hipLaunchKernelGGL((cb_encode_kernel<uint16_t>), dim3(grid), dim3(256), lds, st, (const uint16_t*)x,
                       rows, cols, cb, K, P, codes);
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
