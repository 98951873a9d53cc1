// Elementwise kernels: the LUT gather behind quantized_ops::vmap, the
// closed-form per-tensor fake-quant (FakeQuantizeFunction) with optional
// format codes, and the setup kernels that tabulate a format over all 2^16
// bf16 patterns (get_quantization_map) and derive level-set boundaries.
#include <math.h>

#include <type_traits>

#include "vqx_kernels.h"

namespace vqx {

// ---------------------------------------------------------------------------
// element access by dtype
// ---------------------------------------------------------------------------
template <typename T>
struct IO;

template <>
struct IO<float> {
  static constexpr int kVec = 8;  // elements per thread per step (2 x 16 B)
  __device__ static void load(const float* p, float (&v)[8]) {
    f32x4 a = ld_nt(reinterpret_cast<const f32x4*>(p));
    f32x4 b = ld_nt(reinterpret_cast<const f32x4*>(p) + 1);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  __device__ static void store(float* p, const float (&v)[8]) {
    f32x4 a = {v[0], v[1], v[2], v[3]};
    f32x4 b = {v[4], v[5], v[6], v[7]};
    st_nt(reinterpret_cast<f32x4*>(p), a);
    st_nt(reinterpret_cast<f32x4*>(p) + 1, b);
  }
  __device__ static float get(const float* p) { return *p; }
  __device__ static void put(float* p, float v) { *p = v; }
};

template <>
struct IO<uint16_t> {  // bf16 stored as raw bits
  static constexpr int kVec = 8;  // 1 x 16 B
  __device__ static void load(const uint16_t* p, float (&v)[8]) {
    u32x4 a = ld_nt(reinterpret_cast<const u32x4*>(p));
    uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = u2f(w[j] << 16);
      v[2 * j + 1] = u2f(w[j] & 0xFFFF0000u);
    }
  }
  // values already rounded to bf16 (their low 16 bits are zero)
  __device__ static void store(uint16_t* p, const float (&v)[8]) {
    u32x4 a;
    a.x = (f2u(v[0]) >> 16) | (f2u(v[1]) & 0xFFFF0000u);
    a.y = (f2u(v[2]) >> 16) | (f2u(v[3]) & 0xFFFF0000u);
    a.z = (f2u(v[4]) >> 16) | (f2u(v[5]) & 0xFFFF0000u);
    a.w = (f2u(v[6]) >> 16) | (f2u(v[7]) & 0xFFFF0000u);
    st_nt(reinterpret_cast<u32x4*>(p), a);
  }
  __device__ static float get(const uint16_t* p) { return u2f((uint32_t)*p << 16); }
  __device__ static void put(uint16_t* p, float v) { *p = (uint16_t)(f2u(v) >> 16); }
};

template <>
struct IO<__half> {
  static constexpr int kVec = 8;
  __device__ static void load(const __half* p, float (&v)[8]) {
    u32x4 a = ld_nt(reinterpret_cast<const u32x4*>(p));
    uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = h2f_exact(w[j] & 0xFFFFu);
      v[2 * j + 1] = h2f_exact(w[j] >> 16);
    }
  }
  __device__ static void store(__half* p, const float (&v)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = f2h_exact(v[2 * j]) | (f2h_exact(v[2 * j + 1]) << 16);
    u32x4 a = {w[0], w[1], w[2], w[3]};
    st_nt(reinterpret_cast<u32x4*>(p), a);
  }
  __device__ static float get(const __half* p) {
    return h2f_exact(*reinterpret_cast<const uint16_t*>(p));
  }
  __device__ static void put(__half* p, float v) {
    *reinterpret_cast<uint16_t*>(p) = (uint16_t)f2h_exact(v);
  }
};

// Rounding of a float to the input dtype, as torch stores an op result.
template <typename T>
__device__ __forceinline__ float to_dtype(float v);
template <>
__device__ __forceinline__ float to_dtype<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_dtype<uint16_t>(float v) { return bf2f(f2bf(v)); }
template <>
__device__ __forceinline__ float to_dtype<__half>(float v) {
  return h2f_exact(f2h_exact(v));
}

// One element of FakeQuantizeFunction.forward (fake_quantize.py:112-115):
//   s = scale.to(x.dtype);  y = vmap(x / s, qmap) * s
// where every op rounds to x's dtype and vmap first casts to bf16
// (quantized.py:107-108).  unit: s == 1, so the division and product are
// identities and are skipped; a bf16 input then indexes the table with its
// raw bits and the table entry is stored as is, like the reference's gather.
template <typename T, typename Enc>
__device__ __forceinline__ float fq_one(float x, float s, bool unit, bool mul, const Enc& enc,
                                        uint32_t& code) {
  constexpr bool kBf16 = std::is_same<T, uint16_t>::value;
  uint32_t h;
  if (unit)
    h = kBf16 ? (f2u(x) >> 16) : f2bf(x);
  else
    h = f2bf(to_dtype<T>(x / s));
  Result r = enc.encode(h);
  code = r.code;
  if (unit) return kBf16 ? u2f(r.value << 16) : to_dtype<T>(bf2f(r.value));
  float v = to_dtype<T>(bf2f(r.value));
  return mul ? to_dtype<T>(v * s) : v;
}

template <int CB>
__device__ __forceinline__ void store_codes8(void* codes, int64_t i, const uint32_t (&c)[8]) {
  if constexpr (CB == 1) {
    u32x2 w;
    w.x = (c[0] & 0xFF) | ((c[1] & 0xFF) << 8) | ((c[2] & 0xFF) << 16) | (c[3] << 24);
    w.y = (c[4] & 0xFF) | ((c[5] & 0xFF) << 8) | ((c[6] & 0xFF) << 16) | (c[7] << 24);
    st_nt(reinterpret_cast<u32x2*>(static_cast<uint8_t*>(codes) + i), w);
  } else if constexpr (CB == 2) {
    u32x4 w;
    w.x = (c[0] & 0xFFFF) | (c[1] << 16);
    w.y = (c[2] & 0xFFFF) | (c[3] << 16);
    w.z = (c[4] & 0xFFFF) | (c[5] << 16);
    w.w = (c[6] & 0xFFFF) | (c[7] << 16);
    st_nt(reinterpret_cast<u32x4*>(static_cast<uint16_t*>(codes) + i), w);
  }
}

template <int CB>
__device__ __forceinline__ void store_code1(void* codes, int64_t i, uint32_t c) {
  if constexpr (CB == 1) static_cast<uint8_t*>(codes)[i] = (uint8_t)c;
  if constexpr (CB == 2) static_cast<uint16_t*>(codes)[i] = (uint16_t)c;
}

// Per-tensor (C == 1) fake-quant, 8 elements per thread per step, 16-byte
// streaming loads/stores.  x, y 16-byte aligned; codes 8 (CB=1) or 16 (CB=2)
// byte aligned; the < 8-element tail is done one element per thread.
template <typename T, typename Enc, int CB>
__global__ __launch_bounds__(256) void fq_vec_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                     void* __restrict__ codes, int64_t n,
                                                     const float* __restrict__ scale, bool mul, Enc enc) {
  float s = scale ? scale[0] : 1.0f;
  s = to_dtype<T>(s);
  bool unit = s == 1.0f;
  const int64_t nvec = n / 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < nvec; g += stride) {
    float v[8];
    uint32_t c[8];
    IO<T>::load(x + g * 8, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = fq_one<T>(v[j], s, unit, mul, enc, c[j]);
    if (y) IO<T>::store(y + g * 8, v);
    if constexpr (CB > 0) store_codes8<CB>(codes, g * 8, c);
  }
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t i = nvec * 8 + t;
  if (i < n) {
    uint32_t c;
    float v = fq_one<T>(IO<T>::get(x + i), s, unit, mul, enc, c);
    if (y) IO<T>::put(y + i, v);
    if constexpr (CB > 0) store_code1<CB>(codes, i, c);
  }
}

// Table path of the per-tensor fake-quant: the format comes from the
// compact LDS table (magnitudes >= S from the full table in global memory).
typedef __attribute__((address_space(3))) const uint32_t lds_cu32;

// Unit scale, per group of 8: when no magnitude reaches the table's special
// threshold S, each element is its magnitude clamped into [T0 - 1, T1] with
// v_med3_f32 (clamping before the bf16 rounding equals clamping after it, the
// bounds being bf16 values), RNE to bf16, one compare against a uniform
// threshold for the sign, and one LDS read giving value and code together.
// Other groups, and every group under a non-unit scale, take the exact
// per-element route (IEEE division, full table beyond S).
// 1024 threads: sixteen waves share one copy of the table, which a 27 KB
// posit8 table would otherwise limit to six workgroups of four waves per CU,
// and each workgroup's fill serves four times the waves (C1 28.4 us with 256
// threads, 27.0-27.5 with 512, 26.2-26.5 with 1024)
constexpr int kFqLutThreads = 1024;

template <typename T, int CB>
__global__ __launch_bounds__(kFqLutThreads) void fq_lut_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                     void* __restrict__ codes, int64_t n,
                                                     const float* __restrict__ scale, bool mul, LutView lv) {
  extern __shared__ uint32_t lds_lut[];
  constexpr bool kBf16 = std::is_same<T, uint16_t>::value;
  constexpr bool kF32 = std::is_same<T, float>::value;
  const int64_t nvec = n / 8;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int lane = threadIdx.x & 63;
  int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  // Element offsets of thread group gg's two 4-element halves.  fp32 is
  // lane-interleaved within a whole wave (lane L: 4 L and 256 + 4 L of the
  // wave's 512 elements), so each 16-byte load / store instruction of the
  // wave covers one contiguous span; 2-byte types already do (one 16-byte
  // access per lane).
  auto halves = [&](int64_t gg, int64_t& e0, int64_t& e1) {
    e0 = gg * 8;
    e1 = e0 + 4;
    if constexpr (kF32) {
      const int64_t w0 = gg - lane;
      if (w0 + 64 <= nvec) {
        e0 = w0 * 8 + lane * 4;
        e1 = e0 + 256;
      }
    }
  };
  auto load8 = [&](int64_t gg, float (&v)[8]) {
    if constexpr (kF32) {
      int64_t e0, e1;
      halves(gg, e0, e1);
      // non-temporal loads: 28.7 -> 27.8 us at C1 with the input streaming
      // from HBM (plain loads won only with the input left in the MALL)
      f32x4 a = ld_nt(reinterpret_cast<const f32x4*>(x + e0)), b = ld_nt(reinterpret_cast<const f32x4*>(x + e1));
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      IO<T>::load(x + gg * 8, v);
    }
  };
  float nxt[8];
  if (g < nvec) load8(g, nxt);  // in flight while the table fills LDS
  LutLds t = lut_to_lds(lv.blob, lv.len, lds_lut);
  const uint32_t* full = lv.blob + kLutHeaderWords + 2 * kLutMaxLen;
  // LDS byte addresses such that entry(h) = base + 4 h for h in [T0 - 1, T1]
  const uint32_t pb = (uint32_t)(size_t)(lds_cu32*)lds_lut - 4u * t.t0m1;
  const uint32_t nb = pb + 4u * t.len;
  const float lo = u2f(t.t0m1 << 16), hi = u2f(t.t1 << 16);
  const uint32_t big = (t.s - 1u) << 16;  // magnitudes (fp32 bits) from here: exact route
  // x rounds to a bf16 below -0 iff x < -2^-134, to -0 or below iff x < 0
  const uint32_t nthr = t.zsign ? 0x7FFFFFFFu : 0x80008000u;
  float s = scale ? scale[0] : 1.0f;
  s = to_dtype<T>(s);
  const bool unit = s == 1.0f;
  // a normal lower bound keeps the clamp and the rounding free of subnormals
  const bool clamp_ok = unit && t.t0m1 >= 0x80u;
  for (; g < nvec; g += stride) {
    float v[8];
    uint32_t c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = nxt[j];
    if (g + stride < nvec) load8(g + stride, nxt);
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = umax32(m, f2u(v[j]) & 0x7FFFFFFFu);
    if (clamp_ok && m < big) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float qc = __builtin_amdgcn_fmed3f(__builtin_fabsf(v[j]), lo, hi);
        uint32_t h = kBf16 ? f2u(qc) >> 16 : pack_bf16x2(qc, 0.0f);
        uint32_t e = *(lds_cu32*)(size_t)((f2u(v[j]) > nthr ? nb : pb) + 4u * h);
        c[j] = e >> 16;
        float q = u2f(e << 16);
        v[j] = kBf16 ? q : to_dtype<T>(q);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t h;
        if (unit)
          h = kBf16 ? (f2u(v[j]) >> 16) : f2bf(v[j]);
        else
          h = f2bf(to_dtype<T>(v[j] / s));
        uint32_t e = (h & 0x7FFFu) < t.s ? lut_entry(t, h) : full[h];
        c[j] = e >> 16;
        float q = u2f(e << 16);
        v[j] = unit ? (kBf16 ? q : to_dtype<T>(q)) : (mul ? to_dtype<T>(to_dtype<T>(q) * s) : to_dtype<T>(q));
      }
    }
    if constexpr (kF32) {
      int64_t e0, e1;
      halves(g, e0, e1);
      if (y) {
        st_nt(reinterpret_cast<f32x4*>(y + e0), f32x4{v[0], v[1], v[2], v[3]});
        st_nt(reinterpret_cast<f32x4*>(y + e1), f32x4{v[4], v[5], v[6], v[7]});
      }
      if constexpr (CB == 1) {
        uint8_t* cb8 = static_cast<uint8_t*>(codes);
        __builtin_nontemporal_store((c[0] & 0xFF) | ((c[1] & 0xFF) << 8) | ((c[2] & 0xFF) << 16) | (c[3] << 24),
                                    reinterpret_cast<uint32_t*>(cb8 + e0));
        __builtin_nontemporal_store((c[4] & 0xFF) | ((c[5] & 0xFF) << 8) | ((c[6] & 0xFF) << 16) | (c[7] << 24),
                                    reinterpret_cast<uint32_t*>(cb8 + e1));
      } else if constexpr (CB == 2) {
        uint16_t* cb16 = static_cast<uint16_t*>(codes);
        st_nt(reinterpret_cast<u32x2*>(cb16 + e0), u32x2{(c[0] & 0xFFFF) | (c[1] << 16), (c[2] & 0xFFFF) | (c[3] << 16)});
        st_nt(reinterpret_cast<u32x2*>(cb16 + e1), u32x2{(c[4] & 0xFFFF) | (c[5] << 16), (c[6] & 0xFFFF) | (c[7] << 16)});
      }
    } else {
      if (y) IO<T>::store(y + g * 8, v);
      if constexpr (CB > 0) store_codes8<CB>(codes, g * 8, c);
    }
  }
  int64_t i = nvec * 8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    float xv = IO<T>::get(x + i);
    uint32_t h = unit ? (kBf16 ? (f2u(xv) >> 16) : f2bf(xv)) : f2bf(to_dtype<T>(xv / s));
    uint32_t e = full[h];
    float q = u2f(e << 16);
    float r = unit ? (kBf16 ? q : to_dtype<T>(q)) : (mul ? to_dtype<T>(to_dtype<T>(q) * s) : to_dtype<T>(q));
    if (y) IO<T>::put(y + i, r);
    if constexpr (CB > 0) store_code1<CB>(codes, i, e >> 16);
  }
}

// General path: any alignment, per-channel scales (channel of element i is
// (i / inner) % C).
template <typename T, typename Enc, int CB>
__global__ __launch_bounds__(256) void fq_scalar_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                        void* __restrict__ codes, int64_t n,
                                                        const float* __restrict__ scale,
                                                        int64_t inner, int64_t C, bool mul, Enc enc) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float s = 1.0f;
    if (scale) s = scale[C > 1 ? (i / inner) % C : 0];
    s = to_dtype<T>(s);
    uint32_t c;
    float v = fq_one<T>(IO<T>::get(x + i), s, s == 1.0f, mul, enc, c);
    if (y) IO<T>::put(y + i, v);
    if constexpr (CB > 0) store_code1<CB>(codes, i, c);
  }
}

template <typename T, typename Enc>
static int launch_fq(const T* x, T* y, void* codes, int code_bytes, int64_t n, const float* scale,
                     int64_t inner, int64_t C, bool mul, const Enc& enc, hipStream_t st) {
  if (n == 0) return kOk;
  const int bs = 256;
  bool vec = C <= 1 && aligned(x, 16) && (!y || aligned(y, 16)) &&
             (code_bytes == 0 || aligned(codes, code_bytes == 1 ? 8 : 16));
  if (vec) {
    unsigned grid = grid_for(n / 8 + 1, bs);
    if (code_bytes == 0)
      hipLaunchKernelGGL((fq_vec_kernel<T, Enc, 0>), dim3(grid), dim3(bs), 0, st, x, y, codes, n, scale, mul, enc);
    else if (code_bytes == 1)
      hipLaunchKernelGGL((fq_vec_kernel<T, Enc, 1>), dim3(grid), dim3(bs), 0, st, x, y, codes, n, scale, mul, enc);
    else
      hipLaunchKernelGGL((fq_vec_kernel<T, Enc, 2>), dim3(grid), dim3(bs), 0, st, x, y, codes, n, scale, mul, enc);
  } else {
    unsigned grid = grid_for(n, bs);
    if (code_bytes == 0)
      hipLaunchKernelGGL((fq_scalar_kernel<T, Enc, 0>), dim3(grid), dim3(bs), 0, st, x, y, codes, n, scale, inner, C, mul, enc);
    else if (code_bytes == 1)
      hipLaunchKernelGGL((fq_scalar_kernel<T, Enc, 1>), dim3(grid), dim3(bs), 0, st, x, y, codes, n, scale, inner, C, mul, enc);
    else
      hipLaunchKernelGGL((fq_scalar_kernel<T, Enc, 2>), dim3(grid), dim3(bs), 0, st, x, y, codes, n, scale, inner, C, mul, enc);
  }
  return check_launch("fake_quant");
}

template <typename Enc>
static int launch_fq_dtype(const void* x, int dtype, void* y, void* codes, int code_bytes, int64_t n,
                           const float* scale, int64_t inner, int64_t C, bool mul, const Enc& enc,
                           hipStream_t st) {
  switch (dtype) {
    case kF32:
      return launch_fq((const float*)x, (float*)y, codes, code_bytes, n, scale, inner, C, mul, enc, st);
    case kBF16:
      return launch_fq((const uint16_t*)x, (uint16_t*)y, codes, code_bytes, n, scale, inner, C, mul, enc, st);
    case kF16:
      return launch_fq((const __half*)x, (__half*)y, codes, code_bytes, n, scale, inner, C, mul, enc, st);
    default:
      return set_error(kErrInvalid, "input dtype %d not supported (float32, bfloat16, float16)", dtype);
  }
}

template <typename T>
static int launch_fq_lut(const T* x, T* y, void* codes, int code_bytes, int64_t n, const float* scale, bool mul,
                         const LutView& lv, hipStream_t st) {
  size_t lds = sizeof(uint32_t) * 2 * lv.len;
  if (code_bytes == 0) {
    auto k = fq_lut_kernel<T, 0>;
    unsigned grid = persistent_grid((const void*)k, kFqLutThreads, lds, n / 8 + 1);
    hipLaunchKernelGGL(k, dim3(grid), dim3(kFqLutThreads), lds, st, x, y, codes, n, scale, mul, lv);
  } else {
    auto k = fq_lut_kernel<T, 1>;
    unsigned grid = persistent_grid((const void*)k, kFqLutThreads, lds, n / 8 + 1);
    hipLaunchKernelGGL(k, dim3(grid), dim3(kFqLutThreads), lds, st, x, y, codes, n, scale, mul, lv);
  }
  return check_launch("fake_quant(lut)");
}

int fake_quant(const void* x, int dtype, int64_t n, const FormatDesc& fmt, const float* scale,
               int64_t scale_numel, int64_t scale_inner, bool mul, void* y, void* codes, int code_bytes,
               hipStream_t st) {
  if (n < 0) return set_error(kErrInvalid, "negative element count");
  if (code_bytes != 0 && code_bytes != 1 && code_bytes != 2)
    return set_error(kErrInvalid, "code width must be 1 or 2 bytes");
  if (scale_numel > 1 && scale_inner < 1) return set_error(kErrInvalid, "scale_inner must be >= 1");
  if (n == 0) return kOk;
  if (fmt.lut && scale_numel <= 1 && code_bytes <= 1 && aligned(x, 16) && (!y || aligned(y, 16)) &&
      (code_bytes == 0 || aligned(codes, 8))) {
    LutView lv{fmt.lut, fmt.lut_len};
    switch (dtype) {
      case kF32: return launch_fq_lut((const float*)x, (float*)y, codes, code_bytes, n, scale, mul, lv, st);
      case kBF16: return launch_fq_lut((const uint16_t*)x, (uint16_t*)y, codes, code_bytes, n, scale, mul, lv, st);
      case kF16: return launch_fq_lut((const __half*)x, (__half*)y, codes, code_bytes, n, scale, mul, lv, st);
      default: break;
    }
  }
  return with_encoder(fmt, [&](auto enc) {
    return launch_fq_dtype(x, dtype, y, codes, code_bytes, n, scale, scale_inner, scale_numel, mul, enc, st);
  });
}

int lut_gather(const void* x, int dtype, int64_t n, const uint16_t* table, void* y, hipStream_t st) {
  if (n < 0) return set_error(kErrInvalid, "negative element count");
  if (!table) return set_error(kErrInvalid, "table is null");
  return launch_fq_dtype(x, dtype, y, nullptr, 0, n, nullptr, 1, 1, false, EncTable{table}, st);
}

// ---------------------------------------------------------------------------
// FusedAmaxObsFakeQuantize.forward for the per-tensor and per-channel
// qschemes (src/vc/quantization/fake_quantize.py:308-341, :418-426), without
// a host synchronisation.  Channel of element i: (i / inner) % C (C == 1 is
// per-tensor).  history: fp32 [H, C]; scale: fp32 [C]; both updated in place.
//  1. obs_prepare_kernel, one thread per channel: the new scale from the
//     history's maximum before this step (torch.amax over dim 0, a NaN
//     anywhere giving NaN), divided by quant_max in IEEE fp32 (the CPU's
//     tensor / Python-scalar division), the previous scale where that
//     maximum is not positive or not finite, optionally 2 ** ceil(log2) as
//     the CPU evaluates it; then torch.roll(history, -1, 0) with row 0
//     cleared for this step's amax.
//  2. obs_fq_kernel: y = vmap(x / s, qmap) * s with s the channel's new scale
//     in x's dtype (FakeQuantizeFunction; skipped when y is null), and |x|
//     folded into history row 0 by integer atomic max on fp32 bit patterns
//     (non-negative floats order as their patterns, and a NaN pattern beats
//     every number, as torch.amax propagates NaN).  A thread keeps a running
//     maximum for its current channel and folds it in when the channel
//     changes and at the end, with the atomic skipped when row 0 already
//     holds at least as much (row 0 only grows during the launch, so a
//     stale read can only cost an unneeded atomic).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void obs_prepare_kernel(float* __restrict__ hist, int H, int64_t C,
                                                          float* __restrict__ scale, float quant_max, bool pow2) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  const float first = hist[c];
  float amax = first;
  bool nan = first != first;
#pragma unroll 4
  for (int h = 1; h < H; ++h) {
    const float v = hist[(int64_t)h * C + c];
    nan |= v != v;
    amax = __builtin_fmaxf(amax, v);
  }
  if (nan) amax = __builtin_nanf("");
  const float prev = scale[c];
  float sf = amax / quant_max;
  sf = amax > 0.0f ? sf : prev;
  sf = __builtin_isfinite(amax) ? sf : prev;
  if (pow2) sf = u2f(pow2_ceil_log2_f32(f2u(sf)));
  scale[c] = sf;
  // roll by -1: row h takes row h + 1, the last row takes row 0
  for (int h = 1; h + 1 < H; ++h) hist[(int64_t)h * C + c] = hist[(int64_t)(h + 1) * C + c];
  if (H > 1) hist[(int64_t)(H - 1) * C + c] = first;
  hist[c] = 0.0f;
}

__device__ __forceinline__ void fold_amax(uint32_t* __restrict__ row, int64_t c, uint32_t m) {
  uint32_t* p = row + c;
  if (m > __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) atomicMax(p, m);
}

__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = umax32(v, (uint32_t)__shfl_xor((int)v, d, 64));
  return v;
}

// VEC: 8 elements per thread and step with 16-byte loads / stores, every
// group of 8 within one channel (C == 1, or inner % 8 == 0).  Otherwise one
// element per step, with a grid stride the host makes a multiple of
// inner * C when it can, which keeps each thread on one channel.
template <typename T, typename Enc, bool VEC>
__global__ __launch_bounds__(256) void obs_fq_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t n,
                                                     int64_t inner, int64_t C, int64_t stride,
                                                     const float* __restrict__ scale, uint32_t* __restrict__ row,
                                                     Enc enc) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t run = 0;
  int64_t run_c = -1;
  auto fold = [&](int64_t c, uint32_t m) {
    if (c != run_c) {
      if (run_c >= 0) fold_amax(row, run_c, run);
      run_c = c;
      run = m;
    } else {
      run = umax32(run, m);
    }
  };
  if constexpr (VEC) {
    const int64_t nvec = n / 8;
    for (int64_t g = t; g < nvec; g += stride) {
      float v[8];
      IO<T>::load(x + g * 8, v);
      const int64_t c = C > 1 ? (g * 8 / inner) % C : 0;
      uint32_t m = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) m = umax32(m, f2u(v[j]) & 0x7FFFFFFFu);
      if (y) {
        const float s = to_dtype<T>(scale[c]);
        uint32_t code;
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = fq_one<T>(v[j], s, s == 1.0f, true, enc, code);
        IO<T>::store(y + g * 8, v);
      }
      if (C == 1) {
        run = umax32(run, m);
        run_c = 0;
      } else {
        // when the whole wave is active and on one channel (rows of a
        // weight), reduce over the wave and let lane 0 fold; the condition
        // is uniform over the wave, so every lane takes the same branch
        const int lane = threadIdx.x & 63;
        const bool full = g - lane + 64 <= nvec;
        const int ci = (int)c;
        if (full && __all(ci == __builtin_amdgcn_readfirstlane(ci))) {
          m = wave_umax(m);
          if (lane == 0) fold(c, m);
        } else {
          fold(c, m);
        }
      }
    }
    // the < 8-element tail, one element per thread
    const int64_t i = nvec * 8 + t;
    if (i < n) {
      const float xv = IO<T>::get(x + i);
      const int64_t c = C > 1 ? (i / inner) % C : 0;
      if (y) {
        const float s = to_dtype<T>(scale[c]);
        uint32_t code;
        IO<T>::put(y + i, fq_one<T>(xv, s, s == 1.0f, true, enc, code));
      }
      fold(c, f2u(xv) & 0x7FFFFFFFu);
    }
  } else {
    for (int64_t i = t; i < n; i += stride) {
      const float xv = IO<T>::get(x + i);
      const int64_t c = C > 1 ? (i / inner) % C : 0;
      if (y) {
        const float s = to_dtype<T>(scale[c]);
        uint32_t code;
        IO<T>::put(y + i, fq_one<T>(xv, s, s == 1.0f, true, enc, code));
      }
      fold(c, f2u(xv) & 0x7FFFFFFFu);
    }
  }
  if (C == 1) {
    // per-tensor: one fold per wave
    const uint32_t m = wave_umax(run_c >= 0 ? run : 0u);
    if ((threadIdx.x & 63) == 0) fold_amax(row, 0, m);
  } else if (run_c >= 0) {
    fold_amax(row, run_c, run);
  }
}

template <typename T, typename Enc>
static int launch_obs_fq(const T* x, T* y, int64_t n, int64_t inner, int64_t C, const float* scale,
                         uint32_t* row, const Enc& enc, hipStream_t st) {
  const int bs = 256;
  const bool vec = (C == 1 || inner % 8 == 0) && aligned(x, 16) && (!y || aligned(y, 16));
  if (vec) {
    const unsigned grid = grid_for(n / 8 + 1, bs);
    hipLaunchKernelGGL((obs_fq_kernel<T, Enc, true>), dim3(grid), dim3(bs), 0, st, x, y, n, inner, C,
                       (int64_t)grid * bs, scale, row, enc);
  } else {
    // a stride that is a multiple of inner * C keeps each thread on one
    // channel; the cap keeps the grid within a few waves per SIMD
    const int64_t period = inner * C;
    const int64_t target = (int64_t)num_cus() * 8 * bs;
    int64_t threads = target;
    if (period <= target) threads = target / period * period;
    else if (period <= (int64_t)1 << 22) threads = period;
    const int64_t need = n < threads ? ((n + bs - 1) / bs) * bs : threads;
    const unsigned grid = (unsigned)((need + bs - 1) / bs);
    hipLaunchKernelGGL((obs_fq_kernel<T, Enc, false>), dim3(grid), dim3(bs), 0, st, x, y, n, inner, C, threads, scale,
                       row, enc);
  }
  return check_launch("amax_observe_fake_quant");
}

int amax_observe_fake_quant(const void* x, int dtype, int64_t n, int64_t C, int64_t inner, const FormatDesc& fmt,
                            float* history, int H, float* scale, float quant_max, bool pow2, void* y,
                            hipStream_t st) {
  if (n <= 0) return set_error(kErrInvalid, "amax_observe_fake_quant: empty input (torch.amax of an empty tensor)");
  if (C < 1 || inner < 1 || H < 1) return set_error(kErrInvalid, "amax_observe_fake_quant: C, inner, H must be >= 1");
  if (C > 1 && (n % (C * inner)) != 0)
    return set_error(kErrInvalid, "amax_observe_fake_quant: n = %lld is not a multiple of C * inner", (long long)n);
  if (C > (int64_t)1 << 30) return set_error(kErrInvalid, "amax_observe_fake_quant: too many channels");
  hipLaunchKernelGGL(obs_prepare_kernel, dim3((unsigned)((C + 255) / 256)), dim3(256), 0, st, history, H, C, scale,
                     quant_max, pow2);
  int rc = check_launch("amax_observe_fake_quant(prepare)");
  if (rc != kOk) return rc;
  uint32_t* row = reinterpret_cast<uint32_t*>(history);
  return with_encoder(fmt, [&](auto enc) {
    switch (dtype) {
      case kF32: return launch_obs_fq((const float*)x, (float*)y, n, inner, C, scale, row, enc, st);
      case kBF16: return launch_obs_fq((const uint16_t*)x, (uint16_t*)y, n, inner, C, scale, row, enc, st);
      case kF16: return launch_obs_fq((const __half*)x, (__half*)y, n, inner, C, scale, row, enc, st);
      default: return set_error(kErrInvalid, "input dtype %d not supported (float32, bfloat16, float16)", dtype);
    }
  });
}

// ---------------------------------------------------------------------------
// quantize / dequantize with any scale layout (vqx_scale_map)
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t scale_index(int64_t i, const ScaleMap& m) {
  int64_t in = i % m.inner;
  int64_t r = i / m.inner;
  int64_t l = r % m.L;
  int64_t o = r / m.L;
  return o * m.s_o + (l / m.block) * m.s_l + in * m.s_in;
}

template <typename T, typename Enc, int CB>
__global__ __launch_bounds__(256) void quant_mapped_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                           void* __restrict__ codes, int64_t n,
                                                           ScaleMap m, bool mul, Enc enc) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    int64_t si = scale_index(i, m);
    float s = IO<T>::get(static_cast<const T*>(m.scale) + si);
    float xv = IO<T>::get(x + i);
    float t = to_dtype<T>(xv / s);
    if (m.zero_point) t = to_dtype<T>(t + IO<T>::get(static_cast<const T*>(m.zero_point) + si));
    Result r = enc.encode(f2bf(t));
    float v = to_dtype<T>(bf2f(r.value));
    if (mul) {
      if (m.zero_point) v = to_dtype<T>(v - IO<T>::get(static_cast<const T*>(m.zero_point) + si));
      v = to_dtype<T>(v * s);
    }
    if (y) IO<T>::put(y + i, v);
    if constexpr (CB > 0) store_code1<CB>(codes, i, r.code);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void dequant_mapped_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                             int64_t n, const uint16_t* __restrict__ in_map,
                                                             ScaleMap m, const uint16_t* __restrict__ out_map) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float v = IO<T>::get(x + i);
    if (in_map) v = to_dtype<T>(bf2f(in_map[f2bf(v)]));
    if (m.scale) {
      int64_t si = scale_index(i, m);
      if (m.zero_point) v = to_dtype<T>(v - IO<T>::get(static_cast<const T*>(m.zero_point) + si));
      v = to_dtype<T>(v * IO<T>::get(static_cast<const T*>(m.scale) + si));
    }
    if (out_map) v = to_dtype<T>(bf2f(out_map[f2bf(v)]));
    IO<T>::put(y + i, v);
  }
}

template <typename T, typename Enc>
static int launch_qmapped(const T* x, T* y, void* codes, int code_bytes, int64_t n, const ScaleMap& m,
                          bool mul, const Enc& enc, hipStream_t st) {
  unsigned grid = grid_for(n, 256);
  if (code_bytes == 0)
    hipLaunchKernelGGL((quant_mapped_kernel<T, Enc, 0>), dim3(grid), dim3(256), 0, st, x, y, codes, n, m, mul, enc);
  else if (code_bytes == 1)
    hipLaunchKernelGGL((quant_mapped_kernel<T, Enc, 1>), dim3(grid), dim3(256), 0, st, x, y, codes, n, m, mul, enc);
  else
    hipLaunchKernelGGL((quant_mapped_kernel<T, Enc, 2>), dim3(grid), dim3(256), 0, st, x, y, codes, n, m, mul, enc);
  return check_launch("quantize_mapped");
}

static int check_map(const ScaleMap& m) {
  if (m.L < 1 || m.inner < 1 || m.block < 1)
    return set_error(kErrInvalid, "scale map: L, inner, block must be >= 1");
  if (m.s_o < 0 || m.s_l < 0 || m.s_in < 0) return set_error(kErrInvalid, "scale map: negative stride");
  return kOk;
}

int quantize_mapped(const void* x, int dtype, int64_t n, const FormatDesc& fmt, const ScaleMap& m,
                    bool mul, void* y, void* codes, int code_bytes, hipStream_t st) {
  if (n < 0) return set_error(kErrInvalid, "negative element count");
  if (n == 0) return kOk;
  if (!m.scale) return set_error(kErrInvalid, "quantize: scale is required");
  int rc = check_map(m);
  if (rc != kOk) return rc;
  if (!codes) code_bytes = 0;
  if (code_bytes < 0 || code_bytes > 2) return set_error(kErrInvalid, "code width must be 1 or 2 bytes");
  return with_encoder(fmt, [&](auto enc) -> int {
    using E = decltype(enc);
    switch (dtype) {
      case kF32: return launch_qmapped<float, E>((const float*)x, (float*)y, codes, code_bytes, n, m, mul, enc, st);
      case kBF16: return launch_qmapped<uint16_t, E>((const uint16_t*)x, (uint16_t*)y, codes, code_bytes, n, m, mul, enc, st);
      case kF16: return launch_qmapped<__half, E>((const __half*)x, (__half*)y, codes, code_bytes, n, m, mul, enc, st);
      default: return set_error(kErrInvalid, "input dtype %d not supported", dtype);
    }
  });
}

int dequantize_mapped(const void* x, int dtype, int64_t n, const uint16_t* in_map, const ScaleMap& m,
                      const uint16_t* out_map, void* y, hipStream_t st) {
  if (n < 0) return set_error(kErrInvalid, "negative element count");
  if (n == 0) return kOk;
  if (m.scale) {
    int rc = check_map(m);
    if (rc != kOk) return rc;
  }
  unsigned grid = grid_for(n, 256);
  switch (dtype) {
    case kF32:
      hipLaunchKernelGGL((dequant_mapped_kernel<float>), dim3(grid), dim3(256), 0, st, (const float*)x, (float*)y, n, in_map, m, out_map);
      break;
    case kBF16:
      hipLaunchKernelGGL((dequant_mapped_kernel<uint16_t>), dim3(grid), dim3(256), 0, st, (const uint16_t*)x, (uint16_t*)y, n, in_map, m, out_map);
      break;
    case kF16:
      hipLaunchKernelGGL((dequant_mapped_kernel<__half>), dim3(grid), dim3(256), 0, st, (const __half*)x, (__half*)y, n, in_map, m, out_map);
      break;
    default:
      return set_error(kErrInvalid, "input dtype %d not supported", dtype);
  }
  return check_launch("dequantize_mapped");
}

// ---------------------------------------------------------------------------
// setup: tabulate a format over every bf16 pattern
// ---------------------------------------------------------------------------
template <typename Enc>
__global__ __launch_bounds__(256) void build_table_kernel(uint16_t* values, uint16_t* codes, Enc enc) {
  uint32_t h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= 65536u) return;
  Result r = enc.encode(h);
  if (values) values[h] = (uint16_t)r.value;
  if (codes) codes[h] = (uint16_t)r.code;
}

int build_table(const FormatDesc& fmt, uint16_t* values, uint16_t* codes, hipStream_t st) {
  return with_encoder(fmt, [&](auto enc) {
    hipLaunchKernelGGL((build_table_kernel<decltype(enc)>), dim3(256), dim3(256), 0, st, values, codes, enc);
    return check_launch("build_table");
  });
}

// Compact LUT (vqx_lut.h): tabulate entries, find the flush and saturation
// runs shared by both signs, copy the table between them.
template <typename Enc>
__global__ __launch_bounds__(256) void lut_full_kernel(uint32_t* full, Enc enc) {
  uint32_t h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= 65536u) return;
  Result r = enc.encode(h);
  full[h] = (r.value & 0xFFFFu) | (r.code << 16);
}

__global__ __launch_bounds__(256) void lut_bounds_kernel(const uint32_t* full, uint32_t S, uint32_t* hdr) {
  uint32_t a = blockIdx.x * blockDim.x + threadIdx.x;
  if (a < 1 || a >= S) return;
  if (full[a] != full[1] || full[0x8000u | a] != full[0x8001u]) atomicMin(&hdr[kLutT0m1], a);
  if (full[a] != full[S - 1] || full[0x8000u | a] != full[0x8000u | (S - 1)]) atomicMax(&hdr[kLutT1], a);
}

__global__ void lut_finalize_kernel(const uint32_t* full, uint32_t S, uint32_t* hdr) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  uint32_t first = hdr[kLutT0m1], last = hdr[kLutT1];
  uint32_t t0m1 = first == 0xFFFFFFFFu ? S - 1 : first - 1;  // >= 1
  if (full[0] != full[t0m1]) t0m1 = 0;  // +0 must share entry 0 with the run below T0
  uint32_t t1 = last == 0 ? t0m1 : last + 1;
  if (t1 > S - 1) t1 = S - 1;
  if (t1 < t0m1) t1 = t0m1;
  uint32_t len = t1 - t0m1 + 1;
  hdr[kLutT0m1] = t0m1;
  hdr[kLutT1] = t1;
  hdr[kLutS] = S;
  hdr[kLutLen] = len;
  // -0 must encode like the tiny negatives or like +0
  uint32_t zsign = full[0x8000u] == full[0x8000u | t0m1] ? 1u : 0u;
  bool zok = zsign || full[0x8000u] == full[t0m1];
  hdr[kLutZeroSign] = zsign;
  hdr[kLutValid] = (len <= (uint32_t)kLutMaxLen && zok) ? 1u : 0u;
}

__global__ __launch_bounds__(256) void lut_copy_kernel(const uint32_t* full, uint32_t* blob) {
  uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (!blob[kLutValid]) return;
  uint32_t len = blob[kLutLen], t0m1 = blob[kLutT0m1];
  if (i >= len) return;
  blob[kLutHeaderWords + i] = full[t0m1 + i];
  blob[kLutHeaderWords + len + i] = full[0x8000u | (t0m1 + i)];
}

__global__ void lut_init_kernel(uint32_t* hdr) {
  if (threadIdx.x < kLutHeaderWords) hdr[threadIdx.x] = threadIdx.x == kLutT0m1 ? 0xFFFFFFFFu : 0u;
}

int build_lut(const FormatDesc& fmt, uint32_t* blob, hipStream_t st) {
  if (fmt.code_bits > 8) return set_error(kErrInvalid, "tables hold codes of at most 8 bits");
  // magnitudes from S up take the closed form: Inf/NaN, and the fp core's
  // NaN region (bf16 log2 = 128)
  uint32_t S = fmt.kind == kFmtFpCore ? 0x7F58u : 0x7F80u;
  uint32_t* full = blob + kLutHeaderWords + 2 * kLutMaxLen;
  FormatDesc d = fmt;
  d.lut = nullptr;
  return with_encoder(d, [&](auto enc) {
    hipLaunchKernelGGL((lut_full_kernel<decltype(enc)>), dim3(256), dim3(256), 0, st, full, enc);
    hipLaunchKernelGGL(lut_init_kernel, dim3(1), dim3(64), 0, st, blob);
    hipLaunchKernelGGL(lut_bounds_kernel, dim3(128), dim3(256), 0, st, full, S, blob);
    hipLaunchKernelGGL(lut_finalize_kernel, dim3(1), dim3(64), 0, st, full, S, blob);
    hipLaunchKernelGGL(lut_copy_kernel, dim3(kLutMaxLen / 256), dim3(256), 0, st, full, blob);
    return check_launch("build_lut");
  });
}

// Index table of a level set for every bf16 pattern:
//  mode 0 (NormalFloat, normal_float.py:58-60): levels are bf16, the input is
//    clamped to [min, max], and |level - x| is rounded to bf16 before argmin;
//  mode 1 (codebook, lcq.py:286-291): levels fp32, clamp and |x - level| fp32.
// argmin takes the first index of the minimum; NaN inputs give index 0.
__global__ __launch_bounds__(256) void level_index_kernel(const float* levels, int K, int mode,
                                                          uint8_t* out) {
  uint32_t h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= 65536u) return;
  float x = bf2f(h);
  if (x != x) {
    out[h] = 0;
    return;
  }
  float lo = levels[0], hi = levels[0];
  for (int k = 1; k < K; ++k) {
    lo = fminf(lo, levels[k]);
    hi = fmaxf(hi, levels[k]);
  }
  float xc = x < lo ? lo : x;
  xc = xc > hi ? hi : xc;
  int best = 0;
  float bd = 0.0f;
  for (int k = 0; k < K; ++k) {
    float d = mode == 0 ? levels[k] - xc : xc - levels[k];
    if (mode == 0) d = bf2f(f2bf(d));
    d = fabsf(d);
    if (k == 0 || d < bd) {
      bd = d;
      best = k;
    }
  }
  out[h] = (uint8_t)best;
}

// Order-preserving key of a float: unsigned comparison of keys = float order.
__device__ __forceinline__ uint32_t order_key(uint32_t bits) {
  return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}
__device__ __forceinline__ uint32_t key_bits(uint32_t key) {
  return (key & 0x80000000u) ? (key & 0x7FFFFFFFu) : ~key;
}

// first[c] = least (order key of a) bf16 value whose index is c.
__global__ __launch_bounds__(256) void level_first_kernel(const uint8_t* idx, uint32_t* first, int K) {
  // per-workgroup minima in LDS first, then one global atomic per level
  __shared__ uint32_t lmin[256];
  for (int k = threadIdx.x; k < K; k += blockDim.x) lmin[k] = 0xFFFFFFFFu;
  __syncthreads();
  uint32_t h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h < 65536u && (h & 0x7FFFu) <= 0x7F80u) atomicMin(&lmin[idx[h]], order_key(h << 16));
  __syncthreads();
  for (int k = threadIdx.x; k < K; k += blockDim.x)
    if (lmin[k] != 0xFFFFFFFFu) atomicMin(&first[k], lmin[k]);
}

// boundaries[j-1] = min_{c >= j} first[c]  (suffix minimum), as fp32 values.
__global__ void level_boundary_kernel(const uint32_t* first, int K, float* boundaries) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  uint32_t m = 0xFFFFFFFFu;
  for (int j = K - 1; j >= 1; --j) {
    m = first[j] < m ? first[j] : m;
    // a code no bf16 value reaches gets a NaN boundary: v >= NaN never holds
    boundaries[j - 1] = m == 0xFFFFFFFFu ? __builtin_nanf("") : u2f(key_bits(m));
  }
}

// Check that counting boundaries reproduces the index table everywhere.
__global__ __launch_bounds__(256) void level_verify_kernel(const uint8_t* idx, const float* boundaries,
                                                           int K, int* bad) {
  uint32_t h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= 65536u) return;
  uint32_t c = count_le(boundaries, K - 1, bf2f(h));
  if (c != idx[h]) atomicAdd(bad, 1);
}

int level_tables(const float* levels, int K, int mode, uint8_t* index_table, float* boundaries,
                 uint32_t* work, int* bad, hipStream_t st) {
  if (K < 1 || K > 256) return set_error(kErrInvalid, "level count %d outside [1,256]", K);
  hipLaunchKernelGGL(level_index_kernel, dim3(256), dim3(256), 0, st, levels, K, mode, index_table);
  if (K == 1) return check_launch("level_tables");
  if (hipMemsetAsync(work, 0xFF, sizeof(uint32_t) * K, st) != hipSuccess ||
      hipMemsetAsync(bad, 0, sizeof(int), st) != hipSuccess)
    return set_error(kErrLaunch, "hipMemsetAsync failed");
  hipLaunchKernelGGL(level_first_kernel, dim3(256), dim3(256), 0, st, index_table, work, K);
  hipLaunchKernelGGL(level_boundary_kernel, dim3(1), dim3(64), 0, st, work, K, boundaries);
  hipLaunchKernelGGL(level_verify_kernel, dim3(256), dim3(256), 0, st, index_table, boundaries, K, bad);
  return check_launch("level_tables");
}

}  // namespace vqx
