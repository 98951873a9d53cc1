// Blockwise kernels: the MX / absmax block scale (calculate_mx_qparam) fused
// with the element encode (quantize / quantize_mx), with every output the
// path needs written in the same pass: the reference's scale and quantized
// values, the fake-quant product, packed codes, fp32 and E8M0 scales.  Plus
// the decode of packed codes back to values (dequantize).
#include <type_traits>

#include "vqx_kernels.h"

namespace vqx {

// ---------------------------------------------------------------------------
// dtype traits for blockwise inputs
// ---------------------------------------------------------------------------
template <typename T>
struct BT;

template <>
struct BT<uint16_t> {  // bf16 bits
  static constexpr uint32_t kSign = 0x8000u;
  static constexpr uint32_t kMagMask = 0x7FFFu;
  static constexpr uint32_t kInf = 0x7F80u;
  __device__ static uint32_t bits(const uint16_t* p) { return *p; }
  __device__ static float val(uint32_t b) { return u2f(b << 16); }
  __device__ static uint32_t round_bits(float f) { return f2bf(f); }
  __device__ static void load16(const uint16_t* p, uint32_t (&b)[16]) {
    const u32x4* q = reinterpret_cast<const u32x4*>(p);
    u32x4 a0 = ld_nt(q), a1 = ld_nt(q + 1);
    uint32_t w[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      b[2 * j] = w[j] & 0xFFFFu;
      b[2 * j + 1] = w[j] >> 16;
    }
  }
  __device__ static void store16(uint16_t* p, const uint32_t (&b)[16]) {
    u32x4* q = reinterpret_cast<u32x4*>(p);
    u32x4 a0 = {b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
    u32x4 a1 = {b[8] | (b[9] << 16), b[10] | (b[11] << 16), b[12] | (b[13] << 16),
                b[14] | (b[15] << 16)};
    st_nt(q, a0);
    st_nt(q + 1, a1);
  }
  __device__ static void put(uint16_t* p, uint32_t b) { *p = (uint16_t)b; }
};

template <>
struct BT<float> {
  static constexpr uint32_t kSign = 0x80000000u;
  static constexpr uint32_t kMagMask = 0x7FFFFFFFu;
  static constexpr uint32_t kInf = 0x7F800000u;
  __device__ static uint32_t bits(const float* p) { return f2u(*p); }
  __device__ static float val(uint32_t b) { return u2f(b); }
  __device__ static uint32_t round_bits(float f) { return f2u(f); }
  __device__ static void load16(const float* p, uint32_t (&b)[16]) {
    const u32x4* q = reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      u32x4 a = ld_nt(q + k);
      b[4 * k] = a.x;
      b[4 * k + 1] = a.y;
      b[4 * k + 2] = a.z;
      b[4 * k + 3] = a.w;
    }
  }
  __device__ static void store16(float* p, const uint32_t (&b)[16]) {
    u32x4* q = reinterpret_cast<u32x4*>(p);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      u32x4 a = {b[4 * k], b[4 * k + 1], b[4 * k + 2], b[4 * k + 3]};
      st_nt(q + k, a);
    }
  }
  __device__ static void put(float* p, uint32_t b) { *reinterpret_cast<uint32_t*>(p) = b; }
};

// ---------------------------------------------------------------------------
// block scale  (ops/quantized.py:442-499, mx_utils.py:16-59)
// ---------------------------------------------------------------------------
// floor(log2) of a block amax, in the input dtype's arithmetic.  bf16: the
// bf16-rounded log (see log2floor_bf16).  fp32: the correctly rounded fp32
// log, which steps up exactly when the 23-bit mantissa reaches
// 2^23 (2^(1 - u/2) - 1), u the fp32 spacing next to the integer above.
__device__ __forceinline__ int log2floor_f32(uint32_t mag) {
  uint32_t E = mag >> 23, m = mag & 0x7FFFFFu;
  if (E == 0) {
    // subnormal amax m * 2^-149, 2^k <= m < 2^(k+1): the fp32 log rounds up
    // to k - 148 for the top J mantissas of the range (J by k = 17..22, from
    // torch's CPU log2 over every subnormal; none below k = 17)
    const int k = 31 - clz32(m);
    const uint32_t kSubTop[6] = {1, 2, 5, 11, 11, 22};
    const uint32_t J = k >= 17 ? kSubTop[k - 17] : 0u;
    return k - 149 + (J != 0 && m >= (2u << k) - J ? 1 : 0);
  }
  int p = (int)E - 127;
  int band;
  if (p >= 0) {
    uint32_t n = (uint32_t)p + 1u;
    band = 31 - clz32(n);
    if ((n & (n - 1u)) == 0) band -= 1;
  } else if (p == -1) {
    return p;
  } else {
    uint32_t n = (uint32_t)(-p - 1);
    band = 31 - clz32(n);
  }
  // The top J = floor(2^24 (1 - 2^(-u/2))) mantissas of the binade round up,
  // u = 2^(band - 23); J by band -1 .. 6.
  const uint32_t kTop[8] = {0, 0, 1, 2, 5, 11, 22, 44};
  uint32_t J = kTop[band + 1];
  return p + (J != 0 && m >= 0x800000u - J ? 1 : 0);
}

// Returns the block scale in the input dtype (as a float holding that value).
template <typename T>
__device__ __forceinline__ float block_scale(uint32_t amax_bits, const ScaleParams& sp) {
  constexpr bool kBf16 = std::is_same<T, uint16_t>::value;
  const uint32_t inf = BT<T>::kInf;
  float scale;
  if (sp.mode == 0) {
    if (amax_bits > inf) return 1.0f;  // NaN amax -> NaN scale -> 1.0
    if (amax_bits == inf) return __builtin_huge_valf();
    // amax == 0 -> log2(2^-126) = -126 (mx_utils.py:45)
    int e = amax_bits == 0 ? -126
                           : (kBf16 ? log2floor_bf16(amax_bits) : log2floor_f32(amax_bits));
    e -= sp.shift;
    // 2**e in the input dtype: bf16 keeps 2^-133 .. 2^127, 2^-134 ties to 0
    int lo = kBf16 ? -133 : -149;
    if (e > 127)
      scale = __builtin_huge_valf();
    else if (e >= lo)
      scale = exp2i(e);
    else
      scale = 0.0f;
  } else {
    float amax = BT<T>::val(amax_bits);
    scale = BT<T>::val(BT<T>::round_bits(amax / sp.quant_max));
    if (sp.scale_qmap) {
      uint32_t h = f2bf(scale);
      scale = BT<T>::val(BT<T>::round_bits(bf2f(sp.scale_qmap[h])));
    }
  }
  // torch.where(scale > 0, scale, 1.0): zero and NaN scales become 1
  return scale > 0.0f ? scale : 1.0f;
}

// E8M0 byte of a scale: 2^(byte - 127) for powers of two in [2^-127, 2^127],
// 0xFF for +Inf; scales below E8M0's range clamp to 0x00 (the exact scale is
// in the bf16/fp32 scale outputs).
__device__ __forceinline__ uint32_t e8m0_of(float s) {
  uint32_t b = f2u(s);
  uint32_t E = (b >> 23) & 0xFFu;
  if (E == 0xFFu) return 0xFFu;
  return E;  // subnormal scales (2^-127 and below) give 0
}

// x / s rounded as the input dtype divides: exactly by the reciprocal when s
// is a power of two whose reciprocal is a normal-or-exact fp32, else IEEE.
// A NaN quotient (a NaN x, or +-Inf / Inf) takes x's sign, so that the code
// of a NaN value (the format's all-ones magnitude) has a defined sign bit:
// the reference's values are NaN either way, and it writes no codes.
template <typename T>
__device__ __forceinline__ uint32_t div_to_bf16(float x, float s, float rcp, bool pow2) {
  float q = pow2 ? x * rcp : x / s;
  const uint32_t h = f2bf(BT<T>::val(BT<T>::round_bits(q)));
  return q == q ? h : (h & 0x7FFFu) | ((f2u(x) >> 16) & 0x8000u);
}

// The outlier bound of an input of type T (0xFFFFFFFF when masking is off).
template <typename T>
__device__ __forceinline__ uint32_t outlier_bound_t(const OutlierArgs& oa) {
  if (!oa.active) return 0xFFFFFFFFu;
  return outlier_bound(oa, [](float f) { return BT<T>::round_bits(f); }, BT<T>::kSign);
}

// ---------------------------------------------------------------------------
// packing helpers: element i of a group of 16 at bits [cb*i, cb*i + cb)
// ---------------------------------------------------------------------------
template <int CB>
__device__ __forceinline__ void store_group_codes(uint8_t* base, int64_t g, const uint32_t (&c)[16]) {
  if constexpr (CB == 4) {
    u32x2 w;
    w.x = 0;
    w.y = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      w.x |= (c[j] & 0xFu) << (4 * j);
      w.y |= (c[j + 8] & 0xFu) << (4 * j);
    }
    st_nt(reinterpret_cast<u32x2*>(base + g * 8), w);
  } else if constexpr (CB == 6) {
    uint32_t k[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) k[j] = c[j] & 0x3Fu;
    uint32_t w0 = k[0] | (k[1] << 6) | (k[2] << 12) | (k[3] << 18) | (k[4] << 24) | (k[5] << 30);
    uint32_t w1 = (k[5] >> 2) | (k[6] << 4) | (k[7] << 10) | (k[8] << 16) | (k[9] << 22) | (k[10] << 28);
    uint32_t w2 = (k[10] >> 4) | (k[11] << 2) | (k[12] << 8) | (k[13] << 14) | (k[14] << 20) | (k[15] << 26);
    uint32_t* q = reinterpret_cast<uint32_t*>(base + g * 12);
    __builtin_nontemporal_store(w0, q);
    __builtin_nontemporal_store(w1, q + 1);
    __builtin_nontemporal_store(w2, q + 2);
  } else if constexpr (CB == 8) {
    u32x4 w;
    w.x = (c[0] & 0xFF) | ((c[1] & 0xFF) << 8) | ((c[2] & 0xFF) << 16) | (c[3] << 24);
    w.y = (c[4] & 0xFF) | ((c[5] & 0xFF) << 8) | ((c[6] & 0xFF) << 16) | (c[7] << 24);
    w.z = (c[8] & 0xFF) | ((c[9] & 0xFF) << 8) | ((c[10] & 0xFF) << 16) | (c[11] << 24);
    w.w = (c[12] & 0xFF) | ((c[13] & 0xFF) << 8) | ((c[14] & 0xFF) << 16) | (c[15] << 24);
    st_nt(reinterpret_cast<u32x4*>(base + g * 16), w);
  } else if constexpr (CB == 16) {
    u32x4* q = reinterpret_cast<u32x4*>(base + g * 32);
    u32x4 a = {(c[0] & 0xFFFF) | (c[1] << 16), (c[2] & 0xFFFF) | (c[3] << 16),
               (c[4] & 0xFFFF) | (c[5] << 16), (c[6] & 0xFFFF) | (c[7] << 16)};
    u32x4 b = {(c[8] & 0xFFFF) | (c[9] << 16), (c[10] & 0xFFFF) | (c[11] << 16),
               (c[12] & 0xFFFF) | (c[13] << 16), (c[14] & 0xFFFF) | (c[15] << 16)};
    st_nt(q, a);
    st_nt(q + 1, b);
  }
}

// Fast path: blocks of 16 * LPB contiguous elements (last-dim blocks), each
// thread one 16-element group, the LPB threads of a block adjacent in the wave.
template <typename T, typename Enc, int CB, int LPB>
__global__ __launch_bounds__(256) void mx_group_kernel(const T* __restrict__ x, int64_t ngroups,
                                                       ScaleParams sp, Enc enc, MxOut out, OutlierArgs oa) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const uint32_t bound = outlier_bound_t<T>(oa);
  uint32_t nskip = 0;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < ngroups; g += stride) {
    uint32_t b[16], xo[16];
    BT<T>::load16(x + g * 16, b);
    uint32_t skip = 0;
    if (oa.active) {
      // outliers: zeros in the block max and the encode, restored below
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        xo[j] = b[j];
        const bool sk = outlier_skip(b[j] & BT<T>::kMagMask, bound, BT<T>::kInf);
        skip |= (uint32_t)sk << j;
        b[j] = sk ? 0u : b[j];
      }
      nskip += __builtin_popcount(skip);
    }
    uint32_t amax = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) amax = umax32(amax, b[j] & BT<T>::kMagMask);
#pragma unroll
    for (int off = 1; off < LPB; off <<= 1) amax = umax32(amax, (uint32_t)__shfl_xor((int)amax, off, 64));
    float s = block_scale<T>(amax, sp);
    uint32_t sb = f2u(s);
    bool pow2 = (sb & 0x7FFFFFu) == 0 && ((sb >> 23) & 0xFF) >= 1 && ((sb >> 23) & 0xFF) <= 253;
    float rcp = pow2 ? u2f((uint32_t)(254 - ((sb >> 23) & 0xFF)) << 23) : 0.0f;
    uint32_t code[16], qv[16], fv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      uint32_t h = div_to_bf16<T>(BT<T>::val(b[j]), s, rcp, pow2);
      Result r = enc.encode(h);
      code[j] = r.code;
      float v = BT<T>::val(BT<T>::round_bits(bf2f(r.value)));
      qv[j] = BT<T>::round_bits(v);
      if (std::is_same<T, uint16_t>::value) qv[j] = r.value;
      fv[j] = BT<T>::round_bits(v * s);
    }
    if (skip) {
#pragma unroll
      for (int j = 0; j < 16; ++j) fv[j] = (skip >> j) & 1u ? xo[j] : fv[j];
    }
    if (out.qvals) BT<T>::store16(static_cast<T*>(out.qvals) + g * 16, qv);
    if (out.fq) BT<T>::store16(static_cast<T*>(out.fq) + g * 16, fv);
    if constexpr (CB > 0) store_group_codes<CB>(static_cast<uint8_t*>(out.codes), g, code);
    if ((threadIdx.x & (LPB - 1)) == 0) {
      int64_t blk = g / LPB;
      if (out.scale) BT<T>::put(static_cast<T*>(out.scale) + blk, BT<T>::round_bits(s));
      if (out.scale_f32) __builtin_nontemporal_store(s, out.scale_f32 + blk);
      if (out.scale_e8m0) __builtin_nontemporal_store((uint8_t)e8m0_of(s), out.scale_e8m0 + blk);
    }
  }
  outlier_tally(nskip, oa);
}

// General path: x viewed as [outer, L, inner], blocks of bs along L (the last
// block may be short: the reference zero-pads it, which leaves its amax
// unchanged).  One thread per block; codes unpacked (1 or 2 bytes each).
template <typename T, typename Enc>
__global__ __launch_bounds__(256) void mx_block_kernel(const T* __restrict__ x, int64_t outer, int64_t L,
                                                       int64_t inner, int64_t bs, ScaleParams sp, Enc enc,
                                                       MxOut out, int code_bytes, OutlierArgs oa) {
  const int64_t nblk_l = (L + bs - 1) / bs;
  const int64_t total = outer * nblk_l * inner;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const uint32_t bound = outlier_bound_t<T>(oa);
  // an outlier reads as zero (+0.0 bits), as masked_fill(skip, 0.0) leaves it
  auto masked = [&](uint32_t b) { return outlier_skip(b & BT<T>::kMagMask, bound, BT<T>::kInf) ? 0u : b; };
  uint32_t nskip = 0;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += stride) {
    // scale tensor index order = [outer, nblk_l, inner]
    int64_t in = t % inner;
    int64_t rest = t / inner;
    int64_t bl = rest % nblk_l;
    int64_t o = rest / nblk_l;
    int64_t l0 = bl * bs;
    int64_t l1 = l0 + bs < L ? l0 + bs : L;
    const T* base = x + (o * L) * inner + in;
    uint32_t amax = 0;
    for (int64_t l = l0; l < l1; ++l) amax = umax32(amax, masked(BT<T>::bits(base + l * inner)) & BT<T>::kMagMask);
    float s = block_scale<T>(amax, sp);
    uint32_t sb = f2u(s);
    bool pow2 = (sb & 0x7FFFFFu) == 0 && ((sb >> 23) & 0xFF) >= 1 && ((sb >> 23) & 0xFF) <= 253;
    float rcp = pow2 ? u2f((uint32_t)(254 - ((sb >> 23) & 0xFF)) << 23) : 0.0f;
    for (int64_t l = l0; l < l1; ++l) {
      int64_t i = (o * L + l) * inner + in;
      const uint32_t xo = BT<T>::bits(x + i);
      const uint32_t xb = masked(xo);
      const bool sk = xb != xo;
      nskip += sk ? 1u : 0u;
      uint32_t h = div_to_bf16<T>(BT<T>::val(xb), s, rcp, pow2);
      Result r = enc.encode(h);
      float v = BT<T>::val(BT<T>::round_bits(bf2f(r.value)));
      uint32_t q = std::is_same<T, uint16_t>::value ? r.value : BT<T>::round_bits(v);
      if (out.qvals) BT<T>::put(static_cast<T*>(out.qvals) + i, q);
      if (out.fq) BT<T>::put(static_cast<T*>(out.fq) + i, sk ? xo : BT<T>::round_bits(v * s));
      if (out.codes) {
        if (code_bytes == 1) static_cast<uint8_t*>(out.codes)[i] = (uint8_t)r.code;
        else static_cast<uint16_t*>(out.codes)[i] = (uint16_t)r.code;
      }
    }
    if (out.scale) BT<T>::put(static_cast<T*>(out.scale) + t, BT<T>::round_bits(s));
    if (out.scale_f32) out.scale_f32[t] = s;
    if (out.scale_e8m0) out.scale_e8m0[t] = (uint8_t)e8m0_of(s);
  }
  outlier_tally(nskip, oa);
}

// Blocks along a middle axis (inner > 1, e.g. ax=-2 of an attention operand):
// x viewed as [outer, L, inner], blocks of bs <= 128 rows along L, inner a
// multiple of VE = 16 / sizeof(T).  A 256-thread workgroup takes a tile of
// bs rows x 16 column chunks of VE elements (256 contiguous bytes per row):
// thread (chunk c = tid % 16, row group g = tid / 16) loads rows g, g + 16,
// ... of its chunk with 16-byte loads, the per-column block maxima meet in
// LDS, and each thread encodes its elements from registers and stores them
// in the layout it loaded.  Rows past L (a short last block, zero-padded in
// the reference) and chunks past inner are left out.  Same per-element
// arithmetic and outputs as mx_block_kernel (codes unpacked, 1 or 2 bytes).
constexpr int kColChunks = 16;
constexpr int kColRowsMax = 8;  // rows per thread: bs <= 128

template <typename T, typename Enc>
__global__ __launch_bounds__(256) void mx_cols_kernel(const T* __restrict__ x, int64_t outer, int64_t L,
                                                      int64_t inner, int bs, ScaleParams sp, Enc enc, MxOut out,
                                                      int code_bytes, OutlierArgs oa) {
  constexpr int VE = 16 / sizeof(T);
  constexpr int TW = kColChunks * VE;  // columns per tile
  __shared__ uint32_t s_amax[256 / kColChunks][TW];
  __shared__ float s_scale[TW];
  const int tid = threadIdx.x, cg = tid % kColChunks, rg = tid / kColChunks;
  const int64_t nblk = (L + bs - 1) / bs;
  const int64_t ntc = (inner + TW - 1) / TW;
  const int64_t ntiles = outer * nblk * ntc;
  const uint32_t bound = outlier_bound_t<T>(oa);
  uint32_t nskip = 0;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t tc = tile % ntc, rest = tile / ntc;
    const int64_t bl = rest % nblk, o = rest / nblk;
    const int64_t l0 = bl * bs;
    const int64_t col = tc * TW + (int64_t)cg * VE;  // first column of this thread's chunk
    const bool cok = col < inner;
    uint32_t v[kColRowsMax][VE];  // the input, outliers included
    uint32_t skip[kColRowsMax];
    uint32_t m[VE];
#pragma unroll
    for (int e = 0; e < VE; ++e) m[e] = 0;
#pragma unroll
    for (int i = 0; i < kColRowsMax; ++i) {
      const int r = rg + 16 * i;
      const int64_t l = l0 + r;
      skip[i] = 0;
      if (r < bs && l < L && cok) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(x + (o * L + l) * inner + col);
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          const uint32_t b = sizeof(T) == 2 ? ((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) : w[e];
          v[i][e] = b;
          const bool sk = outlier_skip(b & BT<T>::kMagMask, bound, BT<T>::kInf);
          skip[i] |= (uint32_t)sk << e;
          m[e] = umax32(m[e], sk ? 0u : b & BT<T>::kMagMask);
        }
        nskip += __builtin_popcount(skip[i]);
      }
    }
#pragma unroll
    for (int e = 0; e < VE; ++e) s_amax[rg][cg * VE + e] = m[e];
    __syncthreads();
    if (tid < TW) {
      uint32_t a = 0;
#pragma unroll
      for (int g = 0; g < 256 / kColChunks; ++g) a = umax32(a, s_amax[g][tid]);
      const float sc = block_scale<T>(a, sp);
      s_scale[tid] = sc;
      const int64_t c = tc * TW + tid;
      if (c < inner) {
        const int64_t si = (o * nblk + bl) * inner + c;
        if (out.scale) BT<T>::put(static_cast<T*>(out.scale) + si, BT<T>::round_bits(sc));
        if (out.scale_f32) out.scale_f32[si] = sc;
        if (out.scale_e8m0) out.scale_e8m0[si] = (uint8_t)e8m0_of(sc);
      }
    }
    __syncthreads();
    float s[VE], rcp[VE];
    bool pw[VE];
#pragma unroll
    for (int e = 0; e < VE; ++e) {
      s[e] = s_scale[cg * VE + e];
      const uint32_t sb = f2u(s[e]);
      pw[e] = (sb & 0x7FFFFFu) == 0 && ((sb >> 23) & 0xFF) >= 1 && ((sb >> 23) & 0xFF) <= 253;
      rcp[e] = pw[e] ? u2f((uint32_t)(254 - ((sb >> 23) & 0xFF)) << 23) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kColRowsMax; ++i) {
      const int r = rg + 16 * i;
      const int64_t l = l0 + r;
      if (!(r < bs && l < L && cok)) continue;
      uint32_t qv[VE], fv[VE], cd[VE];
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        const bool sk = (skip[i] >> e) & 1u;  // an outlier: encoded as +0, output unchanged
        const uint32_t h = div_to_bf16<T>(BT<T>::val(sk ? 0u : v[i][e]), s[e], rcp[e], pw[e]);
        const Result rr = enc.encode(h);
        const float val = BT<T>::val(BT<T>::round_bits(bf2f(rr.value)));
        qv[e] = std::is_same<T, uint16_t>::value ? rr.value : BT<T>::round_bits(val);
        fv[e] = sk ? v[i][e] : BT<T>::round_bits(val * s[e]);
        cd[e] = rr.code;
      }
      const int64_t base = (o * L + l) * inner + col;
      auto store = [&](void* p, const uint32_t(&b)[VE]) {
        u32x4 w;
        if constexpr (sizeof(T) == 2) {
#pragma unroll
          for (int j = 0; j < 4; ++j) w[j] = (b[2 * j] & 0xFFFFu) | (b[2 * j + 1] << 16);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) w[j] = b[j];
        }
        *reinterpret_cast<u32x4*>(static_cast<T*>(p) + base) = w;
      };
      if (out.qvals) store(out.qvals, qv);
      if (out.fq) store(out.fq, fv);
      if (out.codes) {
        if (code_bytes == 1) {
#pragma unroll
          for (int e = 0; e < VE; ++e) static_cast<uint8_t*>(out.codes)[base + e] = (uint8_t)cd[e];
        } else {
#pragma unroll
          for (int e = 0; e < VE; ++e) static_cast<uint16_t*>(out.codes)[base + e] = (uint16_t)cd[e];
        }
      }
    }
    __syncthreads();  // s_amax / s_scale are rewritten by the next tile
  }
  outlier_tally(nskip, oa);
}

// ---------------------------------------------------------------------------
// Group-wise affine fake-quant (GroupWiseAffineFakeQuantFunction.forward,
// quantization/fake_quantize.py:162-211): per block of bs along L, min and
// max (a short last block is zero-padded, which pulls both towards 0),
//   sf = (max - min) / (qmax - qmin), 1 where not > 0;  zp = -min / sf + qmin;
// optionally both through scale_qmap (vmap); then per element
//   (clamp(round(x / sf + zp), qmin, qmax) - zp) * sf.
// Every step rounds to the input dtype as torch's ops on that dtype do (the
// fp32 result of each operation, then RNE to bf16 for bf16 inputs), the
// divisions are IEEE-correct, and NaN propagates as in torch (amin / amax
// and clamp keep it).  One thread per block, x viewed as [outer, L, inner].
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float round_to(float f) {
  return BT<T>::val(BT<T>::round_bits(f));
}

template <typename T>
__global__ __launch_bounds__(256) void gwa_fq_kernel(const T* __restrict__ x, int64_t outer, int64_t L,
                                                     int64_t inner, int64_t bs, float qmin, float qmax,
                                                     const uint16_t* __restrict__ scale_qmap, T* scale_out,
                                                     T* zp_out, T* __restrict__ y) {
  const int64_t nblk_l = (L + bs - 1) / bs;
  const int64_t total = outer * nblk_l * inner;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const float qrange = qmax - qmin;
  auto vmap = [&](float v) { return round_to<T>(bf2f(scale_qmap[f2bf(v)])); };
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += stride) {
    const int64_t in = t % inner;
    const int64_t rest = t / inner;
    const int64_t bl = rest % nblk_l;
    const int64_t o = rest / nblk_l;
    const int64_t l0 = bl * bs;
    const int64_t l1 = l0 + bs < L ? l0 + bs : L;
    const T* base = x + (o * L) * inner + in;
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
    bool nan = false;
    for (int64_t l = l0; l < l1; ++l) {
      const float v = BT<T>::val(BT<T>::bits(base + l * inner));
      nan |= v != v;
      mn = v < mn ? v : mn;
      mx = v > mx ? v : mx;
    }
    if (l1 - l0 < bs) {  // the zero padding of a short last block
      mn = mn < 0.0f ? mn : 0.0f;
      mx = mx > 0.0f ? mx : 0.0f;
    }
    if (nan) mn = mx = __builtin_nanf("");
    float sf = round_to<T>(round_to<T>(mx - mn) / qrange);
    sf = sf > 0.0f ? sf : 1.0f;
    float zp = round_to<T>(round_to<T>(-mn / sf) + qmin);
    if (scale_qmap) {
      sf = vmap(sf);
      zp = vmap(zp);
    }
    if (scale_out) BT<T>::put(scale_out + t, BT<T>::round_bits(sf));
    if (zp_out) BT<T>::put(zp_out + t, BT<T>::round_bits(zp));
    for (int64_t l = l0; l < l1; ++l) {
      const int64_t i = (o * L + l) * inner + in;
      const float v = BT<T>::val(BT<T>::bits(x + i));
      float q = __builtin_rintf(round_to<T>(round_to<T>(v / sf) + zp));
      q = q < qmin ? qmin : (q > qmax ? qmax : q);  // NaN stays NaN
      BT<T>::put(y + i, BT<T>::round_bits(round_to<T>(q - zp) * sf));
    }
  }
}

// Blocks along the last axis (inner == 1, L % bs == 0, bs = 8 G with G in
// 1, 2, 4, 8): G consecutive lanes share a block, each loading 8 consecutive
// elements with vector loads, and reduce min / max / NaN with XOR shuffles.
// The per-element arithmetic is gwa_fq_kernel's.  The only freedom the tree
// order adds is which of +0 and -0 a min or max keeps, and neither sf
// (max - min, then 1 where not > 0) nor zp (-min / sf + qmin) nor y changes
// with it.
// v from the lane that DPP control CTRL names (within rows of 16 lanes)
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}

template <typename T, int G>
__global__ __launch_bounds__(256) void gwa_fq_rows_kernel(const T* __restrict__ x, int64_t nchunks, float qmin,
                                                          float qmax, const uint16_t* __restrict__ scale_qmap,
                                                          T* scale_out, T* zp_out, T* __restrict__ y) {
  const float qrange = qmax - qmin;
  // qrange as a bf16 value (at most 8 significant bits) and its reciprocal
  const bool qr_exact = (f2u(qrange) & 0xFFFFu) == 0 && ((f2u(qrange) >> 23) & 0xFFu) - 1u < 252u;
  const float qr_rcp = __builtin_amdgcn_rcpf(qrange);
  // 0 < |q| < 2^-125: a quotient among the subnormals, or within one binade
  // of them (a margin for the rounding of the fast quotient)
  auto tiny = [](float q) { return (f2u(q) & 0x7FFFFFFFu) - 1u < 0x00FFFFFFu; };
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  // every lane runs the same number of iterations (nchunks is a multiple of
  // G and the stride of 256), so the shuffles see whole groups
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c - threadIdx.x % 64 < nchunks; c += stride) {
    const bool live = c < nchunks;
    const int64_t cc = live ? c : nchunks - 1;
    float v[8];
    if constexpr (sizeof(T) == 2) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(x + cc * 8);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = u2f(w[i] << 16);
        v[2 * i + 1] = u2f(w[i] & 0xFFFF0000u);
      }
    } else {
      const float4 a = *reinterpret_cast<const float4*>(x + cc * 8);
      const float4 b = *reinterpret_cast<const float4*>(x + cc * 8 + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
    int nan = 0;
    // fminf / fmaxf (v_min / v_max) skip NaN operands; the NaN flag stands in
    // for them, and which zero a min or max keeps changes nothing (see above)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      nan |= v[i] != v[i];
      mn = __builtin_fminf(mn, v[i]);
      mx = __builtin_fmaxf(mx, v[i]);
    }
    // over the block's G lanes with DPP: XOR 1 and XOR 2 within quads, then
    // the half-row mirror, which pairs the two quads of 8 lanes
    auto combine = [&](float omn, float omx, int onan) {
      nan |= onan;
      mn = __builtin_fminf(mn, omn);
      mx = __builtin_fmaxf(mx, omx);
    };
    if constexpr (G >= 2) combine(dpp_f<0xB1>(mn), dpp_f<0xB1>(mx), dpp_i<0xB1>(nan));
    if constexpr (G >= 4) combine(dpp_f<0x4E>(mn), dpp_f<0x4E>(mx), dpp_i<0x4E>(nan));
    if constexpr (G >= 8) combine(dpp_f<0x141>(mn), dpp_f<0x141>(mx), dpp_i<0x141>(nan));
    if (nan) mn = mx = __builtin_nanf("");
    float sf, zp;
    if constexpr (sizeof(T) == 2) {
      // both quotients have bf16 operands (qrange a bf16 integer), so a
      // reciprocal multiply rounds like the IEEE division (as for x / sf
      // below), with the same fallback
      const float d = round_to<T>(mx - mn);
      float q1 = d * qr_rcp;
      if (!qr_exact || tiny(q1)) q1 = d / qrange;
      sf = round_to<T>(q1);
      sf = sf > 0.0f ? sf : 1.0f;
      const uint32_t se = (f2u(sf) >> 23) & 0xFFu;
      float q2 = -mn * __builtin_amdgcn_rcpf(sf);
      if (se - 1u >= 252u || tiny(q2)) q2 = -mn / sf;
      zp = round_to<T>(round_to<T>(q2) + qmin);
    } else {
      sf = round_to<T>(round_to<T>(mx - mn) / qrange);
      sf = sf > 0.0f ? sf : 1.0f;
      zp = round_to<T>(round_to<T>(-mn / sf) + qmin);
    }
    if (scale_qmap) {
      sf = round_to<T>(bf2f(scale_qmap[f2bf(sf)]));
      zp = round_to<T>(bf2f(scale_qmap[f2bf(zp)]));
    }
    if (!live) continue;
    if (c % G == 0) {
      // plain stores: these scattered 2-byte words merge in L2 (non-temporal
      // ones took the same time and wrote 3.7 MB more at F3)
      if (scale_out) BT<T>::put(scale_out + c / G, BT<T>::round_bits(sf));
      if (zp_out) BT<T>::put(zp_out + c / G, BT<T>::round_bits(zp));
    }
    // x / sf, rounded to the element type.  bf16: x and sf are both bf16
    // values, so x * rcp(sf) rounds to bf16 exactly as the IEEE quotient does
    // (an exact quotient of two 8-bit significands lies at least 2^-16.86
    // relative from every bf16 rounding midpoint, hazard H7, far beyond the
    // few fp32 ulps of v_rcp_f32 and the product).  A quotient below 2^-124
    // (where bf16 subnormal midpoints can be hit exactly) may round
    // differently, but the output does not depend on it beyond its sign,
    // which the product keeps: with |zp| >= 2^-116 the sum with zp rounds to
    // zp whatever it is; otherwise the sum rounds to an integer zero, and
    // the output is bf16((0 - zp) * sf), or the sign of that zero when zp is
    // 0.  Only where 1 / sf is not a normal float do the elements take the
    // IEEE division.
    float qd[8];
    bool slow = true;
    if constexpr (sizeof(T) == 2) {
      const uint32_t se = (f2u(sf) >> 23) & 0xFFu;
      const float rs = __builtin_amdgcn_rcpf(sf);
      slow = se - 1u >= 252u;
#pragma unroll
      for (int i = 0; i < 8; ++i) qd[i] = v[i] * rs;
    }
    if (slow) {
#pragma unroll
      for (int i = 0; i < 8; ++i) qd[i] = v[i] / sf;
    }
    float o[8];
    // bf16, only finite values in all of the wave's blocks, a normal sf
    // whose reciprocal is normal, and a finite zp: then no intermediate is a
    // NaN (a quotient can still overflow to +-Inf, which v_med3 clamps as the
    // compares do), so the clamp is one v_med3 and the stores go through
    // v_cvt_pk_bf16_f32.  A scale_qmap can round sf to 0 (fp8_e5m3 below its
    // subnormals): then 0 / 0 is a NaN that must reach the output, and
    // v_med3 would turn it into quant_min, so such waves take the compares.
    const bool finite = __builtin_isfinite(mn) && __builtin_isfinite(mx) && __builtin_isfinite(zp) && !slow;
    const bool fast = sizeof(T) == 2 && __builtin_amdgcn_ballot_w64(!finite) == 0;
    if (fast) {
      u32x4 w;
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        uint32_t p = pack_bf16x2(qd[i], qd[i + 1]);
        float a = u2f(p << 16) + zp, b = u2f(p & 0xFFFF0000u) + zp;
        p = pack_bf16x2(a, b);
        a = __builtin_amdgcn_fmed3f(__builtin_rintf(u2f(p << 16)), qmin, qmax) - zp;
        b = __builtin_amdgcn_fmed3f(__builtin_rintf(u2f(p & 0xFFFF0000u)), qmin, qmax) - zp;
        p = pack_bf16x2(a, b);
        w[i / 2] = pack_bf16x2(u2f(p << 16) * sf, u2f(p & 0xFFFF0000u) * sf);
      }
      // the output non-temporally (42.0-42.5 against 42.9-43.6 us at F3
      // with plain stores; non-temporal loads as well were slower)
      if constexpr (sizeof(T) == 2) st_nt(reinterpret_cast<u32x4*>(y + c * 8), w);
      continue;
    }
    if constexpr (sizeof(T) == 2) {
      // the intermediate bf16 roundings two at a time (v_cvt_pk_bf16_f32:
      // RNE as f2bf for every non-NaN value; a NaN stays a NaN, and the
      // final store gives it f2bf's pattern)
      auto rnd2 = [](float& a, float& b) {
        const uint32_t p = pack_bf16x2(a, b);
        a = u2f(p << 16);
        b = u2f(p & 0xFFFF0000u);
      };
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        float a = qd[i], b = qd[i + 1];
        rnd2(a, b);
        a += zp;
        b += zp;
        rnd2(a, b);
        a = __builtin_rintf(a);
        b = __builtin_rintf(b);
        a = a < qmin ? qmin : (a > qmax ? qmax : a);  // NaN stays NaN
        b = b < qmin ? qmin : (b > qmax ? qmax : b);
        a -= zp;
        b -= zp;
        rnd2(a, b);
        o[i] = a * sf;
        o[i + 1] = b * sf;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float q = __builtin_rintf(round_to<T>(round_to<T>(qd[i]) + zp));
        q = q < qmin ? qmin : (q > qmax ? qmax : q);  // NaN stays NaN
        o[i] = round_to<T>(q - zp) * sf;
      }
    }
    if constexpr (sizeof(T) == 2) {
      u32x4 w;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = (uint32_t)BT<T>::round_bits(o[2 * i]) | ((uint32_t)BT<T>::round_bits(o[2 * i + 1]) << 16);
      st_nt(reinterpret_cast<u32x4*>(y + c * 8), w);
    } else {
      *reinterpret_cast<float4*>(y + c * 8) = float4{o[0], o[1], o[2], o[3]};
      *reinterpret_cast<float4*>(y + c * 8 + 4) = float4{o[4], o[5], o[6], o[7]};
    }
  }
}

template <typename T>
static void launch_gwa_rows(const void* x, int64_t n, int64_t bs, float qmin, float qmax, const uint16_t* sq,
                            void* sc, void* zp, void* y, hipStream_t st) {
  const int64_t nchunks = n / 8;
  const unsigned grid = grid_for(nchunks, 256);
  const T* xx = static_cast<const T*>(x);
  T *s = static_cast<T*>(sc), *z = static_cast<T*>(zp), *yy = static_cast<T*>(y);
  switch (bs) {
    case 8: hipLaunchKernelGGL((gwa_fq_rows_kernel<T, 1>), dim3(grid), dim3(256), 0, st, xx, nchunks, qmin, qmax, sq, s, z, yy); break;
    case 16: hipLaunchKernelGGL((gwa_fq_rows_kernel<T, 2>), dim3(grid), dim3(256), 0, st, xx, nchunks, qmin, qmax, sq, s, z, yy); break;
    case 32: hipLaunchKernelGGL((gwa_fq_rows_kernel<T, 4>), dim3(grid), dim3(256), 0, st, xx, nchunks, qmin, qmax, sq, s, z, yy); break;
    default: hipLaunchKernelGGL((gwa_fq_rows_kernel<T, 8>), dim3(grid), dim3(256), 0, st, xx, nchunks, qmin, qmax, sq, s, z, yy); break;
  }
}

int gwa_fake_quant(const void* x, int dtype, int64_t outer, int64_t L, int64_t inner, int64_t bs, float qmin,
                   float qmax, const uint16_t* scale_qmap, void* scale_out, void* zp_out, void* y,
                   hipStream_t st) {
  if (outer < 0 || L < 0 || inner < 0) return set_error(kErrInvalid, "gwa_fake_quant: negative shape");
  if (bs < 1) return set_error(kErrInvalid, "gwa_fake_quant: block_size must be >= 1");
  if (!(qmax > qmin)) return set_error(kErrInvalid, "gwa_fake_quant: quant_max must exceed quant_min");
  const int64_t total = outer * ((L + bs - 1) / bs) * inner;
  if (total == 0) return kOk;
  if (!x || !y) return set_error(kErrInvalid, "gwa_fake_quant: null tensor");
  const bool rows = inner == 1 && (bs == 8 || bs == 16 || bs == 32 || bs == 64) && L % bs == 0 &&
                    aligned(x, 32) && aligned(y, 32) && (dtype == kBF16 || dtype == kF32);
  if (rows) {
    if (dtype == kBF16)
      launch_gwa_rows<uint16_t>(x, outer * L, bs, qmin, qmax, scale_qmap, scale_out, zp_out, y, st);
    else
      launch_gwa_rows<float>(x, outer * L, bs, qmin, qmax, scale_qmap, scale_out, zp_out, y, st);
    return check_launch("gwa_fake_quant");
  }
  const unsigned grid = grid_for(total, 256);
  if (dtype == kBF16)
    hipLaunchKernelGGL(gwa_fq_kernel<uint16_t>, dim3(grid), dim3(256), 0, st, (const uint16_t*)x, outer, L, inner,
                       bs, qmin, qmax, scale_qmap, (uint16_t*)scale_out, (uint16_t*)zp_out, (uint16_t*)y);
  else if (dtype == kF32)
    hipLaunchKernelGGL(gwa_fq_kernel<float>, dim3(grid), dim3(256), 0, st, (const float*)x, outer, L, inner, bs,
                       qmin, qmax, scale_qmap, (float*)scale_out, (float*)zp_out, (float*)y);
  else
    return set_error(kErrInvalid, "gwa_fake_quant: input dtype %d not supported (bf16 or fp32)", dtype);
  return check_launch("gwa_fake_quant");
}

// ---------------------------------------------------------------------------
// LUT fast path: bf16 input, blocks of 16*LPB along the last dim.
// ---------------------------------------------------------------------------
// RN_bf16(x / s) for bf16-valued x and s (s normal with a normal reciprocal):
// q = x * rcp(s) is within 1.5 ulp32 of x / s, so its bf16 rounding is the
// exact one unless q lies within a few ulp32 of a bf16 midpoint, where the
// IEEE division decides.  (An exact quotient of two 8-bit significands is
// either a bf16 midpoint itself or at least 2^-17 away from every midpoint,
// so the fp32 division's own rounding never moves it across one.)
__device__ __forceinline__ uint32_t div_bf16_fast(float x, float s, float r) {
  float q = x * r;
  uint32_t qb = f2u(q);
  if ((qb & 0xFFFFu) - 0x7FFCu <= 8u) qb = f2u(x / s);
  return f2bf(u2f(qb));
}


typedef __attribute__((address_space(3))) const uint32_t lds_cu32;
typedef __attribute__((address_space(3))) const uint8_t lds_cu8;
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Power-of-two block scale of a bf16 block (block_scale<uint16_t> mode 0)
// with the floor(bf16 log2) step thresholds read from an LDS byte table
// indexed by the exponent field.
__device__ __forceinline__ float block_scale_pow2_lds(uint32_t amax, int shift, const uint8_t* thr) {
  uint32_t E = amax >> 7, m = amax & 0x7Fu;
  int lf = (int)E - 127 + (m >= thr[E] ? 1 : 0);
  if (E == 0) lf = amax == 0 ? -126 : log2floor_bf16(amax);  // zero or subnormal amax
  int e = lf - shift;
  float sc = e > 127 ? __builtin_huge_valf() : (e >= -133 ? exp2i(e) : 1.0f);
  sc = amax == 0x7F80u ? __builtin_huge_valf() : sc;
  return amax > 0x7F80u ? 1.0f : sc;
}

// Wave layout of the table kernels.  A wave streams 1024-element chunks,
// lane L taking group L of the chunk (elements 16 L .. 16 L + 15), with each
// load instruction covering one contiguous 1 KiB: load a brings the first
// half of the chunk and load b the second, lanes 0-31 taking the even
// 16-byte slots of a half (elements 16 L .. 16 L + 7 of it) and lanes 32-63
// the odd ones (16 (L - 32) + 8 .. + 15).  One v_permlane32_swap per dword
// then gives lane L < 32 its group as (a, a of lane L + 32) and lane L >= 32
// as (b of lane L - 32, b).  (Loading each lane's own 32 contiguous bytes
// instead leaves every load instruction half-filling its cache lines, which
// costs about a fifth of the read rate at these sizes.)  The swap is its own
// inverse, so it also turns a lane's 16 outputs back into two contiguous
// 1 KiB stores at the same slots.
__device__ __forceinline__ uint32_t half_slot(int lane) { return lane < 32 ? 2 * lane : 2 * (lane - 32) + 1; }

__device__ __forceinline__ void half_swap(u32x4& a, u32x4& b) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(a[i], b[i], false, false);
    a[i] = r[0];
    b[i] = r[1];
  }
}

// WANT: bit 0 = reference quantize() values, bit 1 = fake-quant values.
// CT: packed codes only (WANT 0, CB 4 or 8), read from the codes-only LDS
// tables (lut_codes_to_lds) and packed with ORs and byte permutes.
//
// Fast path per element: the quotient (one multiply; for absmax scales a
// reciprocal multiply whose rare near-midpoint cases are redone by IEEE
// division for the whole group), its magnitude clamped into the table range
// [T0 - 1, T1] with v_med3_f32 (clamping before the bf16 rounding equals
// clamping after it, the bounds being bf16 values), one compare against a
// uniform threshold picking the sign's table base, and one LDS read at that
// base plus the clamped quotient's bf16 bits, scaled to the entry size.
// 1024 threads: sixteen waves share one copy of the tables and each
// workgroup's fill serves them all (C2 20.1-20.4 us with 256 threads,
// 19.8-19.9 with 1024; C3 e4m3 36.7 -> 35.4, e2m1 31.0 -> 30.2, fake-quant
// 51.2 -> 49.4; e3m2 unchanged)
constexpr int kMxLutThreads = 1024;

// OUTL: outlier masking (fake-quant output only): elements with |x| at or
// above the threshold are zeros for the block max and the encode, and the
// output restores them; the kernel counts them into the device stats.
template <int CB, int LPB, bool ABSMAX, int WANT, bool CT, bool OUTL = false>
__global__ __launch_bounds__(kMxLutThreads) void mx_lut_kernel(const uint16_t* __restrict__ x, int64_t ngroups,
                                                     ScaleParams sp, LutView lv, MxOut out, OutlierArgs oa) {
  static_assert(!CT || (WANT == 0 && (CB == 4 || CB == 8)), "code tables serve packed 4- or 8-bit codes only");
  static_assert(!OUTL || (WANT == 2 && CB == 0 && !CT), "outlier masking serves the fake-quant output only");
  const uint32_t obound = OUTL ? outlier_bound_t<uint16_t>(oa) : 0xFFFFFFFFu;
  uint32_t nskip = 0;
  extern __shared__ uint32_t lds_lut[];
  __shared__ uint8_t thr8[256];
  const int lane = threadIdx.x & 63;
  // whole 1024-element chunks, one per wave and trip (wave-uniform indices),
  // in the swapped layout; the groups past the last whole chunk after them,
  // one per thread, in the plain layout
  const int64_t nchunks = ngroups / 64;
  const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x / 64);
  int64_t c = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6)));
  const u32x4* xv = reinterpret_cast<const u32x4*>(x);
  // input loads non-temporal: with the input streaming from HBM (inputs
  // larger than the MALL, or not left there by the launch before) they are
  // faster than plain loads (C3 e4m3 38.5 -> 36.9, e3m2 35.4 -> 33.9, e2m1
  // 33.6 -> 32.1, fake-quant 51.5 -> 50.6 us); plain loads win only when the
  // same input is re-read from the MALL back to back
  auto ld_x = [](const u32x4* p) { return ld_nt(p); };
  const uint32_t slot = half_slot(lane);
  // the first chunk's loads are in flight while the tables fill LDS
  u32x4 n0 = {0, 0, 0, 0}, n1 = {0, 0, 0, 0};
  if (c < nchunks) {
    n0 = ld_x(xv + c * 128 + slot);
    n1 = ld_x(xv + c * 128 + 64 + slot);
  }
  if constexpr (!ABSMAX)
    for (int i = threadIdx.x; i < 256; i += blockDim.x) thr8[i] = (uint8_t)log2_step_threshold(i);
  LutLds t;
  if constexpr (CT)
    t = lut_codes_to_lds<CB>(lv.blob, lv.len, lds_lut);
  else
    t = lut_to_lds(lv.blob, lv.len, lds_lut);
  const uint32_t* full = lv.blob + kLutHeaderWords + 2 * kLutMaxLen;
  // LDS byte addresses such that entry(h) = base + ES h for h in [T0 - 1, T1]
  // (ES = 4 bytes per entry, 1 for the code tables); nb passes through
  // readfirstlane so that the compiler keeps the per-element form
  // select(pb, nb) + ES h
  constexpr uint32_t ES = CT ? 1u : 4u;
  const uint32_t pb = (uint32_t)(size_t)(lds_cu32*)lds_lut - ES * t.t0m1;
  const uint32_t nb = __builtin_amdgcn_readfirstlane(pb + ES * t.len);
  const float lo = u2f(t.t0m1 << 16), hi = u2f(t.t1 << 16);
  // absmax: a power-of-two quant_max divides exactly as a multiply
  const bool qmax_pow2 = (f2u(sp.quant_max) & 0x807FFFFFu) == 0 && ((f2u(sp.quant_max) >> 23) - 1u) < 253u;
  const float qmax_rcp = u2f((254u - (f2u(sp.quant_max) >> 23)) << 23);

  // One group of 16 consecutive elements (wx, as bf16 pairs), group index gl.
  // SW: a whole chunk in the swapped layout (every lane of the wave active).
  auto group = [&](auto sw, const uint32_t(&wx)[8], int64_t gl) {
    constexpr bool SW = decltype(sw)::value;
    // w: the group with its outliers zeroed (OUTL), else the input itself
    uint32_t w[8];
    uint32_t skip = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      w[j] = wx[j];
      if constexpr (OUTL) {
        const bool lo = outlier_skip(wx[j] & 0x7FFFu, obound, 0x7F80u);
        const bool hi = outlier_skip((wx[j] >> 16) & 0x7FFFu, obound, 0x7F80u);
        skip |= ((uint32_t)lo << (2 * j)) | ((uint32_t)hi << (2 * j + 1));
        w[j] &= (lo ? 0xFFFF0000u : 0xFFFFFFFFu) & (hi ? 0x0000FFFFu : 0xFFFFFFFFu);
      }
    }
    if constexpr (OUTL) nskip += __builtin_popcount(skip);
    u16x2 m2 = {0, 0};  // magnitude maxima of the low and high halves
#pragma unroll
    for (int j = 0; j < 8; ++j) m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, w[j] & 0x7FFF7FFFu));
    const uint32_t amax = block_max<LPB>((uint32_t)(m2.x > m2.y ? m2.x : m2.y));
    float s;
    if constexpr (ABSMAX) {
      if (qmax_pow2 && !sp.scale_qmap) {
        // the hardware RNE; a NaN or Inf amax gives NaN / Inf either way,
        // and NaN then takes scale 1 below as with the software rounding
        const float sc = u2f(pack_bf16x2(u2f(amax << 16) * qmax_rcp, 0.0f) << 16);
        s = sc > 0.0f ? sc : 1.0f;
      } else {
        s = block_scale_bf16<true>(amax, sp);
      }
    } else {
      s = block_scale_pow2_lds(amax, sp.shift, thr8);
    }
    uint32_t sb = f2u(s);
    uint32_t sE = (sb >> 23) & 0xFFu;
    const float amaxf = u2f(amax << 16);
    bool fast;
    float rcp;
    uint32_t nthr;  // sign rule: the negative table iff (fp32 bits) > nthr
    if constexpr (!ABSMAX) {
      // a power of two in [2^-100, 2^100]: x / s and v * s are exact
      // scalings (quotients below bf16's normal range only reach the table's
      // entry 0, as T0 is above it), and the largest quotient stays below S;
      // a quotient keeps its sign unless it rounds to a bf16 zero, i.e.
      // unless |x| <= 2^-134 s: compared on x's bits
      rcp = u2f((254u - sE) << 23);
      fast = (sb & 0x7FFFFFu) == 0 && sE >= 27 && sE <= 227 && amax < 0x7F80u && t.t0m1 >= 0x80u &&
             (f2u(amaxf * rcp) >> 16) < t.s;
      int ze = (int)sE - 127 - 134;
      float sz = ze >= -149 ? exp2i(ze) : 0.0f;
      nthr = t.zsign ? 0x7FFFFFFFu : (0x80000000u | f2u(sz));
    } else {
      // the quotient q rounds to a bf16 below -0 iff q < -2^-134 (2^-134 is
      // a midpoint, so q is exact there), or to -0 or below iff q is negative
      rcp = __builtin_amdgcn_rcpf(s);
      fast = sE >= 2 && sE <= 252 && amax < 0x7F80u && t.t0m1 >= 0x80u &&
             (f2u(amaxf * rcp) >> 16) + 1u < t.s;
      nthr = t.zsign ? 0x7FFFFFFFu : 0x80008000u;
    }
    uint32_t ent[16];
    if (fast) {
      uint32_t addr[16];
      if constexpr (!ABSMAX) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          uint32_t xb = (j & 1) ? (w[j >> 1] & 0xFFFF0000u) : (w[j >> 1] << 16);
          float qc = __builtin_amdgcn_fmed3f(__builtin_fabsf(u2f(xb) * rcp), lo, hi);
          addr[j] = (xb > nthr ? nb : pb) + ES * (f2u(qc) >> 16);  // qc is a bf16 value
        }
      } else {
        // x and s are bf16 values (8-bit significands), so x / s is at least
        // 2^-17 (relative) away from every bf16 rounding midpoint, while
        // x * rcp(s) is within 2^-22 of x / s (v_rcp_f32: 1 ulp, then the
        // product's rounding): its bf16 rounding is that of the reference's
        // fp32 division, with no check needed
        float q[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          uint32_t xb = (j & 1) ? (w[j >> 1] & 0xFFFF0000u) : (w[j >> 1] << 16);
          q[j] = u2f(xb) * rcp;
        }
#pragma unroll
        for (int j = 0; j < 16; j += 2) {
          // clamped magnitudes are normal and finite: hardware RNE is exact;
          // one conversion rounds the pair
          const uint32_t hh = pack_bf16x2(__builtin_amdgcn_fmed3f(__builtin_fabsf(q[j]), lo, hi),
                                          __builtin_amdgcn_fmed3f(__builtin_fabsf(q[j + 1]), lo, hi));
          addr[j] = (f2u(q[j]) > nthr ? nb : pb) + ES * (hh & 0xFFFFu);
          addr[j + 1] = (f2u(q[j + 1]) > nthr ? nb : pb) + ES * (hh >> 16);
        }
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if constexpr (CT)
          ent[j] = *(lds_cu8*)(size_t)(addr[j] + ((CB == 4 && (j & 1)) ? (uint32_t)kCodeCopy2 : 0u));
        else
          ent[j] = *(lds_cu32*)(size_t)addr[j];
      }
    } else {
      // scale 1 (NaN block), Inf, subnormal or extreme: exact division and
      // the full table (unrolled: a rolled loop would index w and ent
      // dynamically and pin their registers for the whole kernel)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        uint32_t xb = (j & 1) ? (w[j >> 1] & 0xFFFF0000u) : (w[j >> 1] << 16);
        const float q = u2f(xb) / s;
        uint32_t h = f2bf(q);
        // a NaN quotient takes x's sign (as div_to_bf16 gives it)
        h = q == q ? h : (h & 0x7FFFu) | ((xb >> 16) & 0x8000u);
        uint32_t e = full[h];
        if constexpr (CT) e = (CB == 4 && (j & 1)) ? (e >> 16) << 4 : e >> 16;
        ent[j] = e;
      }
    }
    if constexpr (WANT != 0) {
      uint32_t qv[16], fv[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        uint32_t v = ent[j] & 0xFFFFu;
        qv[j] = v;
        // pow2 scales on the fast path multiply exactly
        fv[j] = (ABSMAX || !fast) ? f2bf(u2f(v << 16) * s) : (f2u(u2f(v << 16) * s) >> 16);
      }
      if constexpr (OUTL) {
        if (skip) {
#pragma unroll
          for (int j = 0; j < 16; ++j)
            fv[j] = (skip >> j) & 1u ? ((j & 1) ? wx[j >> 1] >> 16 : wx[j >> 1] & 0xFFFFu) : fv[j];
        }
      }
      auto store = [&](uint16_t* base, const uint32_t(&b)[16]) {
        if constexpr (SW) {
          u32x4 a0 = {b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
          u32x4 a1 = {b[8] | (b[9] << 16), b[10] | (b[11] << 16), b[12] | (b[13] << 16), b[14] | (b[15] << 16)};
          half_swap(a0, a1);
          u32x4* p = reinterpret_cast<u32x4*>(base + (gl - lane) * 16);
          st_nt(p + slot, a0);
          st_nt(p + 64 + slot, a1);
        } else {
          BT<uint16_t>::store16(base + gl * 16, b);
        }
      };
      if constexpr (WANT & 1) store(static_cast<uint16_t*>(out.qvals), qv);
      if constexpr (WANT & 2) store(static_cast<uint16_t*>(out.fq), fv);
    }
    if constexpr (CT && CB == 4) {
      uint32_t b[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) b[k] = ent[2 * k] | ent[2 * k + 1];
      u32x2 cw = {pack_low_bytes(b[0], b[1], b[2], b[3]), pack_low_bytes(b[4], b[5], b[6], b[7])};
      st_nt(reinterpret_cast<u32x2*>(static_cast<uint8_t*>(out.codes) + gl * 8), cw);
    } else if constexpr (CT) {
      u32x4 cw = {pack_low_bytes(ent[0], ent[1], ent[2], ent[3]), pack_low_bytes(ent[4], ent[5], ent[6], ent[7]),
                  pack_low_bytes(ent[8], ent[9], ent[10], ent[11]),
                  pack_low_bytes(ent[12], ent[13], ent[14], ent[15])};
      st_nt(reinterpret_cast<u32x4*>(static_cast<uint8_t*>(out.codes) + gl * 16), cw);
    } else if constexpr (CB > 0) {
      uint32_t code[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) code[j] = ent[j] >> 16;
      store_group_codes<CB>(static_cast<uint8_t*>(out.codes), gl, code);
    }
    if ((gl & (LPB - 1)) == 0) {
      int64_t blk = gl / LPB;
      // plain stores: a chunk's scales are 32-64 contiguous bytes, and the
      // L2 merges the neighbouring chunks' pieces into whole lines before
      // they reach HBM (non-temporal stores sent each piece on its own:
      // C3 e4m3 36.9 -> 35.8, fake-quant 50.6 -> 49.4, C2 22.6 -> 22.1 us)
      if (out.scale) static_cast<uint16_t*>(out.scale)[blk] = (uint16_t)f2bf(s);
      if (out.scale_f32) out.scale_f32[blk] = s;
      if (out.scale_e8m0) out.scale_e8m0[blk] = (uint8_t)e8m0_of(s);
    }
  };

  for (; c < nchunks; c += nwaves) {
    u32x4 a = n0, b = n1;
    if (c + nwaves < nchunks) {  // prefetch the next chunk
      n0 = ld_x(xv + (c + nwaves) * 128 + slot);
      n1 = ld_x(xv + (c + nwaves) * 128 + 64 + slot);
    }
    half_swap(a, b);
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    group(std::true_type{}, w, c * 64 + lane);
  }
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t g = nchunks * 64 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < ngroups; g += stride) {
    const u32x4 a = ld_x(xv + 2 * g), b = ld_x(xv + 2 * g + 1);
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    group(std::false_type{}, w, g);
  }
  if constexpr (OUTL) outlier_tally(nskip, oa);
}

template <int CB, int LPB, bool ABSMAX, int WANT>
static int launch_lut_k(const uint16_t* x, int64_t ngroups, const ScaleParams& sp, const LutView& lv,
                        const MxOut& out, hipStream_t st) {
  const int bs = kMxLutThreads;
  // codes-only outputs use the code tables where they fit
  constexpr bool kCodes = WANT == 0 && (CB == 4 || CB == 8);
  if (kCodes && (CB == 8 || (int64_t)lv.len * 2 <= kCodeCopy2)) {
    auto k = mx_lut_kernel<CB, LPB, ABSMAX, WANT, kCodes>;
    size_t lds = CB == 4 ? kCodeCopy2 + (size_t)lv.len * 2 : (size_t)lv.len * 2;
    unsigned grid = persistent_grid((const void*)k, bs, lds, ngroups);
    hipLaunchKernelGGL(k, dim3(grid), dim3(bs), lds, st, x, ngroups, sp, lv, out, OutlierArgs{});
  } else {
    auto k = mx_lut_kernel<CB, LPB, ABSMAX, WANT, false>;
    size_t lds = sizeof(uint32_t) * 2 * lv.len;
    unsigned grid = persistent_grid((const void*)k, bs, lds, ngroups);
    hipLaunchKernelGGL(k, dim3(grid), dim3(bs), lds, st, x, ngroups, sp, lv, out, OutlierArgs{});
  }
  return check_launch("mx_quantize(lut)");
}

// Blocks along a middle axis of a bf16 input, table-driven: the layout and
// per-column block scales of mx_cols_kernel, the per-element path of
// mx_lut_kernel.  A persistent workgroup copies the format's compact table
// (value | code << 16 per magnitude, both signs) into LDS once; a column's
// block whose scale passes the same checks as mx_lut_kernel's fast path
// (ABSMAX: x * rcp(s) rounds to the bf16 of the reference's x / s, as x and s
// are bf16 values; power-of-two scales: an exact scaling) takes a clamp and
// one LDS read per element, any other block the exact division and the full
// table.  Outputs and outlier handling as mx_cols_kernel (OUTL: outlier
// masking active).
//
// A tile is one block by 128 columns; thread (rg, cg) = (tid / 16, tid % 16)
// holds 16 bytes (8 columns) of rows rg, rg + 16, ... (R rows).  The work is
// done on bf16 pairs as loaded: block maxima with packed 16-bit maxima,
// outliers as per-pair masks, two quotients rounded by one conversion, and
// the fake-quant pair assembled by one conversion (or one byte permute for
// the exact power-of-two products) and one bit select restoring outliers.
// A tile's R rows are loaded together, one tile ahead: the next tile's loads
// are issued once this tile's scales are known (its last global read) and
// land while it is encoded and stored.  A row outside the block or the
// tensor, or a chunk past inner, reads the block's first row at column 0
// (in bounds) and is replaced by zeros before use, so no branch sits between
// the loads; past the last tile the last one is read again.
template <bool ABSMAX, int R, bool OUTL>
__global__ __launch_bounds__(256) void mx_cols_lut_kernel(const uint16_t* __restrict__ x, int64_t outer, int64_t L,
                                                          int64_t inner, int bs, ScaleParams sp, LutView lv,
                                                          MxOut out, int code_bytes, OutlierArgs oa) {
  static_assert(R >= 1 && R <= kColRowsMax, "rows per thread");
  constexpr int VE = 8;
  constexpr int TW = kColChunks * VE;
  extern __shared__ uint32_t lds_lut[];
  __shared__ uint32_t s_amax[256 / kColChunks][TW / 2];  // column maxima of each row group, as pairs
  __shared__ float s_scale[TW];
  __shared__ uint32_t s_cmax[TW];
  const LutLds t = lut_to_lds(lv.blob, lv.len, lds_lut);
  const uint32_t* full = lv.blob + kLutHeaderWords + 2 * kLutMaxLen;
  const uint32_t pb = (uint32_t)(size_t)(lds_cu32*)lds_lut - 4u * t.t0m1;
  const uint32_t nb = pb + 4u * t.len;
  const float lo = u2f(t.t0m1 << 16), hi = u2f(t.t1 << 16);
  const int tid = threadIdx.x, cg = tid % kColChunks, rg = tid / kColChunks;
  // tile coordinates in 32-bit arithmetic (the host checks ntiles < 2^31)
  const uint32_t nblk = (uint32_t)((L + bs - 1) / bs);
  const uint32_t ntc = (uint32_t)((inner + TW - 1) / TW);
  const uint32_t ntiles = (uint32_t)(outer * nblk * ntc);
  // outlier bound on the magnitude bits (0xFFFF: nothing is an outlier)
  const uint32_t bound = OUTL ? outlier_bound_t<uint16_t>(oa) : 0xFFFFFFFFu;
  const u16x2 b16 = {(unsigned short)(bound > 0xFFFFu ? 0xFFFFu : bound),
                     (unsigned short)(bound > 0xFFFFu ? 0xFFFFu : bound)};
  uint32_t nskip = 0;
  auto load_tile = [&](uint32_t tile, u32x4(&dst)[R]) {
    const uint32_t tc = tile % ntc, rest = tile / ntc;
    const uint32_t bl = rest % nblk, o = rest / nblk;
    const int64_t l0 = (int64_t)bl * bs;
    const int64_t col = (int64_t)tc * TW + (int64_t)cg * VE;
    const bool cok = col < inner;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int64_t l = l0 + rg + 16 * i;
      const bool ok = rg + 16 * i < bs && l < L;
      dst[i] = *reinterpret_cast<const u32x4*>(x + ((int64_t)o * L + (ok ? l : l0)) * inner + (cok ? col : 0));
    }
  };
  u32x4 w[R], wn[R];
  load_tile(blockIdx.x < ntiles ? blockIdx.x : ntiles - 1, w);
  for (uint32_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const uint32_t tc = tile % ntc, rest = tile / ntc;
    const uint32_t bl = rest % nblk, o = rest / nblk;
    const int64_t l0 = (int64_t)bl * bs;
    const int64_t col = (int64_t)tc * TW + (int64_t)cg * VE;
    const bool cok = col < inner;
    bool rok[R];
    u32x4 mk[R];  // OUTL: 0xFFFF over the outlier halves
    u16x2 mp[4] = {{0, 0}, {0, 0}, {0, 0}, {0, 0}};  // magnitude maxima of columns 2j, 2j + 1
    u16x2 cnt = {0, 0};                               // outliers among the low / high halves
#pragma unroll
    for (int i = 0; i < R; ++i) {
      rok[i] = rg + 16 * i < bs && l0 + rg + 16 * i < L && cok;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        w[i][j] = rok[i] ? w[i][j] : 0u;
        u16x2 mg = __builtin_bit_cast(u16x2, w[i][j] & 0x7FFF7FFFu);
        if constexpr (OUTL) {
          // outlier_skip on both halves with packed 16-bit arithmetic:
          // bound <= mag (mag + 1 - bound > 0) and mag <= 0x7F80 (not NaN),
          // each a saturating difference, and-ed as 0 / 1 by minima
          const u16x2 ge = __builtin_elementwise_sub_sat(mg + (u16x2){1, 1}, b16);
          const u16x2 le = __builtin_elementwise_sub_sat((u16x2){0x7F81, 0x7F81}, mg);
          u16x2 one = __builtin_elementwise_min(__builtin_elementwise_min(ge, le), (u16x2){1, 1});
          one = rok[i] ? one : (u16x2){0, 0};  // the zeros standing in for rows or chunks outside
          cnt += one;
          mk[i][j] = __builtin_bit_cast(uint32_t, (u16x2){0, 0} - one);
          mg = __builtin_bit_cast(u16x2, __builtin_bit_cast(uint32_t, mg) & ~mk[i][j]);
        } else {
          mk[i][j] = 0u;
        }
        mp[j] = __builtin_elementwise_max(mp[j], mg);
      }
    }
    if constexpr (OUTL) nskip += (uint32_t)cnt.x + (uint32_t)cnt.y;
#pragma unroll
    for (int j = 0; j < 4; ++j) s_amax[rg][cg * 4 + j] = __builtin_bit_cast(uint32_t, mp[j]);
    __syncthreads();
    if (tid < TW) {
      uint32_t a = 0;
#pragma unroll
      for (int g = 0; g < 256 / kColChunks; ++g) a = umax32(a, (s_amax[g][tid >> 1] >> (16 * (tid & 1))) & 0xFFFFu);
      const float sc = block_scale<uint16_t>(a, sp);
      s_scale[tid] = sc;
      s_cmax[tid] = a;
      const int64_t c = (int64_t)tc * TW + tid;
      if (c < inner) {
        const int64_t si = ((int64_t)o * nblk + bl) * inner + c;
        if (out.scale) static_cast<uint16_t*>(out.scale)[si] = (uint16_t)BT<uint16_t>::round_bits(sc);
        if (out.scale_f32) out.scale_f32[si] = sc;
        if (out.scale_e8m0) out.scale_e8m0[si] = (uint8_t)e8m0_of(sc);
      }
    }
    __syncthreads();
    {
      const uint32_t next = tile + gridDim.x;  // < 2^32: tile < 2^31, gridDim.x < 2^31
      load_tile(next < ntiles ? next : ntiles - 1, wn);
    }
    // per column: the scale, its reciprocal, whether the table path holds
    // for the column's block, and the sign rule (the negative table iff the
    // fp32 bits of the quotient (ABSMAX) or of x (power of two) > nthr)
    float s[VE], rcp[VE];
    bool fast[VE];
    uint32_t nthr[VE];
    bool all_fast = true;
#pragma unroll
    for (int e = 0; e < VE; ++e) {
      s[e] = s_scale[cg * VE + e];
      const uint32_t amax = s_cmax[cg * VE + e];
      const uint32_t sb = f2u(s[e]), sE = (sb >> 23) & 0xFFu;
      const float amaxf = u2f(amax << 16);
      if constexpr (ABSMAX) {
        rcp[e] = __builtin_amdgcn_rcpf(s[e]);
        fast[e] = sE >= 2 && sE <= 252 && amax < 0x7F80u && t.t0m1 >= 0x80u && (f2u(amaxf * rcp[e]) >> 16) + 1u < t.s;
        nthr[e] = t.zsign ? 0x7FFFFFFFu : 0x80008000u;
      } else {
        rcp[e] = u2f((254u - sE) << 23);
        fast[e] = (sb & 0x7FFFFFu) == 0 && sE >= 27 && sE <= 227 && amax < 0x7F80u && t.t0m1 >= 0x80u &&
                  (f2u(amaxf * rcp[e]) >> 16) < t.s;
        const int ze = (int)sE - 127 - 134;
        const float sz = ze >= -149 ? exp2i(ze) : 0.0f;
        nthr[e] = t.zsign ? 0x7FFFFFFFu : (0x80000000u | f2u(sz));
      }
      rcp[e] = cok ? rcp[e] : 0.0f;  // a chunk past inner: quotients of 0 (its rows are zeros)
      all_fast = all_fast && fast[e];
    }
    // Row i's outputs from its eight entries (value | code << 16), as pairs.
    auto emit = [&](int i, const uint32_t(&ent)[VE]) {
      u32x4 qv, fv;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t el = ent[2 * j], eh = ent[2 * j + 1];
        qv[j] = __builtin_amdgcn_perm(eh, el, 0x05040100u);
        const float vl = u2f(el << 16) * s[2 * j], vh = u2f(eh << 16) * s[2 * j + 1];
        uint32_t f;
        if (ABSMAX || !(fast[2 * j] && fast[2 * j + 1]))
          f = pack_bf16x2(vl, vh);  // RNE (the products are finite: table values times normal scales)
        else
          f = __builtin_amdgcn_perm(f2u(vh), f2u(vl), 0x07060302u);  // exact power-of-two products
        fv[j] = (mk[i][j] & w[i][j]) | (~mk[i][j] & f);  // an outlier keeps its input
      }
      const int64_t base = ((int64_t)o * L + l0 + rg + 16 * i) * inner + col;
      if (out.qvals) *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out.qvals) + base) = qv;
      if (out.fq) *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out.fq) + base) = fv;
      if (out.codes) {
        if (code_bytes == 1) {
#pragma unroll
          for (int e = 0; e < VE; ++e) static_cast<uint8_t*>(out.codes)[base + e] = (uint8_t)(ent[e] >> 16);
        } else {
#pragma unroll
          for (int e = 0; e < VE; ++e) static_cast<uint16_t*>(out.codes)[base + e] = (uint16_t)(ent[e] >> 16);
        }
      }
    };
    // A chunk past inner takes no part in the wave's choice (its scales are
    // those of empty columns).  When every chunk of the wave is on the table
    // path, all its entries are read with no branch between the reads.
    if (__all(all_fast || !cok)) {
      uint32_t ent[R][VE];
#pragma unroll
      for (int i = 0; i < R; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t wmj = w[i][j] & ~mk[i][j];  // outliers encode as +0
          const float xl = u2f(wmj << 16), xh = u2f(wmj & 0xFFFF0000u);
          uint32_t al, ah;
          if constexpr (ABSMAX) {
            const float ql = xl * rcp[2 * j], qh = xh * rcp[2 * j + 1];
            // clamped magnitudes are normal and finite: hardware RNE is exact
            const uint32_t hh = pack_bf16x2(__builtin_amdgcn_fmed3f(__builtin_fabsf(ql), lo, hi),
                                            __builtin_amdgcn_fmed3f(__builtin_fabsf(qh), lo, hi));
            al = (f2u(ql) > nthr[2 * j] ? nb : pb) + 4u * (hh & 0xFFFFu);
            ah = (f2u(qh) > nthr[2 * j + 1] ? nb : pb) + 4u * (hh >> 16);
          } else {
            // the clamped quotients are bf16 values: their high halves
            const float cl = __builtin_amdgcn_fmed3f(__builtin_fabsf(xl * rcp[2 * j]), lo, hi);
            const float ch = __builtin_amdgcn_fmed3f(__builtin_fabsf(xh * rcp[2 * j + 1]), lo, hi);
            al = (f2u(xl) > nthr[2 * j] ? nb : pb) + 4u * (f2u(cl) >> 16);
            ah = (f2u(xh) > nthr[2 * j + 1] ? nb : pb) + 4u * (f2u(ch) >> 16);
          }
          ent[i][2 * j] = *(lds_cu32*)(size_t)al;
          ent[i][2 * j + 1] = *(lds_cu32*)(size_t)ah;
        }
      }
#pragma unroll
      for (int i = 0; i < R; ++i)
        if (rok[i]) emit(i, ent[i]);
    } else {
#pragma unroll
      for (int i = 0; i < R; ++i) {
        if (!rok[i]) continue;
        uint32_t ent[VE];
#pragma unroll
        for (int e = 0; e < VE; ++e) {
          const uint32_t wmj = w[i][e >> 1] & ~mk[i][e >> 1];
          const uint32_t xb = (e & 1) ? (wmj & 0xFFFF0000u) : (wmj << 16);
          if (fast[e]) {
            uint32_t addr;
            if constexpr (ABSMAX) {
              const float q = u2f(xb) * rcp[e];
              const uint32_t h = pack_bf16x2(__builtin_amdgcn_fmed3f(__builtin_fabsf(q), lo, hi), 0.0f);
              addr = (f2u(q) > nthr[e] ? nb : pb) + 4u * h;
            } else {
              const float qc = __builtin_amdgcn_fmed3f(__builtin_fabsf(u2f(xb) * rcp[e]), lo, hi);
              addr = (xb > nthr[e] ? nb : pb) + 4u * (f2u(qc) >> 16);
            }
            ent[e] = *(lds_cu32*)(size_t)addr;
          } else {
            const float q = u2f(xb) / s[e];
            uint32_t h = f2bf(q);
            h = q == q ? h : (h & 0x7FFFu) | ((xb >> 16) & 0x8000u);
            ent[e] = full[h];
          }
        }
        emit(i, ent);
      }
    }
    __syncthreads();  // s_amax / s_scale / s_cmax are rewritten by the next tile
#pragma unroll
    for (int i = 0; i < R; ++i) w[i] = wn[i];
  }
  if constexpr (OUTL) outlier_tally(nskip, oa);
}

// The fake-quant output with outlier masking (mx_lut_kernel's OUTL form).
template <int LPB, bool ABSMAX>
static int launch_lut_outlier(const uint16_t* x, int64_t ngroups, const ScaleParams& sp, const LutView& lv,
                              const MxOut& out, const OutlierArgs& oa, hipStream_t st) {
  auto k = mx_lut_kernel<0, LPB, ABSMAX, 2, false, true>;
  const size_t lds = sizeof(uint32_t) * 2 * lv.len;
  const unsigned grid = persistent_grid((const void*)k, kMxLutThreads, lds, ngroups);
  hipLaunchKernelGGL(k, dim3(grid), dim3(kMxLutThreads), lds, st, x, ngroups, sp, lv, out, oa);
  return check_launch("mx_quantize(lut, outliers)");
}

template <int CB, int LPB, bool ABSMAX>
static int launch_lut_want(const uint16_t* x, int64_t ngroups, const ScaleParams& sp, const LutView& lv,
                           const MxOut& out, hipStream_t st) {
  switch ((out.qvals ? 1 : 0) | (out.fq ? 2 : 0)) {
    case 0: return launch_lut_k<CB, LPB, ABSMAX, 0>(x, ngroups, sp, lv, out, st);
    case 1: return launch_lut_k<CB, LPB, ABSMAX, 1>(x, ngroups, sp, lv, out, st);
    case 2: return launch_lut_k<CB, LPB, ABSMAX, 2>(x, ngroups, sp, lv, out, st);
    default: return launch_lut_k<CB, LPB, ABSMAX, 3>(x, ngroups, sp, lv, out, st);
  }
}

template <int CB, bool ABSMAX>
static int launch_lut_lpb(const uint16_t* x, int64_t ngroups, int lpb, const ScaleParams& sp,
                          const LutView& lv, const MxOut& out, hipStream_t st) {
  switch (lpb) {
    case 1: return launch_lut_want<CB, 1, ABSMAX>(x, ngroups, sp, lv, out, st);
    case 2: return launch_lut_want<CB, 2, ABSMAX>(x, ngroups, sp, lv, out, st);
    case 4: return launch_lut_want<CB, 4, ABSMAX>(x, ngroups, sp, lv, out, st);
    case 8: return launch_lut_want<CB, 8, ABSMAX>(x, ngroups, sp, lv, out, st);
    default: return set_error(kErrInvalid, "block size %d not supported on the table path", lpb * 16);
  }
}

static int launch_lut(const uint16_t* x, int64_t n, int lpb, int cb, const ScaleParams& sp, const LutView& lv,
                      const MxOut& out, hipStream_t st) {
  int64_t ngroups = n / 16;
  bool absmax = sp.mode == 1;
#define VQX_LUT_CB(C)                                                                        \
  return absmax ? launch_lut_lpb<C, true>(x, ngroups, lpb, sp, lv, out, st)                  \
                : launch_lut_lpb<C, false>(x, ngroups, lpb, sp, lv, out, st);
  switch (cb) {
    case 0: VQX_LUT_CB(0)
    case 4: VQX_LUT_CB(4)
    case 6: VQX_LUT_CB(6)
    case 8: VQX_LUT_CB(8)
    default: return set_error(kErrInvalid, "table path packs 4-, 6- or 8-bit codes, not %d", cb);
  }
#undef VQX_LUT_CB
}

template <typename T, typename Enc, int CB>
static int launch_group(const T* x, int64_t n, int lpb, const ScaleParams& sp, const Enc& enc,
                        const MxOut& out, hipStream_t st, const OutlierArgs& oa = OutlierArgs{}) {
  int64_t ngroups = n / 16;
  const int bs = 256;
  unsigned grid = grid_for(ngroups, bs);
  switch (lpb) {
#define VQX_LPB(L)                                                                                 \
  case L:                                                                                          \
    hipLaunchKernelGGL((mx_group_kernel<T, Enc, CB, L>), dim3(grid), dim3(bs), 0, st, x, ngroups, \
                       sp, enc, out, oa);                                                          \
    break;
    VQX_LPB(1)
    VQX_LPB(2)
    VQX_LPB(4)
    VQX_LPB(8)
#undef VQX_LPB
    default:
      return set_error(kErrInvalid, "block size %d not supported on the packed path", lpb * 16);
  }
  return check_launch("mx_quantize");
}

template <typename T, typename Enc>
static int mx_quantize_t(const T* x, int64_t outer, int64_t L, int64_t inner, int64_t bs,
                         const ScaleParams& sp, const Enc& enc, const MxOut& out, int code_layout,
                         int code_bits, hipStream_t st, const OutlierArgs& oa) {
  int64_t n = outer * L * inner;
  if (n == 0) return kOk;
  int64_t lpb = bs / 16;
  bool fast = inner == 1 && bs % 16 == 0 && L % bs == 0 && lpb >= 1 && lpb <= 8 &&
              (lpb & (lpb - 1)) == 0 && aligned(x, 16) &&
              (!out.qvals || aligned(out.qvals, 16)) && (!out.fq || aligned(out.fq, 16)) &&
              (!out.codes || aligned(out.codes, 16));
  if (out.codes && code_layout == 0) {  // packed codes need the group path
    if (!fast)
      return set_error(kErrInvalid,
                       "packed codes need last-dim blocks (inner == 1), block size 16, 32, 64 or 128 "
                       "dividing the row, and 16-byte aligned buffers");
    if constexpr (Enc::kBits != 0) {
      if (code_bits != Enc::kBits)
        return set_error(kErrInvalid, "format packs %d-bit codes, not %d", Enc::kBits, code_bits);
      return launch_group<T, Enc, Enc::kBits>(x, n, (int)lpb, sp, enc, out, st);
    } else {
      switch (code_bits) {
        case 4: return launch_group<T, Enc, 4>(x, n, (int)lpb, sp, enc, out, st);
        case 6: return launch_group<T, Enc, 6>(x, n, (int)lpb, sp, enc, out, st);
        case 8: return launch_group<T, Enc, 8>(x, n, (int)lpb, sp, enc, out, st);
        case 16: return launch_group<T, Enc, 16>(x, n, (int)lpb, sp, enc, out, st);
        default: return set_error(kErrInvalid, "packed code width %d not in {4, 6, 8, 16}", code_bits);
      }
    }
  }
  if (fast && !out.codes) return launch_group<T, Enc, 0>(x, n, (int)lpb, sp, enc, out, st, oa);
  if (out.codes && code_layout != 1 && code_layout != 2)
    return set_error(kErrInvalid, "unpacked code layout must be 1 or 2 bytes");
  constexpr int VE = 16 / sizeof(T);
  if (inner > 1 && inner % VE == 0 && bs <= 16 * kColRowsMax && aligned(x, 16) &&
      (!out.qvals || aligned(out.qvals, 16)) && (!out.fq || aligned(out.fq, 16))) {
    const int64_t tiles = outer * ((L + bs - 1) / bs) * ((inner + kColChunks * VE - 1) / (kColChunks * VE));
    const unsigned grid = persistent_grid((const void*)mx_cols_kernel<T, Enc>, 256, 0, tiles * 256);
    hipLaunchKernelGGL((mx_cols_kernel<T, Enc>), dim3(grid), dim3(256), 0, st, x, outer, L, inner, (int)bs, sp,
                       enc, out, code_layout, oa);
    return check_launch("mx_quantize(cols)");
  }
  int64_t nblocks = outer * ((L + bs - 1) / bs) * inner;
  unsigned grid = grid_for(nblocks, 256);
  hipLaunchKernelGGL((mx_block_kernel<T, Enc>), dim3(grid), dim3(256), 0, st, x, outer, L, inner, bs, sp,
                     enc, out, code_layout, oa);
  return check_launch("mx_quantize");
}

int mx_quantize(const void* x, int dtype, int64_t outer, int64_t L, int64_t inner, int64_t bs,
                const FormatDesc& fmt, const ScaleParams& sp, const MxOut& out, int code_layout,
                hipStream_t st, const OutlierArgs* oap) {
  const OutlierArgs oa = oap ? *oap : OutlierArgs{};
  if (oa.active && (out.qvals || out.codes || out.scale_e8m0))
    return set_error(kErrInvalid, "mx_quantize: outlier masking writes the fake-quant values and scales only");
  if (outer < 0 || L < 0 || inner < 1 || bs < 1)
    return set_error(kErrInvalid, "bad block geometry outer=%lld L=%lld inner=%lld bs=%lld",
                     (long long)outer, (long long)L, (long long)inner, (long long)bs);
  if (code_layout < 0 || code_layout > 2) return set_error(kErrInvalid, "code layout must be 0, 1 or 2");
  if (out.scale_e8m0 && sp.mode != 0)
    return set_error(kErrInvalid, "E8M0 scales need power-of-two scaling");
  {
    int64_t n = outer * L * inner;
    int64_t lpb = bs / 16;
    bool packed = out.codes && code_layout == 0;
    bool fast = dtype == kBF16 && fmt.lut && inner == 1 && bs % 16 == 0 && L % bs == 0 && lpb >= 1 &&
                lpb <= 8 && (lpb & (lpb - 1)) == 0 && aligned(x, 16) &&
                (!out.qvals || aligned(out.qvals, 16)) && (!out.fq || aligned(out.fq, 16)) &&
                (!out.codes || aligned(out.codes, 16)) && (!out.codes || packed);
    if (n == 0) return kOk;
    if (fast && oa.active) {
      if (!out.fq) return set_error(kErrInvalid, "mx_quantize: outlier masking needs the fake-quant output");
      LutView lv{fmt.lut, fmt.lut_len};
      const int64_t ng = n / 16;
      const bool am = sp.mode == 1;
      switch (lpb) {
        case 1: return am ? launch_lut_outlier<1, true>((const uint16_t*)x, ng, sp, lv, out, oa, st)
                          : launch_lut_outlier<1, false>((const uint16_t*)x, ng, sp, lv, out, oa, st);
        case 2: return am ? launch_lut_outlier<2, true>((const uint16_t*)x, ng, sp, lv, out, oa, st)
                          : launch_lut_outlier<2, false>((const uint16_t*)x, ng, sp, lv, out, oa, st);
        case 4: return am ? launch_lut_outlier<4, true>((const uint16_t*)x, ng, sp, lv, out, oa, st)
                          : launch_lut_outlier<4, false>((const uint16_t*)x, ng, sp, lv, out, oa, st);
        default: return am ? launch_lut_outlier<8, true>((const uint16_t*)x, ng, sp, lv, out, oa, st)
                           : launch_lut_outlier<8, false>((const uint16_t*)x, ng, sp, lv, out, oa, st);
      }
    }
    if (fast) {
      LutView lv{fmt.lut, fmt.lut_len};
      return launch_lut((const uint16_t*)x, n, (int)lpb, packed ? fmt.code_bits : 0, sp, lv, out, st);
    }
    // blocks along a middle axis of a bf16 input: the table-driven column kernel
    const bool cols = dtype == kBF16 && fmt.lut && inner > 1 && inner % 8 == 0 && bs <= 16 * kColRowsMax &&
                      !packed && (out.codes == nullptr || code_layout == 1 || code_layout == 2) &&
                      aligned(x, 16) && (!out.qvals || aligned(out.qvals, 16)) && (!out.fq || aligned(out.fq, 16));
    const int64_t col_tiles = outer * ((L + bs - 1) / bs) * ((inner + kColChunks * 8 - 1) / (kColChunks * 8));
    if (cols && col_tiles < ((int64_t)1 << 31)) {
      LutView lv{fmt.lut, fmt.lut_len};
      const int64_t tiles = col_tiles;
      const size_t lds = sizeof(uint32_t) * 2 * (size_t)lv.len;
      auto go = [&](auto kern) {
        const unsigned grid = persistent_grid((const void*)kern, 256, lds, tiles * 256);
        hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, st, (const uint16_t*)x, outer, L, inner, (int)bs, sp,
                           lv, out, code_layout, oa);
        return check_launch("mx_quantize(cols, table)");
      };
      // rows per thread: the 16 row groups of a workgroup cover bs rows
      const int rows = (int)((bs + 15) / 16);
      auto by_rows = [&](auto absmax, auto outl) {
        constexpr bool A = decltype(absmax)::value, O = decltype(outl)::value;
        if (rows <= 1) return go(mx_cols_lut_kernel<A, 1, O>);
        if (rows <= 2) return go(mx_cols_lut_kernel<A, 2, O>);
        if (rows <= 4) return go(mx_cols_lut_kernel<A, 4, O>);
        return go(mx_cols_lut_kernel<A, 8, O>);
      };
      if (sp.mode == 1)
        return oa.active ? by_rows(std::true_type{}, std::true_type{}) : by_rows(std::true_type{}, std::false_type{});
      return oa.active ? by_rows(std::false_type{}, std::true_type{}) : by_rows(std::false_type{}, std::false_type{});
    }
  }
  return with_encoder(fmt, [&](auto enc) -> int {
    using E = decltype(enc);
    if (dtype == kBF16)
      return mx_quantize_t<uint16_t, E>((const uint16_t*)x, outer, L, inner, bs, sp, enc, out,
                                        code_layout, fmt.code_bits, st, oa);
    if (dtype == kF32)
      return mx_quantize_t<float, E>((const float*)x, outer, L, inner, bs, sp, enc, out, code_layout,
                                     fmt.code_bits, st, oa);
    return set_error(kErrInvalid, "blockwise input dtype %d not supported (float32, bfloat16)", dtype);
  });
}

// ---------------------------------------------------------------------------
// decode: codes -> value table -> times the block scale, in the output dtype
// (dequantize, ops/quantized.py:211-222; linear_mx's weight decode :319-326)
// ---------------------------------------------------------------------------
// scale_kind: 0 fp32, 1 bf16, 2 E8M0
__device__ __forceinline__ float load_scale(const void* s, int kind, int64_t i) {
  if (kind == 0) return static_cast<const float*>(s)[i];
  if (kind == 1) return bf2f(static_cast<const uint16_t*>(s)[i]);
  uint32_t e = static_cast<const uint8_t*>(s)[i];
  return e == 0xFFu ? __builtin_huge_valf() : (e == 0 ? u2f(0x00400000u) : u2f(e << 23));
}

// Decode of packed codes: out = round(table[code] * scale[block]).
// 4- and 8-bit codes take a lane-interleaved layout: a wave handles 1024
// elements per step as chunks of 16 output bytes per lane (E = 8 bf16 or 4
// fp32 elements), chunk q of lane L at element 64 E q + E L, so every load
// and store instruction of the wave covers one contiguous span; each chunk
// lies inside one block (block sizes are multiples of 16).  6-bit codes and
// any elements past the last whole 1024 take 16-element groups per thread.
// The codes are read with plain loads (non-temporal ones made the C2 decode
// 22.5 us against 16.9), the output is stored non-temporally.
template <typename T, int CB>
__device__ __forceinline__ void decode_chunks(const uint8_t* __restrict__ codes, const void* scale, int scale_kind,
                                              const uint16_t* tab, T* __restrict__ out, int64_t base, int lane,
                                              int64_t bs) {
  constexpr int E = 16 / (int)sizeof(T);  // elements per 16-byte output chunk
  constexpr int Q = 16 / E;               // chunks per lane per step
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int64_t e = base + (int64_t)q * 64 * E + (int64_t)lane * E;
    uint32_t c[E];
    if constexpr (CB == 4 && E == 8) {
      uint32_t w = *reinterpret_cast<const uint32_t*>(codes + e / 2);
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = (w >> (4 * j)) & 0xFu;
    } else if constexpr (CB == 4) {  // E == 4
      uint32_t w = *reinterpret_cast<const uint16_t*>(codes + e / 2);
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = (w >> (4 * j)) & 0xFu;
    } else if constexpr (E == 8) {  // CB == 8
      u32x2 w = *reinterpret_cast<const u32x2*>(codes + e);
#pragma unroll
      for (int j = 0; j < 8; ++j) c[j] = ((j < 4 ? w.x : w.y) >> (8 * (j & 3))) & 0xFFu;
    } else {  // CB == 8, E == 4
      uint32_t w = *reinterpret_cast<const uint32_t*>(codes + e);
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = (w >> (8 * j)) & 0xFFu;
    }
    const float s = load_scale(scale, scale_kind, e / bs);
    if constexpr (E == 8) {
      u32x4 v;
      if (__builtin_isfinite(s)) {
        // finite products: v_cvt_pk_bf16_f32 rounds them as f2bf does
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[j] = pack_bf16x2(bf2f(tab[c[2 * j]]) * s, bf2f(tab[c[2 * j + 1]]) * s);
      } else {
        uint32_t o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = f2bf(bf2f(tab[c[j]]) * s);
        v = u32x4{o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16)};
      }
      st_nt(reinterpret_cast<u32x4*>(out + e), v);
    } else {
      f32x4 v = {bf2f(tab[c[0]]) * s, bf2f(tab[c[1]]) * s, bf2f(tab[c[2]]) * s, bf2f(tab[c[3]]) * s};
      st_nt(reinterpret_cast<f32x4*>(out + e), v);
    }
  }
}

template <typename T, int CB, int LPB>
__global__ __launch_bounds__(256) void decode_group_kernel(const uint8_t* __restrict__ codes,
                                                           const void* __restrict__ scale, int scale_kind,
                                                           const uint16_t* __restrict__ dtab, int ntab,
                                                           T* __restrict__ out, int64_t ngroups) {
  __shared__ uint16_t tab[1 << (CB > 8 ? 8 : CB)];
  for (int i = threadIdx.x; i < ntab && i < (1 << (CB > 8 ? 8 : CB)); i += blockDim.x) tab[i] = dtab[i];
  __syncthreads();
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t g0 = 0;  // first group left to the per-thread loop
  if constexpr (CB == 4 || CB == 8) {
    const int lane = threadIdx.x & 63;
    const int64_t nsteps = ngroups / 64;  // whole 1024-element wave steps
    const int64_t wstride = stride / 64;
    for (int64_t w = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / 64; w < nsteps; w += wstride)
      decode_chunks<T, CB>(codes, scale, scale_kind, tab, out, w * 1024, lane, 16 * LPB);
    g0 = nsteps * 64;
  }
  for (int64_t g = g0 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < ngroups; g += stride) {
    uint32_t c[16];
    if constexpr (CB == 4) {
      u32x2 w = *reinterpret_cast<const u32x2*>(codes + g * 8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        c[j] = (w.x >> (4 * j)) & 0xFu;
        c[j + 8] = (w.y >> (4 * j)) & 0xFu;
      }
    } else if constexpr (CB == 6) {
      const uint32_t* q = reinterpret_cast<const uint32_t*>(codes + g * 12);
      uint32_t w0 = q[0], w1 = q[1], w2 = q[2];
      uint64_t lo = (uint64_t)w0 | ((uint64_t)w1 << 32);
#pragma unroll
      for (int j = 0; j < 10; ++j) c[j] = (uint32_t)(lo >> (6 * j)) & 0x3Fu;
      c[10] = ((w1 >> 28) | (w2 << 4)) & 0x3Fu;
#pragma unroll
      for (int j = 11; j < 16; ++j) c[j] = (w2 >> (6 * j - 64)) & 0x3Fu;
    } else {
      u32x4 w = *reinterpret_cast<const u32x4*>(codes + g * 16);
      uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 16; ++j) c[j] = (ww[j >> 2] >> (8 * (j & 3))) & 0xFFu;
    }
    float s = load_scale(scale, scale_kind, g / LPB);
    uint32_t o[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) o[j] = BT<T>::round_bits(bf2f(tab[c[j]]) * s);
    BT<T>::store16(out + g * 16, o);
  }
}

int mx_decode(const uint8_t* codes, int code_bits, const uint16_t* decode_table, int ntab,
              const void* scale, int scale_kind, int64_t n, int64_t bs, void* out, int out_dtype,
              hipStream_t st) {
  if (n == 0) return kOk;
  int64_t lpb = bs / 16;
  if (n % bs != 0 || bs % 16 != 0 || lpb > 8 || (lpb & (lpb - 1)) != 0 || !aligned(codes, 16) ||
      !aligned(out, 16))
    return set_error(kErrInvalid, "decode needs n %% bs == 0, bs in {16, 32, 64, 128}, aligned buffers");
  if (code_bits != 4 && code_bits != 6 && code_bits != 8)
    return set_error(kErrInvalid, "decode code width %d not in {4, 6, 8}", code_bits);
  if (scale_kind < 0 || scale_kind > 2) return set_error(kErrInvalid, "scale kind must be 0, 1 or 2");
  int64_t ngroups = n / 16;
  unsigned grid = grid_for(ngroups, 256);
#define VQX_DEC(T, CB, L)                                                                      \
  hipLaunchKernelGGL((decode_group_kernel<T, CB, L>), dim3(grid), dim3(256), 0, st, codes, scale, \
                     scale_kind, decode_table, ntab, (T*)out, ngroups)
#define VQX_DEC_L(T, CB)            \
  switch (lpb) {                    \
    case 1: VQX_DEC(T, CB, 1); break;  \
    case 2: VQX_DEC(T, CB, 2); break;  \
    case 4: VQX_DEC(T, CB, 4); break;  \
    default: VQX_DEC(T, CB, 8); break;  \
  }
  if (out_dtype == kBF16) {
    if (code_bits == 4) { VQX_DEC_L(uint16_t, 4) }
    else if (code_bits == 6) { VQX_DEC_L(uint16_t, 6) }
    else { VQX_DEC_L(uint16_t, 8) }
  } else if (out_dtype == kF32) {
    if (code_bits == 4) { VQX_DEC_L(float, 4) }
    else if (code_bits == 6) { VQX_DEC_L(float, 6) }
    else { VQX_DEC_L(float, 8) }
  } else {
    return set_error(kErrInvalid, "decode output dtype %d not supported", out_dtype);
  }
#undef VQX_DEC_L
#undef VQX_DEC
  return check_launch("mx_decode");
}

// Inverse table of a format: dtab[code] = value for every code some bf16
// pattern encodes to (all patterns sharing a code share its value).
template <typename Enc>
__global__ __launch_bounds__(256) void decode_table_kernel(uint16_t* dtab, int ntab, Enc enc) {
  uint32_t h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= 65536u) return;
  Result r = enc.encode(h);
  if ((int)r.code < ntab && (h & 0x7FFFu) <= 0x7F80u) dtab[r.code] = (uint16_t)r.value;
}

int decode_table(const FormatDesc& fmt, uint16_t* dtab, int ntab, hipStream_t st) {
  return with_encoder(fmt, [&](auto enc) {
    hipLaunchKernelGGL((decode_table_kernel<decltype(enc)>), dim3(256), dim3(256), 0, st, dtab, ntab, enc);
    return check_launch("decode_table");
  });
}

}  // namespace vqx
