// Element-format encoders for the Voyager quantization hot path.
//
// Every reference quantizer is a function of the bf16 bit pattern of its
// input: get_quantization_map() tabulates it over all 2^16 patterns
// (src/voyager_compiler/quantization/fake_quantize.py:30-98) and vmap()
// gathers from that table (src/voyager_compiler/ops/quantized.py:101-121).
// This header computes the same functions in closed form on the bit pattern,
// with integer bit manipulation, so a kernel needs no 128 KiB table.  Each
// encoder returns the format code (what the packed outputs store) and the
// fake-quant value as a bf16 pattern (what the reference's table holds).
//
// The header is plain C++ (no HIP types): hipcc builds it into the kernels and
// g++ builds it into the CPU harness that checks every encoder against the
// reference tables over all 65536 inputs.

#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define VQX_HD __host__ __device__ __forceinline__
#else
#define VQX_HD inline
#endif

// Every fp expression below is one IEEE operation whose rounding is part of
// the reference's semantics: never fuse a multiply into an add.
#if defined(__clang__)
#define VQX_NO_CONTRACT _Pragma("clang fp contract(off)")
#else
#define VQX_NO_CONTRACT
#endif

namespace vqx {

// ---------------------------------------------------------------------------
// bit casts and bf16 rounding
// ---------------------------------------------------------------------------
VQX_HD uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
VQX_HD float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
VQX_HD float bf2f(uint32_t h) { return u2f(h << 16); }

// fp32 -> bf16, round to nearest even; every NaN becomes 0x7FC0 (what torch's
// c10::BFloat16 conversion produces for .to(bfloat16) and bf16 arithmetic).
VQX_HD uint32_t f2bf(float f) {
  uint32_t u = f2u(f);
  uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  return ((u & 0x7FFFFFFFu) > 0x7F800000u) ? 0x7FC0u : r;
}

VQX_HD int clz32(uint32_t x) {
#if defined(__HIPCC__) || defined(__GNUC__)
  return x ? __builtin_clz(x) : 32;
#else
  int n = 0;
  while (n < 32 && !(x & (0x80000000u >> n))) ++n;
  return n;
#endif
}

// 2^e as an fp32 value for e in [-149, 127] (exact, including subnormals).
VQX_HD float exp2i(int e) {
  return e >= -126 ? u2f((uint32_t)(e + 127) << 23) : u2f(1u << (e + 149));
}

// ---------------------------------------------------------------------------
// floor(log2(a)) as torch evaluates it on a bf16 tensor
// ---------------------------------------------------------------------------
// mx_utils.py:43-47 and fp8.py:193-197 take torch.log2 of bf16 data: the log
// is computed in fp32 and rounded to bf16 before the floor, so for a mantissa
// close to 2 the result is one above the true exponent (31.75 -> 5).  For a
// normal a = 2^p (1 + m/128) the floor is p or p + 1, and it is p + 1 exactly
// when log2(1 + m/128) >= 1 - u/2, u being the bf16 spacing of log values next
// to the integer p + 1 on the side a's log lies.  That spacing is 2^(b-7) with
// b = floor(log2 |p + 1|) (one less when p + 1 > 0 is a power of two, since
// the log then lies in the binade below); the smallest such m for each b is
// ceil(128 * (2^(1 - 2^(b-8)) - 1)).  Subnormal a = m 2^-133 has |log| in
// [126, 133], where bf16 spacing is 1 or 1/2; the mantissa thresholds at which
// the result steps up are listed directly.  Every entry is checked against
// torch's own bf16 log2 for all 2^16 patterns by the CPU test suite.
VQX_HD uint32_t log2_step_threshold(int E) {
  // thresholds for b = -1 .. 6 (128 = never), one byte each, b + 1 = byte index:
  // 128, 128, 127, 126, 123, 118, 107, 88
  const uint64_t kByBand = 0x586B767B7E7F8080ull;
  int p = E - 127;
  // n = p + 1 for p >= 0, -(p + 1) below; p == -1 gives n = 0 and band -1
  uint32_t n = p >= 0 ? (uint32_t)p + 1u : (uint32_t)(-p - 1);
  int band = 31 - clz32(n);
  band -= (p >= 0 && (n & (n - 1u)) == 0) ? 1 : 0;
  return (uint32_t)(kByBand >> (8 * (band + 1))) & 0xFFu;
}

// floor(bf16(log2(a))) for a positive finite bf16 magnitude pattern (1..0x7F7F).
VQX_HD int log2floor_bf16(uint32_t mag) {
  uint32_t E = mag >> 7, m = mag & 0x7Fu;
  int sub = -133 + (m >= 2) + (m >= 3) + (m >= 6) + (m >= 12) + (m >= 23) + (m >= 54) + (m >= 108);
  int nrm = (int)E - 127 + (m >= log2_step_threshold((int)E) ? 1 : 0);
  return E == 0 ? sub : nrm;
}

// 2 ** ceil(log2(f)) for an fp32 bit pattern f, as torch evaluates
// torch.pow(2, torch.ceil(torch.log2(sf))) on the CPU
// (src/vc/quantization/fake_quantize.py:339-340).  The CPU's fp32 log2 is
// correctly rounded, so for f = 2^p (1 + d 2^-q) just above a power of two
// (q = 23 for a normal f, q = the bit length - 1 of a subnormal's mantissa)
// the log rounds down to the integer p while log2(1 + d 2^-q) is below half
// the fp32 spacing next to p: the ceiling then stays p for d <= J.  J depends
// on p's band (normal f) or on q (subnormal f) only.  Zero gives +0,
// negative or NaN gives NaN, +Inf stays +Inf.
VQX_HD uint32_t pow2_ceil_log2_f32(uint32_t b) {
  if ((b & 0x7FFFFFFFu) == 0) return 0u;                // log2(0) = -inf, 2^-inf = 0
  if ((b >> 31) || b > 0x7F800000u) return 0x7FC00000u;  // log2 < 0 or NaN: NaN
  if (b == 0x7F800000u) return b;
  const uint32_t E = b >> 23, m = b & 0x7FFFFFu;
  int p;
  uint32_t d, J;
  if (E != 0) {
    p = (int)E - 127;
    d = m;
    // band of the integer p: floor(log2 p) above 0, floor(log2(-p - 1))
    // below (the spacing just above a negative power of two is the finer
    // one of the binade below it); J by band 2 .. 6
    const uint32_t n = p > 0 ? (uint32_t)p : (p < -1 ? (uint32_t)(-p - 1) : 0u);
    const int band = n ? 31 - clz32(n) : -1;
    J = band >= 2 && band <= 6 ? (0x16'0B'05'02'01ull >> (8 * (band - 2))) & 0xFFu : 0u;
  } else {
    const int k = 31 - clz32(m);  // m = 2^k + d
    p = k - 149;
    d = m - (1u << k);
    J = k >= 18 ? (0x0B'05'05'02'01ull >> (8 * (k - 18))) & 0xFFu : 0u;
  }
  if (d == 0) return b;  // an exact power of two
  const int e = d <= J ? p : p + 1;
  if (e >= 128) return 0x7F800000u;
  return e >= -126 ? (uint32_t)(e + 127) << 23 : 1u << (e + 149);
}

// Round-to-nearest-even of mant / 2^sh for sh >= 0 (sh may exceed 31).
VQX_HD uint32_t rne_shift(uint32_t mant, int sh) {
  if (sh <= 0) return mant << (-sh);
  if (sh > 31) return 0;
  uint32_t q = mant >> sh;
  uint32_t rem = mant & ((1u << sh) - 1u);
  uint32_t half = 1u << (sh - 1);
  return q + ((rem > half) | ((rem == half) & (q & 1u)));
}

// ---------------------------------------------------------------------------
// Format descriptors
// ---------------------------------------------------------------------------
enum FormatKind : int32_t {
  kFmtIdentity = 0,  // "float32" / "bfloat16": value = bf16(x)
  kFmtFp16 = 1,      // "float16": bf16(fp16(x))
  kFmtInt = 2,       // int<n> / uint<n>: clamp(round_half_even(x))
  kFmtFpCore = 3,    // fp<N>_e<E>m<M>: MX element core (fp8.py:160-225)
  kFmtNvFp8 = 4,     // e4m3 / e5m2: fp32-bit RNE (fp8.py:13-74)
  kFmtPosit = 5,     // posit<n>_<es> (posit.py:8-73)
  kFmtLevels = 6,    // nf<k>[_<b>] or a sorted codebook: boundary search
  kFmtTable = 7,     // any 65536-entry bf16 table (a caller's qmap)
};

enum FormatFlags : int32_t {
  kFlagUnsigned = 1,  // fp core with N == E + M: input magnitude only
};

struct Result {
  uint32_t code;   // format code, nbits wide (two's complement for int/posit)
  uint32_t value;  // fake-quant value as a bf16 bit pattern
};

// ---------------------------------------------------------------------------
// posit(n, es), n <= 16, es <= 3   (dtypes/posit.py:8-73)
// ---------------------------------------------------------------------------
// Code = round-to-nearest-even of the posit bit string (regime run and its
// terminator, es exponent bits, the 7 fraction bits of the bf16 input) cut to
// n - 1 bits; a carry out of the fraction runs into the exponent and regime,
// which is exactly the next posit.  Special rules of the reference:
//   |x| < 2^floor(-(n-1) 2^es + 2^(es-1))  -> 0        (posit.py:52-57)
//   scale above (n-2) 2^es -> maxpos, below -(n-2) 2^es -> minpos (:20-21,:42)
//   both zeros -> 0; Inf/NaN -> NaR                     (:60-61)
struct Posit {
  int n, es;

  VQX_HD int flush_exp() const {
    // floor(-(n-1) 2^es + 2^(es-1)); for es = 0 the 1/2 floors away.
    int base = -(n - 1) * (1 << es);
    return es == 0 ? base : base + (1 << (es - 1));
  }

  // Magnitude code (n-1 bits) for a finite nonzero bf16 magnitude.
  VQX_HD uint32_t mag_code(uint32_t a) const {
    int E = (int)(a >> 7);
    uint32_t f = a & 0x7Fu;
    int scale = E - 127;
    int maxs = (n - 2) << es;
    int fe = flush_exp();
    uint32_t thr = fe >= -126 ? (uint32_t)(fe + 127) << 7 : (1u << (fe + 133));
    if (a < thr) return 0;
    if (scale > maxs) return (1u << (n - 1)) - 1u;
    if (scale < -maxs) return 1u;
    int k = scale >> es;  // arithmetic shift = floor division
    uint32_t e = (uint32_t)scale & ((1u << es) - 1u);
    uint32_t reg;
    int rlen;
    if (k >= 0) {
      reg = ((2u << k) - 1u) << 1;  // k+1 ones, then the terminating zero
      rlen = k + 2;
    } else {
      reg = 1u;  // -k zeros (implicit), then the terminating one
      rlen = 1 - k;
    }
    uint32_t body = (((reg << es) | e) << 7) | f;
    int cut = rlen + es + 7 - (n - 1);
    return rne_shift(body, cut);
  }

  // Decode an (n-1)-bit magnitude code to fp32 (exact for n <= 16).
  VQX_HD float mag_value(uint32_t c) const {
    if (c == 0) return 0.0f;
    int w = n - 1;
    uint32_t top = (c >> (w - 1)) & 1u;
    // run length of the leading bit, within the w-bit field
    uint32_t x = top ? (~c) & ((1u << w) - 1u) : c;
    int run = x ? (clz32(x) - (32 - w)) : w;
    int k = top ? run - 1 : -run;
    int rest = w - run - 1;  // bits after the terminator
    if (rest < 0) rest = 0;
    uint32_t tail = c & ((1u << rest) - 1u);
    uint32_t e, frac;
    int fbits;
    if (rest >= es) {
      e = tail >> (rest - es);
      fbits = rest - es;
      frac = tail & ((1u << fbits) - 1u);
    } else {
      e = tail << (es - rest);
      fbits = 0;
      frac = 0;
    }
    int sc = k * (1 << es) + (int)e;
    // (1 + frac / 2^fbits) * 2^sc with fbits <= 13: build it in fp32.
    uint32_t mant = frac << (23 - fbits);
    return u2f((uint32_t)(sc + 127) << 23 | mant);
  }

  VQX_HD Result encode(uint32_t h) const {
    uint32_t a = h & 0x7FFFu;
    uint32_t neg = h >> 15;
    Result r;
    if (a >= 0x7F80u) {  // Inf / NaN -> NaR
      r.code = 1u << (n - 1);
      r.value = 0x7FC0u;
      return r;
    }
    uint32_t c = a ? mag_code(a) : 0u;
    float v = mag_value(c);
    uint32_t mask = (n >= 32) ? 0xFFFFFFFFu : ((1u << n) - 1u);
    r.code = (neg && c) ? ((0u - c) & mask) : c;
    uint32_t vb = f2bf(v);
    r.value = (neg && c) ? (vb | 0x8000u) : vb;
    return r;
  }
};

// ---------------------------------------------------------------------------
// fp<N>_e<E>m<M> through the microscaling element core (fp8.py:160-225),
// as routed by fake_quantize.py:63-80 with round="even", saturate_normals.
// ---------------------------------------------------------------------------
// On the bf16 data the reference evaluates:
//   pe  = max(floor(bf16 log2(|A| + [A == 0])), 2 - 2^(E-1))
//   q   = round_half_even(|A| / 2^pe * 2^M)
//   out = clamp(sign(A) q / 2^M * 2^pe, +-max_norm), Inf restored, NaN kept
// With M <= 6 every intermediate is exact in bf16, so integer RNE of the bf16
// mantissa reproduces it; pe uses the bf16-log2 floor above.  When pe = 128
// the reference computes 0 * 2^128 = NaN, so bf16 magnitudes from
// 2^127 * 1.6875 up map to NaN; both zeros map to +0 and a nonzero input that
// rounds to zero keeps its sign.  M >= 7 formats take the op-by-op bf16 path
// (encode_emulated), because there the reference's own rounding steps round.
struct FpCore {
  int ebits, mbits;        // element exponent / mantissa bits
  float max_norm;          // saturation bound
  bool is_unsigned;        // N == E + M: magnitude of the input is quantized

  VQX_HD int min_exp() const { return 2 - (1 << (ebits - 1)); }
  VQX_HD int nbits() const { return ebits + mbits + (is_unsigned ? 0 : 1); }

  // OCP-style code of a (finite, saturated) result given as q * 2^(pe - M).
  VQX_HD uint32_t pack(uint32_t neg, uint32_t q, int pe) const {
    int M = mbits;
    if (q == 0) return neg << (ebits + mbits);
    if (q >> (M + 1)) {  // rounding carried into the next binade
      q >>= 1;
      pe += 1;
    }
    uint32_t field, mant;
    if (q >> M) {
      field = (uint32_t)(pe - min_exp() + 1);
      mant = q - (1u << M);
    } else {
      field = 0;
      mant = q;
    }
    uint32_t mag = (field << M) | mant;
    return is_unsigned ? mag : ((neg << (ebits + mbits)) | mag);
  }

  // Largest finite code: the saturation value max_norm.
  VQX_HD uint32_t max_code(uint32_t neg) const {
    // max_norm = 2^emax * (2 - 2^-M) or e4m3's 448 = 2^8 * 1.75
    uint32_t mb = f2u(max_norm);
    int e = (int)((mb >> 23) & 0xFF) - 127;
    uint32_t mant = (mb >> (23 - mbits)) & ((1u << mbits) - 1u);
    uint32_t field = (uint32_t)(e - min_exp() + 1);
    uint32_t mag = (field << mbits) | mant;
    return is_unsigned ? mag : ((neg << (ebits + mbits)) | mag);
  }

  VQX_HD uint32_t nan_code(uint32_t neg) const {
    // Formats without a NaN encoding saturate; e4m3/e5m2 use S.1..1.1..1.
    uint32_t all = (1u << (ebits + mbits)) - 1u;
    return is_unsigned ? all : ((neg << (ebits + mbits)) | all);
  }

  VQX_HD Result encode(uint32_t h) const {
    Result r;
    if (is_unsigned) h &= 0x7FFFu;
    uint32_t neg = h >> 15;
    uint32_t a = h & 0x7FFFu;
    if (a > 0x7F80u) {  // NaN
      r.value = 0x7FC0u;
      r.code = nan_code(neg);
      return r;
    }
    if (a == 0x7F80u) {  // +-Inf restored (fp8.py:221-222)
      r.value = h;
      r.code = nan_code(neg);
      return r;
    }
    if (a == 0) {
      r.value = 0u;
      r.code = 0u;
      return r;
    }
    int lf = log2floor_bf16(a);
    int pe = lf > min_exp() ? lf : min_exp();
    if (pe >= 128) {  // 2^pe overflows bf16: 0 * inf = NaN
      r.value = 0x7FC0u;
      r.code = nan_code(neg);
      return r;
    }
    if (mbits >= 7) return encode_emulated(h);
    int E = (int)(a >> 7);
    uint32_t mant = (E ? 128u : 0u) | (a & 0x7Fu);
    int Eeff = E ? E : 1;
    // |A| = mant * 2^(Eeff - 134); q = RNE(|A| * 2^(M - pe))
    int sh = pe - mbits - (Eeff - 134);
    uint32_t q = rne_shift(mant, sh);
    // The reference's floor(bf16(|a| + 0.5)) rounds 0.5 - 2^-9 (mantissa
    // 255, nine places below the point) up to 1: fp8.py:136-140 in bf16.
    q |= (uint32_t)(mant == 255u && sh == 9);
    // value = q * 2^(pe - M)
    float v = (float)q * exp2i(pe - mbits);
    if (v > max_norm) {
      r.value = f2bf(max_norm) | (neg << 15);
      r.code = max_code(neg);
      return r;
    }
    r.value = f2bf(v) | (neg << 15);
    r.code = pack(neg, q, pe);
    return r;
  }

  // Op-by-op bf16 evaluation of the reference core, for formats where its
  // intermediate steps round (M >= 7).  Codes are not defined for these.
  VQX_HD Result encode_emulated(uint32_t h) const {
    VQX_NO_CONTRACT
    Result r;
    r.code = 0;
    float A = bf2f(h);
    uint32_t a = h & 0x7FFFu;
    int lf = a ? log2floor_bf16(a) : 0;
    int pe = lf > min_exp() ? lf : min_exp();
    float p2 = bf2f(f2bf(exp2i(pe)));
    float out = bf2f(f2bf(A / p2));
    out = bf2f(f2bf(out * exp2i(mbits)));
    float absA = out < 0 ? -out : out;
    float t1 = bf2f(f2bf(absA - 0.5f));
    float t1m = t1 - 2.0f * __builtin_floorf(t1 * 0.5f);
    float mask = (t1m == 0.0f) ? 1.0f : 0.0f;
    float t2 = __builtin_floorf(bf2f(f2bf(absA + 0.5f)));
    float sgn = out > 0 ? 1.0f : (out < 0 ? -1.0f : 0.0f);
    float q = bf2f(f2bf(sgn * bf2f(f2bf(t2 - mask))));
    out = bf2f(f2bf(q / exp2i(mbits)));
    out = bf2f(f2bf(out * p2));
    float mn = bf2f(f2bf(max_norm));
    if (out > mn) out = mn;
    if (out < -mn) out = -mn;
    r.value = f2bf(out);
    return r;
  }
};

// ---------------------------------------------------------------------------
// NVIDIA-style e4m3 / e5m2   (dtypes/fp8.py:13-74, fake_quantize.py:55-60)
// ---------------------------------------------------------------------------
// RNE onto the grid with min normal 2^emin and subnormals below, saturating at
// fmax; |x| <= 2^emin 2^-(M+1) and both zeros give +0; non-finite gives NaN.
struct NvFp8 {
  int ebits, mbits, emin, bias;
  float fmax;

  VQX_HD static NvFp8 e4m3() { return NvFp8{4, 3, -6, 7, 448.0f}; }
  VQX_HD static NvFp8 e5m2() { return NvFp8{5, 2, -14, 15, 57344.0f}; }

  VQX_HD Result encode(uint32_t h) const {
    Result r;
    uint32_t neg = h >> 15;
    uint32_t a = h & 0x7FFFu;
    uint32_t all = (1u << (ebits + mbits)) - 1u;
    if (a >= 0x7F80u) {
      r.value = 0x7FC0u;
      r.code = (neg << 7) | all;
      return r;
    }
    // flush threshold 2^(emin - M - 1) as a bf16 pattern
    uint32_t flush = (uint32_t)(emin - mbits - 1 + 127) << 7;
    if (a <= flush) {
      r.value = 0u;
      r.code = 0u;
      return r;
    }
    int E = (int)(a >> 7);
    uint32_t mant = (E ? 128u : 0u) | (a & 0x7Fu);
    int Eeff = E ? E : 1;
    int ex = Eeff - 127;
    int pe = ex > emin ? ex : emin;
    // q = RNE(|x| / 2^(pe - M)),  |x| = mant 2^(Eeff - 134)
    uint32_t q = rne_shift(mant, pe - mbits - (Eeff - 134));
    float v = (float)q * exp2i(pe - mbits);
    if (v >= fmax) {
      r.value = f2bf(fmax) | (neg << 15);
      // fmax = 1.75 * 2^(emax): exponent field emax + bias, mantissa 110
      uint32_t fb = f2u(fmax);
      uint32_t fe = ((fb >> 23) & 0xFF) - 127 + bias;
      uint32_t fm = (fb >> (23 - mbits)) & ((1u << mbits) - 1u);
      r.code = (neg << 7) | (fe << mbits) | fm;
      return r;
    }
    r.value = f2bf(v) | (neg << 15);
    if (q >> (mbits + 1)) {
      q >>= 1;
      pe += 1;
    }
    uint32_t field = (q >> mbits) ? (uint32_t)(pe + bias) : 0u;
    uint32_t m = (q >> mbits) ? q - (1u << mbits) : q;
    r.code = (neg << 7) | (field << mbits) | m;
    return r;
  }
};

// ---------------------------------------------------------------------------
// int<n> / uint<n>: clamp(round_half_even(x), qmin, qmax) in bf16
// (fake_quantize.py:43-52).  Codes are two's complement (n bits) / unsigned.
// ---------------------------------------------------------------------------
struct IntFmt {
  int nbits;
  bool is_signed;

  VQX_HD Result encode(uint32_t h) const {
    Result r;
    uint32_t a = h & 0x7FFFu;
    uint32_t neg = h >> 15;
    int qmin = is_signed ? -(1 << (nbits - 1)) : 0;
    int qmax = is_signed ? (1 << (nbits - 1)) - 1 : (1 << nbits) - 1;
    float lo = bf2f(f2bf((float)qmin));
    float hi = bf2f(f2bf((float)qmax));
    if (a > 0x7F80u) {
      r.value = 0x7FC0u;
      r.code = 0u;
      return r;
    }
    float x = bf2f(h);
    float rx = __builtin_rintf(x);  // half to even, keeps -0.0
    if (rx < lo) rx = lo;
    if (rx > hi) rx = hi;
    r.value = f2bf(rx);
    int iv = (int)rx;
    uint32_t mask = (nbits >= 32) ? 0xFFFFFFFFu : ((1u << nbits) - 1u);
    r.code = (uint32_t)iv & mask;
    (void)neg;
    return r;
  }
};

// ---------------------------------------------------------------------------
// Sorted levels searched by boundaries: NormalFloat (normal_float.py:54-60) and
// per-tensor codebook tables (lcq.py:270-291).  The reference's argmin index,
// as a function of the input's bf16 value, is non-decreasing, so it equals the
// number of boundaries b_j <= v, with b_j the least bf16 value whose index is
// >= j (NaN compares false and gets index 0, as torch.argmin gives).  The
// boundaries are derived once per level set from the exhaustive index table.
// ---------------------------------------------------------------------------
VQX_HD uint32_t count_le(const float* b, int nb, float v) {
  // branch-free binary search over nb sorted boundaries (nb + 1 a power of 2
  // is not required)
  uint32_t lo = 0;
  int len = nb;
  while (len > 0) {
    int half = len >> 1;
    bool ge = v >= b[lo + half];
    lo = ge ? lo + half + 1 : lo;
    len = ge ? len - half - 1 : half;
  }
  return lo;
}

}  // namespace vqx
