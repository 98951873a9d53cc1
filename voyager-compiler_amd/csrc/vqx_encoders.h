// Device-side encoder objects: one per format family, each with
//   Result encode(uint32_t bf16_bits) const
// Compile-time specialisations for the hot formats let the compiler fold the
// format constants into the bit manipulation.
#pragma once

#include <hip/hip_fp16.h>

#include "vqx_common.h"

namespace vqx {

// C-ABI format descriptor (mirrors vqx_format in include/vqx.h).
struct FormatDesc {
  int32_t kind;
  int32_t p0;
  int32_t p1;
  int32_t flags;
  float max_norm;
  int32_t code_bits;
  const float* boundaries;   // kFmtLevels: nlevels - 1 fp32 boundaries
  const uint16_t* levels;    // kFmtLevels: nlevels bf16 patterns
  const uint8_t* code_table; // kFmtLevels: 65536 codes, one byte each
  const uint16_t* value_table; // kFmtTable: 65536 bf16 values
  const uint32_t* lut;         // compact LDS table blob (vqx_lut.h), or null
  int32_t lut_len;             // entries per sign of that table
};

// kBits: the packed code width an encoder always produces (0 = depends on the
// runtime format); kernels instantiate only the packers an encoder can use.
struct EncIdentity {
  static constexpr int kBits = 16;
  __device__ __forceinline__ Result encode(uint32_t h) const { return Result{h, h}; }
};

struct EncFp16 {
  static constexpr int kBits = 16;
  __device__ __forceinline__ Result encode(uint32_t h) const {
    uint32_t b = f2bf(h2f_exact(f2h_exact(bf2f(h))));
    return Result{b, b};
  }
};

template <int N, int ES>
struct EncPositC {
  static constexpr int kBits = N <= 4 ? 4 : (N <= 6 ? 6 : (N <= 8 ? 8 : 16));
  __device__ __forceinline__ Result encode(uint32_t h) const {
    return Posit{N, ES}.encode(h);
  }
};

struct EncPosit {
  static constexpr int kBits = 0;
  Posit p;
  __device__ __forceinline__ Result encode(uint32_t h) const { return p.encode(h); }
};

template <int EB, int MB, bool UNS>
struct EncFpCoreC {
  static constexpr int kBits = EB + MB + (UNS ? 0 : 1);
  float max_norm;
  __device__ __forceinline__ Result encode(uint32_t h) const {
    return FpCore{EB, MB, max_norm, UNS}.encode(h);
  }
};

struct EncFpCore {
  static constexpr int kBits = 0;
  FpCore f;
  __device__ __forceinline__ Result encode(uint32_t h) const { return f.encode(h); }
};

struct EncNvFp8 {
  static constexpr int kBits = 8;
  NvFp8 f;
  __device__ __forceinline__ Result encode(uint32_t h) const { return f.encode(h); }
};

struct EncInt {
  static constexpr int kBits = 0;
  IntFmt f;
  __device__ __forceinline__ Result encode(uint32_t h) const { return f.encode(h); }
};

// Sorted level set with a precomputed 65536-entry code table (NormalFloat and
// per-tensor codebooks); value = levels[code].
struct EncLevels {
  static constexpr int kBits = 0;
  const uint8_t* codes;
  const uint16_t* levels;
  __device__ __forceinline__ Result encode(uint32_t h) const {
    uint32_t c = codes[h & 0xFFFFu];
    return Result{c, levels[c]};
  }
};

// Any 65536-entry bf16 table (a caller's qmap): value = table[h], no code.
struct EncTable {
  static constexpr int kBits = 16;
  const uint16_t* t;
  __device__ __forceinline__ Result encode(uint32_t h) const {
    return Result{0u, (uint32_t)t[h & 0xFFFFu]};
  }
};

// Calls f(encoder) with the encoder object for a descriptor; returns
// kErrInvalid for a descriptor no encoder handles.
template <typename F>
int with_encoder(const FormatDesc& d, F&& f) {
  switch (d.kind) {
    case kFmtIdentity:
      return f(EncIdentity{});
    case kFmtFp16:
      return f(EncFp16{});
    case kFmtPosit:
      if (d.p0 < 2 || d.p0 > 16 || d.p1 < 0 || d.p1 > 3)
        return set_error(kErrInvalid, "posit(%d,%d) outside n in [2,16], es in [0,3]", d.p0, d.p1);
      if (d.p0 == 8 && d.p1 == 1) return f(EncPositC<8, 1>{});
      return f(EncPosit{Posit{d.p0, d.p1}});
    case kFmtFpCore: {
      bool uns = (d.flags & kFlagUnsigned) != 0;
      if (d.p0 < 1 || d.p0 > 8 || d.p1 < 0 || d.p1 > 23)
        return set_error(kErrInvalid, "fp e%dm%d outside supported range", d.p0, d.p1);
      if (!uns && d.p0 == 4 && d.p1 == 3) return f(EncFpCoreC<4, 3, false>{d.max_norm});
      if (!uns && d.p0 == 3 && d.p1 == 2) return f(EncFpCoreC<3, 2, false>{d.max_norm});
      if (!uns && d.p0 == 2 && d.p1 == 1) return f(EncFpCoreC<2, 1, false>{d.max_norm});
      return f(EncFpCore{FpCore{d.p0, d.p1, d.max_norm, uns}});
    }
    case kFmtNvFp8:
      if (d.p0 == 4) return f(EncNvFp8{NvFp8::e4m3()});
      if (d.p0 == 5) return f(EncNvFp8{NvFp8::e5m2()});
      return set_error(kErrInvalid, "NVIDIA fp8 expects e4m3 or e5m2");
    case kFmtInt:
      if (d.p0 < 1 || d.p0 > 31)
        return set_error(kErrInvalid, "int%d outside [1,31]", d.p0);
      return f(EncInt{IntFmt{d.p0, d.p1 != 0}});
    case kFmtLevels:
      if (!d.code_table || !d.levels)
        return set_error(kErrInvalid, "level format needs its code table and levels");
      return f(EncLevels{d.code_table, d.levels});
    case kFmtTable:
      if (!d.value_table) return set_error(kErrInvalid, "table format needs its 65536-entry table");
      return f(EncTable{d.value_table});
    default:
      return set_error(kErrInvalid, "unknown format kind %d", d.kind);
  }
}

}  // namespace vqx
