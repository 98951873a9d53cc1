// Compact code/value lookup tables for the streaming kernels.
//
// For a format with codes of at most 8 bits, every bf16 magnitude below some
// T0 encodes like the smallest positive magnitude (flush / round to zero) and
// every magnitude from T1 up to the special threshold S encodes like the
// largest (saturation), separately for each sign.  Between them the table
// holds, for both signs, one 32-bit entry per bf16 magnitude:
//   entry = value (bf16 bits) | code << 16
// so one LDS read gives both outputs.  Index of a bf16 pattern h with
// magnitude a = h & 0x7FFF < S:  med3(a, T0 - 1, T1) - (T0 - 1)  (entry 0
// stands for every magnitude below T0, which also covers +0; -0 has its own
// entry because the reference maps it to +0 while tiny negatives keep -0).
// Magnitudes >= S (Inf, NaN and the fp formats' NaN region) take the exact
// closed-form encoder.  The table is built on the GPU by the closed-form
// encoders themselves (vqx_build_lut), so it is exact by construction.
#pragma once

#include "vqx_common.h"

namespace vqx {

// Blob layout in device memory (uint32 words).
enum LutHeader : int {
  kLutValid = 0,    // 1 when the table is usable
  kLutT0m1 = 1,     // T0 - 1
  kLutT1 = 2,       // T1
  kLutS = 3,        // special threshold S
  kLutLen = 4,      // entries per sign = T1 - (T0 - 1) + 1
  kLutZeroSign = 5,  // 1: -0 encodes like tiny negatives; 0: like +0
  kLutHeaderWords = 16,
};

constexpr int kLutMaxLen = 8192;  // entries per sign (64 KiB of LDS for both signs)
// full table scratch (65536 entries) + header + two signed tables
constexpr int64_t kLutBytes = (int64_t)(kLutHeaderWords + 2 * kLutMaxLen + 65536) * 4;

// Host-side view, filled from the format descriptor.
struct LutView {
  const uint32_t* blob;  // device blob (header + tables)
  int32_t len;           // entries per sign (host copy of kLutLen)
};

// Device-side parameters after the LDS copy.
struct LutLds {
  const uint32_t* pos;  // LDS: len entries for h >= 0, then len entries for h < 0
  uint32_t len, t0m1, t1, s, zsign;
};

// The blob's header words (uniform loads) and the LDS view of its tables.
__device__ __forceinline__ LutLds lut_header(const uint32_t* blob, int len, const uint32_t* lds) {
  LutLds v;
  v.pos = lds;
  v.len = (uint32_t)len;
  v.t0m1 = blob[kLutT0m1];
  v.t1 = blob[kLutT1];
  v.s = blob[kLutS];
  v.zsign = blob[kLutZeroSign];
  return v;
}

// The copy loops below issue kLutCopyBatch loads per thread before the first
// LDS store (clamped indices, no branch between the loads), so a workgroup's
// prologue waits for one round trip per batch rather than one per word.
constexpr int kLutCopyBatch = 8;
template <typename F>
__device__ __forceinline__ void lut_copy_batched(const uint32_t* __restrict__ src, int n, F&& put) {
  for (int b = 0; b < n; b += kLutCopyBatch * (int)blockDim.x) {
    uint32_t r[kLutCopyBatch];
#pragma unroll
    for (int u = 0; u < kLutCopyBatch; ++u) {
      const int i = b + u * (int)blockDim.x + (int)threadIdx.x;
      r[u] = src[i < n ? i : n - 1];
    }
#pragma unroll
    for (int u = 0; u < kLutCopyBatch; ++u) {
      const int i = b + u * (int)blockDim.x + (int)threadIdx.x;
      if (i < n) put(i, r[u]);
    }
  }
}

// Cooperative copy of the two signed tables into LDS; returns the view.
// Call with all threads of the workgroup; includes the barrier.
__device__ __forceinline__ LutLds lut_to_lds(const uint32_t* blob, int len, uint32_t* lds) {
  const LutLds v = lut_header(blob, len, lds);
  lut_copy_batched(blob + kLutHeaderWords, 2 * len, [&](int i, uint32_t w) { lds[i] = w; });
  __syncthreads();
  return v;
}

// Codes-only copy of the two signed tables into LDS, for kernels that write
// packed codes and nothing else: one byte per magnitude holding the code, so
// an entry's address is the table base plus the bf16 bits themselves; CB 4
// adds a second copy kCodeCopy2 bytes further on holding the code shifted into
// the high nibble, so a byte of two codes is the OR of an even and an odd
// element's entries (read at the same address plus an immediate offset).
// Call with all threads of the workgroup; includes the barrier.
constexpr int kCodeCopy2 = 4096;  // CB 4 needs 2 * len <= kCodeCopy2
template <int CB>
__device__ __forceinline__ LutLds lut_codes_to_lds(const uint32_t* blob, int len, uint32_t* lds) {
  static_assert(CB == 4 || CB == 8, "code tables hold 4- or 8-bit codes");
  const LutLds v = lut_header(blob, len, lds);
  uint8_t* l8 = reinterpret_cast<uint8_t*>(lds);
  lut_copy_batched(blob + kLutHeaderWords, 2 * len, [&](int i, uint32_t w) {
    const uint32_t c = w >> 16;
    l8[i] = (uint8_t)c;
    if constexpr (CB == 4) l8[kCodeCopy2 + i] = (uint8_t)(c << 4);
  });
  __syncthreads();
  return v;
}

// Entry for a bf16 pattern whose magnitude is below S.
__device__ __forceinline__ uint32_t lut_index(const LutLds& t, uint32_t h) {
  uint32_t a = h & 0x7FFFu;
  uint32_t c = a < t.t0m1 ? t.t0m1 : a;  // clamp into [T0 - 1, T1] (v_med3_u32)
  c = c > t.t1 ? t.t1 : c;
  uint32_t neg = ((a != 0u) | t.zsign) ? (h >> 15) & 1u : 0u;
  return c - t.t0m1 + neg * t.len;
}

__device__ __forceinline__ uint32_t lut_entry(const LutLds& t, uint32_t h) { return t.pos[lut_index(t, h)]; }

}  // namespace vqx
