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

// Decision thresholds.  With v clamped into [c[0], c[K-1]] and d_j =
// |fl(v - c_j)| the reference's distance to entry j, the code is the first
// index of the smallest d_j.  If every two distinct neighbouring entries differ
// by at least four ulps of the row's range R = c[K-1] - c[0] (no two distinct
// entries on one side of v can then round to equal distances), the code is
// non-decreasing in v and exceeds i exactly when d_b < d_a, with a = c[i] and
// b the first later entry above a (duplicates of a never win: the lowest index
// does).  That predicate is false up to a, true from b on and monotone in
// between, so the code is the number of thresholds at or below the value's
// key, t[i] = the smallest key with d_b < d_a, found by binary search over the
// bf16 keys.  No later entry above a: no threshold (0x10000, above every
// key).  A row that fails the gap condition (entries closer than the fp32
// resolution of its distances, where several entries round to the same
// distance and counting pairwise decisions misses the first of them) is
// encoded by nearest_sorted instead.

// Smallest gap between distinct entries under which the threshold search is
// exact (+Inf when the range is not finite: every pair fails).
__device__ __forceinline__ float exact_gap(float lo, float hi) {
  const float r = hi - lo;
  if (!(r < __builtin_huge_valf())) return __builtin_huge_valf();
  const uint32_t e = f2u(r) >> 23;  // r >= 0: biased exponent
  const float ulp = e > 23 ? u2f((e - 23) << 23) : u2f(1u << (e > 0 ? e - 1 : 0));
  return 4.0f * ulp;
}

// Threshold i of the row; clears ok when the pair (a, b) is closer than gap.
__device__ uint32_t code_threshold(const float* cb, int K, int i, float gap, bool& ok) {
  const float a = cb[i];
  int j = i + 1;
  while (j < K && !(cb[j] > a)) ++j;
  if (j == K) return 0x10000u;
  const float b = cb[j];
  if (!(b - a >= gap)) ok = false;
  const float vmin = cb[0], vmax = cb[K - 1];
  auto closer_to_b = [&](int k) {
    float v = bf2f(key_bf16((uint32_t)k));
    v = v < vmin ? vmin : (v > vmax ? vmax : v);
    return __builtin_fabsf(b - v) < __builtin_fabsf(v - a);
  };
  // Invariant: closer_to_b(lo) is false, closer_to_b(hi) true.  The switch
  // usually sits within a key or two of the midpoint, so a bracket of the
  // midpoint's key is tried first (it checks itself); where fp32 absorption
  // moves the switch away from the midpoint (entries of opposite signs close
  // to zero) the bracket fails and the search covers [a, b]: lo below a
  // (or -Inf), hi above b (or +Inf, which clamps to c[K-1] >= b).
  const int km = (int)bf16_key(f2bf(0.5f * a + 0.5f * b));
  int lo, hi;
  if (km - 2 >= 0x7F && km + 2 <= 0xFF80 && !closer_to_b(km - 2) && closer_to_b(km + 2)) {
    lo = km - 2;
    hi = km + 2;
  } else {
    lo = (int)bf16_key(f2bf(a)) - 2;
    hi = (int)bf16_key(f2bf(b)) + 2;
    lo = lo < 0x7F ? 0x7F : lo;      // -Inf
    hi = hi > 0xFF80 ? 0xFF80 : hi;  // +Inf
  }
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
constexpr int kCbMaxK = 256;    // entries per row, one per thread of the workgroup

// Search tree of the decision thresholds.  A row with 2^L - 1 thresholds
// (L = 0 .. 8) uses the top of a breadth-first (Eytzinger) tree of 255 slots:
// slot n has children 2n and 2n + 1, the root sits at slot 2^(8 - L), and L
// steps n -> 2n + (threshold(n) <= v) end at slot 256 + code, so the code is
// the low byte of the final slot.  Sorted threshold j has in-order rank
// j + 1 = (2m + 1) 2^h: height h, m-th of its level, slot 2^(7 - h) + m.
// Each level's slots are contiguous, so a level's reads hit distinct LDS
// banks down to 64 slots.
__device__ __forceinline__ uint32_t tree_slot(uint32_t j) {
  const uint32_t r = j + 1;
  const int h = __builtin_ctz(r);
  return (1u << (7 - h)) + (r >> (h + 1));
}

// Threshold key as a value for fp32 comparisons with the bf16 input value:
// keys order like values except that -0 sits just below +0, and no threshold
// separates -0 from +0 (both are at the same distance from every entry), so
// key(t) <= key(v) is t <= v; "no threshold" is NaN, below nothing, and a NaN
// input is below every threshold (code 0, the reference's NaN code).
__device__ __forceinline__ float threshold_value(uint32_t key) {
  return key > 0xFFFFu ? u2f(0x7FC00000u) : bf2f(key_bf16(key));
}

typedef __attribute__((address_space(3))) const float lds_cf32;
__device__ __forceinline__ float lds_f32(uint32_t byte_addr) { return *(lds_cf32*)(size_t)byte_addr; }

// NT: non-temporal loads (faster for the shallow trees, K <= 16: 15.1
// against 16.4 us at C4 K=16; plain loads are faster for the deep ones: 22.7
// against 23.0 us at K=256)
template <bool NT, typename T>
__device__ __forceinline__ void load_chunk(const T* xr, int64_t base, int lane, float (&v)[16]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t e = base + q * 256 + lane * 4;
    if constexpr (std::is_same<T, float>::value) {
      const f32x4* p = reinterpret_cast<const f32x4*>(xr + e);
      f32x4 a = NT ? ld_nt(p) : *p;
      v[4 * q] = a.x; v[4 * q + 1] = a.y; v[4 * q + 2] = a.z; v[4 * q + 3] = a.w;
    } else {
      const u32x2* p = reinterpret_cast<const u32x2*>(xr + e);
      u32x2 a = NT ? ld_nt(p) : *p;
      v[4 * q] = u2f(a.x << 16); v[4 * q + 1] = u2f(a.x & 0xFFFF0000u);
      v[4 * q + 2] = u2f(a.y << 16); v[4 * q + 3] = u2f(a.y & 0xFFFF0000u);
    }
  }
}

// Per-channel encode.  Each row is shared by `split` waves (1, 2 or 4: waves
// gw and gw' with gw / split = gw' / split take the row's chunks s, s + split,
// ... for s = gw % split), and each wave works through its own rows (row
// gw / split, then + nw / split, ... for global wave gw of nw) with no
// workgroup barriers; the items it streams are its 1024-element chunks of
// those rows in order, in two register buffers used in turn: the next item's
// load is issued before the current one is encoded, also across a row
// boundary, so loads stay in flight while a row's search tree is built (each
// wave builds its own copy).  Rows and chunks are wave-uniform (the wave index
// goes through readfirstlane), so the loop's branches are scalar.  The tree
// (see tree_slot) holds the row's K - 1 decision thresholds, padded with "no threshold" to 2^LOGP - 1, in the
// wave's 1 KiB LDS slice.  The search walks LDS byte addresses A = B + 4n
// (B: the slice, 1 KiB aligned): a step is A -> 2A - B + 4c, the root level
// compares against a register copy, and the last step yields
// A / 2 + c = B / 2 + 256 + code, whose low byte is the code.  A lane searches
// G of its values at once, level by level, so G independent LDS reads are in
// flight per wave at each level (G = 16 for the deep trees of 32 entries and
// more, whose waves are few and long; G = 4 for the shallow ones, held to 64
// registers so that 8 waves fit on each SIMD).  fp32 inputs
// are rounded to bf16 two at a time (v_cvt_pk_bf16_f32: round to nearest
// even, NaN kept, subnormals kept under the kernel's f32 denormal mode).
template <typename T, int LOGP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(LOGP <= 4 ? 8 : 1))) void cb_encode_kernel(const T* __restrict__ x, int64_t rows, int64_t cols,
                                                        const float* __restrict__ cb, int K,
                                                        uint8_t* __restrict__ codes, int split) {
  constexpr uint32_t kRoot = 1u << (8 - LOGP);
  __shared__ __attribute__((aligned(1024))) float s_tw[4][256];  // slot n of wave w at s_tw[w][n]
  __shared__ float s_cbw[4][kCbMaxK];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* s_cb = s_cbw[wave];
  float* s_t = s_tw[wave];
  const uint32_t B = (uint32_t)(size_t)(lds_cf32*)s_t;
  const uint32_t kStep0 = 0u - B, kStep1 = 4u - B;               // 2A + these: A -> B + 4(2n + c)
  const uint32_t kLeft = B + 8u * kRoot, kRight = B + 8u * kRoot + 4u;  // A after the root level
  const int64_t gw = (int64_t)blockIdx.x * 4 + wave, nw = (int64_t)gridDim.x * 4;
  const int64_t nchunk = cols / kCbChunk, full = nchunk * kCbChunk;
  float root = 0.0f;
  bool tree = true;  // the row's tree is exact (else nearest_sorted)
  // a word whose low byte is the code of bf16 value f
  auto search = [&](float f) -> uint32_t {
    if constexpr (LOGP == 0) {
      return 0u;
    } else if constexpr (LOGP == 1) {
      return root <= f ? 1u : 0u;
    } else {
      uint32_t A = root <= f ? kRight : kLeft;
#pragma unroll
      for (int l = 1; l < LOGP - 1; ++l) A = (A << 1) + (lds_f32(A) <= f ? kStep1 : kStep0);
      return (A >> 1) + (lds_f32(A) <= f ? 1u : 0u);
    }
  };
  // search for G values at once, level by level
  constexpr int G = LOGP <= 4 ? 4 : 16;
  auto searchG = [&](const float (&f)[G], uint32_t (&out)[G]) {
    if constexpr (LOGP == 0) {
#pragma unroll
      for (int k = 0; k < G; ++k) out[k] = 0u;
    } else if constexpr (LOGP == 1) {
#pragma unroll
      for (int k = 0; k < G; ++k) out[k] = root <= f[k] ? 1u : 0u;
    } else {
      uint32_t A[G];
#pragma unroll
      for (int k = 0; k < G; ++k) A[k] = root <= f[k] ? kRight : kLeft;
#pragma unroll
      for (int l = 1; l < LOGP - 1; ++l) {
        float t[G];
#pragma unroll
        for (int k = 0; k < G; ++k) t[k] = lds_f32(A[k]);
#pragma unroll
        for (int k = 0; k < G; ++k) A[k] = (A[k] << 1) + (t[k] <= f[k] ? kStep1 : kStep0);
      }
      float t[G];
#pragma unroll
      for (int k = 0; k < G; ++k) t[k] = lds_f32(A[k]);
#pragma unroll
      for (int k = 0; k < G; ++k) out[k] = (A[k] >> 1) + (t[k] <= f[k] ? 1u : 0u);
    }
  };
  auto load_cb = [&](int64_t r, float (&c)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] = (r < rows && lane + 64 * j < K) ? cb[r * K + lane + 64 * j] : 0.0f;
  };
  const int64_t nwr = nw / split, s = gw % split;
  float cbn[4];
  load_cb(gw / split, cbn);
  int64_t r = gw / split, c = s;  // current item: chunk c of row r
  // one item: encode chunk (r, c) from cur after loading the next item into nxt
  auto step = [&](const float (&cur)[16], float (&nxt)[16]) {
    if (c == s) {  // new row: its tree from the prefetched codebook
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (lane + 64 * j < K) s_cb[lane + 64 * j] = cbn[j];
      wave_lds_sync();
      const float gap = exact_gap(s_cb[0], s_cb[K - 1]);
      bool ok = true;
      for (int j = lane; j < (1 << LOGP) - 1; j += 64)
        s_t[tree_slot(j)] = threshold_value(j < K - 1 ? code_threshold(s_cb, K, j, gap, ok) : 0x10000u);
      tree = __builtin_amdgcn_ballot_w64(!ok) == 0;
      load_cb(r + nwr, cbn);
      wave_lds_sync();
      if constexpr (LOGP > 0) root = s_t[kRoot];
    }
    const bool last = c + split >= nchunk;
    const int64_t rn = last ? r + nwr : r, cn = last ? s : c + split;
    if (nchunk > 0) {
      if (rn < rows) load_chunk<(LOGP <= 4)>(x + rn * cols, cn * kCbChunk, lane, nxt);  // wave-uniform branch
      uint8_t* cr = codes + r * cols + c * kCbChunk;
#pragma unroll
      for (int h = 0; h < 16; h += G) {
        float f[G];
#pragma unroll
        for (int k = 0; k < G; k += 2) {
          if constexpr (std::is_same<T, float>::value) {
            const uint32_t p = pack_bf16x2(cur[h + k], cur[h + k + 1]);
            f[k] = u2f(p << 16);
            f[k + 1] = u2f(p & 0xFFFF0000u);
          } else {
            f[k] = cur[h + k];  // bf16 values already
            f[k + 1] = cur[h + k + 1];
          }
        }
        uint32_t code[G];
        if (tree) {
          searchG(f, code);
        } else {
#pragma unroll
          for (int k = 0; k < G; ++k) code[k] = nearest_sorted(s_cb, K, f[k]);
        }
#pragma unroll
        for (int q = 0; q < G / 4; ++q) {
          const uint32_t w = pack_low_bytes(code[4 * q], code[4 * q + 1], code[4 * q + 2], code[4 * q + 3]);
          __builtin_nontemporal_store(w, reinterpret_cast<uint32_t*>(cr + (h / 4 + q) * 256 + lane * 4));
        }
      }
    }
    if (last) {  // row done: its tail
      const T* xr = x + r * cols;
      for (int64_t i = full + lane + (s == 0 ? 0 : cols); i < cols; i += 64) {
        float xv = std::is_same<T, float>::value ? u2f(pack_bf16x2((float)xr[i], 0.0f) << 16)
                                                 : u2f((uint32_t)((const uint16_t*)xr)[i] << 16);
        codes[r * cols + i] = (uint8_t)(tree ? search(xv) : nearest_sorted(s_cb, K, xv));
      }
      wave_lds_sync();  // all lanes are done with this row's tree
    }
    r = rn;
    c = cn;
  };
  float va[16], vb[16];
  if (r < rows && nchunk > 0) load_chunk<(LOGP <= 4)>(x + r * cols, c * kCbChunk, lane, va);
  while (r < rows) {
    step(va, vb);
    if (r >= rows) break;
    step(vb, va);
  }
}

// Per-channel decode, organised like the encode: rows shared by `split` waves
// in the same way, each wave streaming its 1024-element chunks of its rows
// through two register buffers, the next chunk's codes loaded before the
// current one is written out, the row's table (bf16 of each entry) in the
// wave's LDS slice.
template <typename T>
__global__ __launch_bounds__(256) void cb_decode_kernel(const uint8_t* __restrict__ codes, int64_t rows,
                                                        int64_t cols, const float* __restrict__ cb, int K,
                                                        T* __restrict__ out, int split) {
  __shared__ float s_cbw[4][kCbMaxK];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  float* s_cb = s_cbw[wave];
  const int64_t gw = (int64_t)blockIdx.x * 4 + wave, nw = (int64_t)gridDim.x * 4;
  const int64_t nchunk = cols / kCbChunk, full = nchunk * kCbChunk;
  auto value = [&](uint32_t c) { return s_cb[c < (uint32_t)K ? c : K - 1]; };
  auto load_cb = [&](int64_t r, float (&c)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] = (r < rows && lane + 64 * j < K) ? cb[r * K + lane + 64 * j] : 0.0f;
  };
  auto load = [&](const uint8_t* p, uint32_t(&d)[4]) {
#pragma unroll
    // plain loads: 12.3 against 16.6 us at C4 with non-temporal ones
    for (int q = 0; q < 4; ++q) d[q] = *reinterpret_cast<const uint32_t*>(p + q * 256 + lane * 4);
  };
  const int64_t nwr = nw / split, s = gw % split;
  float cbn[4];
  load_cb(gw / split, cbn);
  int64_t r = gw / split, c = s;
  auto step = [&](const uint32_t(&cur)[4], uint32_t(&nxt)[4]) {
    if (c == s) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (lane + 64 * j < K) s_cb[lane + 64 * j] = bf2f(f2bf(cbn[j]));
      load_cb(r + nwr, cbn);
      wave_lds_sync();
    }
    const bool last = c + split >= nchunk;
    const int64_t rn = last ? r + nwr : r, cn = last ? s : c + split;
    if (nchunk > 0) {
      if (rn < rows) load(codes + rn * cols + cn * kCbChunk, nxt);  // wave-uniform branch
      T* orow = out + r * cols + c * kCbChunk;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v0 = value(cur[q] & 0xFFu), v1 = value((cur[q] >> 8) & 0xFFu), v2 = value((cur[q] >> 16) & 0xFFu),
              v3 = value(cur[q] >> 24);
        const int e = q * 256 + lane * 4;
        if constexpr (std::is_same<T, float>::value) {
          st_nt(reinterpret_cast<f32x4*>(orow + e), f32x4{v0, v1, v2, v3});
        } else {
          u32x2 a = {(f2u(v0) >> 16) | (f2u(v1) & 0xFFFF0000u), (f2u(v2) >> 16) | (f2u(v3) & 0xFFFF0000u)};
          st_nt(reinterpret_cast<u32x2*>(orow + e), a);
        }
      }
    }
    if (last) {
      const uint8_t* cr = codes + r * cols;
      T* orow = out + r * cols;
      for (int64_t i = full + lane + (s == 0 ? 0 : cols); i < cols; i += 64) {
        float v = value(cr[i]);
        if constexpr (std::is_same<T, float>::value) orow[i] = v;
        else ((uint16_t*)orow)[i] = (uint16_t)(f2u(v) >> 16);
      }
      wave_lds_sync();
    }
    r = rn;
    c = cn;
  };
  uint32_t wa[4], wb[4];
  if (r < rows && nchunk > 0) load(codes + r * cols + c * kCbChunk, wa);
  while (r < rows) {
    step(wa, wb);
    if (r >= rows) break;
    step(wb, wa);
  }
}

// Waves per row for the codebook kernels: 1, 2 or 4 (at most the row's whole
// chunks), whichever leaves the fewest rows' worth of chunks to the busiest
// of the grid's waves (grid: the resident workgroups of 4 waves); the grid is
// then trimmed to the waves that have work.
static int row_split(unsigned& grid, int64_t rows, int64_t nchunk) {
  const int64_t nw = (int64_t)grid * 4;
  int split = 1;
  for (int sp = 2; sp <= 4 && sp <= nchunk; sp *= 2)
    if ((rows * sp + nw - 1) / nw * split < (rows * split + nw - 1) / nw * sp) split = sp;
  grid = (unsigned)std::min<int64_t>(grid, (rows * split + 3) / 4);
  return split;
}

// row_split waves per row, as many waves as fit on the device at once
template <typename T>
static void launch_encode(int logp, hipStream_t st, const T* x, int64_t rows, int64_t cols, const float* cb,
                          int K, uint8_t* codes) {
  const int64_t nchunk = cols / kCbChunk;
#define VQX_CB_CASE(L)                                                                                    \
  case L: {                                                                                               \
    unsigned grid = persistent_grid((const void*)cb_encode_kernel<T, L>, 256, 0, rows * 64 * 4);          \
    const int split = row_split(grid, rows, nchunk);                                                      \
    hipLaunchKernelGGL((cb_encode_kernel<T, L>), dim3(grid), dim3(256), 0, st, x, rows, cols, cb, K, codes, \
                       split);                                                                            \
  } break;
  switch (logp) {
    VQX_CB_CASE(0) VQX_CB_CASE(1) VQX_CB_CASE(2) VQX_CB_CASE(3) VQX_CB_CASE(4)
    VQX_CB_CASE(5) VQX_CB_CASE(6) VQX_CB_CASE(7) default: VQX_CB_CASE(8)
  }
#undef VQX_CB_CASE
}

int codebook_encode(const void* x, int dtype, int64_t rows, int64_t cols, const float* cb, int K,
                    uint8_t* codes, hipStream_t st) {
  if (K < 1 || K > kCbMaxK) return set_error(kErrInvalid, "codebook size %d outside [1,%d]", K, kCbMaxK);
  if (rows < 0 || cols < 0) return set_error(kErrInvalid, "negative shape");
  if (rows == 0 || cols == 0) return kOk;
  if (!aligned(x, 16) || !aligned(codes, 16) || (cols % 16) != 0)
    return set_error(kErrInvalid, "codebook encode needs 16-byte aligned rows (cols %% 16 == 0)");
  int logp = 0;
  while ((1 << logp) < K) ++logp;  // K - 1 thresholds padded to 2^logp - 1 nodes (codes up to 2^logp - 1)
  if (dtype == kF32)
    launch_encode<float>(logp, st, (const float*)x, rows, cols, cb, K, codes);
  else if (dtype == kBF16)
    launch_encode<uint16_t>(logp, st, (const uint16_t*)x, rows, cols, cb, K, codes);
  else
    return set_error(kErrInvalid, "codebook input dtype %d not supported", dtype);
  return check_launch("codebook_encode");
}

int codebook_decode(const uint8_t* codes, int64_t rows, int64_t cols, const float* cb, int K, void* out,
                    int dtype, hipStream_t st) {
  if (K < 1 || K > kCbMaxK) return set_error(kErrInvalid, "codebook size %d outside [1,%d]", K, kCbMaxK);
  if (rows < 0 || cols < 0) return set_error(kErrInvalid, "negative shape");
  if (rows == 0 || cols == 0) return kOk;
  if (!aligned(out, 16) || !aligned(codes, 16) || (cols % 16) != 0)
    return set_error(kErrInvalid, "codebook decode needs 16-byte aligned rows (cols %% 16 == 0)");
  const int64_t work = rows * 64 * 4, nchunk = cols / kCbChunk;  // up to four waves per row
  if (dtype == kF32) {
    unsigned grid = persistent_grid((const void*)cb_decode_kernel<float>, 256, 0, work);
    const int split = row_split(grid, rows, nchunk);
    hipLaunchKernelGGL((cb_decode_kernel<float>), dim3(grid), dim3(256), 0, st, codes, rows, cols, cb, K,
                       (float*)out, split);
  } else if (dtype == kBF16) {
    unsigned grid = persistent_grid((const void*)cb_decode_kernel<uint16_t>, 256, 0, work);
    const int split = row_split(grid, rows, nchunk);
    hipLaunchKernelGGL((cb_decode_kernel<uint16_t>), dim3(grid), dim3(256), 0, st, codes, rows, cols, cb, K,
                       (uint16_t*)out, split);
  } else
    return set_error(kErrInvalid, "codebook output dtype %d not supported", dtype);
  return check_launch("codebook_decode");
}

}  // namespace vqx
