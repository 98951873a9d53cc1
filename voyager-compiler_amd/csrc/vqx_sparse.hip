// Outlier split and CSR kernels behind filter_outlier, quantize_mx_outlier,
// slice_csr_tensor and spmm_csr (src/voyager_compiler/ops/quantized.py:532-895).
//
// filter_outlier over a [batches, rows, cols] input is three launches:
//   1. outlier_count_kernel  one wave per row counts the outliers (|x| > t and
//                            x != 0) and stores the count where the row's end
//                            pointer goes (indptr[b][r + 1]);
//   2. csr_scan_kernel       one workgroup per batch turns those counts into
//                            row pointers in place, clamped to the capacity;
//   3. outlier_split_kernel  one wave per row reads the row again, writes the
//                            inliers, gathers the outliers in column order in
//                            LDS and writes them to their CSR slots as one
//                            contiguous run;
//                            the whole grid then pads data / indices past the
//                            last entry with 0 / -1.
// An outlier's slot is its row's pointer plus its rank within the row; ranks
// come from wave ballots (lane-major, so column order is kept).  Entries past
// the capacity are dropped, which keeps the first max_nnz in row-major order.
//
// The one-pass form (the _ws entry points) reads x once, in two launches:
//   1. outlier_split_kernel<.., STAGE>  as 3. above, but each row's outliers
//                            go to the row's own staging slots in a caller's
//                            workspace (the first `slots` of them) and its
//                            count to counts[row];
//   2. outlier_finalize_kernel  one workgroup per chunk of rows: row pointers
//                            from the counts, the staged entries copied to
//                            their slots, rows that overflowed their staging
//                            read again from x, and the padding.
//
// The column slice of a CSR matrix reuses the same count -> scan -> scatter
// shape over the stored entries; the row slice is one gather launch.
//
// spmm_csr: one wave per (row, 1 KiB column chunk) of the output runs down
// the row's entries in order and accumulates a * B[k, n] in fp32 (B row-major
// [K, N]).  A "kc"-stored or coded/scaled B is first decoded and transposed
// into that layout by csr_decode_kernel, in the dtype the reference's decode
// produces.
#include "vqx_common.h"
#include "vqx_kernels.h"

namespace vqx {
namespace {

// ---------------------------------------------------------------------------
// element traits: storage type, exact widening, round-to-nearest-even narrowing
// ---------------------------------------------------------------------------
template <int DT>
struct FT;
template <>
struct FT<kF32> {
  using S = uint32_t;
  static constexpr int kVec = 4;  // elements per 16 bytes
  __device__ static float val(uint32_t b) { return u2f(b); }
  __device__ static uint32_t bits(float f) { return f2u(f); }
};
template <>
struct FT<kBF16> {
  using S = uint16_t;
  static constexpr int kVec = 8;
  __device__ static float val(uint32_t b) { return bf2f(b); }
  __device__ static uint32_t bits(float f) { return f2bf(f); }
};
template <>
struct FT<kF16> {
  using S = uint16_t;
  static constexpr int kVec = 8;
  __device__ static float val(uint32_t b) { return h2f_exact(b); }
  __device__ static uint32_t bits(float f) { return f2h_exact(f); }
};

// V consecutive elements starting at p: one 16-byte or 4-byte load when V
// fills it, else V element loads.  Element j of the group is get(j).
template <typename S, int V>
struct Group {
  static constexpr int kBytes = V * (int)sizeof(S);
  static constexpr bool kWide = kBytes == 16;
  static constexpr bool kWord = kBytes == 4 && V > 1;
  uint32_t w[kBytes / 4 > 0 ? kBytes / 4 : 1];
  S e[(kWide || kWord) ? 1 : V];
  __device__ void load(const S* p) {
    if constexpr (kWide) {
      u32x4 v = *(const u32x4*)p;
      w[0] = v[0], w[1] = v[1], w[2] = v[2], w[3] = v[3];
    } else if constexpr (kWord) {
      w[0] = *(const uint32_t*)p;
    } else {
#pragma unroll
      for (int j = 0; j < V; ++j) e[j] = p[j];
    }
  }
  __device__ uint32_t get(int j) const {
    if constexpr (kWide || kWord) {
      if constexpr (sizeof(S) == 4) return w[j];
      else return (w[j >> 1] >> ((j & 1) * 16)) & 0xFFFFu;
    } else {
      return (uint32_t)e[j];
    }
  }
};

// NT: non-temporal (streaming) store, so that a write-once output does not
// push re-read data out of the caches.
template <typename S, int V, bool NT = false>
__device__ __forceinline__ void store_group(S* p, const uint32_t (&b)[V]) {
  if constexpr (V * sizeof(S) == 16) {
    u32x4 v;
    if constexpr (sizeof(S) == 4) {
      v = u32x4{b[0], b[1], b[2], b[3]};
    } else {
      v = u32x4{b[0] | b[1] << 16, b[2] | b[3] << 16, b[4] | b[5] << 16, b[6] | b[7] << 16};
    }
    if constexpr (NT) st_nt((u32x4*)p, v);
    else *(u32x4*)p = v;
  } else if constexpr (V * sizeof(S) == 4 && V == 2) {
    *(uint32_t*)p = b[0] | b[1] << 16;
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) p[j] = (S)b[j];
  }
}

__device__ __forceinline__ int64_t min64(int64_t a, int64_t b) { return a < b ? a : b; }

__device__ __forceinline__ bool is_outlier(float v, float t) { return fabsf(v) > t && v != 0.f; }

__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ int64_t wave_sum64(int64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ int64_t wave_incl_scan(int64_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int64_t u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  return v;
}

// ---------------------------------------------------------------------------
// filter_outlier
// ---------------------------------------------------------------------------
// Pass 1 counts each row's outliers.  Row group loads are clamped into the
// row (cols >= V), so every lane loads unconditionally and lanes past the end
// only drop their flags.
template <int DT, int V>
__global__ __launch_bounds__(256) void outlier_count_kernel(const typename FT<DT>::S* __restrict__ x,
                                                            int64_t nrows, int64_t rows, int64_t cols,
                                                            float t, int32_t* __restrict__ indptr) {
  using S = typename FT<DT>::S;
  constexpr int U = 4;
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * 4;
  for (int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); g < nrows; g += nw) {
    const S* row = x + g * cols;
    uint32_t cnt = 0;
    for (int64_t c0 = 0; c0 < cols; c0 += U * 64 * V) {
      Group<S, V> grp[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + (int64_t)(u * 64 + lane) * V;
        ok[u] = c < cols;
        grp[u].load(row + (ok[u] ? c : cols - V));
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < V; ++j) cnt += (ok[u] && is_outlier(FT<DT>::val(grp[u].get(j)), t)) ? 1u : 0u;
    }
    cnt = wave_sum(cnt);
    if (lane == 0) {
      const int64_t b = g / rows, r = g - b * rows;
      indptr[b * (rows + 1) + r + 1] = (int32_t)cnt;
    }
  }
}

// In place: indptr[b][r + 1] holds row r's count on entry and
// min(prefix, max_nnz) + offset on exit (int32 wrap-around, as the
// reference's int32 add); indptr[b][0] = offset.
__global__ __launch_bounds__(1024) void csr_scan_kernel(int32_t* __restrict__ indptr, int64_t rows, int64_t max_nnz,
                                                        int32_t offset) {
  __shared__ int64_t wsum[16];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t b = blockIdx.x;
  int32_t* ptr = indptr + b * (rows + 1);
  const int64_t per = (rows + 1023) / 1024;
  const int64_t r0 = min64(tid * per, rows), r1 = min64(r0 + per, rows);
  int64_t s = 0;
  for (int64_t r = r0; r < r1; ++r) s += ptr[r + 1];
  const int64_t incl = wave_incl_scan(s, lane);
  if (lane == 63) wsum[wv] = incl;
  __syncthreads();
  int64_t before = 0;
  for (int w = 0; w < wv; ++w) before += wsum[w];
  int64_t run = before + incl - s;
  for (int64_t r = r0; r < r1; ++r) {
    run += ptr[r + 1];
    const int64_t c = run < max_nnz ? run : max_nnz;
    ptr[r + 1] = (int32_t)((uint32_t)c + (uint32_t)offset);
  }
  if (tid == 0) ptr[0] = offset;
}

// Slots [indptr[b][rows] - indptr[b][0], max_nnz) of every batch's data /
// indices get 0 / -1, spread over the whole grid (the pointers are clamped,
// so the kept entries never reach past max_nnz).
template <typename S>
__device__ void pad_tail(const int32_t* __restrict__ indptr, int64_t rows, int64_t nb, int64_t max_nnz,
                         S* __restrict__ data, int32_t* __restrict__ indices) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x, nt = (int64_t)gridDim.x * blockDim.x;
  for (int64_t b = 0; b < nb; ++b) {
    const int32_t* ptr = indptr + b * (rows + 1);
    const int64_t used = (int64_t)(uint32_t)((uint32_t)ptr[rows] - (uint32_t)ptr[0]);
    for (int64_t j = used + tid; j < max_nnz; j += nt) {
      data[b * max_nnz + j] = (S)0;
      indices[b * max_nnz + j] = -1;
    }
  }
}

// Pass 2 reads each row again, writes the inliers (every |x| > t becomes +0,
// zeros too when t is negative) and moves the outliers (the nonzero ones), in
// column order, to their CSR slots.  Each wave gathers its row's outliers in
// an LDS buffer
// (slot = running count + rank from the ballots) and writes them out as one
// contiguous run when the row ends or the buffer nears full, instead of
// scattering 2- and 4-byte stores.
// quantize_mx_outlier's inlier quantization fused into the split (bf16,
// blocks of V * LPB along the row): the inliers' block scale as
// calculate_mx_qparam forms it and qmap[bf16(inlier / scale)] as quantize
// does (quantized.py:688-699), in place of the inliers themselves.
struct MxFuse {
  ScaleParams sp;
  const uint16_t* qmap;  // 65536 bf16 values
  uint16_t* scale;       // [rows, cols / (V * LPB)] bf16
};

// The one-pass form (STAGE) has no row pointers yet: each row's outliers go
// to the row's own staging slots (the first `slots` of them, in column
// order) and its count to counts[row]; outlier_finalize_kernel then places
// them.
struct Stage {
  int32_t* counts;  // [nb * rows]
  int32_t* col;     // [nb * rows][slots]
  void* val;        // [nb * rows][slots], x's storage type
  int64_t slots;
};

template <int DT, int V, bool MXQ = false, int LPB = 1, bool STAGE = false>
__global__ __launch_bounds__(256) void outlier_split_kernel(const typename FT<DT>::S* __restrict__ x,
                                                            int64_t nb, int64_t rows, int64_t cols,
                                                            float t, const int32_t* __restrict__ indptr,
                                                            int64_t max_nnz, typename FT<DT>::S* __restrict__ inlier,
                                                            typename FT<DT>::S* __restrict__ data,
                                                            int32_t* __restrict__ indices, MxFuse mf = {},
                                                            Stage sg = {}) {
  static_assert(!MXQ || (DT == kBF16 && V == 8), "the fused MX quantization takes bf16 groups of 8");
  using S = typename FT<DT>::S;
  constexpr int U = 4;
  constexpr uint32_t CAP = 1024, FLUSH = CAP - 64 * V;  // a group adds at most 64 * V
  __shared__ S s_val[4][CAP];
  __shared__ uint32_t s_col[4][CAP];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  S* bval = s_val[wv];
  uint32_t* bcol = s_col[wv];
  const int64_t nw = (int64_t)gridDim.x * 4;
  const int64_t nrows = nb * rows;
  for (int64_t g = (int64_t)blockIdx.x * 4 + wv; g < nrows; g += nw) {
    const int64_t b = g / rows, r = g - b * rows;
    int64_t pos, lim;
    S* drow;
    int32_t* crow;
    if constexpr (STAGE) {
      pos = 0;
      lim = sg.slots;
      drow = (S*)sg.val + g * sg.slots;
      crow = sg.col + g * sg.slots;
    } else {
      const int32_t* ptr = indptr + b * (rows + 1);
      pos = (int64_t)(uint32_t)((uint32_t)ptr[r] - (uint32_t)ptr[0]);
      lim = max_nnz;
      drow = data + b * max_nnz;
      crow = indices + b * max_nnz;
    }
    const S* row = x + g * cols;
    S* irow = inlier + g * cols;
    uint32_t nbuf = 0;
    auto flush = [&]() {
      wave_lds_sync();
      for (uint32_t i = lane; i < nbuf; i += 64) {
        const int64_t p = pos + i;
        if (p < lim) {
          drow[p] = (S)bval[i];
          crow[p] = (int32_t)bcol[i];
        }
      }
      wave_lds_sync();
      pos += nbuf;
      nbuf = 0;
    };
    for (int64_t c0 = 0; c0 < cols; c0 += U * 64 * V) {
      Group<S, V> grp[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + (int64_t)(u * 64 + lane) * V;
        ok[u] = c < cols;
        grp[u].load(row + (ok[u] ? c : cols - V));
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t c = (uint32_t)(c0 + (u * 64 + lane) * V);
        bool f[V];
        uint32_t keep[V];
        uint32_t below = 0, n = 0;
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const uint32_t e = grp[u].get(j);
          const float v = FT<DT>::val(e);
          keep[j] = fabsf(v) > t ? 0u : e;
          f[j] = ok[u] && is_outlier(v, t);
          const uint64_t m = __ballot(f[j]);
          below += lanes_below(m);
          n += (uint32_t)__popcll(m);
        }
        if constexpr (MXQ) {
          // the block's scale from its inliers' magnitudes over LPB lanes (a
          // block is wholly inside or wholly past the row, as cols % (8 LPB)
          // == 0), then each inlier quantized through the table
          uint32_t am = 0;
#pragma unroll
          for (int j = 0; j < V; ++j) am = umax32(am, keep[j] & 0x7FFFu);
          am = block_max<LPB>(am);
          const float sc = mf.sp.mode == 0 ? block_scale_bf16<false>(am, mf.sp) : block_scale_bf16<true>(am, mf.sp);
          // a power-of-two scale with a representable reciprocal divides
          // exactly as a multiply (both round the same real x / s once)
          const uint32_t sb = f2u(sc), se = (sb >> 23) & 0xFFu;
          const bool p2 = (sb & 0x807FFFFFu) == 0 && se - 1u < 253u;
          uint32_t qv[V];
          if (__builtin_amdgcn_ballot_w64(!p2 || am > 0x7F80u) == 0) {
            // no NaN inlier in the wave: v_cvt_pk_bf16_f32 rounds the
            // quotients two at a time, as f2bf does for every non-NaN value
            const float rc = u2f((254u - se) << 23);
#pragma unroll
            for (int j = 0; j < V; j += 2) {
              const uint32_t h = pack_bf16x2(bf2f(keep[j]) * rc, bf2f(keep[j + 1]) * rc);
              qv[j] = mf.qmap[h & 0xFFFFu];
              qv[j + 1] = mf.qmap[h >> 16];
            }
          } else if (__builtin_amdgcn_ballot_w64(!p2) == 0) {
            const float rc = u2f((254u - se) << 23);
#pragma unroll
            for (int j = 0; j < V; ++j) qv[j] = mf.qmap[f2bf(bf2f(keep[j]) * rc)];
          } else {
#pragma unroll
            for (int j = 0; j < V; ++j) qv[j] = mf.qmap[f2bf(bf2f(keep[j]) / sc)];
          }
          if (ok[u]) {
            store_group<S, V, true>(irow + c, qv);
            if (lane % LPB == 0) mf.scale[g * (cols / (V * LPB)) + c / (V * LPB)] = (uint16_t)f2bf(sc);
          }
        } else {
          if (ok[u]) store_group<S, V, true>(irow + c, keep);
        }
        if (n != 0) {
          uint32_t q = nbuf + below;
#pragma unroll
          for (int j = 0; j < V; ++j) {
            if (f[j]) {
              bval[q] = (S)grp[u].get(j);
              bcol[q] = c + j;
              ++q;
            }
          }
          nbuf += n;
          if (nbuf >= FLUSH) flush();
        }
      }
    }
    if (nbuf != 0) flush();
    if constexpr (STAGE) {
      if (lane == 0) sg.counts[g] = (int32_t)pos;
    }
  }
  if constexpr (!STAGE) pad_tail(indptr, rows, nb, max_nnz, data, indices);
}

// The one-pass form's second launch, one workgroup per (batch, chunk of 16
// to 256 rows): the chunk's row pointers (the batch's counts before the
// chunk summed, then a scan over the chunk's own), its rows' staged
// outliers copied to their slots, and its share of the batch's unused slots
// padded with 0 / -1.  The chunk's entries fill one contiguous run of slots,
// so each thread takes slots of that run (a binary search over the chunk's
// row starts names the row) and all the copies are independent.  A row with
// more outliers than staging slots reads its row of x again and places all
// of them, in column order, directly.  The pointers clamp to max_nnz and add
// the offset as csr_scan_kernel does, and every entry lands where the
// two-pass form puts it.  Each workgroup reads the batch's whole count array
// (L2-resident: 4 bytes per row).
template <int DT, int V>
__global__ __launch_bounds__(256) void outlier_finalize_kernel(const typename FT<DT>::S* __restrict__ x,
                                                               int64_t rows, int64_t cols, float t, Stage sg,
                                                               int64_t chunk, int64_t nchunk, int64_t max_nnz,
                                                               int32_t offset, typename FT<DT>::S* __restrict__ data,
                                                               int32_t* __restrict__ indices,
                                                               int32_t* __restrict__ indptr) {
  using S = typename FT<DT>::S;
  constexpr int U = 16;
  __shared__ int64_t red[2][4];
  __shared__ int64_t wtot[4];
  __shared__ int64_t first[256];  // slot of each chunk row's first outlier, before clamping
  __shared__ int32_t ncnt[256];   // each chunk row's count
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t b = blockIdx.x / nchunk, c = blockIdx.x - b * nchunk;
  const int64_t r0 = c * chunk, r1 = min64(r0 + chunk, rows), nr = r1 - r0;
  const int32_t* cnt = sg.counts + b * rows;
  // every load unconditional (indices clamped into the array, values
  // masked), so that all of a thread's loads are in flight together
  const int64_t r = r0 + tid;
  int32_t v = rows > 0 ? cnt[min64(r, rows - 1)] : 0;
  v = tid < nr ? v : 0;
  int64_t pre = 0, tot = 0;
  const int last = (int)rows - 1;  // rows < 2^31
  for (int q = tid; q <= last; q += 256 * U) {
    int32_t w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = cnt[min(q + 256 * u, last)];
    // all U loads issue before the first use
    __builtin_amdgcn_sched_barrier(0);
    int64_t st = 0, sp = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = q + 256 * u;
      st += i <= last ? w[u] : 0;
      sp += i < r0 ? w[u] : 0;
    }
    tot += st;
    pre += sp;
  }
  pre = wave_sum64(pre);
  tot = wave_sum64(tot);
  if (lane == 0) red[0][wv] = pre, red[1][wv] = tot;
  const int64_t incl = wave_incl_scan(v, lane);
  if (lane == 63) wtot[wv] = incl;
  __syncthreads();
  pre = red[0][0] + red[0][1] + red[0][2] + red[0][3];
  tot = red[1][0] + red[1][1] + red[1][2] + red[1][3];
  int64_t before = pre;
  for (int w = 0; w < wv; ++w) before += wtot[w];
  first[tid] = before + incl - v;
  ncnt[tid] = v;
  if (tid < nr) {
    const int64_t e = before + incl;
    indptr[b * (rows + 1) + r + 1] = (int32_t)((uint32_t)(e < max_nnz ? e : max_nnz) + (uint32_t)offset);
  }
  if (c == 0 && tid == 0) indptr[b * (rows + 1)] = offset;
  __syncthreads();
  S* drow = data + b * max_nnz;
  int32_t* crow = indices + b * max_nnz;
  {
    const int64_t lo = tot < max_nnz ? tot : max_nnz, span = max_nnz - lo;
    const int64_t a1 = lo + span * (c + 1) / nchunk;
    for (int64_t j = lo + span * c / nchunk + tid; j < a1; j += 256) {
      drow[j] = (S)0;
      crow[j] = -1;
    }
  }
  const int64_t run0 = first[0];
  const int64_t run1 = min64(pre + (wtot[0] + wtot[1] + wtot[2] + wtot[3]), max_nnz);
  constexpr int P = 4;  // slots per thread in flight
  for (int64_t p0 = run0 + tid; sg.slots > 0 && p0 < run1; p0 += 256 * P) {
    S dv[P];
    int32_t cv[P];
    bool take[P];
#pragma unroll
    for (int u = 0; u < P; ++u) {
      const int64_t p = p0 + 256 * u;
      // the chunk row whose run holds slot p: the last i < nr with first[i] <= p
      int lo = 0, hi = (int)nr - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (first[mid] <= p) lo = mid;
        else hi = mid - 1;
      }
      take[u] = p < run1 && ncnt[lo] <= sg.slots;
      // a slot not taken reads staging entry 0 (slots > 0 here)
      const int64_t k = take[u] ? (b * rows + r0 + lo) * sg.slots + (p - first[lo]) : 0;
      dv[u] = ((const S*)sg.val)[k];
      cv[u] = sg.col[k];
    }
#pragma unroll
    for (int u = 0; u < P; ++u) {
      if (take[u]) {
        drow[p0 + 256 * u] = dv[u];
        crow[p0 + 256 * u] = cv[u];
      }
    }
  }
  for (int64_t i = wv; i < nr; i += 4) {
    const int64_t p0 = first[i], n = ncnt[i];
    if (n <= sg.slots || p0 >= max_nnz) continue;
    const S* row = x + (b * rows + r0 + i) * cols;
    int64_t pos = p0;
    for (int64_t c0 = 0; c0 < cols && pos < max_nnz; c0 += 64 * V) {
      const int64_t cc = c0 + (int64_t)lane * V;
      const bool ok = cc < cols;
      Group<S, V> grp;
      grp.load(row + (ok ? cc : cols - V));
      bool f[V];
      uint32_t below = 0, n_grp = 0;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        f[j] = ok && is_outlier(FT<DT>::val(grp.get(j)), t);
        const uint64_t m = __ballot(f[j]);
        below += lanes_below(m);
        n_grp += (uint32_t)__popcll(m);
      }
      int64_t q = pos + below;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        if (f[j]) {
          if (q < max_nnz) {
            drow[q] = (S)grp.get(j);
            crow[q] = (int32_t)(cc + j);
          }
          ++q;
        }
      }
      pos += n_grp;
    }
  }
}

// ---------------------------------------------------------------------------
// slice_csr_tensor
// ---------------------------------------------------------------------------
// Rows [start, start + nrows_out): rebased pointers and the entries they cover.
template <typename S>
__global__ __launch_bounds__(256) void csr_slice_rows_kernel(const S* __restrict__ data,
                                                             const int32_t* __restrict__ indices,
                                                             const int32_t* __restrict__ indptr, int64_t nnz_in,
                                                             int64_t start, int64_t nrows_out, int64_t max_nnz,
                                                             S* __restrict__ data_out, int32_t* __restrict__ indices_out,
                                                             int32_t* __restrict__ indptr_out) {
  const int64_t s0 = indptr[start];
  const int64_t nse = (int64_t)indptr[start + nrows_out] - s0;
  const bool over = nse > max_nnz;
  const int64_t n = max_nnz > nrows_out + 1 ? max_nnz : nrows_out + 1;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    if (i <= nrows_out) {
      int64_t v = (int64_t)indptr[start + i] - s0;
      if (over && v > max_nnz) v = max_nnz;
      indptr_out[i] = (int32_t)v;
    }
    if (i < max_nnz) {
      const int64_t p = s0 + i;
      const bool real = i < nse && p >= 0 && p < nnz_in;
      data_out[i] = real ? data[p] : (S)0;
      indices_out[i] = real ? indices[p] : -1;
    }
  }
}

// Column slice [start, end): per-row count of the stored entries in range,
// written where the row's end pointer goes (csr_scan_kernel follows, then
// csr_cols_scatter_kernel).
__global__ __launch_bounds__(256) void csr_cols_count_kernel(const int32_t* __restrict__ indices,
                                                             const int32_t* __restrict__ indptr, int64_t rows,
                                                             int64_t nnz_in, int64_t start, int64_t end,
                                                             int32_t* __restrict__ indptr_out) {
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * 4;
  for (int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += nw) {
    int64_t p0 = indptr[r], p1 = indptr[r + 1];
    p0 = p0 < 0 ? 0 : (p0 > nnz_in ? nnz_in : p0);
    p1 = p1 < p0 ? p0 : (p1 > nnz_in ? nnz_in : p1);
    uint32_t cnt = 0;
    for (int64_t p = p0 + lane; p < p1; p += 64) {
      const int64_t k = indices[p];
      cnt += (k >= start && k < end) ? 1u : 0u;
    }
    cnt = wave_sum(cnt);
    if (lane == 0) indptr_out[r + 1] = (int32_t)cnt;
  }
}

template <typename S>
__global__ __launch_bounds__(256) void csr_cols_scatter_kernel(const S* __restrict__ data,
                                                               const int32_t* __restrict__ indices,
                                                               const int32_t* __restrict__ indptr, int64_t rows,
                                                               int64_t nnz_in, int64_t start, int64_t end,
                                                               int64_t max_nnz, const int32_t* __restrict__ indptr_out,
                                                               S* __restrict__ data_out,
                                                               int32_t* __restrict__ indices_out) {
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * 4;
  for (int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += nw) {
    int64_t p0 = indptr[r], p1 = indptr[r + 1];
    p0 = p0 < 0 ? 0 : (p0 > nnz_in ? nnz_in : p0);
    p1 = p1 < p0 ? p0 : (p1 > nnz_in ? nnz_in : p1);
    int64_t pos = indptr_out[r];
    for (int64_t q0 = p0; q0 < p1 && pos < max_nnz; q0 += 64) {
      const int64_t p = q0 + lane;
      const bool live = p < p1;
      const int64_t k = live ? indices[p] : -1;
      const bool f = live && k >= start && k < end;
      const uint64_t m = __ballot(f);
      const int64_t o = pos + lanes_below(m);
      if (f && o < max_nnz) {
        data_out[o] = data[p];
        indices_out[o] = (int32_t)(k - start);
      }
      pos += __popcll(m);
    }
  }
  pad_tail(indptr_out, rows, 1, max_nnz, data_out, indices_out);
}

// ---------------------------------------------------------------------------
// spmm_csr
// ---------------------------------------------------------------------------
__device__ __forceinline__ float load_f(const void* p, int dt, int64_t i) {
  switch (dt) {
    case kF32: return ((const float*)p)[i];
    case kBF16: return bf2f(((const uint16_t*)p)[i]);
    case kF16: return h2f_exact(((const uint16_t*)p)[i]);
    default: return (float)((const uint8_t*)p)[i];
  }
}

__device__ __forceinline__ float round_as(float v, int dt) {
  switch (dt) {
    case kBF16: return bf2f(f2bf(v));
    case kF16: return h2f_exact(f2h_exact(v));
    default: return v;
  }
}

__device__ __forceinline__ void store_f(void* p, int dt, int64_t i, float v) {
  switch (dt) {
    case kF32: ((float*)p)[i] = v; break;
    case kBF16: ((uint16_t*)p)[i] = (uint16_t)f2bf(v); break;
    default: ((uint16_t*)p)[i] = (uint16_t)f2h_exact(v); break;
  }
}

// Bt[b][k][n] = decode(B[b][n][k]) ("kc", transpose) or decode(B[b][k][n])
// ("ck"), 64x64 tiles through LDS.  decode(v) = code[trunc(v)] (negative
// indices count from the end; out of range -> NaN) and, with a scale,
// round_to(out_dtype, value * scale) with the scale expanded by block.
__global__ __launch_bounds__(256) void csr_decode_kernel(CsrDecode d) {
  __shared__ float tile[64][65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t tr = (d.br + 63) / 64, tc = (d.bc + 63) / 64;
  const int64_t ntiles = d.nb * tr * tc;
  for (int64_t tIdx = blockIdx.x; tIdx < ntiles; tIdx += gridDim.x) {
    const int64_t b = tIdx / (tr * tc), rem = tIdx - b * tr * tc;
    const int64_t r0 = rem / tc * 64, c0 = rem % tc * 64;
    const int64_t c = c0 + tx;
    for (int i = ty; i < 64; i += 4) {
      const int64_t r = r0 + i;
      float v = 0.f;
      if (r < d.br && c < d.bc) {
        v = load_f(d.B, d.b_dtype, (b * d.br + r) * d.bc + c);
        if (d.code) {
          if (!(v == v) || fabsf(v) >= (float)d.code_len + 1.f) {
            v = __builtin_nanf("");
          } else {
            int64_t k = (int64_t)v;
            if (k < 0) k += d.code_len;
            v = (k >= 0 && k < d.code_len) ? load_f(d.code, d.code_dtype, k) : __builtin_nanf("");
          }
        }
        if (d.scale) {
          const int64_t si = b * d.sb_stride + (r / d.rdiv) * d.sc + c / d.cdiv;
          v = round_as(v * load_f(d.scale, d.scale_dtype, si), d.out_dtype);
        }
      }
      tile[i][tx] = v;
    }
    __syncthreads();
    if (d.transpose) {
      // out[b][c0 + i][r0 + tx] = tile[tx][i]: out is [nb, bc, br]
      for (int i = ty; i < 64; i += 4) {
        const int64_t oc = c0 + i, orow = r0 + tx;
        if (oc < d.bc && orow < d.br) store_f(d.out, d.out_dtype, (b * d.bc + oc) * d.br + orow, tile[tx][i]);
      }
    } else {
      for (int i = ty; i < 64; i += 4) {
        const int64_t r = r0 + i;
        if (r < d.br && c < d.bc) store_f(d.out, d.out_dtype, (b * d.br + r) * d.bc + c, tile[i][tx]);
      }
    }
    __syncthreads();
  }
}

// out[g][n] = round(sum over the row's entries p, in order, of a_p * B[k_p][n])
// (+ addend[g][n], rounded again, when given).  One wave per (row, slice of
// 64*V columns: 1 KiB of a B row); entries are read eight at a time.  Each
// entry reads its piece of a B row from L2 / MALL: nnz * N * sizeof(B) bytes
// gathered in all, so the items are ordered for the L2s: taken slice by
// slice (all rows of a column slice, then the next slice), the sequence is
// cut into kXcds equal runs, and run x goes to the workgroups x, x + kXcds,
// ..., which the dispatcher places on XCD x (workgroups go to the XCDs in
// turn).  Each XCD then gathers from one or two B slices at a time instead of
// from all of B (11 MB of B rows per XCD at O3 instead of 90 MB).  The grid is
// a multiple of kXcds; where the workgroups land affects speed only.
constexpr int kXcds = 8;

template <int DT, int V>
__global__ __launch_bounds__(256) void spmm_csr_kernel(SpmmArgs a) {
  using S = typename FT<DT>::S;
  constexpr int U = 8;
  const int lane = threadIdx.x & 63;
  const int64_t nch = (a.N + 64 * V - 1) / (64 * V);
  const int64_t nrow = a.nb * a.rows, items = nrow * nch;
  const S* B = (const S*)a.B;
  const int xcd = blockIdx.x % kXcds;
  const int64_t lo = items * xcd / kXcds, hi = items * (xcd + 1) / kXcds;
  const int64_t nwx = (int64_t)(gridDim.x / kXcds) * 4;
  for (int64_t w = lo + (int64_t)(blockIdx.x / kXcds) * 4 + (threadIdx.x >> 6); w < hi; w += nwx) {
    const int64_t ch = w / nrow, g = w - ch * nrow;
    const int64_t n = ch * 64 * V + (int64_t)lane * V;
    const bool nok = n < a.N;
    const int64_t nn = nok ? n : a.N - V;
    {
      const int64_t b = g / a.rows, r = g - b * a.rows;
      const int32_t* ptr = a.indptr + b * (a.rows + 1);
      const int64_t base = ptr[0];
      int64_t p0 = (int64_t)ptr[r] - base, p1 = (int64_t)ptr[r + 1] - base;
      p0 = p0 < 0 ? 0 : (p0 > a.nnz_stride ? a.nnz_stride : p0);
      p1 = p1 < p0 ? p0 : (p1 > a.nnz_stride ? a.nnz_stride : p1);
      if (a.K == 0) p1 = p0;  // no row of B to read
      const S* Bb = B + b * a.b_stride + nn;
      const int32_t* idx = a.indices + b * a.nnz_stride;
      const int64_t dbase = b * a.nnz_stride;
      float acc[V];
#pragma unroll
      for (int j = 0; j < V; ++j) acc[j] = 0.f;
      // The row's entries 64 at a time: lane j loads entry p + j's column and
      // value once, and the B loads of a group of U entries take them from
      // the lanes as scalars, so they issue back to back without waiting on
      // index loads.  The FMAs run in entry order, as before.
      for (int64_t p = p0; p < p1; p += 64) {
        const int cnt = (int)(p1 - p < 64 ? p1 - p : 64);
        const int32_t kl = lane < cnt ? idx[p + lane] : -1;
        const float al = lane < cnt ? load_f(a.data, a.data_dtype, dbase + p + lane) : 0.f;
        int q = 0;
        for (; q + U <= cnt; q += U) {
          Group<S, V> grp[U];
          float av[U];
          bool ok[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int k = __builtin_amdgcn_readlane(kl, q + u);
            ok[u] = (uint32_t)k < (uint64_t)a.K;
            av[u] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, al), q + u));
            grp[u].load(Bb + (ok[u] ? (int64_t)k : 0) * a.N);
          }
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int j = 0; j < V; ++j)
              if (ok[u]) acc[j] = fmaf(av[u], FT<DT>::val(grp[u].get(j)), acc[j]);
        }
        for (; q < cnt; ++q) {
          const int k = __builtin_amdgcn_readlane(kl, q);
          const bool ok = (uint32_t)k < (uint64_t)a.K;
          const float av = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, al), q));
          Group<S, V> grp;
          grp.load(Bb + (ok ? (int64_t)k : 0) * a.N);
#pragma unroll
          for (int j = 0; j < V; ++j)
            if (ok) acc[j] = fmaf(av, FT<DT>::val(grp.get(j)), acc[j]);
        }
      }
      if (nok) {
        uint32_t o[V];
        if (a.addend) {
          Group<S, V> ad;
          ad.load((const S*)a.addend + g * a.N + n);
#pragma unroll
          for (int j = 0; j < V; ++j)
            o[j] = FT<DT>::bits(FT<DT>::val(ad.get(j)) + FT<DT>::val(FT<DT>::bits(acc[j])));
        } else {
#pragma unroll
          for (int j = 0; j < V; ++j) o[j] = FT<DT>::bits(acc[j]);
        }
        // non-temporal: the write-once output does not displace the B
        // slices the XCD's L2 holds (142.5-143.2 against 144.0-146.7 us)
        store_group<S, V, true>((S*)a.out + g * a.N + n, o);
      }
    }
  }
}

template <int DT>
int launch_filter(const void* x, int64_t nb, int64_t rows, int64_t cols, float t, int64_t max_nnz, int32_t offset,
                  void* data, int32_t* indices, int32_t* indptr, void* inlier, hipStream_t st) {
  using S = typename FT<DT>::S;
  constexpr int V = FT<DT>::kVec;
  const int64_t nrows = nb * rows;
  const bool wide = cols % V == 0 && aligned(x, 16) && aligned(inlier, 16);
  // cols == 0 runs the count kernel too: its row loop is empty and it
  // stores zero counts.
  if (nrows > 0) {
    if (wide) {
      hipLaunchKernelGGL((outlier_count_kernel<DT, V>), dim3(grid_for(nrows, 4, 16)), dim3(256), 0, st,
                         (const S*)x, nrows, rows, cols, t, indptr);
    } else {
      hipLaunchKernelGGL((outlier_count_kernel<DT, 1>), dim3(grid_for(nrows, 4, 16)), dim3(256), 0, st,
                         (const S*)x, nrows, rows, cols, t, indptr);
    }
  }
  hipLaunchKernelGGL(csr_scan_kernel, dim3((unsigned)nb), dim3(1024), 0, st, indptr, rows, max_nnz, offset);
  // the split kernel also pads every batch's tail, so it runs when rows == 0
  const unsigned grid = grid_for(nrows > 0 ? nrows : 1, 4, 16);
  if (wide) {
    hipLaunchKernelGGL((outlier_split_kernel<DT, V>), dim3(grid), dim3(256), 0, st, (const S*)x, nb, rows, cols, t,
                       indptr, max_nnz, (S*)inlier, (S*)data, indices);
  } else {
    hipLaunchKernelGGL((outlier_split_kernel<DT, 1>), dim3(grid), dim3(256), 0, st, (const S*)x, nb, rows, cols, t,
                       indptr, max_nnz, (S*)inlier, (S*)data, indices);
  }
  return check_launch("filter_outlier");
}

template <int LPB>
void launch_split_mx(const uint16_t* x, int64_t nb, int64_t rows, int64_t cols, float t, int32_t* indptr,
                     int64_t max_nnz, uint16_t* values, uint16_t* data, int32_t* indices, const MxFuse& mf,
                     hipStream_t st) {
  const int64_t nrows = nb * rows;
  hipLaunchKernelGGL((outlier_split_kernel<kBF16, 8, true, LPB>), dim3(grid_for(nrows > 0 ? nrows : 1, 4, 16)),
                     dim3(256), 0, st, x, nb, rows, cols, t, indptr, max_nnz, values, data, indices, mf);
}

// One-pass workspace: counts [nrows] int32 (256-byte aligned block), then the
// staging columns [nrows][slots] int32 and values [nrows][slots] (x's
// storage type).  The slots per row follow from the bytes given.
size_t stage_counts_bytes(int64_t nrows) { return ((size_t)nrows * 4 + 255) & ~(size_t)255; }

int stage_from_workspace(void* ws, int64_t ws_bytes, int64_t nrows, int64_t cols, int es, Stage* sg,
                         const char* what) {
  *sg = Stage{};
  if (nrows == 0) return kOk;
  const size_t cb = stage_counts_bytes(nrows);
  if (!ws || ws_bytes < 0 || (size_t)ws_bytes < cb)
    return set_error(kErrInvalid, "%s: workspace of %lld bytes, at least %zu needed", what, (long long)ws_bytes, cb);
  if (((uintptr_t)ws & 255) != 0) return set_error(kErrInvalid, "%s: workspace must be 256-byte aligned", what);
  int64_t slots = (int64_t)(((size_t)ws_bytes - cb) / ((size_t)nrows * (size_t)(4 + es)));
  if (slots > cols) slots = cols;
  sg->counts = (int32_t*)ws;
  sg->col = (int32_t*)((char*)ws + cb);
  sg->val = (char*)ws + cb + (size_t)nrows * (size_t)slots * 4;
  sg->slots = slots;
  return kOk;
}

template <int DT>
int launch_finalize(const void* x, bool wide, int64_t nb, int64_t rows, int64_t cols, float t, const Stage& sg,
                    int64_t max_nnz, int32_t offset, void* data, int32_t* indices, int32_t* indptr, hipStream_t st) {
  using S = typename FT<DT>::S;
  constexpr int V = FT<DT>::kVec;
  // about 256 workgroups per batch: chunks of 16 to 256 rows
  const int64_t chunk = std::min<int64_t>(256, std::max<int64_t>(16, (rows + 255) / 256));
  const int64_t nchunk = rows > 0 ? (rows + chunk - 1) / chunk : 1;
  if (nb * nchunk > INT32_MAX) return set_error(kErrInvalid, "filter_outlier: too many row chunks");
  const dim3 grid((unsigned)(nb * nchunk));
  if (wide)
    hipLaunchKernelGGL((outlier_finalize_kernel<DT, V>), grid, dim3(256), 0, st, (const S*)x, rows, cols, t, sg,
                       chunk, nchunk, max_nnz, offset, (S*)data, indices, indptr);
  else
    hipLaunchKernelGGL((outlier_finalize_kernel<DT, 1>), grid, dim3(256), 0, st, (const S*)x, rows, cols, t, sg,
                       chunk, nchunk, max_nnz, offset, (S*)data, indices, indptr);
  return kOk;
}

template <int DT>
int launch_filter_ws(const void* x, int64_t nb, int64_t rows, int64_t cols, float t, int64_t max_nnz, int32_t offset,
                     void* data, int32_t* indices, int32_t* indptr, void* inlier, const Stage& sg, hipStream_t st) {
  using S = typename FT<DT>::S;
  constexpr int V = FT<DT>::kVec;
  const int64_t nrows = nb * rows;
  const bool wide = cols % V == 0 && aligned(x, 16) && aligned(inlier, 16);
  if (nrows > 0) {
    const unsigned grid = grid_for(nrows, 4, 16);
    if (wide)
      hipLaunchKernelGGL((outlier_split_kernel<DT, V, false, 1, true>), dim3(grid), dim3(256), 0, st, (const S*)x,
                         nb, rows, cols, t, nullptr, max_nnz, (S*)inlier, nullptr, nullptr, MxFuse{}, sg);
    else
      hipLaunchKernelGGL((outlier_split_kernel<DT, 1, false, 1, true>), dim3(grid), dim3(256), 0, st, (const S*)x,
                         nb, rows, cols, t, nullptr, max_nnz, (S*)inlier, nullptr, nullptr, MxFuse{}, sg);
  }
  const int rc = launch_finalize<DT>(x, wide, nb, rows, cols, t, sg, max_nnz, offset, data, indices, indptr, st);
  if (rc != kOk) return rc;
  return check_launch("filter_outlier");
}

template <int LPB>
void launch_split_mx_stage(const uint16_t* x, int64_t nb, int64_t rows, int64_t cols, float t, uint16_t* values,
                           const MxFuse& mf, const Stage& sg, hipStream_t st) {
  hipLaunchKernelGGL((outlier_split_kernel<kBF16, 8, true, LPB, true>), dim3(grid_for(nb * rows, 4, 16)),
                     dim3(256), 0, st, x, nb, rows, cols, t, nullptr, (int64_t)0, values, nullptr, nullptr, mf, sg);
}

template <int DT>
int launch_spmm(const SpmmArgs& a, hipStream_t st) {
  constexpr int V = FT<DT>::kVec;
  const bool wide = a.N % V == 0 && aligned(a.B, 16) && aligned(a.out, 16) && (a.b_stride % V == 0) &&
                    (!a.addend || aligned(a.addend, 16));
  const int v = wide ? V : 1;
  const int64_t items = a.nb * a.rows * ((a.N + 64 * v - 1) / (64 * v));
  // resident workgroups only (the slice order relies on them running
  // together), a multiple of kXcds, no more than the items need
  auto grid_of = [&](const void* k) {
    const int64_t need = ((items + 3) / 4 + kXcds - 1) / kXcds * kXcds;
    const int64_t res = (int64_t)persistent_grid(k, 256, 0, items * 64) / kXcds * kXcds;
    return (unsigned)std::max<int64_t>(kXcds, std::min(need, res));
  };
  if (wide)
    hipLaunchKernelGGL((spmm_csr_kernel<DT, V>), dim3(grid_of((const void*)spmm_csr_kernel<DT, V>)), dim3(256), 0,
                       st, a);
  else
    hipLaunchKernelGGL((spmm_csr_kernel<DT, 1>), dim3(grid_of((const void*)spmm_csr_kernel<DT, 1>)), dim3(256), 0,
                       st, a);
  return check_launch("spmm_csr");
}

}  // namespace

int filter_outlier(const void* x, int dtype, int64_t nb, int64_t rows, int64_t cols, float threshold,
                   int64_t max_nnz, int32_t indptr_offset, void* data, int32_t* indices, int32_t* indptr,
                   void* inlier, hipStream_t st) {
  if (nb < 0 || rows < 0 || cols < 0 || max_nnz < 0) return set_error(kErrInvalid, "filter_outlier: negative size");
  if (nb == 0) return kOk;
  if (!indptr || (max_nnz > 0 && (!data || !indices)) || (rows * cols > 0 && (!x || !inlier)))
    return set_error(kErrInvalid, "filter_outlier: null buffer");
  if (max_nnz > INT32_MAX || rows >= INT32_MAX || cols > INT32_MAX)
    return set_error(kErrInvalid, "filter_outlier: sizes beyond int32 indices");
  switch (dtype) {
    case kF32: return launch_filter<kF32>(x, nb, rows, cols, threshold, max_nnz, indptr_offset, data, indices, indptr, inlier, st);
    case kBF16: return launch_filter<kBF16>(x, nb, rows, cols, threshold, max_nnz, indptr_offset, data, indices, indptr, inlier, st);
    case kF16: return launch_filter<kF16>(x, nb, rows, cols, threshold, max_nnz, indptr_offset, data, indices, indptr, inlier, st);
    default: return set_error(kErrInvalid, "filter_outlier: dtype %d not supported (fp32, bf16, fp16)", dtype);
  }
}

int quantize_mx_outlier_fused(const void* x, int64_t nb, int64_t rows, int64_t cols, float threshold,
                              int64_t max_nnz, int32_t indptr_offset, int64_t block_size, const ScaleParams& sp,
                              const uint16_t* qmap, void* data, int32_t* indices, int32_t* indptr, void* scale,
                              void* values, hipStream_t st) {
  if (nb < 0 || rows < 0 || cols < 0 || max_nnz < 0)
    return set_error(kErrInvalid, "quantize_mx_outlier: negative size");
  if (block_size != 8 && block_size != 16 && block_size != 32 && block_size != 64)
    return set_error(kErrUnsupported, "quantize_mx_outlier: fused form takes blocks of 8, 16, 32 or 64");
  if (cols % block_size) return set_error(kErrUnsupported, "quantize_mx_outlier: cols must be whole blocks");
  if (nb == 0) return kOk;
  if (!indptr || !qmap || (max_nnz > 0 && (!data || !indices)) ||
      (rows * cols > 0 && (!x || !values || !scale)))
    return set_error(kErrInvalid, "quantize_mx_outlier: null buffer");
  if (max_nnz > INT32_MAX || rows >= INT32_MAX || cols > INT32_MAX)
    return set_error(kErrInvalid, "quantize_mx_outlier: sizes beyond int32 indices");
  if (!aligned(x, 16) || !aligned(values, 16))
    return set_error(kErrInvalid, "quantize_mx_outlier: input and values must be 16-byte aligned");
  const int64_t nrows = nb * rows;
  const uint16_t* xs = (const uint16_t*)x;
  if (nrows > 0)
    hipLaunchKernelGGL((outlier_count_kernel<kBF16, 8>), dim3(grid_for(nrows, 4, 16)), dim3(256), 0, st, xs, nrows,
                       rows, cols, threshold, indptr);
  hipLaunchKernelGGL(csr_scan_kernel, dim3((unsigned)nb), dim3(1024), 0, st, indptr, rows, max_nnz, indptr_offset);
  MxFuse mf{sp, qmap, (uint16_t*)scale};
  uint16_t* v = (uint16_t*)values;
  uint16_t* d = (uint16_t*)data;
  switch (block_size) {
    case 8: launch_split_mx<1>(xs, nb, rows, cols, threshold, indptr, max_nnz, v, d, indices, mf, st); break;
    case 16: launch_split_mx<2>(xs, nb, rows, cols, threshold, indptr, max_nnz, v, d, indices, mf, st); break;
    case 32: launch_split_mx<4>(xs, nb, rows, cols, threshold, indptr, max_nnz, v, d, indices, mf, st); break;
    default: launch_split_mx<8>(xs, nb, rows, cols, threshold, indptr, max_nnz, v, d, indices, mf, st); break;
  }
  return check_launch("quantize_mx_outlier");
}

// The one-pass finalize sums, in each of its (about 256) workgroups, the
// counts of every row of the batch before its chunk, so its reads grow as
// rows^2 / chunk; past this many rows per matrix the _ws entry points take
// the two-pass form (count, one scan per batch, split), whose reads are
// linear in rows.
constexpr int64_t kOnePassMaxRows = 16384;

int64_t outlier_stage_slots(int64_t rows, int64_t cols, int64_t max_nnz) {
  if (max_nnz <= 0 || rows <= 0 || cols <= 0) return 0;
  const int64_t per = (max_nnz + rows - 1) / rows;
  int64_t s = (2 * per + 63) / 64 * 64;
  s = s < 64 ? 64 : (s > 1024 ? 1024 : s);
  return s < cols ? s : cols;
}

int outlier_workspace_size(int dtype, int64_t nb, int64_t rows, int64_t cols, int64_t max_nnz, int64_t* bytes) {
  if (!bytes) return set_error(kErrInvalid, "outlier_workspace_size: null result pointer");
  if (nb < 0 || rows < 0 || cols < 0 || max_nnz < 0)
    return set_error(kErrInvalid, "outlier_workspace_size: negative size");
  int es;
  switch (dtype) {
    case kF32: es = 4; break;
    case kBF16:
    case kF16: es = 2; break;
    default: return set_error(kErrInvalid, "outlier_workspace_size: dtype %d not supported (fp32, bf16, fp16)", dtype);
  }
  const int64_t nrows = nb * rows;
  *bytes = nrows == 0 || rows > kOnePassMaxRows ? 0
                      : (int64_t)(stage_counts_bytes(nrows) +
                                  (size_t)nrows * (size_t)outlier_stage_slots(rows, cols, max_nnz) * (size_t)(4 + es));
  return kOk;
}

int filter_outlier_ws(const void* x, int dtype, int64_t nb, int64_t rows, int64_t cols, float threshold,
                      int64_t max_nnz, int32_t indptr_offset, void* data, int32_t* indices, int32_t* indptr,
                      void* inlier, void* workspace, int64_t workspace_bytes, hipStream_t st) {
  if (nb < 0 || rows < 0 || cols < 0 || max_nnz < 0) return set_error(kErrInvalid, "filter_outlier: negative size");
  if (nb == 0) return kOk;
  if (!indptr || (max_nnz > 0 && (!data || !indices)) || (rows * cols > 0 && (!x || !inlier)))
    return set_error(kErrInvalid, "filter_outlier: null buffer");
  if (max_nnz > INT32_MAX || rows >= INT32_MAX || cols > INT32_MAX)
    return set_error(kErrInvalid, "filter_outlier: sizes beyond int32 indices");
  const int es = dtype == kF32 ? 4 : 2;
  if (dtype != kF32 && dtype != kBF16 && dtype != kF16)
    return set_error(kErrInvalid, "filter_outlier: dtype %d not supported (fp32, bf16, fp16)", dtype);
  if (rows > kOnePassMaxRows)
    return filter_outlier(x, dtype, nb, rows, cols, threshold, max_nnz, indptr_offset, data, indices, indptr, inlier,
                          st);
  Stage sg;
  if (stage_from_workspace(workspace, workspace_bytes, nb * rows, cols, es, &sg, "filter_outlier") != kOk)
    return kErrInvalid;
  switch (dtype) {
    case kF32: return launch_filter_ws<kF32>(x, nb, rows, cols, threshold, max_nnz, indptr_offset, data, indices, indptr, inlier, sg, st);
    case kBF16: return launch_filter_ws<kBF16>(x, nb, rows, cols, threshold, max_nnz, indptr_offset, data, indices, indptr, inlier, sg, st);
    default: return launch_filter_ws<kF16>(x, nb, rows, cols, threshold, max_nnz, indptr_offset, data, indices, indptr, inlier, sg, st);
  }
}

int quantize_mx_outlier_fused_ws(const void* x, int64_t nb, int64_t rows, int64_t cols, float threshold,
                                 int64_t max_nnz, int32_t indptr_offset, int64_t block_size, const ScaleParams& sp,
                                 const uint16_t* qmap, void* data, int32_t* indices, int32_t* indptr, void* scale,
                                 void* values, void* workspace, int64_t workspace_bytes, hipStream_t st) {
  if (nb < 0 || rows < 0 || cols < 0 || max_nnz < 0)
    return set_error(kErrInvalid, "quantize_mx_outlier: negative size");
  if (block_size != 8 && block_size != 16 && block_size != 32 && block_size != 64)
    return set_error(kErrUnsupported, "quantize_mx_outlier: fused form takes blocks of 8, 16, 32 or 64");
  if (cols % block_size) return set_error(kErrUnsupported, "quantize_mx_outlier: cols must be whole blocks");
  if (nb == 0) return kOk;
  if (!indptr || !qmap || (max_nnz > 0 && (!data || !indices)) ||
      (rows * cols > 0 && (!x || !values || !scale)))
    return set_error(kErrInvalid, "quantize_mx_outlier: null buffer");
  if (max_nnz > INT32_MAX || rows >= INT32_MAX || cols > INT32_MAX)
    return set_error(kErrInvalid, "quantize_mx_outlier: sizes beyond int32 indices");
  if (!aligned(x, 16) || !aligned(values, 16))
    return set_error(kErrInvalid, "quantize_mx_outlier: input and values must be 16-byte aligned");
  if (rows > kOnePassMaxRows)
    return quantize_mx_outlier_fused(x, nb, rows, cols, threshold, max_nnz, indptr_offset, block_size, sp, qmap, data,
                                     indices, indptr, scale, values, st);
  Stage sg;
  if (stage_from_workspace(workspace, workspace_bytes, nb * rows, cols, 2, &sg, "quantize_mx_outlier") != kOk)
    return kErrInvalid;
  const uint16_t* xs = (const uint16_t*)x;
  if (nb * rows > 0) {
    MxFuse mf{sp, qmap, (uint16_t*)scale};
    uint16_t* v = (uint16_t*)values;
    switch (block_size) {
      case 8: launch_split_mx_stage<1>(xs, nb, rows, cols, threshold, v, mf, sg, st); break;
      case 16: launch_split_mx_stage<2>(xs, nb, rows, cols, threshold, v, mf, sg, st); break;
      case 32: launch_split_mx_stage<4>(xs, nb, rows, cols, threshold, v, mf, sg, st); break;
      default: launch_split_mx_stage<8>(xs, nb, rows, cols, threshold, v, mf, sg, st); break;
    }
  }
  const int rc = launch_finalize<kBF16>(x, true, nb, rows, cols, threshold, sg, max_nnz, indptr_offset, data, indices,
                                        indptr, st);
  if (rc != kOk) return rc;
  return check_launch("quantize_mx_outlier");
}

int csr_slice(const void* data, int dtype, const int32_t* indices, const int32_t* indptr, int64_t nnz_in,
              int64_t rows, int dim, int64_t start, int64_t end, int64_t max_nnz, void* data_out,
              int32_t* indices_out, int32_t* indptr_out, hipStream_t st) {
  if (rows < 0 || nnz_in < 0 || max_nnz < 0) return set_error(kErrInvalid, "slice_csr_tensor: negative size");
  if (max_nnz > INT32_MAX) return set_error(kErrInvalid, "slice_csr_tensor: capacity beyond int32 indices");
  if (!indptr || !indptr_out || (max_nnz > 0 && (!data_out || !indices_out)) || (nnz_in > 0 && (!data || !indices)))
    return set_error(kErrInvalid, "slice_csr_tensor: null buffer");
  const bool wide16 = dtype == kBF16 || dtype == kF16;
  if (!wide16 && dtype != kF32)
    return set_error(kErrInvalid, "slice_csr_tensor: dtype %d not supported (fp32, bf16, fp16)", dtype);
  if (dim == 0) {
    if (start < 0 || end < start || end > rows)
      return set_error(kErrInvalid, "slice_csr_tensor: rows [%lld, %lld] outside [0, %lld]", (long long)start,
                       (long long)end, (long long)rows);
    const int64_t nrows_out = end - start;
    const int64_t n = max_nnz > nrows_out + 1 ? max_nnz : nrows_out + 1;
    if (wide16)
      hipLaunchKernelGGL(csr_slice_rows_kernel<uint16_t>, dim3(grid_for(n, 256)), dim3(256), 0, st,
                         (const uint16_t*)data, indices, indptr, nnz_in, start, nrows_out, max_nnz,
                         (uint16_t*)data_out, indices_out, indptr_out);
    else
      hipLaunchKernelGGL(csr_slice_rows_kernel<uint32_t>, dim3(grid_for(n, 256)), dim3(256), 0, st,
                         (const uint32_t*)data, indices, indptr, nnz_in, start, nrows_out, max_nnz,
                         (uint32_t*)data_out, indices_out, indptr_out);
    return check_launch("slice_csr_tensor");
  }
  if (dim != 1) return set_error(kErrInvalid, "slice_csr_tensor: cannot slice along dim %d", dim);
  if (start < 0) return set_error(kErrInvalid, "slice_csr_tensor: column start must be >= 0");
  if (rows > 0)
    hipLaunchKernelGGL(csr_cols_count_kernel, dim3(grid_for(rows, 4, 16)), dim3(256), 0, st, indices, indptr, rows,
                       nnz_in, start, end, indptr_out);
  hipLaunchKernelGGL(csr_scan_kernel, dim3(1), dim3(1024), 0, st, indptr_out, rows, max_nnz, 0);
  // the scatter kernel also pads the tail, so it runs when rows == 0
  const unsigned grid = grid_for(rows > 0 ? rows : 1, 4, 16);
  if (wide16)
    hipLaunchKernelGGL(csr_cols_scatter_kernel<uint16_t>, dim3(grid), dim3(256), 0, st, (const uint16_t*)data,
                       indices, indptr, rows, nnz_in, start, end, max_nnz, indptr_out, (uint16_t*)data_out,
                       indices_out);
  else
    hipLaunchKernelGGL(csr_cols_scatter_kernel<uint32_t>, dim3(grid), dim3(256), 0, st, (const uint32_t*)data,
                       indices, indptr, rows, nnz_in, start, end, max_nnz, indptr_out, (uint32_t*)data_out,
                       indices_out);
  return check_launch("slice_csr_tensor");
}

int csr_decode(const CsrDecode& d, hipStream_t st) {
  if (d.nb < 0 || d.br < 0 || d.bc < 0) return set_error(kErrInvalid, "csr_decode: negative size");
  const int64_t n = d.nb * d.br * d.bc;
  if (n == 0) return kOk;
  if (!d.B || !d.out) return set_error(kErrInvalid, "csr_decode: null buffer");
  if (d.b_dtype < kF32 || d.b_dtype > kU8) return set_error(kErrInvalid, "csr_decode: B dtype %d", d.b_dtype);
  if (d.out_dtype < kF32 || d.out_dtype > kF16) return set_error(kErrInvalid, "csr_decode: out dtype %d", d.out_dtype);
  if (d.code && (d.code_len < 1 || d.code_dtype < kF32 || d.code_dtype > kF16))
    return set_error(kErrInvalid, "csr_decode: bad code table");
  if (d.scale && (d.scale_dtype < kF32 || d.scale_dtype > kF16 || d.rdiv < 1 || d.cdiv < 1 || d.sr < 1 || d.sc < 1 ||
                  (d.br - 1) / d.rdiv >= d.sr || (d.bc - 1) / d.cdiv >= d.sc))
    return set_error(kErrInvalid, "csr_decode: scale does not cover B");
  const int64_t tiles = d.nb * ((d.br + 63) / 64) * ((d.bc + 63) / 64);
  hipLaunchKernelGGL(csr_decode_kernel, dim3(grid_for(tiles, 1, 8)), dim3(256), 0, st, d);
  return check_launch("csr_decode");
}

int spmm_csr(const SpmmArgs& a, hipStream_t st) {
  if (a.nb < 0 || a.rows < 0 || a.K < 0 || a.N < 0 || a.nnz_stride < 0 || a.b_stride < 0)
    return set_error(kErrInvalid, "spmm_csr: negative size");
  if (a.nb * a.rows * a.N == 0) return kOk;
  if (!a.indptr || !a.B || !a.out || (a.nnz_stride > 0 && (!a.data || !a.indices)))
    return set_error(kErrInvalid, "spmm_csr: null buffer");
  if (a.data_dtype < kF32 || a.data_dtype > kF16) return set_error(kErrInvalid, "spmm_csr: data dtype %d", a.data_dtype);
  switch (a.b_dtype) {
    case kF32: return launch_spmm<kF32>(a, st);
    case kBF16: return launch_spmm<kBF16>(a, st);
    case kF16: return launch_spmm<kF16>(a, st);
    default: return set_error(kErrInvalid, "spmm_csr: B dtype %d not supported (fp32, bf16, fp16)", a.b_dtype);
  }
}

}  // namespace vqx
