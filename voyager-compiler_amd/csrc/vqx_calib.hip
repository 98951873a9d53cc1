// LCQ calibration statistics: the weighted per-bin moments that the learned
// codebook solver reads (src/voyager_compiler/quantization/lcq.py:44-119
// Histogram.add, with unit_scale :136-150 as _accumulate :603-626 applies it).
//
// Per element v -- x itself, or x / blockscale with blockscale =
// max(amax |block|, 1e-12) / quant_max in fp32 and IEEE division -- the bin
// is the number of edges <= v, minus one, clamped to [0, bins - 1]
// (torch.bucketize(right=True); NaN counts every edge), and
//   weight[bin] += w,  total[bin] += w v,  square[bin] += (w v) v
// in fp64 (w v is exact in fp64; the second product rounds as torch's does).
// Only the order of the fp64 additions differs from the reference's
// index_add_.
//
// Each workgroup keeps the three histograms in LDS (fp64 LDS atomics) with
// the fp32 edges beside them, works through a grid-stride share of the
// elements (four per lane per load, a block's amax a butterfly over its
// lanes; odd block sizes one thread per block), then adds its histograms to
// the global sums with fp64 atomics.  The bin of v starts from
// the arithmetic guess of a uniform grid and is corrected against the actual
// edges, so it is exact whatever rounding the edges carry.
#include <type_traits>

#include "vqx_common.h"
#include "vqx_kernels.h"

namespace vqx {
namespace {

constexpr int kHistThreads = 1024;

template <int DT>
__device__ __forceinline__ float load_elem(const void* x, int64_t i) {
  if constexpr (DT == kF32) return ((const float*)x)[i];
  else if constexpr (DT == kBF16) return bf2f(((const uint16_t*)x)[i]);
  else return h2f_exact(((const uint16_t*)x)[i]);
}

struct HistLds {
  double* w;
  double* t;
  double* s;
  const float* e;  // bins + 1 edges
};

// The bin guess on the uniform grid [e0, e0 + bins * step]: the number of
// edges <= v if the edges were exactly uniform.  Monotone in v.
__device__ __forceinline__ int grid_guess(float v, float e0, float inv_step, int bins) {
  // fmaxf / fminf also send a NaN guess (degenerate edges) into [1, bins]
  return (int)fminf(fmaxf(__builtin_floorf((v - e0) * inv_step) + 1.0f, 1.0f), (float)bins);
}

// Number of edges <= v (0 .. bins + 1).  With `tight` (every edge checked
// at set-up: grid_guess(e[j]) >= j and grid_guess(just below e[j]) <= j + 1)
// the guess is within one of the answer for every v between e[0] and
// e[bins] (the guess is monotone), so one look at the two edges around it
// settles the count; otherwise the guess is walked to the answer.
__device__ __forceinline__ int edges_at_or_below(float v, const float* e, int bins, float e0, float elast,
                                                 float inv_step, bool tight) {
  if (!(v == v)) return bins + 1;  // NaN: bucketize places it past every edge
  if (v >= elast) return bins + 1;
  if (v < e0) return 0;
  // e[0] <= v < e[bins]: the answer lies in [1, bins]
  int g = grid_guess(v, e0, inv_step, bins);
  if (tight) {
    const float lo = e[g - 1], hi = e[g < bins ? g : bins];
    return g - (lo > v ? 1 : 0) + (g < bins && hi <= v ? 1 : 0);
  }
  while (g > 1 && !(e[g - 1] <= v)) --g;
  while (g < bins && e[g] <= v) ++g;
  return g;
}

__device__ __forceinline__ void hist_add(const HistLds& h, int bins, float e0, float elast, float inv_step, bool tight,
                                         float v, float w) {
  int c = edges_at_or_below(v, h.e, bins, e0, elast, inv_step, tight) - 1;
  c = c < 0 ? 0 : (c > bins - 1 ? bins - 1 : c);
  const double vd = (double)v, wd = (double)w;
  const double wv = wd * vd;
  atomicAdd(&h.w[c], wd);
  atomicAdd(&h.t[c], wv);
  atomicAdd(&h.s[c], wv * vd);
}

// The bin of v when the guess is tight, without branches: the count from the
// two edges around the guess, then NaN and v >= e[bins] to the last bin and
// v < e[0] to the first (bucketize's count, minus one, clamped).
__device__ __forceinline__ int bin_tight(float v, const float* e, int bins, float e0, float elast, float inv_step) {
  const int g = grid_guess(v, e0, inv_step, bins);  // in [1, bins] for every v
  const float lo = e[g - 1], hi = e[g];
  const int c = g - (lo > v ? 1 : 0) + (g < bins && hi <= v ? 1 : 0);
  return (!(v == v) || v >= elast) ? bins - 1 : (v < e0 ? 0 : c - 1);
}

// Adds of one element, the products in fp64 as the reference forms them
// (w v is exact; w = 1 gives v and v v exactly).
__device__ __forceinline__ void add_moments(const HistLds& h, int c, float v, float w) {
  const double vd = (double)v, wd = (double)w;
  const double wv = wd * vd;
  atomicAdd(&h.w[c], wd);
  atomicAdd(&h.t[c], wv);
  atomicAdd(&h.s[c], wv * vd);
}

// max over a segment of lanes (xor butterfly over `span` lanes), NaN winning
__device__ __forceinline__ float seg_max_nan(float a, int span) {
  for (int o = 1; o < span; o <<= 1) {
    const float b = __shfl_xor(a, o, 64);
    a = (!(a == a) || !(b == b)) ? __builtin_nanf("") : (b > a ? b : a);
  }
  return a;
}

// Four consecutive elements as fp32 (one 16-byte or 8-byte load).
template <int DT>
__device__ __forceinline__ void load4(const void* x, int64_t i, float (&v)[4]) {
  if constexpr (DT == kF32) {
    const f32x4 q = *(const f32x4*)((const float*)x + i);
    v[0] = q[0], v[1] = q[1], v[2] = q[2], v[3] = q[3];
  } else {
    const u32x2 q = *(const u32x2*)((const uint16_t*)x + i);
    const uint32_t h[4] = {q[0] & 0xFFFFu, q[0] >> 16, q[1] & 0xFFFFu, q[1] >> 16};
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = DT == kBF16 ? bf2f(h[j]) : h2f_exact(h[j]);
  }
}

// VEC: n % 4 == 0 and block_size is 0 or a power of two in [4, 256].  Each
// lane takes four consecutive elements (one load), so a wave covers 256
// elements and a block is block_size / 4 consecutive lanes, whose amax is a
// butterfly over those lanes.  Otherwise one thread per block (or element).
template <int DT, bool VEC, bool W>
__global__ __launch_bounds__(kHistThreads) void lcq_hist_kernel(const void* __restrict__ x, int64_t n, int64_t bs,
                                                                float quant_max, const float* __restrict__ wts,
                                                                int64_t wper, const float* __restrict__ edges,
                                                                int bins, double* __restrict__ gw,
                                                                double* __restrict__ gt, double* __restrict__ gs) {
  __shared__ double s_w[kHistMaxBins], s_t[kHistMaxBins], s_s[kHistMaxBins];
  __shared__ float s_e[kHistMaxBins + 1];
  __shared__ int s_loose;
  if (threadIdx.x == 0) s_loose = 0;
  for (int j = threadIdx.x; j < bins; j += kHistThreads) s_w[j] = s_t[j] = s_s[j] = 0.0;
  for (int j = threadIdx.x; j <= bins; j += kHistThreads) s_e[j] = edges[j];
  __syncthreads();
  const float e0 = s_e[0], elast = s_e[bins];
  const float inv_step = (float)bins / (elast - e0);
  {
    // can the guess be trusted to within one?  (edges ascending, and the
    // guess at and just below every edge within one of its count)
    bool loose = false;
    for (int j = threadIdx.x; j <= bins; j += kHistThreads) {
      const float ej = s_e[j];
      // the float just below ej (finite ej)
      const uint32_t eb = f2u(ej);
      const float below = (eb & 0x7FFFFFFFu) == 0 ? u2f(0x80000001u) : u2f((eb >> 31) ? eb + 1u : eb - 1u);
      loose |= !(ej == ej) || (j > 0 && !(s_e[j - 1] < ej));
      if (j >= 1 && j <= bins - 1) {
        loose |= grid_guess(ej, e0, inv_step, bins) < j;
        loose |= grid_guess(below, e0, inv_step, bins) > j + 1;
      }
    }
    if (loose) s_loose = 1;
  }
  __syncthreads();
  const bool tight = s_loose == 0;
  const HistLds h{s_w, s_t, s_s, s_e};
  // the vectorised unit-weight path counts in the first half of s_w's bytes
  uint32_t* const s_n = reinterpret_cast<uint32_t*>(s_w);
  constexpr bool kCounts = VEC && !W;
  const float eps = 1e-12f;
  if constexpr (VEC) {
    constexpr int U = 4;  // groups of 256 elements per wave in flight
    const int lane = threadIdx.x & 63;
    const int span = bs > 0 ? (int)(bs / 4) : 1;
    const int64_t groups = (n + 255) / 256;
    const int64_t wv = (int64_t)blockIdx.x * (kHistThreads / 64) + (threadIdx.x >> 6);
    const int64_t nw = (int64_t)gridDim.x * (kHistThreads / 64);
    const uint32_t per = (uint32_t)wper;
    // the element loop, compiled once per kind of bin search (the choice is
    // uniform, so it is made outside the loop)
    auto run = [&](auto tight_c) {
      constexpr bool T = decltype(tight_c)::value;
      for (int64_t g0 = wv * U; g0 < groups; g0 += nw * U) {
        float v[U][4];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t i = (g0 + u) * 256 + lane * 4;
          ok[u] = g0 + u < groups && i < n;
          load4<DT>(x, ok[u] ? i : 0, v[u]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (bs > 0) {
            float a = 0.0f;
            bool nan = false;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float m = fabsf(v[u][j]);
              nan |= !(m == m);
              a = m > a ? m : a;
            }
            // blocks lie wholly inside or wholly outside n, so lanes past n
            // only meet each other in the butterfly
            a = seg_max_nan(nan ? __builtin_nanf("") : a, span);
            // torch's amax propagates NaN; clamp_min keeps it
            const float scale = ((a == a) ? (a > eps ? a : eps) : a) / quant_max;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[u][j] = v[u][j] / scale;
          }
          // lanes past n add v = 0 with weight 0, which changes no sum
          float w[4] = {1.0f, 1.0f, 1.0f, 1.0f};
          if constexpr (W) {
            // weight of element i: wts[i % period], from the group's start
            // (wave-uniform) plus the lane's offset below 256
            const uint32_t base = (uint32_t)(((g0 + u) * 256) % wper);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint32_t k = base + (uint32_t)(lane * 4 + j);
              w[j] = wts[per >= 256u ? (k >= per ? k - per : k) : k % per];
            }
          }
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float vj = ok[u] ? v[u][j] : 0.0f;
            const int c = T ? bin_tight(vj, s_e, bins, e0, elast, inv_step)
                            : min(max(edges_at_or_below(vj, s_e, bins, e0, elast, inv_step, false) - 1, 0), bins - 1);
            if constexpr (W) {
              add_moments(h, c, vj, ok[u] ? w[j] : 0.0f);
            } else if (ok[u]) {
              // unit weights: the weight sum is a count (exact in fp64 at
              // the flush), one 32-bit LDS atomic instead of an fp64 one
              const double vd = (double)vj;
              atomicAdd(&s_n[c], 1u);
              atomicAdd(&h.t[c], vd);
              atomicAdd(&h.s[c], vd * vd);
            }
          }
        }
      }
    };
    if (tight)
      run(std::integral_constant<bool, true>());
    else
      run(std::integral_constant<bool, false>());
  } else {
    const int64_t tid = (int64_t)blockIdx.x * kHistThreads + threadIdx.x, nt = (int64_t)gridDim.x * kHistThreads;
    if (bs == 0) {
      for (int64_t i = tid; i < n; i += nt)
        hist_add(h, bins, e0, elast, inv_step, tight, load_elem<DT>(x, i), wts ? wts[i % wper] : 1.0f);
    } else {
      for (int64_t b = tid; b < n / bs; b += nt) {
        const int64_t i0 = b * bs;
        float amax = 0.0f;
        bool nan = false;
        for (int64_t i = i0; i < i0 + bs; ++i) {
          const float a = fabsf(load_elem<DT>(x, i));
          nan |= !(a == a);
          amax = a > amax ? a : amax;
        }
        const float scale = (nan ? __builtin_nanf("") : (amax > eps ? amax : eps)) / quant_max;
        for (int64_t i = i0; i < i0 + bs; ++i)
          hist_add(h, bins, e0, elast, inv_step, tight, load_elem<DT>(x, i) / scale, wts ? wts[i % wper] : 1.0f);
      }
    }
  }
  __syncthreads();
  // every workgroup starts its flush at a different bin, so that workgroups
  // finishing together do not queue on the same addresses
  const int rot = (int)(((int64_t)blockIdx.x * 521) % bins);
  for (int jj = threadIdx.x; jj < bins; jj += kHistThreads) {
    const int j = jj + rot < bins ? jj + rot : jj + rot - bins;
    const double a = kCounts ? (double)s_n[j] : s_w[j], t = s_t[j], q = s_s[j];
    if (a != 0.0 || t != 0.0 || q != 0.0) {
      atomicAdd(gw + j, a);
      atomicAdd(gt + j, t);
      atomicAdd(gs + j, q);
    }
  }
}

template <int DT, bool VEC>
void launch_hist_w(unsigned grid, const void* x, int64_t n, int64_t bs, float quant_max, const float* w, int64_t wper,
                   const float* edges, int bins, double* gw, double* gt, double* gs, hipStream_t st) {
  if (w)
    hipLaunchKernelGGL((lcq_hist_kernel<DT, VEC, true>), dim3(grid), dim3(kHistThreads), 0, st, x, n, bs, quant_max, w,
                       wper, edges, bins, gw, gt, gs);
  else
    hipLaunchKernelGGL((lcq_hist_kernel<DT, VEC, false>), dim3(grid), dim3(kHistThreads), 0, st, x, n, bs, quant_max,
                       w, wper, edges, bins, gw, gt, gs);
}

template <int DT>
int launch_hist(const void* x, int64_t n, int64_t bs, float quant_max, const float* w, int64_t wper,
                const float* edges, int bins, double* gw, double* gt, double* gs, hipStream_t st) {
  const bool vec = n % 4 == 0 && (bs == 0 || (bs >= 4 && bs <= 256 && (bs & (bs - 1)) == 0)) &&
                   aligned(x, DT == kF32 ? 16 : 8);
  if (vec)
    launch_hist_w<DT, true>(grid_for((n + 255) / 256 * 64, kHistThreads * 4, 1), x, n, bs, quant_max, w, wper, edges,
                            bins, gw, gt, gs, st);
  else
    launch_hist_w<DT, false>(grid_for(bs > 0 ? n / bs : n, kHistThreads, 1), x, n, bs, quant_max, w, wper, edges,
                             bins, gw, gt, gs, st);
  return check_launch("lcq_histogram");
}

}  // namespace

int lcq_histogram(const void* x, int dtype, int64_t n, int64_t block_size, float quant_max, const float* weights,
                  int64_t weights_period, const float* edges, int bins, double* weight, double* total,
                  double* square, hipStream_t st) {
  if (n < 0 || block_size < 0) return set_error(kErrInvalid, "lcq_histogram: negative size");
  if (bins < 1 || bins > kHistMaxBins)
    return set_error(kErrInvalid, "lcq_histogram: bins must be in [1, %d] (got %d)", kHistMaxBins, bins);
  if (block_size > 0 && n % block_size != 0)
    return set_error(kErrInvalid, "lcq_histogram: %lld elements do not split into blocks of %lld", (long long)n,
                     (long long)block_size);
  if (weights && (weights_period < 1 || weights_period > INT32_MAX))
    return set_error(kErrInvalid, "lcq_histogram: weights_period must be in [1, 2^31)");
  if (!edges || !weight || !total || !square) return set_error(kErrInvalid, "lcq_histogram: null buffer");
  if (n == 0) return kOk;
  if (!x) return set_error(kErrInvalid, "lcq_histogram: null input");
  switch (dtype) {
    case kF32: return launch_hist<kF32>(x, n, block_size, quant_max, weights, weights_period, edges, bins, weight, total, square, st);
    case kBF16: return launch_hist<kBF16>(x, n, block_size, quant_max, weights, weights_period, edges, bins, weight, total, square, st);
    case kF16: return launch_hist<kF16>(x, n, block_size, quant_max, weights, weights_period, edges, bins, weight, total, square, st);
    default: return set_error(kErrInvalid, "lcq_histogram: dtype %d not supported (fp32, bf16, fp16)", dtype);
  }
}

}  // namespace vqx

// ---------------------------------------------------------------------------
// GPTQ column loop of one microscaling block
// (src/voyager_compiler/quantization/gptq.py:241-262): for each row r and
// block column j = 0 .. ncols - 1 in order, with c = col0 + j,
//   q        = float(qmap[bf16(w[r, c] / scale[r])]) * scale[r]
//   out[r,c] = q
//   d        = (w[r, c] - q) / max(hinv[c, c], 1e-12)
//   deltas[r, j] = d
//   w[r, c + k] -= d * hinv[c, c + k]   for the block's later columns
// every operation rounded to fp32 as torch performs it (the product and the
// difference rounded separately, no fused multiply-add).  Each row's block
// sits in the registers of a quad of lanes; the table and the block's corner
// of hinv are staged in LDS (see gptq_block_kernel).  The block's columns of
// w are left as they were.
// ---------------------------------------------------------------------------
namespace vqx {
namespace {

constexpr int kGptqMaxCols = 64;
constexpr int kGptqThreads = 256;
constexpr int kGptqLanes = 4;                          // lanes per row: one DPP quad
constexpr int kGptqSlots = kGptqMaxCols / kGptqLanes;  // columns per lane
constexpr int kGptqRowsPerBlock = kGptqThreads / kGptqLanes;

// Lane o's value in every lane of its quad (o is a constant after unrolling).
__device__ __forceinline__ float quad_bcast(float v, int o) {
  const int x = __float_as_int(v);
  int y;
  switch (o) {
    case 0: y = __builtin_amdgcn_mov_dpp(x, 0x00, 0xF, 0xF, false); break;
    case 1: y = __builtin_amdgcn_mov_dpp(x, 0x55, 0xF, 0xF, false); break;
    case 2: y = __builtin_amdgcn_mov_dpp(x, 0xAA, 0xF, 0xF, false); break;
    default: y = __builtin_amdgcn_mov_dpp(x, 0xFF, 0xF, 0xF, false); break;
  }
  return __int_as_float(y);
}

// Each row is split over a quad of lanes: lane q keeps columns 4i + q
// (i < 16) in registers.  For column j the owning lane's value is broadcast
// in the quad, all four lanes quantize it and form the delta (the same
// arithmetic, so the same bits), and each lane subtracts delta times the
// factor from its own later columns.  Every column still sees the
// reference's sequence of updates, in the same order.  Slots whose column is
// not after j may be updated too: they are no longer read.  The 65536-entry
// bf16 table, the block's 64x64 corner of the factor (laid out so a lane's
// 16 values are contiguous) and its diagonal are staged in LDS; the next
// column's factor row is read while the current column is processed.
// Multiply and subtract round separately, as the reference's two torch ops.
__global__ __launch_bounds__(kGptqThreads) void gptq_block_kernel(
    const float* __restrict__ work, int64_t rows, int64_t ld, int64_t col0, int ncols,
    const float* __restrict__ scale, float quant_max, const uint16_t* __restrict__ scale_qmap,
    const float* __restrict__ hinv, int64_t ldh, const uint16_t* __restrict__ qmap, float* __restrict__ out,
    float* __restrict__ deltas, int64_t ldd) {
#pragma clang fp contract(off)
  __shared__ __align__(16) uint16_t lut[65536];
  __shared__ __align__(16) float hq[kGptqMaxCols * kGptqMaxCols];  // [j][lane][slot] = U[j][4 slot + lane]
  __shared__ __align__(16) float hd[kGptqMaxCols];                 // U[j][j]
  {
    // all of a thread's loads are issued before the first LDS store, so the
    // staging takes a few L2 round trips, not one per load
    constexpr int kLutLoads = 65536 / 8 / kGptqThreads;                      // 32 x 16 bytes
    constexpr int kHLoads = kGptqMaxCols * kGptqMaxCols / kGptqThreads;      // 16 floats
    const uint4* src = reinterpret_cast<const uint4*>(qmap);
    uint4* dst = reinterpret_cast<uint4*>(lut);
    uint4 t[kLutLoads];
#pragma unroll
    for (int u = 0; u < kLutLoads; ++u) t[u] = src[threadIdx.x + u * kGptqThreads];
    float h[kHLoads];
#pragma unroll
    for (int u = 0; u < kHLoads; ++u) {
      const int i = threadIdx.x + u * kGptqThreads, j = i / kGptqMaxCols, k = i % kGptqMaxCols;
      h[u] = (j < ncols && k < ncols) ? hinv[(col0 + j) * ldh + col0 + k] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kLutLoads; ++u) dst[threadIdx.x + u * kGptqThreads] = t[u];
#pragma unroll
    for (int u = 0; u < kHLoads; ++u) {
      const int i = threadIdx.x + u * kGptqThreads, j = i / kGptqMaxCols, k = i % kGptqMaxCols;
      hq[j * kGptqMaxCols + (k % kGptqLanes) * kGptqSlots + k / kGptqLanes] = h[u];
      if (j == k) hd[j] = h[u];
    }
  }
  __syncthreads();
  const int lane = threadIdx.x % kGptqLanes;
  const int64_t r = (int64_t)blockIdx.x * kGptqRowsPerBlock + threadIdx.x / kGptqLanes;
  if (r >= rows) return;  // whole quads leave together
  float w[kGptqSlots], oq[kGptqSlots], od[kGptqSlots];
  const float* wr = work + r * ld + col0;
#pragma unroll
  for (int i = 0; i < kGptqSlots; ++i) {
    const int k = i * kGptqLanes + lane;
    w[i] = k < ncols ? wr[k] : 0.0f;
    oq[i] = 0.0f;
    od[i] = 0.0f;
  }
  float s;
  if (scale) {
    s = scale[r];
  } else {
    // the block's scale as calculate_mx_qparam forms it from the current
    // weights (quantized.py:491-498, gptq.py:103-113): amax of the block
    // (NaN wins), / quant_max (IEEE), through the scale codebook, 1 where not
    // positive, then at least 1e-12
    float m = 0.0f;
    int nan = 0;
#pragma unroll
    for (int i = 0; i < kGptqSlots; ++i) {
      const float a = fabsf(w[i]);  // columns past ncols hold 0
      nan |= a != a;
      m = a > m ? a : m;
    }
    {  // over the quad: lanes ^1, then ^2
      float o = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0xB1, 0xF, 0xF, false));
      nan |= __builtin_amdgcn_mov_dpp(nan, 0xB1, 0xF, 0xF, false);
      m = o > m ? o : m;
      o = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x4E, 0xF, 0xF, false));
      nan |= __builtin_amdgcn_mov_dpp(nan, 0x4E, 0xF, 0xF, false);
      m = o > m ? o : m;
    }
    float sc = nan ? __builtin_nanf("") : m / quant_max;
    if (scale_qmap) sc = bf2f(scale_qmap[f2bf(sc)]);
    sc = sc > 0.0f ? sc : 1.0f;
    s = sc > 1e-12f ? sc : 1e-12f;
  }
  const float* hl = hq + lane * kGptqSlots;
  float hr[kGptqSlots];
#pragma unroll
  for (int i = 0; i < kGptqSlots; ++i) hr[i] = hl[i];
#pragma unroll
  for (int j = 0; j < kGptqMaxCols; ++j) {
    if (j < ncols) {
      const int owner = j % kGptqLanes, slot = j / kGptqLanes;
      float hn[kGptqSlots];
      if (j + 1 < kGptqMaxCols) {
#pragma unroll
        for (int i = (j + 2) / kGptqLanes; i < kGptqSlots; ++i) hn[i] = hl[(j + 1) * kGptqMaxCols + i];
      }
      const float hcc = hd[j];
      const float v = quad_bcast(w[slot], owner);
      const float q = bf2f(lut[f2bf(v / s)]) * s;
      const float d = (v - q) / (hcc > 1e-12f ? hcc : 1e-12f);
      oq[slot] = lane == owner ? q : oq[slot];
      od[slot] = lane == owner ? d : od[slot];
#pragma unroll
      for (int i = (j + 1) / kGptqLanes; i < kGptqSlots; ++i) {
        const float t = d * hr[i];
        w[i] = w[i] - t;
      }
      if (j + 1 < kGptqMaxCols) {
#pragma unroll
        for (int i = (j + 2) / kGptqLanes; i < kGptqSlots; ++i) hr[i] = hn[i];
      }
    }
  }
  float* orow = out + r * ld + col0;
  float* drow = deltas + r * ldd;
#pragma unroll
  for (int i = 0; i < kGptqSlots; ++i) {
    const int k = i * kGptqLanes + lane;
    if (k < ncols) {
      orow[k] = oq[i];
      drow[k] = od[i];
    }
  }
}

// Cholesky factor and its inverse for a diagonal block of at most 64 rows
// (the leaves of the blocked factorisation of the reversed Hessian, whose
// inverse factor is GPTQ's U; gptq.py:32-71 computes U with torch.linalg).
// Four waves; lane i of wave w holds row i, columns 16 w .. 16 w + 15.
//  * Factor, right-looking: for column j the owning wave publishes the
//    updated column in LDS; after the barrier every thread reads the pivot,
//    forms its row's L[i][j] and updates its own later columns with the
//    published column.
//  * L goes to LDS column-major.  Inverse, right-looking: lane c of wave w
//    holds rows 16 w .. 16 w + 15 of column c of L^-1; for row m the owning
//    wave finishes it with the pivot and publishes it, and every thread
//    subtracts column m of L times it from its later rows.
// One barrier per step (the published values alternate between two
// buffers).  Rows n .. 63 are padded with the identity, so the block is
// diag(A, I).  Every load reads a clamped, in-bounds address and selects, so
// all are issued together.  A pivot that is not positive (or NaN) sets
// *info to 1.
constexpr int kCholLeaf = 64;
constexpr int kCholWaves = 4;
constexpr int kCholCols = kCholLeaf / kCholWaves;  // columns (then rows) per thread

__global__ __launch_bounds__(kCholLeaf* kCholWaves) void chol_inv_leaf_kernel(const float* __restrict__ a,
                                                                              int64_t lda, int n,
                                                                              float* __restrict__ li, int64_t ldl,
                                                                              int* __restrict__ info) {
  __shared__ __align__(16) float pub[2][kCholLeaf];
  __shared__ __align__(16) float lt[kCholLeaf * kCholLeaf];  // lt[m * 64 + q] = L[q][m]
  __shared__ __align__(16) float rdiag[kCholLeaf];           // 1 / L[m][m]
  const int lane = threadIdx.x % kCholLeaf;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kCholLeaf);
  const int k0 = w * kCholCols;
  const int ic = lane < n ? lane : n - 1;
  float r[kCholCols];
#pragma unroll
  for (int t = 0; t < kCholCols; ++t) {
    const int k = k0 + t;
    const float v = a[ic * lda + (k < n ? k : n - 1)];
    r[t] = (lane < n && k <= lane) ? v : (k == lane ? 1.0f : 0.0f);
  }
  bool bad = false;
#pragma unroll
  for (int j = 0; j < kCholLeaf; ++j) {
    float* cb = pub[j & 1];
    if (w == j / kCholCols) cb[lane] = r[j % kCholCols];
    __syncthreads();
    // the factor needs fp32 accuracy, not correct rounding: the hardware
    // reciprocal square root keeps the per-column chain short
    const float djj = cb[j];
    const float cl = cb[lane];  // read with the pivot, not behind it
    bad |= !(djj > 0.0f);
    const float inv = __builtin_amdgcn_rsqf(djj);
    const float d = djj * inv;
    if (threadIdx.x == 0) rdiag[j] = inv;
    const float lsc = cl * inv;
    const float lij = lane > j ? lsc : (lane == j ? d : 0.0f);
    if (w == j / kCholCols) r[j % kCholCols] = lij;
    if (k0 + kCholCols - 1 > j) {
#pragma unroll
      for (int t = 0; t < kCholCols; ++t) {
        const float u = fmaf(-lij, cb[k0 + t] * inv, r[t]);
        r[t] = k0 + t > j ? u : r[t];
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kCholCols; ++t) lt[(k0 + t) * kCholLeaf + lane] = r[t];
  __syncthreads();
  // x[t] = (L^-1)[q][c] for q = k0 + t, c = lane
  float x[kCholCols];
#pragma unroll
  for (int t = 0; t < kCholCols; ++t) x[t] = k0 + t == lane ? 1.0f : 0.0f;
#pragma unroll
  for (int m = 0; m < kCholLeaf; ++m) {
    float* xb = pub[m & 1];
    if (w == m / kCholCols) {
      x[m % kCholCols] = x[m % kCholCols] * rdiag[m];
      xb[lane] = x[m % kCholCols];
    }
    __syncthreads();
    const float xm = xb[lane];
    if (k0 + kCholCols - 1 > m) {
#pragma unroll
      for (int t = 0; t < kCholCols; ++t) {
        const float u = fmaf(-lt[m * kCholLeaf + k0 + t], xm, x[t]);
        x[t] = k0 + t > m ? u : x[t];
      }
    }
  }
  if (lane < n) {
#pragma unroll
    for (int t = 0; t < kCholCols; ++t)
      if (k0 + t < n) li[(k0 + t) * ldl + lane] = x[t];
  }
  if (bad && threadIdx.x == 0) info[0] = 1;
}

}  // namespace

int gptq_block(const float* work, int64_t rows, int64_t ld, int64_t col0, int ncols, const float* scale,
               float quant_max, const uint16_t* scale_qmap, const float* hinv, int64_t ldh, const uint16_t* qmap,
               float* out, float* deltas, int64_t ldd, hipStream_t st) {
  if (rows < 0 || ld < 0 || col0 < 0 || ldh < 0) return set_error(kErrInvalid, "gptq_block: negative size");
  if (ncols < 1 || ncols > kGptqMaxCols)
    return set_error(kErrInvalid, "gptq_block: ncols must be in [1, %d] (got %d)", kGptqMaxCols, ncols);
  if (col0 + ncols > ld || col0 + ncols > ldh)
    return set_error(kErrInvalid, "gptq_block: columns %lld..%lld past the row length", (long long)col0,
                     (long long)(col0 + ncols));
  if (ldd < ncols) return set_error(kErrInvalid, "gptq_block: deltas row stride below ncols");
  if (rows == 0) return kOk;
  if (!work || !hinv || !qmap || !out || !deltas) return set_error(kErrInvalid, "gptq_block: null buffer");
  if (!scale && !(quant_max > 0.0f))
    return set_error(kErrInvalid, "gptq_block: quant_max must be positive when the kernel forms the scale");
  if (reinterpret_cast<uintptr_t>(qmap) % 16)
    return set_error(kErrInvalid, "gptq_block: the table must be 16-byte aligned");
  hipLaunchKernelGGL(gptq_block_kernel, dim3((unsigned)((rows + kGptqRowsPerBlock - 1) / kGptqRowsPerBlock)),
                     dim3(kGptqThreads), 0, st, work, rows, ld, col0, ncols, scale, quant_max, scale_qmap, hinv, ldh,
                     qmap, out, deltas, ldd);
  return check_launch("gptq_block");
}

int chol_inverse_block(const float* a, int64_t lda, int n, float* li, int64_t ldl, int* info, hipStream_t st) {
  if (n < 1 || n > kCholLeaf)
    return set_error(kErrInvalid, "chol_inverse_block: n must be in [1, %d] (got %d)", kCholLeaf, n);
  if (lda < n || ldl < n) return set_error(kErrInvalid, "chol_inverse_block: leading dimension below n");
  if (!a || !li || !info) return set_error(kErrInvalid, "chol_inverse_block: null buffer");
  hipLaunchKernelGGL(chol_inv_leaf_kernel, dim3(1), dim3(kCholLeaf * kCholWaves), 0, st, a, lda, n, li, ldl, info);
  return check_launch("chol_inverse_block");
}

}  // namespace vqx
