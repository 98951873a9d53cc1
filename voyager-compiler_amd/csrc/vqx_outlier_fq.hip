// FakeQuantize outlier masking (FusedAmaxObsFakeQuantize.forward,
// src/voyager_compiler/quantization/fake_quantize.py:373-395) on the device:
//
//  * the outlier share's threshold, threshold = min(topk(|x|, k)) with
//    k = max(1, ceil(outlier_pct * numel)), and its running average
//    (fake_quantize.py:373-387), by a radix select on the bit patterns of
//    |x| (no sort, no host round trip);
//  * for the quantization schemes other than microscaling (whose kernels
//    mask, count and restore in their own pass), one pass that writes the
//    input with its outliers zeroed (x.masked_fill(|x| >= t, 0)) and counts
//    them, and one that puts them back into the fake-quantized output
//    (torch.where(skip, x, y)).
//
// The order of non-negative floats is the order of their bit patterns, so
// the k-th largest |x| is found digit by digit: a pass over x histograms the
// next digit of the magnitudes that share the digits chosen so far, and the
// last workgroup of the pass picks the digit where the count from the top
// reaches the rank still wanted.  15-bit magnitudes (bf16, fp16) take two
// passes (11 + 4 bits), fp32 three (11 + 10 + 10).  torch.topk ranks NaN
// above every number and min() propagates it, so any NaN in x makes the
// threshold NaN; pass 0 counts NaNs and settles that case.
#include "vqx_kernels.h"

namespace vqx {
namespace {

struct EltBF16 {
  using S = uint16_t;
  static constexpr uint32_t kMag = 0x7FFFu, kInf = 0x7F80u, kSign = 0x8000u;
  static constexpr int kBits = 15;
  __device__ static float val(uint32_t b) { return u2f(b << 16); }
  __device__ static uint32_t round(float f) { return f2bf(f); }
};
struct EltF16 {
  using S = uint16_t;
  static constexpr uint32_t kMag = 0x7FFFu, kInf = 0x7C00u, kSign = 0x8000u;
  static constexpr int kBits = 15;
  __device__ static float val(uint32_t b) { return h2f_exact(b); }
  __device__ static uint32_t round(float f) { return f2h_exact(f); }
};
struct EltF32 {
  using S = uint32_t;
  static constexpr uint32_t kMag = 0x7FFFFFFFu, kInf = 0x7F800000u, kSign = 0x80000000u;
  static constexpr int kBits = 31;
  __device__ static float val(uint32_t b) { return u2f(b); }
  __device__ static uint32_t round(float f) { return f2u(f); }
};

constexpr int kTopkBins = 2048;  // the widest digit: 11 bits
constexpr int kTopkThreads = 1024;

// Radix-select state in caller-owned device memory, zero-initialised once.
// A call leaves hist, ticket and nan at zero again; prefix, remaining and
// done pass a pass's choice to the next and are rewritten by every call.
constexpr int kTopkFine = 256;  // pass 0's window of 15-bit magnitudes
struct TopkState {
  uint32_t hist[kTopkBins];
  uint32_t fine[kTopkFine];  // pass 0's counts of the magnitudes in its window
  uint32_t ticket;
  uint32_t prefix;     // the magnitude's digits chosen so far
  uint64_t remaining;  // the rank (1 = largest) still wanted among those magnitudes
  uint32_t nan;        // NaNs seen by pass 0
  uint32_t done;       // 1: pass 0 found a NaN and wrote the threshold
};

// The digit of a pass: bits [shift, shift + width) of the magnitude.
struct Digit {
  int shift, width;
};

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The new threshold value (fake_quantize.py:379-387): the first call copies
// the top-k minimum into the fp32 buffer; later calls take
// t * decay + (threshold * (1 - decay)), each operation rounded as torch
// rounds it: t * decay in fp32 (the buffer's dtype), threshold * (1 - decay)
// in x's dtype, the sum in fp32 (three roundings: no contraction into an FMA,
// which rounds once and differs at ties).
template <typename E>
__device__ __forceinline__ void write_threshold(float v, int ema, float decay, float omd, float* thr) {
#pragma clang fp contract(off)
  if (!ema) {
    *thr = v;
    return;
  }
  const float a = *thr * decay;
  const float b = E::val(E::round(v * omd));
  *thr = a + b;
}

// One radix pass.  Every workgroup counts its share of x into an LDS
// histogram and adds the nonzero bins to st->hist; the last one to finish
// picks the digit.  Pass 0 also counts NaNs.  Later passes do nothing when
// pass 0 settled the threshold (a NaN, or the window below).
//
// For 15-bit magnitudes with a previous threshold t (the running average),
// pass 0 also counts every magnitude in a window of 256 from one binade
// below t, one bin each.  When the digit it picks lies inside the window,
// those counts are the second pass's histogram for that digit, so the last
// workgroup finishes the select itself and pass 1 returns at once; a digit
// outside the window leaves it to pass 1 as before.  Either way the result
// is the same k-th largest magnitude.
template <typename E>
__global__ __launch_bounds__(kTopkThreads) void topk_pass_kernel(const typename E::S* __restrict__ x, int64_t n,
                                                                 int64_t k, int pass, Digit dg, int last,
                                                                 TopkState* st, float* thr, int ema, float decay,
                                                                 float omd) {
  using S = typename E::S;
  __shared__ uint32_t h[kTopkBins];
  __shared__ uint32_t s_fine[kTopkFine];
  __shared__ uint32_t s_nan, s_ticket;
  __shared__ uint64_t s_wsum[kTopkThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (pass > 0 && ld_agent(&st->done)) return;  // uniform over the grid
  const uint32_t prefix = pass > 0 ? ld_agent(&st->prefix) : 0u;
  const int nbins = 1 << dg.width;
  const uint32_t dmask = (uint32_t)nbins - 1u;
  // pass 0's window [w0, w0 + 256), 16-aligned (whole second-pass digits),
  // from one binade (128 magnitudes) below the previous threshold
  bool win = false;
  uint32_t w0 = 0;
  if (E::kBits == 15 && pass == 0 && ema) {
    const float tp = *thr;
    if (tp > 0.0f && tp < __builtin_huge_valf()) {
      const uint32_t tb = E::round(tp) & E::kMag;
      w0 = (tb > 128u ? tb - 128u : 0u) & ~15u;
      win = w0 + kTopkFine <= E::kInf;
    }
  }
  for (int i = tid; i < kTopkBins; i += kTopkThreads) h[i] = 0;
  if (win)
    for (int i = tid; i < kTopkFine; i += kTopkThreads) s_fine[i] = 0;
  if (tid == 0) s_nan = 0;
  __syncthreads();
  uint32_t nan = 0;
  auto count = [&](uint32_t b) {
    const uint32_t mag = b & E::kMag;
    if (mag > E::kInf) {
      ++nan;
      return;
    }
    if (pass > 0 && (mag >> (dg.shift + dg.width)) != prefix) return;
    atomicAdd(&h[(mag >> dg.shift) & dmask], 1u);
    if (win && mag - w0 < (uint32_t)kTopkFine) atomicAdd(&s_fine[mag - w0], 1u);
  };
  constexpr int V = 16 / sizeof(S);
  constexpr int U = 4;  // loads in flight per thread
  const int64_t nv = n / V;
  const int64_t stride = (int64_t)gridDim.x * kTopkThreads;
  const u32x4* xv = reinterpret_cast<const u32x4*>(x);
  auto count4 = [&](const u32x4& w) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (sizeof(S) == 2) {
        count(w[j] & 0xFFFFu);
        count(w[j] >> 16);
      } else {
        count(w[j]);
      }
    }
  };
  int64_t i = (int64_t)blockIdx.x * kTopkThreads + tid;
  for (; i + (U - 1) * stride < nv; i += U * stride) {
    u32x4 w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = ld_nt(xv + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) count4(w[u]);
  }
  for (; i < nv; i += stride) count4(ld_nt(xv + i));
  for (int64_t i = nv * V + (int64_t)blockIdx.x * kTopkThreads + tid; i < n; i += stride) count(x[i]);
  if (pass == 0 && nan) atomicAdd(&s_nan, nan);
  __syncthreads();
  for (int i = tid; i < nbins; i += kTopkThreads)
    if (h[i]) __hip_atomic_fetch_add(&st->hist[i], h[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (win)
    for (int i = tid; i < kTopkFine; i += kTopkThreads)
      if (s_fine[i]) __hip_atomic_fetch_add(&st->fine[i], s_fine[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (tid == 0 && s_nan) __hip_atomic_fetch_add(&st->nan, s_nan, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);  // this wave's bin additions have completed
  __syncthreads();
  if (tid == 0) s_ticket = __hip_atomic_fetch_add(&st->ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (s_ticket != gridDim.x - 1) return;

  // ---- the last workgroup: every other workgroup's bins are in st->hist
  __syncthreads();  // every thread has read s_ticket before s_nan is reused
  if (tid == 0) {
    st_agent(&st->ticket, 0u);
    s_nan = pass == 0 ? __hip_atomic_exchange(&st->nan, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
  }
  // the bins into LDS, and cleared for the next pass / call
  for (int i = tid; i < nbins; i += kTopkThreads) {
    h[i] = ld_agent(&st->hist[i]);
    st_agent(&st->hist[i], 0u);
  }
  if (win) {
    for (int i = tid; i < kTopkFine; i += kTopkThreads) {
      s_fine[i] = ld_agent(&st->fine[i]);
      st_agent(&st->fine[i], 0u);
    }
  }
  __syncthreads();
  if (s_nan) {  // a NaN ranks first: the threshold is NaN
    if (tid == 0) {
      write_threshold<E>(__builtin_nanf(""), ema, decay, omd, thr);
      st_agent(&st->done, 1u);
    }
    return;
  }
  const uint64_t want = pass == 0 ? (uint64_t)k
                                  : __hip_atomic_load(&st->remaining, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // each thread owns bins 2 tid and 2 tid + 1; the count above a thread's
  // bins is a suffix sum over the higher threads
  const uint64_t b0 = 2 * tid < nbins ? h[2 * tid] : 0u, b1 = 2 * tid + 1 < nbins ? h[2 * tid + 1] : 0u;
  const uint64_t mine = b0 + b1;
  // inclusive suffix sum within the wave (lanes above this one)
  uint64_t suf = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t u = __shfl_down(suf, o, 64);
    if (lane + o < 64) suf += u;
  }
  if (lane == 0) s_wsum[wv] = suf;  // the wave's total
  __syncthreads();
  uint64_t above = suf - mine;  // bins of the higher lanes of this wave
  for (int w = wv + 1; w < kTopkThreads / 64; ++w) above += s_wsum[w];
  // the selected bin: the count from the top first reaches `want` in it
  int sel = -1;
  uint64_t rem = 0;
  if (above < want && above + b1 >= want) {
    sel = 2 * tid + 1;
    rem = want - above;
  } else if (above + b1 < want && above + mine >= want) {
    sel = 2 * tid;
    rem = want - above - b1;
  }
  if (sel < 0) return;
  const uint32_t digits = (prefix << dg.width) | (uint32_t)sel;
  if (last) {
    write_threshold<E>(E::val(digits << dg.shift), ema, decay, omd, thr);
    return;
  }
  // pass 0 (the one thread that picked the digit): the window's counts of the
  // digit's 16 magnitudes finish the select when they cover it
  const uint32_t m0 = digits << dg.shift;
  if (win && dg.shift == 4 && m0 >= w0 && m0 + 16u <= w0 + kTopkFine) {
    uint64_t c = 0;
    for (int j = 15; j >= 0; --j) {
      c += s_fine[m0 + (uint32_t)j - w0];
      if (c >= rem) {
        write_threshold<E>(E::val(m0 + (uint32_t)j), ema, decay, omd, thr);
        st_agent(&st->done, 1u);
        return;
      }
    }
  }
  if (pass == 0) st_agent(&st->done, 0u);
  st_agent(&st->prefix, digits);
  __hip_atomic_store(&st->remaining, rem, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename E>
int launch_topk(const void* x, int64_t n, int64_t k, int ema, float decay, float omd, float* thr, TopkState* st,
                hipStream_t s) {
  using S = typename E::S;
  constexpr int V = 16 / sizeof(S);
  int64_t need = (n / V + kTopkThreads - 1) / kTopkThreads;
  // one workgroup per CU: each pass ends in a flush of its bins (device-scope
  // atomics), which more workgroups make longer (two per CU measured slower)
  int64_t grid = std::min<int64_t>(std::max<int64_t>(need, 1), num_cus());
  const Digit d15[2] = {{4, 11}, {0, 4}};
  const Digit d31[3] = {{20, 11}, {10, 10}, {0, 10}};
  const int npass = E::kBits == 15 ? 2 : 3;
  for (int p = 0; p < npass; ++p) {
    const Digit dg = E::kBits == 15 ? d15[p] : d31[p];
    hipLaunchKernelGGL(topk_pass_kernel<E>, dim3((unsigned)grid), dim3(kTopkThreads), 0, s, (const S*)x, n, k, p,
                       dg, p == npass - 1 ? 1 : 0, st, thr, ema, decay, omd);
  }
  return check_launch("outlier_topk_threshold");
}

// x with its outliers zeroed (masked: optional, else only the count).
template <typename E>
__global__ __launch_bounds__(256) void outlier_mask_kernel(const typename E::S* __restrict__ x, int64_t n,
                                                           OutlierArgs oa, typename E::S* __restrict__ masked) {
  using S = typename E::S;
  const uint32_t bound = outlier_bound(oa, [](float f) { return E::round(f); }, E::kSign);
  uint32_t cnt = 0;
  constexpr int V = 16 / sizeof(S);
  const int64_t nv = n / V;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const u32x4* xv = reinterpret_cast<const u32x4*>(x);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += stride) {
    u32x4 w = ld_nt(xv + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (sizeof(S) == 2) {
        const bool lo = outlier_skip(w[j] & E::kMag, bound, E::kInf);
        const bool hi = outlier_skip((w[j] >> 16) & E::kMag, bound, E::kInf);
        cnt += (lo ? 1u : 0u) + (hi ? 1u : 0u);
        w[j] &= (lo ? 0xFFFF0000u : 0xFFFFFFFFu) & (hi ? 0x0000FFFFu : 0xFFFFFFFFu);
      } else {
        const bool sk = outlier_skip(w[j] & E::kMag, bound, E::kInf);
        cnt += sk ? 1u : 0u;
        w[j] = sk ? 0u : w[j];
      }
    }
    if (masked) st_nt(reinterpret_cast<u32x4*>(masked) + i, w);
  }
  for (int64_t i = nv * V + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint32_t b = x[i];
    const bool sk = outlier_skip(b & E::kMag, bound, E::kInf);
    cnt += sk ? 1u : 0u;
    if (masked) masked[i] = sk ? (S)0 : (S)b;
  }
  outlier_tally(cnt, oa);
}

// y[i] = x[i] where x[i] is an outlier (torch.where(skip, x, y)); y is only
// written there.
template <typename E>
__global__ __launch_bounds__(256) void outlier_restore_kernel(const typename E::S* __restrict__ x, int64_t n,
                                                              OutlierArgs oa, typename E::S* __restrict__ y) {
  using S = typename E::S;
  const uint32_t bound = outlier_bound(oa, [](float f) { return E::round(f); }, E::kSign);
  constexpr int V = 16 / sizeof(S);
  const int64_t nv = n / V;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const u32x4* xv = reinterpret_cast<const u32x4*>(x);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv; i += stride) {
    const u32x4 w = ld_nt(xv + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (sizeof(S) == 2) {
        if (outlier_skip(w[j] & E::kMag, bound, E::kInf)) y[i * V + 2 * j] = (S)(w[j] & 0xFFFFu);
        if (outlier_skip((w[j] >> 16) & E::kMag, bound, E::kInf)) y[i * V + 2 * j + 1] = (S)(w[j] >> 16);
      } else {
        if (outlier_skip(w[j] & E::kMag, bound, E::kInf)) y[i * V + j] = w[j];
      }
    }
  }
  for (int64_t i = nv * V + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint32_t b = x[i];
    if (outlier_skip(b & E::kMag, bound, E::kInf)) y[i] = (S)b;
  }
}

template <typename F>
int with_elt(int dtype, const char* what, F f) {
  switch (dtype) {
    case kBF16: return f(EltBF16{});
    case kF16: return f(EltF16{});
    case kF32: return f(EltF32{});
    default: return set_error(kErrInvalid, "%s: dtype %d not supported (fp32, bf16, fp16)", what, dtype);
  }
}

}  // namespace

int64_t outlier_topk_workspace_bytes() { return (int64_t)((sizeof(TopkState) + 255) & ~(size_t)255); }

int outlier_topk_threshold(const void* x, int dtype, int64_t n, int64_t k, int ema, float decay, float omd,
                           float* thr, void* workspace, int64_t workspace_bytes, hipStream_t st) {
  if (n < 1) return set_error(kErrInvalid, "outlier_topk_threshold: empty input (torch.topk needs k <= numel)");
  if (k < 1 || k > n)
    return set_error(kErrInvalid, "outlier_topk_threshold: k = %lld outside [1, numel = %lld]", (long long)k,
                     (long long)n);
  if (!x || !thr || !workspace) return set_error(kErrInvalid, "outlier_topk_threshold: null buffer");
  if (workspace_bytes < outlier_topk_workspace_bytes())
    return set_error(kErrInvalid, "outlier_topk_threshold: workspace of %lld bytes, %lld needed",
                     (long long)workspace_bytes, (long long)outlier_topk_workspace_bytes());
  if (!aligned(x, 16) || !aligned(workspace, 16))
    return set_error(kErrInvalid, "outlier_topk_threshold: input and workspace must be 16-byte aligned");
  return with_elt(dtype, "outlier_topk_threshold", [&](auto e) {
    using E = decltype(e);
    return launch_topk<E>(x, n, k, ema, decay, omd, thr, (TopkState*)workspace, st);
  });
}

int outlier_mask(const void* x, int dtype, int64_t n, const OutlierArgs& oa, void* masked, hipStream_t st) {
  if (n == 0) return kOk;
  if (!x) return set_error(kErrInvalid, "outlier_mask: null input");
  if (!aligned(x, 16) || (masked && !aligned(masked, 16)))
    return set_error(kErrInvalid, "outlier_mask: buffers must be 16-byte aligned");
  return with_elt(dtype, "outlier_mask", [&](auto e) {
    using E = decltype(e);
    using S = typename E::S;
    const unsigned grid = grid_for(n / (16 / sizeof(S)) + 1, 256, 8);
    hipLaunchKernelGGL(outlier_mask_kernel<E>, dim3(grid), dim3(256), 0, st, (const S*)x, n, oa, (S*)masked);
    return check_launch("outlier_mask");
  });
}

int outlier_restore(const void* x, int dtype, int64_t n, const OutlierArgs& oa, void* y, hipStream_t st) {
  if (n == 0) return kOk;
  if (!x || !y) return set_error(kErrInvalid, "outlier_restore: null buffer");
  if (!aligned(x, 16)) return set_error(kErrInvalid, "outlier_restore: input must be 16-byte aligned");
  return with_elt(dtype, "outlier_restore", [&](auto e) {
    using E = decltype(e);
    using S = typename E::S;
    const unsigned grid = grid_for(n / (16 / sizeof(S)) + 1, 256, 8);
    hipLaunchKernelGGL(outlier_restore_kernel<E>, dim3(grid), dim3(256), 0, st, (const S*)x, n, oa, (S*)y);
    return check_launch("outlier_restore");
  });
}

}  // namespace vqx
