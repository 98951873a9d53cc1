// Block-scaled product with both operands decoded on the fly:
//   out[b, m, n] = sum_k A'[b, m, k] * B'[b, k, n]  (+ bias[n]),  bf16 out,
// where each operand X' is the decode linear_mx / matmul_mx apply before
// their dense product (src/voyager_compiler/ops/quantized.py:313-326 and
// :388-398): X' = bf16(code[trunc(X)] * scale[block of k]) with the code
// lookup and the scale each optional.  X holds bf16 values or integer-valued
// bf16 code indices; the scales are bf16, one per block of `bs` along K.
// This is the path of the converted models' operands that are not a
// 16-level weight with blocks of 64 (that one runs vqx_nf4_gemm.hip with a
// packed weight): int6 / nf4_6 attention operands coded on both sides, int8
// weights with blocks of 16, activations coded with input_code / input_scale.
//
// bf16 MFMA (v_mfma_f32_32x32x16_bf16), fp32 accumulation.  A workgroup of
// 256 threads computes a 128 x 128 tile; wave w owns the 64 x 64 block at
// rows 64 (w >> 1), columns 64 (w & 1).  The K loop steps by 64.  Each step
// the raw operand bytes of step s + 2 are loaded into registers (two register
// sets, so a load has two steps to land), those of step s + 1 are decoded and
// written to the other of two LDS stages, and the MFMAs of step s read their
// fragments from the current stage; one barrier per step.  Two workgroups fit
// a CU (72 KiB of LDS each), so one's decode runs under the other's MFMAs.
//  * K-major operands ([rows][K], A always): 16-byte loads, 8 lanes per
//    128-byte row; each 8-value chunk shares one scale (the block size is a
//    power of two >= 8).
//  * An N-major right operand ([K][N], matmul_mx's "ck" layout): each thread
//    loads 4 k rows x 8 columns, decodes them with the 8 columns' scales (one
//    16-byte load) and transposes them with v_perm into 8 column rows of 4 k,
//    written as 8-byte LDS stores.
//  * Code lookups: the decode of a pattern depends only on its sign and on
//    its magnitude clamped to [0x3F7F, 0x4381] (every |v| < 1 truncates to
//    index 0 like 0.996; |v| >= 258, Inf and NaN are outside any table of up
//    to 256 entries), so each workgroup tabulates 2 x 1027 decoded bf16 values
//    in LDS once and a lookup is a clamp and one 2-byte LDS read.  An index
//    outside the table (the reference raises IndexError) decodes to NaN.
// Tiles are numbered batch-major, then by row tile, then by column tile, and
// handed out so each XCD runs a contiguous range (whole row slabs of A, and
// for batched attention products whole heads, stay in its L2).
#include <type_traits>

#include "vqx_kernels.h"

namespace vqx {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTK = 64;  // k per step
constexpr uint32_t kCodeLo = 0x3F7Fu, kCodeHi = 0x4381u;
constexpr int kCodeSpan = (int)(kCodeHi - kCodeLo) + 1;  // entries per sign
constexpr int kMaxCode = 256;

enum Dec : int { kPlain = 0, kScale = 1, kCode = 2, kCodeScale = 3 };

struct MxOpArgs {
  const uint16_t* data;
  const uint16_t* scale;
  const uint16_t* code;
  int64_t bstride, ld, sbstride, sld;
  int32_t code_len, bs_shift;  // block size = 1 << bs_shift
};

// byte offset of 16-byte chunk c (0..7) of row r in a [rows][64] bf16 tile;
// the slot is c ^ (r & 7) ^ ((r >> 3) & 7).  Fragment reads (16 aligned
// consecutive rows, one chunk) meet 16 distinct (row parity, slot) pairs and
// row-wise 16-byte writes 16 distinct pairs per 16 lanes, so both are
// conflict free; the N-major operand's 8-byte column writes meet at most two
// lanes per bank group.
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t c) {
  return r * 128u + ((c ^ (r & 7u) ^ ((r >> 3) & 7u)) << 4);
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Decoded bf16 value of code pattern h through the LDS table.
__device__ __forceinline__ uint32_t code_value(const uint16_t* tab, uint32_t h) {
  uint32_t a = h & 0x7FFFu;
  a = a < kCodeLo ? kCodeLo : (a > kCodeHi ? kCodeHi : a);
  return tab[a - kCodeLo + ((h >> 15) & 1u) * (uint32_t)kCodeSpan];
}

// The table: entry e of sign s is the decode of the bf16 pattern
// s << 15 | (kCodeLo + e), the reference's code[index.to(long)] (trunc
// toward zero, a negative index counting from the end).
template <int THREADS>
__device__ void build_code_table(uint16_t* tab, const uint16_t* code, int len) {
  for (int e = threadIdx.x; e < 2 * kCodeSpan; e += THREADS) {
    const uint32_t s = e >= kCodeSpan ? 1u : 0u;
    const uint32_t h = (s << 15) | (kCodeLo + (uint32_t)(e - (int)s * kCodeSpan));
    const float t = __builtin_truncf(u2f(h << 16));
    const bool ok = t >= -(float)len && t < (float)len;
    const int i = ok ? (int)t : 0;
    tab[e] = ok ? code[i < 0 ? i + len : i] : (uint16_t)0x7FC0u;
  }
}

// Decode one dword (two bf16 patterns, low half first) with scales s0 / s1.
template <int D>
__device__ __forceinline__ uint32_t decode2(uint32_t w, float s0, float s1, const uint16_t* tab) {
  if constexpr (D == kPlain) {
    return w;
  } else if constexpr (D == kScale) {
    return pack_bf16x2(u2f(w << 16) * s0, u2f(w & 0xFFFF0000u) * s1);
  } else {
    const uint32_t lo = code_value(tab, w & 0xFFFFu), hi = code_value(tab, w >> 16);
    if constexpr (D == kCode) return lo | (hi << 16);
    else return pack_bf16x2(u2f(lo << 16) * s0, u2f(hi << 16) * s1);
  }
}

__device__ __forceinline__ float bf_lo(uint32_t w) { return u2f(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return u2f(w & 0xFFFF0000u); }

// One operand's raw bytes of one step: up to four 16-byte chunks and their scales.
struct Raw {
  u32x4 v[4];
  u32x4 s;  // K-major: s[q] low half = scale of chunk q; N-major: the 8 columns' scales
  bool in;  // the chunks lie inside K (past K they are zero and must decode to zero)
};

// K-major staging of ROWS tile rows (A, or B stored [N][K]) by THREADS
// threads: chunk q of thread t is chunk t % 8 of tile row t / 8 + q THREADS / 8.
// Loads are never skipped (a branch around a load makes the compiler wait for
// every load in flight at the join): past the last row the last row is read,
// past K the last chunk, and in a checked step the chunk is zeroed after the
// load.  Addresses are a uniform base (the batch item) plus 32-bit byte
// offsets; LDS addresses are precomputed.
template <int D, int ROWS, int THREADS>
struct KMajor {
  static constexpr int kCh = ROWS * 8 / THREADS;  // chunks per thread
  static_assert(kCh >= 1 && kCh <= 4, "chunks per thread");
  const char* base;   // data of the batch item
  const char* sbase;  // scales of the batch item
  uint32_t off[kCh];  // byte offset of the thread's chunk in step 0, per row
  uint32_t soff[kCh];
  uint32_t lds[kCh];  // LDS byte offset of the thread's chunks in a stage
  int sh;

  __device__ __forceinline__ void init(const MxOpArgs& o, int64_t b, int r0, int rows_valid) {
    const int t = threadIdx.x;
    base = reinterpret_cast<const char*>(o.data + b * o.bstride);
    if constexpr (D == kScale || D == kCodeScale) sbase = reinterpret_cast<const char*>(o.scale + b * o.sbstride);
#pragma unroll
    for (int q = 0; q < kCh; ++q) {
      int r = r0 + (t >> 3) + (THREADS / 8) * q;
      r = r < rows_valid ? r : rows_valid - 1;
      off[q] = 2u * ((uint32_t)r * (uint32_t)o.ld + (uint32_t)(t & 7) * 8u);
      if constexpr (D == kScale || D == kCodeScale) soff[q] = 2u * (uint32_t)r * (uint32_t)o.sld;
      lds[q] = swz((t >> 3) + (THREADS / 8) * q, t & 7);
    }
    sh = o.bs_shift;
  }
  template <bool CHECK>
  __device__ __forceinline__ void load(Raw& x, int ks, int K) {
    int k = ks * kTK + (threadIdx.x & 7) * 8;
    x.in = true;
    if constexpr (CHECK) {
      x.in = k < K;
      k = x.in ? k : K - 8;
    }
    const uint32_t kb = 2u * (uint32_t)(k - (int)(threadIdx.x & 7) * 8);
#pragma unroll
    for (int q = 0; q < kCh; ++q) {
      x.v[q] = *reinterpret_cast<const u32x4*>(base + (off[q] + kb));
      if constexpr (D == kScale || D == kCodeScale)
        x.s[q] = *reinterpret_cast<const uint16_t*>(sbase + (soff[q] + 2u * (uint32_t)(k >> sh)));
    }
  }
  // decode and write to the stage; in a checked step chunks past K are
  // written as zeros
  template <bool CHECK>
  __device__ __forceinline__ void store(const Raw& x, uint8_t* stage, const uint16_t* tab) {
#pragma unroll
    for (int q = 0; q < kCh; ++q) {
      const float s = bf_lo(x.s[q]);
      u32x4 d;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        d[j] = decode2<D>(x.v[q][j], s, s, tab);
        if constexpr (CHECK) d[j] = x.in ? d[j] : 0u;
      }
      *reinterpret_cast<u32x4*>(stage + lds[q]) = d;
    }
  }
};

// N-major staging of COLS tile columns (B stored [K][N]): a 64-deep step is
// 16 blocks of 4 k rows by COLS / 8 blocks of 8 columns; thread t < 2 COLS
// loads block (k rows 4 (t / (COLS / 8)) .. +3, columns 8 (t % (COLS / 8))
// .. +7) (past N the last 8 columns, past K the last 4 rows, zeroed after the
// load in a checked step), decodes it with the 8 columns' scales and
// transposes it into 8 column rows of 4 k.
template <int D, int COLS, int THREADS>
struct NMajor {
  static constexpr int kOct = COLS / 8;  // column blocks per k-row block
  static_assert(2 * COLS <= THREADS, "one block per thread");
  const char* base;
  const char* sbase;
  uint32_t coff;   // byte offset of the thread's first column (clamped)
  uint32_t ldb;    // bytes between k rows
  uint32_t sldb;   // bytes between block rows of the scales
  int sh;

  __device__ __forceinline__ static bool active() { return 2 * COLS == THREADS || (int)threadIdx.x < 2 * COLS; }

  __device__ __forceinline__ void init(const MxOpArgs& o, int64_t b, int n0, int N) {
    const int t = threadIdx.x;
    int n = n0 + (t % kOct) * 8;
    n = n < N ? n : N - 8;
    base = reinterpret_cast<const char*>(o.data + b * o.bstride);
    if constexpr (D == kScale || D == kCodeScale) sbase = reinterpret_cast<const char*>(o.scale + b * o.sbstride);
    coff = 2u * (uint32_t)n;
    ldb = 2u * (uint32_t)o.ld;
    sldb = 2u * (uint32_t)o.sld;
    sh = o.bs_shift;
  }
  template <bool CHECK>
  __device__ __forceinline__ void load(Raw& x, int ks, int K) {
    if (!active()) return;
    int k = ks * kTK + ((int)threadIdx.x / kOct) * 4;
    x.in = true;
    if constexpr (CHECK) {
      x.in = k < K;  // K % 8 == 0: the four rows are all in or all out
      k = x.in ? k : K - 4;
    }
    const uint32_t r0 = (uint32_t)k * ldb + coff;
#pragma unroll
    for (int i = 0; i < 4; ++i) x.v[i] = *reinterpret_cast<const u32x4*>(base + (r0 + (uint32_t)i * ldb));
    if constexpr (D == kScale || D == kCodeScale)
      x.s = *reinterpret_cast<const u32x4*>(sbase + ((uint32_t)(k >> sh) * sldb + coff));
  }
  template <bool CHECK>
  __device__ __forceinline__ void store(const Raw& x, uint8_t* stage, const uint16_t* tab) {
    if (!active()) return;
    const int t = threadIdx.x, o = t % kOct, kq = t / kOct;
    u32x4 d[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        d[i][j] = decode2<D>(x.v[i][j], bf_lo(x.s[j]), bf_hi(x.s[j]), tab);
        if constexpr (CHECK) d[i][j] = x.in ? d[i][j] : 0u;
      }
    // column 2 j takes the low halves of dword j of rows 0..3, column 2 j + 1
    // the high halves
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x2 ev = {__builtin_amdgcn_perm(d[1][j], d[0][j], 0x05040100u),
                        __builtin_amdgcn_perm(d[3][j], d[2][j], 0x05040100u)};
      const u32x2 od = {__builtin_amdgcn_perm(d[1][j], d[0][j], 0x07060302u),
                        __builtin_amdgcn_perm(d[3][j], d[2][j], 0x07060302u)};
      *reinterpret_cast<u32x2*>(stage + swz(8 * o + 2 * j, kq >> 1) + 8 * (kq & 1)) = ev;
      *reinterpret_cast<u32x2*>(stage + swz(8 * o + 2 * j + 1, kq >> 1) + 8 * (kq & 1)) = od;
    }
  }
};

// Output of one wave's (32 FM) x 64 block, staged through LDS: the wave
// writes its bf16 results (bias added) as rows of 144 bytes (64 values and
// 16 bytes of padding, which spreads a column of 32 rows over the banks)
// into its own region, then stores 8 whole 128-byte row segments per
// instruction (16 bytes a lane, non-temporal: the output is not read again
// by this kernel).  The accumulator layout has each lane hold 4 consecutive
// columns of 32 different rows, which would otherwise make every store
// instruction write 16-byte pieces of 32 rows.
constexpr int kOutRow = 144;  // bytes per staged row

template <int FM>
__device__ __forceinline__ void store_block(f32x16 (&acc)[FM][2], uint8_t* region, const uint16_t* __restrict__ bias,
                                            uint16_t* __restrict__ ob, int M, int N, int mrow0, int ncol0) {
  const int lane = threadIdx.x & 63, lr = lane & 31, lk = lane >> 5;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = j * 32 + 8 * g + 4 * lk;  // column within the block
      if (bias) {
        const int n = ncol0 + c < N ? ncol0 + c : N - 4;  // N % 4 == 0
        const u32x2 bb = *reinterpret_cast<const u32x2*>(bias + n);
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          acc[i][j][4 * g] += bf_lo(bb.x);
          acc[i][j][4 * g + 1] += bf_hi(bb.x);
          acc[i][j][4 * g + 2] += bf_lo(bb.y);
          acc[i][j][4 * g + 3] += bf_hi(bb.y);
        }
      }
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const u32x2 o = {pack_bf16x2(acc[i][j][4 * g], acc[i][j][4 * g + 1]),
                         pack_bf16x2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3])};
        *reinterpret_cast<u32x2*>(region + (i * 32 + lr) * kOutRow + c * 2) = o;
      }
    }
  wave_lds_sync();
  const int c = (lane & 7) * 8, n = ncol0 + c;
#pragma unroll
  for (int q = 0; q < FM * 4; ++q) {
    const int r = q * 8 + (lane >> 3), m = mrow0 + r;
    const u32x4 v = *reinterpret_cast<const u32x4*>(region + r * kOutRow + c * 2);
    if (m >= M || n >= N) continue;
    uint16_t* dst = ob + (int64_t)m * N + n;
    if ((N & 7) == 0) {
      st_nt(reinterpret_cast<u32x4*>(dst), v);
    } else {  // rows are only 8-byte aligned; the last chunk may be half inside
      *reinterpret_cast<u32x2*>(dst) = u32x2{v.x, v.y};
      if (n + 4 < N) *reinterpret_cast<u32x2*>(dst + 4) = u32x2{v.z, v.w};
    }
  }
}

// Tile shapes: TM x TN outputs per workgroup of THREADS threads; the waves
// form a (TM / WROWS) x (TN / 64) grid, each owning WROWS x 64 outputs as
// (WROWS / 32) x 2 MFMA tiles of 32 x 32.
//   128 x 128, 256 threads: 64 x 64 per wave, two workgroups per CU;
//   256 x 128, 512 threads: 64 x 64 per wave, one workgroup per CU: three
//                           quarters of the 128 x 128 tile's decode per
//                           product.
// (256 x 256 with 128 x 64 per wave needs more than the 256 registers a wave
// has at two waves per SIMD: its accumulators alone take 128.)
template <int TM, int TN>
struct Shape {
  static constexpr int kThreads = (TM == 128 && TN == 128) ? 256 : 512;  // as in the launch bounds below
  static constexpr int kWavesN = TN / 64;
  static constexpr int kWavesM = kThreads / 64 / kWavesN;
  static constexpr int kWRows = TM / kWavesM;
  static constexpr int kFM = kWRows / 32;
  static constexpr int kStageA = TM * kTK * 2, kStageB = TN * kTK * 2;
};

template <int DA, int DB, bool BK, int TM, int TN>
__global__ __launch_bounds__((TM == 128 && TN == 128) ? 256 : 512, 2) void mx_gemm_kernel(
    MxOpArgs a, MxOpArgs b, const uint16_t* __restrict__ bias, uint16_t* __restrict__ out, int M, int N, int K, int tm,
    int tn, int ntiles) {
  using S = Shape<TM, TN>;
  constexpr int kThreads = S::kThreads, kFM = S::kFM, kStageA = S::kStageA, kStageB = S::kStageB;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * (kStageA + kStageB)];
  static_assert(kThreads / 64 * kFM * 32 * kOutRow <= 2 * (kStageA + kStageB), "output staging fits the stages");
  uint8_t* const la = lds;
  uint8_t* const lb = lds + 2 * kStageA;
  __shared__ uint16_t ta[DA >= kCode ? 2 * kCodeSpan : 1];
  __shared__ uint16_t tb[DB >= kCode ? 2 * kCodeSpan : 1];

  const int bid = blockIdx.x;
  const int per_xcd = (ntiles + 7) / 8;
  const int tile = ntiles % 8 == 0 ? (bid & 7) * per_xcd + (bid >> 3) : bid;
  const int per_batch = tm * tn;
  const int64_t bi = tile / per_batch;
  const int rem = tile - (int)bi * per_batch;
  const int m0 = (rem / tn) * TM, n0 = (rem % tn) * TN;

  if constexpr (DA >= kCode) build_code_table<kThreads>(ta, a.code, a.code_len);
  if constexpr (DB >= kCode) build_code_table<kThreads>(tb, b.code, b.code_len);
  if constexpr (DA >= kCode || DB >= kCode) __syncthreads();

  KMajor<DA, TM, kThreads> sa;
  sa.init(a, bi, m0, M);
  typename std::conditional<BK, KMajor<DB, TN, kThreads>, NMajor<DB, TN, kThreads>>::type sb;
  sb.init(b, bi, n0, N);

  const int nk = (K + kTK - 1) / kTK;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / S::kWavesN, wn = wave % S::kWavesN, lr = lane & 31, lk = lane >> 5;

  f32x16 acc[kFM][2];
#pragma unroll
  for (int i = 0; i < kFM; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  auto compute = [&](uint32_t sta, uint32_t stb) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      bf16x8 fb[2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        fb[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(lb + stb + swz(wn * 64 + j * 32 + lr, kk * 2 + lk)));
#pragma unroll
      for (int i = 0; i < kFM; ++i) {
        const bf16x8 fa = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const u32x4*>(la + sta + swz(wm * S::kWRows + i * 32 + lr, kk * 2 + lk)));
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[j], fa, acc[i][j], 0, 0, 0);
      }
    }
  };

  // step s lives in registers ra/rb[s % 2] and in LDS stage s % 2
  Raw ra[2], rb[2];
  sa.template load<true>(ra[0], 0, K);
  sb.template load<true>(rb[0], 0, K);
  if (nk > 1) {
    sa.template load<true>(ra[1], 1, K);
    sb.template load<true>(rb[1], 1, K);
  }
  sa.template store<true>(ra[0], la, ta);
  sb.template store<true>(rb[0], lb, tb);
  if (nk > 2) {
    sa.template load<true>(ra[0], 2, K);
    sb.template load<true>(rb[0], 2, K);
  }
  lds_barrier();

  // FULL: ks + 3 < nk and step ks + 3 lies wholly inside K (so do the steps
  // before it), so the step stores and loads unconditionally and without
  // range checks: no branch in the steady state, and the compiler waits only
  // for the loads of the step it decodes, not for those issued after them
  auto step = [&](int ks, auto par, auto full) {
    constexpr int P = decltype(par)::value;  // ks % 2
    constexpr bool kFull = decltype(full)::value;
    compute(P * kStageA, P * kStageB);
    if (kFull || ks + 1 < nk) {
      sa.template store<!kFull>(ra[1 - P], la + (1 - P) * kStageA, ta);
      sb.template store<!kFull>(rb[1 - P], lb + (1 - P) * kStageB, tb);
    }
    lds_barrier();
    if (kFull || ks + 3 < nk) {
      sa.template load<!kFull>(ra[1 - P], ks + 3, K);
      sb.template load<!kFull>(rb[1 - P], ks + 3, K);
    }
  };
  const std::integral_constant<int, 0> p0;
  const std::integral_constant<int, 1> p1;
  const std::true_type all;
  const std::false_type checked;
  const int nfull = K / kTK;  // steps wholly inside K
  int ks = 0;
  for (; ks + 4 < nfull; ks += 2) {
    step(ks, p0, all);
    step(ks + 1, p1, all);
  }
  for (; ks < nk; ks += 2) {
    step(ks, p0, checked);
    if (ks + 1 < nk) step(ks + 1, p1, checked);
  }

  // every wave has passed the last step's barrier: the stages are free for
  // the output staging
  store_block<kFM>(acc, lds + wave * (kFM * 32 * kOutRow), bias, out + bi * (int64_t)M * N, M, N,
                   m0 + wm * S::kWRows, n0 + wn * 64);
}

// The decode of one operand into dense bf16 in its own layout: the pass the
// host runs ahead of the product for an operand that many output tiles read.
// Item b of the operand is [R][C] (row stride o.ld), out is [items][R][C]
// contiguous; K-major: C = K, blocks along C; N-major: R = K, blocks along R.
// Each thread decodes 8 consecutive values of a row per iteration.
template <int D, bool KMAJ>
__global__ __launch_bounds__(256) void mx_decode_kernel(MxOpArgs o, uint16_t* __restrict__ out, int R, int C,
                                                        uint32_t chunks) {
  __shared__ uint16_t tab[D >= kCode ? 2 * kCodeSpan : 1];
  if constexpr (D >= kCode) {
    build_code_table<256>(tab, o.code, o.code_len);
    __syncthreads();
  }
  const uint32_t cpr = (uint32_t)C / 8u;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < chunks; i += gridDim.x * 256u) {
    const uint32_t row = i / cpr;  // over all items
    const int c = (int)(i - row * cpr) * 8;
    const uint32_t bi = row / (uint32_t)R;
    const int r = (int)(row - bi * (uint32_t)R);
    const u32x4 v = ld_nt(reinterpret_cast<const u32x4*>(o.data + (int64_t)bi * o.bstride + (int64_t)r * o.ld + c));
    u32x4 d;
    if constexpr (KMAJ) {
      float s = 1.0f;
      if constexpr (D == kScale || D == kCodeScale)
        s = bf_lo(o.scale[(int64_t)bi * o.sbstride + (int64_t)r * o.sld + (c >> o.bs_shift)]);
#pragma unroll
      for (int j = 0; j < 4; ++j) d[j] = decode2<D>(v[j], s, s, tab);
    } else {
      u32x4 sc = {0u, 0u, 0u, 0u};
      if constexpr (D == kScale || D == kCodeScale)
        sc = *reinterpret_cast<const u32x4*>(o.scale + (int64_t)bi * o.sbstride + (int64_t)(r >> o.bs_shift) * o.sld + c);
#pragma unroll
      for (int j = 0; j < 4; ++j) d[j] = decode2<D>(v[j], bf_lo(sc[j]), bf_hi(sc[j]), tab);
    }
    st_nt(reinterpret_cast<u32x4*>(out + (int64_t)row * C + c), d);
  }
}

template <int DA, int DB, bool BK, int TM, int TN>
int launch_one(const MxOpArgs& a, const MxOpArgs& b, const uint16_t* bias, uint16_t* out, int M, int N, int K,
               int batch, hipStream_t stream) {
  const int tm = (M + TM - 1) / TM, tn = (N + TN - 1) / TN;
  const int64_t ntiles = (int64_t)batch * tm * tn;
  if (ntiles > INT32_MAX) return set_error(kErrInvalid, "mx_gemm: too many tiles");
  hipLaunchKernelGGL((mx_gemm_kernel<DA, DB, BK, TM, TN>), dim3((unsigned)ntiles), dim3(Shape<TM, TN>::kThreads), 0,
                     stream, a, b, bias, out, M, N, K, tm, tn, (int)ntiles);
  return check_launch("mx_gemm_kernel");
}

// The tile, from measurement (LLaMA-7B shapes on one MI355X): 256 x 128
// for products with N > 128 and K > 128 that still give every CU a tile
// (the MXINT8 MLP linear: 253 against 282 us), else 128 x 128 (two
// workgroups per CU: the attention products, K = 128 or N = 128, run 9% and
// 6% faster on it).
enum TileKind : int { kT128 = 0, kT256x128 = 1 };

int pick_tile(int64_t batch, int64_t M, int64_t N, int64_t K) {
  if (N <= 128 || K <= 128) return kT128;
  const int64_t tiles = batch * ((M + 255) / 256) * ((N + 127) / 128);
  return tiles >= num_cus() ? kT256x128 : kT128;
}

template <int DA, int DB, bool BK>
int launch_tile(int tile, const MxOpArgs& a, const MxOpArgs& b, const uint16_t* bias, uint16_t* out, int M, int N,
                int K, int batch, hipStream_t stream) {
  if (tile == kT256x128) return launch_one<DA, DB, BK, 256, 128>(a, b, bias, out, M, N, K, batch, stream);
  return launch_one<DA, DB, BK, 128, 128>(a, b, bias, out, M, N, K, batch, stream);
}

template <int DA, int DB>
int launch_layout(bool bk, int tile, const MxOpArgs& a, const MxOpArgs& b, const uint16_t* bias, uint16_t* out, int M,
                  int N, int K, int batch, hipStream_t stream) {
  return bk ? launch_tile<DA, DB, true>(tile, a, b, bias, out, M, N, K, batch, stream)
            : launch_tile<DA, DB, false>(tile, a, b, bias, out, M, N, K, batch, stream);
}

template <int DA>
int launch_b(int db, bool bk, int tile, const MxOpArgs& a, const MxOpArgs& b, const uint16_t* bias, uint16_t* out,
             int M, int N, int K, int batch, hipStream_t stream) {
  switch (db) {
    case kPlain: return launch_layout<DA, kPlain>(bk, tile, a, b, bias, out, M, N, K, batch, stream);
    case kScale: return launch_layout<DA, kScale>(bk, tile, a, b, bias, out, M, N, K, batch, stream);
    case kCode: return launch_layout<DA, kCode>(bk, tile, a, b, bias, out, M, N, K, batch, stream);
    default: return launch_layout<DA, kCodeScale>(bk, tile, a, b, bias, out, M, N, K, batch, stream);
  }
}

int dec_of(const MxOperand& o) { return (o.code ? kCode : kPlain) | (o.scale ? kScale : kPlain); }

// The kernels address each matrix (and its scales) of a batch item with
// 32-bit byte offsets from the item's base.
constexpr int64_t kMaxItemBytes = (int64_t)1 << 32;

int check_operand(const MxOperand& o, const char* name, bool k_major_only, int64_t K, int64_t cols) {
  if (!o.data || !aligned(o.data, 16)) return set_error(kErrInvalid, "%s: data must be a 16-byte aligned pointer", name);
  if (k_major_only && !o.k_major) return set_error(kErrInvalid, "%s: the left operand is K-major ([M][K])", name);
  const int64_t need = o.k_major ? K : cols;
  if (o.ld < need || o.ld % 8) return set_error(kErrInvalid, "%s: ld %lld must be >= %lld and a multiple of 8", name,
                                                (long long)o.ld, (long long)need);
  if (o.batch_stride < 0 || o.batch_stride % 8)
    return set_error(kErrInvalid, "%s: batch_stride must be >= 0 and a multiple of 8", name);
  const int64_t span = o.k_major ? (cols - 1) * o.ld + K : (K - 1) * o.ld + cols;
  if (2 * span >= kMaxItemBytes)
    return set_error(kErrInvalid, "%s: one batch item spans more than 4 GiB", name);
  if (o.code && (o.code_len < 1 || o.code_len > kMaxCode))
    return set_error(kErrInvalid, "%s: code_len %d outside 1..%d", name, (int)o.code_len, kMaxCode);
  if (o.scale) {
    if (o.block_size < 8 || (o.block_size & (o.block_size - 1)))
      return set_error(kErrInvalid, "%s: block_size %d must be a power of two >= 8", name, (int)o.block_size);
    const int64_t nkb = (K + o.block_size - 1) / o.block_size;
    if (o.scale_batch_stride < 0) return set_error(kErrInvalid, "%s: scale_batch_stride must be >= 0", name);
    const int64_t sspan = o.k_major ? (cols - 1) * o.scale_ld + nkb : (nkb - 1) * o.scale_ld + cols;
    if (2 * sspan >= kMaxItemBytes)
      return set_error(kErrInvalid, "%s: one batch item's scales span more than 4 GiB", name);
    if (o.k_major) {
      if (o.scale_ld < nkb) return set_error(kErrInvalid, "%s: scale_ld must be >= %lld", name, (long long)nkb);
    } else {
      if (!aligned(o.scale, 16) || o.scale_ld < cols || o.scale_ld % 8 || o.scale_batch_stride % 8)
        return set_error(kErrInvalid,
                         "%s: N-major scales need a 16-byte aligned pointer, scale_ld >= %lld and strides that are "
                         "multiples of 8",
                         name, (long long)cols);
    }
  }
  return kOk;
}

MxOpArgs args_of(const MxOperand& o) {
  MxOpArgs r;
  r.data = static_cast<const uint16_t*>(o.data);
  r.scale = static_cast<const uint16_t*>(o.scale);
  r.code = static_cast<const uint16_t*>(o.code);
  r.bstride = o.batch_stride;
  r.ld = o.ld;
  r.sbstride = o.scale_batch_stride;
  r.sld = o.scale_ld;
  r.code_len = o.code ? o.code_len : 0;
  r.bs_shift = o.scale ? __builtin_ctz((unsigned)o.block_size) : 0;
  return r;
}

}  // namespace

int mx_gemm(const MxOperand& a, const MxOperand& b, const uint16_t* bias, uint16_t* out, int64_t batch, int64_t M,
            int64_t N, int64_t K, hipStream_t stream) {
  if (batch < 1 || M < 1 || N < 1 || K < 1) return set_error(kErrInvalid, "mx_gemm: empty product");
  if (K % 8) return set_error(kErrInvalid, "mx_gemm: K (%lld) must be a multiple of 8", (long long)K);
  if (N % 4) return set_error(kErrInvalid, "mx_gemm: N (%lld) must be a multiple of 4", (long long)N);
  if (!b.k_major && N % 8) return set_error(kErrInvalid, "mx_gemm: an N-major right operand needs N %% 8 == 0");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX) return set_error(kErrInvalid, "mx_gemm: dimension too large");
  int rc = check_operand(a, "mx_gemm A", true, K, M);
  if (rc) return rc;
  rc = check_operand(b, "mx_gemm B", false, K, N);
  if (rc) return rc;
  if (!out || !aligned(out, 8)) return set_error(kErrInvalid, "mx_gemm: out must be 8-byte aligned");
  if (bias && !aligned(bias, 8)) return set_error(kErrInvalid, "mx_gemm: bias must be 8-byte aligned");
  if (batch > INT32_MAX) return set_error(kErrInvalid, "mx_gemm: batch too large");
  const MxOpArgs aa = args_of(a), bb = args_of(b);
  const int db = dec_of(b);
  const bool bk = b.k_major != 0;
  const int tile = pick_tile(batch, M, N, K);
  const int iM = (int)M, iN = (int)N, iK = (int)K, ib = (int)batch;
  switch (dec_of(a)) {
    case kPlain: return launch_b<kPlain>(db, bk, tile, aa, bb, bias, out, iM, iN, iK, ib, stream);
    case kScale: return launch_b<kScale>(db, bk, tile, aa, bb, bias, out, iM, iN, iK, ib, stream);
    case kCode: return launch_b<kCode>(db, bk, tile, aa, bb, bias, out, iM, iN, iK, ib, stream);
    default: return launch_b<kCodeScale>(db, bk, tile, aa, bb, bias, out, iM, iN, iK, ib, stream);
  }
}

template <int D>
int launch_decode(bool kmaj, const MxOpArgs& o, uint16_t* out, int R, int C, uint32_t chunks, hipStream_t stream) {
  const unsigned grid = grid_for(chunks, 256, 8);
  if (kmaj)
    hipLaunchKernelGGL((mx_decode_kernel<D, true>), dim3(grid), dim3(256), 0, stream, o, out, R, C, chunks);
  else
    hipLaunchKernelGGL((mx_decode_kernel<D, false>), dim3(grid), dim3(256), 0, stream, o, out, R, C, chunks);
  return check_launch("mx_decode_kernel");
}

int mx_decode(const MxOperand& x, int64_t batch, int64_t rows, int64_t K, uint16_t* out, hipStream_t stream) {
  if (batch < 1 || rows < 1 || K < 1) return set_error(kErrInvalid, "mx_decode: empty operand");
  if (K % 8) return set_error(kErrInvalid, "mx_decode: K (%lld) must be a multiple of 8", (long long)K);
  if (!x.k_major && rows % 8)
    return set_error(kErrInvalid, "mx_decode: an N-major operand needs a multiple of 8 columns");
  int rc = check_operand(x, "mx_decode", false, K, rows);
  if (rc) return rc;
  if (!out || !aligned(out, 16)) return set_error(kErrInvalid, "mx_decode: out must be 16-byte aligned");
  const int64_t R = x.k_major ? rows : K, C = x.k_major ? K : rows;
  const int64_t chunks = batch * R * (C / 8);
  if (chunks > INT32_MAX || batch * R > INT32_MAX) return set_error(kErrInvalid, "mx_decode: operand too large");
  const MxOpArgs o = args_of(x);
  const bool km = x.k_major != 0;
  switch (dec_of(x)) {
    case kPlain: return launch_decode<kPlain>(km, o, out, (int)R, (int)C, (uint32_t)chunks, stream);
    case kScale: return launch_decode<kScale>(km, o, out, (int)R, (int)C, (uint32_t)chunks, stream);
    case kCode: return launch_decode<kCode>(km, o, out, (int)R, (int)C, (uint32_t)chunks, stream);
    default: return launch_decode<kCodeScale>(km, o, out, (int)R, (int)C, (uint32_t)chunks, stream);
  }
}

}  // namespace vqx
