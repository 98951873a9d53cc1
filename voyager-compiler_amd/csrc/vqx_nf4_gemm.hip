// NF4-dequant-fused linear:  out[M, N] = A[M, K] . W[N, K]^T (+ bias)
// with W[n, k] = bf16(level[code[n, k]] * scale[n, k / 64]) decoded on the fly
// (the weight decode of linear_mx, src/voyager_compiler/ops/quantized.py:
// 319-326, fused into the product of :330-331).  bf16 MFMA
// (v_mfma_f32_32x32x16_bf16), fp32 accumulation, bf16 output.
//
// Tiling: a workgroup of 256 threads (4 waves) computes a 256 x 128 tile of
// out; wave w owns rows 64w .. 64w+63 and all 128 columns (2 x 4 MFMA tiles of
// 32 x 32).  The K loop steps by 64 (one NF4 scale block).
//  * A never touches LDS: each wave's rows are private to it, so its MFMA
//    operands are loaded straight from global memory (one 16-byte load per
//    lane per fragment), one k-step ahead in registers.
//  * W is decoded once per workgroup into LDS (128 x 64 bf16 = 16 KiB per
//    step, 16-byte chunks XOR-swizzled by row): each thread turns 32 codes per
//    step into bf16 with a v_perm byte-table lookup of the levels, the fp32
//    product with the block scale and RNE.  A ring of three LDS buffers lets
//    the decode run two k-steps ahead of the MFMAs, so one barrier per step
//    suffices and the next step's first fragments are already in registers
//    when it starts.
//  * The MFMA takes the W fragment as its first operand, so each lane ends
//    with four consecutive output columns per group: 8-byte stores.
// Workgroups are ordered so each XCD runs whole 256-row slabs of A, which stay
// in its L2 while W streams past.
#include <type_traits>

#include "vqx_kernels.h"

namespace vqx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kBM = 256, kBN = 128, kBK = 64;
constexpr int kThreads = 256;
constexpr int kWTile = kBN * kBK * 2;  // decoded W bytes per k-step
constexpr int kWBufs = 3;

// byte offset of 16-byte chunk c (0..7) of row r in a [rows][64] bf16 tile
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t c) { return r * 128u + ((c ^ (r & 7u)) << 4); }

// Decode 8 codes (one dword: byte i holds codes 2i (low nibble), 2i+1) into
// four bf16 pairs in k order.  hl/hh: level high bytes for codes 0-7 / 8-15
// (as two dwords each: bytes 0-3 and 4-7), ll/lh likewise for the low bytes.
struct LevelBytes {
  uint32_t h0, h1, h2, h3;  // high bytes of levels 0-3, 4-7, 8-11, 12-15
  uint32_t l0, l1, l2, l3;  // low bytes
};

__device__ __forceinline__ void lookup4(uint32_t nib, const LevelBytes& lb, uint32_t& hi, uint32_t& lo) {
  // nib: four 4-bit codes, one per byte.  v_perm picks bytes 0-7 of a pair of
  // dwords; the code's bit 3 chooses between the 0-7 and 8-15 tables.
  uint32_t sel = nib & 0x07070707u;
  uint32_t m = ((nib >> 3) & 0x01010101u) * 0xFFu;
  uint32_t ha = __builtin_amdgcn_perm(lb.h1, lb.h0, sel);
  uint32_t hb = __builtin_amdgcn_perm(lb.h3, lb.h2, sel);
  uint32_t la = __builtin_amdgcn_perm(lb.l1, lb.l0, sel);
  uint32_t lbb = __builtin_amdgcn_perm(lb.l3, lb.l2, sel);
  hi = (hb & m) | (ha & ~m);
  lo = (lbb & m) | (la & ~m);
}

// 8 codes -> 4 dwords of bf16 pairs = bf16(level * s), k ascending.
__device__ __forceinline__ void decode8(uint32_t w, float s, const LevelBytes& lb, uint32_t (&out)[4]) {
  uint32_t he, le, ho, lo;
  lookup4(w & 0x0F0F0F0Fu, lb, he, le);         // even k: codes 0, 2, 4, 6
  lookup4((w >> 4) & 0x0F0F0F0Fu, lb, ho, lo);  // odd k:  codes 1, 3, 5, 7
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // fp32 of the levels: level bf16 in the high half
    uint32_t se = 0x00000C0Cu | ((4u + i) << 24) | ((uint32_t)i << 16);  // bytes: 0, 0, le[i], he[i]
    float ve = u2f(__builtin_amdgcn_perm(he, le, se));
    float vo = u2f(__builtin_amdgcn_perm(ho, lo, se));
    out[i] = pack_bf16x2(ve * s, vo * s);
  }
}

// LDS-only workgroup barrier: waits for this wave's LDS traffic, not for the
// global loads still in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__global__ __launch_bounds__(kThreads) void nf4_gemm_kernel(const uint16_t* __restrict__ A,
                                                             const uint8_t* __restrict__ codes,
                                                             const float* __restrict__ scale,
                                                             const uint16_t* __restrict__ levels,
                                                             const uint16_t* __restrict__ bias,
                                                             uint16_t* __restrict__ out, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) uint8_t wl[kWBufs * kWTile];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lr = lane & 31;  // fragment row within a 32-tile
  const int lk = lane >> 5;  // which 8-wide k group

  // XCD-aware tile order: consecutive workgroup ids go round-robin over the 8
  // XCDs; give each XCD a contiguous range of tiles, M-major, so an XCD works
  // through whole A slabs.
  const int ntn = N / kBN, ntm = M / kBM;
  const int ntiles = ntn * ntm;
  int bid = blockIdx.x;
  int per_xcd = (ntiles + 7) / 8;
  int tile = (bid & 7) * per_xcd + (bid >> 3);
  if (ntiles % 8 != 0) tile = bid;  // uneven split: plain order
  if (tile >= ntiles) return;
  const int tm = tile / ntn, tn = tile % ntn;
  const int m0 = tm * kBM, n0 = tn * kBN;

  // level byte tables (uniform)
  LevelBytes lb;
  {
    uint32_t hb[4] = {0, 0, 0, 0}, lbv[4] = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      uint32_t v = levels[c];
      hb[c >> 2] |= ((v >> 8) & 0xFFu) << (8 * (c & 3));
      lbv[c >> 2] |= (v & 0xFFu) << (8 * (c & 3));
    }
    lb.h0 = hb[0]; lb.h1 = hb[1]; lb.h2 = hb[2]; lb.h3 = hb[3];
    lb.l0 = lbv[0]; lb.l1 = lbv[1]; lb.l2 = lbv[2]; lb.l3 = lbv[3];
  }

  const int nk = K / kBK;
  const int kb = K / 64;  // scale blocks per row

  // A fragment (i, kk) of a step: lane (lr, lk) holds
  // A[m0 + 64 wave + 32 i + lr][64 ks + 16 kk + 8 lk .. +8]; stored as a[2 kk + i].
  const uint16_t* ap = A + (size_t)(m0 + wave * 64 + lr) * K + lk * 8;
  const size_t a32 = (size_t)32 * K;
  // W decode assignment: row wr, codes for k 32 wh .. 32 wh + 31 of a step
  const int wr = tid >> 1, wh = tid & 1;
  const uint8_t* wsrc = codes + (size_t)(n0 + wr) * (K / 2) + wh * 16;
  const float* ssrc = scale + (size_t)(n0 + wr) * kb;

  auto load_a = [&](u32x4(&a)[8], int ks) {
    const uint16_t* p = ap + (size_t)ks * kBK;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      a[2 * kk] = *reinterpret_cast<const u32x4*>(p + kk * 16);
      a[2 * kk + 1] = *reinterpret_cast<const u32x4*>(p + a32 + kk * 16);
    }
  };
  auto decode_store = [&](uint32_t base, uint32_t w, float s, int j) {
    uint32_t o[4];
    decode8(w, s, lb, o);
    u32x4 v = {o[0], o[1], o[2], o[3]};
    *reinterpret_cast<u32x4*>(wl + base + swz(wr, wh * 4 + j)) = v;
  };
  auto read_b = [&](bf16x8(&b)[4], uint32_t base, int kk) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      b[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(wl + base + swz(j * 32 + lr, kk * 2 + lk)));
  };

  f32x16 acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  auto mma = [&](const bf16x8(&b)[4], const u32x4(&a)[8], int kk) {
    bf16x8 a0 = __builtin_bit_cast(bf16x8, a[2 * kk]);
    bf16x8 a1 = __builtin_bit_cast(bf16x8, a[2 * kk + 1]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[j], a0, acc[0][j], 0, 0, 0);
      acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[j], a1, acc[1][j], 0, 0, 0);
    }
  };

  // codes in flight: wc/ws hold the codes of step ks + 2 while step ks runs
  u32x4 wc;
  float ws;
  // prologue: W of steps 0 and 1 decoded into buffers 0 and 1, A of step 0
  // and the codes of step 2 in flight, fragments of step 0, kk 0 read
  u32x4 a0[8], a1[8];
  bf16x8 bA[4], bB[4];
  load_a(a0, 0);
  {
    u32x4 c0 = *reinterpret_cast<const u32x4*>(wsrc);
    float s0 = ssrc[0];
    u32x4 c1 = c0;
    float s1 = s0;
    if (nk > 1) {
      c1 = *reinterpret_cast<const u32x4*>(wsrc + kBK / 2);
      s1 = ssrc[1];
    }
    if (nk > 2) {
      wc = *reinterpret_cast<const u32x4*>(wsrc + 2 * (kBK / 2));
      ws = ssrc[2];
    }
    decode_store(0, c0.x, s0, 0);
    decode_store(0, c0.y, s0, 1);
    decode_store(0, c0.z, s0, 2);
    decode_store(0, c0.w, s0, 3);
    if (nk > 1) {
      decode_store(kWTile, c1.x, s1, 0);
      decode_store(kWTile, c1.y, s1, 1);
      decode_store(kWTile, c1.z, s1, 2);
      decode_store(kWTile, c1.w, s1, 3);
    }
  }
  lds_barrier();
  read_b(bA, 0, 0);

  // One k-step.  On entry bA holds the kk 0 fragments of step ks and acur its
  // A fragments; on exit bA holds the kk 0 fragments of step ks + 1 and anxt
  // its A fragments.  full: ks + 3 < nk, so every prefetch and decode is live
  // and the step compiles without branches.
  auto step = [&](auto full, int ks, int buf, const u32x4(&acur)[8], u32x4(&anxt)[8]) {
    constexpr bool kFull = decltype(full)::value;
    const uint32_t cur = buf * kWTile;
    const uint32_t nxt = (buf == kWBufs - 1 ? 0 : buf + 1) * kWTile;
    const uint32_t dec = (buf == 0 ? kWBufs - 1 : buf - 1) * kWTile;  // (ks + 2) % 3
    const bool more = kFull || ks + 1 < nk;
    const bool do_dec = kFull || ks + 2 < nk;
    if (more) load_a(anxt, ks + 1);
    const uint32_t w0 = wc.x, w1 = wc.y, w2 = wc.z, w3 = wc.w;
    const float s = ws;
    if (kFull || ks + 3 < nk) {
      wc = *reinterpret_cast<const u32x4*>(wsrc + (size_t)(ks + 3) * (kBK / 2));
      ws = ssrc[ks + 3];
    }
    read_b(bB, cur, 1);
    if (do_dec) decode_store(dec, w0, s, 0);
    mma(bA, acur, 0);
    read_b(bA, cur, 2);
    if (do_dec) decode_store(dec, w1, s, 1);
    mma(bB, acur, 1);
    read_b(bB, cur, 3);
    if (do_dec) decode_store(dec, w2, s, 2);
    mma(bA, acur, 2);
    if (more) read_b(bA, nxt, 0);
    if (do_dec) decode_store(dec, w3, s, 3);
    mma(bB, acur, 3);
    lds_barrier();
  };
  const std::integral_constant<bool, true> kAll;
  const std::integral_constant<bool, false> kChecked;

  int buf = 0;
  int ks = 0;
  for (; ks + 4 < nk; ks += 2) {
    step(kAll, ks, buf, a0, a1);
    buf = buf == kWBufs - 1 ? 0 : buf + 1;
    step(kAll, ks + 1, buf, a1, a0);
    buf = buf == kWBufs - 1 ? 0 : buf + 1;
  }
  for (; ks < nk; ks += 2) {
    step(kChecked, ks, buf, a0, a1);
    buf = buf == kWBufs - 1 ? 0 : buf + 1;
    if (ks + 1 < nk) step(kChecked, ks + 1, buf, a1, a0);
    buf = buf == kWBufs - 1 ? 0 : buf + 1;
  }

  // epilogue: lane holds output row m = lr of each A fragment and columns
  // 8 g + 4 lk .. +3 (g = 0..3) of each W fragment, in acc[i][j][4 g .. 4 g + 3]
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = n0 + j * 32 + 8 * g + 4 * lk;
      float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f, b3 = 0.0f;
      if (bias) {
        u32x2 bb = *reinterpret_cast<const u32x2*>(bias + n);
        b0 = u2f(bb.x << 16);
        b1 = u2f(bb.x & 0xFFFF0000u);
        b2 = u2f(bb.y << 16);
        b3 = u2f(bb.y & 0xFFFF0000u);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int m = m0 + wave * 64 + i * 32 + lr;
        u32x2 o = {pack_bf16x2(acc[i][j][4 * g] + b0, acc[i][j][4 * g + 1] + b1),
                   pack_bf16x2(acc[i][j][4 * g + 2] + b2, acc[i][j][4 * g + 3] + b3)};
        *reinterpret_cast<u32x2*>(out + (size_t)m * N + n) = o;
      }
    }
  }
}

int nf4_gemm(const uint16_t* A, const uint8_t* codes, const float* scale, const uint16_t* levels,
             const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K, hipStream_t st) {
  if (M <= 0 || N <= 0 || K <= 0) return set_error(kErrInvalid, "nf4_gemm: empty shape");
  if (M % kBM || N % kBN || K % kBK)
    return set_error(kErrUnsupported, "nf4_gemm: needs M %% 256 == 0, N %% 128 == 0, K %% 64 == 0 "
                     "(got %lld x %lld x %lld)", (long long)M, (long long)N, (long long)K);
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30)) return set_error(kErrInvalid, "nf4_gemm: shape too large");
  if (!aligned(A, 16) || !aligned(codes, 16) || !aligned(out, 8) || (bias && !aligned(bias, 8)))
    return set_error(kErrInvalid, "nf4_gemm: A and codes must be 16-byte aligned, out and bias 8-byte aligned");
  int ntiles = (int)((M / kBM) * (N / kBN));
  hipLaunchKernelGGL(nf4_gemm_kernel, dim3(ntiles), dim3(kThreads), 0, st, A, codes, scale, levels, bias, out,
                     (int)M, (int)N, (int)K);
  return check_launch("nf4_gemm");
}

}  // namespace vqx
