// NF4-dequant-fused linear:  out[M, N] = A[M, K] . W[N, K]^T (+ bias)
// with W[n, k] = bf16(level[code[n, k]] * scale[n, k / 64]) decoded on the fly
// (the weight decode of linear_mx, src/voyager_compiler/ops/quantized.py:
// 319-326, fused into the product of :330-331).  bf16 MFMA
// (v_mfma_f32_32x32x16_bf16), fp32 accumulation, bf16 output.
//
// Tiling: a workgroup of 512 threads (8 waves, two per SIMD) computes a
// 256 x 128 tile of out; wave w owns the 64 x 64 block at rows 64 (w >> 1),
// columns 64 (w & 1) (2 x 2 MFMA tiles of 32 x 32).  The K loop steps by 64
// (one NF4 scale block) and is unrolled by 3 so every ring index below is
// static.  Two waves per SIMD let one wave's decode VALU and memory
// instructions issue while the other's MFMAs run.
//  * A: a ring of three LDS stages filled two steps ahead of use: fully
//    coalesced 16-byte loads (8 lanes per 128-byte row; wave w loads rows
//    32 w .. 32 w + 31) into registers, written in the swizzled layout one
//    step after the load.
//  * W: decoded once per workgroup into a ring of three LDS buffers two
//    steps ahead (128 x 64 bf16 per step; each thread 16 codes of one row).
//    The quad of lanes on a row shares the row's scale: each lane scales
//    four of the 16 levels (fp32 product, RNE to bf16), DPP broadcasts give
//    every lane the 16 scaled values as v_perm byte tables, and the codes
//    are byte lookups into them.  One barrier per step publishes both rings.
//  * Fragments of both operands are read from LDS one 16-deep k slice ahead
//    of their MFMAs (16-byte chunks XOR-swizzled by row: conflict-free).
//  * The MFMA takes the W fragment as its first operand, so each lane ends
//    with four consecutive output columns per group: 8-byte stores.
// Workgroups are ordered so each XCD runs whole 256-row slabs of A, which stay
// in its L2 while W streams past.  A partial last row tile runs as a launch
// of its own that loads row M - 1 in place of the missing rows and stores
// only rows < M.  M <= 16 takes the skinny kernel further down instead.
#include <mutex>
#include <type_traits>

#include "vqx_kernels.h"

namespace vqx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 128, kBK = 64;
constexpr int kThreads = 512;
constexpr int kWTile = kBN * kBK * 2;  // decoded W bytes per k-step
constexpr int kATile = kBM * kBK * 2;  // A bytes per k-step

// byte offset of 16-byte chunk c (0..7) of row r in a [rows][64] bf16 tile.
// The chunk slot is c ^ (r & 7) ^ ((r >> 3) & 1): for a fixed c, any 8
// aligned consecutive rows use 8 different slots (distinct 16-byte bank
// groups within 128 bytes) and any 16 aligned consecutive rows use 16
// different (row parity, slot) pairs (distinct bank groups within 256 bytes),
// so a fragment read of 32 consecutive rows is conflict free whether LDS
// serves 8 lanes over 32 banks or 16 lanes over 64 banks per cycle.
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t c) {
  return r * 128u + ((c ^ (r & 7u) ^ ((r >> 3) & 1u)) << 4);
}

// Decode 8 codes (one dword: byte i holds codes 2i (low nibble), 2i+1) into
// four bf16 pairs in k order.  hl/hh: level high bytes for codes 0-7 / 8-15
// (as two dwords each: bytes 0-3 and 4-7), ll/lh likewise for the low bytes.
struct LevelBytes {
  uint32_t h0, h1, h2, h3;  // high bytes of levels 0-3, 4-7, 8-11, 12-15
  uint32_t l0, l1, l2, l3;  // low bytes
};

__device__ __forceinline__ void lookup4(uint32_t sel, uint32_t m, const LevelBytes& lb, uint32_t& hi, uint32_t& lo) {
  // sel: four 3-bit code bits 0-2, one per byte; m: 0xFF in the bytes whose
  // code has bit 3 set.  v_perm picks bytes 0-7 of a pair of dwords; m
  // chooses between the tables of codes 0-7 and 8-15.
  uint32_t ha = __builtin_amdgcn_perm(lb.h1, lb.h0, sel);
  uint32_t hb = __builtin_amdgcn_perm(lb.h3, lb.h2, sel);
  uint32_t la = __builtin_amdgcn_perm(lb.l1, lb.l0, sel);
  uint32_t lbb = __builtin_amdgcn_perm(lb.l3, lb.l2, sel);
  hi = (hb & m) | (ha & ~m);
  lo = (lbb & m) | (la & ~m);
}

// Byte masks of bit 7 of each byte of y: v_perm selectors 8, 9, 10, 11
// replicate the sign bit of bytes 1, 3, 5, 7 of the pair {y, y << 8}, i.e.
// of bytes 0, 2, 1, 3 of y.
__device__ __forceinline__ uint32_t byte_sign_mask(uint32_t y) {
  return __builtin_amdgcn_perm(y, y << 8, 0x0B090A08u);
}

// The 16 values bf16(level[c] * s) of one scale block, as high and low byte
// tables in the LevelBytes layout: pair p[i] holds entries 2i (low half) and
// 2i + 1; the high bytes of entries 4j .. 4j + 3 are bytes 1, 3 of p[2j] and
// of p[2j + 1], the low bytes bytes 0, 2.
__device__ __forceinline__ LevelBytes scaled_levels(const float (&lv)[16], float s) {
  uint32_t p[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) p[i] = pack_bf16x2(lv[2 * i] * s, lv[2 * i + 1] * s);
  LevelBytes t;
  t.h0 = __builtin_amdgcn_perm(p[1], p[0], 0x07050301u);
  t.h1 = __builtin_amdgcn_perm(p[3], p[2], 0x07050301u);
  t.h2 = __builtin_amdgcn_perm(p[5], p[4], 0x07050301u);
  t.h3 = __builtin_amdgcn_perm(p[7], p[6], 0x07050301u);
  t.l0 = __builtin_amdgcn_perm(p[1], p[0], 0x06040200u);
  t.l1 = __builtin_amdgcn_perm(p[3], p[2], 0x06040200u);
  t.l2 = __builtin_amdgcn_perm(p[5], p[4], 0x06040200u);
  t.l3 = __builtin_amdgcn_perm(p[7], p[6], 0x06040200u);
  return t;
}

// scaled_levels for the four lanes of a DPP quad that share one scale: lane
// q of the quad scales levels 4 q .. 4 q + 3 (lq, its own four) and builds
// byte tables h_q, l_q; quad broadcasts give every lane all eight.  The
// same bytes as scaled_levels, for a quarter of its products and
// conversions plus 8 DPP moves.
__device__ __forceinline__ LevelBytes quad_scaled_levels(const float (&lq)[4], float s) {
  const uint32_t pa = pack_bf16x2(lq[0] * s, lq[1] * s), pb = pack_bf16x2(lq[2] * s, lq[3] * s);
  const int h = (int)__builtin_amdgcn_perm(pb, pa, 0x07050301u), l = (int)__builtin_amdgcn_perm(pb, pa, 0x06040200u);
  LevelBytes t;
  t.h0 = (uint32_t)__builtin_amdgcn_mov_dpp(h, 0x00, 0xF, 0xF, true);  // quad_perm [0,0,0,0]
  t.h1 = (uint32_t)__builtin_amdgcn_mov_dpp(h, 0x55, 0xF, 0xF, true);  // [1,1,1,1]
  t.h2 = (uint32_t)__builtin_amdgcn_mov_dpp(h, 0xAA, 0xF, 0xF, true);  // [2,2,2,2]
  t.h3 = (uint32_t)__builtin_amdgcn_mov_dpp(h, 0xFF, 0xF, 0xF, true);  // [3,3,3,3]
  t.l0 = (uint32_t)__builtin_amdgcn_mov_dpp(l, 0x00, 0xF, 0xF, true);
  t.l1 = (uint32_t)__builtin_amdgcn_mov_dpp(l, 0x55, 0xF, 0xF, true);
  t.l2 = (uint32_t)__builtin_amdgcn_mov_dpp(l, 0xAA, 0xF, 0xF, true);
  t.l3 = (uint32_t)__builtin_amdgcn_mov_dpp(l, 0xFF, 0xF, 0xF, true);
  return t;
}

// decode8 with the scale already applied (tables from scaled_levels): the
// byte lookups give the final bf16 bytes, which four pairs of v_perm
// interleave into the same k-ascending bf16 pairs decode8 returns.
__device__ __forceinline__ void decode8_scaled(uint32_t w, const LevelBytes& tb, uint32_t (&out)[4]) {
  uint32_t he, le, ho, lo;
  lookup4(w & 0x07070707u, byte_sign_mask(w << 4), tb, he, le);    // codes 0, 2, 4, 6
  lookup4((w >> 4) & 0x07070707u, byte_sign_mask(w), tb, ho, lo);  // codes 1, 3, 5, 7
  const uint32_t e01 = __builtin_amdgcn_perm(he, le, 0x05010400u);  // values of codes 0, 2
  const uint32_t o01 = __builtin_amdgcn_perm(ho, lo, 0x05010400u);  // codes 1, 3
  const uint32_t e23 = __builtin_amdgcn_perm(he, le, 0x07030602u);  // codes 4, 6
  const uint32_t o23 = __builtin_amdgcn_perm(ho, lo, 0x07030602u);  // codes 5, 7
  out[0] = __builtin_amdgcn_perm(o01, e01, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(o01, e01, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(o23, e23, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(o23, e23, 0x07060302u);
}

// LDS-only workgroup barrier: waits for this wave's LDS traffic, not for the
// global loads still in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// k-steps ks0 .. ks0 + nk - 1 of the 256 x 128 tile at rows m0, columns n0,
// into acc (zeroed here).  PARTIAL: rows past M load row M - 1.  Ends with
// an LDS barrier after the last fragment read, so the rings can be refilled
// for another tile right away.  The rings are declared here, so their LDS
// addresses are constants and fold into the instructions' offsets.
template <bool PARTIAL>
__device__ __forceinline__ void tile_steps(const uint16_t* __restrict__ A, const uint8_t* __restrict__ codes,
                                           const float* __restrict__ scale, const uint16_t* __restrict__ levels,
                                           int M, int K, int m0, int n0, int ks0, int nk, f32x16 (&acc)[2][2]) {
  __shared__ __attribute__((aligned(16))) uint8_t wl[3 * kWTile];
  __shared__ __attribute__((aligned(16))) uint8_t al[3 * kATile];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;  // 64-row block
  const int wn = wave & 1;   // 64-column block
  const int lr = lane & 31;  // fragment row within a 32-tile
  const int lk = lane >> 5;  // which 8-wide k group
  const int kb = K / 64;  // scale blocks per row

  // A staging: load q (0..3) of a step covers rows 32 wave + 8 q .. +7, lane
  // L chunk L % 8 of row 32 wave + 8 q + L / 8.  In a partial tile, rows
  // past M load row M - 1 instead; their outputs are not stored.
  const uint16_t* asrc = A + (size_t)(m0 + wave * 32 + (lane >> 3)) * K + (lane & 7) * 8 + (size_t)ks0 * kBK;
  int aoff[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r = m0 + wave * 32 + 8 * q + (lane >> 3);
    aoff[q] = PARTIAL ? ((r < M ? r : M - 1) - (m0 + wave * 32 + (lane >> 3))) * K : 8 * q * K;
  }
  u32x4 areg[4];
  auto load_a = [&](int ks) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if constexpr (PARTIAL)
        areg[q] = *reinterpret_cast<const u32x4*>(asrc + aoff[q] + (size_t)ks * kBK);
      else
        areg[q] = *reinterpret_cast<const u32x4*>(asrc + (size_t)(8 * q) * K + (size_t)ks * kBK);
    }
  };
  auto store_a = [&](uint32_t stage) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<u32x4*>(al + stage + swz(wave * 32 + 8 * q + (lane >> 3), lane & 7)) = areg[q];
  };
  // W decode assignment: row wr, codes for k 16 wq .. 16 wq + 15 of a step.
  // The quad of lanes on one row shares the row's scale: each lane scales
  // four of the levels (lq) and the quad shares the byte tables.
  const int wr = tid >> 2, wq = tid & 3;
  float lq[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) lq[i] = u2f((uint32_t)levels[4 * wq + i] << 16);
  const uint8_t* wsrc = codes + (size_t)(n0 + wr) * (K / 2) + wq * 8 + (size_t)ks0 * (kBK / 2);
  const float* ssrc = scale + (size_t)(n0 + wr) * kb + ks0;

  auto decode_store = [&](uint32_t base, uint32_t w, const LevelBytes& tb, int j) {
    uint32_t o[4];
    decode8_scaled(w, tb, o);
    u32x4 v = {o[0], o[1], o[2], o[3]};
    *reinterpret_cast<u32x4*>(wl + base + swz(wr, wq * 2 + j)) = v;
  };
  auto read_b = [&](bf16x8(&b)[2], uint32_t base, int kk) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      b[j] = __builtin_bit_cast(bf16x8,
                                *reinterpret_cast<const u32x4*>(wl + base + swz(wn * 64 + j * 32 + lr, kk * 2 + lk)));
  };
  auto read_a = [&](bf16x8(&a)[2], uint32_t base, int kk) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      a[i] = __builtin_bit_cast(bf16x8,
                                *reinterpret_cast<const u32x4*>(al + base + swz(wm * 64 + i * 32 + lr, kk * 2 + lk)));
  };

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  auto mma = [&](const bf16x8(&b)[2], const bf16x8(&a)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      acc[0][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[j], a[0], acc[0][j], 0, 0, 0);
      acc[1][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[j], a[1], acc[1][j], 0, 0, 0);
    }
  };

  // codes in flight, one slot per step mod 3: step ks decodes the codes of
  // step ks + 2 from its slot and, once they are consumed, reloads the slot
  // with those of step ks + 5 (no register copies, so no early waits)
  u32x2 wc0 = {0, 0}, wc1 = {0, 0}, wc2 = {0, 0};
  float ws0 = 0.0f, ws1 = 0.0f, ws2 = 0.0f;
  auto load_codes = [&](u32x2& c, float& sc, int ks) {
    c = *reinterpret_cast<const u32x2*>(wsrc + (size_t)ks * (kBK / 2));
    sc = ssrc[ks];
  };

  // prologue: A of steps 0 and 1 staged and of step 2 in registers, W of
  // steps 0 and 1 decoded, the codes of steps 2..4 in flight, fragments of
  // step 0, first slice, read
  load_a(0);
  store_a(0);
  if (nk > 1) {
    load_a(1);
    store_a(kATile);
  }
  if (nk > 2) load_a(2);
  {
    u32x2 c0, c1 = {0, 0};
    float s0, s1 = 0.0f;
    load_codes(c0, s0, 0);
    if (nk > 1) load_codes(c1, s1, 1);
    if (nk > 2) load_codes(wc0, ws0, 2);
    if (nk > 3) load_codes(wc1, ws1, 3);
    if (nk > 4) load_codes(wc2, ws2, 4);
    const LevelBytes t0 = quad_scaled_levels(lq, s0);
    decode_store(0, c0.x, t0, 0);
    decode_store(0, c0.y, t0, 1);
    if (nk > 1) {
      const LevelBytes t1 = quad_scaled_levels(lq, s1);
      decode_store(kWTile, c1.x, t1, 0);
      decode_store(kWTile, c1.y, t1, 1);
    }
  }
  lds_barrier();
  bf16x8 bA[2], bB[2], aA[2], aB[2];
  read_b(bA, 0, 0);
  read_a(aA, 0, 0);

  // One k-step; T = ks % 3 selects the ring slots.  On entry bA/aA hold the
  // kk 0 fragments of step ks; on exit those of step ks + 1.  full:
  // ks + 5 < nk, so every prefetch and decode is live and the step compiles
  // without branches.
  //
  // Issue order: each kk first sends the LDS reads of the next kk's
  // fragments, then a scheduling fence, then its 4 MFMAs alternating with
  // the VALU of the decode (kk 0 and 2) or the A staging (kk 1) or the code
  // loads (kk 3); the fences keep the compiler from sinking the fragment
  // reads next to their MFMAs.
  auto step = [&](auto full, auto tt, int ks, u32x2& wc, float& ws) {
    constexpr bool kFull = decltype(full)::value;
    constexpr int T = decltype(tt)::value;
    constexpr uint32_t a_cur = T * kATile, a_nxt = ((T + 1) % 3) * kATile, a_new = ((T + 2) % 3) * kATile;
    constexpr uint32_t w_cur = T * kWTile, w_nxt = ((T + 1) % 3) * kWTile, w_new = ((T + 2) % 3) * kWTile;
    const bool more = kFull || ks + 1 < nk;
    const bool ahead2 = kFull || ks + 2 < nk;
    const uint32_t w0 = wc.x, w1 = wc.y;
    LevelBytes tb;  // the step's scaled tables, built before its first decode
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      bf16x8(&bcur)[2] = (kk & 1) ? bB : bA;
      bf16x8(&bnext)[2] = (kk & 1) ? bA : bB;
      bf16x8(&acur)[2] = (kk & 1) ? aB : aA;
      bf16x8(&anext)[2] = (kk & 1) ? aA : aB;
      if (kk < 3) {
        read_b(bnext, w_cur, kk + 1);
        read_a(anext, a_cur, kk + 1);
      } else if (more) {
        read_b(bnext, w_nxt, 0);
        read_a(anext, a_nxt, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (kk == 0 && ahead2) {
        tb = quad_scaled_levels(lq, ws);
        decode_store(w_new, w0, tb, 0);
      }
      if (kk == 2 && ahead2) decode_store(w_new, w1, tb, 1);
      mma(bcur, acur);
      if (kk == 1) {
        if (ahead2) store_a(a_new);  // A of step ks + 2, loaded during step ks - 1
        __builtin_amdgcn_sched_barrier(0);
        if (kFull || ks + 3 < nk) load_a(ks + 3);
      }
      if (kk == 3 && (kFull || ks + 5 < nk)) load_codes(wc, ws, ks + 5);
      if constexpr (kFull) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // VALU
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    lds_barrier();
  };
  const std::integral_constant<bool, true> kAll;
  const std::integral_constant<bool, false> kChecked;
  const std::integral_constant<int, 0> k0;
  const std::integral_constant<int, 1> k1;
  const std::integral_constant<int, 2> k2;

  int ks = 0;
  for (; ks + 7 < nk; ks += 3) {
    step(kAll, k0, ks, wc0, ws0);
    step(kAll, k1, ks + 1, wc1, ws1);
    step(kAll, k2, ks + 2, wc2, ws2);
  }
  for (; ks < nk; ks += 3) {
    step(kChecked, k0, ks, wc0, ws0);
    if (ks + 1 < nk) step(kChecked, k1, ks + 1, wc1, ws1);
    if (ks + 2 < nk) step(kChecked, k2, ks + 2, wc2, ws2);
  }

}

// Output of one tile: lane holds output row m = lr of each A fragment and
// columns 8 g + 4 lk .. +3 (g = 0..3) of each W fragment, in
// acc[i][j][4 g .. 4 g + 3]; bf16 (RNE) of acc + bias, rows < M only when
// PARTIAL.
template <bool PARTIAL>
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[2][2], const uint16_t* __restrict__ bias,
                                           uint16_t* __restrict__ out, int M, int N, int m0, int n0) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1, lr = lane & 31, lk = lane >> 5;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int n = n0 + wn * 64 + j * 32 + 8 * g + 4 * lk;
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
        const int m = m0 + wm * 64 + i * 32 + lr;
        u32x2 o = {pack_bf16x2(acc[i][j][4 * g] + b0, acc[i][j][4 * g + 1] + b1),
                   pack_bf16x2(acc[i][j][4 * g + 2] + b2, acc[i][j][4 * g + 3] + b3)};
        if (!PARTIAL || m < M) *reinterpret_cast<u32x2*>(out + (size_t)m * N + n) = o;
      }
    }
  }
}

// Whole tiles, one per workgroup.  PARTIAL: the launch covers the one row
// tile starting at row m_base with fewer than 256 rows left; otherwise it
// covers the first ntiles full tiles from row m_base, M-major.  zero/nzero:
// counters of a stream-K launch that follows on the same stream, cleared by
// workgroup 0 after its tile (stores ahead of the k loop would make the
// compiler's memory-counter waits inside it more conservative).
template <bool PARTIAL>
__global__ __launch_bounds__(kThreads) void nf4_gemm_kernel(const uint16_t* __restrict__ A,
                                                             const uint8_t* __restrict__ codes,
                                                             const float* __restrict__ scale,
                                                             const uint16_t* __restrict__ levels,
                                                             const uint16_t* __restrict__ bias,
                                                             uint16_t* __restrict__ out, int M, int N, int K,
                                                             int m_base, int ntiles, int* __restrict__ zero,
                                                             int nzero) {
  // XCD-aware tile order: consecutive workgroup ids go round-robin over the 8
  // XCDs; give each XCD a contiguous range of tiles, M-major, so an XCD works
  // through whole A slabs.
  const int ntn = N / kBN;
  int bid = blockIdx.x;
  int per_xcd = (ntiles + 7) / 8;
  int tile = (bid & 7) * per_xcd + (bid >> 3);
  if (ntiles % 8 != 0) tile = bid;  // uneven split: plain order
  if (tile >= ntiles) return;
  const int m0 = m_base + (tile / ntn) * kBM, n0 = (tile % ntn) * kBN;
  f32x16 acc[2][2];
  tile_steps<PARTIAL>(A, codes, scale, levels, M, K, m0, n0, 0, K / kBK, acc);
  store_tile<PARTIAL>(acc, bias, out, M, N, m0, n0);
  if (zero && blockIdx.x == 0)
    for (int i = threadIdx.x; i < nzero; i += kThreads) zero[i] = 0;
}

// Stream-K tail: the last sk_tiles full tiles (from tile index tile_base,
// M-major) as sk_tiles * nk k-steps split evenly over the gridDim.x
// workgroups: workgroup i takes steps [U i / g, U (i + 1) / g) of the
// tile-major step sequence (U = sk_tiles * nk, g = gridDim.x), i.e. the end
// of one tile, possibly whole tiles, and the start of another.  A whole tile
// is stored directly.  A piece of a tile leaves its fp32 sums in the
// workspace, slot 2 i for the workgroup's first tile and 2 i + 1 for its last
// (slot layout: float pair q of thread t at (q * 512 + t) * 2), then bumps the
// tile's counter; the workgroup that brings the counter to the number of
// contributors adds the slots in contributor order (so the result does not
// depend on which one arrives last), adds the bias and stores the tile.
// Nothing waits on another workgroup.  The counters start at zero (cleared
// by the launch before this one on the stream).
//
// The slots are written and read with device-scope atomic stores and loads,
// which the hardware keeps coherent across the XCDs' separate L2 caches at
// the access itself (the sc1 policy).  A device-scope fence would instead
// write back (release) or invalidate (acquire) the whole L2 of the XCD, in
// every wave of every piece, and cost the other workgroups there their
// cached operands.  Each wave waits for its slot stores to complete before
// the workgroup barrier that precedes the counter increment, and the
// finisher issues its slot loads only after it has read the counter.
constexpr int kPartFloats = kBM * kBN;  // one tile of fp32 sums
constexpr int kMaxContrib = 6;          // workgroups sharing one tile, at most (the plan ensures it)

__device__ __forceinline__ int sk_group_of(int64_t step, int g, int64_t U) {
  return (int)(((step + 1) * g - 1) / U);  // the workgroup whose range holds step
}

__global__ __launch_bounds__(kThreads) void nf4_gemm_sk_kernel(const uint16_t* __restrict__ A,
                                                                const uint8_t* __restrict__ codes,
                                                                const float* __restrict__ scale,
                                                                const uint16_t* __restrict__ levels,
                                                                const uint16_t* __restrict__ bias,
                                                                uint16_t* __restrict__ out, int M, int N, int K,
                                                                int tile_base, int sk_tiles, float* __restrict__ part,
                                                                int* __restrict__ cnt) {
  __shared__ int s_arrived;
  const int tid = threadIdx.x;
  // workgroup ids go round-robin over the 8 XCDs: renumber them so each XCD
  // runs a contiguous run of ranges (the pieces of one tile on one XCD, its
  // operands in that XCD's L2)
  const int g = gridDim.x;
  const int me = g % 8 == 0 ? (int)(blockIdx.x & 7) * (g >> 3) + (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const int nk = K / kBK, ntn = N / kBN;
  const int64_t U = (int64_t)sk_tiles * nk;
  const int64_t u0 = U * me / g, u1 = U * (me + 1) / g;
  const int t_first = (int)(u0 / nk);
  for (int64_t u = u0; u < u1;) {
    const int t = (int)(u / nk);
    const int k_lo = (int)(u - (int64_t)t * nk);
    const int k_hi = (int)((u1 - (int64_t)t * nk) < nk ? (u1 - (int64_t)t * nk) : nk);
    const int tile = tile_base + t;
    const int m0 = (tile / ntn) * kBM, n0 = (tile % ntn) * kBN;
    f32x16 acc[2][2];
    tile_steps<false>(A, codes, scale, levels, M, K, m0, n0, k_lo, k_hi - k_lo, acc);
    u = (int64_t)(t + 1) * nk;
    if (k_lo == 0 && k_hi == nk) {
      store_tile<false>(acc, bias, out, M, N, m0, n0);
      continue;
    }
    uint64_t* mine = reinterpret_cast<uint64_t*>(part + (size_t)(2 * me + (t == t_first ? 0 : 1)) * kPartFloats);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const f32x2 v = {acc[i][j][2 * q], acc[i][j][2 * q + 1]};
          __hip_atomic_store(mine + (size_t)((i * 2 + j) * 8 + q) * kThreads + tid, __builtin_bit_cast(uint64_t, v),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's slot stores have completed
    __syncthreads();
    const int c_first = sk_group_of((int64_t)t * nk, g, U);
    const int c_last = sk_group_of((int64_t)t * nk + nk - 1, g, U);
    if (tid == 0) s_arrived = __hip_atomic_fetch_add(cnt + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (s_arrived != c_last - c_first) continue;  // another contributor is still running
    // the slots in contributor order (32 loads of one slot in flight at a time)
    f32x16 tot[2][2] = {};
    for (int c = c_first; c <= c_last; ++c) {
      const int tf = (int)((U * c / g) / nk);
      const uint64_t* src = reinterpret_cast<const uint64_t*>(part + (size_t)(2 * c + (t == tf ? 0 : 1)) * kPartFloats);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int q = 0; q < 8; ++q) {
            f32x2 v;
            if (c == me) {
              v = f32x2{acc[i][j][2 * q], acc[i][j][2 * q + 1]};
            } else {
              v = __builtin_bit_cast(f32x2, __hip_atomic_load(src + (size_t)((i * 2 + j) * 8 + q) * kThreads + tid,
                                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            }
#pragma unroll
            for (int e = 0; e < 2; ++e) tot[i][j][2 * q + e] = c == c_first ? v[e] : tot[i][j][2 * q + e] + v[e];
          }
    }
    store_tile<false>(tot, bias, out, M, N, m0, n0);
  }
}

__global__ void nf4_zero_counters(int* __restrict__ cnt, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) cnt[i] = 0;
}

// ---------------------------------------------------------------------------
// Skinny form for M <= 16 (decode-time batches).  Each wave computes a
// 16 x 16 output tile (all of A's rows, padded to 16; 16 output columns)
// over a quarter of K with v_mfma_f32_16x16x32_bf16; the workgroup's 4 waves
// take the 4 quarters of K for the same columns and add their tiles in LDS in
// wave (k) order.  Per 128-k step lane l loads 32 codes (16 bytes) of its
// column's W row and the 32 matching A values (64 bytes) of its A row, for
// row / column l % 16 and k = 128 s + 32 (l / 16) .. +31; MFMA c (0..3) of
// the step takes the lane's k 32 (l / 16) + 8 c .. + 7 from both operands (one
// permutation of k for both, so every product pairs the same k).  W is
// decoded exactly as in the tile kernel (bf16(level * scale)).  The MFMAs
// are idle most of the time: the decode's VALU and the weight's bytes bound
// the kernel.
// ---------------------------------------------------------------------------
// Waves per workgroup (each a 1/W share of K): 4, or 8 / 16 when N is too
// small for 16-column workgroups of 4 waves to give every CU about eight
// waves (N = 4096 at M = 1: 256 workgroups).
constexpr int kSkinnyWavesMin = 4, kSkinnyWavesMax = 16;

// scaled_levels for two 16-lane rows that share one scale (rows 2 j and
// 2 j + 1 of the wave): the even row scales levels 0-7, the odd row levels
// 8-15 (lh, the row's own eight) and v_permlane16_swap gives both rows all
// sixteen.  The same bytes as scaled_levels, for half its products and
// conversions plus 4 swaps.
__device__ __forceinline__ LevelBytes row_pair_scaled_levels(const float (&lh)[8], float s) {
  const uint32_t p0 = pack_bf16x2(lh[0] * s, lh[1] * s), p1 = pack_bf16x2(lh[2] * s, lh[3] * s);
  const uint32_t p2 = pack_bf16x2(lh[4] * s, lh[5] * s), p3 = pack_bf16x2(lh[6] * s, lh[7] * s);
  const uint32_t ha = __builtin_amdgcn_perm(p1, p0, 0x07050301u), hb = __builtin_amdgcn_perm(p3, p2, 0x07050301u);
  const uint32_t la = __builtin_amdgcn_perm(p1, p0, 0x06040200u), lb = __builtin_amdgcn_perm(p3, p2, 0x06040200u);
  // r[0]: the even row's value, r[1]: the odd row's, in every lane
  const auto xha = __builtin_amdgcn_permlane16_swap(ha, ha, false, false);
  const auto xhb = __builtin_amdgcn_permlane16_swap(hb, hb, false, false);
  const auto xla = __builtin_amdgcn_permlane16_swap(la, la, false, false);
  const auto xlb = __builtin_amdgcn_permlane16_swap(lb, lb, false, false);
  LevelBytes t;
  t.h0 = xha[0];
  t.h1 = xhb[0];
  t.h2 = xha[1];
  t.h3 = xhb[1];
  t.l0 = xla[0];
  t.l1 = xlb[0];
  t.l2 = xla[1];
  t.l3 = xlb[1];
  return t;
}

template <int W>
__global__ __launch_bounds__(64 * W) void nf4_skinny_kernel(const uint16_t* __restrict__ A,
                                                                        const uint8_t* __restrict__ codes,
                                                                        const float* __restrict__ scale,
                                                                        const uint16_t* __restrict__ levels,
                                                                        const uint16_t* __restrict__ bias,
                                                                        uint16_t* __restrict__ out, int M, int N,
                                                                        int K) {
  __shared__ float part[W][16][16];  // [wave][row m][column]
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int nn = n0 + r < N ? n0 + r : N - 1;
  const int mm = r < M ? r : M - 1;
  const int kb = K / 64;
  const int steps = (K + 127) / 128;
  const int s0 = steps * wave / W, s1 = steps * (wave + 1) / W;
  float lh[8];  // the row's eight levels as fp32: 0-7 in even 16-lane rows, 8-15 in odd
#pragma unroll
  for (int c = 0; c < 8; ++c) lh[c] = u2f((uint32_t)levels[c + 8 * (g & 1)] << 16);
  const uint8_t* wrow = codes + (size_t)nn * (K / 2);
  const float* srow = scale + (size_t)nn * kb;
  const uint16_t* arow = A + (size_t)mm * K;
  f32x4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
  // One 128-k step.  CHECK: the step may reach past K (K % 64 == 0, so a
  // 32-k group is either wholly inside K or wholly past it: the last step of
  // an odd number of 64-blocks); past it A = 0 and the loads are clamped to
  // the last group.  Only that step is checked.
  auto step = [&](int st, auto check) {
    constexpr bool kCheck = decltype(check)::value;
    const int k = st * 128 + g * 32;
    const bool kok = !kCheck || k < K;
    const int kk = kok ? k : K - 32;
    const u32x4 w = *reinterpret_cast<const u32x4*>(wrow + kk / 2);
    const float sc = srow[kk / 64];
    u32x4 a[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      a[c] = *reinterpret_cast<const u32x4*>(arow + kk + 8 * c);
      if (kCheck && !kok) a[c] = u32x4{0u, 0u, 0u, 0u};
    }
    // the lane's 32 codes share one scale block with those of the other row
    // of its row pair (k 64-aligned): scale the 16 levels once per pair
    const LevelBytes tb = row_pair_scaled_levels(lh, sc);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint32_t o[4];
      decode8_scaled(w[c], tb, o);
      const u32x4 b = {o[0], o[1], o[2], o[3]};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[c]), __builtin_bit_cast(bf16x8, b),
                                                    acc, 0, 0, 0);
    }
  };
  const int whole = K / 128;  // steps wholly inside K
  const int s_end = s1 < whole ? s1 : whole;
  for (int st = s0; st < s_end; ++st) step(st, std::false_type{});
  for (int st = s_end > s0 ? s_end : s0; st < s1; ++st) step(st, std::true_type{});
  // lane holds rows 4 (l / 16) .. + 3 of column l % 16
#pragma unroll
  for (int j = 0; j < 4; ++j) part[wave][4 * g + j][r] = acc[j];
  __syncthreads();
  if (threadIdx.x < 256) {
    const int t = threadIdx.x, m = t >> 4, c = t & 15;
    float v = part[0][m][c];
#pragma unroll
    for (int w = 1; w < W; ++w) v += part[w][m][c];
    const int n = n0 + c;
    if (m < M && n < N) {
      const float b = bias ? u2f((uint32_t)bias[n] << 16) : 0.0f;
      out[(size_t)m * N + n] = (uint16_t)f2bf(v + b);
    }
  }
}

// Stream-K plan for the full tiles of an M > 16 product: when the tile count
// is not a multiple of the CU count, the tiles of the last, partly filled
// round are split into k-step ranges over up to one workgroup per CU, at
// least max(16, nk / 4) steps each.  A split tile costs each workgroup a
// second pipeline fill and the fp32 exchange, about 20 us at K = 4096
// (measured: 81 us for 44-step ranges against 61 us of steps), so the split
// is taken only when a range is at least kSkSaving steps shorter than a
// whole tile: C5's last round (176 of 256 CUs, 44-step ranges) stays whole
// tiles (measured even), a 256-row product (86 tiles, 22-step ranges) splits
// (51 us against 66 us).  dp_tiles run first, one per workgroup.
struct SkPlan {
  int64_t dp_tiles = 0, sk_tiles = 0, groups = 0, bytes = 0;
};

constexpr int64_t kCounterBytes = 256;  // alignment of the counter block
constexpr int64_t kSkSaving = 24;       // k-steps a split must save over a whole tile

static SkPlan plan_stream_k(int64_t M, int64_t N, int64_t K) {
  SkPlan p;
  if (M <= 16 || N % kBN || K % kBK || K <= 0) return p;
  const int64_t tiles = (M / kBM) * (N / kBN), nk = K / kBK;
  const int64_t cus = num_cus();
  p.dp_tiles = tiles;
  const int64_t rem = tiles % cus;
  if (rem == 0) return p;
  const int64_t U = rem * nk, min_steps = nk / 4 > 16 ? nk / 4 : 16;
  const int64_t g = U / min_steps < cus ? U / min_steps : cus;
  if (g < 1 || (U + g - 1) / g + kSkSaving > nk) return p;
  // a tile meets at most ceil(nk / shortest range) + 1 ranges
  if ((nk + U / g - 1) / (U / g) + 1 > kMaxContrib) return p;
  p.dp_tiles = tiles - rem;
  p.sk_tiles = rem;
  p.groups = g;
  p.bytes = (rem * 4 + kCounterBytes - 1) / kCounterBytes * kCounterBytes + 2 * g * kPartFloats * 4;
  return p;
}

int64_t nf4_gemm_workspace(int64_t M, int64_t N, int64_t K) { return plan_stream_k(M, N, K).bytes; }

// ---------------------------------------------------------------------------
// Allocation-free form of nf4_gemm with a workspace: the workspace is
// `scratch`, a device array of this library that each GPU holds for the
// life of the process.  Its size covers every stream-K plan on a device of up
// to 256 CUs: two 256 x 128 fp32 partial tiles per CU plus the tile counters
// (64 MiB + 1 KiB).  A plan that needs more (a device with more CUs) is
// rejected.  In host code `scratch` names a host-side stand-in, so kernels get
// its device address, looked up once per device with that device current.
// Every call on one device shares the array: the counters are cleared on the
// stream ahead of the split launch (by nf4_gemm, as with a caller's
// workspace), the partial slots need no initial contents, and calls that
// overlap on one device race.
// ---------------------------------------------------------------------------
constexpr int64_t kScratchBytes = (64ll << 20) + 1024;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

static int scratch_of_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(kErrLaunch, "nf4_linear_noalloc: no current device (or device index >= %d)", kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(kErrLaunch, "nf4_linear_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return kOk;
}

int nf4_gemm_noalloc(const uint16_t* A, const uint8_t* codes, const float* scale, const uint16_t* levels,
                     const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K, hipStream_t st) {
  const int64_t need = plan_stream_k(M, N, K).bytes;
  if (need > kScratchBytes)
    return set_error(kErrUnsupported, "nf4_linear_noalloc: this shape needs %lld bytes of scratch, the maximum is %lld",
                     (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_of_current_device(&ws);
  if (rc != kOk) return rc;
  return nf4_gemm(A, codes, scale, levels, bias, out, M, N, K, need > 0 ? ws : nullptr, need > 0 ? kScratchBytes : 0,
                  st);
}

// ---------------------------------------------------------------------------
// The packed operands from linear_mx's convert format
// (src/vc/quantization/quantize_pt2e.py:456-508: the weight holds integer-
// valued code indices in a float tensor, weight_code the levels, weight_scale
// one value per 64-element block along K).  The index of element (n, k) is
// trunc(w) (torch's .to(long)); a negative index counts from the end of the
// code table, as torch's indexing does (quantized.py:319-320).  A NaN, an
// infinity or an index outside the table sets *bad: the reference raises
// IndexError there, and the caller takes the unfused path.  transposed: the
// weight is stored [K, N] ("ck") with its scale [K/64, N]; otherwise [N, K]
// and [N, K/64].  One 64 (n) x 64 (k) tile per loop trip: thread t packs 16
// codes of column n0 + t / 4, from its own loads ([N, K]) or through an LDS
// transpose ([K, N]); threads 0-63 convert the tile's 64 scales to fp32.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float elem_as_f32(const void* p, int dt, int64_t i) {
  if (dt == kF32) return static_cast<const float*>(p)[i];
  const uint32_t h = static_cast<const uint16_t*>(p)[i];
  return dt == kBF16 ? bf2f(h) : h2f_exact(h);
}

__device__ __forceinline__ uint32_t code_index(float v, int ncode, bool& bad) {
  // |v| < ncode + 1 keeps the truncation in int range and fails NaN / Inf
  if (!(__builtin_fabsf(v) < (float)(ncode + 1))) {
    bad = true;
    return 0;
  }
  int k = (int)v;  // toward zero
  if (k < 0) k += ncode;
  if (k < 0 || k >= ncode) {
    bad = true;
    return 0;
  }
  return (uint32_t)k;
}

__global__ __launch_bounds__(256) void nf4_pack_kernel(const void* __restrict__ w, int wdt,
                                                       const void* __restrict__ s, int sdt, int N, int K,
                                                       int transposed, int ncode, uint8_t* __restrict__ codes,
                                                       float* __restrict__ scale_out, int* __restrict__ bad) {
  __shared__ uint8_t idx[64][65];  // [k][n] of a transposed tile
  const int t = threadIdx.x;
  const int tn = (N + 63) / 64, kb = K / 64;
  const int64_t ntiles = (int64_t)tn * kb;
  bool my_bad = false;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int n0 = (int)(tile % tn) * 64, b = (int)(tile / tn), k0 = b * 64;
    const int n = n0 + (t >> 2), kq = 16 * (t & 3);
    uint32_t c[16];
    if (!transposed) {
      if (n < N) {
#pragma unroll
        for (int j = 0; j < 16; ++j) c[j] = code_index(elem_as_f32(w, wdt, (int64_t)n * K + k0 + kq + j), ncode, my_bad);
      }
    } else {
      // load: row k0 + t / 4 of [K, N], columns n0 + 16 (t % 4) .. + 15
      const int kr = k0 + (t >> 2);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int nc = n0 + kq + j;
        idx[t >> 2][kq + j] = nc < N ? (uint8_t)code_index(elem_as_f32(w, wdt, (int64_t)kr * N + nc), ncode, my_bad) : 0;
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 16; ++j) c[j] = idx[kq + j][t >> 2];
      __syncthreads();
    }
    if (n < N) {
      u32x2 v = {0u, 0u};
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j >> 2] |= (c[2 * j] | c[2 * j + 1] << 4) << (8 * (j & 3));
      *reinterpret_cast<u32x2*>(codes + (size_t)n * (K / 2) + (k0 + kq) / 2) = v;
    }
    if (t < 64 && n0 + t < N) {
      const int sn = n0 + t;
      scale_out[(size_t)sn * kb + b] =
          s ? elem_as_f32(s, sdt, transposed ? (int64_t)b * N + sn : (int64_t)sn * kb + b) : 1.0f;
    }
  }
  if (my_bad) atomicOr(bad, 1);
}

int nf4_pack(const void* weight, int w_dtype, const void* scale, int s_dtype, int64_t N, int64_t K, int transposed,
             int ncode, uint8_t* codes, float* scale_out, int* bad, hipStream_t st) {
  if (N <= 0 || K <= 0) return set_error(kErrInvalid, "nf4_pack: empty shape");
  if (N > (1 << 30) || K > (1 << 30)) return set_error(kErrInvalid, "nf4_pack: shape too large");
  if (K % 64) return set_error(kErrUnsupported, "nf4_pack: needs K %% 64 == 0 (got K = %lld)", (long long)K);
  if (ncode < 1 || ncode > 16) return set_error(kErrInvalid, "nf4_pack: code tables of 1..16 entries (got %d)", ncode);
  if (w_dtype != kF32 && w_dtype != kBF16 && w_dtype != kF16)
    return set_error(kErrInvalid, "nf4_pack: weight dtype must be F32, BF16 or F16");
  if (scale && s_dtype != kF32 && s_dtype != kBF16 && s_dtype != kF16)
    return set_error(kErrInvalid, "nf4_pack: scale dtype must be F32, BF16 or F16");
  if (!aligned(codes, 8) || !aligned(scale_out, 4)) return set_error(kErrInvalid, "nf4_pack: codes must be 8-byte aligned");
  const int64_t tiles = (N + 63) / 64 * (K / 64);
  hipLaunchKernelGGL(nf4_pack_kernel, dim3(grid_for(tiles, 1, 8)), dim3(256), 0, st, weight, w_dtype, scale, s_dtype,
                     (int)N, (int)K, transposed, ncode, codes, scale_out, bad);
  return check_launch("nf4_pack");
}

int nf4_gemm(const uint16_t* A, const uint8_t* codes, const float* scale, const uint16_t* levels,
             const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K, void* workspace,
             int64_t workspace_bytes, hipStream_t st) {
  if (M <= 0 || N <= 0 || K <= 0) return set_error(kErrInvalid, "nf4_gemm: empty shape");
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30)) return set_error(kErrInvalid, "nf4_gemm: shape too large");
  if (K % kBK) return set_error(kErrUnsupported, "nf4_gemm: needs K %% 64 == 0 (got K = %lld)", (long long)K);
  if (!aligned(A, 16) || !aligned(codes, 16) || !aligned(out, 8) || (bias && !aligned(bias, 8)))
    return set_error(kErrInvalid, "nf4_gemm: A and codes must be 16-byte aligned, out and bias 8-byte aligned");
  if (M <= 16) {
    const unsigned tiles = (unsigned)((N + 15) / 16);
    // about eight waves per CU, at most one wave per 128-k step
    int w = kSkinnyWavesMin;
    while (w < kSkinnyWavesMax && (int64_t)tiles * w < (int64_t)num_cus() * 8 && 2 * w <= (K + 127) / 128) w *= 2;
    if (w == 16)
      hipLaunchKernelGGL(nf4_skinny_kernel<16>, dim3(tiles), dim3(64 * 16), 0, st, A, codes, scale, levels, bias, out,
                         (int)M, (int)N, (int)K);
    else if (w == 8)
      hipLaunchKernelGGL(nf4_skinny_kernel<8>, dim3(tiles), dim3(64 * 8), 0, st, A, codes, scale, levels, bias, out,
                         (int)M, (int)N, (int)K);
    else
      hipLaunchKernelGGL(nf4_skinny_kernel<4>, dim3(tiles), dim3(64 * 4), 0, st, A, codes, scale, levels, bias, out,
                         (int)M, (int)N, (int)K);
    return check_launch("nf4_skinny");
  }
  if (N % kBN)
    return set_error(kErrUnsupported, "nf4_gemm: needs N %% 128 == 0 for M > 16 (got N = %lld)", (long long)N);
  const int64_t mfull = M / kBM * kBM;
  const int64_t ntiles = mfull / kBM * (N / kBN);
  SkPlan plan;
  plan.dp_tiles = ntiles;
  if (workspace) {
    plan = plan_stream_k(M, N, K);
    if (plan.sk_tiles > 0 && workspace_bytes < plan.bytes)
      return set_error(kErrInvalid, "nf4_gemm: workspace of %lld bytes, this shape needs %lld",
                       (long long)workspace_bytes, (long long)plan.bytes);
    if (!aligned(workspace, 256)) return set_error(kErrInvalid, "nf4_gemm: workspace must be 256-byte aligned");
  }
  int* cnt = plan.sk_tiles > 0 ? static_cast<int*>(workspace) : nullptr;
  if (cnt && plan.dp_tiles == 0)
    hipLaunchKernelGGL(nf4_zero_counters, dim3((unsigned)((plan.sk_tiles + 255) / 256)), dim3(256), 0, st, cnt,
                       (int)plan.sk_tiles);
  if (plan.dp_tiles > 0)
    hipLaunchKernelGGL(nf4_gemm_kernel<false>, dim3((unsigned)plan.dp_tiles), dim3(kThreads), 0, st, A, codes, scale,
                       levels, bias, out, (int)M, (int)N, (int)K, 0, (int)plan.dp_tiles, cnt, (int)plan.sk_tiles);
  if (plan.sk_tiles > 0) {
    float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                           (plan.sk_tiles * 4 + kCounterBytes - 1) / kCounterBytes * kCounterBytes);
    hipLaunchKernelGGL(nf4_gemm_sk_kernel, dim3((unsigned)plan.groups), dim3(kThreads), 0, st, A, codes, scale, levels,
                       bias, out, (int)M, (int)N, (int)K, (int)plan.dp_tiles, (int)plan.sk_tiles, part, cnt);
  }
  if (mfull < M)
    hipLaunchKernelGGL(nf4_gemm_kernel<true>, dim3((unsigned)(N / kBN)), dim3(kThreads), 0, st, A, codes, scale,
                       levels, bias, out, (int)M, (int)N, (int)K, (int)mfull, (int)(N / kBN), nullptr, 0);
  return check_launch("nf4_gemm");
}

}  // namespace vqx
