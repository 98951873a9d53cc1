// NF4-dequant-fused linear:  out[M, N] = A[M, K] . W[N, K]^T (+ bias)
// with W[n, k] = bf16(level[code[n, k]] * scale[n, k / 64]) decoded on the fly
// (the weight decode of linear_mx, src/voyager_compiler/ops/quantized.py:
// 319-326, fused into the product of :330-331).  bf16 MFMA
// (v_mfma_f32_32x32x16_bf16), fp32 accumulation, bf16 output.
//
// Tiling: a workgroup of 256 threads (4 waves as 2 x 2) computes a 256 x 128
// tile of out; each wave a 128 x 64 sub-tile = 4 x 2 MFMA tiles of 32 x 32.
// The K loop steps by 64 (one NF4 scale block).  Per step the workgroup stages
// the A tile (256 x 64 bf16, 32 KiB) and the decoded W tile (128 x 64 bf16,
// 16 KiB) in LDS, double buffered; 16-byte chunks are XOR-swizzled by row so
// the fragment reads are bank-conflict free.  Each thread decodes 32 weights
// per step: one 16-byte load of packed codes, a byte-table lookup of the bf16
// levels with v_perm, the fp32 product with the block scale and RNE to bf16.
// Workgroups are ordered so each XCD runs whole 256-row slabs of A, which stay
// in its L2 while W streams past.
#include "vqx_kernels.h"

namespace vqx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kBM = 256, kBN = 128, kBK = 64;
constexpr int kThreads = 256;
constexpr int kALds = kBM * kBK * 2;  // bytes
constexpr int kWLds = kBN * kBK * 2;
constexpr int kStage = kALds + kWLds;

// byte offset of 16-byte chunk c (0..7) of row r in a [rows][64] bf16 tile
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t c) { return r * 128u + ((c ^ (r & 7u)) << 4); }

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  f32x2 f = {a, b};
  bf16x2 h = __builtin_convertvector(f, bf16x2);
  return __builtin_bit_cast(uint32_t, h);
}

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

__global__ __launch_bounds__(kThreads) void nf4_gemm_kernel(const uint16_t* __restrict__ A,
                                                             const uint8_t* __restrict__ codes,
                                                             const float* __restrict__ scale,
                                                             const uint16_t* __restrict__ levels,
                                                             const uint16_t* __restrict__ bias,
                                                             uint16_t* __restrict__ out, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // XCD-aware tile order: consecutive workgroup ids go round-robin over the 8
  // XCDs; give each XCD a contiguous range of tiles, M-major, so an XCD works
  // through whole A slabs.
  const int ntn = N / kBN, ntm = M / kBM;
  const int ntiles = ntn * ntm;
  int bid = blockIdx.x;
  int per_xcd = (ntiles + 7) / 8;
  int xcd = bid & 7, local = bid >> 3;
  int tile = xcd * per_xcd + local;
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

  // this thread's load assignments
  // A: 2048 16-byte chunks per step, 8 per thread: chunk q = tid + 256 i,
  // row q / 8, chunk q % 8
  // W: row n = tid / 2, half = tid % 2 (codes for k 0-31 or 32-63 of the step)
  const int wr = tid >> 1, wh = tid & 1;
  const uint8_t* wsrc = codes + (size_t)(n0 + wr) * (K / 2) + wh * 16;
  const float* ssrc = scale + (size_t)(n0 + wr) * kb;

  u32x4 areg[8];
  u32x4 wreg;
  float sreg;

  auto load_global = [&](int ks) {
    const uint16_t* asrc = A + (size_t)m0 * K + ks * kBK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int q = tid + kThreads * i;
      int r = q >> 3, c = q & 7;
      areg[i] = *reinterpret_cast<const u32x4*>(asrc + (size_t)r * K + c * 8);
    }
    wreg = *reinterpret_cast<const u32x4*>(wsrc + ks * (kBK / 2));
    sreg = ssrc[ks];
  };

  auto store_lds = [&](int buf) {
    uint8_t* sa = smem + buf * kStage;
    uint8_t* sw = sa + kALds;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int q = tid + kThreads * i;
      int r = q >> 3, c = q & 7;
      *reinterpret_cast<u32x4*>(sa + swz(r, c)) = areg[i];
    }
    uint32_t w4[4] = {wreg.x, wreg.y, wreg.z, wreg.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t o[4];
      decode8(w4[j], sreg, lb, o);
      u32x4 v = {o[0], o[1], o[2], o[3]};
      *reinterpret_cast<u32x4*>(sw + swz(wr, wh * 4 + j)) = v;
    }
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  load_global(0);
  store_lds(0);
  __syncthreads();

  const int lr = lane & 31;   // fragment row / column within a 32-tile
  const int lk = lane >> 5;   // which 8-wide k group

  for (int ks = 0; ks < nk; ++ks) {
    const int buf = ks & 1;
    if (ks + 1 < nk) load_global(ks + 1);
    const uint8_t* sa = smem + buf * kStage;
    const uint8_t* sw = sa + kALds;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      bf16x8 af[4], bfr[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int r = wm * 128 + i * 32 + lr;
        u32x4 v = *reinterpret_cast<const u32x4*>(sa + swz(r, kk * 2 + lk));
        af[i] = __builtin_bit_cast(bf16x8, v);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        int r = wn * 64 + j * 32 + lr;
        u32x4 v = *reinterpret_cast<const u32x4*>(sw + swz(r, kk * 2 + lk));
        bfr[j] = __builtin_bit_cast(bf16x8, v);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (ks + 1 < nk) store_lds(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds column lr, rows 8*(e/4) + 4*lk + (e%4) of each tile
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    int n = n0 + wn * 64 + j * 32 + lr;
    float bv = bias ? bf2f(bias[n]) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        int m = m0 + wm * 128 + i * 32 + 8 * (e >> 2) + 4 * lk + (e & 3);
        out[(size_t)m * N + n] = (uint16_t)f2bf(acc[i][j][e] + bv);
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
  if (!aligned(A, 16) || !aligned(codes, 16) || !aligned(out, 4))
    return set_error(kErrInvalid, "nf4_gemm: A and codes must be 16-byte aligned");
  int ntiles = (int)((M / kBM) * (N / kBN));
  static thread_local bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)nf4_gemm_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                            2 * kStage) != hipSuccess)
      return set_error(kErrLaunch, "nf4_gemm: cannot reserve %d bytes of LDS", 2 * kStage);
    attr_set = true;
  }
  hipLaunchKernelGGL(nf4_gemm_kernel, dim3(ntiles), dim3(kThreads), 2 * kStage, st, A, codes, scale, levels, bias,
                     out, (int)M, (int)N, (int)K);
  return check_launch("nf4_gemm");
}

}  // namespace vqx
