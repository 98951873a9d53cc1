// Shared HIP plumbing for the vqx kernels: error state, launch sizing,
// streaming loads/stores and wave64 reductions.  gfx950 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vqx_formats.h"

namespace vqx {

// ---------------------------------------------------------------------------
// error state (thread-local message; entry points return a negative status)
// ---------------------------------------------------------------------------
enum Status : int {
  kOk = 0,
  kErrInvalid = -1,   // bad argument: shape, dtype, alignment, format
  kErrLaunch = -2,    // kernel launch / HIP runtime failure
  kErrUnsupported = -3,
};

int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
int num_cus();

// dtype tags used across the C ABI
enum DType : int32_t {
  kF32 = 0,
  kBF16 = 1,
  kF16 = 2,
  kU8 = 3,
  kI64 = 4,
};

// ---------------------------------------------------------------------------
// memory helpers
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ T ld_nt(const T* p) {
  return __builtin_nontemporal_load(p);
}
template <typename T>
__device__ __forceinline__ void st_nt(T* p, T v) {
  __builtin_nontemporal_store(v, p);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t umax32(uint32_t a, uint32_t b) {
  return a > b ? a : b;
}
__device__ __forceinline__ uint32_t umin32(uint32_t a, uint32_t b) {
  return a < b ? a : b;
}

// Round-to-nearest-even fp32 -> bf16 pattern, every NaN to 0x7FC0.
__device__ __forceinline__ uint32_t f2bf_dev(float f) { return f2bf(f); }

// Two fp32 -> bf16 (RNE, v_cvt_pk_bf16_f32), a in the low half.  Matches
// f2bf for every non-NaN input.
typedef __bf16 vqx_bf16x2 __attribute__((ext_vector_type(2)));
typedef float vqx_f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  vqx_f32x2 f = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, vqx_bf16x2));
}

// Low bytes of four words, packed a | b << 8 | c << 16 | d << 24 (three v_perm).
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_amdgcn_perm(__builtin_amdgcn_perm(d, c, 0x0C0C0400u), __builtin_amdgcn_perm(b, a, 0x0C0C0400u),
                               0x05040100u);
}

// Wave-level LDS hand-off: the wave's own LDS writes are complete and visible
// to all its lanes before any lane reads past this point.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// Exact fp16 <-> fp32 conversions in integer arithmetic (subnormals and signed
// zeros kept, round to nearest even), independent of the device's fp16
// denormal mode; torch's CPU conversions are the reference.
__device__ __forceinline__ float h2f_exact(uint32_t hb) {
  uint32_t s = (hb & 0x8000u) << 16;
  uint32_t e = (hb >> 10) & 0x1Fu, m = hb & 0x3FFu;
  uint32_t nrm = s | ((e + 112u) << 23) | (m << 13);
  uint32_t inf = s | 0x7F800000u | (m << 13);
  uint32_t sub = s | f2u((float)m * 0x1p-24f);  // m * 2^-24 is exact in fp32
  return u2f(e == 0x1Fu ? inf : (e != 0 ? nrm : sub));
}

__device__ __forceinline__ uint32_t f2h_exact(float f) {
  uint32_t b = f2u(f);
  uint32_t s = (b >> 16) & 0x8000u;
  uint32_t a = b & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return s | 0x7E00u;        // NaN
  if (a >= 0x477FF000u) return s | 0x7C00u;       // rounds to >= 65520: Inf
  if (a >= 0x38800000u) {                         // normal fp16 range
    uint32_t r = a + 0xFFFu + ((a >> 13) & 1u);   // RNE at bit 13
    return s | ((r >> 13) - (112u << 10));
  }
  // subnormal fp16: multiples of 2^-24; round |f| * 2^24 to an integer
  float q = u2f(a) * 0x1p24f;                     // exact scaling
  return s | (uint32_t)__builtin_rintf(q);
}

// Grid sizing: enough workgroups to cover the work, capped at a few per CU;
// kernels loop grid-stride beyond that.
inline unsigned grid_for(int64_t work_items, int per_block, int max_per_cu = 8) {
  int64_t need = (work_items + per_block - 1) / per_block;
  int64_t cap = (int64_t)num_cus() * max_per_cu;
  if (need < 1) need = 1;
  return (unsigned)(need < cap ? need : cap);
}

// Persistent launch: as many workgroups as fit on the device at once (from
// the kernel's register use and the dynamic LDS size), no more than the work
// needs; the kernels loop grid-stride.
unsigned persistent_grid(const void* kernel, int block, size_t lds_bytes, int64_t work_items);

inline bool aligned(const void* p, unsigned a) {
  return ((uintptr_t)p & (a - 1)) == 0;
}

}  // namespace vqx
