// CPU harness for vqx_formats.h: evaluates the same encoder code the HIP
// kernels run, over caller-given bf16 patterns, so the tests can compare it
// with the oracle over all 65536 inputs without a GPU.  Test-only.
#include "vqx_formats.h"

extern "C" {

// 2 ** ceil(log2(f)) of fp32 bit patterns (the observer's power-of-two scale).
int vqx_host_pow2_ceil_log2(const uint32_t* in, int64_t n, uint32_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = vqx::pow2_ceil_log2_f32(in[i]);
  return 0;
}

// kind/params follow vqx::FormatKind; levels/boundaries for kFmtLevels.
int vqx_host_encode(int kind, int p0, int p1, float max_norm, int flags,
                    const float* boundaries, const uint16_t* levels, int nlev,
                    const uint16_t* in, int64_t n, uint32_t* code,
                    uint16_t* value) {
  for (int64_t i = 0; i < n; ++i) {
    uint32_t h = in[i];
    vqx::Result r{0, 0};
    switch (kind) {
      case vqx::kFmtPosit:
        r = vqx::Posit{p0, p1}.encode(h);
        break;
      case vqx::kFmtFpCore:
        r = vqx::FpCore{p0, p1, max_norm, (flags & 1) != 0}.encode(h);
        break;
      case vqx::kFmtNvFp8:
        r = (p0 == 4 ? vqx::NvFp8::e4m3() : vqx::NvFp8::e5m2()).encode(h);
        break;
      case vqx::kFmtInt:
        r = vqx::IntFmt{p0, p1 != 0}.encode(h);
        break;
      case vqx::kFmtLevels: {
        uint32_t c = vqx::count_le(boundaries, nlev - 1, vqx::bf2f(h));
        r.code = c;
        r.value = levels[c];
        break;
      }
      default:
        return -1;
    }
    code[i] = r.code;
    value[i] = (uint16_t)r.value;
  }
  return 0;
}

int vqx_host_log2floor(const uint16_t* in, int64_t n, int32_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = vqx::log2floor_bf16(in[i] & 0x7FFFu);
  return 0;
}
}
