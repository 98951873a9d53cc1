// Host-side entry points of the kernel families (one translation unit each),
// called by the C ABI in vqx_capi.hip.
#pragma once

#include "vqx_encoders.h"
#include "vqx_lut.h"

namespace vqx {

struct ScaleParams {
  int32_t mode;                // 0: power of two (force_scale_power_of_two), 1: absmax
  int32_t shift;               // mode 0: floor(log2(quant_max))
  float quant_max;             // mode 1
  const uint16_t* scale_qmap;  // mode 1: optional bf16 table applied to the scale
};

struct MxOut {
  void* scale;          // input dtype [blocks]
  float* scale_f32;     // [blocks]
  uint8_t* scale_e8m0;  // [blocks]
  void* qvals;          // input dtype [n]: the reference's quantize() output
  void* fq;             // input dtype [n]: qvals * scale (MXFakeQuantizeFunction)
  void* codes;          // codes: packed bitstream or one uint8/uint16 per element
};

struct ScaleMap {
  const void* scale;
  const void* zero_point;
  int64_t L, inner, block;
  int64_t s_o, s_l, s_in;
};

// vqx_elementwise.hip
int quantize_mapped(const void* x, int dtype, int64_t n, const FormatDesc& fmt, const ScaleMap& m,
                    bool mul, void* y, void* codes, int code_bytes, hipStream_t st);
int dequantize_mapped(const void* x, int dtype, int64_t n, const uint16_t* in_map, const ScaleMap& m,
                      const uint16_t* out_map, void* y, hipStream_t st);
int fake_quant(const void* x, int dtype, int64_t n, const FormatDesc& fmt, const float* scale,
               int64_t scale_numel, int64_t scale_inner, bool mul, void* y, void* codes, int code_bytes,
               hipStream_t st);
int lut_gather(const void* x, int dtype, int64_t n, const uint16_t* table, void* y, hipStream_t st);
int build_table(const FormatDesc& fmt, uint16_t* values, uint16_t* codes, hipStream_t st);
int build_lut(const FormatDesc& fmt, uint32_t* blob, hipStream_t st);
int level_tables(const float* levels, int K, int mode, uint8_t* index_table, float* boundaries,
                 uint32_t* work, int* bad, hipStream_t st);

// vqx_blockwise.hip
int mx_quantize(const void* x, int dtype, int64_t outer, int64_t L, int64_t inner, int64_t bs,
                const FormatDesc& fmt, const ScaleParams& sp, const MxOut& out, int code_layout,
                hipStream_t st);
int mx_decode(const uint8_t* codes, int code_bits, const uint16_t* decode_table, int ntab,
              const void* scale, int scale_kind, int64_t n, int64_t bs, void* out, int out_dtype,
              hipStream_t st);
int decode_table(const FormatDesc& fmt, uint16_t* dtab, int ntab, hipStream_t st);
int gwa_fake_quant(const void* x, int dtype, int64_t outer, int64_t L, int64_t inner, int64_t bs, float qmin,
                   float qmax, const uint16_t* scale_qmap, void* scale_out, void* zp_out, void* y,
                   hipStream_t st);

// vqx_codebook.hip
int codebook_encode(const void* x, int dtype, int64_t rows, int64_t cols, const float* cb, int K,
                    uint8_t* codes, hipStream_t st);
int codebook_decode(const uint8_t* codes, int64_t rows, int64_t cols, const float* cb, int K, void* out,
                    int dtype, hipStream_t st);

// vqx_nf4_gemm.hip
int nf4_gemm(const uint16_t* A, const uint8_t* codes, const float* scale, const uint16_t* levels,
             const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K, hipStream_t st);

}  // namespace vqx
