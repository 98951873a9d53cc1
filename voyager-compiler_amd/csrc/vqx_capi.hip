// C ABI of libvqx.so (declared in include/vqx.h): argument checks, the
// thread-local error message, and dispatch into the kernel families.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/vqx.h"
#include "vqx_kernels.h"

namespace vqx {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(kErrLaunch, "%s: %s", what, hipGetErrorString(e));
  return kOk;
}

int num_cus() {
  static thread_local int cached_dev = -1, cached_cus = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev != cached_dev) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cached_dev = dev;
    cached_cus = cus;
  }
  return cached_cus;
}

unsigned persistent_grid(const void* kernel, int block, size_t lds_bytes, int64_t work_items) {
  // occupancy by (kernel, block, LDS), cached per thread and device
  struct Entry {
    const void* k;
    int block, dev;
    size_t lds;
    int per_cu;
  };
  static thread_local Entry cache[32];
  static thread_local int used = 0;
  int dev = 0;
  (void)hipGetDevice(&dev);
  int per_cu = 0;
  for (int i = 0; i < used; ++i)
    if (cache[i].k == kernel && cache[i].block == block && cache[i].lds == lds_bytes && cache[i].dev == dev)
      per_cu = cache[i].per_cu;
  if (per_cu == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, lds_bytes) != hipSuccess ||
        per_cu <= 0)
      per_cu = 1;
    Entry e{kernel, block, dev, lds_bytes, per_cu};
    cache[used < 32 ? used++ : 31] = e;
  }
  int64_t need = (work_items + block - 1) / block;
  int64_t cap = (int64_t)num_cus() * per_cu;
  if (need < 1) need = 1;
  return (unsigned)(need < cap ? need : cap);
}

static int to_desc(const vqx_format* f, FormatDesc* d) {
  if (!f) return set_error(kErrInvalid, "format descriptor is NULL");
  d->kind = f->kind;
  d->p0 = f->p0;
  d->p1 = f->p1;
  d->flags = f->flags;
  d->max_norm = f->max_norm;
  d->code_bits = f->code_bits;
  d->boundaries = f->boundaries;
  d->levels = f->levels;
  d->code_table = f->code_table;
  d->value_table = f->value_table;
  d->lut = f->lut;
  d->lut_len = f->lut_len;
  if (d->lut && (d->lut_len < 1 || d->lut_len > kLutMaxLen))
    return set_error(kErrInvalid, "lut_len %d outside [1, %d]", d->lut_len, kLutMaxLen);
  return kOk;
}

static int to_map(const vqx_scale_map* sm, ScaleMap* m) {
  if (!sm) {
    *m = ScaleMap{nullptr, nullptr, 1, 1, 1, 0, 0, 0};
    return kOk;
  }
  *m = ScaleMap{sm->scale, sm->zero_point, sm->L, sm->inner, sm->block, sm->s_o, sm->s_l, sm->s_in};
  return kOk;
}

}  // namespace vqx

using namespace vqx;

#define VQX_TRY(expr)          \
  do {                         \
    int _rc = (expr);          \
    if (_rc != kOk) return _rc; \
  } while (0)

extern "C" {

const char* vqx_version(void) { return "vqx 0.1.0 gfx950"; }

const char* vqx_last_error(void) { return g_err; }

int vqx_device_cus(void) { return num_cus(); }

int vqx_vmap(const void* x, int32_t x_dtype, int64_t n, const uint16_t* table, void* y,
             vqx_stream_t stream) {
  g_err[0] = 0;
  if (n > 0 && (!x || !y)) return set_error(kErrInvalid, "vmap: null tensor");
  return lut_gather(x, x_dtype, n, table, y, (hipStream_t)stream);
}

int vqx_fake_quant(const void* x, int32_t x_dtype, int64_t n, const vqx_format* fmt,
                   const float* scale, int64_t scale_numel, int64_t scale_inner, int32_t mul_back,
                   void* y, void* codes, int32_t code_bytes, vqx_stream_t stream) {
  g_err[0] = 0;
  FormatDesc d;
  VQX_TRY(to_desc(fmt, &d));
  if (n > 0 && !x) return set_error(kErrInvalid, "fake_quant: null input");
  if (!codes) code_bytes = 0;
  if (scale && scale_numel < 1) return set_error(kErrInvalid, "fake_quant: scale_numel must be >= 1");
  return fake_quant(x, x_dtype, n, d, scale, scale ? scale_numel : 1, scale_inner, mul_back != 0, y,
                    codes, code_bytes, (hipStream_t)stream);
}

int vqx_amax_observe_fake_quant(const void* x, int32_t x_dtype, int64_t n, int64_t channels, int64_t inner,
                                const vqx_format* fmt, float* amax_history, int32_t history_len, float* scale,
                                float quant_max, int32_t force_scale_power_of_two, void* y, vqx_stream_t stream) {
  g_err[0] = 0;
  FormatDesc d;
  VQX_TRY(to_desc(fmt, &d));
  if (!x || !amax_history || !scale) return set_error(kErrInvalid, "amax_observe_fake_quant: null buffer");
  return amax_observe_fake_quant(x, x_dtype, n, channels, inner, d, amax_history, history_len, scale, quant_max,
                                 force_scale_power_of_two != 0, y, (hipStream_t)stream);
}

int vqx_quantize_mapped(const void* x, int32_t x_dtype, int64_t n, const vqx_format* fmt,
                        const vqx_scale_map* sm, int32_t mul_back, void* y, void* codes,
                        int32_t code_bytes, vqx_stream_t stream) {
  g_err[0] = 0;
  FormatDesc d;
  VQX_TRY(to_desc(fmt, &d));
  ScaleMap m;
  VQX_TRY(to_map(sm, &m));
  if (n > 0 && !x) return set_error(kErrInvalid, "quantize: null input");
  return quantize_mapped(x, x_dtype, n, d, m, mul_back != 0, y, codes, code_bytes, (hipStream_t)stream);
}

int vqx_dequantize_mapped(const void* x, int32_t x_dtype, int64_t n, const uint16_t* input_qmap,
                          const vqx_scale_map* sm, const uint16_t* output_qmap, void* y,
                          vqx_stream_t stream) {
  g_err[0] = 0;
  ScaleMap m;
  VQX_TRY(to_map(sm, &m));
  if (n > 0 && (!x || !y)) return set_error(kErrInvalid, "dequantize: null tensor");
  return dequantize_mapped(x, x_dtype, n, input_qmap, m, output_qmap, y, (hipStream_t)stream);
}

int vqx_build_table(const vqx_format* fmt, uint16_t* values, uint16_t* codes, vqx_stream_t stream) {
  g_err[0] = 0;
  FormatDesc d;
  VQX_TRY(to_desc(fmt, &d));
  return build_table(d, values, codes, (hipStream_t)stream);
}

int64_t vqx_lut_bytes(void) { return kLutBytes; }

int vqx_build_lut(const vqx_format* fmt, uint32_t* blob, vqx_stream_t stream) {
  g_err[0] = 0;
  FormatDesc d;
  VQX_TRY(to_desc(fmt, &d));
  if (!blob) return set_error(kErrInvalid, "build_lut: null blob");
  return build_lut(d, blob, (hipStream_t)stream);
}

int vqx_level_tables(const float* levels, int32_t K, int32_t mode, uint8_t* index_table,
                     float* boundaries, uint32_t* work, int32_t* bad, vqx_stream_t stream) {
  g_err[0] = 0;
  if (!levels || !index_table || (K > 1 && (!boundaries || !work || !bad)))
    return set_error(kErrInvalid, "level_tables: null buffer");
  if (mode != 0 && mode != 1) return set_error(kErrInvalid, "level_tables: mode must be 0 or 1");
  return level_tables(levels, K, mode, index_table, boundaries, work, bad, (hipStream_t)stream);
}

int vqx_mx_quantize(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner,
                    int64_t block_size, const vqx_format* fmt, int32_t scale_mode, int32_t pow2_shift,
                    float quant_max, const uint16_t* scale_qmap, void* scale_out, float* scale_f32,
                    uint8_t* scale_e8m0, void* qvals, void* fq, void* codes, int32_t code_layout,
                    vqx_stream_t stream) {
  g_err[0] = 0;
  FormatDesc d;
  VQX_TRY(to_desc(fmt, &d));
  if (!x && outer * L * inner > 0) return set_error(kErrInvalid, "mx_quantize: null input");
  if (scale_mode != 0 && scale_mode != 1) return set_error(kErrInvalid, "mx_quantize: scale_mode must be 0 or 1");
  ScaleParams sp{scale_mode, pow2_shift, quant_max, scale_qmap};
  MxOut out{scale_out, scale_f32, scale_e8m0, qvals, fq, codes};
  return mx_quantize(x, x_dtype, outer, L, inner, block_size, d, sp, out, code_layout, (hipStream_t)stream);
}

int vqx_outlier_stats_size(int64_t* bytes) {
  g_err[0] = 0;
  if (!bytes) return set_error(kErrInvalid, "outlier_stats_size: null result pointer");
  *bytes = kOutlierStatsBytes;
  return kOk;
}

int vqx_outlier_topk_workspace_size(int64_t* bytes) {
  g_err[0] = 0;
  if (!bytes) return set_error(kErrInvalid, "outlier_topk_workspace_size: null result pointer");
  *bytes = outlier_topk_workspace_bytes();
  return kOk;
}

int vqx_outlier_topk_threshold(const void* x, int32_t x_dtype, int64_t n, int64_t k, int32_t ema, float decay,
                               float one_minus_decay, float* threshold, void* workspace, int64_t workspace_bytes,
                               vqx_stream_t stream) {
  g_err[0] = 0;
  if (ema != 0 && ema != 1) return set_error(kErrInvalid, "outlier_topk_threshold: ema must be 0 or 1");
  return outlier_topk_threshold(x, x_dtype, n, k, ema, decay, one_minus_decay, threshold, workspace,
                                workspace_bytes, (hipStream_t)stream);
}

static OutlierArgs outlier_args(const float* threshold_dev, float threshold, void* stats, int64_t numel,
                                int32_t parity) {
  return OutlierArgs{1, threshold_dev, threshold, (OutlierStats*)stats, numel, parity};
}

int vqx_mx_fake_quant_outlier(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner,
                              int64_t block_size, const vqx_format* fmt, int32_t scale_mode, int32_t pow2_shift,
                              float quant_max, const uint16_t* scale_qmap, const float* threshold_dev,
                              float threshold, void* stats, int32_t stats_parity, void* scale_out,
                              float* scale_f32, void* fq, vqx_stream_t stream) {
  g_err[0] = 0;
  FormatDesc d;
  VQX_TRY(to_desc(fmt, &d));
  if (!x && outer * L * inner > 0) return set_error(kErrInvalid, "mx_fake_quant_outlier: null input");
  if (!fq && outer * L * inner > 0) return set_error(kErrInvalid, "mx_fake_quant_outlier: null output");
  if (scale_mode != 0 && scale_mode != 1)
    return set_error(kErrInvalid, "mx_fake_quant_outlier: scale_mode must be 0 or 1");
  if (stats && !aligned(stats, 256)) return set_error(kErrInvalid, "mx_fake_quant_outlier: stats must be 256-byte aligned");
  if (stats_parity != 0 && stats_parity != 1) return set_error(kErrInvalid, "mx_fake_quant_outlier: parity must be 0 or 1");
  ScaleParams sp{scale_mode, pow2_shift, quant_max, scale_qmap};
  MxOut out{scale_out, scale_f32, nullptr, nullptr, fq, nullptr};
  const OutlierArgs oa = outlier_args(threshold_dev, threshold, stats, outer * L * inner, stats_parity);
  return mx_quantize(x, x_dtype, outer, L, inner, block_size, d, sp, out, 1, (hipStream_t)stream, &oa);
}

int vqx_outlier_mask(const void* x, int32_t x_dtype, int64_t n, const float* threshold_dev, float threshold,
                     void* stats, int32_t stats_parity, void* masked, vqx_stream_t stream) {
  g_err[0] = 0;
  if (n < 0) return set_error(kErrInvalid, "outlier_mask: negative size");
  if (stats && !aligned(stats, 256)) return set_error(kErrInvalid, "outlier_mask: stats must be 256-byte aligned");
  if (stats_parity != 0 && stats_parity != 1) return set_error(kErrInvalid, "outlier_mask: parity must be 0 or 1");
  return outlier_mask(x, x_dtype, n, outlier_args(threshold_dev, threshold, stats, n, stats_parity), masked,
                      (hipStream_t)stream);
}

int vqx_outlier_restore(const void* x, int32_t x_dtype, int64_t n, const float* threshold_dev, float threshold,
                        void* y, vqx_stream_t stream) {
  g_err[0] = 0;
  if (n < 0) return set_error(kErrInvalid, "outlier_restore: negative size");
  return outlier_restore(x, x_dtype, n, outlier_args(threshold_dev, threshold, nullptr, n, 0), y, (hipStream_t)stream);
}

int vqx_mx_decode(const uint8_t* codes, int32_t code_bits, const uint16_t* decode_table, int32_t ntab,
                  const void* scale, int32_t scale_kind, int64_t n, int64_t block_size, void* out,
                  int32_t out_dtype, vqx_stream_t stream) {
  g_err[0] = 0;
  if (n > 0 && (!codes || !decode_table || !scale || !out))
    return set_error(kErrInvalid, "mx_decode: null buffer");
  if (block_size < 1) return set_error(kErrInvalid, "mx_decode: block_size must be >= 1");
  return mx_decode(codes, code_bits, decode_table, ntab, scale, scale_kind, n, block_size, out, out_dtype,
                   (hipStream_t)stream);
}

int vqx_gwa_fake_quant(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner,
                       int64_t block_size, float quant_min, float quant_max, const uint16_t* scale_qmap,
                       void* scale_out, void* zero_point_out, void* y, vqx_stream_t stream) {
  g_err[0] = 0;
  return gwa_fake_quant(x, x_dtype, outer, L, inner, block_size, quant_min, quant_max, scale_qmap, scale_out,
                        zero_point_out, y, (hipStream_t)stream);
}

int vqx_decode_table(const vqx_format* fmt, uint16_t* dtab, int32_t ntab, vqx_stream_t stream) {
  g_err[0] = 0;
  FormatDesc d;
  VQX_TRY(to_desc(fmt, &d));
  if (!dtab || ntab < 1 || ntab > 65536) return set_error(kErrInvalid, "decode_table: bad table");
  return decode_table(d, dtab, ntab, (hipStream_t)stream);
}

int vqx_codebook_encode(const void* x, int32_t x_dtype, int64_t rows, int64_t cols, const float* cb,
                        int32_t K, uint8_t* codes, vqx_stream_t stream) {
  g_err[0] = 0;
  if (rows * cols > 0 && (!x || !cb || !codes)) return set_error(kErrInvalid, "codebook_encode: null buffer");
  return codebook_encode(x, x_dtype, rows, cols, cb, K, codes, (hipStream_t)stream);
}

int vqx_codebook_decode(const uint8_t* codes, int64_t rows, int64_t cols, const float* cb, int32_t K,
                        void* out, int32_t out_dtype, vqx_stream_t stream) {
  g_err[0] = 0;
  if (rows * cols > 0 && (!codes || !cb || !out)) return set_error(kErrInvalid, "codebook_decode: null buffer");
  return codebook_decode(codes, rows, cols, cb, K, out, out_dtype, (hipStream_t)stream);
}

int vqx_nf4_linear(const uint16_t* A, const uint8_t* codes, const float* scale, const uint16_t* levels,
                   const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K,
                   vqx_stream_t stream) {
  g_err[0] = 0;
  if (!A || !codes || !scale || !levels || !out) return set_error(kErrInvalid, "nf4_linear: null buffer");
  return nf4_gemm(A, codes, scale, levels, bias, out, M, N, K, nullptr, 0, (hipStream_t)stream);
}

int vqx_nf4_linear_workspace_size(int64_t M, int64_t N, int64_t K, int64_t* bytes) {
  g_err[0] = 0;
  if (!bytes) return set_error(kErrInvalid, "nf4_linear_workspace_size: null bytes");
  *bytes = nf4_gemm_workspace(M, N, K);
  return kOk;
}

int vqx_nf4_linear_ws(const uint16_t* A, const uint8_t* codes, const float* scale, const uint16_t* levels,
                      const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K, void* workspace,
                      int64_t workspace_bytes, vqx_stream_t stream) {
  g_err[0] = 0;
  if (!A || !codes || !scale || !levels || !out) return set_error(kErrInvalid, "nf4_linear: null buffer");
  if (!workspace && nf4_gemm_workspace(M, N, K) > 0)
    return set_error(kErrInvalid, "nf4_linear_ws: null workspace (this shape needs %lld bytes)",
                     (long long)nf4_gemm_workspace(M, N, K));
  return nf4_gemm(A, codes, scale, levels, bias, out, M, N, K, workspace, workspace_bytes, (hipStream_t)stream);
}

int vqx_nf4_linear_noalloc(const uint16_t* A, const uint8_t* codes, const float* scale, const uint16_t* levels,
                           const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K,
                           vqx_stream_t stream) {
  g_err[0] = 0;
  if (!A || !codes || !scale || !levels || !out) return set_error(kErrInvalid, "nf4_linear: null buffer");
  return nf4_gemm_noalloc(A, codes, scale, levels, bias, out, M, N, K, (hipStream_t)stream);
}

int vqx_mx_matmul(const VqxMxOperand* a, const VqxMxOperand* b, const uint16_t* bias, uint16_t* out,
                  int64_t batch, int64_t M, int64_t N, int64_t K, vqx_stream_t stream) {
  g_err[0] = 0;
  static_assert(sizeof(VqxMxOperand) == sizeof(MxOperand), "VqxMxOperand and MxOperand differ");
  if (!a || !b) return set_error(kErrInvalid, "mx_matmul: null operand descriptor");
  return mx_gemm(*reinterpret_cast<const MxOperand*>(a), *reinterpret_cast<const MxOperand*>(b), bias, out, batch, M,
                 N, K, (hipStream_t)stream);
}

int vqx_mx_operand_decode(const VqxMxOperand* x, int64_t batch, int64_t rows, int64_t K, uint16_t* out,
                          vqx_stream_t stream) {
  g_err[0] = 0;
  if (!x) return set_error(kErrInvalid, "mx_decode: null operand descriptor");
  return mx_decode(*reinterpret_cast<const MxOperand*>(x), batch, rows, K, out, (hipStream_t)stream);
}

int vqx_nf4_pack_weight(const void* weight, int32_t w_dtype, const void* scale, int32_t s_dtype, int64_t N,
                        int64_t K, int32_t transposed, int32_t ncode, uint8_t* codes, float* scale_out,
                        int32_t* bad, vqx_stream_t stream) {
  g_err[0] = 0;
  if (!weight || !codes || !scale_out || !bad) return set_error(kErrInvalid, "nf4_pack_weight: null buffer");
  return nf4_pack(weight, w_dtype, scale, s_dtype, N, K, transposed, ncode, codes, scale_out, bad,
                  (hipStream_t)stream);
}

int vqx_filter_outlier(const void* x, int32_t x_dtype, int64_t batches, int64_t rows, int64_t cols,
                       float threshold, int64_t max_nnz, int32_t indptr_offset, void* data, int32_t* indices,
                       int32_t* indptr, void* inlier, vqx_stream_t stream) {
  g_err[0] = 0;
  return filter_outlier(x, x_dtype, batches, rows, cols, threshold, max_nnz, indptr_offset, data, indices, indptr,
                        inlier, (hipStream_t)stream);
}

int vqx_quantize_mx_outlier(const void* x, int64_t batches, int64_t rows, int64_t cols, float threshold,
                            int64_t max_nnz, int32_t indptr_offset, int64_t block_size, int32_t scale_mode,
                            int32_t shift, float quant_max, const uint16_t* scale_qmap, const uint16_t* qmap,
                            void* data, int32_t* indices, int32_t* indptr, void* scale, void* values,
                            vqx_stream_t stream) {
  g_err[0] = 0;
  if (scale_mode != 0 && scale_mode != 1) return set_error(kErrInvalid, "quantize_mx_outlier: scale_mode 0 or 1");
  ScaleParams sp{scale_mode, shift, quant_max, scale_mode == 1 ? scale_qmap : nullptr};
  return quantize_mx_outlier_fused(x, batches, rows, cols, threshold, max_nnz, indptr_offset, block_size, sp, qmap,
                                   data, indices, indptr, scale, values, (hipStream_t)stream);
}

int vqx_outlier_workspace_size(int32_t x_dtype, int64_t batches, int64_t rows, int64_t cols, int64_t max_nnz,
                               int64_t* bytes) {
  g_err[0] = 0;
  return outlier_workspace_size(x_dtype, batches, rows, cols, max_nnz, bytes);
}

int vqx_filter_outlier_ws(const void* x, int32_t x_dtype, int64_t batches, int64_t rows, int64_t cols,
                          float threshold, int64_t max_nnz, int32_t indptr_offset, void* data, int32_t* indices,
                          int32_t* indptr, void* inlier, void* workspace, int64_t workspace_bytes,
                          vqx_stream_t stream) {
  g_err[0] = 0;
  return filter_outlier_ws(x, x_dtype, batches, rows, cols, threshold, max_nnz, indptr_offset, data, indices, indptr,
                           inlier, workspace, workspace_bytes, (hipStream_t)stream);
}

int vqx_quantize_mx_outlier_ws(const void* x, int64_t batches, int64_t rows, int64_t cols, float threshold,
                               int64_t max_nnz, int32_t indptr_offset, int64_t block_size, int32_t scale_mode,
                               int32_t shift, float quant_max, const uint16_t* scale_qmap, const uint16_t* qmap,
                               void* data, int32_t* indices, int32_t* indptr, void* scale, void* values,
                               void* workspace, int64_t workspace_bytes, vqx_stream_t stream) {
  g_err[0] = 0;
  if (scale_mode != 0 && scale_mode != 1) return set_error(kErrInvalid, "quantize_mx_outlier: scale_mode 0 or 1");
  ScaleParams sp{scale_mode, shift, quant_max, scale_mode == 1 ? scale_qmap : nullptr};
  return quantize_mx_outlier_fused_ws(x, batches, rows, cols, threshold, max_nnz, indptr_offset, block_size, sp, qmap,
                                      data, indices, indptr, scale, values, workspace, workspace_bytes,
                                      (hipStream_t)stream);
}

int vqx_slice_csr(const void* data, int32_t dtype, const int32_t* indices, const int32_t* indptr, int64_t nnz,
                  int64_t rows, int32_t dim, int64_t start, int64_t end, int64_t max_nnz, void* data_out,
                  int32_t* indices_out, int32_t* indptr_out, vqx_stream_t stream) {
  g_err[0] = 0;
  return csr_slice(data, dtype, indices, indptr, nnz, rows, dim, start, end, max_nnz, data_out, indices_out,
                   indptr_out, (hipStream_t)stream);
}

int vqx_csr_decode_weight(const void* B, int32_t B_dtype, int64_t batches, int64_t rows, int64_t cols,
                          int32_t transpose, const void* code, int32_t code_dtype, int64_t code_len,
                          const void* scale, int32_t scale_dtype, int64_t scale_batch_stride, int64_t scale_rows,
                          int64_t scale_cols, int64_t row_block, int64_t col_block, void* out, int32_t out_dtype,
                          vqx_stream_t stream) {
  g_err[0] = 0;
  CsrDecode d{B, B_dtype, batches, rows, cols, transpose, code, code_dtype, code_len, scale, scale_dtype,
              scale_batch_stride, scale_rows, scale_cols, row_block, col_block, out, out_dtype};
  return csr_decode(d, (hipStream_t)stream);
}

int vqx_spmm_csr(const void* data, int32_t data_dtype, const int32_t* indices, const int32_t* indptr,
                 int64_t batches, int64_t rows, int64_t nnz_stride, const void* B, int32_t B_dtype,
                 int64_t B_batch_stride, int64_t K, int64_t N, const void* addend, void* out, vqx_stream_t stream) {
  g_err[0] = 0;
  SpmmArgs a{data, data_dtype, indices, indptr, batches, rows, nnz_stride, B, B_dtype, B_batch_stride, K, N,
             addend, out};
  return spmm_csr(a, (hipStream_t)stream);
}

int vqx_lcq_histogram(const void* x, int32_t x_dtype, int64_t n, int64_t block_size, float quant_max,
                      const float* weights, int64_t weights_period, const float* edges, int32_t bins,
                      double* weight, double* total, double* square, vqx_stream_t stream) {
  g_err[0] = 0;
  return lcq_histogram(x, x_dtype, n, block_size, quant_max, weights, weights_period, edges, bins, weight, total,
                       square, (hipStream_t)stream);
}

int vqx_gptq_block(const float* work, int64_t rows, int64_t ld, int64_t col0, int32_t ncols, const float* scale,
                   float quant_max, const uint16_t* scale_qmap, const float* hinv, int64_t ldh,
                   const uint16_t* qmap, float* out, float* deltas, int64_t ldd, vqx_stream_t stream) {
  g_err[0] = 0;
  return gptq_block(work, rows, ld, col0, ncols, scale, quant_max, scale_qmap, hinv, ldh, qmap, out, deltas, ldd,
                    (hipStream_t)stream);
}

int vqx_chol_inverse_block(const float* a, int64_t lda, int32_t n, float* li, int64_t ldl, int32_t* info,
                           vqx_stream_t stream) {
  g_err[0] = 0;
  return chol_inverse_block(a, lda, n, li, ldl, info, (hipStream_t)stream);
}

}  // extern "C"
