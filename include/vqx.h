/*
 * vqx — MI355X (gfx950) kernels for the Voyager quantization hot path.
 *
 * C ABI of libvqx.so.  Every pointer argument named as a tensor is a device
 * pointer (hipMalloc / torch CUDA-device memory) unless stated otherwise; sizes
 * are element counts.  Every call enqueues work on `stream` and returns
 * without synchronizing; it returns VQX_OK (0) or a negative status, with a
 * message from vqx_last_error() (thread-local).  The library keeps no device
 * allocations of its own: callers own every buffer.
 *
 * Reference interfaces (paths relative to the voyager-compiler repository,
 * src/vc = src/voyager_compiler) are cited on each entry point.
 */
#ifndef VQX_H_
#define VQX_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* vqx_stream_t; /* hipStream_t; NULL = the default stream */

enum {
  VQX_OK = 0,
  VQX_ERR_INVALID = -1,     /* bad argument: shape, dtype, alignment, format */
  VQX_ERR_LAUNCH = -2,      /* HIP runtime / kernel launch failure */
  VQX_ERR_UNSUPPORTED = -3, /* valid request this build does not implement */
};

/* dtype tags */
enum {
  VQX_F32 = 0,
  VQX_BF16 = 1,
  VQX_F16 = 2,
  VQX_U8 = 3,
};

/* Element format kinds (the dtype strings get_quantization_map accepts,
 * src/vc/quantization/fake_quantize.py:30-98). */
enum {
  VQX_FMT_IDENTITY = 0, /* "float32", "bfloat16" */
  VQX_FMT_FP16 = 1,     /* "float16" */
  VQX_FMT_INT = 2,      /* "int<n>" / "uint<n>":   p0 = n, p1 = signed (1) */
  VQX_FMT_FP = 3,       /* "fp<N>_e<E>m<M>":       p0 = E, p1 = M, max_norm */
  VQX_FMT_NV_FP8 = 4,   /* "e4m3" / "e5m2":        p0 = 4 or 5 */
  VQX_FMT_POSIT = 5,    /* "posit<n>_<es>":        p0 = n, p1 = es */
  VQX_FMT_LEVELS = 6,   /* "nf<k>[_<b>]", codebook tables: levels + code table */
  VQX_FMT_TABLE = 7,    /* any 65536-entry bf16 table (a user qmap); no codes */
};

#define VQX_FLAG_UNSIGNED 1 /* fp<N>_e<E>m<M> with N == E + M */

/* Format descriptor.  Host struct; its table pointers are device pointers,
 * read only for VQX_FMT_LEVELS (boundaries, levels, code_table) and
 * VQX_FMT_TABLE (value_table). */
typedef struct vqx_format {
  int32_t kind;
  int32_t p0;
  int32_t p1;
  int32_t flags;
  float max_norm;
  int32_t code_bits;           /* width of one packed code: 4, 6, 8 or 16 */
  const float* boundaries;     /* LEVELS: nlevels-1 fp32 boundaries */
  const uint16_t* levels;      /* LEVELS: nlevels bf16 level patterns */
  const uint8_t* code_table;   /* LEVELS: 65536 codes, one per bf16 pattern */
  const uint16_t* value_table; /* TABLE: 65536 bf16 values, one per bf16 pattern */
  const uint32_t* lut;         /* optional: table blob from vqx_build_lut (formats with
                                  codes of at most 8 bits); NULL = closed form only */
  int32_t lut_len;             /* that blob's entries per sign (blob word 4) */
} vqx_format;

/* Where element i of x finds its scale / zero point.  x is viewed as
 * [outer, L, inner] (i = (o * L + l) * inner + in) and reads
 * scale[o * s_o + (l / block) * s_l + in * s_in]; strides of 0 broadcast.
 * Per-tensor: all strides 0.  Per-channel along the middle axis: block 1,
 * s_l 1.  Blocks of `block` along L: s_o = ceil(L/block) * inner,
 * s_l = inner, s_in = 1.  scale / zero_point are in x's dtype. */
typedef struct vqx_scale_map {
  const void* scale;
  const void* zero_point; /* optional */
  int64_t L, inner, block;
  int64_t s_o, s_l, s_in;
} vqx_scale_map;

/* Library version string. */
const char* vqx_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* vqx_last_error(void);

/* Number of compute units of the current device (used for launch sizing). */
int vqx_device_cus(void);

/*
 * quantized_ops::vmap  (src/vc/ops/quantized.py:98-121)
 * y[i] = table[bf16_bits(x[i])], returned in x's dtype.  x: n elements of
 * x_dtype (F32, BF16, F16); table: 65536 bf16 patterns; y: n elements of x_dtype.
 */
int vqx_vmap(const void* x, int32_t x_dtype, int64_t n, const uint16_t* table, void* y,
             vqx_stream_t stream);

/*
 * FusedAmaxObsFakeQuantize.forward with the observer on, per-tensor or
 * per-channel qscheme (src/vc/quantization/fake_quantize.py:308-341 observer
 * step, :418-426 forward, :112-115 fake-quant), on the device and without a
 * host synchronisation.  Element i of x belongs to channel
 * (i / inner) % channels (channels = 1: per-tensor).  amax_history: fp32
 * [history_len, channels] and scale: fp32 [channels], read and updated in
 * place exactly as the reference updates its buffers: the scale is the
 * history's maximum from before this step divided by quant_max (IEEE fp32),
 * kept where that maximum is not positive or not finite, optionally
 * 2 ** ceil(log2(scale)) as torch computes it on the CPU; the history is
 * rolled by one and row 0 becomes this step's max |x| per channel (NaN if
 * any element is NaN).  y (NULL: observe only) = vmap(x / s, qmap) * s with
 * the new scale s in x's dtype.  Two launches (the scales, then one pass over
 * x).  n > 0, a multiple of channels * inner.
 */
int vqx_amax_observe_fake_quant(const void* x, int32_t x_dtype, int64_t n, int64_t channels, int64_t inner,
                                const vqx_format* fmt, float* amax_history, int32_t history_len, float* scale,
                                float quant_max, int32_t force_scale_power_of_two, void* y, vqx_stream_t stream);

/*
 * FakeQuantizeFunction.forward  (src/vc/quantization/fake_quantize.py:101-115)
 * and quantized_ops::quantize without block_size (src/vc/ops/quantized.py:131-172):
 *   y = vmap(x / s, qmap) * s   (mul_back = 1)   or   y = vmap(x / s, qmap)
 * with the format's table computed in closed form.  scale: NULL (s = 1) or
 * scale_numel fp32 values; element i uses scale[(i / scale_inner) % scale_numel].
 * codes (optional, NULL to skip): one code per element, code_bytes (1 or 2)
 * wide: posit/int two's complement, fp OCP-style bits, level index.
 */
int vqx_fake_quant(const void* x, int32_t x_dtype, int64_t n, const vqx_format* fmt,
                   const float* scale, int64_t scale_numel, int64_t scale_inner,
                   int32_t mul_back, void* y, void* codes, int32_t code_bytes,
                   vqx_stream_t stream);

/*
 * quantized_ops::quantize  (src/vc/ops/quantized.py:124-172) with any scale
 * layout: y = vmap(x / s [+ zp], qmap) with the format (or a TABLE format for
 * an arbitrary qmap), every op rounded to x's dtype (F32, BF16, F16).
 * mul_back = 1 multiplies back (y = vmap(...) * s: fake-quant).
 * codes: optional, code_bytes (1 or 2) per element.
 */
int vqx_quantize_mapped(const void* x, int32_t x_dtype, int64_t n, const vqx_format* fmt,
                        const vqx_scale_map* sm, int32_t mul_back, void* y, void* codes,
                        int32_t code_bytes, vqx_stream_t stream);

/*
 * quantized_ops::dequantize  (src/vc/ops/quantized.py:175-227):
 * y = out_map((in_map(x) [- zp]) * s), in_map / out_map optional 65536-entry
 * bf16 tables (input_qmap / output_qmap), every op in x's dtype.
 */
int vqx_dequantize_mapped(const void* x, int32_t x_dtype, int64_t n, const uint16_t* input_qmap,
                          const vqx_scale_map* sm, const uint16_t* output_qmap, void* y,
                          vqx_stream_t stream);

/*
 * get_quantization_map  (src/vc/quantization/fake_quantize.py:30-98)
 * values[h] = the format's value for bf16 pattern h (65536 bf16 patterns);
 * codes[h] (optional) = its code.
 */
int vqx_build_table(const vqx_format* fmt, uint16_t* values, uint16_t* codes,
                    vqx_stream_t stream);

/* Bytes of the table blob vqx_build_lut writes. */
int64_t vqx_lut_bytes(void);

/*
 * Compact code/value table of a format (codes of at most 8 bits) for the
 * streaming kernels: blob word 0 = 1 if usable, word 4 = entries per sign
 * (copy it to fmt->lut_len).  Built on the GPU from the closed-form encoder,
 * so a kernel using it gives the same results.  blob: vqx_lut_bytes() bytes.
 */
int vqx_build_lut(const vqx_format* fmt, uint32_t* blob, vqx_stream_t stream);

/*
 * Level-set tables for quantize_to_nf (src/vc/quantization/dtypes/normal_float.py:54-60,
 * mode 0: bf16 arithmetic) and codebook_qmap (src/vc/quantization/lcq.py:270-291,
 * mode 1: fp32 arithmetic).  levels: K fp32 values (the bf16 levels for mode 0).
 * Writes index_table[65536] (argmin index per bf16 pattern) and boundaries[K-1];
 * work: K uint32 scratch; bad: one int, set to the number of patterns whose
 * index the boundaries do not reproduce (0 = the level set is monotone).
 */
int vqx_level_tables(const float* levels, int32_t K, int32_t mode, uint8_t* index_table,
                     float* boundaries, uint32_t* work, int32_t* bad, vqx_stream_t stream);

/*
 * quantized_ops::calculate_mx_qparam + quantize / quantize_mx fused
 * (src/vc/ops/quantized.py:435-529) and MXFakeQuantizeFunction.forward
 * (src/vc/quantization/fake_quantize.py:123-153).
 * x viewed as [outer, L, inner] with blocks of block_size along L.
 * scale_mode 0: power of two, pow2_shift = floor(log2(quant_max));
 * scale_mode 1: absmax / quant_max, then scale_qmap (65536 bf16, optional).
 * Outputs (each optional): scale_out [outer, ceil(L/bs), inner] in x's dtype;
 * scale_f32 (same shape, fp32); scale_e8m0 (uint8, power-of-two mode only);
 * qvals [n] in x's dtype = quantize()'s output; fq [n] = qvals * scale;
 * codes: code_layout 0 = packed bitstream of fmt->code_bits per element
 * (element i at bits [cb*i, cb*i+cb), little endian; needs inner == 1,
 * block_size 16, 32, 64 or 128 dividing L, 16-byte aligned buffers),
 * 1 / 2 = one uint8 / uint16 per element.
 */
int vqx_mx_quantize(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner,
                    int64_t block_size, const vqx_format* fmt, int32_t scale_mode,
                    int32_t pow2_shift, float quant_max, const uint16_t* scale_qmap,
                    void* scale_out, float* scale_f32, uint8_t* scale_e8m0, void* qvals,
                    void* fq, void* codes, int32_t code_layout, vqx_stream_t stream);

/*
 * FakeQuantize outlier masking (FusedAmaxObsFakeQuantize.forward,
 * src/vc/quantization/fake_quantize.py:373-395).  An element is an outlier
 * when |x| >= t, compared in x's dtype (t rounded to it, as torch casts the
 * threshold); a NaN t skips nothing, a t <= -0 every non-NaN element.  t is
 * read from threshold_dev (fp32, device) when it is not NULL, else it is
 * `threshold`.
 * stats (optional): vqx_outlier_stats_size bytes of 256-byte aligned device
 * memory, zeroed once by the caller, that keep the largest fraction of
 * outliers seen (max_outlier_pct, :389-391; count / numel as Python divides).
 * A call counts into one of two sets, named by stats_parity; calls sharing a
 * buffer must be ordered (one stream) and alternate parities.  Each call
 * folds the other set (the previous call's) into the fp64 at byte offset 0.
 * Set p starts at byte 256 + 2176 p: its uint64 numel (the last call's
 * element count), then 16 uint64 partial counts 128 bytes apart (bytes
 * 128, 256, ..., 2048 of the set).  The current fraction is the maximum of
 * the fp64 and the last call's set (sum of its counts / its numel).
 */
int vqx_outlier_stats_size(int64_t* bytes);

/*
 * The outlier_pct threshold (fake_quantize.py:373-387): the k-th largest |x|
 * (torch.topk(|x|, k).values.min(); NaN when x holds a NaN), k in [1, n],
 * then written to *threshold (fp32, device): ema 0 stores it, ema 1 updates
 * *threshold = *threshold * decay + (value * one_minus_decay rounded to x's
 * dtype), in fp32 (F32, BF16 or F16 x; 16-byte aligned).  workspace:
 * vqx_outlier_topk_workspace_size bytes of 16-byte aligned device memory,
 * zeroed once before its first use (calls leave it ready for the next);
 * calls sharing one workspace must be ordered.
 */
int vqx_outlier_topk_workspace_size(int64_t* bytes);
int vqx_outlier_topk_threshold(const void* x, int32_t x_dtype, int64_t n, int64_t k, int32_t ema, float decay,
                               float one_minus_decay, float* threshold, void* workspace, int64_t workspace_bytes,
                               vqx_stream_t stream);

/*
 * MXFakeQuantizeFunction.forward between the outlier mask and restore
 * (fake_quantize.py:388-395 around :397-408) in one pass: vqx_mx_quantize's
 * fake-quant values and scale of x with its outliers zeroed, the outliers
 * written back unchanged into fq, and counted into stats.  Same geometry and
 * scale arguments as vqx_mx_quantize; the scale goes to scale_out (x's
 * dtype) and / or scale_f32 (its value in fp32), each optional.
 */
int vqx_mx_fake_quant_outlier(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner,
                              int64_t block_size, const vqx_format* fmt, int32_t scale_mode, int32_t pow2_shift,
                              float quant_max, const uint16_t* scale_qmap, const float* threshold_dev,
                              float threshold, void* stats, int32_t stats_parity, void* scale_out,
                              float* scale_f32, void* fq, vqx_stream_t stream);

/*
 * The mask and the restore around the other quantization schemes
 * (fake_quantize.py:388-391, :429-430): masked = x.masked_fill(|x| >= t, 0)
 * (optional: with masked NULL only the count is taken, into stats), and
 * y[i] = x[i] where x[i] is an outlier (y is written only there).  F32, BF16
 * or F16; 16-byte aligned x and masked.
 */
int vqx_outlier_mask(const void* x, int32_t x_dtype, int64_t n, const float* threshold_dev, float threshold,
                     void* stats, int32_t stats_parity, void* masked, vqx_stream_t stream);
int vqx_outlier_restore(const void* x, int32_t x_dtype, int64_t n, const float* threshold_dev, float threshold,
                        void* y, vqx_stream_t stream);

/*
 * quantized_ops::dequantize with input_qmap (src/vc/ops/quantized.py:175-227),
 * on packed codes: out[i] = decode_table[code(i)] * scale[i / block_size],
 * rounded to out_dtype (F32 or BF16).  scale_kind 0 = fp32, 1 = bf16,
 * 2 = E8M0 uint8.  decode_table: ntab bf16 values indexed by code.
 */
int vqx_mx_decode(const uint8_t* codes, int32_t code_bits, const uint16_t* decode_table,
                  int32_t ntab, const void* scale, int32_t scale_kind, int64_t n,
                  int64_t block_size, void* out, int32_t out_dtype, vqx_stream_t stream);

/*
 * GroupWiseAffineFakeQuantFunction.forward
 * (src/vc/quantization/fake_quantize.py:162-211), the group_wise_affine
 * qscheme's fake-quant (e.g. uint2 KV caches).  x viewed as [outer, L, inner]
 * with blocks of block_size along L (a short last block is zero-padded, as
 * mx_utils.py:62-108 pads it).  Per block: sf = (max - min) / (quant_max -
 * quant_min), 1 where not > 0; zp = -min / sf + quant_min; both through
 * scale_qmap when given; y = (clamp(round(x / sf + zp), quant_min, quant_max)
 * - zp) * sf, every step rounded to x's dtype (BF16 or F32) as torch does.
 * scale_out / zero_point_out (optional): [outer, ceil(L/bs), inner] in x's dtype.
 */
int vqx_gwa_fake_quant(const void* x, int32_t x_dtype, int64_t outer, int64_t L, int64_t inner,
                       int64_t block_size, float quant_min, float quant_max, const uint16_t* scale_qmap,
                       void* scale_out, void* zero_point_out, void* y, vqx_stream_t stream);

/* decode_table[code] = value of the format, for codes < ntab. */
int vqx_decode_table(const vqx_format* fmt, uint16_t* decode_table, int32_t ntab,
                     vqx_stream_t stream);

/*
 * Per-channel codebook encode (the per-row form of codebook_qmap + vmap,
 * src/vc/quantization/lcq.py:270-291, src/vc/ops/quantized.py:101-121):
 * codes[r, c] = argmin_k |clamp(bf16(x[r, c])) - cb[r, k]| in fp32, lowest k
 * on ties, NaN -> 0.  cb: [rows, K] fp32, each row sorted ascending, K <= 256.
 * x: [rows, cols] F32 or BF16, cols % 16 == 0.
 */
int vqx_codebook_encode(const void* x, int32_t x_dtype, int64_t rows, int64_t cols,
                        const float* cb, int32_t K, uint8_t* codes, vqx_stream_t stream);

/* out[r, c] = bf16(cb[r, codes[r, c]]) stored as out_dtype (F32 or BF16). */
int vqx_codebook_decode(const uint8_t* codes, int64_t rows, int64_t cols, const float* cb,
                        int32_t K, void* out, int32_t out_dtype, vqx_stream_t stream);

/*
 * quantized_ops::linear_mx with an NF4 block-64 weight, dequant fused into the
 * product (src/vc/ops/quantized.py:286-348: decoded = weight_code[codes] *
 * expand(weight_scale), then aten.linear):
 *   out[M, N] = A[M, K] . W[N, K]^T + bias,  W[n, k] = bf16(levels[c] * scale[n, k/64])
 * A: bf16 row-major [M, K]; codes: packed 4-bit [N, K/2] (low nibble = even k);
 * scale: fp32 [N, K/64]; levels: 16 bf16 patterns; bias: bf16 [N] or NULL;
 * out: bf16 [M, N], fp32 accumulation.  Any M >= 1: M <= 16 runs a skinny
 * kernel bound by the weight's bytes (any N); larger M the bf16 MFMA tile
 * kernel (256 x 128 tiles, a partial last row tile; needs N % 128 == 0).
 * K % 64 == 0 always (VQX_ERR_UNSUPPORTED otherwise).
 */
int vqx_nf4_linear(const uint16_t* A, const uint8_t* codes, const float* scale, const uint16_t* levels,
                   const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K,
                   vqx_stream_t stream);

/*
 * The same product (src/vc/ops/quantized.py:286-348) with a caller-owned
 * workspace, which lets the M > 16 tile kernel balance its last round: when
 * the count of 256 x 128 tiles is not a multiple of the CU count, the last
 * round's tiles are split along K over all CUs (stream-K) and their fp32
 * partial sums meet in the workspace.  Sums are added in a fixed order, so
 * the result is deterministic; it can differ from vqx_nf4_linear's in the
 * last bf16 bit where the fp32 grouping of a sum differs.
 * vqx_nf4_linear_workspace_size gives the bytes needed on the current device
 * (0: the shape runs whole tiles only and workspace may be NULL).  workspace:
 * 256-byte aligned device memory, no initial contents needed; calls that
 * share one workspace must be ordered (one stream).
 */
int vqx_nf4_linear_workspace_size(int64_t M, int64_t N, int64_t K, int64_t* bytes);
int vqx_nf4_linear_ws(const uint16_t* A, const uint8_t* codes, const float* scale, const uint16_t* levels,
                      const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K, void* workspace,
                      int64_t workspace_bytes, vqx_stream_t stream);

/*
 * vqx_nf4_linear_ws without a workspace argument and without any allocation:
 * the same product, the same stream-K plan and therefore the same bits.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The workspace is a device array of the library,
 * 64 MiB + 1 KiB, which each GPU the library runs on holds until the process
 * ends; a shape whose plan needs more (a device with more than 256 CUs)
 * returns VQX_ERR_UNSUPPORTED.  Every call on one GPU shares that array: the
 * call clears what must start at zero on `stream` before using it, and calls
 * that overlap on one GPU (other streams, other threads) race.
 */
int vqx_nf4_linear_noalloc(const uint16_t* A, const uint8_t* codes, const float* scale, const uint16_t* levels,
                           const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K,
                           vqx_stream_t stream);

/*
 * The operands of vqx_nf4_linear from the convert format that linear_mx /
 * matmul_mx receive after convert_pt2e (src/vc/quantization/quantize_pt2e.py:
 * 456-508 stores the weight as integer-valued code indices in a float tensor,
 * the levels as weight_code and one scale per 64-element block along K;
 * src/vc/ops/quantized.py:319-326 decodes them as
 * weight_code[weight.to(long)] * expand(weight_scale)).
 * weight: [N, K] (transposed = 0, linear_mx "kc" / matmul_mx "kc") or [K, N]
 * (transposed = 1, "ck"), dtype F32, BF16 or F16; scale: [N, K/64] or
 * [K/64, N] in F32, BF16 or F16, or NULL (all ones).  Writes codes: packed
 * 4-bit [N, K/2] (8-byte aligned) and scale_out: fp32 [N, K/64], which widen
 * the scale exactly.  Index = trunc(w), a negative index counting from the
 * end of the ncode-entry table (1..16); a NaN, an infinity or an index out of
 * range sets *bad to 1 (device int, cleared by the caller; the reference
 * raises IndexError there).  K % 64 == 0.
 */
int vqx_nf4_pack_weight(const void* weight, int32_t w_dtype, const void* scale, int32_t s_dtype, int64_t N,
                        int64_t K, int32_t transposed, int32_t ncode, uint8_t* codes, float* scale_out,
                        int32_t* bad, vqx_stream_t stream);

/*
 * One operand of vqx_mx_matmul in the convert format, read in place: `data`
 * holds bf16 values, or integer-valued bf16 code indices when `code` is set;
 * the decoded operand is bf16(code[trunc(data)] * scale[block]) with either
 * part optional, as src/vc/ops/quantized.py:313-326 (linear_mx) and :388-398
 * (matmul_mx) decode it.  An index outside the code table (the reference
 * raises IndexError) decodes to NaN.
 *   k_major = 1: rows of K contiguous values, row r at data + r * ld;
 *                scales [rows][ceil(K / block_size)], row r at
 *                scale + r * scale_ld.
 *   k_major = 0: K rows of contiguous columns, k row at data + k * ld (right
 *                operand only); scales [ceil(K / block_size)][cols], block
 *                row at scale + j * scale_ld (16-byte aligned, scale_ld and
 *                scale_batch_stride multiples of 8).
 * batch_stride / scale_batch_stride: elements between batch items (0: the
 * same matrix for every item).  data 16-byte aligned, ld and batch_stride
 * multiples of 8; block_size a power of two >= 8; code: bf16, code_len
 * 1..256 entries.
 */
typedef struct VqxMxOperand {
  const void* data;
  const void* scale;
  const void* code;
  int64_t batch_stride;
  int64_t ld;
  int64_t scale_batch_stride;
  int64_t scale_ld;
  int32_t k_major;
  int32_t block_size;
  int32_t code_len;
  int32_t reserved;
} VqxMxOperand;

/*
 * The dense product of linear_mx / matmul_mx (src/vc/ops/quantized.py:
 * 295-348 and 371-421) with both operands decoded inside the kernel:
 * out[b][M][N] = A'[b] . B'[b] (+ bias), fp32 accumulation, bf16 out
 * (contiguous, 8-byte aligned).  a: the left operand [M][K], k_major = 1;
 * b: the right operand, [N][K] (k_major = 1: linear_mx "kc", matmul_mx
 * "kc") or [K][N] (k_major = 0: matmul_mx "ck", linear_mx "ck").  bias: bf16
 * [N] (8-byte aligned) or NULL.  K % 8 == 0, N % 4 == 0 (N % 8 == 0 when
 * b is N-major).  Replaces the decode + aten.linear / aten.matmul sequence
 * for operands outside vqx_nf4_linear's format (code tables of more than
 * 16 entries, no code table, blocks other than 64, coded activations,
 * batched right operands).
 */
int vqx_mx_matmul(const VqxMxOperand* a, const VqxMxOperand* b, const uint16_t* bias, uint16_t* out,
                  int64_t batch, int64_t M, int64_t N, int64_t K, vqx_stream_t stream);

/*
 * The operand decode of linear_mx / matmul_mx (src/vc/ops/quantized.py:
 * 313-326, 388-398) on its own: x (a VqxMxOperand: k_major = 1 for
 * [rows][K], 0 for [K][rows]) decoded to dense bf16 in the same layout,
 * out contiguous [batch][rows][K] or [batch][K][rows] (16-byte aligned).
 * The host runs it ahead of vqx_mx_matmul for an operand that many output
 * tiles read (decoding once instead of once per tile).  K % 8 == 0;
 * rows % 8 == 0 when k_major = 0.
 */
int vqx_mx_operand_decode(const VqxMxOperand* x, int64_t batch, int64_t rows, int64_t K, uint16_t* out,
                          vqx_stream_t stream);

/*
 * quantized_ops::filter_outlier (src/vc/ops/quantized.py:532-630, with
 * _pad_csr at :537-569), and the outlier half of quantize_mx_outlier
 * (:633-712, indptr_offset added to the row pointers).
 * x: [batches, rows, cols] F32, BF16 or F16.  An outlier is an element with
 * |x| > threshold and x != 0, threshold given already rounded to x's dtype
 * (torch casts the Python scalar to the tensor's dtype before comparing).
 * Outputs per batch b, each matrix's outliers in row-major order:
 *   inlier [batches, rows, cols]  x with outliers replaced by +0
 *   indptr [batches, rows + 1]    int32, min(prefix count, max_nnz) + indptr_offset
 *                                 (int32 wrap-around)
 *   data, indices [batches, max_nnz]  values (x's dtype) and int32 columns of
 *                                 the first max_nnz outliers; unused slots 0 / -1.
 */
int vqx_filter_outlier(const void* x, int32_t x_dtype, int64_t batches, int64_t rows, int64_t cols,
                       float threshold, int64_t max_nnz, int32_t indptr_offset, void* data, int32_t* indices,
                       int32_t* indptr, void* inlier, vqx_stream_t stream);

/*
 * quantized_ops::quantize_mx_outlier in one pass over the inliers
 * (src/vc/ops/quantized.py:649-699): the CSR of filter_outlier (as
 * vqx_filter_outlier, row pointers + indptr_offset), then for each block of
 * block_size (8, 16, 32 or 64; cols % block_size == 0) inliers along a row
 * the block's scale as calculate_mx_qparam forms it (scale_mode 0: power of
 * two with shift = floor(log2(quant_max)); 1: amax / quant_max through
 * scale_qmap when given) and values = qmap[bf16(inlier / scale)], without
 * writing the inliers.  x, data, scale, values: BF16 only; x and values
 * 16-byte aligned; scale [batches * rows, cols / block_size]; values like x.
 */
int vqx_quantize_mx_outlier(const void* x, int64_t batches, int64_t rows, int64_t cols, float threshold,
                            int64_t max_nnz, int32_t indptr_offset, int64_t block_size, int32_t scale_mode,
                            int32_t shift, float quant_max, const uint16_t* scale_qmap, const uint16_t* qmap,
                            void* data, int32_t* indices, int32_t* indptr, void* scale, void* values,
                            vqx_stream_t stream);

/*
 * One-pass forms of vqx_filter_outlier and vqx_quantize_mx_outlier (same
 * arguments, same outputs bit for bit), which read x once: the first launch
 * writes the inliers (or the quantized inliers and their scales), each row's
 * outlier count, and the row's first outliers to staging slots in
 * `workspace`; the second places them behind the row pointers, reading again
 * only the rows whose outliers did not fit their slots, and pads the unused
 * entries.  Same reference interfaces as the two entry points above
 * (src/vc/ops/quantized.py:532-630, :633-712).
 * Matrices of more than 16384 rows take the two-pass form instead (the
 * second launch's reads would grow as rows^2), and ignore the workspace.
 * vqx_outlier_workspace_size gives the bytes for the default slots per row
 * (0 when batches * rows == 0 or rows > 16384; workspace may then be NULL).
 * Otherwise any workspace of
 * at least the 256-byte-aligned 4 * batches * rows bytes of the counts works:
 * the rest sets the slots per row (fewer slots, more rows read again).
 * workspace: 256-byte aligned device memory, contents ignored; calls that
 * share one workspace must be ordered (one stream).
 */
int vqx_outlier_workspace_size(int32_t x_dtype, int64_t batches, int64_t rows, int64_t cols, int64_t max_nnz,
                               int64_t* bytes);
int vqx_filter_outlier_ws(const void* x, int32_t x_dtype, int64_t batches, int64_t rows, int64_t cols,
                          float threshold, int64_t max_nnz, int32_t indptr_offset, void* data, int32_t* indices,
                          int32_t* indptr, void* inlier, void* workspace, int64_t workspace_bytes,
                          vqx_stream_t stream);
int vqx_quantize_mx_outlier_ws(const void* x, int64_t batches, int64_t rows, int64_t cols, float threshold,
                               int64_t max_nnz, int32_t indptr_offset, int64_t block_size, int32_t scale_mode,
                               int32_t shift, float quant_max, const uint16_t* scale_qmap, const uint16_t* qmap,
                               void* data, int32_t* indices, int32_t* indptr, void* scale, void* values,
                               void* workspace, int64_t workspace_bytes, vqx_stream_t stream);

/*
 * quantized_ops::slice_csr_tensor (src/vc/ops/quantized.py:715-777) of one CSR
 * matrix: data [nnz] (F32, BF16 or F16), indices [nnz] int32, indptr [rows + 1]
 * int32 starting at 0; entries past indptr[rows] are padding (index -1).
 * dim 0: rows [start, end), 0 <= start <= end <= rows; indptr_out [end - start + 1].
 * dim 1: columns [start, end), start >= 0, indices rebased by -start;
 *        indptr_out [rows + 1].
 * data_out / indices_out [max_nnz]: the kept entries in order, padded with
 * 0 / -1; past max_nnz they are dropped and indptr_out clamped to max_nnz.
 */
int vqx_slice_csr(const void* data, int32_t dtype, const int32_t* indices, const int32_t* indptr, int64_t nnz,
                  int64_t rows, int32_t dim, int64_t start, int64_t end, int64_t max_nnz, void* data_out,
                  int32_t* indices_out, int32_t* indptr_out, vqx_stream_t stream);

/*
 * The weight decode of quantized_ops::spmm_csr (src/vc/ops/quantized.py:816-836):
 * B [batches, rows, cols] (F32, BF16, F16 or U8) ->
 *   v = code ? code[trunc(B)] : B        (negative index from the end; out of range -> NaN)
 *   v = scale ? round_out(v * scale[b * scale_batch_stride + (r / row_block) * scale_cols
 *                                   + c / col_block]) : v
 * stored as out_dtype (F32, BF16 or F16: the dtype torch's decode produces),
 * transposed to [batches, cols, rows] when transpose != 0 (the "kc" layout).
 * scale_rows / scale_cols must cover B through row_block / col_block.
 */
int vqx_csr_decode_weight(const void* B, int32_t B_dtype, int64_t batches, int64_t rows, int64_t cols,
                          int32_t transpose, const void* code, int32_t code_dtype, int64_t code_len,
                          const void* scale, int32_t scale_dtype, int64_t scale_batch_stride, int64_t scale_rows,
                          int64_t scale_cols, int64_t row_block, int64_t col_block, void* out, int32_t out_dtype,
                          vqx_stream_t stream);

/*
 * quantized_ops::spmm_csr product (src/vc/ops/quantized.py:838-878):
 *   out[b, r, n] = round_B(sum over the row's entries p, in order, of
 *                  fp32(data[b, p]) * B[b, indices[b, p], n])
 * accumulated in fp32; with an addend, out = round_B(addend + round_B(sum))
 * (the dense + sparse sum of linear_mx / matmul_mx, :335-348, :408-420).
 * data / indices [batches, nnz_stride]; indptr [batches, rows + 1], a batch's
 * entries at positions indptr[b][r] - indptr[b][0] (row pointers lifted out
 * of a longer array).  B: [K, N] row-major (F32, BF16 or F16; also the
 * output dtype) at B + b * B_batch_stride (0 = shared).  Entries whose index
 * is outside [0, K) add nothing; positions are clamped to [0, nnz_stride).
 */
int vqx_spmm_csr(const void* data, int32_t data_dtype, const int32_t* indices, const int32_t* indptr,
                 int64_t batches, int64_t rows, int64_t nnz_stride, const void* B, int32_t B_dtype,
                 int64_t B_batch_stride, int64_t K, int64_t N, const void* addend, void* out, vqx_stream_t stream);

/*
 * LCQ calibration statistics: Histogram.add (src/vc/quantization/lcq.py:44-119),
 * optionally fused with unit_scale (:136-150) as _accumulate (:603-626) applies it.
 * block_size = 0: v[i] = x[i];  block_size > 0 (n % block_size == 0):
 * v[i] = x[i] / (max(amax |block|, 1e-12) / quant_max), fp32, IEEE division.
 * bin = (number of edges <= v) - 1 clamped to [0, bins - 1] (torch.bucketize
 * right=True; NaN counts every edge); with w = weights[i % weights_period]
 * (weights NULL: w = 1):  weight[bin] += w, total[bin] += w v,
 * square[bin] += (w v) v, in fp64, added to what the arrays hold (zero them
 * before the first call).  x: n elements, F32, BF16 or F16; edges: bins + 1
 * ascending fp32 values; bins <= 4096; weight / total / square: bins doubles.
 * The fp64 sums are added in an unspecified order (as index_add_ on a GPU).
 */
int vqx_lcq_histogram(const void* x, int32_t x_dtype, int64_t n, int64_t block_size, float quant_max,
                      const float* weights, int64_t weights_period, const float* edges, int32_t bins,
                      double* weight, double* total, double* square, vqx_stream_t stream);

/*
 * The column loop of GPTQ's compensate_weight for one microscaling block
 * (src/vc/quantization/gptq.py:241-262).  work, out: fp32 [rows, ld] row-major;
 * the block is columns col0 .. col0 + ncols - 1 (ncols <= 64).  For each row r
 * and block column j in order, c = col0 + j:
 *   q = float(qmap[bf16(w[r, c] / s[r])]) * s[r];  out[r, c] = q
 *   d = (w[r, c] - q) / max(hinv[c, c], 1e-12);    deltas[r, j] = d
 *   w[r, c + k] -= d * hinv[c, c + k] for the block's later columns (on a
 *   private copy: work is not written)
 * each operation rounded to fp32 as torch performs it (no fused multiply-add).
 * s[r] = scale[r] when scale is given (fp32 [rows]); with scale NULL the
 * kernel forms block_scale's unshrunk scale from the block's current weights
 * (gptq.py:103-113 through calculate_mx_qparam, quantized.py:491-498):
 * amax over the block (NaN propagates) / quant_max, through scale_qmap
 * (65536 bf16 patterns) when given, 1 where not positive, at least 1e-12.
 * hinv: fp32 upper Cholesky factor of the inverse Hessian, row stride ldh;
 * qmap: 65536 bf16 patterns, 16-byte aligned; deltas: fp32, row stride
 * ldd >= ncols.
 */
int vqx_gptq_block(const float* work, int64_t rows, int64_t ld, int64_t col0, int32_t ncols, const float* scale,
                   float quant_max, const uint16_t* scale_qmap, const float* hinv, int64_t ldh,
                   const uint16_t* qmap, float* out, float* deltas, int64_t ldd, vqx_stream_t stream);

/*
 * One diagonal block of the factorisation behind GPTQ's inverse-Hessian
 * factor (src/vc/quantization/gptq.py:32-71, which calls torch.linalg's
 * cholesky, cholesky_inverse and cholesky).  The host factors the reversed
 * Hessian blockwise with library GEMMs between these blocks.  a: fp32, row
 * stride lda, its lower n x n triangle read (n <= 64); li: fp32, row stride
 * ldl, receives the inverse of the lower Cholesky factor of that block
 * (zeros above the diagonal); *info is set to 1 if a pivot is not positive
 * (the matrix is not positive definite) and left alone otherwise.
 */
int vqx_chol_inverse_block(const float* a, int64_t lda, int32_t n, float* li, int64_t ldl, int32_t* info,
                           vqx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VQX_H_ */
