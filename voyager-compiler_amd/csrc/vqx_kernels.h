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

// Device helpers shared by the MX kernels and the fused outlier split.
// Block scale of a bf16 block, specialised by mode (branch-free).
template <bool ABSMAX>
__device__ __forceinline__ float block_scale_bf16(uint32_t amax, const ScaleParams& sp) {
  if constexpr (!ABSMAX) {
    // e = floor(bf16 log2(amax)) - shift (amax 0 -> -126); 2**e in bf16 keeps
    // 2^-133 .. 2^127 and rounds 2^-134 and below to 0, which becomes 1
    int e = (amax == 0 ? -126 : log2floor_bf16(amax)) - sp.shift;
    float sc = e > 127 ? __builtin_huge_valf() : (e >= -133 ? exp2i(e) : 1.0f);
    sc = amax == 0x7F80u ? __builtin_huge_valf() : sc;
    return amax > 0x7F80u ? 1.0f : sc;
  } else {
    float sc = bf2f(f2bf(bf2f(amax) / sp.quant_max));
    if (sp.scale_qmap) sc = bf2f(f2bf(bf2f(sp.scale_qmap[f2bf(sc)])));
    return sc > 0.0f ? sc : 1.0f;
  }
}

// Max over the LPB adjacent lanes of a block: DPP quad permutes for lane
// distances 1 and 2, a shuffle beyond.
template <int LPB>
__device__ __forceinline__ uint32_t block_max(uint32_t v) {
  if constexpr (LPB >= 2) v = umax32(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
  if constexpr (LPB >= 4) v = umax32(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
  if constexpr (LPB >= 8) v = umax32(v, (uint32_t)__shfl_xor((int)v, 4, 64));
  return v;
}

// ---------------------------------------------------------------------------
// FakeQuantize outlier masking (quantization/fake_quantize.py:373-395): the
// elements with |x| >= threshold are left out of the quantization (zeroed
// before it, so they drop out of block maxima) and come back unchanged after
// it; the largest skipped fraction seen so far is kept on the device.
// ---------------------------------------------------------------------------
// Device state of the skipped-element counts (kOutlierStatsBytes, zeroed
// once by the caller).  A launch adds its count into the 16 slots of the set
// its parity names (workgroup i into slot i % 16, one fire-and-forget atomic
// each, the slots 128 bytes apart so they do not contend), and its workgroup
// 0 records the launch's numel there and folds the other set (the previous
// launch's, complete by then) into `best`, then clears it.  Launches that
// share a stats buffer alternate parities; the host folds the last launch's
// set when it reads the fraction.
constexpr int kOutlierSlots = 16;
constexpr int kOutlierStride = 128;                                     // bytes between slots
constexpr int kOutlierBest = 0;                                         // fp64 bits of the largest fraction
constexpr int kOutlierSet0 = 256;                                       // set p at kOutlierSet0 + p * kOutlierSetBytes
constexpr int kOutlierSetBytes = kOutlierStride * (1 + kOutlierSlots);  // numel, then the slots
constexpr int kOutlierStatsBytes = kOutlierSet0 + 2 * kOutlierSetBytes;
struct OutlierStats;  // opaque: the byte layout above

struct OutlierArgs {
  int32_t active;        // 0: no masking (the other fields unused)
  const float* thr_dev;  // the threshold in device memory (fp32), or null: thr_host
  float thr_host;
  OutlierStats* stats;   // null: nothing counted
  int64_t numel;         // the fraction's denominator (the whole tensor)
  int32_t parity;        // the stats set this launch counts into (0 or 1)
};

// The threshold as a bound on the magnitude bits of x's dtype: |x| >= t is
// compared in x's dtype, so t rounds (RNE) to it first, as torch casts the
// fp32 threshold (or the Python float) to the tensor's dtype.  A NaN t skips
// nothing (0xFFFFFFFF), a t at or below -0 every non-NaN element (0).
// round_bits: fp32 -> the dtype's bits; sign: the dtype's sign bit.
template <typename F>
__device__ __forceinline__ uint32_t outlier_bound(const OutlierArgs& oa, F round_bits, uint32_t sign) {
  const float t = oa.thr_dev ? *oa.thr_dev : oa.thr_host;
  if (t != t) return 0xFFFFFFFFu;
  const uint32_t tb = round_bits(t);
  return (tb & sign) ? 0u : tb;
}

// Whether an element of magnitude bits mag (NaN: above inf) is an outlier.
__device__ __forceinline__ bool outlier_skip(uint32_t mag, uint32_t bound, uint32_t inf) {
  return mag >= bound && mag <= inf;
}

__device__ __forceinline__ unsigned long long* outlier_word(OutlierStats* st, int byte_offset) {
  return reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(st) + byte_offset);
}

// End of an outlier-masking launch: the workgroup's skipped elements (cnt per
// thread) go into a slot of the launch's set with one atomic whose result
// nobody waits for; workgroup 0 also records the launch's numel and folds
// the previous launch's set into the largest fraction (count / numel in
// fp64: both below 2^53, so this is the quotient Python's int / int gives)
// and clears that set.  Every thread of every workgroup calls it once.
__device__ __forceinline__ void outlier_tally(uint32_t cnt, const OutlierArgs& oa) {
  if (!oa.stats) return;
  __shared__ unsigned long long s_tot;
  if (threadIdx.x == 0) s_tot = 0;
  __syncthreads();
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) cnt += (uint32_t)__shfl_xor((int)cnt, o, 64);
  if ((threadIdx.x & 63) == 0 && cnt) atomicAdd(&s_tot, (unsigned long long)cnt);
  __syncthreads();
  if (threadIdx.x != 0) return;
  OutlierStats* st = oa.stats;
  const int cur = kOutlierSet0 + oa.parity * kOutlierSetBytes, prev = kOutlierSet0 + (1 - oa.parity) * kOutlierSetBytes;
  const unsigned bid = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  if (s_tot)
    __hip_atomic_fetch_add(outlier_word(st, cur + kOutlierStride * (1 + (int)(bid % kOutlierSlots))), s_tot,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (bid != 0) return;
  __hip_atomic_store(outlier_word(st, cur), (unsigned long long)oa.numel, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the previous set's numel and slots and the best fraction are read
  // together (one round trip at the end of the launch, not one per word)
  unsigned long long v[kOutlierSlots + 1];
#pragma unroll
  for (int s = 0; s <= kOutlierSlots; ++s)
    v[s] = __hip_atomic_load(outlier_word(st, prev + kOutlierStride * s), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  unsigned long long* best = outlier_word(st, kOutlierBest);
  const double b = __builtin_bit_cast(double, __hip_atomic_load(best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  const unsigned long long n = v[0];
  if (n == 0) return;
  unsigned long long c = 0;
#pragma unroll
  for (int s = 1; s <= kOutlierSlots; ++s) c += v[s];
#pragma unroll
  for (int s = 0; s <= kOutlierSlots; ++s)
    __hip_atomic_store(outlier_word(st, prev + kOutlierStride * s), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const double f = (double)c / (double)n;
  if (f > b) __hip_atomic_store(best, __builtin_bit_cast(unsigned long long, f), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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
int amax_observe_fake_quant(const void* x, int dtype, int64_t n, int64_t C, int64_t inner, const FormatDesc& fmt,
                            float* history, int H, float* scale, float quant_max, bool pow2, void* y,
                            hipStream_t st);
int build_table(const FormatDesc& fmt, uint16_t* values, uint16_t* codes, hipStream_t st);
int build_lut(const FormatDesc& fmt, uint32_t* blob, hipStream_t st);
int level_tables(const float* levels, int K, int mode, uint8_t* index_table, float* boundaries,
                 uint32_t* work, int* bad, hipStream_t st);

// vqx_blockwise.hip
// oa: optional outlier masking (the fake-quant output restores the skipped
// elements; they count as zeros in the block maxima and the other outputs)
int mx_quantize(const void* x, int dtype, int64_t outer, int64_t L, int64_t inner, int64_t bs,
                const FormatDesc& fmt, const ScaleParams& sp, const MxOut& out, int code_layout,
                hipStream_t st, const OutlierArgs* oa = nullptr);
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
             const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K, void* workspace,
             int64_t workspace_bytes, hipStream_t st);
int64_t nf4_gemm_workspace(int64_t M, int64_t N, int64_t K);
int nf4_gemm_noalloc(const uint16_t* A, const uint8_t* codes, const float* scale, const uint16_t* levels,
                     const uint16_t* bias, uint16_t* out, int64_t M, int64_t N, int64_t K, hipStream_t st);
int nf4_pack(const void* weight, int w_dtype, const void* scale, int s_dtype, int64_t N, int64_t K, int transposed,
             int ncode, uint8_t* codes, float* scale_out, int* bad, hipStream_t st);

// vqx_mx_gemm.hip (the layout of VqxMxOperand in vqx.h)
struct MxOperand {
  const void* data;          // bf16 values or integer-valued bf16 code indices
  const void* scale;         // bf16 scales, one per block_size along K, or null
  const void* code;          // bf16 code table of code_len entries, or null
  int64_t batch_stride;      // elements between batch items (0: one matrix for every item)
  int64_t ld;                // elements between rows ([rows][K]) or between k rows ([K][cols])
  int64_t scale_batch_stride;
  int64_t scale_ld;          // scale elements between rows, or between block rows
  int32_t k_major;           // 1: [rows][K], K contiguous; 0: [K][cols]
  int32_t block_size;
  int32_t code_len;
  int32_t reserved;
};
int mx_gemm(const MxOperand& a, const MxOperand& b, const uint16_t* bias, uint16_t* out, int64_t batch, int64_t M,
            int64_t N, int64_t K, hipStream_t st);
int mx_decode(const MxOperand& x, int64_t batch, int64_t rows, int64_t K, uint16_t* out, hipStream_t st);

// vqx_sparse.hip
struct CsrDecode {
  const void* B;        // [nb, br, bc], dtype b_dtype (float tags or kU8)
  int b_dtype;
  int64_t nb, br, bc;
  int transpose;        // out [nb, bc, br] ("kc") or [nb, br, bc] ("ck")
  const void* code;     // optional [code_len] lookup of trunc(B)
  int code_dtype;
  int64_t code_len;
  const void* scale;    // optional; element (b, r, c) -> b*sb_stride + (r/rdiv)*sc + c/cdiv
  int scale_dtype;
  int64_t sb_stride, sr, sc, rdiv, cdiv;
  void* out;
  int out_dtype;        // the decoded dtype; value * scale is rounded to it
};

struct SpmmArgs {
  const void* data;     // [nb, nnz_stride]
  int data_dtype;
  const int32_t* indices;  // [nb, nnz_stride]
  const int32_t* indptr;   // [nb, rows + 1]; a batch's entries start at indptr[b][0]
  int64_t nb, rows, nnz_stride;
  const void* B;        // [.., K, N] row-major, batch stride b_stride (0: shared)
  int b_dtype;          // also the output dtype
  int64_t b_stride, K, N;
  const void* addend;   // optional [nb, rows, N]
  void* out;            // [nb, rows, N]
};

int filter_outlier(const void* x, int dtype, int64_t nb, int64_t rows, int64_t cols, float threshold,
                   int64_t max_nnz, int32_t indptr_offset, void* data, int32_t* indices, int32_t* indptr,
                   void* inlier, hipStream_t st);
int quantize_mx_outlier_fused(const void* x, int64_t nb, int64_t rows, int64_t cols, float threshold,
                              int64_t max_nnz, int32_t indptr_offset, int64_t block_size, const ScaleParams& sp,
                              const uint16_t* qmap, void* data, int32_t* indices, int32_t* indptr, void* scale,
                              void* values, hipStream_t st);
int64_t outlier_stage_slots(int64_t rows, int64_t cols, int64_t max_nnz);
int outlier_workspace_size(int dtype, int64_t nb, int64_t rows, int64_t cols, int64_t max_nnz, int64_t* bytes);
int filter_outlier_ws(const void* x, int dtype, int64_t nb, int64_t rows, int64_t cols, float threshold,
                      int64_t max_nnz, int32_t indptr_offset, void* data, int32_t* indices, int32_t* indptr,
                      void* inlier, void* workspace, int64_t workspace_bytes, hipStream_t st);
int quantize_mx_outlier_fused_ws(const void* x, int64_t nb, int64_t rows, int64_t cols, float threshold,
                                 int64_t max_nnz, int32_t indptr_offset, int64_t block_size, const ScaleParams& sp,
                                 const uint16_t* qmap, void* data, int32_t* indices, int32_t* indptr, void* scale,
                                 void* values, void* workspace, int64_t workspace_bytes, hipStream_t st);
int csr_slice(const void* data, int dtype, const int32_t* indices, const int32_t* indptr, int64_t nnz_in,
              int64_t rows, int dim, int64_t start, int64_t end, int64_t max_nnz, void* data_out,
              int32_t* indices_out, int32_t* indptr_out, hipStream_t st);
int csr_decode(const CsrDecode& d, hipStream_t st);
int spmm_csr(const SpmmArgs& a, hipStream_t st);

// vqx_outlier_fq.hip
int64_t outlier_topk_workspace_bytes();
int outlier_topk_threshold(const void* x, int dtype, int64_t n, int64_t k, int ema, float decay, float omd,
                           float* thr, void* workspace, int64_t workspace_bytes, hipStream_t st);
int outlier_mask(const void* x, int dtype, int64_t n, const OutlierArgs& oa, void* masked, hipStream_t st);
int outlier_restore(const void* x, int dtype, int64_t n, const OutlierArgs& oa, void* y, hipStream_t st);

// vqx_calib.hip
constexpr int kHistMaxBins = 4096;
int lcq_histogram(const void* x, int dtype, int64_t n, int64_t block_size, float quant_max, const float* weights,
                  int64_t weights_period, const float* edges, int bins, double* weight, double* total,
                  double* square, hipStream_t st);
int gptq_block(const float* work, int64_t rows, int64_t ld, int64_t col0, int ncols, const float* scale,
               float quant_max, const uint16_t* scale_qmap, const float* hinv, int64_t ldh, const uint16_t* qmap,
               float* out, float* deltas, int64_t ldd, hipStream_t st);

// Lower Cholesky factor L of the leading n x n block of a (n <= 64, lower
// triangle read) and its inverse into li (zeros above the diagonal); *info
// set to 1 on a non-positive pivot.
int chol_inverse_block(const float* a, int64_t lda, int n, float* li, int64_t ldl, int* info, hipStream_t st);

}  // namespace vqx
