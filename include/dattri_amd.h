/*
 * dattri_amd.h -- C ABI of the MI355X (gfx950) gradient-scoring library.
 *
 * Every entry point takes device pointers, element counts/strides (in
 * elements, int64), a dtype code and a HIP stream (hipStream_t passed as
 * void*), launches stream-ordered work and returns a status code.  Nothing is
 * synchronised and nothing is allocated by the library: temporary storage is a
 * caller-provided workspace whose size the matching *_workspace query returns.
 * All entry points are re-entrant (no global mutable state besides a
 * thread-local error message), so they may be called from concurrent autograd
 * hook threads on different streams.
 *
 * Results are fp32 unless an output dtype is given.  Inputs are never written.
 *
 * Reference interface each entry point replaces is cited as
 * dattri_llm/<file>:<line> (TRAIS-Lab/dattri-llm 0.1.0).
 */
#ifndef DATTRI_AMD_H
#define DATTRI_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. */
enum { DA_F32 = 0, DA_F16 = 1, DA_BF16 = 2 };

/* Status codes.  A non-zero status leaves a message in da_last_error(). */
enum {
  DA_OK = 0,
  DA_ERR_INVALID = 1,     /* bad argument: shape, stride, alignment, size    */
  DA_ERR_UNSUPPORTED = 2, /* valid request this build does not implement     */
  DA_ERR_HIP = 3,         /* a HIP runtime call or kernel launch failed      */
  DA_ERR_WORKSPACE = 4    /* workspace pointer missing or too small          */
};

/* ABI version (bumped on any signature change). */
int da_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* da_last_error(void);

/*
 * One side of a per-sample factor product: B samples, each a set of token
 * rows of an activation factor (width K) and an output-gradient factor
 * (width D).  Two addressing modes:
 *
 *   dense     (seg_offsets == NULL): row t < tokens of sample b is at
 *             act + b*act_bstride + t*act_tstride (elements), likewise grad.
 *   segmented (seg_offsets != NULL, B+1 int32 entries): sample b owns flat
 *             rows [seg_offsets[b], seg_offsets[b+1]); flat row r is physical
 *             row p = row_index ? row_index[r] : r, found at
 *             act + p*act_tstride (grad likewise).  `tokens` must be >= the
 *             longest segment.  This is the expert-segmented MoE layout.
 *
 * has_bias = 1 means the activation carries an implicit trailing ones column
 * (a linear layer's bias folded as in dattri_llm/gradient/ops/preprocess.py:436-437),
 * which is never stored.
 *
 * Rows must be 16-byte aligned and K, D multiples of 16 bytes / element size.
 */
typedef struct da_factor_side {
  const void* act;
  const void* grad;
  int64_t batch;
  int64_t tokens;
  int64_t act_bstride;
  int64_t act_tstride;
  int64_t grad_bstride;
  int64_t grad_tstride;
  const int32_t* seg_offsets;
  const int32_t* row_index;
  int32_t has_bias;
  int32_t reserved;
} da_factor_side;

/*
 * Fused ghost inner product (factorized cross-gram) of one linear layer:
 *
 *   out[i*ld_out + j] (+)= sum_{t,s} (a1_it . a2_js) * (g1_it . g2_js)
 *
 * for i < s1->batch, j < s2->batch; fp32 accumulation throughout, the two
 * (S1 x S2) Gram tiles never leave registers.  accumulate != 0 adds to out
 * (multi-layer sums); otherwise out is overwritten.  Deterministic.
 *
 * Replaces the factorized route of cross_gram,
 * dattri_llm/gradient/ops/dot.py:115-118 (and the per-sample norm form at
 * dot.py:409-411 when both sides are the same block).
 */
int da_ghost_gram_workspace(const da_factor_side* s1, const da_factor_side* s2, int64_t K,
                            int64_t D, int dtype, size_t* bytes);
int da_ghost_gram(const da_factor_side* s1, const da_factor_side* s2, int64_t K, int64_t D,
                  int dtype, float* out, int64_t ld_out, int accumulate, void* workspace,
                  size_t workspace_bytes, void* stream);

/*
 * Per-sample weight gradient of a linear layer (materialized route):
 *
 *   out[b*out_bstride + o*out_rstride + k] = sum_t g[b,t,o] * a[b,t,k]   (k < K)
 *   out[b*out_bstride + o*out_rstride + K] = sum_t g[b,t,o]              (has_bias)
 *
 * a is (B, T, K), g is (B, T, D) with element strides (bstride, tstride) and
 * unit feature stride; out is written in out_dtype (fp32 accumulation).
 * Replaces materialize_factors for linear layers,
 * dattri_llm/gradient/ops/materialize.py:114-116 (bmm(g^T, a) flattened to
 * (B, out*in)), with the bias column of preprocess.py:436-437.
 */
int da_materialize_linear(const void* a, const void* g, int dtype, int64_t batch, int64_t tokens,
                          int64_t K, int64_t D, int64_t a_bstride, int64_t a_tstride,
                          int64_t g_bstride, int64_t g_tstride, int has_bias, void* out,
                          int out_dtype, int64_t out_bstride, int64_t out_rstride, void* stream);

/*
 * One dense layer of a score GEMM: m1 is (B1, width), m2 is (B2, width), row
 * strides ld1/ld2 in elements, unit column stride.
 */
typedef struct da_dense_layer {
  const void* m1;
  const void* m2;
  int64_t width;
  int64_t ld1;
  int64_t ld2;
} da_dense_layer;

/*
 * Multi-layer score GEMM (dense route), fp32 accumulation:
 *
 *   out[i*ld_row + j*ld_col] (+)= sum_L sum_c m1_L[i,c] * m2_L[j,c]
 *
 * All layers share one dtype; at most 32 layers per call.  Deterministic
 * (fixed-order split-K reduction through the workspace).
 * Replaces the dense products of cross_gram / cross_dot,
 * dattri_llm/gradient/ops/dot.py:114 and :501-505, and the layer sum of
 * layerwise_cross_dot, dot.py:599-604.
 */
int da_score_gemm_workspace(int64_t b1, int64_t b2, const da_dense_layer* layers, int n_layers,
                            int dtype, size_t* bytes);
int da_score_gemm(int64_t b1, int64_t b2, const da_dense_layer* layers, int n_layers, int dtype,
                  float* out, int64_t ld_row, int64_t ld_col, int accumulate, void* workspace,
                  size_t workspace_bytes, void* stream);

/*
 * Per-sample weight gradient of a token norm layer (kind 0 = RMSNorm,
 * 1 = LayerNorm), one pass over x and g:
 *
 *   x_hat = x * rsqrt(mean(x^2) + eps)  |  (x - mean) * rsqrt(var + eps)
 *   out[b*out_bstride + f]     = sum_t x_hat[b,t,f] * g[b,t,f]      (f < d)
 *   out[b*out_bstride + d + f] = sum_t g[b,t,f]                     (has_bias)
 *
 * eps is the caller's resolved epsilon (the reference's eps=None means the
 * activation dtype's machine epsilon, gradient/ops/norm.py:38-39).
 * Replaces preprocess_factors' norm branches (dattri_llm/gradient/ops/preprocess.py:366-384,
 * norm.py:25-41, :95-110) followed by materialize_factors' token sum
 * (materialize.py:96-98).
 */
int da_norm_weight_grad_workspace(int64_t batch, int64_t tokens, int64_t d, int has_bias,
                                  size_t* bytes);
int da_norm_weight_grad(const void* x, const void* g, int dtype, int64_t batch, int64_t tokens,
                        int64_t d, int64_t x_bstride, int64_t x_tstride, int64_t g_bstride,
                        int64_t g_tstride, int kind, float eps, int has_bias, void* out,
                        int out_dtype, int64_t out_bstride, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * Normalised rows x_hat of a token norm layer (the activation factor
 * preprocess_factors returns, dattri_llm/gradient/ops/norm.py:10-41):
 * x is (rows, d) with row stride x_rstride, out (rows, d) in out_dtype.
 */
int da_norm_xhat(const void* x, int dtype, int64_t rows, int64_t d, int64_t x_rstride, int kind,
                 float eps, void* out, int out_dtype, int64_t out_rstride, void* stream);

/*
 * Lane-layout self test of the 32x32 MFMA convention every kernel relies on:
 * a (32 x k) and b (32 x k) row-major (k = 16 for bf16/f16, 8 for f32, i.e.
 * one 16-byte chunk per lane), out receives 64 lanes x 16 accumulator values
 * of C = a . b^T exactly as the registers hold them (out[lane*16 + r]).
 * No counterpart in the reference: used by tests and smoke checks.
 */
int da_selftest_mfma(int dtype, const void* a, const void* b, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DATTRI_AMD_H */
