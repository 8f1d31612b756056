/*
 * dattri_amd.h -- C ABI of the MI355X (gfx950) gradient-scoring library.
 *
 * Every entry point takes device pointers, element counts/strides (in
 * elements, int64), a dtype code and a HIP stream (hipStream_t passed as
 * void*), launches stream-ordered work and returns a status code.  Nothing is
 * synchronised and nothing is allocated by the library: temporary storage is a
 * caller-provided workspace whose size the matching *_workspace query returns.
 * All entry points but one are re-entrant (no global mutable state besides a
 * thread-local error message), so they may be called from concurrent autograd
 * hook threads on different streams.  The exception is da_score_gemm_noalloc,
 * whose partials live in one library-owned device array per GPU.
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
 * The ghost inner product on the diagonal pairs only: per-sample dots of two
 * blocks of one batch size B, or per-sample squared norms when both sides
 * are the same block,
 *
 *   out[i*out_stride] (+)= sum_{t,s} (a1_it . a2_is + bias) * (g1_it . g2_is),  i < B,
 *
 * in one launch over the B pairs' tiles (fp32, deterministic).  Replaces the
 * factorized per-sample norm of grad_norm_sq_factors,
 * dattri_llm/gradient/ops/dot.py:409-411 (the einsums "btk,bsk->bts" and
 * "btd,bsd->bts" summed per sample), and the per-sample dots of dot_factors,
 * dot.py:307-357.  DA_ERR_INVALID when the batch sizes differ.
 */
int da_ghost_gram_diag_workspace(const da_factor_side* s1, const da_factor_side* s2, int64_t K, int64_t D,
                                 int dtype, size_t* bytes);
int da_ghost_gram_diag(const da_factor_side* s1, const da_factor_side* s2, int64_t K, int64_t D, int dtype,
                       float* out, int64_t out_stride, int accumulate, void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * Cross-gram of two embedding sides (nn.Embedding, and nn.EmbeddingBag once
 * its per-bag gradient is spread over its tokens).  The weight gradient is
 * sum_t e_{tok_t} g_t^T, so
 *
 *   out[i*ld_out + j] (+)= sum_t g1[i,t,:] . G2_j[tok1[i,t], :],
 *   G2_j[v] = sum over s with tok2[j,s] == v of g2[j,s,:]
 *
 * side->act holds int64 token ids (B, T) with element strides (act_bstride,
 * act_tstride); side->grad the (B, T, E) gradient rows (16-byte aligned).  A
 * negative id matches nothing (a padding position).  No segments, row index
 * or bias column.  diag = 1 takes the pairs (i, i) only, into out[i*ld_out]
 * (both batches equal): per-sample dots, or squared norms when both sides are
 * one block.  Side 2 is compacted to its samples' distinct ids (fp32 row sums,
 * sorted ids), and every side-1 token is looked up in every side-2 sample:
 * O(B1 T1 B2 log T2) searches plus one E-long dot per match.  fp32,
 * deterministic.  Replaces the embedding branches of cross_gram,
 * dattri_llm/gradient/ops/dot.py:58-74 (a scatter_add_ into a (vocab, E)
 * table per side-2 sample, then a gather), of dot_factors, dot.py:325-337,
 * and of grad_norm_sq_factors, dot.py:383-384.
 */
int da_embedding_cross_gram_workspace(const da_factor_side* s1, const da_factor_side* s2, int64_t E, int dtype,
                                      int diag, size_t* bytes);
int da_embedding_cross_gram(const da_factor_side* s1, const da_factor_side* s2, int64_t E, int dtype, int diag,
                            float* out, int64_t ld_out, int accumulate, void* workspace, size_t workspace_bytes,
                            void* stream);

/*
 * The same products kept per side-1 token: out[i*ld_b1 + t*ld_t + j*ld_b2]
 * (+)= g1[i,t,:] . G2_j[tok1[i,t], :], fp32 (B1, T1, B2); summing over t gives
 * da_embedding_cross_gram.  A gradient token stride of 0 is allowed (a bag's
 * one gradient row spread over its tokens).  Replaces the embedding branch of
 * cross_gram_per_token, dattri_llm/gradient/ops/dot.py:189-203.
 */
int da_embedding_cross_gram_per_token_workspace(const da_factor_side* s1, const da_factor_side* s2, int64_t E,
                                                int dtype, size_t* bytes);
int da_embedding_cross_gram_per_token(const da_factor_side* s1, const da_factor_side* s2, int64_t E, int dtype,
                                      float* out, int64_t ld_b1, int64_t ld_t, int64_t ld_b2, int accumulate,
                                      void* workspace, size_t workspace_bytes, void* stream);

/*
 * Per-token product of an embedding side against dense per-sample gradients,
 *
 *   out[i*ld_b1 + t*ld_t + j*ld_b2] (+)= sum_e g[i,t,e] * m2[j*m2_bstride + tok[i,t]*E + e]
 *
 * fp32; m2 holds each sample's (vocab, E) block (da_materialize_embedding's
 * layout) in dtype.  tok int64 (B1, T1), g (B1, T1, E), element strides as
 * for da_materialize_embedding; a negative id gives 0, ids must be < vocab.
 * Replaces the embedding branch of cross_gram_per_token_dense,
 * dattri_llm/gradient/ops/dot.py:239-245 (a gather of m2's rows, then an
 * einsum).
 */
int da_dense_per_token_embedding(const int64_t* tok, const void* g, int dtype, int64_t b1, int64_t len1, int64_t E,
                                 int64_t vocab, int64_t tok_bstride, int64_t tok_tstride, int64_t g_bstride,
                                 int64_t g_tstride, const void* m2, int64_t m2_bstride, int64_t b2, float* out,
                                 int64_t ld_b1, int64_t ld_t, int64_t ld_b2, int accumulate, void* stream);

/*
 * Per-token cross-gram of two factorized sides: side 1's token axis kept,
 * side 2's summed out,
 *
 *   out[i*ld_b1 + t*ld_t + j*ld_b2] (+)= sum_s (a1[i,t,:].a2[j,s,:] + bias) * (g1[i,t,:].g2[j,s,:])
 *                                     = a1_it^T (sum_s a2_js g2_js^T) g1_it,
 *
 * fp32, (B1, T1, B2).  Summing over t gives da_ghost_gram's (B1, B2).
 * Replaces cross_gram_per_token for linear layers,
 * dattri_llm/gradient/ops/dot.py:171-222 (einsum over the materialized side-2
 * gradient, :220-222), which cross_dot_per_token (:266-299) and
 * layerwise_cross_dot_per_token (:607-669) call.  Dense sides only (no
 * seg_offsets), D > 0; DA_ERR_UNSUPPORTED for rows beyond 32-bit offsets.
 */
int da_ghost_gram_per_token_workspace(const da_factor_side* s1, const da_factor_side* s2, int64_t K, int64_t D,
                                      int dtype, size_t* bytes);
int da_ghost_gram_per_token(const da_factor_side* s1, const da_factor_side* s2, int64_t K, int64_t D, int dtype,
                            float* out, int64_t ld_b1, int64_t ld_t, int64_t ld_b2, int accumulate,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Per-token cross-gram against a dense side 2 (materialized or
 * preconditioned per-sample gradients):
 *
 *   out[i*ld_b1 + t*ld_t + j*ld_b2] (+)= sum_o (a1[i,t,:] . M2_j[o,:] + mb_j[o]) * g1[i,t,o]
 *
 * with M2_j[o, k] at m2 + j*m2_bstride + o*m2_rstride + k (elements, K
 * columns, 16-byte aligned rows) and, when s1->has_bias, the bias column's
 * gradients mb_j[o] = m2_bias[j*m2_bias_ld + o] (fp32).  Only s1's factors
 * are read (act (B1, T1, K), grad (B1, T1, D)).  Replaces
 * cross_gram_per_token_dense for linear layers,
 * dattri_llm/gradient/ops/dot.py:225-263 (einsum "btk,btd,cdk->btc").
 */
int da_dense_per_token_workspace(const da_factor_side* s1, int64_t b2, int64_t K, int64_t D, int dtype,
                                 size_t* bytes);
int da_dense_per_token(const da_factor_side* s1, const void* m2, int64_t b2, int64_t m2_bstride, int64_t m2_rstride,
                       const float* m2_bias, int64_t m2_bias_ld, int64_t K, int64_t D, int dtype, float* out,
                       int64_t ld_b1, int64_t ld_t, int64_t ld_b2, int accumulate, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * Segment-summed ghost product over experts (MoE routed layers):
 *
 *   out[i*ld_out + j] (+)= sum_e sum_{t in seg1_e(i), s in seg2_e(j)}
 *                            (a1_e,t . a2_e,s) * (g1_e,t . g2_e,s)
 *
 * s1[e], s2[e] (e < n_groups) describe group e -- one expert of one linear
 * layer -- in packed segmented form: seg_offsets (B+1 int32, non-decreasing)
 * split the expert's rows by sample, `tokens` is the expert's total row count
 * (>= seg_offsets[B]), row_index optionally gathers physical rows,
 * act/grad_tstride are row strides, has_bias (equal on both sides) adds the
 * implicit ones column.  K[e], D[e] are the group's activation and gradient
 * widths, so the experts of several layers can share one launch (the launch
 * orders the groups by decreasing K + D itself).  All groups share the batch
 * sizes (B1, B2) and dtype.  Tiles run over each expert's rows as packed (no
 * per-sample padding); each tile's products are binned by (sample, sample) and
 * reduced in a fixed order (deterministic).  Empty experts and samples are
 * allowed.
 *
 * Replaces, for routed experts, the per-expert regroup to zero-filled
 * (B, T, d) captures (dattri_llm/gradient/hooks/routing.py:71-86) followed by
 * the factorized cross_gram (dattri_llm/gradient/ops/dot.py:115-118), summed
 * over experts and layers as layerwise_cross_dot sums layers (dot.py:599-604).
 */
int da_ghost_gram_grouped_workspace(const da_factor_side* s1, const da_factor_side* s2, int n_groups,
                                    const int64_t* K, const int64_t* D, int dtype, size_t* bytes);
int da_ghost_gram_grouped(const da_factor_side* s1, const da_factor_side* s2, int n_groups,
                          const int64_t* K, const int64_t* D, int dtype, float* out, int64_t ld_out,
                          int accumulate, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Per-sample weight gradient of a linear layer (materialized route):
 *
 *   out[b*out_bstride + o*out_rstride + k] = sum_t g[b,t,o] * a[b,t,k]   (k < K)
 *   out[b*out_bstride + o*out_rstride + K] = sum_t g[b,t,o]              (has_bias)
 *
 * a is (B, T, K), g is (B, T, D) with element strides (bstride, tstride) and
 * unit feature stride; out is written in out_dtype (fp32 accumulation).
 * Output addressing: flat index c = o*out_rstride + k of sample b is stored at
 * out + b*out_bstride + (c/64)*out_blk + c%64 (elements).  out_blk = 64 (or 0)
 * is plain row-major; out_bstride = 64, out_blk = B*64 (needs K % 64 == 0 and
 * no bias) writes the k-blocked layout da_score_gemm streams contiguously.
 * Replaces materialize_factors for linear layers,
 * dattri_llm/gradient/ops/materialize.py:114-116 (bmm(g^T, a) flattened to
 * (B, out*in)), with the bias column of preprocess.py:436-437.
 */
int da_materialize_linear(const void* a, const void* g, int dtype, int64_t batch, int64_t tokens,
                          int64_t K, int64_t D, int64_t a_bstride, int64_t a_tstride,
                          int64_t g_bstride, int64_t g_tstride, int has_bias, void* out,
                          int out_dtype, int64_t out_bstride, int64_t out_rstride,
                          int64_t out_blk, void* stream);

/*
 * Per-sample embedding weight gradient (scatter-add):
 *
 *   out[b*out_bstride + v*E + e] = sum over t with tok[b,t] == v of g[b,t,e]
 *
 * for v < vocab, in dtype: each row summed in fp32 in ascending t and rounded
 * once (what the reference's scatter_add_ gives on the CPU, where the
 * reduced-precision path accumulates in fp32; deterministic).  tok is int64
 * (B, T) with element strides (tok_bstride, tok_tstride); g is (B, T, E) with
 * element strides (g_bstride, g_tstride), rows 16-byte aligned, E a multiple
 * of 16 bytes / element size.  Every block is zeroed first; ids outside
 * [0, vocab) add nothing (callers reject them beforehand; a negative id is a
 * padding position).  vocab, T < 2^31; B <= 65535.  The workspace (size from
 * da_materialize_embedding_workspace, 256-byte aligned) holds each token's
 * first occurrence and, for 2-byte dtypes, the fp32 (B, T, E) sums.
 * Replaces _materialize_embedding, dattri_llm/gradient/ops/materialize.py:22-48
 * (result.scatter_add_ into (B, vocab, E), flattened to (B, vocab*E)).
 */
int da_materialize_embedding_workspace(int64_t batch, int64_t tokens, int64_t E, int dtype, size_t* bytes);
int da_materialize_embedding(const int64_t* tok, const void* g, int dtype, int64_t batch, int64_t tokens,
                             int64_t E, int64_t vocab, int64_t tok_bstride, int64_t tok_tstride,
                             int64_t g_bstride, int64_t g_tstride, void* out, int64_t out_bstride,
                             void* workspace, size_t workspace_bytes, void* stream);

/*
 * Kept entries of the per-sample embedding gradient, without forming it:
 *
 *   out[b*ld_out + q] = sum over t with tok[b,t] == rows[q] of g[b,t,cols[q]],  q < k,
 *
 * fp32, tokens in ascending order.  tok int64 (B, T) and g (B, T, E) with
 * element strides as for da_materialize_embedding (no alignment needed);
 * rows / cols int64 (k,).  A negative id or a column outside [0, E) adds
 * nothing.  Replaces the embedding branch of mask_factors,
 * dattri_llm/gradient/ops/projection.py:718-735 (a one-hot indicator times
 * the gathered gradient columns, summed over tokens).
 */
int da_gather_embedding_entries(const int64_t* tok, const void* g, int dtype, int64_t batch, int64_t tokens,
                                int64_t E, int64_t tok_bstride, int64_t tok_tstride, int64_t g_bstride,
                                int64_t g_tstride, const int64_t* rows, const int64_t* cols, int64_t k, float* out,
                                int64_t ld_out, void* stream);

/*
 * Row Gram: out (+)= x^T x, fp32 (width, width) with row stride ld_out, of the
 * bf16/fp16 rows x (rows, width) with row stride x_stride (elements; width and
 * x_stride multiples of 8, rows 16-byte aligned).  accumulate = 0 overwrites,
 * 1 adds to a symmetric out (the tiles below the diagonal are rewritten as the
 * mirror of those above it); rows = 0 (x may then be NULL) zeroes or leaves out.  The symmetric product is computed once per pair of tiles (the ones
 * on or above the diagonal) and mirrored.  Returns DA_ERR_UNSUPPORTED for
 * other dtypes.  Replaces the covariance products of the K-FAC factors and the
 * empirical Fisher, dattri_llm/gradient/ops/kronecker.py:111-112
 * ((a_f^T a_f), (g_f^T g_f)), :136 (grad^T grad) and the accumulators'
 * :512-513 and :594.
 */
int da_row_gram(const void* x, int dtype, int64_t rows, int64_t width, int64_t x_stride, float* out,
                int64_t ld_out, int accumulate, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Workspace bytes da_row_gram can use on the current device for (rows, width)
 * packed rows (x_stride == width): the tiles past the triangle's last whole
 * round of CUs run as token splits into compact fp32 256 x 256 partial tiles,
 * so a partly filled round (or a small triangle) fills the GPU.  0 when one
 * pass is best.  A smaller or NULL workspace is accepted: the call then uses
 * the splits that fit (down to none).  Calls sharing a workspace must be
 * ordered on one stream.  No reference counterpart (workspace sizing).
 */
int da_row_gram_workspace(int64_t rows, int64_t width, int dtype, size_t* bytes);

/*
 * Gradient-free rows: out[r] = 1 if some entry of row r of x (rows, width),
 * row stride x_stride (elements), compares unequal to zero, else 0 (-0.0 is
 * zero; NaN, inf and subnormals are not).  Rows 16-byte aligned, width and
 * x_stride multiples of 16 bytes.  Replaces the mask of
 * dattri_llm/gradient/ops/kronecker.py:65-81 ((g_f != 0).any(dim=1)).
 */
int da_nonzero_rows(const void* x, int dtype, int64_t rows, int64_t width, int64_t x_stride, uint8_t* out,
                    void* stream);

/*
 * One dense layer of a score GEMM: m1 is (B1, width), m2 is (B2, width).
 * Element c of row r of side s lives at  m_s + r*ld_s + (c/64)*blk_s + c%64
 * (elements): rows are sequences of 64-element blocks.  blk_s = 64 (or 0) is
 * plain row-major; blk_s = B_s*64 with ld_s = 64 is the k-blocked layout, in
 * which block b of every row is one contiguous B_s*64 run (what
 * da_materialize_linear writes with out_blk = B*64).
 */
typedef struct da_dense_layer {
  const void* m1;
  const void* m2;
  int64_t width;
  int64_t ld1;
  int64_t ld2;
  int64_t blk1;
  int64_t blk2;
} da_dense_layer;

/*
 * Multi-layer score GEMM (dense route), fp32 accumulation:
 *
 *   out[i*ld_row + j*ld_col] (+)= sum_L sum_c m1_L[i,c] * m2_L[j,c]
 *
 * All layers share one dtype; at most 32 layers per call.  Deterministic
 * (fixed-order split-K reduction through the workspace).  For 2-byte dtypes
 * the workspace size depends on the current device's CU count (one partial
 * tile per CU): query it with the device current on which the call will run.
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
 * Per-row dot products of dense layers, summed over layers, fp32:
 *
 *   out[r*out_stride] (+)= sum_L sum_c m1_L[r, c] * m2_L[r, c]
 *
 * with the layers' addressing of da_dense_layer (row-major or k-blocked); a
 * layer whose m2 is NULL contributes its squared row norms.  One pass over
 * every weight, deterministic (fixed-order reduction through the workspace,
 * whose size depends on the current device's CU count).  At most 32 layers
 * per call.  Replaces the dense per-sample squared norms of grad_norm_sq,
 * dattri_llm/gradient/ops/dot.py:426-428 ((flat * flat).sum(-1)), summed
 * over layers as TracInAttributor._norm sums them
 * (dattri_llm/attribution/algorithm/tracin.py:129-148), and the dense
 * per-sample dots of dot_factors, dot.py:307-357.
 */
int da_row_dots_workspace(int64_t rows, const da_dense_layer* layers, int n_layers, int dtype, size_t* bytes);
int da_row_dots(int64_t rows, const da_dense_layer* layers, int n_layers, int dtype, float* out,
                int64_t out_stride, int accumulate, void* workspace, size_t workspace_bytes, void* stream);

/*
 * da_score_gemm without a workspace, for callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  No counterpart in the reference.
 *
 * Same arguments and results as da_score_gemm (bit-identical: same kernels,
 * same fixed-order reduction) minus the workspace.  The split-K partials live
 * in a library-owned device array of DA_SCORE_GEMM_SCRATCH_BYTES on each GPU
 * the library runs on, held until the process ends; its address is resolved
 * once per device on the first call there.  A problem whose
 * da_score_gemm_workspace exceeds that size returns DA_ERR_WORKSPACE (for
 * 2-byte dtypes one partial tile per CU: e.g. 8 x 64 outputs need 0.5 MiB on
 * 256 CUs).  Nothing is allocated or freed and no memset is issued; every
 * partial is written before it is read, so nothing carries over between
 * calls.  All calls on one GPU share the array: calls that overlap on it
 * (different streams or threads) race, so order them on one stream.
 */
#define DA_SCORE_GEMM_SCRATCH_BYTES ((size_t)8 << 20)
int da_score_gemm_noalloc(int64_t b1, int64_t b2, const da_dense_layer* layers, int n_layers, int dtype,
                          float* out, int64_t ld_row, int64_t ld_col, int accumulate, void* stream);

/*
 * Per-sample weight gradient of a token norm layer (kind 0 = RMSNorm,
 * 1 = LayerNorm, 2 = x already normalised, i.e. x_hat = x), one pass over x
 * and g:
 *
 *   x_hat = x * rsqrt(mean(x^2) + eps)  |  (x - mean) * rsqrt(var + eps)
 *   out[b*out_bstride + f]     = sum_t x_hat[b,t,f] * g[b,t,f]      (f < d)
 *   out[b*out_bstride + d + f] = sum_t g[b,t,f]                     (has_bias)
 *
 * eps is the caller's resolved epsilon (the reference's eps=None means the
 * activation dtype's machine epsilon, gradient/ops/norm.py:38-39).  Rows start
 * 16-byte aligned and are read in whole 16-byte chunks: when d is not a
 * multiple of a chunk, the row stride must leave room for the last chunk,
 * whose elements past d are read and ignored.
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
 * Rows are read in whole 16-byte chunks, as for da_norm_weight_grad.
 */
int da_norm_xhat(const void* x, int dtype, int64_t rows, int64_t d, int64_t x_rstride, int kind,
                 float eps, void* out, int out_dtype, int64_t out_rstride, void* stream);

/*
 * Channel norms (GroupNorm; InstanceNorm is one group per channel).  x and g
 * are contiguous (N, C, S) (S = the flattened spatial axes), G groups of C/G
 * consecutive channels; x_hat = (x - mean) / sqrt(var + eps) over each
 * (sample, group) block of C/G x S values (biased variance), as
 * dattri_llm/gradient/ops/norm.py:44-62 computes it.
 *
 * da_channel_norm_weight_grad: out[n*out_ld + c] = sum_s x_hat[n,c,s] g[n,c,s]
 * and, with has_bias, out[n*out_ld + C + c] = sum_s g[n,c,s] (fp32 sums, out in
 * out_dtype) -- the token sum of the (N, S, C) factors of
 * _augment_channel_norm, norm.py:120-141, that materialize_factors forms
 * (materialize.py:96-98).  S > 0.
 * da_channel_norm_xhat: x_hat in x's layout, in out_dtype (the normalisation
 * preprocess_factors applies, preprocess.py:386-401).
 * Both need a workspace of da_channel_norm_workspace bytes (the statistics).
 */
int da_channel_norm_workspace(int64_t N, int64_t G, size_t* bytes);
int da_channel_norm_weight_grad(const void* x, const void* g, int dtype, int64_t N, int64_t C, int64_t S, int64_t G,
                                float eps, int has_bias, void* out, int out_dtype, int64_t out_ld, void* workspace,
                                size_t workspace_bytes, void* stream);
int da_channel_norm_xhat(const void* x, int dtype, int64_t N, int64_t C, int64_t S, int64_t G, float eps, void* out,
                         int out_dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Random projection of factor rows (ProjectionMatrix.__call__,
 * dattri_llm/gradient/ops/projection.py:363-370):
 *
 *   out[r*out_rstride + c] = sum_j x[r*x_rstride + j] * P[j, c] (+ bias[c])
 *
 * The projection matrix is passed TRANSPOSED: pt is (k, d) with row stride
 * pt_rstride, so both operands are read along d.  bias is k fp32 values or
 * NULL (the bias row of a linear layer's (d+1, k) matrix, projection.py:276-277).
 */
int da_project_rows(const void* x, int dtype, int64_t rows, int64_t d, int64_t x_rstride,
                    const void* pt, int64_t k, int64_t pt_rstride, const float* bias, void* out,
                    int out_dtype, int64_t out_rstride, void* stream);

/*
 * Fused capture-time projection and per-sample outer-product sum of a linear
 * layer (the LoGRA capture of dattri_llm/gradient/hooks/hooks.py:631-648 with
 * materialize_factors(a_p, g_p, "nn.Linear"), materialize.py:114-116):
 *
 *   a_p = a . P_in (+ bias_in)     (B, T, ka)      P_in^T  = pin_t  (ka, K)
 *   g_p = g . P_out                (B, T, kg)      P_out^T = pout_t (kg, D)
 *   out[b*out_bstride + o*ka + i] = sum_t g_p[b,t,o] * a_p[b,t,i]
 *
 * ka, kg <= 64 (DA_ERR_UNSUPPORTED above).  One pass over a and g.  The
 * workspace size depends on the current device's CU count (one partial
 * projection per CU at most): query it with the device current on which the
 * call will run.
 */
int da_project_outer_workspace(int64_t batch, int64_t tokens, int64_t ka, int64_t kg, size_t* bytes);
int da_project_outer(const void* a, const void* g, int dtype, int64_t batch, int64_t tokens, int64_t K,
                     int64_t D, int64_t a_bstride, int64_t a_tstride, int64_t g_bstride,
                     int64_t g_tstride, const void* pin_t, int64_t ka, int64_t pin_rstride,
                     const float* bias_in, const void* pout_t, int64_t kg, int64_t pout_rstride,
                     void* out, int out_dtype, int64_t out_bstride, void* workspace,
                     size_t workspace_bytes, void* stream);

/*
 * A coordinate subset of per-sample linear weight gradients (the "mask"
 * projection style), gathered from the factors without forming the gradient:
 *
 *   out[b*out_ld + k] = sum_t g[b, t, rows[k]] * A[b, t, cols[k]],   k < n,
 *
 * fp32, where A is a (B, T, K) with, when has_bias, an implicit ones column at
 * index K.  rows/cols (int64, device) are the coordinates' output and input
 * indices (flat index o*(K+bias) + i of the materialized gradient); entries
 * outside the layer contribute 0.  Replaces mask_factors for linear layers,
 * dattri_llm/gradient/ops/projection.py:687-783 (_gather_pairs,
 * projection.py:786-811).
 */
int da_gather_entries(const void* a, const void* g, int dtype, int64_t batch, int64_t tokens, int64_t K, int64_t D,
                      int64_t a_bstride, int64_t a_tstride, int64_t g_bstride, int64_t g_tstride, int has_bias,
                      const int64_t* rows, const int64_t* cols, int64_t n, float* out, int64_t out_ld,
                      void* stream);

/*
 * MoE router: per token, top-k of softmax(logits) (fp32, a NaN or +inf logit
 * or an all -inf row gives NaN probabilities as torch's softmax does), weights
 * renormalised over the k, indices in the order torch.topk returns on the CPU,
 * ties and NaN rows included (ATen's nth_element / partial_sort selection) --
 * the router contract of transformers' MixtralTopKRouter.forward used by
 * dattri_llm/gradient/hooks/override_layers/fused_experts.py:210-237.
 * logits (n_tokens, n_experts) with row stride row_stride; weights (n, k)
 * fp32; index (n, k) int64.  n_experts <= 256, k <= 16.
 */
int da_moe_topk(const void* logits, int dtype, int64_t n_tokens, int n_experts, int k,
                int64_t row_stride, float* weights, int64_t* index, void* stream);

/*
 * Stable counting sort of integer keys into `bins` bins (<= 8192).
 * keys: keys32 or keys64 (n entries), or with slot_major != 0 the int64
 * (rows, k) matrix keys64 read slot-major (entry p = keys64[(p % rows)*k + p / rows]).
 * key_div > 1 divides each key first (e.g. flat token -> sample).  Writes
 * offsets (bins+1: bin b holds sorted positions [offsets[b], offsets[b+1]))
 * and perm (sorted position -> input entry).  Keys outside [0, bins) are
 * dropped (offsets[bins] counts the kept ones).  On top-k indices read
 * slot-major this yields the expert segments in the order of
 * fused_experts.py:219-228 (torch.where over one_hot(idx).permute(2,1,0)[e]).
 */
int da_counting_sort(const int32_t* keys32, const int64_t* keys64, int64_t n, int64_t rows,
                     int64_t k, int slot_major, int64_t key_div, int bins, int32_t* offsets,
                     int32_t* perm, void* stream);

/*
 * Expert routing of one side in one launch.  index is the (n_tokens, k) int64
 * top-k matrix (da_moe_topk), n_tokens = batch * tokens (flat token
 * b*tokens + t).  Entries p = slot*n_tokens + token are taken in the
 * reference's order (slot-major, token ascending: torch.where over
 * one_hot(idx).permute(2,1,0)[e], fused_experts.py:219-228) and sorted
 * stably twice in one pass:
 *   expert_offsets (n_experts+1): expert e owns routed rows
 *       [expert_offsets[e], expert_offsets[e+1]);
 *   entries (n*k): entries[expert_offsets[e] + r] = p of expert e's row r;
 *   seg (n_experts * (batch+1)): seg[e*(batch+1) + b] = number of expert e's
 *       rows from samples < b (per-expert relative offsets);
 *   rows (n*k): rows[expert_offsets[e] + q] = expert e's local row numbers
 *       grouped by sample (stable): the (seg, row_index) pair of a group of
 *       da_ghost_gram_grouped.
 * Replaces the per-expert torch.where loop of fused_experts.py:219-228 plus
 * the regroup bookkeeping of hooks/routing.py:71-86.  n_experts <= 256,
 * n_experts * batch <= 8192; indices outside [0, n_experts) are dropped.
 */
int da_moe_route(const int64_t* index, int64_t n_tokens, int k, int n_experts, int64_t batch,
                 int64_t tokens, int32_t* expert_offsets, int32_t* entries, int32_t* seg, int32_t* rows,
                 void* stream);

/*
 * Routed-row compaction: of the batch * tokens rows (row p = b * tokens + t of
 * sample b), the ones whose mask byte is non-zero, in increasing order:
 * rows[seg_offsets[b] .. seg_offsets[b+1]) are sample b's (seg_offsets has
 * batch + 1 entries; rows holds up to batch * tokens entries, seg_offsets[batch]
 * of them written).  With the mask of da_nonzero_rows this finds the
 * gradient-carrying rows of the zero-filled (B, T, d) captures the
 * reference's routed-token layout produces for MoE experts
 * (dattri_llm/gradient/hooks/routing.py:71-86: "zero where a sample's token
 * was not routed to the layer"), as the (seg_offsets, row_index) pair of
 * da_ghost_gram_grouped -- without a host round trip.
 */
int da_compact_rows(const uint8_t* mask, int64_t batch, int64_t tokens, int32_t* seg_offsets, int32_t* rows,
                    void* stream);

/*
 * Exact location of routed token rows: x (n_x, width) holds rows gathered
 * from the block input src (n_src, width) (row strides in elements, rows
 * 16-byte aligned, width * element size a multiple of 16).  The k-th
 * occurrence of a row value among x's rows is matched to the k-th token, in
 * ascending order, of src holding the same value, and verified element by
 * element (float equality: -0 == +0, NaN equals nothing):
 * token[r] (int64) = the matched src row of x row r, or -1.  *status (device
 * int32) is set to 0, then to 1 when any row fails (a value absent from src,
 * more copies than src holds, or a fingerprint collision).  Workspace from
 * da_match_rows_workspace.  Replaces RoutedTokenTracker._match,
 * dattri_llm/gradient/hooks/routing.py:300-333 (fingerprints, a stable sort,
 * searchsorted, torch.equal).
 */
int da_match_rows_workspace(int64_t n_src, int64_t n_x, size_t* bytes);
int da_match_rows(const void* src, int64_t n_src, int64_t src_rstride, const void* x, int64_t n_x, int64_t x_rstride,
                  int64_t width, int dtype, int64_t* token, int32_t* status, void* workspace, size_t workspace_bytes,
                  void* stream);

/*
 * Lane-layout self test of the MFMA conventions every kernel relies on.
 * shape 32: a and b are (32 x k) row-major with k = 16 (bf16/f16) or 8 (f32),
 *           one 16-byte chunk per lane half; out receives 64 lanes x 16
 *           accumulator values of C = a . b^T as the registers hold them
 *           (out[lane*16 + r]).
 * shape 16: a and b are (16 x k), k = 32 (bf16/f16) or 16 (f32); out receives
 *           64 lanes x 4 values (out[lane*4 + r]).
 * No counterpart in the reference: used by tests and smoke checks.
 */
int da_selftest_mfma(int dtype, int shape, const void* a, const void* b, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DATTRI_AMD_H */
