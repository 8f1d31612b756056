// Embedding layers (nn.Embedding, and nn.EmbeddingBag spread over its tokens)
// on gfx950: the weight-gradient scatter and the per-token product against a
// dense side 2.  Both are HBM-bound gathers/scatters of 16-byte row chunks; no
// MFMA.  (The factorized cross-gram of two embedding sides runs on the ghost
// engine, ghost_gram.hip.)
#include <algorithm>

#include "common.h"

namespace da {
namespace {

// Embedding weight gradient (materialize.py:22-48): for each sample b,
//
//   out[b, v, :] = sum over t with tok[b, t] == v of g[b, t, :]
//
// the (vocab, E) block of sample b at out + b * out_bstride (row v at v * E),
// summed in fp32 in ascending t and rounded once to the output dtype -- what
// the reference's scatter_add_ along the vocab axis gives on the CPU (its
// reduced-precision path accumulates in fp32), and deterministic.
//
// fp32 output: the rows are summed in place (the blocks are zeroed first).
// bf16 / fp16 output: each token's row is the first occurrence of its id in
// the sample (its "slot", embed_first_slot); the sums build up in an fp32
// (B, T, E) scratch at the slot rows (the first occurrence writes, later ones
// add), and embed_write_slots rounds each slot row into its id's row.
//
// Summing: one thread owns one 16-byte column chunk of one sample and adds the
// token rows in ascending t.  Blocks along z split the target rows by
// row % gridDim.z, so a thread's chain of read-modify-writes covers only its
// slice's tokens; every block stages the sample's target rows through LDS in
// runs of kEmbedIds.  Ids outside [0, vocab) add nothing (the host rejects
// them first; a negative id is a padding position); vocab < 2^31.
constexpr int kEmbedIds = 2048;

// slot[b, t] = the first t' <= t with tok[b, t'] == tok[b, t]; -1 for an id
// outside [0, vocab).  A block covers 256 consecutive t and scans the ids
// before them in LDS runs of kSlotRun (every lane reads the same id at once).
constexpr int kSlotRun = 2048;

__global__ __launch_bounds__(256) void embed_first_slot(const int64_t* __restrict__ tok, int64_t tok_bs,
                                                        int64_t tok_ts, int64_t tokens, int64_t vocab,
                                                        int32_t* __restrict__ slot) {
  __shared__ int64_t run[kSlotRun];
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  const int64_t* tb = tok + b * tok_bs;
  const int64_t v = t < tokens ? tb[t * tok_ts] : -1;
  const bool live = v >= 0 && v < vocab;
  int64_t first = live ? t : -1;
  bool found = !live;
  const int64_t end = std::min<int64_t>(tokens, (int64_t)(blockIdx.x + 1) * blockDim.x);  // ids before the last t
  for (int64_t u0 = 0; u0 < end; u0 += kSlotRun) {
    const int n = (int)std::min<int64_t>(kSlotRun, end - u0);
    __syncthreads();  // the previous run is consumed
    for (int i = threadIdx.x; i < n; i += blockDim.x) run[i] = tb[(u0 + i) * tok_ts];
    __syncthreads();
    if (!found) {
      const int m = (int)std::min<int64_t>(n, t - u0);  // ids strictly before t
      for (int i = 0; i < m; ++i)
        if (run[i] == v) {
          first = u0 + i;
          found = true;
          break;
        }
    }
  }
  if (t < tokens) slot[b * tokens + t] = (int32_t)first;
}

// kSlots = false: rows are ids into the fp32 output; true: rows are slots into
// the fp32 scratch, and the first occurrence (slot == t) writes instead of adds.
template <int DT, bool kSlots>
__global__ __launch_bounds__(256) void embed_accumulate(const int64_t* __restrict__ tok, int64_t tok_bs,
                                                        int64_t tok_ts, const int32_t* __restrict__ slot,
                                                        const char* __restrict__ g, int64_t g_bs, int64_t g_ts,
                                                        int64_t tokens, int64_t E, int64_t vocab,
                                                        float* acc, int64_t acc_bstride) {
  constexpr int VEC = Elem<DT>::kVec;
  __shared__ int32_t rows[kEmbedIds];
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 16-byte chunk of the gradient row
  const int64_t b = blockIdx.y;
  const int64_t slices = gridDim.z, slice = blockIdx.z;
  const bool active = c * VEC < E;
  const int64_t* tb = tok + b * tok_bs;
  const char* gb = g + b * g_bs + c * 16;
  float* ab = acc + b * acc_bstride + c * VEC;
  for (int64_t t0 = 0; t0 < tokens; t0 += kEmbedIds) {
    const int n = (int)(tokens - t0 < kEmbedIds ? tokens - t0 : kEmbedIds);
    __syncthreads();  // the previous run's rows are consumed
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      int64_t r;
      if constexpr (kSlots) {
        r = slot[b * tokens + t0 + i];
      } else {
        const int64_t v = tb[(t0 + i) * tok_ts];
        r = (v >= 0 && v < vocab) ? v : -1;
      }
      rows[i] = (r >= 0 && r % slices == slice) ? (int32_t)r : -1;
    }
    __syncthreads();
    if (!active) continue;
    for (int i = 0; i < n; ++i) {
      const int32_t r = rows[i];
      if (r < 0) continue;
      float x[VEC];
      unpack16<DT>(ld16(gb + (t0 + i) * g_ts), x);
      float* o = ab + (int64_t)r * E;
      if (kSlots && r == t0 + i) {  // first occurrence: the slot row starts here
#pragma unroll
        for (int h = 0; h < VEC / 4; ++h)
          *(f32x4*)(o + 4 * h) = f32x4{x[4 * h], x[4 * h + 1], x[4 * h + 2], x[4 * h + 3]};
      } else {
#pragma unroll
        for (int h = 0; h < VEC / 4; ++h) {
          f32x4 y = *(const f32x4*)(o + 4 * h);
          y[0] += x[4 * h];
          y[1] += x[4 * h + 1];
          y[2] += x[4 * h + 2];
          y[3] += x[4 * h + 3];
          *(f32x4*)(o + 4 * h) = y;
        }
      }
    }
  }
}

// out[b, tok[b, t], :] = round(scratch[b, t, :]) for every first occurrence t.
template <int DT>
__global__ __launch_bounds__(256) void embed_write_slots(const int64_t* __restrict__ tok, int64_t tok_bs,
                                                         int64_t tok_ts, const int32_t* __restrict__ slot,
                                                         const float* __restrict__ scratch, int64_t tokens,
                                                         int64_t E, int64_t chunk_blocks, char* out,
                                                         int64_t out_bstride) {
  constexpr int VEC = Elem<DT>::kVec, ES = Elem<DT>::kBytes;
  const int64_t t = blockIdx.x / chunk_blocks;
  const int64_t c = (blockIdx.x % chunk_blocks) * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (c * VEC >= E || slot[b * tokens + t] != t) return;
  const int64_t v = tok[b * tok_bs + t * tok_ts];
  const float* src = scratch + (b * tokens + t) * E + c * VEC;
  u32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint16_t lo, hi;
    if constexpr (DT == DA_BF16) {
      lo = f32_to_bf16_bits(src[2 * e]);
      hi = f32_to_bf16_bits(src[2 * e + 1]);
    } else {
      lo = f32_to_f16_bits(src[2 * e]);
      hi = f32_to_f16_bits(src[2 * e + 1]);
    }
    r[e] = (uint32_t)lo | ((uint32_t)hi << 16);
  }
  st16(out + (b * out_bstride + v * E + c * VEC) * ES, r);
}

// Zero `rows` runs of `chunks` 16-byte chunks, run r at out + r * stride bytes
// (grid-stride, so any size fits one launch).
__global__ __launch_bounds__(256) void zero_runs16(char* out, int64_t rows, int64_t chunks, int64_t stride) {
  const int64_t n = rows * chunks;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / chunks;
    st16(out + r * stride + (i - r * chunks) * 16, u32x4{0u, 0u, 0u, 0u});
  }
}

// Per-token product of an embedding side against dense per-sample gradients
// (dot.py:225-263, the embedding branch :239-245):
//
//   out[i, t, j] = sum_e g1[i, t, e] * m2[j, tok1[i, t], e]
//
// m2 is sample j's (vocab, E) block at m2 + j * m2_bstride.  One wave per
// token (i, t): its lanes stride the row's 16-byte chunks and the wave sum
// fixes the order.  A negative id (padding) gives 0; ids must be < vocab.
template <int DT>
__global__ __launch_bounds__(256) void embed_dense_per_token(const int64_t* __restrict__ tok, int64_t tok_bs,
                                                             int64_t tok_ts, const char* __restrict__ g, int64_t g_bs,
                                                             int64_t g_ts, int64_t b1, int64_t len1, int64_t E,
                                                             int64_t vocab, const char* __restrict__ m2,
                                                             int64_t m2_bs, int64_t b2, float* __restrict__ out,
                                                             int64_t ld_b1, int64_t ld_t, int64_t ld_b2,
                                                             int accumulate) {
  constexpr int VEC = Elem<DT>::kVec, ES = Elem<DT>::kBytes;
  const int lane = threadIdx.x & 63;
  const int64_t u = (int64_t)blockIdx.x * (blockDim.x / kWave) + (threadIdx.x >> 6);
  if (u >= b1 * len1) return;  // uniform per wave; no barrier below
  const int64_t i = u / len1, t = u - i * len1;
  const int64_t v = tok[i * tok_bs + t * tok_ts];
  const bool live = v >= 0 && v < vocab;
  const char* grow = g + i * g_bs + t * g_ts;
  const int64_t chunks = E / VEC;
  float* o = out + i * ld_b1 + t * ld_t;
  for (int64_t j = 0; j < b2; ++j) {
    float acc = 0.f;
    if (live) {
      const char* mrow = m2 + (j * m2_bs + v * E) * ES;
      for (int64_t c = lane; c < chunks; c += kWave) {
        float x[VEC], y[VEC];
        unpack16<DT>(ld16(grow + c * 16), x);
        unpack16<DT>(ld16(mrow + c * 16), y);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc = fmaf(x[e], y[e], acc);
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) o[j * ld_b2] = accumulate ? o[j * ld_b2] + acc : acc;
  }
}


// Entries of the per-sample embedding gradient without forming it
// (projection.py:718-735, the "mask" capture of an embedding):
//
//   out[b, q] = sum over t with tok[b, t] == rows[q] of g[b, t, cols[q]]
//
// fp32, the tokens in ascending order.  One thread per kept entry, the
// sample's ids staged through LDS in runs; a column outside [0, E) or a
// negative id adds nothing.
template <int DT>
__global__ __launch_bounds__(256) void embed_gather_entries(const int64_t* __restrict__ tok, int64_t tok_bs,
                                                            int64_t tok_ts, const char* __restrict__ g,
                                                            int64_t g_bs, int64_t g_ts, int64_t tokens, int64_t E,
                                                            const int64_t* __restrict__ rows,
                                                            const int64_t* __restrict__ cols, int64_t k,
                                                            float* __restrict__ out, int64_t ld_out) {
  __shared__ int64_t ids[kEmbedIds];
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  const bool live = q < k;
  const int64_t v = live ? rows[q] : -1, e = live ? cols[q] : -1;
  const bool use = live && v >= 0 && e >= 0 && e < E;
  const int64_t* tb = tok + b * tok_bs;
  const char* gb = g + b * g_bs;
  float acc = 0.f;
  for (int64_t t0 = 0; t0 < tokens; t0 += kEmbedIds) {
    const int n = (int)(tokens - t0 < kEmbedIds ? tokens - t0 : kEmbedIds);
    __syncthreads();  // the previous run is consumed
    for (int i = threadIdx.x; i < n; i += blockDim.x) ids[i] = tb[(t0 + i) * tok_ts];
    __syncthreads();
    if (!use) continue;
    for (int i = 0; i < n; ++i)
      if (ids[i] == v) acc += Elem<DT>::load(gb + (t0 + i) * g_ts, e);
  }
  if (live) out[b * ld_out + q] = acc;
}

}  // namespace
}  // namespace da

namespace da {
namespace {
// Scratch of da_materialize_embedding: the int32 slots, then (2-byte outputs)
// the fp32 (B, T, E) sums, 256-byte aligned.
size_t embed_ws(int64_t batch, int64_t tokens, int64_t E, int dtype, size_t* scratch_off) {
  const size_t slots = ((size_t)(batch * tokens) * sizeof(int32_t) + 255) & ~(size_t)255;
  *scratch_off = slots;
  return slots + (dtype == DA_F32 ? 0 : (size_t)(batch * tokens * E) * sizeof(float));
}
}  // namespace
}  // namespace da

extern "C" int da_materialize_embedding_workspace(int64_t batch, int64_t tokens, int64_t E, int dtype,
                                                  size_t* bytes) {
  using namespace da;
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "da_materialize_embedding_workspace: bad dtype");
  if (batch < 0 || tokens < 0 || E < 0 || !bytes)
    return set_error(DA_ERR_INVALID, "da_materialize_embedding_workspace: bad argument");
  size_t off;
  *bytes = embed_ws(batch, tokens, E, dtype, &off);
  return DA_OK;
}

extern "C" int da_materialize_embedding(const int64_t* tok, const void* g, int dtype, int64_t batch, int64_t tokens,
                                        int64_t E, int64_t vocab, int64_t tok_bstride, int64_t tok_tstride,
                                        int64_t g_bstride, int64_t g_tstride, void* out, int64_t out_bstride,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  using namespace da;
  const char* who = "da_materialize_embedding";
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "%s: bad dtype", who);
  if (batch < 0 || tokens < 0 || E < 0 || vocab < 0) return set_error(DA_ERR_INVALID, "%s: negative size", who);
  if (batch == 0 || E == 0 || vocab == 0) return DA_OK;
  const int64_t es = (int64_t)elem_bytes(dtype), vec = 16 / es;
  if (!out || (tokens > 0 && (!tok || !g))) return set_error(DA_ERR_INVALID, "%s: NULL pointer", who);
  if (E % vec || ((uintptr_t)g & 15) || ((uintptr_t)out & 15) || (g_bstride * es) % 16 || (g_tstride * es) % 16 ||
      (out_bstride * es) % 16 || ((uintptr_t)tok & 7))
    return set_error(DA_ERR_INVALID, "%s: rows must be 16-byte aligned (E a multiple of %lld)", who, (long long)vec);
  if (out_bstride < vocab * E) return set_error(DA_ERR_INVALID, "%s: out batch stride below vocab * E", who);
  if (vocab > INT32_MAX || tokens > INT32_MAX)
    return set_error(DA_ERR_INVALID, "%s: vocab and tokens must be below 2^31", who);
  if (batch > 65535) return set_error(DA_ERR_INVALID, "%s: batch above 65535", who);
  size_t scratch_off;
  const size_t need = embed_ws(batch, tokens, E, dtype, &scratch_off);
  if (tokens > 0 && (!workspace || workspace_bytes < need))
    return set_error(DA_ERR_WORKSPACE, "%s: workspace needs %zu bytes, got %zu", who, need, workspace_bytes);
  hipStream_t st = (hipStream_t)stream;
  // zero the blocks (a fill kernel, so the call can be captured in a graph)
  {
    const int64_t chunks = vocab * E * es / 16, n = batch * chunks;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 8192);
    zero_runs16<<<(unsigned)blocks, 256, 0, st>>>((char*)out, batch, chunks, out_bstride * es);
  }
  int rc = check_launch(who);
  if (rc || tokens == 0) return rc;
  int32_t* slot = (int32_t*)workspace;
  float* scratch = (float*)((char*)workspace + scratch_off);
  // row slices: enough blocks to fill the chip, each thread's add chain ~tokens / slices long
  const int64_t xg = (E / vec + 255) / 256;
  int64_t slices = (4096 + xg * batch - 1) / (xg * batch);
  slices = std::max<int64_t>(1, std::min<int64_t>({slices, 256, dtype == DA_F32 ? vocab : tokens}));
  dim3 grid((unsigned)xg, (unsigned)batch, (unsigned)slices);
  if (dtype == DA_F32) {
    embed_accumulate<DA_F32, false><<<grid, 256, 0, st>>>(tok, tok_bstride, tok_tstride, nullptr, (const char*)g,
                                                          g_bstride * es, g_tstride * es, tokens, E, vocab,
                                                          (float*)out, out_bstride);
    return check_launch(who);
  }
  embed_first_slot<<<dim3((unsigned)((tokens + 255) / 256), (unsigned)batch), 256, 0, st>>>(
      tok, tok_bstride, tok_tstride, tokens, vocab, slot);
  rc = check_launch(who);
  if (rc) return rc;
  const int64_t wblocks = tokens * xg;
  if (wblocks > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: too many tokens", who);
  if (dtype == DA_BF16) {
    embed_accumulate<DA_BF16, true><<<grid, 256, 0, st>>>(tok, tok_bstride, tok_tstride, slot, (const char*)g,
                                                          g_bstride * es, g_tstride * es, tokens, E, vocab, scratch,
                                                          tokens * E);
    embed_write_slots<DA_BF16><<<dim3((unsigned)wblocks, (unsigned)batch), 256, 0, st>>>(
        tok, tok_bstride, tok_tstride, slot, scratch, tokens, E, xg, (char*)out, out_bstride);
  } else {
    embed_accumulate<DA_F16, true><<<grid, 256, 0, st>>>(tok, tok_bstride, tok_tstride, slot, (const char*)g,
                                                         g_bstride * es, g_tstride * es, tokens, E, vocab, scratch,
                                                         tokens * E);
    embed_write_slots<DA_F16><<<dim3((unsigned)wblocks, (unsigned)batch), 256, 0, st>>>(
        tok, tok_bstride, tok_tstride, slot, scratch, tokens, E, xg, (char*)out, out_bstride);
  }
  return check_launch(who);
}

extern "C" int da_dense_per_token_embedding(const int64_t* tok, const void* g, int dtype, int64_t b1, int64_t len1,
                                            int64_t E, int64_t vocab, int64_t tok_bstride, int64_t tok_tstride,
                                            int64_t g_bstride, int64_t g_tstride, const void* m2, int64_t m2_bstride,
                                            int64_t b2, float* out, int64_t ld_b1, int64_t ld_t, int64_t ld_b2,
                                            int accumulate, void* stream) {
  using namespace da;
  const char* who = "da_dense_per_token_embedding";
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "%s: bad dtype", who);
  if (b1 < 0 || len1 < 0 || E < 0 || vocab < 0 || b2 < 0) return set_error(DA_ERR_INVALID, "%s: negative size", who);
  if (b1 == 0 || len1 == 0 || b2 == 0) return DA_OK;
  if (!tok || !g || !m2 || !out) return set_error(DA_ERR_INVALID, "%s: NULL pointer", who);
  const int64_t es = (int64_t)elem_bytes(dtype), vec = 16 / es;
  if (E % vec || ((uintptr_t)g & 15) || ((uintptr_t)m2 & 15) || (g_bstride * es) % 16 || (g_tstride * es) % 16 ||
      (m2_bstride * es) % 16 || ((uintptr_t)tok & 7))
    return set_error(DA_ERR_INVALID, "%s: rows must be 16-byte aligned (E a multiple of %lld)", who, (long long)vec);
  if (m2_bstride < vocab * E) return set_error(DA_ERR_INVALID, "%s: m2 batch stride below vocab * E", who);
  const int64_t waves = b1 * len1, blocks = (waves + 3) / 4;
  if (blocks > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: too many tokens", who);
  hipStream_t st = (hipStream_t)stream;
#define DA_EDPT(DT)                                                                                          \
  embed_dense_per_token<DT><<<(unsigned)blocks, 256, 0, st>>>(tok, tok_bstride, tok_tstride, (const char*)g,  \
                                                              g_bstride * es, g_tstride * es, b1, len1, E,    \
                                                              vocab, (const char*)m2, m2_bstride, b2, out,    \
                                                              ld_b1, ld_t, ld_b2, accumulate)
  switch (dtype) {
    case DA_BF16: DA_EDPT(DA_BF16); break;
    case DA_F16: DA_EDPT(DA_F16); break;
    default: DA_EDPT(DA_F32); break;
  }
#undef DA_EDPT
  return check_launch(who);
}

extern "C" int da_gather_embedding_entries(const int64_t* tok, const void* g, int dtype, int64_t batch,
                                           int64_t tokens, int64_t E, int64_t tok_bstride, int64_t tok_tstride,
                                           int64_t g_bstride, int64_t g_tstride, const int64_t* rows,
                                           const int64_t* cols, int64_t k, float* out, int64_t ld_out,
                                           void* stream) {
  using namespace da;
  const char* who = "da_gather_embedding_entries";
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "%s: bad dtype", who);
  if (batch < 0 || tokens < 0 || E < 0 || k < 0) return set_error(DA_ERR_INVALID, "%s: negative size", who);
  if (batch == 0 || k == 0) return DA_OK;
  if (!out || !rows || !cols || (tokens > 0 && (!tok || !g))) return set_error(DA_ERR_INVALID, "%s: NULL pointer", who);
  if (ld_out < k) return set_error(DA_ERR_INVALID, "%s: ld_out below k", who);
  if (batch > 65535 || (k + 255) / 256 > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: problem too large", who);
  const int64_t es = (int64_t)elem_bytes(dtype);
  dim3 grid((unsigned)((k + 255) / 256), (unsigned)batch);
  hipStream_t st = (hipStream_t)stream;
#define DA_EGE(DT)                                                                                             \
  embed_gather_entries<DT><<<grid, 256, 0, st>>>(tok, tok_bstride, tok_tstride, (const char*)g, g_bstride * es, \
                                                 g_tstride * es, tokens, E, rows, cols, k, out, ld_out)
  switch (dtype) {
    case DA_BF16: DA_EGE(DA_BF16); break;
    case DA_F16: DA_EGE(DA_F16); break;
    default: DA_EGE(DA_F32); break;
  }
#undef DA_EGE
  return check_launch(who);
}

