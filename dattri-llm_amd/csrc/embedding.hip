// Embedding layers (nn.Embedding, and nn.EmbeddingBag spread over its tokens)
// on gfx950: the weight-gradient scatter, the cross-gram of two factorized
// sides and the per-token products.  All are HBM/L2-bound gathers and
// scatters of 16-byte row chunks; no MFMA.
#include <algorithm>

#include <rocprim/device/device_segmented_radix_sort.hpp>

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


// ---------------------------------------------------------------------------
// Cross-gram of two embedding sides (dot.py:58-74, :189-203, :325-337).
//
// An embedding's weight gradient is sum_t e_{tok_t} g_t^T, so
//
//   K[i, t, j] = g1[i, t, :] . G2_j[tok1[i, t], :],   G2_j[v] = sum over s with tok2[j, s] == v of g2[j, s, :]
//
// and K[i, j] = sum_t K[i, t, j].  The reference scatters each side-2 sample
// into a (vocab, E) table and gathers from it.  Here side 2 is compacted
// instead: its tokens' first occurrences (embed_first_slot) carry the fp32
// row sums (embed_accumulate), and a segmented radix sort gives every sample
// its ascending distinct ids with their slots.  Then one wave per side-1
// token looks its id up in 64 side-2 samples at once (one binary search per
// lane) and runs a wave-wide dot for each sample that holds it.  Work is
// O(B1 T1 B2 log T2) searches plus one E-long dot per match, never a
// (T1 x T2) product.
// ---------------------------------------------------------------------------

// keys[b*T + t] = the id of a first occurrence (slot == t), else all ones
// (past every id); vals = t.  Also the segment offsets b*T.
__global__ void embed_keys(const int64_t* __restrict__ tok, int64_t tok_bs, int64_t tok_ts,
                           const int32_t* __restrict__ slot, int64_t batch, int64_t tokens,
                           uint64_t* __restrict__ keys, int32_t* __restrict__ vals, int32_t* __restrict__ seg) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i <= batch) seg[i < batch ? i : batch] = (int32_t)((i < batch ? i : batch) * tokens);
  if (i >= batch * tokens) return;
  const int64_t b = i / tokens, t = i - b * tokens;
  const bool first = slot[i] == t;
  keys[i] = first ? (uint64_t)tok[b * tok_bs + t * tok_ts] : ~0ULL;
  vals[i] = (int32_t)t;
}

// One wave per side-1 token (i, t): out[i*ld_b1 + t*ld_t + j*ld_b2] (+)= g1[i,t] . rows2[j, slot]
// for every side-2 sample j holding the token's id (0 otherwise); with diag,
// only j = i, into out[i*ld_b1 + t*ld_t].
template <int DT>
__global__ __launch_bounds__(256) void embed_lookup_dot(const int64_t* __restrict__ tok1, int64_t tok1_bs,
                                                        int64_t tok1_ts, const char* __restrict__ g1, int64_t g1_bs,
                                                        int64_t g1_ts, int64_t b1, int64_t len1, int64_t E,
                                                        const uint64_t* __restrict__ keys2,
                                                        const int32_t* __restrict__ slots2,
                                                        const float* __restrict__ rows2, int64_t b2, int64_t len2,
                                                        int diag, float* __restrict__ out, int64_t ld_b1,
                                                        int64_t ld_t, int64_t ld_b2, int accumulate) {
  constexpr int VEC = Elem<DT>::kVec;
  const int lane = threadIdx.x & 63;
  const int64_t u = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (u >= b1 * len1) return;  // uniform per wave
  const int64_t i = u / len1, t = u - i * len1;
  const int64_t v = tok1[i * tok1_bs + t * tok1_ts];
  const char* grow = g1 + i * g1_bs + t * g1_ts;
  float* o = out + i * ld_b1 + t * ld_t;
  const int64_t chunks = E / VEC;
  const int64_t nj = diag ? 1 : b2;
  for (int64_t j0 = 0; j0 < nj; j0 += kWave) {
    // lane l searches sample j0 + l
    const int64_t jl = diag ? i : j0 + lane;
    bool hit = false;
    int64_t slot = 0;
    if ((diag ? lane == 0 : j0 + lane < nj) && v >= 0) {
      const uint64_t* k = keys2 + jl * len2;
      int64_t lo = 0, hi = len2;
      while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (k[mid] < (uint64_t)v) lo = mid + 1; else hi = mid;
      }
      hit = lo < len2 && k[lo] == (uint64_t)v;
      if (hit) slot = slots2[jl * len2 + lo];
    }
    if (!accumulate && (diag ? lane == 0 : j0 + lane < nj) && !hit) o[(diag ? 0 : j0 + lane) * ld_b2] = 0.f;
    uint64_t mask = __ballot(hit);
    while (mask) {
      const int l = __builtin_ctzll(mask);
      mask &= mask - 1;
      const int64_t j = diag ? i : j0 + l;
      const int64_t sj = __shfl((long long)slot, l);
      const float* r2 = rows2 + (j * len2 + sj) * E;
      float acc = 0.f;
      for (int64_t c = lane; c < chunks; c += kWave) {
        float x[VEC];
        unpack16<DT>(ld16(grow + c * 16), x);
#pragma unroll
        for (int e = 0; e < VEC; e += 4) {
          const f32x4 y = *(const f32x4*)(r2 + c * VEC + e);
          acc = fmaf(x[e], y[0], acc);
          acc = fmaf(x[e + 1], y[1], acc);
          acc = fmaf(x[e + 2], y[2], acc);
          acc = fmaf(x[e + 3], y[3], acc);
        }
      }
      acc = wave_sum(acc);
      if (lane == 0) {
        float* d = o + (diag ? 0 : j0 + l) * ld_b2;
        *d = accumulate ? *d + acc : acc;
      }
    }
  }
}

// out[i*ld_out + j] (+)= sum_t pt[(i*len1 + t)*nj + j]: one block per (i, 64
// consecutive j), each of its 4 waves summing a quarter of the tokens in
// ascending order (lane = j), the quarters then added in wave order.
__global__ __launch_bounds__(256) void embed_token_sum(const float* __restrict__ pt, int64_t b1, int64_t len1,
                                                       int64_t nj, float* __restrict__ out, int64_t ld_out,
                                                       int accumulate) {
  __shared__ float part[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t i = blockIdx.y, j = (int64_t)blockIdx.x * 64 + lane;
  const int64_t per = (len1 + 3) / 4, t0 = wave * per, t1 = t0 + per < len1 ? t0 + per : len1;
  float s = 0.f;
  if (j < nj) {
    const float* p = pt + i * len1 * nj + j;
#pragma unroll 8
    for (int64_t t = t0; t < t1; ++t) s += p[t * nj];
  }
  part[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && j < nj) {
    const float tot = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
    float* d = out + i * ld_out + j;
    *d = accumulate ? *d + tot : tot;
  }
}

size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

// Workspace of the embedding cross-gram: side 2's slots, fp32 slot rows, sort
// keys / values (twice), segment offsets, the sort's scratch, and (sum over t)
// the per-token products.
struct EmbGramWs {
  size_t slot, rows, keys, keys2, vals, vals2, seg, sort, pt, total, sort_bytes;
};

int emb_gram_plan(const da_factor_side* s1, const da_factor_side* s2, int64_t E, int dtype, bool diag, bool per_token,
                  EmbGramWs* w) {
  const char* who = "da_embedding_cross_gram";
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "%s: bad dtype %d", who, dtype);
  if (!s1 || !s2) return set_error(DA_ERR_INVALID, "%s: NULL side", who);
  const int64_t es = (int64_t)elem_bytes(dtype);
  if (E <= 0 || (E * es) % 16)
    return set_error(DA_ERR_INVALID, "%s: E=%lld must be a positive multiple of %lld elements", who, (long long)E,
                     (long long)(16 / es));
  const da_factor_side* sd[2] = {s1, s2};
  for (int q = 0; q < 2; ++q) {
    const da_factor_side* s = sd[q];
    if (s->batch < 0 || s->tokens < 0) return set_error(DA_ERR_INVALID, "%s: negative batch/tokens", who);
    if (s->seg_offsets || s->row_index || s->has_bias)
      return set_error(DA_ERR_INVALID, "%s: embedding sides are dense, without a bias column", who);
    if (s->batch == 0 || s->tokens == 0) continue;
    if (!s->act || !s->grad) return set_error(DA_ERR_INVALID, "%s: NULL factor", who);
    if (((uintptr_t)s->act & 7) || ((uintptr_t)s->grad & 15) || (s->grad_tstride * es) % 16 ||
        (s->grad_bstride * es) % 16)
      return set_error(DA_ERR_INVALID, "%s: gradient rows must be 16-byte aligned", who);
  }
  if (s1->batch > 65535) return set_error(DA_ERR_INVALID, "%s: side 1 batch above 65535", who);
  if (diag && s1->batch != s2->batch)
    return set_error(DA_ERR_INVALID, "%s: diag needs one batch size on both sides (%lld vs %lld)", who,
                     (long long)s1->batch, (long long)s2->batch);
  const int64_t n2 = s2->batch * s2->tokens;
  if (n2 > 0x7fffffffLL || s2->batch > 65535) return set_error(DA_ERR_INVALID, "%s: side 2 too large", who);
  size_t sort_bytes = 0;
  if (n2 > 0) {
    hipError_t e = rocprim::segmented_radix_sort_pairs(
        nullptr, sort_bytes, (const uint64_t*)nullptr, (uint64_t*)nullptr, (const int32_t*)nullptr,
        (int32_t*)nullptr, (unsigned int)n2, (unsigned int)s2->batch, (const int32_t*)nullptr,
        (const int32_t*)nullptr, 0, 64, (hipStream_t)0);
    if (e != hipSuccess) return set_error(DA_ERR_HIP, "%s: sort sizing failed: %s", who, hipGetErrorString(e));
  }
  size_t o = 0;
  w->slot = o; o = a256(o + (size_t)n2 * 4);
  w->rows = o; o = a256(o + (size_t)n2 * E * 4);
  w->keys = o; o = a256(o + (size_t)n2 * 8);
  w->keys2 = o; o = a256(o + (size_t)n2 * 8);
  w->vals = o; o = a256(o + (size_t)n2 * 4);
  w->vals2 = o; o = a256(o + (size_t)n2 * 4);
  w->seg = o; o = a256(o + (size_t)(s2->batch + 1) * 4);
  w->sort = o; o = a256(o + sort_bytes);
  w->pt = o;
  if (!per_token) o = a256(o + (size_t)(s1->batch * s1->tokens * (diag ? 1 : s2->batch)) * 4);
  w->total = o;
  w->sort_bytes = sort_bytes;
  return DA_OK;
}

// Side 2 compacted: slot rows (fp32 sums) and sorted ids per sample.
template <int DT>
int emb_compact(const da_factor_side* s2, int64_t E, char* ws, const EmbGramWs& w, hipStream_t st) {
  const int64_t b2 = s2->batch, len2 = s2->tokens, n2 = b2 * len2;
  constexpr int64_t es = Elem<DT>::kBytes, vec = 16 / es;
  const int64_t* tok = (const int64_t*)s2->act;
  int32_t* slot = (int32_t*)(ws + w.slot);
  float* rows = (float*)(ws + w.rows);
  embed_first_slot<<<dim3((unsigned)((len2 + 255) / 256), (unsigned)b2), 256, 0, st>>>(
      tok, s2->act_bstride, s2->act_tstride, len2, INT64_MAX, slot);
  const int64_t xg = (E / vec + 255) / 256;
  int64_t slices = (4096 + xg * b2 - 1) / (xg * b2);
  slices = std::max<int64_t>(1, std::min<int64_t>({slices, 256, len2}));
  embed_accumulate<DT, true><<<dim3((unsigned)xg, (unsigned)b2, (unsigned)slices), 256, 0, st>>>(
      tok, s2->act_bstride, s2->act_tstride, slot, (const char*)s2->grad, s2->grad_bstride * es,
      s2->grad_tstride * es, len2, E, INT64_MAX, rows, len2 * E);
  embed_keys<<<(unsigned)((std::max<int64_t>(n2, b2 + 1) + 255) / 256), 256, 0, st>>>(
      tok, s2->act_bstride, s2->act_tstride, slot, b2, len2, (uint64_t*)(ws + w.keys), (int32_t*)(ws + w.vals),
      (int32_t*)(ws + w.seg));
  int rc = check_launch("da_embedding_cross_gram(compact)");
  if (rc) return rc;
  size_t tb = w.sort_bytes;
  const int32_t* seg = (const int32_t*)(ws + w.seg);
  hipError_t e = rocprim::segmented_radix_sort_pairs(
      ws + w.sort, tb, (const uint64_t*)(ws + w.keys), (uint64_t*)(ws + w.keys2), (const int32_t*)(ws + w.vals),
      (int32_t*)(ws + w.vals2), (unsigned int)n2, (unsigned int)b2, seg, seg + 1, 0, 64, st);
  if (e != hipSuccess) return set_error(DA_ERR_HIP, "da_embedding_cross_gram: sort failed: %s", hipGetErrorString(e));
  return DA_OK;
}

template <int DT>
int emb_gram_run(const da_factor_side* s1, const da_factor_side* s2, int64_t E, bool diag, bool per_token,
                 float* out, int64_t ld_b1, int64_t ld_t, int64_t ld_b2, int accumulate, char* ws,
                 const EmbGramWs& w, hipStream_t st) {
  const int64_t b1 = s1->batch, len1 = s1->tokens, b2 = s2->batch, len2 = s2->tokens;
  const int64_t nj = diag ? 1 : b2;
  constexpr int64_t es = Elem<DT>::kBytes;
  if (len2 > 0) {
    int rc = emb_compact<DT>(s2, E, ws, w, st);
    if (rc) return rc;
  }
  float* pt = per_token ? out : (float*)(ws + w.pt);
  const int64_t pb1 = per_token ? ld_b1 : len1 * nj, pt_t = per_token ? ld_t : nj, pb2 = per_token ? ld_b2 : 1;
  const int acc_pt = per_token ? accumulate : 0;
  // (with no side-2 tokens every search misses and the products are written as zeros)
  const int64_t waves = b1 * len1;
  if ((waves + 3) / 4 > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "da_embedding_cross_gram: too many tokens");
  embed_lookup_dot<DT><<<(unsigned)((waves + 3) / 4), 256, 0, st>>>(
      (const int64_t*)s1->act, s1->act_bstride, s1->act_tstride, (const char*)s1->grad, s1->grad_bstride * es,
      s1->grad_tstride * es, b1, len1, E, (const uint64_t*)(ws + w.keys2), (const int32_t*)(ws + w.vals2),
      (const float*)(ws + w.rows), b2, len2, diag ? 1 : 0, pt, pb1, pt_t, pb2, acc_pt);
  int rc = check_launch("da_embedding_cross_gram(lookup)");
  if (rc || per_token) return rc;
  embed_token_sum<<<dim3((unsigned)((nj + 63) / 64), (unsigned)b1), 256, 0, st>>>(pt, b1, len1, nj, out, ld_b1,
                                                                                   accumulate);
  return check_launch("da_embedding_cross_gram(sum)");
}

int emb_gram_entry(const da_factor_side* s1, const da_factor_side* s2, int64_t E, int dtype, bool diag,
                   bool per_token, float* out, int64_t ld_b1, int64_t ld_t, int64_t ld_b2, int accumulate,
                   void* workspace, size_t workspace_bytes, hipStream_t st) {
  const char* who = per_token ? "da_embedding_cross_gram_per_token" : "da_embedding_cross_gram";
  EmbGramWs w;
  int rc = emb_gram_plan(s1, s2, E, dtype, diag, per_token, &w);
  if (rc) return rc;
  if (s1->batch == 0 || s2->batch == 0) return DA_OK;
  if (!out) return set_error(DA_ERR_INVALID, "%s: out is NULL", who);
  if (s1->tokens == 0) {
    if (accumulate || per_token) return DA_OK;
    return zero_f32_2d(out, s1->batch, diag ? 1 : s2->batch, ld_b1, st);
  }
  if (!workspace || workspace_bytes < w.total)
    return set_error(DA_ERR_WORKSPACE, "%s: workspace needs %zu bytes, got %zu", who, w.total, workspace_bytes);
  switch (dtype) {
    case DA_BF16:
      return emb_gram_run<DA_BF16>(s1, s2, E, diag, per_token, out, ld_b1, ld_t, ld_b2, accumulate, (char*)workspace,
                                   w, st);
    case DA_F16:
      return emb_gram_run<DA_F16>(s1, s2, E, diag, per_token, out, ld_b1, ld_t, ld_b2, accumulate, (char*)workspace,
                                  w, st);
    default:
      return emb_gram_run<DA_F32>(s1, s2, E, diag, per_token, out, ld_b1, ld_t, ld_b2, accumulate, (char*)workspace,
                                  w, st);
  }
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

extern "C" int da_embedding_cross_gram_workspace(const da_factor_side* s1, const da_factor_side* s2, int64_t E,
                                                 int dtype, int diag, size_t* bytes) {
  using namespace da;
  if (!bytes) return set_error(DA_ERR_INVALID, "da_embedding_cross_gram_workspace: bytes is NULL");
  EmbGramWs w;
  int rc = emb_gram_plan(s1, s2, E, dtype, diag != 0, false, &w);
  if (rc) return rc;
  *bytes = w.total;
  return DA_OK;
}

extern "C" int da_embedding_cross_gram(const da_factor_side* s1, const da_factor_side* s2, int64_t E, int dtype,
                                       int diag, float* out, int64_t ld_out, int accumulate, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  return da::emb_gram_entry(s1, s2, E, dtype, diag != 0, false, out, ld_out, 0, 0, accumulate, workspace,
                            workspace_bytes, (hipStream_t)stream);
}

extern "C" int da_embedding_cross_gram_per_token_workspace(const da_factor_side* s1, const da_factor_side* s2,
                                                           int64_t E, int dtype, size_t* bytes) {
  using namespace da;
  if (!bytes) return set_error(DA_ERR_INVALID, "da_embedding_cross_gram_per_token_workspace: bytes is NULL");
  EmbGramWs w;
  int rc = emb_gram_plan(s1, s2, E, dtype, false, true, &w);
  if (rc) return rc;
  *bytes = w.total;
  return DA_OK;
}

extern "C" int da_embedding_cross_gram_per_token(const da_factor_side* s1, const da_factor_side* s2, int64_t E,
                                                 int dtype, float* out, int64_t ld_b1, int64_t ld_t, int64_t ld_b2,
                                                 int accumulate, void* workspace, size_t workspace_bytes,
                                                 void* stream) {
  return da::emb_gram_entry(s1, s2, E, dtype, false, true, out, ld_b1, ld_t, ld_b2, accumulate, workspace,
                            workspace_bytes, (hipStream_t)stream);
}

