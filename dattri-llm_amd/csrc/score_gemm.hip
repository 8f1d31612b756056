// K3a: multi-layer score GEMM on the dense (materialized) route.
//
//   out[i, j] (+)= sum_L sum_c m1_L[i, c] * m2_L[j, c]
//
// Follows the dense cross-gram of cross_gram / cross_dot,
// dattri_llm/gradient/ops/dot.py:114 and :501-505 (M1 @ M2.T per layer), summed
// over layers as in layerwise_cross_dot, dot.py:599-604 -- but all layers in one
// launch with fp32 accumulation throughout.
//
// The product is skinny (B1, B2 in the tens, widths up to 10^8) and bound by
// streaming both operands from HBM once.  The flattened width of every layer
// is cut into chunks; a workgroup owns one chunk of one layer for a 16-row x
// 64-row (side-1 x side-2) output tile and runs 16x16x32 MFMAs straight from
// registers (every element is used by exactly one MFMA of the tile, so there
// is nothing to share through LDS).  In a 16x16 MFMA four lanes serve one
// row; they read 64 contiguous bytes of it per load instruction, and the same
// element-to-k assignment is used on both sides, so the sum is exact in any
// order.  The four waves split the chunk, combine through LDS and write one
// fp32 partial tile; a second kernel sums the partials in a fixed order.
#include "common.h"

namespace da {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxLayers = 32;
constexpr int kTileM = 16;   // side-1 rows per workgroup
constexpr int kTileN = 64;   // side-2 rows per workgroup (4 MFMA blocks)
constexpr int kStep = 256;   // bytes of width per row and wave iteration
constexpr int kUnit = 4 * kStep;  // chunk granularity: one iteration of every wave

struct LayerDev {
  const char* m1;
  const char* m2;
  int64_t bytes;       // row width in bytes (multiple of 16)
  int64_t ld1, ld2;    // row strides in bytes
  int64_t blk1, blk2;  // strides between consecutive 64-element blocks of a row, in bytes
  int64_t chunk0;      // first global chunk index of this layer
};

// Byte address of logical byte `off` of a row: rows are sequences of
// 64-element blocks (kBlk bytes) placed blk bytes apart -- blk == kBlk is the
// plain row-major layout, blk == rows * kBlk the k-blocked (sample-interleaved)
// layout in which one block of every row is contiguous.
template <int kBlk>
__device__ __forceinline__ const char* at(const char* row, int64_t blk, int64_t off) {
  return row + (off / kBlk) * blk + (off % kBlk);
}

struct ScoreArgs {
  LayerDev layers[kMaxLayers];
  int n_layers;
  int64_t chunk_bytes;  // bytes of width per chunk (multiple of kUnit)
  int64_t n_chunks;
  int64_t b1, b2;
  int64_t tiles_n;      // ceil(b2 / kTileN)
  float* partial;       // [b1][b2][n_chunks]
};

template <int DT>
__global__ __launch_bounds__(kThreads) void score_gemm_chunks(ScoreArgs s) {
  constexpr int kBlk = 64 * Elem<DT>::kBytes;  // bytes of one 64-element block
  __shared__ float red[3][kTileM * kTileN];

  const int64_t chunk = blockIdx.x;
  const int64_t tm = blockIdx.y / s.tiles_n, tn = blockIdx.y % s.tiles_n;
  int l = 0;
  while (l + 1 < s.n_layers && s.layers[l + 1].chunk0 <= chunk) ++l;
  const LayerDev L = s.layers[l];
  const int64_t c0 = (chunk - L.chunk0) * s.chunk_bytes;
  const int64_t c1 = min(c0 + s.chunk_bytes, L.bytes);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t i = tm * kTileM + r;
  const char* p1 = i < s.b1 ? L.m1 + i * L.ld1 : nullptr;
  const char* p2[4];
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    const int64_t j = tn * kTileN + 16 * blk + r;
    p2[blk] = j < s.b2 ? L.m2 + j * L.ld2 : nullptr;
  }

  f32x4 acc[4] = {};
  const int64_t span = c1 - c0;
  const int64_t quarter = ((span + kUnit - 1) / kUnit) * kStep;
  const int64_t w0 = c0 + wave * quarter;
  const int64_t w1 = min(w0 + quarter, c1);
  for (int64_t base = w0; base < w1; base += kStep) {
    // MFMA step st reads bytes [base + 64*st + 16*q, +16) of the lane's row.
    u32x4 va[4], vb[4][4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int64_t off = base + 64 * st + 16 * q;
      const bool in = off < w1;
      va[st] = (p1 && in) ? ld16(at<kBlk>(p1, L.blk1, off)) : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int blk = 0; blk < 4; ++blk)
        vb[blk][st] = (p2[blk] && in) ? ld16(at<kBlk>(p2[blk], L.blk2, off)) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) Mfma16<DT>::mma(acc[blk], va[st], vb[blk][st]);
  }

  // Combine the four waves' tiles: waves 1..3 park theirs in LDS, wave 0 sums.
  if (wave > 0) {
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        red[wave - 1][acc16_row(e, lane) * kTileN + 16 * blk + acc16_col(lane)] = acc[blk][e];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = acc16_row(e, lane), col = 16 * blk + acc16_col(lane);
        const int x = row * kTileN + col;
        const float v = acc[blk][e] + red[0][x] + red[1][x] + red[2][x];
        const int64_t oi = tm * kTileM + row, oj = tn * kTileN + col;
        if (oi < s.b1 && oj < s.b2) s.partial[(oi * s.b2 + oj) * s.n_chunks + chunk] = v;
      }
  }
}

// One workgroup per output: its n_chunks partials are contiguous; each thread
// sums a fixed strided subset, then a fixed tree combines the threads.
__global__ __launch_bounds__(256) void score_gemm_reduce(const float* __restrict__ partial,
                                                         int64_t n_chunks, int64_t b1, int64_t b2,
                                                         float* __restrict__ out, int64_t ld_row,
                                                         int64_t ld_col, int accumulate) {
  __shared__ float red[4];
  const int64_t idx = blockIdx.x;
  const float* p = partial + idx * n_chunks;
  float v = 0.f;
  for (int64_t c = threadIdx.x; c < n_chunks; c += 256) v += p[c];
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float sum = (red[0] + red[1]) + (red[2] + red[3]);
    const int64_t i = idx / b2, j = idx - i * b2;
    float* o = out + i * ld_row + j * ld_col;
    *o = accumulate ? *o + sum : sum;
  }
}

struct Plan {
  int64_t chunk_bytes, n_chunks;
  size_t ws;
};

int make_plan(int64_t b1, int64_t b2, const da_dense_layer* layers, int n_layers, int dtype,
              Plan* p) {
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "da_score_gemm: bad dtype %d", dtype);
  if (b1 < 0 || b2 < 0) return set_error(DA_ERR_INVALID, "da_score_gemm: negative batch");
  if (n_layers < 0 || (n_layers > 0 && !layers))
    return set_error(DA_ERR_INVALID, "da_score_gemm: bad layer list");
  if (n_layers > kMaxLayers)
    return set_error(DA_ERR_INVALID, "da_score_gemm: at most %d layers per call", kMaxLayers);
  const int64_t es = (int64_t)elem_bytes(dtype);
  int64_t total = 0;
  for (int l = 0; l < n_layers; ++l) {
    const da_dense_layer& L = layers[l];
    if (L.width < 0) return set_error(DA_ERR_INVALID, "da_score_gemm: layer %d negative width", l);
    if ((L.width * es) % 16 || (L.ld1 * es) % 16 || (L.ld2 * es) % 16)
      return set_error(DA_ERR_INVALID,
                       "da_score_gemm: layer %d width/strides must be multiples of 16 bytes", l);
    if (L.width > 0 && (!L.m1 || !L.m2 || (((uintptr_t)L.m1 | (uintptr_t)L.m2) & 15)))
      return set_error(DA_ERR_INVALID, "da_score_gemm: layer %d pointers NULL or misaligned", l);
    if (L.blk1 < 0 || L.blk2 < 0 || ((L.blk1 * es) % 16) || ((L.blk2 * es) % 16))
      return set_error(DA_ERR_INVALID, "da_score_gemm: layer %d block strides must be >= 0 and 16-byte multiples", l);
    total += L.width * es;
  }
  // Aim for ~4096 chunks over all layers (16 waves per CU), at least one
  // iteration of every wave (kUnit bytes) per chunk.
  const int64_t unit = kUnit;
  int64_t cb = (total / 4096 + unit - 1) / unit * unit;
  if (cb < unit) cb = unit;
  p->chunk_bytes = cb;
  int64_t n = 0;
  for (int l = 0; l < n_layers; ++l) n += (layers[l].width * es + cb - 1) / cb;
  p->n_chunks = n;
  p->ws = (size_t)(n * b1 * b2) * sizeof(float);
  return DA_OK;
}

}  // namespace
}  // namespace da

extern "C" {

int da_score_gemm_workspace(int64_t b1, int64_t b2, const da_dense_layer* layers, int n_layers,
                            int dtype, size_t* bytes) {
  da::Plan p;
  int rc = da::make_plan(b1, b2, layers, n_layers, dtype, &p);
  if (rc) return rc;
  if (!bytes) return da::set_error(DA_ERR_INVALID, "da_score_gemm_workspace: bytes is NULL");
  *bytes = p.ws;
  return DA_OK;
}

int da_score_gemm(int64_t b1, int64_t b2, const da_dense_layer* layers, int n_layers, int dtype,
                  float* out, int64_t ld_row, int64_t ld_col, int accumulate, void* workspace,
                  size_t workspace_bytes, void* stream) {
  using namespace da;
  Plan p;
  int rc = make_plan(b1, b2, layers, n_layers, dtype, &p);
  if (rc) return rc;
  if (b1 == 0 || b2 == 0) return DA_OK;
  if (!out) return set_error(DA_ERR_INVALID, "da_score_gemm: out is NULL");
  hipStream_t st = (hipStream_t)stream;
  if (p.n_chunks == 0) {
    if (accumulate) return DA_OK;
    if (ld_col != 1) return set_error(DA_ERR_INVALID, "da_score_gemm: empty product needs ld_col == 1");
    return zero_f32_2d(out, b1, b2, ld_row, st);
  }
  if (!workspace || workspace_bytes < p.ws)
    return set_error(DA_ERR_WORKSPACE, "da_score_gemm: workspace needs %zu bytes, got %zu", p.ws,
                     workspace_bytes);
  const int64_t es = (int64_t)elem_bytes(dtype);
  ScoreArgs s;
  s.n_layers = n_layers;
  int64_t c = 0;
  for (int l = 0; l < n_layers; ++l) {
    s.layers[l].m1 = (const char*)layers[l].m1;
    s.layers[l].m2 = (const char*)layers[l].m2;
    s.layers[l].bytes = layers[l].width * es;
    s.layers[l].ld1 = layers[l].ld1 * es;
    s.layers[l].ld2 = layers[l].ld2 * es;
    s.layers[l].blk1 = (layers[l].blk1 ? layers[l].blk1 : 64) * es;
    s.layers[l].blk2 = (layers[l].blk2 ? layers[l].blk2 : 64) * es;
    s.layers[l].chunk0 = c;
    c += (s.layers[l].bytes + p.chunk_bytes - 1) / p.chunk_bytes;
  }
  for (int l = n_layers; l < kMaxLayers; ++l) s.layers[l] = s.layers[n_layers - 1];
  s.chunk_bytes = p.chunk_bytes;
  s.n_chunks = p.n_chunks;
  s.b1 = b1;
  s.b2 = b2;
  s.tiles_n = (b2 + kTileN - 1) / kTileN;
  s.partial = (float*)workspace;
  const int64_t tiles = ((b1 + kTileM - 1) / kTileM) * s.tiles_n;
  if (p.n_chunks > 0x7fffffffLL || tiles > 65535)
    return set_error(DA_ERR_INVALID, "da_score_gemm: problem too large for one launch");
  dim3 grid((unsigned)p.n_chunks, (unsigned)tiles);
  switch (dtype) {
    case DA_BF16: score_gemm_chunks<DA_BF16><<<grid, kThreads, 0, st>>>(s); break;
    case DA_F16: score_gemm_chunks<DA_F16><<<grid, kThreads, 0, st>>>(s); break;
    default: score_gemm_chunks<DA_F32><<<grid, kThreads, 0, st>>>(s); break;
  }
  rc = check_launch("da_score_gemm(chunks)");
  if (rc) return rc;
  const int64_t n = b1 * b2;
  if (n > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "da_score_gemm: too many outputs");
  score_gemm_reduce<<<(unsigned)n, 256, 0, st>>>(
      (const float*)workspace, p.n_chunks, b1, b2, out, ld_row, ld_col, accumulate);
  return check_launch("da_score_gemm(reduce)");
}

}  // extern "C"
