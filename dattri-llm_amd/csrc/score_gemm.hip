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
// is cut into chunks; a workgroup owns one chunk of one layer for a 32-row x
// 64-row (side-1 x side-2) output tile.  Each lane loads 16-byte pieces of a
// 128-byte run of its row straight into MFMA operand registers (no LDS: every
// element is used by exactly one MFMA of the tile), the four waves split the
// chunk, combine through LDS, and write one fp32 partial tile; a second kernel
// sums the partials of each output in a fixed order.
#include "common.h"

namespace da {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxLayers = 32;
constexpr int kTileM = 32;  // side-1 rows per workgroup
constexpr int kTileN = 64;  // side-2 rows per workgroup
constexpr int kRun = 128;   // bytes of one row a lane reads per step group (8 x 16 B)

struct LayerDev {
  const char* m1;
  const char* m2;
  int64_t bytes;     // row width in bytes (multiple of 16)
  int64_t ld1, ld2;  // row strides in bytes
  int64_t chunk0;    // first global chunk index of this layer
};

struct ScoreArgs {
  LayerDev layers[kMaxLayers];
  int n_layers;
  int64_t chunk_bytes;  // bytes of width per chunk (multiple of 4 * 2 * kRun)
  int64_t n_chunks;
  int64_t b1, b2;
  int64_t tiles_n;      // ceil(b2 / kTileN)
  float* partial;       // [n_chunks][b1][b2]
};

template <int DT>
__global__ __launch_bounds__(kThreads) void score_gemm_chunks(ScoreArgs s) {
  __shared__ float red[3][kTileM * kTileN];

  const int64_t chunk = blockIdx.x;
  const int64_t tm = blockIdx.y / s.tiles_n, tn = blockIdx.y % s.tiles_n;
  int l = 0;
  while (l + 1 < s.n_layers && s.layers[l + 1].chunk0 <= chunk) ++l;
  const LayerDev L = s.layers[l];
  const int64_t c0 = (chunk - L.chunk0) * s.chunk_bytes;
  const int64_t c1 = min(c0 + s.chunk_bytes, L.bytes);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 31, h = lane >> 5;
  // Side-1 row (one 32-row block) and side-2 rows (two 32-row blocks) of this lane.
  const int64_t i = tm * kTileM + r;
  const int64_t j0 = tn * kTileN + r, j1 = j0 + 32;
  const char* p1 = i < s.b1 ? L.m1 + i * L.ld1 : nullptr;
  const char* q0 = j0 < s.b2 ? L.m2 + j0 * L.ld2 : nullptr;
  const char* q1 = j1 < s.b2 ? L.m2 + j1 * L.ld2 : nullptr;

  f32x16 acc0 = {}, acc1 = {};
  // The chunk is split into 4 quarter ranges, one per wave; each wave walks its
  // range in groups of 2 * kRun bytes: lane half h reads the run at
  // base + h * kRun, 16 bytes per MFMA step (same k-permutation on both sides).
  const int64_t span = c1 - c0;
  const int64_t quarter = ((span + 4 * 2 * kRun - 1) / (4 * 2 * kRun)) * (2 * kRun);
  const int64_t w0 = c0 + wave * quarter;
  const int64_t w1 = min(w0 + quarter, c1);
  for (int64_t base = w0; base < w1; base += 2 * kRun) {
    const int64_t run = base + h * kRun;
    u32x4 va[8], vb0[8], vb1[8];
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const int64_t off = run + 16 * st;
      const bool in = off < w1;
      va[st] = (p1 && in) ? ld16(p1 + off) : u32x4{0, 0, 0, 0};
      vb0[st] = (q0 && in) ? ld16(q0 + off) : u32x4{0, 0, 0, 0};
      vb1[st] = (q1 && in) ? ld16(q1 + off) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      Mfma32<DT>::mma(acc0, va[st], vb0[st]);
      Mfma32<DT>::mma(acc1, va[st], vb1[st]);
    }
  }

  // Combine the four waves' tiles: waves 1..3 park theirs in LDS, wave 0 sums.
  if (wave > 0) {
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int row = acc_row(q, lane), col = acc_col(lane);
      red[wave - 1][row * kTileN + col] = acc0[q];
      red[wave - 1][row * kTileN + 32 + col] = acc1[q];
    }
  }
  __syncthreads();
  if (wave == 0) {
    float* dst = s.partial + chunk * s.b1 * s.b2;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int row = acc_row(q, lane), col = acc_col(lane);
      const int64_t oi = tm * kTileM + row;
      const int e0 = row * kTileN + col, e1 = e0 + 32;
      const float v0 = acc0[q] + red[0][e0] + red[1][e0] + red[2][e0];
      const float v1 = acc1[q] + red[0][e1] + red[1][e1] + red[2][e1];
      const int64_t oj0 = tn * kTileN + col, oj1 = oj0 + 32;
      if (oi < s.b1) {
        if (oj0 < s.b2) dst[oi * s.b2 + oj0] = v0;
        if (oj1 < s.b2) dst[oi * s.b2 + oj1] = v1;
      }
    }
  }
}

__global__ void score_gemm_reduce(const float* __restrict__ partial, int64_t n_chunks, int64_t b1,
                                  int64_t b2, float* __restrict__ out, int64_t ld_row,
                                  int64_t ld_col, int accumulate) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= b1 * b2) return;
  const int64_t i = idx / b2, j = idx - i * b2;
  float s = 0.f;
  for (int64_t c = 0; c < n_chunks; ++c) s += partial[c * b1 * b2 + idx];
  float* o = out + i * ld_row + j * ld_col;
  *o = accumulate ? *o + s : s;
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
    total += L.width * es;
  }
  // Aim for ~4096 chunks over all layers (16 waves per CU), at least one
  // 4-wave step group (4 * 2 * kRun bytes) per chunk.
  const int64_t unit = 4 * 2 * kRun;
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
  score_gemm_reduce<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(
      (const float*)workspace, p.n_chunks, b1, b2, out, ld_row, ld_col, accumulate);
  return check_launch("da_score_gemm(reduce)");
}

}  // extern "C"
