// K1: fused ghost inner product (factorized cross-gram) on gfx950 MFMA.
//
//   out[i, j] = sum_{t < S1, s < S2} (a1[i,t,:] . a2[j,s,:]) * (g1[i,t,:] . g2[j,s,:])
//
// Follows the factorized route of cross_gram, dattri_llm/gradient/ops/dot.py:115-118,
// which forms K_a = A1 A2^T and K_g = G1 G2^T as two (B1*S1) x (B2*S2) matrices in
// HBM and then reduces their Hadamard product over each (S1 x S2) block.
//
// Here the same two products are computed as ONE tiled GEMM pair over the row
// spaces (B1*S1) x (B2*S2): a workgroup owns a tile that lies inside a single
// (i, j) sample pair, runs the activation K-loop into one set of fp32 MFMA
// accumulators and the gradient K-loop into a second set, and reduces
// (K_a + bias) * K_g in registers.  Only one fp32 per tile reaches HBM; a
// second tiny kernel sums the per-tile partials of each pair in a fixed order,
// so results are deterministic.
//
// Tile engines: the 256 x 128 tile on 8 waves (ghost_gram_tiles_v3 and the
// grouped MoE form ghost_grouped_tiles_v3, below) takes dense and grouped
// launches whose rows it can address with 32-bit offsets; the same tile on 4
// waves runs the per-token form; the 128 x 128 kernels first in this file
// take per-sample segmented sides and the rest.  Tile order:
// workgroups are remapped so each XCD owns a contiguous run of tiles, grouped
// a few row tiles wide, so the concurrently running tiles on one XCD share
// their operand row blocks through that XCD's L2.
#include <algorithm>
#include <vector>

#include "common.h"

namespace da {
namespace {

constexpr int kBM = 128;           // side-1 rows per tile
constexpr int kBN = 128;           // side-2 rows per tile
constexpr int kRowBytes = 128;     // bytes of K consumed per pipeline stage
constexpr int kLdsRow = kRowBytes + 16;  // padded LDS row (bank spread)
constexpr int kThreads = 256;      // 4 waves, 2 x 2 arrangement of 64 x 64
constexpr int kGroup = 8;          // row tiles per swizzle group
constexpr int kStageBytes = (kBM + kBN) * kLdsRow;

struct SideDev {
  const char* act;
  const char* grad;
  int64_t batch, tokens;
  int64_t act_bstride, act_tstride;    // bytes
  int64_t grad_bstride, grad_tstride;  // bytes
  const int32_t* seg;
  const int32_t* idx;
};

struct GhostArgs {
  SideDev s1, s2;
  int64_t kbytes_a, kbytes_g;  // K * esize, D * esize
  int64_t tiles_r, tiles_c;    // tiles per sample on each side
  int64_t n_r, n_c;            // total row / column tiles (diag: n_c = tiles_c)
  float bias;
  int diag;                    // only the pairs (i, i): sample i of side 1 with sample i of side 2
  float* partial;              // [B1][B2][tiles_r][tiles_c], diag: [B][tiles_r][tiles_c]
};

// Sample of side 2 for column tile C of row sample i, and the pair's slot in
// the partials.
__device__ __forceinline__ int64_t pair_col_sample(const GhostArgs& g, int64_t i, int64_t C) {
  return g.diag ? i : C / g.tiles_c;
}
__device__ __forceinline__ int64_t pair_slot(const GhostArgs& g, int64_t i, int64_t j) {
  return g.diag ? i : i * g.s2.batch + j;
}

__device__ __forceinline__ int64_t seg_start(const SideDev& s, int64_t b) {
  return s.seg ? (int64_t)s.seg[b] : 0;
}
__device__ __forceinline__ int64_t seg_len(const SideDev& s, int64_t b) {
  return s.seg ? (int64_t)(s.seg[b + 1] - s.seg[b]) : s.tokens;
}
// Byte offset of row t of sample b (t < length) for a factor with the given strides.
__device__ __forceinline__ int64_t row_off(const SideDev& s, int64_t b, int64_t start, int64_t t,
                                           int64_t bstride, int64_t tstride) {
  if (s.seg) {
    const int64_t r = start + t;
    const int64_t p = s.idx ? (int64_t)s.idx[r] : r;
    return p * tstride;
  }
  return b * bstride + t * tstride;
}

// One K-loop of the tile: acc[x][y] += P1[rows 64wm+32x..] . P2[rows 64wn+32y..]^T,
// operands staged through double-buffered LDS, next stage prefetched to registers.
template <int DT>
__device__ __forceinline__ void gram_tile(char* __restrict__ smem, const char* const (&p1)[4],
                                          const char* const (&p2)[4], int64_t kbytes,
                                          f32x16 (&acc)[2][2], int tid, int lane, int wm, int wn) {
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) acc[x][y] = f32x16{};
  const int lr = tid >> 3, lc = tid & 7;
  const int nk = (int)((kbytes + kRowBytes - 1) / kRowBytes);
  u32x4 r1[4], r2[4];

  auto gload = [&](int kt) {
    const int64_t off = (int64_t)kt * kRowBytes + 16 * lc;
    const bool kin = off < kbytes;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      r1[p] = (p1[p] && kin) ? ld16(p1[p] + off) : u32x4{0, 0, 0, 0};
      r2[p] = (p2[p] && kin) ? ld16(p2[p] + off) : u32x4{0, 0, 0, 0};
    }
  };
  auto lstore = [&](int buf) {
    char* base = smem + buf * kStageBytes;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      st16(base + (lr + 32 * p) * kLdsRow + 16 * lc, r1[p]);
      st16(base + (kBM + lr + 32 * p) * kLdsRow + 16 * lc, r2[p]);
    }
  };

  gload(0);
  lstore(0);
  __syncthreads();
  const int frow = lane & 31, fhalf = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    const char* base = smem + buf * kStageBytes;
#pragma unroll
    for (int kg = 0; kg < kRowBytes / 32; ++kg) {
      u32x4 fa[2], fb[2];
#pragma unroll
      for (int x = 0; x < 2; ++x)
        fa[x] = ld16(base + (64 * wm + 32 * x + frow) * kLdsRow + 32 * kg + 16 * fhalf);
#pragma unroll
      for (int y = 0; y < 2; ++y)
        fb[y] = ld16(base + (kBM + 64 * wn + 32 * y + frow) * kLdsRow + 32 * kg + 16 * fhalf);
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y) Mfma32<DT>::mma(acc[x][y], fa[x], fb[y]);
    }
    if (kt + 1 < nk) lstore(buf ^ 1);
    __syncthreads();
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads, 2) void ghost_gram_tiles(GhostArgs g) {
  __shared__ __attribute__((aligned(16))) char smem[2 * kStageBytes];
  __shared__ float red[kThreads / kWave];

  const int64_t logical = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t per_group = (int64_t)kGroup * g.n_c;
  const int64_t group = logical / per_group;
  const int64_t first_r = group * kGroup;
  const int64_t gsize = min(g.n_r - first_r, (int64_t)kGroup);
  const int64_t in_group = logical - group * per_group;
  const int64_t R = first_r + in_group % gsize;
  const int64_t C = in_group / gsize;
  const int64_t i = R / g.tiles_r, tt = R % g.tiles_r;
  const int64_t j = pair_col_sample(g, i, C), ss = C % g.tiles_c;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int64_t len1 = seg_len(g.s1, i), len2 = seg_len(g.s2, j);
  const int64_t t0 = tt * kBM, s0 = ss * kBN;
  float* dst = g.partial + (pair_slot(g, i, j) * g.tiles_r + tt) * g.tiles_c + ss;
  if (t0 >= len1 || s0 >= len2) {  // tile entirely past a segment end: contributes 0
    if (tid == 0) *dst = 0.f;
    return;
  }

  const int lr = tid >> 3;
  const int64_t st1 = seg_start(g.s1, i), st2 = seg_start(g.s2, j);
  const char* a1[4];
  const char* g1[4];
  const char* a2[4];
  const char* g2[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int64_t t = t0 + lr + 32 * p;
    const int64_t s = s0 + lr + 32 * p;
    const bool v1 = t < len1, v2 = s < len2;
    a1[p] = v1 ? g.s1.act + row_off(g.s1, i, st1, t, g.s1.act_bstride, g.s1.act_tstride) : nullptr;
    g1[p] = v1 ? g.s1.grad + row_off(g.s1, i, st1, t, g.s1.grad_bstride, g.s1.grad_tstride) : nullptr;
    a2[p] = v2 ? g.s2.act + row_off(g.s2, j, st2, s, g.s2.act_bstride, g.s2.act_tstride) : nullptr;
    g2[p] = v2 ? g.s2.grad + row_off(g.s2, j, st2, s, g.s2.grad_bstride, g.s2.grad_tstride) : nullptr;
  }

  f32x16 ka[2][2], kg[2][2];
  gram_tile<DT>(smem, a1, a2, g.kbytes_a, ka, tid, lane, wm, wn);
  gram_tile<DT>(smem, g1, g2, g.kbytes_g, kg, tid, lane, wm, wn);

  // Rows past a segment end have zero gradient rows, so K_g is 0 there and the
  // bias term (the implicit ones column) contributes nothing for them.
  float s = 0.f;
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += (ka[x][y][r] + g.bias) * kg[x][y][r];
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (tid == 0) *dst = (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ void ghost_gram_reduce(const float* __restrict__ partial, int64_t b1, int64_t b2,
                                  int64_t per_pair, float* __restrict__ out, int64_t ld_out,
                                  int accumulate) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= b1 * b2) return;
  const int64_t i = idx / b2, j = idx - i * b2;
  const float* p = partial + idx * per_pair;
  float s = 0.f;
  for (int64_t q = 0; q < per_pair; ++q) s += p[q];
  float* o = out + i * ld_out + j;
  *o = accumulate ? *o + s : s;
}

// ---------------------------------------------------------------------------
// Grouped (MoE) form: tiles over each expert's packed, sample-sorted rows.
// ---------------------------------------------------------------------------
constexpr int kMaxGroups = 16;  // groups per launch (the table travels as kernel arguments)
constexpr int kPRow = kBN + 1; // padded fp32 row of the parked product tile

struct GroupDev {
  const char* a1;
  const char* g1;
  const char* a2;
  const char* g2;
  const int32_t* seg1;
  const int32_t* seg2;
  const int32_t* idx1;
  const int32_t* idx2;
  int64_t rows1, rows2;               // packed rows per side (seg[B])
  int64_t a1_ts, g1_ts, a2_ts, g2_ts; // row strides, bytes
  int64_t tile0;                      // first tile of this group in the launch
  int64_t tiles_r, tiles_c;
  int64_t part_off, part_ld;          // partial region (floats) and its row length
  int64_t meta_off;                   // int32 offset of this group's span tables
  int64_t kbytes_a, kbytes_g;         // K * esize, D * esize
  float bias;                         // 1 with an implicit ones column, else 0
};

struct GroupedArgs {
  GroupDev grp[kMaxGroups];
  int n_groups;
  int tile_r, tile_c;  // tile heights on side 1 / side 2 (the spans are counted in tiles)
  int64_t b1, b2;
  float* partial;
  int32_t* meta;  // per group: first1[B1], pre1[B1+1], first2[B2], pre2[B2+1]
};
static_assert(sizeof(GroupedArgs) <= 3584, "grouped kernel arguments must stay well under 4 KB");

// Sample owning packed row p (p < seg[B]): the last b with seg[b] <= p.
__device__ __forceinline__ int64_t sample_of(const int32_t* seg, int64_t nb, int64_t p) {
  int64_t lo = 0, hi = nb;  // seg[lo] <= p < seg[hi]
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)seg[mid] <= p) lo = mid; else hi = mid;
  }
  return lo;
}

// Span tables of one side of one group: first[b] = first row tile of sample b,
// pre[b] = sum of spans (row tiles touched) of samples < b.  One workgroup per
// (group, side); sequential per thread chunk, then a scan of the chunk sums.
__global__ __launch_bounds__(256) void grouped_spans(GroupedArgs ga) {
  __shared__ int32_t part[256];
  const int e = blockIdx.x >> 1, side = blockIdx.x & 1;
  const GroupDev& G = ga.grp[e];
  const int64_t nb = side ? ga.b2 : ga.b1;
  const int32_t* seg = side ? G.seg2 : G.seg1;
  int32_t* first = ga.meta + G.meta_off + (side ? (2 * ga.b1 + 1) : 0);
  int32_t* pre = first + nb;
  const int tid = threadIdx.x;
  const int64_t per = (nb + 255) / 256;
  const int64_t b0 = tid * per, b1e = min(b0 + per, nb);
  const int32_t th = side ? ga.tile_c : ga.tile_r;
  int32_t local = 0;
  for (int64_t b = b0; b < b1e; ++b) {
    const int32_t s0 = seg[b], s1 = seg[b + 1];
    first[b] = s0 / th;
    local += s1 > s0 ? (s1 - 1) / th - s0 / th + 1 : 0;
  }
  part[tid] = local;
  __syncthreads();
  if (tid == 0) {
    int32_t run = 0;
    for (int q = 0; q < 256; ++q) { const int32_t v = part[q]; part[q] = run; run += v; }
    pre[nb] = run;
  }
  __syncthreads();
  int32_t run = part[tid];
  for (int64_t b = b0; b < b1e; ++b) {
    pre[b] = run;
    const int32_t s0 = seg[b], s1 = seg[b + 1];
    run += s1 > s0 ? (s1 - 1) / th - s0 / th + 1 : 0;
  }
}

// Bins of one tile's parked products P (rows x cols, row stride prow): the
// (sample i, sample j) pairs meeting rows [t0, t0 + rows) ∩ [0, n1) and columns
// [s0, s0 + cols) ∩ [0, n2); one wave per bin, lanes over rows, each lane
// summing its rows' columns in order, then a fixed butterfly.  Bin (i, j) of
// tile (m, n) goes to slot (pre1[i] + m - first1[i], pre2[j] + n - first2[j])
// of the group's region (clamped to it).
__device__ __forceinline__ void grouped_bins(const float* P, int prow, int rows, int cols, int64_t t0, int64_t s0,
                                             int64_t n1, int64_t n2, int64_t m, int64_t n, const GroupDev& G,
                                             const GroupedArgs& ga) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t last_r = min(t0 + rows, n1) - 1, last_c = min(s0 + cols, n2) - 1;
  if (last_r < t0 || last_c < s0) return;  // no live rows on a side: no bins
  const int64_t i_lo = sample_of(G.seg1, ga.b1, t0), i_hi = sample_of(G.seg1, ga.b1, last_r);
  const int64_t j_lo = sample_of(G.seg2, ga.b2, s0), j_hi = sample_of(G.seg2, ga.b2, last_c);
  const int64_t nj = j_hi - j_lo + 1, nbins = (i_hi - i_lo + 1) * nj;
  const int32_t* first1 = ga.meta + G.meta_off;
  const int32_t* pre1 = first1 + ga.b1;
  const int32_t* first2 = pre1 + ga.b1 + 1;
  const int32_t* pre2 = first2 + ga.b2;
  for (int64_t bin = wave; bin < nbins; bin += (int64_t)(blockDim.x / kWave)) {
    const int64_t i = i_lo + bin / nj, j = j_lo + bin % nj;
    const int64_t r0 = max((int64_t)G.seg1[i], t0) - t0, r1 = min((int64_t)G.seg1[i + 1], t0 + rows) - t0;
    const int64_t c0 = max((int64_t)G.seg2[j], s0) - s0, c1 = min((int64_t)G.seg2[j + 1], s0 + cols) - s0;
    if (r1 <= r0 || c1 <= c0) continue;  // an empty sample: it owns no slot
    float v = 0.f;
    for (int64_t t = r0 + lane; t < r1; t += kWave)
      for (int64_t c = c0; c < c1; ++c) v += P[t * prow + c];
    v = wave_sum(v);
    const int64_t row = pre1[i] + m - first1[i], col = pre2[j] + n - first2[j];
    if (lane == 0 && row >= 0 && row < G.tiles_r + ga.b1 && col >= 0 && col < G.part_ld)
      ga.partial[G.part_off + row * G.part_ld + col] = v;
  }
}

template <int DT>
__global__ __launch_bounds__(kThreads, 2) void ghost_grouped_tiles(GroupedArgs ga) {
  __shared__ __attribute__((aligned(16))) char smem[2 * kStageBytes];
  static_assert(kBM * kPRow * 4 <= 2 * kStageBytes, "product tile must fit the stage buffers");

  const int64_t logical = xcd_remap(blockIdx.x, gridDim.x);
  int e = 0;
  while (e + 1 < ga.n_groups && ga.grp[e + 1].tile0 <= logical) ++e;
  const GroupDev& G = ga.grp[e];
  const int64_t local = logical - G.tile0;
  const int64_t per_group = (int64_t)kGroup * G.tiles_c;
  const int64_t grp = local / per_group;
  const int64_t first_r = grp * kGroup;
  const int64_t gsize = min(G.tiles_r - first_r, (int64_t)kGroup);
  const int64_t in_group = local - grp * per_group;
  const int64_t m = first_r + in_group % gsize;
  const int64_t n = in_group / gsize;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lr = tid >> 3;
  const int64_t t0 = m * kBM, s0 = n * kBN;
  // Rows at or past seg[B] belong to no sample (and may have no row_index
  // entry): treat them as absent; a tile wholly past them has nothing to do.
  const int64_t n1 = min(G.rows1, (int64_t)G.seg1[ga.b1]), n2 = min(G.rows2, (int64_t)G.seg2[ga.b2]);
  if (t0 >= n1 || s0 >= n2) return;
  const char* a1[4];
  const char* g1[4];
  const char* a2[4];
  const char* g2[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int64_t t = t0 + lr + 32 * p, s = s0 + lr + 32 * p;
    const bool v1 = t < n1, v2 = s < n2;
    const int64_t r1 = v1 ? (G.idx1 ? (int64_t)G.idx1[t] : t) : 0;
    const int64_t r2 = v2 ? (G.idx2 ? (int64_t)G.idx2[s] : s) : 0;
    a1[p] = v1 ? G.a1 + r1 * G.a1_ts : nullptr;
    g1[p] = v1 ? G.g1 + r1 * G.g1_ts : nullptr;
    a2[p] = v2 ? G.a2 + r2 * G.a2_ts : nullptr;
    g2[p] = v2 ? G.g2 + r2 * G.g2_ts : nullptr;
  }

  f32x16 ka[2][2], kg[2][2];
  gram_tile<DT>(smem, a1, a2, G.kbytes_a, ka, tid, lane, wm, wn);
  gram_tile<DT>(smem, g1, g2, G.kbytes_g, kg, tid, lane, wm, wn);

  // Park (K_a + bias) * K_g in LDS (rows past an end are zero rows: K_g = 0).
  float* P = (float*)smem;
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 64 * wm + 32 * x + acc_row(r, lane), col = 64 * wn + 32 * y + acc_col(lane);
        P[row * kPRow + col] = (ka[x][y][r] + G.bias) * kg[x][y][r];
      }
  __syncthreads();

  grouped_bins(P, kPRow, kBM, kBN, t0, s0, n1, n2, m, n, G, ga);
}

// out[i, j] (+)= sum over groups of the (span1 x span2) slot block, in a fixed order.
__global__ void grouped_reduce(GroupedArgs ga, float* __restrict__ out, int64_t ld_out, int accumulate) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= ga.b1 * ga.b2) return;
  const int64_t i = idx / ga.b2, j = idx - i * ga.b2;
  float v = 0.f;
  for (int e = 0; e < ga.n_groups; ++e) {
    const GroupDev& G = ga.grp[e];
    const int32_t* pre1 = ga.meta + G.meta_off + ga.b1;
    const int32_t* pre2 = pre1 + ga.b1 + 1 + ga.b2;
    const float* base = ga.partial + G.part_off;
    const int64_t r_end = min((int64_t)pre1[i + 1], G.tiles_r + ga.b1);
    const int64_t c_end = min((int64_t)pre2[j + 1], G.part_ld);
    for (int64_t r = max((int64_t)pre1[i], (int64_t)0); r < r_end; ++r)
      for (int64_t c = max((int64_t)pre2[j], (int64_t)0); c < c_end; ++c) v += base[r * G.part_ld + c];
  }
  float* o = out + i * ld_out + j;
  *o = accumulate ? *o + v : v;
}

// ---------------------------------------------------------------------------
// 256 x 128 tile engine (the gfx950 path).
//
// Both Gram products of a tile -- K_a over the activation width, then K_g over
// the gradient width -- run as ONE stream of 128-byte K stages (one cache line
// of every operand row) through a ring of three LDS stages (48 KB each, two in
// flight).  Operand rows go HBM -> LDS untouched by buffer loads with the
// LDS-direct bit (16 bytes per lane); rows past a sample's end, and chunks past
// the width, read as zero (offset past the buffer range).  Eight waves, two per
// SIMD, each own a 64 x 64 block of both products (2 x 2 MFMA blocks of
// 32 x 32, 128 accumulators), so one wave of a SIMD keeps the MFMA pipe busy
// while the other waits at a barrier, for a load or on LDS.  As in the dW
// kernel, the loads are issued as inline assembly with explicit vmcnt waits,
// interleaved with the MFMAs (a quarter stage of loads per quarter stage of
// MFMAs), and the last quarter of each stage is multiplied after the barrier
// that opens the next.
// ---------------------------------------------------------------------------
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

namespace v2 {
constexpr int kBM = 256;                 // side-1 rows per tile
constexpr int kBN = 128;                 // side-2 rows per tile
constexpr int kRows = kBM + kBN;         // LDS rows per stage
constexpr int kSB = 128;                 // bytes of K per row and stage: one cache line, four 32-byte slices
constexpr int kStage = kRows * kSB;      // 48 KB
constexpr int kNBuf = 3;                 // ring: two stages in flight
constexpr uint32_t kOob = 0x80000000u;
constexpr int kPRow = kBN + 1;           // parked fp32 product row (grouped epilogue)
constexpr int kRing = kNBuf * kStage;
constexpr int kPark = kBM * kPRow * 4;
constexpr int kSmem = kPark > kRing ? kPark : kRing;
static_assert(kSmem <= 160 * 1024, "LDS");
// 16-byte chunk c of LDS row r sits in slot c ^ (r & 7): the 8 lanes one LDS
// cycle serves (8 consecutive rows, one chunk) read 8 distinct bank groups.
}  // namespace v2

// ---------------------------------------------------------------------------
// The engine's per-wave layout: wave w owns the 64 x 64 block at side-1 rows
// 64 (w / 2) and side-2 rows 64 (w % 2); a 32-byte K slice costs it 4 fragment
// reads per 4 MFMAs.  Each wave issues 6 DMA instructions per stage (wave w
// loads tile rows 48w .. 48w+47).
// ---------------------------------------------------------------------------
namespace v3 {
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kDma = v2::kRows * (v2::kSB / 16) / (kWave * kWaves);  // 6 per wave and stage
static_assert(kDma == 6, "the vmcnt wait and the quarter split assume 6 DMA instructions per stage");
// instructions [kLo[q], kLo[q + 1]) of a stage go out in quarter q
__device__ __forceinline__ constexpr int lo(int q) { return q == 0 ? 0 : q == 1 ? 2 : q == 2 ? 3 : q == 3 ? 5 : 6; }
}  // namespace v3

struct TileSrc8 {
  u32x4 ra1, rg1, ra2, rg2;
  uint32_t roff_a[v3::kDma], roff_g[v3::kDma];
  int64_t kbytes_a, kbytes_g;
};

__device__ __forceinline__ int dma_row8(int w, int j, int lane) { return 8 * (v3::kDma * w + j) + (lane >> 3); }

struct DmaState8 {
  u32x4 ra1, rg1, ra2, rg2;
  uint32_t roa[v3::kDma], rog[v3::kDma];
  uint32_t cbyte, lds0;
  int uwave, na, nst;
  int64_t kba, kbg;
};

// Instructions [j0, j1) of stage st's loads for this wave (6 per wave and
// stage).  Instruction j of wave w loads tile rows 8*(6w + j) .. +7 (rows <
// 256 are side 1); lane l -> row 8*(6w+j) + l/8, slot l%8 holding logical
// chunk (l%8) ^ (l/8), which is cbyte / 16.  A select between the four
// descriptors would be turned into a pointer select over stack copies (a
// scratch load, and the compiler then waits for every outstanding load before
// using it), so the descriptor is picked by mask arithmetic.
__device__ __forceinline__ void dma_part8(const DmaState8& D, int st, int j0, int j1) {
  const bool act = st < D.na;
  const uint32_t koff = (uint32_t)(act ? st : st - D.na) * v2::kSB;
  const int64_t kb = act ? D.kba : D.kbg;
  const bool kin = st < D.nst && (int64_t)(koff + D.cbyte) < kb;
  const uint32_t base = D.lds0 + (uint32_t)((st % v2::kNBuf) * v2::kStage + v3::kDma * D.uwave * 8 * v2::kSB);
#pragma unroll
  for (int j = j0; j < j1; ++j) {
    const bool side1 = v3::kDma * D.uwave + j < v2::kBM / 8;  // uniform
    const uint32_t m = act ? 0xffffffffu : 0u;
    const uint32_t roff = (D.roa[j] & m) | (D.rog[j] & ~m);
    const uint32_t ms = side1 ? 0xffffffffu : 0u;
    u32x4 rs;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      rs[c] = (((D.ra1[c] & m) | (D.rg1[c] & ~m)) & ms) | (((D.ra2[c] & m) | (D.rg2[c] & ~m)) & ~ms);
    dma16(rs, base + (uint32_t)(j * 8 * v2::kSB), (kin && roff != v2::kOob) ? roff + koff + D.cbyte : v2::kOob);
  }
}

// One slice: the 4 MFMAs of (ua, ub) into acc, with rd the 4 fragment reads
// of the slice two ahead (stage base sb, chunk offset coff) into (na, nb), and
// with qd >= 0 quarter qd's share of stage dst's loads (after MFMAs 1 and 3).
template <int DT>
__device__ __forceinline__ void ghost_quarter8(f32x16 (&acc)[2][2], const u32x4 (&ua)[2], const u32x4 (&ub)[2],
                                               bool rd, const lds_char* sb, int coff, int wm, int wn,
                                               u32x4 (&na)[2], u32x4 (&nb)[2], const DmaState8& D, int qd, int dst) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (rd) {
      if (i < 2) na[i] = *(const u32x4*)(sb + (64 * wm + 32 * i) * v2::kSB + coff);
      else nb[i - 2] = *(const u32x4*)(sb + (v2::kBM + 64 * wn + 32 * (i - 2)) * v2::kSB + coff);
    }
    Mfma32<DT>::mma(acc[i >> 1][i & 1], ua[i >> 1], ub[i & 1]);
    if (qd >= 0 && i == 1) dma_part8(D, dst, v3::lo(qd), v3::lo(qd) + 1);
    if (qd >= 0 && i == 3 && v3::lo(qd + 1) - v3::lo(qd) > 1) dma_part8(D, dst, v3::lo(qd) + 1, v3::lo(qd + 1));
    __builtin_amdgcn_sched_barrier(0);
  }
}

__device__ __forceinline__ void ghost_stage_sync8() {
  static_assert(v2::kNBuf == 3, "vmcnt below is one stage of 6 instructions");
  asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("s_barrier" ::: "memory");
}

// Runs the tile's K stages; returns with every wave done reading the ring
// (so the caller may reuse the LDS) and no load in flight.
// kHasA: the tile has activation stages (K > 0), multiplied into ka before
// the gradient stages into kg; otherwise every stage goes to kg and ka stays 0.
// Fragment offsets inside a stage: A fragment x = rows 64wm + 32x + l%32, B
// fragment y = rows 256 + 64wn + 32y + l%32; slice kk reads logical chunk
// 2kk + l/32, stored in slot (2kk + l/32) ^ (l%8).  Fragments are read two
// slices ahead of their MFMAs, so a read has a whole slice of MFMAs to come
// back while the DMA writes share the LDS.  A loop body starts right after a
// barrier (no read in flight, so the loop header needs no wait): it
// multiplies slices 2 and 3 of stage st and slices 0 and 1 of st + 1 while
// reading slices 0..3 of st + 1, loads stage st + 3 into the buffer stage st
// left (its reads all ended before that barrier), then waits for stage st + 2.
// Exactly the 6 instructions of the body's own loads follow the awaited
// stage's last one at every barrier.
template <int DT, bool kHasA>
__device__ __forceinline__ void ghost_tile_engine8(const TileSrc8& S, char* smem, f32x16 (&ka)[2][2],
                                                   f32x16 (&kg)[2][2]) {
  lds_char* const L = (lds_char*)smem;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  DmaState8 D;
  D.uwave = __builtin_amdgcn_readfirstlane(wave);
  D.na = (int)((S.kbytes_a + v2::kSB - 1) / v2::kSB);
  D.nst = D.na + (int)((S.kbytes_g + v2::kSB - 1) / v2::kSB);
  D.ra1 = uniform4(S.ra1);
  D.rg1 = uniform4(S.rg1);
  D.ra2 = uniform4(S.ra2);
  D.rg2 = uniform4(S.rg2);
  D.kba = S.kbytes_a;
  D.kbg = S.kbytes_g;
  D.lds0 = (uint32_t)(uintptr_t)L;
  D.cbyte = 16u * (uint32_t)((lane & 7) ^ (lane >> 3));
#pragma unroll
  for (int j = 0; j < v3::kDma; ++j) {
    D.roa[j] = S.roff_a[j];
    D.rog[j] = S.roff_g[j];
  }
  const int na = D.na, nst = D.nst;

  const int lrow = lane & 31, hh = lane >> 5;
  const int c0 = lrow * v2::kSB + (((0 + hh) ^ (lane & 7)) << 4), c1 = lrow * v2::kSB + (((2 + hh) ^ (lane & 7)) << 4);
  const int c2 = lrow * v2::kSB + (((4 + hh) ^ (lane & 7)) << 4), c3 = lrow * v2::kSB + (((6 + hh) ^ (lane & 7)) << 4);
  u32x4 fa[4][2], fb[4][2];

#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      ka[x][y] = f32x16{};
      kg[x][y] = f32x16{};
    }

#pragma unroll
  for (int s0 = 0; s0 < v2::kNBuf - 1; ++s0) dma_part8(D, s0, 0, v3::kDma);
  ghost_stage_sync8();
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const int co = kk == 0 ? c0 : c1;
#pragma unroll
    for (int x = 0; x < 2; ++x) fa[kk][x] = *(const u32x4*)(L + (64 * wm + 32 * x) * v2::kSB + co);
#pragma unroll
    for (int y = 0; y < 2; ++y) fb[kk][y] = *(const u32x4*)(L + (v2::kBM + 64 * wn + 32 * y) * v2::kSB + co);
  }
  dma_part8(D, v2::kNBuf - 1, v3::lo(0), v3::lo(2));
  {
    f32x16(&acc0)[2][2] = kHasA ? ka : kg;
    ghost_quarter8<DT>(acc0, fa[0], fb[0], true, L, c2, wm, wn, fa[2], fb[2], D, 2, v2::kNBuf - 1);
    ghost_quarter8<DT>(acc0, fa[1], fb[1], true, L, c3, wm, wn, fa[3], fb[3], D, 3, v2::kNBuf - 1);
  }
  ghost_stage_sync8();

#define DA_GHOST_BODY8(A1, A2)                                                                        \
  {                                                                                                   \
    const lds_char* nxt = L + ((st + 1) % v2::kNBuf) * v2::kStage;                                    \
    ghost_quarter8<DT>(A1, fa[2], fb[2], true, nxt, c0, wm, wn, fa[0], fb[0], D, 0, st + 3);          \
    ghost_quarter8<DT>(A1, fa[3], fb[3], true, nxt, c1, wm, wn, fa[1], fb[1], D, 1, st + 3);          \
    ghost_quarter8<DT>(A2, fa[0], fb[0], true, nxt, c2, wm, wn, fa[2], fb[2], D, 2, st + 3);          \
    ghost_quarter8<DT>(A2, fa[1], fb[1], true, nxt, c3, wm, wn, fa[3], fb[3], D, 3, st + 3);          \
    ghost_stage_sync8();                                                                              \
  }
  if constexpr (kHasA) {
    for (int st = 0; st + 1 < na; ++st) DA_GHOST_BODY8(ka, ka)
    {
      const int st = na - 1;
      DA_GHOST_BODY8(ka, kg)
    }
  }
  for (int st = kHasA ? na : 0; st + 1 < nst; ++st) DA_GHOST_BODY8(kg, kg)
#undef DA_GHOST_BODY8
  ghost_quarter8<DT>(kg, fa[2], fb[2], false, L, c0, wm, wn, fa[0], fb[0], D, -1, 0);
  ghost_quarter8<DT>(kg, fa[3], fb[3], false, L, c1, wm, wn, fa[1], fb[1], D, -1, 0);
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Dense / per-sample segmented mode: a 256 x 128 tile inside one sample pair on
// the 8-wave engine.  Its fp32 partial (the 8 waves' shares summed in a fixed
// order) goes to the pair's slot; ghost_gram_reduce adds a pair's tiles.
template <int DT>
__global__ __launch_bounds__(v3::kThreads, 1) void ghost_gram_tiles_v3(GhostArgs g) {
  __shared__ __attribute__((aligned(1024))) char smem[v2::kRing];
  __shared__ float red[v3::kWaves];
  // Each XCD runs 32 tiles at once; grouping 4 row tiles (4 MB of operand rows
  // each at d = 4096) with 8 column tiles (2 MB each) minimises the rows its L2
  // streams per block of concurrent tiles (measured: groups of 4 rows beat 8,
  // 16 and 32 by 6%, 17% and 40% on the 256 x 64 pair, T = 512 workload).
  constexpr int64_t kRowGroup = 4;
  const int64_t logical = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t per_group = kRowGroup * g.n_c;
  const int64_t group = logical / per_group;
  const int64_t first_r = group * kRowGroup;
  const int64_t gsize = min(g.n_r - first_r, kRowGroup);
  const int64_t in_group = logical - group * per_group;
  const int64_t R = first_r + in_group % gsize;
  const int64_t C = in_group / gsize;
  const int64_t i = R / g.tiles_r, tt = R % g.tiles_r;
  const int64_t j = pair_col_sample(g, i, C), ss = C % g.tiles_c;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  const int64_t len1 = seg_len(g.s1, i), len2 = seg_len(g.s2, j);
  const int64_t t0 = tt * v2::kBM, s0 = ss * v2::kBN;
  float* dst = g.partial + (pair_slot(g, i, j) * g.tiles_r + tt) * g.tiles_c + ss;
  if (t0 >= len1 || s0 >= len2) {
    if (tid == 0) *dst = 0.f;
    return;
  }
  const int64_t st1 = seg_start(g.s1, i), st2 = seg_start(g.s2, j);
  // Buffer bases: the sample's first row (dense) or the factor (segmented);
  // the host checked that every offset stays below 2^31.
  const char* ba1 = g.s1.seg ? g.s1.act : g.s1.act + i * g.s1.act_bstride;
  const char* bg1 = g.s1.seg ? g.s1.grad : g.s1.grad + i * g.s1.grad_bstride;
  const char* ba2 = g.s2.seg ? g.s2.act : g.s2.act + j * g.s2.act_bstride;
  const char* bg2 = g.s2.seg ? g.s2.grad : g.s2.grad + j * g.s2.grad_bstride;
  TileSrc8 S;
  S.ra1 = make_rsrc(ba1, 0x7fffffffu);
  S.rg1 = make_rsrc(bg1, 0x7fffffffu);
  S.ra2 = make_rsrc(ba2, 0x7fffffffu);
  S.rg2 = make_rsrc(bg2, 0x7fffffffu);
  S.kbytes_a = g.kbytes_a;
  S.kbytes_g = g.kbytes_g;
#pragma unroll
  for (int q = 0; q < v3::kDma; ++q) {
    const int row = dma_row8(wave, q, lane);
    const bool side1 = row < v2::kBM;
    const SideDev& sd = side1 ? g.s1 : g.s2;
    const int64_t t = side1 ? t0 + row : s0 + row - v2::kBM;
    const int64_t len = side1 ? len1 : len2;
    const int64_t start = side1 ? st1 : st2;
    if (t < len) {
      const int64_t r = sd.seg ? (sd.idx ? (int64_t)sd.idx[start + t] : start + t) : t;
      S.roff_a[q] = (uint32_t)(r * sd.act_tstride);
      S.roff_g[q] = (uint32_t)(r * sd.grad_tstride);
    } else {
      S.roff_a[q] = v2::kOob;
      S.roff_g[q] = v2::kOob;
    }
  }
  f32x16 ka[2][2], kg[2][2];
  ghost_tile_engine8<DT, true>(S, smem, ka, kg);
  float s = 0.f;
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += (ka[x][y][r] + g.bias) * kg[x][y][r];
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (tid == 0) *dst = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
}

// Grouped (MoE) mode: tiles over each group's packed rows, the tile's
// products parked in LDS and binned by sample pair.
template <int DT>
__global__ __launch_bounds__(v3::kThreads, 1) void ghost_grouped_tiles_v3(GroupedArgs ga) {
  __shared__ __attribute__((aligned(1024))) char smem[v2::kSmem];
  // Tiles go to the XCDs round-robin in launch order (no XCD remap): the host
  // orders the groups longest reduction first, so every XCD gets the same mix
  // of tile lengths, longest first.  A contiguous range per XCD would hand the
  // long groups' tiles to some XCDs and the short ones to the rest.
  const int64_t logical = blockIdx.x;
  int e = 0;
  while (e + 1 < ga.n_groups && ga.grp[e + 1].tile0 <= logical) ++e;
  const GroupDev& G = ga.grp[e];
  const int64_t local = logical - G.tile0;
  constexpr int64_t kRowGroup = 4;
  const int64_t per_group = kRowGroup * G.tiles_c;
  const int64_t grp = local / per_group;
  const int64_t first_r = grp * kRowGroup;
  const int64_t gsize = min(G.tiles_r - first_r, kRowGroup);
  const int64_t in_group = local - grp * per_group;
  const int64_t m = first_r + in_group % gsize;
  const int64_t n = in_group / gsize;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t t0 = m * v2::kBM, s0 = n * v2::kBN;
  // Rows at or past seg[B] belong to no sample (and may have no row_index
  // entry); a tile wholly past the packed rows of a side owns no bin.
  const int64_t n1 = min(G.rows1, (int64_t)G.seg1[ga.b1]), n2 = min(G.rows2, (int64_t)G.seg2[ga.b2]);
  if (t0 >= n1 || s0 >= n2) return;
  TileSrc8 S;
  S.ra1 = make_rsrc(G.a1, 0x7fffffffu);
  S.rg1 = make_rsrc(G.g1, 0x7fffffffu);
  S.ra2 = make_rsrc(G.a2, 0x7fffffffu);
  S.rg2 = make_rsrc(G.g2, 0x7fffffffu);
  S.kbytes_a = G.kbytes_a;
  S.kbytes_g = G.kbytes_g;
#pragma unroll
  for (int q = 0; q < v3::kDma; ++q) {
    const int row = dma_row8(wave, q, lane);
    const bool side1 = row < v2::kBM;
    const int64_t t = side1 ? t0 + row : s0 + row - v2::kBM;
    const bool live = t < (side1 ? n1 : n2);
    const int32_t* idx = side1 ? G.idx1 : G.idx2;
    const int64_t r = live ? (idx ? (int64_t)idx[t] : t) : 0;
    S.roff_a[q] = live ? (uint32_t)(r * (side1 ? G.a1_ts : G.a2_ts)) : v2::kOob;
    S.roff_g[q] = live ? (uint32_t)(r * (side1 ? G.g1_ts : G.g2_ts)) : v2::kOob;
  }
  f32x16 ka[2][2], kg[2][2];
  ghost_tile_engine8<DT, true>(S, smem, ka, kg);
  float* P = (float*)smem;
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 64 * wm + 32 * x + acc_row(r, lane), col = 64 * wn + 32 * y + acc_col(lane);
        P[row * v2::kPRow + col] = (ka[x][y][r] + G.bias) * kg[x][y][r];
      }
  __syncthreads();
  grouped_bins(P, v2::kPRow, v2::kBM, v2::kBN, t0, s0, n1, n2, m, n, G, ga);
}


// ---------------------------------------------------------------------------
// Per-token cross-gram on the 256 x 128 engine: K[i, t, j] keeps side 1's
// token t and sums side 2 out (the token decomposition of the score).
//
//   factorized side 2:  K[i,t,j] = sum_s (a1_it . a2_js + bias)(g1_it . g2_js)
//   dense side 2:       K[i,t,j] = sum_o (a1_it . M2_j[o,:] + mb_j[o]) g1_it[o]
//
// The factorized form is the ghost tile with a row epilogue; the dense form
// runs the engine's second product alone over a1 rows against M2_j's rows (the
// output channels o play side 2's tokens) and multiplies by g1 in the
// epilogue.  Each tile parks its (256 x 128) products in LDS and sums every
// row over its 128 columns; a second kernel adds the column tiles in order.
// ---------------------------------------------------------------------------
struct PerTokArgs {
  SideDev s1, s2;                  // dense form: s2.grad = M2 rows (tokens = D)
  int64_t kbytes_a, kbytes_g;
  int64_t tiles_r, tiles_c, n_r, n_c;
  float bias;                      // factorized: the implicit ones column
  const float* m2bias;             // dense: (B2, D) fp32 bias-column gradients, or nullptr
  int64_t m2bias_ld;               // floats between samples
  int64_t tpad;                    // tiles_r * 256
  float* partial;                  // [B1][B2][tpad][tiles_c]
};

template <int DT, bool kDense>
__global__ __launch_bounds__(v3::kThreads, 1) void ghost_per_token_v3(PerTokArgs g) {
  __shared__ __attribute__((aligned(1024))) char smem[v2::kSmem];
  constexpr int64_t kRowGroup = 4;
  const int64_t logical = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t per_group = kRowGroup * g.n_c;
  const int64_t group = logical / per_group;
  const int64_t first_r = group * kRowGroup;
  const int64_t gsize = min(g.n_r - first_r, kRowGroup);
  const int64_t in_group = logical - group * per_group;
  const int64_t R = first_r + in_group % gsize;
  const int64_t C = in_group / gsize;
  const int64_t i = R / g.tiles_r, tt = R % g.tiles_r;
  const int64_t j = C / g.tiles_c, ss = C % g.tiles_c;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t len1 = g.s1.tokens, len2 = g.s2.tokens;
  const int64_t t0 = tt * v2::kBM, s0 = ss * v2::kBN;
  if (t0 >= len1) return;  // uniform: no row of this tile is read back
  TileSrc8 S;
  S.ra1 = make_rsrc(g.s1.act + i * g.s1.act_bstride, 0x7fffffffu);
  S.rg1 = make_rsrc((kDense ? g.s1.act : g.s1.grad) + i * (kDense ? g.s1.act_bstride : g.s1.grad_bstride),
                    0x7fffffffu);
  S.ra2 = make_rsrc(g.s2.grad + j * g.s2.grad_bstride, 0x7fffffffu);
  S.rg2 = make_rsrc(g.s2.grad + j * g.s2.grad_bstride, 0x7fffffffu);
  if (!kDense) S.ra2 = make_rsrc(g.s2.act + j * g.s2.act_bstride, 0x7fffffffu);
  S.kbytes_a = g.kbytes_a;
  S.kbytes_g = g.kbytes_g;
#pragma unroll
  for (int q = 0; q < v3::kDma; ++q) {
    const int row = dma_row8(wave, q, lane);
    const bool side1 = row < v2::kBM;
    const int64_t t = side1 ? t0 + row : s0 + row - v2::kBM;
    if (t < (side1 ? len1 : len2)) {
      // dense form: side 1 streams a1 rows and side 2 M2_j rows, both in the gradient loop
      const int64_t ts1 = kDense ? g.s1.act_tstride : g.s1.grad_tstride;
      S.roff_a[q] = (uint32_t)(t * (side1 ? g.s1.act_tstride : g.s2.act_tstride));
      S.roff_g[q] = (uint32_t)(t * (side1 ? ts1 : g.s2.grad_tstride));
    } else {
      S.roff_a[q] = v2::kOob;
      S.roff_g[q] = v2::kOob;
    }
  }
  f32x16 ka[2][2], kg[2][2];
  ghost_tile_engine8<DT, !kDense>(S, smem, ka, kg);
  float* P = (float*)smem;
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 64 * wm + 32 * x + acc_row(r, lane), col = 64 * wn + 32 * y + acc_col(lane);
        float v;
        if constexpr (kDense) {
          const int64_t t = t0 + row, o = s0 + col;
          const bool ok = t < len1 && o < len2;
          const float gv = ok ? Elem<DT>::load(g.s1.grad + i * g.s1.grad_bstride + t * g.s1.grad_tstride, o) : 0.f;
          const float mb = (ok && g.m2bias) ? g.m2bias[j * g.m2bias_ld + o] : 0.f;
          v = (kg[x][y][r] + mb) * gv;
        } else {
          v = (ka[x][y][r] + g.bias) * kg[x][y][r];
        }
        P[row * v2::kPRow + col] = v;
      }
  __syncthreads();
  // one thread per row: the row's 128 columns in order (zero past side 2's end)
  const int64_t t = t0 + tid;
  if (tid < v2::kBM && t < len1) {
    const float* pr = P + tid * v2::kPRow;
    float sum = 0.f;
    for (int c = 0; c < v2::kBN; ++c) sum += pr[c];
    g.partial[((i * g.s2.batch + j) * g.tpad + t) * g.tiles_c + ss] = sum;
  }
}

// out[i*ld_b1 + t*ld_t + j*ld_b2] (+)= sum over column tiles, in order.
__global__ void per_token_reduce(const float* __restrict__ partial, int64_t b1, int64_t len1, int64_t b2,
                                 int64_t tpad, int64_t tiles_c, float* __restrict__ out, int64_t ld_b1,
                                 int64_t ld_t, int64_t ld_b2, int accumulate) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= b1 * len1 * b2) return;
  const int64_t j = idx % b2, t = (idx / b2) % len1, i = idx / (b2 * len1);
  const float* p = partial + ((i * b2 + j) * tpad + t) * tiles_c;
  float s = 0.f;
  for (int64_t q = 0; q < tiles_c; ++q) s += p[q];
  float* o = out + i * ld_b1 + t * ld_t + j * ld_b2;
  *o = accumulate ? *o + s : s;
}

struct Plan {
  int64_t tiles_r, tiles_c, n_r, n_c, per_pair;
  size_t ws;
  bool v2;  // the 256 x 128 tile engine (dense sides whose offsets fit 31 bits, D > 0)
};

// The tile engine addresses a sample's rows with 32-bit buffer offsets.
bool fits_v2(const da_factor_side* s, int64_t K, int64_t D, int64_t es) {
  if (s->seg_offsets) return false;
  const int64_t ts = s->act_tstride > s->grad_tstride ? s->act_tstride : s->grad_tstride;
  const int64_t w = K > D ? K : D;
  return s->act_tstride >= 0 && s->grad_tstride >= 0 && (s->tokens * ts + w) * es < (1LL << 31) - (1LL << 20);
}

int validate_side(const da_factor_side* s, int64_t K, int64_t D, int dtype, const char* name) {
  if (!s) return set_error(DA_ERR_INVALID, "da_ghost_gram: %s is NULL", name);
  if (s->batch < 0 || s->tokens < 0)
    return set_error(DA_ERR_INVALID, "da_ghost_gram: %s has negative batch/tokens", name);
  if (s->batch == 0 || s->tokens == 0) return DA_OK;
  if (!s->act || !s->grad) return set_error(DA_ERR_INVALID, "da_ghost_gram: %s has NULL factor", name);
  const int64_t es = (int64_t)elem_bytes(dtype);
  if (((uintptr_t)s->act | (uintptr_t)s->grad) & 15)
    return set_error(DA_ERR_INVALID, "da_ghost_gram: %s factors must be 16-byte aligned", name);
  const int64_t strides[4] = {s->act_bstride, s->act_tstride, s->grad_bstride, s->grad_tstride};
  for (int q = 0; q < 4; ++q) {
    if (s->seg_offsets && (q == 0 || q == 2)) continue;  // batch strides unused when segmented
    if ((strides[q] * es) % 16)
      return set_error(DA_ERR_INVALID, "da_ghost_gram: %s strides must be multiples of 16 bytes", name);
  }
  (void)K;
  (void)D;
  return DA_OK;
}

int make_plan(const da_factor_side* s1, const da_factor_side* s2, int64_t K, int64_t D, int dtype,
              Plan* plan, bool diag = false) {
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "da_ghost_gram: bad dtype %d", dtype);
  if (K < 0 || D < 0) return set_error(DA_ERR_INVALID, "da_ghost_gram: negative width");
  const int64_t es = (int64_t)elem_bytes(dtype);
  if ((K * es) % 16 || (D * es) % 16)
    return set_error(DA_ERR_INVALID,
                     "da_ghost_gram: K=%lld and D=%lld must be multiples of %lld elements",
                     (long long)K, (long long)D, (long long)(16 / es));
  int rc = validate_side(s1, K, D, dtype, "s1");
  if (rc) return rc;
  rc = validate_side(s2, K, D, dtype, "s2");
  if (rc) return rc;
  if (s1->has_bias != s2->has_bias)
    return set_error(DA_ERR_INVALID, "da_ghost_gram: both sides must agree on has_bias");
  plan->v2 = fits_v2(s1, K, D, es) && fits_v2(s2, K, D, es) && D > 0 && K > 0;
  const int64_t bm = plan->v2 ? v2::kBM : kBM, bn = plan->v2 ? v2::kBN : kBN;
  plan->tiles_r = (s1->tokens + bm - 1) / bm;
  plan->tiles_c = (s2->tokens + bn - 1) / bn;
  if (diag && s1->batch != s2->batch)
    return set_error(DA_ERR_INVALID, "da_ghost_gram_diag: the two sides need one batch size (%lld vs %lld)",
                     (long long)s1->batch, (long long)s2->batch);
  plan->n_r = s1->batch * plan->tiles_r;
  plan->n_c = (diag ? 1 : s2->batch) * plan->tiles_c;
  plan->per_pair = plan->tiles_r * plan->tiles_c;
  plan->ws = (size_t)(s1->batch * (diag ? 1 : s2->batch) * plan->per_pair) * sizeof(float);
  return DA_OK;
}

SideDev to_dev(const da_factor_side* s, int64_t es) {
  SideDev d;
  d.act = (const char*)s->act;
  d.grad = (const char*)s->grad;
  d.batch = s->batch;
  d.tokens = s->tokens;
  d.act_bstride = s->act_bstride * es;
  d.act_tstride = s->act_tstride * es;
  d.grad_bstride = s->grad_bstride * es;
  d.grad_tstride = s->grad_tstride * es;
  d.seg = s->seg_offsets;
  d.idx = s->row_index;
  return d;
}


// Per-token plans.  Both forms need dense sides (one row range per sample)
// whose rows the 256 x 128 engine addresses with 32-bit offsets.
struct PerTokPlan {
  int64_t tiles_r, tiles_c, tpad;
  size_t ws;
};

int per_token_plan(const da_factor_side* s1, int64_t b2, int64_t len2, int64_t K, int64_t D, int dtype,
                   const char* who, PerTokPlan* p) {
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "%s: bad dtype %d", who, dtype);
  if (K < 0 || D < 0 || b2 < 0 || len2 < 0) return set_error(DA_ERR_INVALID, "%s: negative size", who);
  const int64_t es = (int64_t)elem_bytes(dtype);
  if ((K * es) % 16 || (D * es) % 16)
    return set_error(DA_ERR_INVALID, "%s: K=%lld and D=%lld must be multiples of %lld elements", who,
                     (long long)K, (long long)D, (long long)(16 / es));
  if (!s1) return set_error(DA_ERR_INVALID, "%s: s1 is NULL", who);
  p->tiles_r = (s1->tokens + v2::kBM - 1) / v2::kBM;
  p->tiles_c = (len2 + v2::kBN - 1) / v2::kBN;
  p->tpad = p->tiles_r * v2::kBM;
  p->ws = (size_t)(s1->batch * b2 * p->tpad * p->tiles_c) * sizeof(float);
  return DA_OK;
}

int per_token_launch(const PerTokArgs& g, bool dense, int dtype, int64_t len1, float* out, int64_t ld_b1,
                     int64_t ld_t, int64_t ld_b2, int accumulate, hipStream_t st, const char* who) {
  const int64_t tiles = g.n_r * g.n_c;
  if (tiles > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: problem too large", who);
#define DA_PT(DT)                                                                  \
  if (dense)                                                                       \
    ghost_per_token_v3<DT, true><<<(unsigned)tiles, v3::kThreads, 0, st>>>(g);     \
  else                                                                             \
    ghost_per_token_v3<DT, false><<<(unsigned)tiles, v3::kThreads, 0, st>>>(g);
  switch (dtype) {
    case DA_BF16: DA_PT(DA_BF16) break;
    case DA_F16: DA_PT(DA_F16) break;
    default: DA_PT(DA_F32) break;
  }
#undef DA_PT
  int rc = check_launch(who);
  if (rc) return rc;
  const int64_t n = g.s1.batch * len1 * g.s2.batch;
  per_token_reduce<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(g.partial, g.s1.batch, len1, g.s2.batch, g.tpad,
                                                                g.tiles_c, out, ld_b1, ld_t, ld_b2, accumulate);
  return check_launch(who);
}
}  // namespace
}  // namespace da

namespace da {
namespace {

struct GroupedPlan {
  size_t meta_ints, part_floats, ws;
  bool v2;         // all groups on the 256 x 128 engine
  int tile_r, tile_c;
};

// Layout of the grouped workspace for the groups [g0, g0 + n): int32 span
// tables first, then the partial regions, per group.
int grouped_plan(const da_factor_side* s1, const da_factor_side* s2, int n_groups, const int64_t* K,
                 const int64_t* D, int dtype, GroupedPlan* p) {
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: bad dtype %d", dtype);
  if (n_groups < 0 || (n_groups > 0 && (!s1 || !s2 || !K || !D)))
    return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: bad group list");
  const int64_t es = (int64_t)elem_bytes(dtype);
  p->meta_ints = 0;
  p->part_floats = 0;
  p->v2 = true;
  for (int e = 0; e < n_groups; ++e) {
    // 32-bit buffer offsets over every group's rows, and both loops non-empty
    const da_factor_side* sd[2] = {&s1[e], &s2[e]};
    for (int q = 0; q < 2; ++q) {
      const int64_t ts = sd[q]->act_tstride > sd[q]->grad_tstride ? sd[q]->act_tstride : sd[q]->grad_tstride;
      const int64_t w = K[e] > D[e] ? K[e] : D[e];
      if (sd[q]->tokens < 0 || ts < 0 || (sd[q]->tokens * ts + w) * es >= (1LL << 31) - (1LL << 20)) p->v2 = false;
    }
    if (D[e] <= 0 || K[e] <= 0) p->v2 = false;
  }
  p->tile_r = p->v2 ? v2::kBM : kBM;
  p->tile_c = p->v2 ? v2::kBN : kBN;
  if (n_groups == 0) { p->ws = 0; return DA_OK; }
  const int64_t b1 = s1[0].batch, b2 = s2[0].batch;
  for (int e = 0; e < n_groups; ++e) {
    if (K[e] < 0 || D[e] < 0) return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: group %d negative width", e);
    if ((K[e] * es) % 16 || (D[e] * es) % 16)
      return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: group %d widths must be multiples of %lld elements",
                       e, (long long)(16 / es));
    if (s1[e].has_bias != s2[e].has_bias)
      return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: group %d sides disagree on has_bias", e);
    const da_factor_side* sides[2] = {&s1[e], &s2[e]};
    for (int q = 0; q < 2; ++q) {
      const da_factor_side* sd = sides[q];
      if (sd->batch != (q ? b2 : b1))
        return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: group %d has a different batch", e);
      if (sd->tokens < 0) return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: negative row count");
      if (sd->batch > 0 && !sd->seg_offsets)
        return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: group %d needs seg_offsets", e);
      if (sd->tokens > 0) {
        if (!sd->act || !sd->grad)
          return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: group %d has a NULL factor", e);
        if (((uintptr_t)sd->act | (uintptr_t)sd->grad) & 15)
          return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: factors must be 16-byte aligned");
        if ((sd->act_tstride * es) % 16 || (sd->grad_tstride * es) % 16)
          return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: row strides must be multiples of 16 bytes");
      }
    }
    const int64_t tr = (s1[e].tokens + p->tile_r - 1) / p->tile_r, tc = (s2[e].tokens + p->tile_c - 1) / p->tile_c;
    p->meta_ints += (size_t)(2 * b1 + 1 + 2 * b2 + 1);
    p->part_floats += (size_t)((tr + b1) * (tc + b2));
  }
  p->ws = ((p->meta_ints * sizeof(int32_t) + 255) / 256) * 256 + p->part_floats * sizeof(float);
  return DA_OK;
}

// Both entry points: all (i, j) pairs into out[i * ld_out + j], or (diag) the
// pairs (i, i) into out[i * ld_out].
int run_ghost(const da_factor_side* s1, const da_factor_side* s2, int64_t K, int64_t D, int dtype, bool diag,
              float* out, int64_t ld_out, int accumulate, void* workspace, size_t workspace_bytes,
              hipStream_t st) {
  Plan plan;
  int rc = make_plan(s1, s2, K, D, dtype, &plan, diag);
  if (rc) return rc;
  const int64_t b1 = s1->batch, b2 = diag ? 1 : s2->batch;
  if (b1 == 0 || s2->batch == 0) return DA_OK;
  if (!out) return set_error(DA_ERR_INVALID, "da_ghost_gram: out is NULL");
  if (ld_out < b2)
    return set_error(DA_ERR_INVALID, diag ? "da_ghost_gram_diag: out_stride < 1" : "da_ghost_gram: ld_out < B2");
  if (s1->tokens == 0 || s2->tokens == 0) {
    return accumulate ? DA_OK : zero_f32_2d(out, b1, b2, ld_out, st);
  }
  if (!workspace || workspace_bytes < plan.ws)
    return set_error(DA_ERR_WORKSPACE, "da_ghost_gram: workspace needs %zu bytes, got %zu", plan.ws,
                     workspace_bytes);
  const int64_t es = (int64_t)elem_bytes(dtype);
  GhostArgs args;
  args.s1 = to_dev(s1, es);
  args.s2 = to_dev(s2, es);
  args.kbytes_a = K * es;
  args.kbytes_g = D * es;
  args.tiles_r = plan.tiles_r;
  args.tiles_c = plan.tiles_c;
  args.n_r = plan.n_r;
  args.n_c = plan.n_c;
  args.bias = s1->has_bias ? 1.f : 0.f;
  args.diag = diag ? 1 : 0;
  args.partial = (float*)workspace;
  const int64_t ntiles = plan.n_r * plan.n_c;
  if (ntiles > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "da_ghost_gram: too many tiles");
  dim3 grid((unsigned)ntiles);
  if (plan.v2) {
    switch (dtype) {
      case DA_BF16: ghost_gram_tiles_v3<DA_BF16><<<grid, v3::kThreads, 0, st>>>(args); break;
      case DA_F16: ghost_gram_tiles_v3<DA_F16><<<grid, v3::kThreads, 0, st>>>(args); break;
      default: ghost_gram_tiles_v3<DA_F32><<<grid, v3::kThreads, 0, st>>>(args); break;
    }
  } else {
    switch (dtype) {
      case DA_BF16: ghost_gram_tiles<DA_BF16><<<grid, kThreads, 0, st>>>(args); break;
      case DA_F16: ghost_gram_tiles<DA_F16><<<grid, kThreads, 0, st>>>(args); break;
      default: ghost_gram_tiles<DA_F32><<<grid, kThreads, 0, st>>>(args); break;
    }
  }
  rc = check_launch("da_ghost_gram(tiles)");
  if (rc) return rc;
  const int64_t pairs = b1 * b2;
  ghost_gram_reduce<<<(unsigned)((pairs + 255) / 256), 256, 0, st>>>(
      (const float*)workspace, b1, b2, plan.per_pair, out, ld_out, accumulate);
  return check_launch("da_ghost_gram(reduce)");
}

}  // namespace
}  // namespace da

extern "C" {

int da_ghost_gram_workspace(const da_factor_side* s1, const da_factor_side* s2, int64_t K,
                            int64_t D, int dtype, size_t* bytes) {
  da::Plan plan;
  int rc = da::make_plan(s1, s2, K, D, dtype, &plan);
  if (rc) return rc;
  if (!bytes) return da::set_error(DA_ERR_INVALID, "da_ghost_gram_workspace: bytes is NULL");
  *bytes = plan.ws;
  return DA_OK;
}

int da_ghost_gram(const da_factor_side* s1, const da_factor_side* s2, int64_t K, int64_t D,
                  int dtype, float* out, int64_t ld_out, int accumulate, void* workspace,
                  size_t workspace_bytes, void* stream) {
  return da::run_ghost(s1, s2, K, D, dtype, false, out, ld_out, accumulate, workspace, workspace_bytes,
                       (hipStream_t)stream);
}

int da_ghost_gram_diag_workspace(const da_factor_side* s1, const da_factor_side* s2, int64_t K, int64_t D,
                                 int dtype, size_t* bytes) {
  da::Plan plan;
  int rc = da::make_plan(s1, s2, K, D, dtype, &plan, true);
  if (rc) return rc;
  if (!bytes) return da::set_error(DA_ERR_INVALID, "da_ghost_gram_diag_workspace: bytes is NULL");
  *bytes = plan.ws;
  return DA_OK;
}

int da_ghost_gram_diag(const da_factor_side* s1, const da_factor_side* s2, int64_t K, int64_t D, int dtype,
                       float* out, int64_t out_stride, int accumulate, void* workspace, size_t workspace_bytes,
                       void* stream) {
  return da::run_ghost(s1, s2, K, D, dtype, true, out, out_stride, accumulate, workspace, workspace_bytes,
                       (hipStream_t)stream);
}

int da_ghost_gram_grouped_workspace(const da_factor_side* s1, const da_factor_side* s2, int n_groups,
                                    const int64_t* K, const int64_t* D, int dtype, size_t* bytes) {
  da::GroupedPlan plan;
  int rc = da::grouped_plan(s1, s2, n_groups, K, D, dtype, &plan);
  if (rc) return rc;
  if (!bytes) return da::set_error(DA_ERR_INVALID, "da_ghost_gram_grouped_workspace: bytes is NULL");
  *bytes = plan.ws;
  return DA_OK;
}

int da_ghost_gram_grouped(const da_factor_side* s1, const da_factor_side* s2, int n_groups,
                          const int64_t* K, const int64_t* D, int dtype, float* out, int64_t ld_out,
                          int accumulate, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace da;
  GroupedPlan plan;
  int rc = grouped_plan(s1, s2, n_groups, K, D, dtype, &plan);
  if (rc) return rc;
  if (n_groups == 0) return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: no groups");
  const int64_t b1 = s1[0].batch, b2 = s2[0].batch;
  if (b1 == 0 || b2 == 0) return DA_OK;
  if (!out) return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: out is NULL");
  if (ld_out < b2) return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: ld_out < B2");
  if (!workspace || workspace_bytes < plan.ws)
    return set_error(DA_ERR_WORKSPACE, "da_ghost_gram_grouped: workspace needs %zu bytes, got %zu", plan.ws,
                     workspace_bytes);
  hipStream_t st = (hipStream_t)stream;
  const int64_t es = (int64_t)elem_bytes(dtype);
  int32_t* meta = (int32_t*)workspace;
  float* part = (float*)((char*)workspace + ((plan.meta_ints * sizeof(int32_t) + 255) / 256) * 256);
  int64_t meta_off = 0, part_off = 0;
  bool first_launch = true;
  // Groups in order of decreasing reduction length K + D (stable): the tile
  // kernel deals tiles to the XCDs round-robin, so this is a longest-first
  // schedule on every XCD.  The partial sums land in the same per-pair bins
  // whatever the order.
  std::vector<int> order(n_groups);
  for (int e = 0; e < n_groups; ++e) order[e] = e;
  std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return K[x] + D[x] > K[y] + D[y]; });
  for (int g0 = 0; g0 < n_groups; g0 += kMaxGroups) {
    const int n = n_groups - g0 < kMaxGroups ? n_groups - g0 : kMaxGroups;
    GroupedArgs ga;
    ga.n_groups = 0;
    ga.tile_r = plan.tile_r;
    ga.tile_c = plan.tile_c;
    ga.b1 = b1;
    ga.b2 = b2;
    ga.partial = part;
    ga.meta = meta;
    int64_t tiles = 0;
    for (int q = 0; q < n; ++q) {
      const int e = order[g0 + q];
      const da_factor_side& x = s1[e];
      const da_factor_side& y = s2[e];
      const int64_t tr = (x.tokens + plan.tile_r - 1) / plan.tile_r, tc = (y.tokens + plan.tile_c - 1) / plan.tile_c;
      GroupDev& G = ga.grp[ga.n_groups++];
      G.a1 = (const char*)x.act;
      G.g1 = (const char*)x.grad;
      G.a2 = (const char*)y.act;
      G.g2 = (const char*)y.grad;
      G.seg1 = x.seg_offsets;
      G.seg2 = y.seg_offsets;
      G.idx1 = x.row_index;
      G.idx2 = y.row_index;
      G.rows1 = x.tokens;
      G.rows2 = y.tokens;
      G.a1_ts = x.act_tstride * es;
      G.g1_ts = x.grad_tstride * es;
      G.a2_ts = y.act_tstride * es;
      G.g2_ts = y.grad_tstride * es;
      G.tile0 = tiles;
      G.tiles_r = tr;
      G.tiles_c = tc;
      G.part_off = part_off;
      G.part_ld = tc + b2;
      G.meta_off = meta_off;
      G.kbytes_a = K[e] * es;
      G.kbytes_g = D[e] * es;
      G.bias = x.has_bias ? 1.f : 0.f;
      tiles += tr * tc;
      part_off += (tr + b1) * (tc + b2);
      meta_off += 2 * b1 + 1 + 2 * b2 + 1;
    }
    if (tiles > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "da_ghost_gram_grouped: too many tiles");
    grouped_spans<<<2 * ga.n_groups, 256, 0, st>>>(ga);
    rc = check_launch("da_ghost_gram_grouped(spans)");
    if (rc) return rc;
    if (tiles > 0) {
      if (plan.v2) {
        switch (dtype) {
          case DA_BF16: ghost_grouped_tiles_v3<DA_BF16><<<(unsigned)tiles, v3::kThreads, 0, st>>>(ga); break;
          case DA_F16: ghost_grouped_tiles_v3<DA_F16><<<(unsigned)tiles, v3::kThreads, 0, st>>>(ga); break;
          default: ghost_grouped_tiles_v3<DA_F32><<<(unsigned)tiles, v3::kThreads, 0, st>>>(ga); break;
        }
      } else {
        switch (dtype) {
          case DA_BF16: ghost_grouped_tiles<DA_BF16><<<(unsigned)tiles, kThreads, 0, st>>>(ga); break;
          case DA_F16: ghost_grouped_tiles<DA_F16><<<(unsigned)tiles, kThreads, 0, st>>>(ga); break;
          default: ghost_grouped_tiles<DA_F32><<<(unsigned)tiles, kThreads, 0, st>>>(ga); break;
        }
      }
      rc = check_launch("da_ghost_gram_grouped(tiles)");
      if (rc) return rc;
    }
    grouped_reduce<<<(unsigned)((b1 * b2 + 255) / 256), 256, 0, st>>>(ga, out, ld_out,
                                                                    (accumulate || !first_launch) ? 1 : 0);
    rc = check_launch("da_ghost_gram_grouped(reduce)");
    if (rc) return rc;
    first_launch = false;
  }
  return DA_OK;
}


int da_ghost_gram_per_token_workspace(const da_factor_side* s1, const da_factor_side* s2, int64_t K, int64_t D,
                                      int dtype, size_t* bytes) {
  using namespace da;
  if (!bytes || !s2) return set_error(DA_ERR_INVALID, "da_ghost_gram_per_token_workspace: NULL argument");
  PerTokPlan p;
  const int rc = per_token_plan(s1, s2->batch, s2->tokens, K, D, dtype, "da_ghost_gram_per_token", &p);
  if (rc) return rc;
  *bytes = p.ws;
  return DA_OK;
}

int da_ghost_gram_per_token(const da_factor_side* s1, const da_factor_side* s2, int64_t K, int64_t D, int dtype,
                            float* out, int64_t ld_b1, int64_t ld_t, int64_t ld_b2, int accumulate,
                            void* workspace, size_t workspace_bytes, void* stream) {
  using namespace da;
  const char* who = "da_ghost_gram_per_token";
  if (!s1 || !s2) return set_error(DA_ERR_INVALID, "%s: NULL side", who);
  PerTokPlan p;
  int rc = per_token_plan(s1, s2->batch, s2->tokens, K, D, dtype, who, &p);
  if (rc) return rc;
  rc = validate_side(s1, K, D, dtype, "s1");
  if (rc) return rc;
  rc = validate_side(s2, K, D, dtype, "s2");
  if (rc) return rc;
  if (s1->has_bias != s2->has_bias) return set_error(DA_ERR_INVALID, "%s: both sides must agree on has_bias", who);
  if (s1->batch == 0 || s1->tokens == 0 || s2->batch == 0) return DA_OK;
  if (!out) return set_error(DA_ERR_INVALID, "%s: out is NULL", who);
  const int64_t es = (int64_t)elem_bytes(dtype);
  if (s1->seg_offsets || s2->seg_offsets || !fits_v2(s1, K, D, es) || !fits_v2(s2, K, D, es) || D == 0 || K == 0)
    return set_error(DA_ERR_UNSUPPORTED,
                     "%s: needs dense sides with rows addressable by 32-bit offsets, K > 0 and D > 0", who);
  if (!workspace || workspace_bytes < p.ws)
    return set_error(DA_ERR_WORKSPACE, "%s: workspace needs %zu bytes", who, p.ws);
  PerTokArgs g;
  g.s1 = to_dev(s1, es);
  g.s2 = to_dev(s2, es);
  g.kbytes_a = K * es;
  g.kbytes_g = D * es;
  g.tiles_r = p.tiles_r;
  g.tiles_c = p.tiles_c;
  g.n_r = s1->batch * p.tiles_r;
  g.n_c = s2->batch * p.tiles_c;
  g.bias = s1->has_bias ? 1.f : 0.f;
  g.m2bias = nullptr;
  g.m2bias_ld = 0;
  g.tpad = p.tpad;
  g.partial = (float*)workspace;
  if (s2->tokens == 0) {  // nothing on side 2: the sums are zero
    g.tiles_c = 0;
    const int64_t n = s1->batch * s1->tokens * s2->batch;
    per_token_reduce<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(
        g.partial, s1->batch, s1->tokens, s2->batch, g.tpad, 0, out, ld_b1, ld_t, ld_b2, accumulate);
    return check_launch(who);
  }
  return per_token_launch(g, false, dtype, s1->tokens, out, ld_b1, ld_t, ld_b2, accumulate, (hipStream_t)stream, who);
}

int da_dense_per_token_workspace(const da_factor_side* s1, int64_t b2, int64_t K, int64_t D, int dtype,
                                 size_t* bytes) {
  using namespace da;
  if (!bytes) return set_error(DA_ERR_INVALID, "da_dense_per_token_workspace: bytes is NULL");
  PerTokPlan p;
  const int rc = per_token_plan(s1, b2, D, K, D, dtype, "da_dense_per_token", &p);
  if (rc) return rc;
  *bytes = p.ws;
  return DA_OK;
}

int da_dense_per_token(const da_factor_side* s1, const void* m2, int64_t b2, int64_t m2_bstride, int64_t m2_rstride,
                       const float* m2_bias, int64_t m2_bias_ld, int64_t K, int64_t D, int dtype, float* out,
                       int64_t ld_b1, int64_t ld_t, int64_t ld_b2, int accumulate, void* workspace,
                       size_t workspace_bytes, void* stream) {
  using namespace da;
  const char* who = "da_dense_per_token";
  PerTokPlan p;
  int rc = per_token_plan(s1, b2, D, K, D, dtype, who, &p);
  if (rc) return rc;
  rc = validate_side(s1, K, D, dtype, "s1");
  if (rc) return rc;
  if (s1->batch == 0 || s1->tokens == 0 || b2 == 0) return DA_OK;
  if (!out) return set_error(DA_ERR_INVALID, "%s: out is NULL", who);
  const int64_t es = (int64_t)elem_bytes(dtype);
  if (K == 0 || D == 0) return set_error(DA_ERR_UNSUPPORTED, "%s: needs K > 0 and D > 0", who);
  if (!m2 || ((uintptr_t)m2 & 15) || (m2_bstride * es) % 16 || (m2_rstride * es) % 16 || m2_rstride < K ||
      m2_bstride < 0)
    return set_error(DA_ERR_INVALID, "%s: m2 rows must be 16-byte aligned, row stride >= K", who);
  if (s1->has_bias && !m2_bias) return set_error(DA_ERR_INVALID, "%s: a bias column needs m2_bias", who);
  const int64_t lim = (1LL << 31) - (1LL << 20);
  if (s1->seg_offsets || !fits_v2(s1, K, D, es) || D * m2_rstride * es + K * es >= lim)
    return set_error(DA_ERR_UNSUPPORTED, "%s: needs a dense side 1 and rows addressable by 32-bit offsets", who);
  if (!workspace || workspace_bytes < p.ws)
    return set_error(DA_ERR_WORKSPACE, "%s: workspace needs %zu bytes", who, p.ws);
  PerTokArgs g;
  g.s1 = to_dev(s1, es);
  g.s2.act = (const char*)m2;
  g.s2.grad = (const char*)m2;
  g.s2.batch = b2;
  g.s2.tokens = D;  // M2_j's rows (output channels) take side 2's tokens
  g.s2.act_bstride = g.s2.grad_bstride = m2_bstride * es;
  g.s2.act_tstride = g.s2.grad_tstride = m2_rstride * es;
  g.s2.seg = nullptr;
  g.s2.idx = nullptr;
  g.kbytes_a = 0;  // one product: a1 rows against M2_j rows over K
  g.kbytes_g = K * es;
  g.tiles_r = p.tiles_r;
  g.tiles_c = p.tiles_c;
  g.n_r = s1->batch * p.tiles_r;
  g.n_c = b2 * p.tiles_c;
  g.bias = 0.f;
  g.m2bias = s1->has_bias ? m2_bias : nullptr;
  g.m2bias_ld = m2_bias_ld;
  g.tpad = p.tpad;
  g.partial = (float*)workspace;
  return per_token_launch(g, true, dtype, s1->tokens, out, ld_b1, ld_t, ld_b2, accumulate, (hipStream_t)stream, who);
}

}  // extern "C"
