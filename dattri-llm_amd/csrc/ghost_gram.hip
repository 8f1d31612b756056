// K1: fused ghost inner product (factorized cross-gram) on gfx950 MFMA.
//
//   out[i, j] = sum_{t < S1, s < S2} (a1[i,t,:] . a2[j,s,:]) * (g1[i,t,:] . g2[j,s,:])
//
// Follows the factorized route of cross_gram, dattri_llm/gradient/ops/dot.py:115-118,
// which forms K_a = A1 A2^T and K_g = G1 G2^T as two (B1*S1) x (B2*S2) matrices in
// HBM and then reduces their Hadamard product over each (S1 x S2) block.
//
// Here the same two products are computed as ONE tiled GEMM pair over the row
// spaces (B1*S1) x (B2*S2): a workgroup owns a 128 x 128 tile that lies inside a
// single (i, j) sample pair, runs the activation K-loop into one set of fp32
// MFMA accumulators and the gradient K-loop into a second set, and reduces
// (K_a + bias) * K_g in registers.  Only one fp32 per tile reaches HBM; a
// second tiny kernel sums the per-tile partials of each pair in a fixed order,
// so results are deterministic.
//
// Tile order: workgroups are remapped so each XCD owns a contiguous run of
// tiles, grouped 8 row-tiles wide, so the concurrently running tiles on one
// XCD share their operand row blocks through that XCD's L2.
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
  int64_t n_r, n_c;            // total row / column tiles
  float bias;
  float* partial;              // [B1][B2][tiles_r][tiles_c]
};

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
  const int64_t j = C / g.tiles_c, ss = C % g.tiles_c;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int64_t len1 = seg_len(g.s1, i), len2 = seg_len(g.s2, j);
  const int64_t t0 = tt * kBM, s0 = ss * kBN;
  float* dst = g.partial + ((i * g.s2.batch + j) * g.tiles_r + tt) * g.tiles_c + ss;
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

struct Plan {
  int64_t tiles_r, tiles_c, n_r, n_c, per_pair;
  size_t ws;
};

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
              Plan* plan) {
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
  plan->tiles_r = (s1->tokens + kBM - 1) / kBM;
  plan->tiles_c = (s2->tokens + kBN - 1) / kBN;
  plan->n_r = s1->batch * plan->tiles_r;
  plan->n_c = s2->batch * plan->tiles_c;
  plan->per_pair = plan->tiles_r * plan->tiles_c;
  plan->ws = (size_t)(s1->batch * s2->batch * plan->per_pair) * sizeof(float);
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
  using namespace da;
  Plan plan;
  int rc = make_plan(s1, s2, K, D, dtype, &plan);
  if (rc) return rc;
  const int64_t b1 = s1->batch, b2 = s2->batch;
  if (b1 == 0 || b2 == 0) return DA_OK;
  if (!out) return set_error(DA_ERR_INVALID, "da_ghost_gram: out is NULL");
  if (ld_out < b2) return set_error(DA_ERR_INVALID, "da_ghost_gram: ld_out < B2");
  hipStream_t st = (hipStream_t)stream;
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
  args.partial = (float*)workspace;
  const int64_t ntiles = plan.n_r * plan.n_c;
  if (ntiles > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "da_ghost_gram: too many tiles");
  dim3 grid((unsigned)ntiles);
  switch (dtype) {
    case DA_BF16: ghost_gram_tiles<DA_BF16><<<grid, kThreads, 0, st>>>(args); break;
    case DA_F16: ghost_gram_tiles<DA_F16><<<grid, kThreads, 0, st>>>(args); break;
    default: ghost_gram_tiles<DA_F32><<<grid, kThreads, 0, st>>>(args); break;
  }
  rc = check_launch("da_ghost_gram(tiles)");
  if (rc) return rc;
  const int64_t pairs = b1 * b2;
  ghost_gram_reduce<<<(unsigned)((pairs + 255) / 256), 256, 0, st>>>(
      (const float*)workspace, b1, b2, plan.per_pair, out, ld_out, accumulate);
  return check_launch("da_ghost_gram(reduce)");
}

}  // extern "C"
