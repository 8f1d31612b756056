// Channel norms (GroupNorm, InstanceNorm = GroupNorm with one group per
// channel) on gfx950: the per-sample weight gradient and the normalised input.
//
// x and g are (N, C, S) contiguous (S = the flattened spatial axes).  Group e
// of sample n is the contiguous block of C/G channels x S positions starting
// at (n*C + e*C/G)*S; x_hat = (x - mean) / sqrt(var + eps) over that block
// (biased variance), as dattri_llm/gradient/ops/norm.py:44-62 computes it.
// The layer's affine parameters are per channel, so the weight gradient of
// sample n is dgamma[c] = sum_s x_hat[n,c,s] g[n,c,s] and, with a bias,
// dbeta[c] = sum_s g[n,c,s] -- the token sum of the (N, S, C) factors that
// _augment_channel_norm (norm.py:120-141) builds, [dgamma | dbeta] per sample.
//
// Everything accumulates in fp32 in a fixed order: per thread a strided
// partial, then a wave butterfly and the waves in order.  HBM-bound: the
// statistics read x twice (sum, then squared deviations), the gradient pass
// reads x and g once.
#include "common.h"

namespace da {
namespace {

constexpr int kChThreads = 256;

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();  // red is free (a previous call's readers are done)
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// stats[2*(n*G + e)] = mean, stats[2*(n*G + e) + 1] = 1/sqrt(var + eps).
template <int DT>
__global__ __launch_bounds__(kChThreads) void chnorm_stats(const char* __restrict__ x, int64_t group_elems,
                                                           float eps, float* __restrict__ stats) {
  __shared__ float red[kChThreads / kWave];
  const int64_t blk = blockIdx.x;
  const char* xb = x + blk * group_elems * Elem<DT>::kBytes;
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < group_elems; i += kChThreads) s += Elem<DT>::load(xb, i);
  const float mean = block_sum(s, red) / (float)group_elems;
  float q = 0.f;
  for (int64_t i = threadIdx.x; i < group_elems; i += kChThreads) {
    const float dv = Elem<DT>::load(xb, i) - mean;
    q = fmaf(dv, dv, q);
  }
  const float var = block_sum(q, red) / (float)group_elems;
  if (threadIdx.x == 0) {
    stats[2 * blk] = mean;
    stats[2 * blk + 1] = 1.f / sqrtf(var + eps);
  }
}

// One block per (n, c): dgamma and (with a bias) dbeta of that channel.
template <int DT, int OT>
__global__ __launch_bounds__(kChThreads) void chnorm_grad(const char* __restrict__ x, const char* __restrict__ g,
                                                          int64_t C, int64_t S, int64_t per_group,
                                                          const float* __restrict__ stats, int has_bias,
                                                          char* __restrict__ out, int64_t out_ld) {
  __shared__ float red[kChThreads / kWave];
  const int64_t row = blockIdx.x;  // n * C + c
  const int64_t n = row / C, c = row - n * C;
  const int64_t grp = n * (C / per_group) + c / per_group;
  const float mean = stats[2 * grp], rstd = stats[2 * grp + 1];
  const int64_t off = row * S * Elem<DT>::kBytes;
  const char* xr = x + off;
  const char* gr = g + off;
  float dg = 0.f, db = 0.f;
  for (int64_t s = threadIdx.x; s < S; s += kChThreads) {
    const float gv = Elem<DT>::load(gr, s);
    dg = fmaf((Elem<DT>::load(xr, s) - mean) * rstd, gv, dg);
    db += gv;
  }
  dg = block_sum(dg, red);
  if (has_bias) db = block_sum(db, red);
  if (threadIdx.x == 0) {
    char* o = out + n * out_ld * Elem<OT>::kBytes;
    Elem<OT>::store(o, c, dg);
    if (has_bias) Elem<OT>::store(o, C + c, db);
  }
}

// x_hat in x's (N, C, S) layout.
template <int DT, int OT>
__global__ __launch_bounds__(kChThreads) void chnorm_xhat(const char* __restrict__ x, int64_t C, int64_t S,
                                                          int64_t per_group, const float* __restrict__ stats,
                                                          char* __restrict__ out) {
  const int64_t row = blockIdx.x;
  const int64_t n = row / C, c = row - n * C;
  const int64_t grp = n * (C / per_group) + c / per_group;
  const float mean = stats[2 * grp], rstd = stats[2 * grp + 1];
  const char* xr = x + row * S * Elem<DT>::kBytes;
  char* orow = out + row * S * Elem<OT>::kBytes;
  for (int64_t s = threadIdx.x; s < S; s += kChThreads) Elem<OT>::store(orow, s, (Elem<DT>::load(xr, s) - mean) * rstd);
}

int ch_check(const char* who, int dtype, int out_dtype, int64_t N, int64_t C, int64_t S, int64_t G) {
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return set_error(DA_ERR_INVALID, "%s: bad dtype", who);
  if (N < 0 || C < 0 || S < 0 || G <= 0) return set_error(DA_ERR_INVALID, "%s: bad sizes", who);
  if (C % G) return set_error(DA_ERR_INVALID, "%s: C=%lld is not a multiple of G=%lld", who, (long long)C, (long long)G);
  if (N * C > 0x7fffffffLL || N * G > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: too many rows", who);
  return DA_OK;
}

int ch_stats(const void* x, int dtype, int64_t N, int64_t C, int64_t S, int64_t G, float eps, float* stats,
             hipStream_t st) {
  const int64_t ge = (C / G) * S;
  switch (dtype) {
    case DA_BF16: chnorm_stats<DA_BF16><<<(unsigned)(N * G), kChThreads, 0, st>>>((const char*)x, ge, eps, stats); break;
    case DA_F16: chnorm_stats<DA_F16><<<(unsigned)(N * G), kChThreads, 0, st>>>((const char*)x, ge, eps, stats); break;
    default: chnorm_stats<DA_F32><<<(unsigned)(N * G), kChThreads, 0, st>>>((const char*)x, ge, eps, stats); break;
  }
  return check_launch("channel norm statistics");
}

template <int DT>
void grad_launch(const void* x, const void* g, int64_t N, int64_t C, int64_t S, int64_t pg, const float* stats,
                 int has_bias, void* out, int out_dtype, int64_t out_ld, hipStream_t st) {
  const unsigned grid = (unsigned)(N * C);
  switch (out_dtype) {
    case DA_BF16:
      chnorm_grad<DT, DA_BF16><<<grid, kChThreads, 0, st>>>((const char*)x, (const char*)g, C, S, pg, stats, has_bias,
                                                            (char*)out, out_ld);
      break;
    case DA_F16:
      chnorm_grad<DT, DA_F16><<<grid, kChThreads, 0, st>>>((const char*)x, (const char*)g, C, S, pg, stats, has_bias,
                                                           (char*)out, out_ld);
      break;
    default:
      chnorm_grad<DT, DA_F32><<<grid, kChThreads, 0, st>>>((const char*)x, (const char*)g, C, S, pg, stats, has_bias,
                                                           (char*)out, out_ld);
      break;
  }
}

template <int DT>
void xhat_launch(const void* x, int64_t N, int64_t C, int64_t S, int64_t pg, const float* stats, void* out,
                 int out_dtype, hipStream_t st) {
  const unsigned grid = (unsigned)(N * C);
  switch (out_dtype) {
    case DA_BF16: chnorm_xhat<DT, DA_BF16><<<grid, kChThreads, 0, st>>>((const char*)x, C, S, pg, stats, (char*)out); break;
    case DA_F16: chnorm_xhat<DT, DA_F16><<<grid, kChThreads, 0, st>>>((const char*)x, C, S, pg, stats, (char*)out); break;
    default: chnorm_xhat<DT, DA_F32><<<grid, kChThreads, 0, st>>>((const char*)x, C, S, pg, stats, (char*)out); break;
  }
}

}  // namespace
}  // namespace da

extern "C" {

int da_channel_norm_workspace(int64_t N, int64_t G, size_t* bytes) {
  if (N < 0 || G <= 0 || !bytes) return da::set_error(DA_ERR_INVALID, "da_channel_norm_workspace: bad arguments");
  *bytes = (size_t)(N * G) * 2 * sizeof(float);
  return DA_OK;
}

int da_channel_norm_weight_grad(const void* x, const void* g, int dtype, int64_t N, int64_t C, int64_t S, int64_t G,
                                float eps, int has_bias, void* out, int out_dtype, int64_t out_ld, void* workspace,
                                size_t workspace_bytes, void* stream) {
  using namespace da;
  const char* who = "da_channel_norm_weight_grad";
  int rc = ch_check(who, dtype, out_dtype, N, C, S, G);
  if (rc) return rc;
  if (N == 0 || C == 0) return DA_OK;
  if (!out || out_ld < C * (has_bias ? 2 : 1)) return set_error(DA_ERR_INVALID, "%s: bad out / out_ld", who);
  if (S == 0) return set_error(DA_ERR_INVALID, "%s: no positions (S = 0)", who);
  if (!x || !g) return set_error(DA_ERR_INVALID, "%s: NULL input", who);
  hipStream_t st = (hipStream_t)stream;
  const size_t need = (size_t)(N * G) * 2 * sizeof(float);
  if (!workspace || workspace_bytes < need)
    return set_error(DA_ERR_WORKSPACE, "%s: workspace needs %zu bytes, got %zu", who, need, workspace_bytes);
  float* stats = (float*)workspace;
  rc = ch_stats(x, dtype, N, C, S, G, eps, stats, st);
  if (rc) return rc;
  const int64_t pg = C / G;
  switch (dtype) {
    case DA_BF16: grad_launch<DA_BF16>(x, g, N, C, S, pg, stats, has_bias, out, out_dtype, out_ld, st); break;
    case DA_F16: grad_launch<DA_F16>(x, g, N, C, S, pg, stats, has_bias, out, out_dtype, out_ld, st); break;
    default: grad_launch<DA_F32>(x, g, N, C, S, pg, stats, has_bias, out, out_dtype, out_ld, st); break;
  }
  return check_launch(who);
}

int da_channel_norm_xhat(const void* x, int dtype, int64_t N, int64_t C, int64_t S, int64_t G, float eps, void* out,
                         int out_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace da;
  const char* who = "da_channel_norm_xhat";
  int rc = ch_check(who, dtype, out_dtype, N, C, S, G);
  if (rc) return rc;
  if (N == 0 || C == 0 || S == 0) return DA_OK;
  if (!x || !out) return set_error(DA_ERR_INVALID, "%s: NULL pointer", who);
  const size_t need = (size_t)(N * G) * 2 * sizeof(float);
  if (!workspace || workspace_bytes < need)
    return set_error(DA_ERR_WORKSPACE, "%s: workspace needs %zu bytes, got %zu", who, need, workspace_bytes);
  hipStream_t st = (hipStream_t)stream;
  float* stats = (float*)workspace;
  rc = ch_stats(x, dtype, N, C, S, G, eps, stats, st);
  if (rc) return rc;
  const int64_t pg = C / G;
  switch (dtype) {
    case DA_BF16: xhat_launch<DA_BF16>(x, N, C, S, pg, stats, out, out_dtype, st); break;
    case DA_F16: xhat_launch<DA_F16>(x, N, C, S, pg, stats, out, out_dtype, st); break;
    default: xhat_launch<DA_F32>(x, N, C, S, pg, stats, out, out_dtype, st); break;
  }
  return check_launch(who);
}

}  // extern "C"
