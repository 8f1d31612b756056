// Exact location of routed token rows in their block input
// (RoutedTokenTracker._match, dattri_llm/gradient/hooks/routing.py:300-333).
//
// A Mixture-of-Experts expert receives (n, d) rows gathered from the block's
// (B*T, d) input.  Row r of x is the k-th occurrence of its value among x's
// rows; it is matched to the k-th token (ascending) of the block input holding
// the same value, and the match is verified by an exact element comparison
// (float equality: -0 equals +0, a NaN equals nothing, as torch.equal).
//
//   1. one wave per row: a 64-bit fingerprint of the row's bits, the sum over
//      its 8-byte words of SplitMix64's finalizer (Steele, Lea & Flood 2014)
//      applied to the word xor a per-position constant -- order-free, so the
//      lanes combine it in any order with the same result;
//   2. stable radix sorts (rocPRIM) of (fingerprint, index) for the block
//      input and for x: equal fingerprints keep ascending index order;
//   3. one wave per sorted x row: its rank among x's equal fingerprints, the
//      block input's run of that fingerprint (binary searches), the token at
//      the run's start + rank, and the comparison of the two rows.
// A fingerprint collision between different rows fails the comparison and
// the whole match fails, as the reference's does.
#include <algorithm>

#include <rocprim/device/device_radix_sort.hpp>

#include "common.h"

namespace da {
namespace {

constexpr int kMatchThreads = 256;
constexpr uint64_t kPosMul = 0x9e3779b97f4a7c15ULL;  // 2^64 / golden ratio: spreads word positions

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += (uint64_t)__shfl_xor((unsigned long long)v, m);
  return v;
}

// keys[r] = fingerprint of row r (row_bytes a multiple of 16, rows 16-byte aligned).
__global__ __launch_bounds__(kMatchThreads) void row_fingerprints(const char* __restrict__ x, int64_t rows,
                                                                  int64_t rstride, int64_t chunks,
                                                                  uint64_t* __restrict__ keys) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (kMatchThreads / kWave) + (threadIdx.x >> 6);
  if (r >= rows) return;  // uniform per wave
  const char* row = x + r * rstride;
  uint64_t h = 0;
  for (int64_t c = lane; c < chunks; c += kWave) {
    const u32x4 v = ld16(row + c * 16);
    const uint64_t lo = (uint64_t)v[0] | ((uint64_t)v[1] << 32), hi = (uint64_t)v[2] | ((uint64_t)v[3] << 32);
    h += mix64(lo ^ ((uint64_t)(2 * c + 1) * kPosMul)) + mix64(hi ^ ((uint64_t)(2 * c + 2) * kPosMul));
  }
  h = wave_sum_u64(h);
  if (lane == 0) keys[r] = h;
}

__global__ void iota_i32(int32_t* __restrict__ v, int64_t n, int32_t* __restrict__ status) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) v[i] = (int32_t)i;
  if (i == 0 && status) *status = 0;
}

// First index in k[0, n) whose value is >= key (upper: > key).
__device__ __forceinline__ int64_t bound(const uint64_t* k, int64_t n, uint64_t key, bool upper) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (upper ? (k[mid] <= key) : (k[mid] < key)) lo = mid + 1; else hi = mid;
  }
  return lo;
}

template <int DT>
__device__ __forceinline__ bool chunk_equal(u32x4 a, u32x4 b) {
  float fa[Elem<DT>::kVec], fb[Elem<DT>::kVec];
  unpack16<DT>(a, fa);
  unpack16<DT>(b, fb);
  bool eq = true;
#pragma unroll
  for (int e = 0; e < Elem<DT>::kVec; ++e) eq &= fa[e] == fb[e];
  return eq;
}

// One wave per sorted x row j: token[ix[j]] = the matched block-input token;
// *status = 1 when a row has no token left or its values differ.
template <int DT>
__global__ __launch_bounds__(kMatchThreads) void match_rows_kernel(
    const char* __restrict__ src, int64_t n_src, int64_t src_rstride, const uint64_t* __restrict__ skeys,
    const int32_t* __restrict__ sorder, const char* __restrict__ x, int64_t n_x, int64_t x_rstride,
    const uint64_t* __restrict__ xkeys, const int32_t* __restrict__ xorder, int64_t chunks,
    int64_t* __restrict__ token, int32_t* __restrict__ status) {
  const int lane = threadIdx.x & 63;
  const int64_t j = (int64_t)blockIdx.x * (kMatchThreads / kWave) + (threadIdx.x >> 6);
  if (j >= n_x) return;  // uniform per wave
  const uint64_t key = xkeys[j];
  const int64_t rank = j - bound(xkeys, n_x, key, false);
  const int64_t pos = bound(skeys, n_src, key, false) + rank;
  const int64_t r = xorder[j];
  if (pos >= bound(skeys, n_src, key, true)) {  // more copies of this row than the block holds
    if (lane == 0) {
      token[r] = -1;
      *status = 1;
    }
    return;
  }
  const int64_t t = sorder[pos];
  const char* a = x + r * x_rstride;
  const char* b = src + t * src_rstride;
  bool eq = true;
  for (int64_t c = lane; c < chunks; c += kWave) eq &= chunk_equal<DT>(ld16(a + c * 16), ld16(b + c * 16));
  const bool all = __all(eq);
  if (lane == 0) {
    token[r] = all ? t : -1;
    if (!all) *status = 1;
  }
}

struct MatchWs {
  size_t sort_bytes, total;
  size_t off_skeys, off_skeys2, off_sidx, off_sorder, off_xkeys, off_xkeys2, off_xidx, off_xorder, off_sort;
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

int match_plan(int64_t n_src, int64_t n_x, MatchWs* w) {
  size_t sort_bytes = 0;
  const int64_t big = n_src > n_x ? n_src : n_x;
  if (big > 0) {
    hipError_t e = rocprim::radix_sort_pairs(nullptr, sort_bytes, (const uint64_t*)nullptr, (uint64_t*)nullptr,
                                             (const int32_t*)nullptr, (int32_t*)nullptr, (unsigned int)big, 0, 64,
                                             (hipStream_t)0);
    if (e != hipSuccess) return set_error(DA_ERR_HIP, "da_match_rows: sort sizing failed: %s", hipGetErrorString(e));
  }
  size_t o = 256;  // the status word
  w->off_skeys = o; o = align256(o + n_src * 8);
  w->off_skeys2 = o; o = align256(o + n_src * 8);
  w->off_sidx = o; o = align256(o + n_src * 4);
  w->off_sorder = o; o = align256(o + n_src * 4);
  w->off_xkeys = o; o = align256(o + n_x * 8);
  w->off_xkeys2 = o; o = align256(o + n_x * 8);
  w->off_xidx = o; o = align256(o + n_x * 4);
  w->off_xorder = o; o = align256(o + n_x * 4);
  w->off_sort = o;
  w->sort_bytes = sort_bytes;
  w->total = o + align256(sort_bytes);
  return DA_OK;
}

}  // namespace
}  // namespace da

extern "C" {

int da_match_rows_workspace(int64_t n_src, int64_t n_x, size_t* bytes) {
  using namespace da;
  if (n_src < 0 || n_x < 0 || !bytes || n_src > 0x7fffffffLL || n_x > 0x7fffffffLL)
    return set_error(DA_ERR_INVALID, "da_match_rows_workspace: bad arguments");
  MatchWs w;
  int rc = match_plan(n_src, n_x, &w);
  if (rc) return rc;
  *bytes = w.total;
  return DA_OK;
}

int da_match_rows(const void* src, int64_t n_src, int64_t src_rstride, const void* x, int64_t n_x, int64_t x_rstride,
                  int64_t width, int dtype, int64_t* token, int32_t* status, void* workspace, size_t workspace_bytes,
                  void* stream) {
  using namespace da;
  const char* who = "da_match_rows";
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "%s: bad dtype", who);
  if (n_src < 0 || n_x < 0 || width <= 0 || n_src > 0x7fffffffLL || n_x > 0x7fffffffLL)
    return set_error(DA_ERR_INVALID, "%s: bad sizes", who);
  const int64_t es = (int64_t)elem_bytes(dtype);
  if ((width * es) % 16 || ((uintptr_t)src & 15) || ((uintptr_t)x & 15) || (src_rstride * es) % 16 ||
      (x_rstride * es) % 16)
    return set_error(DA_ERR_INVALID, "%s: rows must be 16-byte aligned and a multiple of 16 bytes wide", who);
  if (!token || !status || !workspace) return set_error(DA_ERR_INVALID, "%s: NULL pointer", who);
  MatchWs w;
  int rc = match_plan(n_src, n_x, &w);
  if (rc) return rc;
  if (workspace_bytes < w.total)
    return set_error(DA_ERR_WORKSPACE, "%s: workspace needs %zu bytes, got %zu", who, w.total, workspace_bytes);
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  uint64_t* skeys = (uint64_t*)(ws + w.off_skeys);
  uint64_t* skeys2 = (uint64_t*)(ws + w.off_skeys2);
  int32_t* sidx = (int32_t*)(ws + w.off_sidx);
  int32_t* sorder = (int32_t*)(ws + w.off_sorder);
  uint64_t* xkeys = (uint64_t*)(ws + w.off_xkeys);
  uint64_t* xkeys2 = (uint64_t*)(ws + w.off_xkeys2);
  int32_t* xidx = (int32_t*)(ws + w.off_xidx);
  int32_t* xorder = (int32_t*)(ws + w.off_xorder);
  void* sort_tmp = ws + w.off_sort;
  iota_i32<<<(unsigned)((std::max<int64_t>(n_src, 1) + 255) / 256), 256, 0, st>>>(sidx, n_src, status);
  if (n_x == 0) return check_launch(who);
  if (n_src == 0) return set_error(DA_ERR_INVALID, "%s: no block rows to match against", who);
  iota_i32<<<(unsigned)((n_x + 255) / 256), 256, 0, st>>>(xidx, n_x, nullptr);
  const int64_t chunks = width * es / 16;
  const int per = kMatchThreads / kWave;
  row_fingerprints<<<(unsigned)((n_src + per - 1) / per), kMatchThreads, 0, st>>>((const char*)src, n_src,
                                                                                  src_rstride * es, chunks, skeys);
  row_fingerprints<<<(unsigned)((n_x + per - 1) / per), kMatchThreads, 0, st>>>((const char*)x, n_x, x_rstride * es,
                                                                                chunks, xkeys);
  rc = check_launch(who);
  if (rc) return rc;
  size_t tb = w.sort_bytes;
  hipError_t e = rocprim::radix_sort_pairs(sort_tmp, tb, skeys, skeys2, sidx, sorder, (unsigned int)n_src, 0, 64, st);
  if (e == hipSuccess) {
    tb = w.sort_bytes;
    e = rocprim::radix_sort_pairs(sort_tmp, tb, xkeys, xkeys2, xidx, xorder, (unsigned int)n_x, 0, 64, st);
  }
  if (e != hipSuccess) return set_error(DA_ERR_HIP, "%s: sort failed: %s", who, hipGetErrorString(e));
  const unsigned grid = (unsigned)((n_x + per - 1) / per);
  const int64_t srs = src_rstride * es, xrs = x_rstride * es;
  switch (dtype) {
    case DA_BF16:
      match_rows_kernel<DA_BF16><<<grid, kMatchThreads, 0, st>>>((const char*)src, n_src, srs, skeys2, sorder,
                                                                 (const char*)x, n_x, xrs, xkeys2, xorder, chunks,
                                                                 token, status);
      break;
    case DA_F16:
      match_rows_kernel<DA_F16><<<grid, kMatchThreads, 0, st>>>((const char*)src, n_src, srs, skeys2, sorder,
                                                                (const char*)x, n_x, xrs, xkeys2, xorder, chunks,
                                                                token, status);
      break;
    default:
      match_rows_kernel<DA_F32><<<grid, kMatchThreads, 0, st>>>((const char*)src, n_src, srs, skeys2, sorder,
                                                                (const char*)x, n_x, xrs, xkeys2, xorder, chunks,
                                                                token, status);
      break;
  }
  return check_launch(who);
}

}  // extern "C"
