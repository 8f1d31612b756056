// K3c: MoE routing and expert segmentation (integer work, bit-exact).
//
//   da_moe_topk:       top-k of softmax(logits) per token, weights renormalised
//                      over the k, indices in torch.topk's CPU order (ties
//                      included, topk_select.h) -- the router of
//                      transformers' MixtralTopKRouter.forward
//                      (softmax(logits.float()) -> topk -> / sum), as consumed by
//                      dattri_llm/gradient/hooks/override_layers/fused_experts.py:210-237.
//   da_counting_sort:  stable counting sort of int32 keys into bins.  With the
//                      top-k indices read slot-major (key[p] = idx[p % N][p / N])
//                      the sorted order is exactly the reference loop's
//                      torch.where(one_hot(idx).permute(2,1,0)[e]) enumeration,
//                      fused_experts.py:219-228 (slot-major, token ascending),
//                      and the bin offsets are the expert segments.  With
//                      key = token // T it groups an expert's rows by sample for
//                      the segmented ghost product (the dense-with-zeros regroup
//                      of hooks/routing.py:71-86, without the zeros).
//
// Both are tiny next to the expert GEMMs; they exist so the routing never
// leaves the device and never depends on a library sort's tie order.
#include "common.h"
#include "topk_select.h"

namespace da {
namespace {

constexpr int kMaxExperts = 256;
constexpr int kMaxTopK = 16;
constexpr int kMaxBins = 8192;

// One router queue per lane in LDS: entry i of lane l at [i * lanes + l], so
// the lanes of a wave touching the same entry hit consecutive words.
struct LdsQueue {
  float* p;
  uint16_t* e;
  int lanes;
  __device__ topk::Entry get(int i) const { return {p[i * lanes], (int)e[i * lanes]}; }
  __device__ void set(int i, topk::Entry x) {
    p[i * lanes] = x.p;
    e[i * lanes] = (uint16_t)x.e;
  }
  __device__ void swap(int i, int j) {
    const topk::Entry a = get(i), b = get(j);
    set(i, b);
    set(j, a);
  }
};

// One lane per token (workgroups of 64 lanes, 32 above 128 experts, so the
// dynamic LDS of 6 bytes per expert and lane stays within 48 KiB).  softmax(logits.float()) as torch computes it -- a maximum that
// propagates NaN, then exp(x - max) / sum -- so a row holding a NaN or +inf
// logit, or only -inf logits, gives NaN probabilities as torch's does; then
// the selection of topk_select.h and weights = top / sum(top).
template <int DT>
__global__ __launch_bounds__(kWave) void moe_topk_kernel(const char* logits, int64_t n, int e, int k,
                                                         int64_t rstride, float* weights, int64_t* index) {
  extern __shared__ __attribute__((aligned(16))) char topk_lds[];
  const int lane = threadIdx.x, lanes = blockDim.x;
  const int64_t tok = (int64_t)blockIdx.x * lanes + lane;
  if (tok >= n) return;
  LdsQueue q{(float*)topk_lds + lane, (uint16_t*)(topk_lds + (size_t)e * lanes * 4) + lane, lanes};
  const char* row = logits + tok * rstride * Elem<DT>::kBytes;
  float mx = -INFINITY;
  for (int x = 0; x < e; ++x) {
    const float v = Elem<DT>::load(row, x);
    if (mx == mx && (v != v || v > mx)) mx = v;
  }
  float sum = 0.f;
  for (int x = 0; x < e; ++x) sum += expf(Elem<DT>::load(row, x) - mx);
  for (int x = 0; x < e; ++x) q.set(x, {expf(Elem<DT>::load(row, x) - mx) / sum, x});
  topk::select_topk(q, e, k);
  float tsum = 0.f;
  for (int s = 0; s < k; ++s) tsum += q.get(s).p;
  for (int s = 0; s < k; ++s) {
    const topk::Entry t = q.get(s);
    weights[tok * k + s] = t.p / tsum;
    index[tok * k + s] = t.e;
  }
}

// Routed-row compaction: the rows p < batch * tokens whose mask byte is
// non-zero, in increasing order, with per-sample offsets (row p = b * tokens
// + t belongs to sample b).  One workgroup: a ballot rank inside each wave,
// the waves' counts in LDS, and a running carry across 1024-row steps.
__global__ __launch_bounds__(1024) void compact_rows_kernel(const uint8_t* __restrict__ mask, int64_t batch,
                                                            int64_t tokens, int32_t* __restrict__ seg,
                                                            int32_t* __restrict__ rows) {
  __shared__ int32_t wave_count[16];
  __shared__ int32_t carry;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t n = batch * tokens;
  for (int64_t b = tid; b <= batch; b += 1024) seg[b] = 0;  // samples with no tokens
  if (tid == 0) carry = 0;
  __syncthreads();
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  for (int64_t base = 0; base < n; base += 1024) {
    const int64_t p = base + tid;
    const bool keep = p < n && mask[p] != 0;
    const uint64_t ballot = __ballot(keep);
    if (lane == 0) wave_count[wave] = __popcll(ballot);
    __syncthreads();
    int32_t rank = carry + __popcll(ballot & below);  // kept rows before p
    for (int w = 0; w < wave; ++w) rank += wave_count[w];
    if (p < n && p % tokens == 0) seg[p / tokens] = rank;
    if (keep) rows[rank] = (int32_t)p;
    __syncthreads();
    if (tid == 0) {
      int32_t total = carry;
      for (int w = 0; w < 16; ++w) total += wave_count[w];
      carry = total;
    }
    __syncthreads();
  }
  if (tid == 0) seg[batch] = carry;
}

// keys are read either directly (slot_major == 0: key[p] = keys[p]) or as the
// slot-major view of an (n/k, k) int64 index matrix (slot_major == 1).
struct SortArgs {
  const int32_t* keys32;
  const int64_t* keys64;  // (rows, k) row-major when slot_major
  int64_t n, rows, k;
  int slot_major;
  int bins;
  int32_t* offsets;       // bins + 1
  int32_t* perm;          // n
  int64_t key_div;        // key = raw / key_div (1 = identity)
};

__device__ __forceinline__ int64_t sort_key(const SortArgs& a, int64_t p) {
  int64_t raw;
  if (a.slot_major) {
    const int64_t slot = p / a.rows, r = p - slot * a.rows;
    raw = a.keys64[r * a.k + slot];
  } else {
    raw = a.keys32 ? (int64_t)a.keys32[p] : a.keys64[p];
  }
  return a.key_div > 1 ? (raw >= 0 ? raw / a.key_div : -1) : raw;
}

// One workgroup: histogram (LDS atomics; counts are order independent), exclusive
// scan, then wave 0 scatters in input order, 64 entries at a time, ranking equal
// keys inside the wave with shuffles -- a stable sort.  Keys outside [0, bins)
// are skipped; offsets[bins] is the number of entries kept.
__global__ __launch_bounds__(256) void counting_sort_kernel(SortArgs a) {
  __shared__ int32_t cnt[kMaxBins];
  const int tid = threadIdx.x;
  for (int b = tid; b < a.bins; b += 256) cnt[b] = 0;
  __syncthreads();
  for (int64_t p = tid; p < a.n; p += 256) {
    const int64_t key = sort_key(a, p);
    if (key >= 0 && key < a.bins) atomicAdd(&cnt[key], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int32_t run = 0;
    for (int b = 0; b < a.bins; ++b) {
      const int32_t c = cnt[b];
      a.offsets[b] = run;
      cnt[b] = run;  // becomes the next free slot of bin b
      run += c;
    }
    a.offsets[a.bins] = run;
  }
  __syncthreads();
  if (tid >= 64) return;
  const int lane = tid;
  for (int64_t base = 0; base < a.n; base += 64) {
    const int64_t p = base + lane;
    const int64_t key = p < a.n ? sort_key(a, p) : -1;
    const bool ok = key >= 0 && key < a.bins;
    int rank = 0, total = 0;
    for (int src = 0; src < 64; ++src) {
      const int64_t other = __shfl(key, src, 64);
      if (ok && other == key) {
        total += 1;
        if (src < lane) rank += 1;
      }
    }
    int32_t slot = 0;
    if (ok) slot = cnt[key] + rank;
    // every lane has read cnt[] before the last lane of each key group bumps it
    __builtin_amdgcn_wave_barrier();
    if (ok) {
      a.perm[slot] = (int32_t)p;
      if (rank == total - 1) cnt[key] = slot + 1;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

// Expert routing of one side in one workgroup.  Entries p = slot*N + token are
// visited in order (the reference's slot-major enumeration); with e = idx[token][slot]
// and b = token / T the kernel runs two stable counting sorts in the same pass:
//   by e      -> entries[off[e] + r] = p for expert e's local row r (routed order);
//   by e*B+b  -> rows[off2[e*B+b] + q] = r, expert e's local rows grouped by sample,
// and seg[e*(B+1) + b] = off2[e*B+b] - off2[e*B] (per-expert relative offsets).
// Histograms and scans use the whole workgroup; the order-dependent scatter
// splits each LDS-resident tile of keys into 16 consecutive segments, one per
// wave, starting from per-wave counters (the cross-wave exclusive sums of
// per-wave histograms), each lane's rank among the lanes of equal key coming
// from one ballot per distinct key in the wave.  When E*B bins do not fit the
// per-wave histograms, the workgroup sorts by e alone and moe_route_rows forms
// the rows, one wave per expert.
struct RouteArgs {
  const int64_t* index;  // (N, k)
  int64_t n, k, experts, batch, tokens;
  int32_t* offsets;  // experts + 1
  int32_t* entries;  // n*k
  int32_t* seg;      // experts * (batch + 1)
  int32_t* rows;     // n*k
};

constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / 64;
constexpr int kRouteTile = 8192;      // keys staged in LDS per pass of the scatter
constexpr int kRouteWaveBins = 1024;  // per-wave histograms of both keys when E*B fits

// In-place exclusive scan of the LDS array a[0, len) by the whole workgroup;
// returns the total.  wsum: kRouteWaves ints of LDS.
__device__ int32_t route_scan(int32_t* a, int len, int32_t* wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (len + kRouteThreads - 1) / kRouteThreads;
  const int beg = tid * per;
  int32_t s = 0;
  for (int i = 0; i < per; ++i)
    if (beg + i < len) s += a[beg + i];
  int32_t x = s;  // inclusive scan over the wave
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int32_t v = lane < kRouteWaves ? wsum[lane] : 0;
    for (int off = 1; off < 64; off <<= 1) {
      const int32_t y = __shfl_up(v, off, 64);
      if (lane >= off) v += y;
    }
    if (lane < kRouteWaves) wsum[lane] = v;
  }
  __syncthreads();
  int32_t run = (wave > 0 ? wsum[wave - 1] : 0) + x - s;
  for (int i = 0; i < per; ++i)
    if (beg + i < len) {
      const int32_t c = a[beg + i];
      a[beg + i] = run;
      run += c;
    }
  const int32_t total = wsum[kRouteWaves - 1];
  __syncthreads();
  return total;
}

// Ranks of this wave's 64 keys among equal keys of the wave (stable), one
// ballot per distinct key; r = lanes below with the same key, t = all of them.
__device__ __forceinline__ void route_ranks(bool ok, int key, uint64_t lt, int& r, int& t) {
  r = 0;
  t = 0;
  for (uint64_t act = __ballot(ok); act;) {
    const int ke = __builtin_amdgcn_readlane(key, __builtin_ctzll(act));
    const bool mine = ok && key == ke;
    const uint64_t m = __ballot(mine);
    if (mine) {
      r = __popcll(m & lt);
      t = __popcll(m);
    }
    act &= ~m;
  }
}

// The ordered scatter of one wave over keys[beg, end) of the tile starting at
// entry t0, advancing the running counters n1 (by expert) and n2 (by expert
// and sample).
template <bool kRows>
__device__ __forceinline__ void route_scatter(const RouteArgs& a, const int32_t* keys, uint32_t t0, uint32_t beg,
                                              uint32_t end, int32_t* n1, int32_t* n2, const int32_t* o1) {
  const int lane = threadIdx.x & 63;
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));  // lanes below this one
  for (uint32_t base = beg; base < end; base += 64) {
    const uint32_t i = base + lane;
    const int32_t kk = i < end ? keys[i] : -1;
    const bool ok = kk >= 0;
    const int e = kk & 511, e2 = kk >> 9;
    int r1, t1, r2 = 0, t2 = 0;
    route_ranks(ok, e, lt, r1, t1);
    if constexpr (kRows) route_ranks(ok, e2, lt, r2, t2);
    int32_t s1 = 0, s2 = 0;
    if (ok) {
      s1 = n1[e] + r1;
      if constexpr (kRows) s2 = n2[e2] + r2;
    }
    // every lane has read the counters before the last lane of each key bumps them
    __builtin_amdgcn_wave_barrier();
    if (ok) {
      a.entries[s1] = (int32_t)(t0 + i);
      if (r1 == t1 - 1) n1[e] = s1 + 1;
      if constexpr (kRows) {
        a.rows[s2] = s1 - o1[e];  // expert-local routed row
        if (r2 == t2 - 1) n2[e2] = s2 + 1;
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(RouteArgs a) {
  __shared__ int32_t c1[kMaxExperts + 1], o1[kMaxExperts + 1];
  __shared__ int32_t c2[kMaxBins + 1];
  __shared__ int32_t keys[kRouteTile];
  __shared__ int32_t h1[kRouteWaves][kMaxExperts];    // per-wave counters by expert
  __shared__ int32_t h2[kRouteWaves][kRouteWaveBins];  // per-wave counters by expert and sample
  __shared__ int32_t wsum[kRouteWaves];
  const int tid = threadIdx.x, wave = tid >> 6;
  const uint32_t n = (uint32_t)a.n, total = (uint32_t)(a.n * a.k), T = (uint32_t)a.tokens;
  const uint32_t B = (uint32_t)a.batch;
  const int E = (int)a.experts, nb2 = E * (int)B;
  const bool per_wave = nb2 <= kRouteWaveBins;  // uniform
  for (int i = tid; i <= E; i += kRouteThreads) c1[i] = 0;
  for (int i = tid; i <= nb2; i += kRouteThreads) c2[i] = 0;
  __syncthreads();
  // entry p -> (e*B + b) << 9 | e, or -1 when its expert index is out of range
  auto key = [&](uint32_t p, int64_t e) __attribute__((always_inline)) {
    const uint32_t slot = p / n, tok = p - slot * n;
    return (e < 0 || e >= E) ? -1 : (int32_t)((((uint32_t)e * B + tok / T) << 9) | (uint32_t)e);
  };
  auto index_of = [&](uint32_t p) __attribute__((always_inline)) {
    const uint32_t slot = p / n, tok = p - slot * n;
    return a.index[(int64_t)tok * a.k + slot];
  };
  // keys of entries p0 + kRouteThreads*j, j < 8, loads first
  auto keys8 = [&](uint32_t p0, uint32_t lim, int32_t (&kk)[8]) __attribute__((always_inline)) {
    int64_t ev[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t p = p0 + (uint32_t)(kRouteThreads * j);
      ev[j] = p < lim ? index_of(p) : -1;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) kk[j] = key(p0 + (uint32_t)(kRouteThreads * j), ev[j]);
  };
  for (uint32_t p0 = tid; p0 < total; p0 += 8 * kRouteThreads) {
    int32_t kk[8];
    keys8(p0, total, kk);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (kk[j] >= 0) {
        atomicAdd(&c1[kk[j] & 511], 1);
        atomicAdd(&c2[kk[j] >> 9], 1);
      }
  }
  __syncthreads();
  const int32_t nvalid = route_scan(c1, E, wsum);
  route_scan(c2, nb2, wsum);
  for (int i = tid; i < E; i += kRouteThreads) {
    o1[i] = c1[i];
    a.offsets[i] = c1[i];
  }
  if (tid == 0) {
    a.offsets[E] = nvalid;
    c2[nb2] = nvalid;
  }
  __syncthreads();
  // per-expert relative offsets (c2 holds bin starts until the scatter advances them)
  for (int q = tid; q < E * ((int)B + 1); q += kRouteThreads) {
    const int e = q / ((int)B + 1), b = q - e * ((int)B + 1);
    a.seg[q] = c2[e * (int)B + b] - c2[e * (int)B];
  }
  __syncthreads();
  for (uint32_t t0 = 0; t0 < total; t0 += kRouteTile) {
    const uint32_t nt = min((uint32_t)kRouteTile, total - t0);
    for (uint32_t i0 = tid; i0 < nt; i0 += 8 * kRouteThreads) {
      int32_t kk[8];
      keys8(t0 + i0, t0 + nt, kk);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (i0 + (uint32_t)(kRouteThreads * j) < nt) keys[i0 + kRouteThreads * j] = kk[j];
    }
    {
      // wave w takes keys [w*seg, (w+1)*seg) of the tile, in order; the
      // (expert, sample) counters only when they fit (per_wave)
      const uint32_t segl = (nt + kRouteWaves - 1) / kRouteWaves;
      for (int i = tid; i < kRouteWaves * E; i += kRouteThreads) (&h1[0][0])[(i / E) * kMaxExperts + i % E] = 0;
      if (per_wave)
        for (int i = tid; i < kRouteWaves * nb2; i += kRouteThreads) (&h2[0][0])[(i / nb2) * kRouteWaveBins + i % nb2] = 0;
      __syncthreads();
      const uint32_t beg = min(nt, wave * segl), end = min(nt, beg + segl);
      for (uint32_t i = beg + (tid & 63); i < end; i += 64) {
        const int32_t kk = keys[i];
        if (kk >= 0) {
          atomicAdd(&h1[wave][kk & 511], 1);
          if (per_wave) atomicAdd(&h2[wave][kk >> 9], 1);
        }
      }
      __syncthreads();
      // per key: wave w starts at the running counter plus the counts of waves < w
      for (int e = tid; e < E; e += kRouteThreads) {
        int32_t run = c1[e];
        for (int w = 0; w < kRouteWaves; ++w) {
          const int32_t c = h1[w][e];
          h1[w][e] = run;
          run += c;
        }
        c1[e] = run;
      }
      if (per_wave)
        for (int q = tid; q < nb2; q += kRouteThreads) {
          int32_t run = c2[q];
          for (int w = 0; w < kRouteWaves; ++w) {
            const int32_t c = h2[w][q];
            h2[w][q] = run;
            run += c;
          }
          c2[q] = run;
        }
      __syncthreads();
      if (per_wave) route_scatter<true>(a, keys, t0, beg, end, h1[wave], h2[wave], o1);
      else route_scatter<false>(a, keys, t0, beg, end, h1[wave], nullptr, o1);
    }
    __syncthreads();
  }
}

// The rows of moe_route when E*B bins do not fit its per-wave histograms:
// wave w of the grid takes expert e = w and walks the expert's entries (the
// by-expert sort, routed order) 64 at a time, so rows[off2[e*B+b] + q] = r for
// expert-local row r runs in the same order as in the one-pass form; the
// per-sample counters start at off2[e*B+b] = off[e] + seg[e*(B+1)+b] and sit
// in LDS (B ints per wave; up to 4 waves per workgroup, as many as keep the
// counters within 64 KB).
constexpr int kRowsWaves = 4;
__global__ __launch_bounds__(kRowsWaves * 64) void moe_route_rows(RouteArgs a) {
  extern __shared__ int32_t cnt_all[];  // (blockDim / 64) * B
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x * (int)(blockDim.x >> 6) + wave;
  const int B = (int)a.batch;
  if (e >= a.experts) return;  // uniform per wave; no barrier below
  int32_t* cnt = cnt_all + wave * B;
  const int32_t o = a.offsets[e], oend = a.offsets[e + 1];
  for (int b = lane; b < B; b += 64) cnt[b] = o + a.seg[e * (B + 1) + b];
  __builtin_amdgcn_wave_barrier();
  const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));  // lanes below this one
  const uint32_t n = (uint32_t)a.n, T = (uint32_t)a.tokens;
  for (int32_t base = o; base < oend; base += 64) {
    const int32_t i = base + lane;
    const bool ok = i < oend;
    int b = 0;
    if (ok) {
      const uint32_t p = (uint32_t)a.entries[i];
      b = (int)((p - (p / n) * n) / T);  // token p % N, its sample
    }
    int r, t;
    route_ranks(ok, b, lt, r, t);
    const int32_t s2 = ok ? cnt[b] + r : 0;
    // every lane has read the counters before the last lane of each sample bumps them
    __builtin_amdgcn_wave_barrier();
    if (ok) {
      a.rows[s2] = i - o;  // expert-local routed row
      if (r == t - 1) cnt[b] = s2 + 1;
    }
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace
}  // namespace da

extern "C" {

int da_moe_topk(const void* logits, int dtype, int64_t n_tokens, int n_experts, int k,
                int64_t row_stride, float* weights, int64_t* index, void* stream) {
  using namespace da;
  const char* who = "da_moe_topk";
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "%s: bad dtype", who);
  if (n_tokens < 0) return set_error(DA_ERR_INVALID, "%s: negative token count", who);
  if (n_experts < 1 || n_experts > kMaxExperts)
    return set_error(DA_ERR_INVALID, "%s: n_experts must be in [1, %d]", who, kMaxExperts);
  if (k < 1 || k > n_experts || k > kMaxTopK)
    return set_error(DA_ERR_INVALID, "%s: k must be in [1, min(n_experts, %d)]", who, kMaxTopK);
  if (row_stride < n_experts) return set_error(DA_ERR_INVALID, "%s: row stride < n_experts", who);
  if (n_tokens == 0) return DA_OK;
  if (!logits || !weights || !index) return set_error(DA_ERR_INVALID, "%s: NULL pointer", who);
  const int lanes = n_experts <= 128 ? kWave : kWave / 2;
  if ((n_tokens + lanes - 1) / lanes > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: too many tokens", who);
  const unsigned blocks = (unsigned)((n_tokens + lanes - 1) / lanes);
  const size_t lds = (size_t)n_experts * lanes * (sizeof(float) + sizeof(uint16_t));  // <= 48 KiB
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case DA_BF16: moe_topk_kernel<DA_BF16><<<blocks, lanes, lds, st>>>((const char*)logits, n_tokens, n_experts, k, row_stride, weights, index); break;
    case DA_F16: moe_topk_kernel<DA_F16><<<blocks, lanes, lds, st>>>((const char*)logits, n_tokens, n_experts, k, row_stride, weights, index); break;
    default: moe_topk_kernel<DA_F32><<<blocks, lanes, lds, st>>>((const char*)logits, n_tokens, n_experts, k, row_stride, weights, index); break;
  }
  return check_launch(who);
}

int da_counting_sort(const int32_t* keys32, const int64_t* keys64, int64_t n, int64_t rows,
                     int64_t k, int slot_major, int64_t key_div, int bins, int32_t* offsets,
                     int32_t* perm, void* stream) {
  using namespace da;
  const char* who = "da_counting_sort";
  if (n < 0 || bins < 1 || bins > kMaxBins)
    return set_error(DA_ERR_INVALID, "%s: need n >= 0 and 1 <= bins <= %d", who, kMaxBins);
  if (n > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: at most 2^31-1 entries", who);
  if (key_div < 1) return set_error(DA_ERR_INVALID, "%s: key_div must be >= 1", who);
  if (slot_major) {
    if (!keys64 || rows < 1 || k < 1 || rows * k != n)
      return set_error(DA_ERR_INVALID, "%s: slot-major keys need an int64 (rows, k) matrix with rows*k == n", who);
  } else if (n > 0 && !keys32 && !keys64) {
    return set_error(DA_ERR_INVALID, "%s: no keys", who);
  }
  if (!offsets || (n > 0 && !perm)) return set_error(DA_ERR_INVALID, "%s: NULL output", who);
  SortArgs a;
  a.keys32 = keys32;
  a.keys64 = keys64;
  a.n = n;
  a.rows = rows;
  a.k = k;
  a.slot_major = slot_major;
  a.bins = bins;
  a.offsets = offsets;
  a.perm = perm;
  a.key_div = key_div;
  counting_sort_kernel<<<1, 256, 0, (hipStream_t)stream>>>(a);
  return check_launch(who);
}

int da_moe_route(const int64_t* index, int64_t n_tokens, int k, int n_experts, int64_t batch,
                 int64_t tokens, int32_t* expert_offsets, int32_t* entries, int32_t* seg, int32_t* rows,
                 void* stream) {
  using namespace da;
  const char* who = "da_moe_route";
  if (n_tokens < 0 || k < 1 || k > kMaxTopK)
    return set_error(DA_ERR_INVALID, "%s: need n_tokens >= 0 and 1 <= k <= %d", who, kMaxTopK);
  if (n_experts < 1 || n_experts > kMaxExperts)
    return set_error(DA_ERR_INVALID, "%s: n_experts must be in [1, %d]", who, kMaxExperts);
  if (batch < 1 || tokens < 1 || batch * tokens != n_tokens)
    return set_error(DA_ERR_INVALID, "%s: n_tokens must equal batch * tokens", who);
  if ((int64_t)n_experts * batch > kMaxBins)
    return set_error(DA_ERR_INVALID, "%s: n_experts * batch must be <= %d", who, kMaxBins);
  if (n_tokens * k > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: at most 2^31-1 entries", who);
  if (!index || !expert_offsets || !entries || !seg || !rows)
    return set_error(DA_ERR_INVALID, "%s: NULL pointer", who);
  RouteArgs a;
  a.index = index;
  a.n = n_tokens;
  a.k = k;
  a.experts = n_experts;
  a.batch = batch;
  a.tokens = tokens;
  a.offsets = expert_offsets;
  a.entries = entries;
  a.seg = seg;
  a.rows = rows;
  hipStream_t st = (hipStream_t)stream;
  moe_route_kernel<<<1, kRouteThreads, 0, st>>>(a);
  const int rc = check_launch(who);
  if (rc || (int64_t)n_experts * batch <= kRouteWaveBins) return rc;
  // the rows, one wave per expert, when the (expert, sample) bins exceed the per-wave histograms
  const int waves = batch <= 4096 ? kRowsWaves : 2;  // batch <= 8192: at most 64 KB of counters
  const unsigned blocks = (unsigned)((n_experts + waves - 1) / waves);
  moe_route_rows<<<blocks, waves * 64, (size_t)waves * batch * sizeof(int32_t), st>>>(a);
  return check_launch(who);
}

int da_compact_rows(const uint8_t* mask, int64_t batch, int64_t tokens, int32_t* seg_offsets, int32_t* rows,
                    void* stream) {
  using namespace da;
  const char* who = "da_compact_rows";
  if (batch < 0 || tokens < 0) return set_error(DA_ERR_INVALID, "%s: negative size", who);
  if (batch * tokens > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: at most 2^31-1 rows", who);
  if (!seg_offsets || (batch * tokens > 0 && (!mask || !rows)))
    return set_error(DA_ERR_INVALID, "%s: NULL pointer", who);
  compact_rows_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(mask, batch, tokens, seg_offsets, rows);
  return check_launch(who);
}

}  // extern "C"
