// K3b: per-sample weight gradient of token norm layers (RMSNorm, LayerNorm).
//
//   x_hat[b,t,:] = x * rsqrt(mean(x^2) + eps)                 (RMSNorm)
//                = (x - mean) * rsqrt(var + eps)              (LayerNorm, biased var)
//   dgamma[b,:]  = sum_t x_hat[b,t,:] * g[b,t,:]
//   dbeta[b,:]   = sum_t g[b,t,:]                             (has_bias: out is [dgamma, dbeta])
//
// Follows preprocess_factors' norm branches, dattri_llm/gradient/ops/preprocess.py:366-384,
// with _compute_rms_x_hat / _compute_layer_norm_x_hat (gradient/ops/norm.py:25-41,
// :10-22), the bias augmentation of norm.py:95-110, and the token contraction of
// materialize_factors, gradient/ops/materialize.py:96-98.  The reference makes
// 3-4 elementwise passes plus a concatenation; here one pass reads x and g once.
//
// One wave owns one token row at a time: the row lives in registers
// (kQ 16-byte chunks per lane), the mean square is a wave reduction, and the
// wave accumulates x_hat*g (and g) for its lanes' features across the rows it
// visits.  The four waves of a workgroup combine through LDS and write one fp32
// partial per (sample, token chunk); a second kernel sums the chunks in order.
// Rows of up to 8 KB stream through a per-wave LDS ring (norm_grad_ring);
// longer rows are loaded straight into registers (norm_grad_chunks).
#include "common.h"

namespace da {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kRowsPerWG = 32;  // token rows per workgroup

struct NormArgs {
  const char* x;
  const char* g;
  int64_t batch, tokens, d;
  int64_t dp;                                          // d rounded up to whole 16-byte chunks
  int64_t x_bstride, x_tstride, g_bstride, g_tstride;  // bytes
  int kind;                                            // 0 RMSNorm, 1 LayerNorm, 2 as given
  float eps;
  int has_bias;
  int64_t chunks;                                      // token chunks per sample
  int64_t ring_rows;                                   // token rows per workgroup of the ring form
  float* partial;                                      // [batch][chunks][(1+bias)*dp]
};

template <int DT>
__device__ __forceinline__ float elem_of(const u32x4& v, int e) {
  if constexpr (DT == DA_F32) return __uint_as_float(v[e]);
  else return Elem<DT>::from_bits((e & 1) ? (v[e >> 1] >> 16) : (v[e >> 1] & 0xffffu));
}

template <int DT, int kQ, bool kBias>
__global__ __launch_bounds__(kThreads) void norm_grad_chunks(NormArgs a) {
  constexpr int VEC = Elem<DT>::kVec;
  extern __shared__ float lds[];  // (1+bias) * d floats: one wave's sums at a time

  const int64_t b = blockIdx.y, chunk = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t nchunk16 = a.dp / VEC;  // 16-byte chunks per row; elements past d are masked
  const float inv_d = 1.f / (float)a.d;

  float dg[kQ][VEC], db[kBias ? kQ : 1][VEC];
#pragma unroll
  for (int q = 0; q < kQ; ++q)
#pragma unroll
    for (int e = 0; e < VEC; ++e) dg[q][e] = 0.f;
#pragma unroll
  for (int q = 0; q < (kBias ? kQ : 1); ++q)
#pragma unroll
    for (int e = 0; e < VEC; ++e) db[q][e] = 0.f;

  const int64_t t_begin = chunk * kRowsPerWG;
  const int64_t t_end = min(t_begin + kRowsPerWG, a.tokens);
  for (int64_t t = t_begin + wave; t < t_end; t += kWaves) {
    const char* xr = a.x + b * a.x_bstride + t * a.x_tstride;
    const char* gr = a.g + b * a.g_bstride + t * a.g_tstride;
    u32x4 vx[kQ], vg[kQ];  // the row stays packed; unpacked on use
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const int64_t c = lane + (int64_t)q * kWave;
      const bool in = c < nchunk16;
      vx[q] = in ? ld16(xr + c * 16) : u32x4{0, 0, 0, 0};
      vg[q] = in ? ld16(gr + c * 16) : u32x4{0, 0, 0, 0};
    }
    float mean = 0.f;
    if (a.kind == 1) {
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < kQ; ++q)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const bool in = (lane + (int64_t)q * kWave) * VEC + e < a.d;
          s += in ? elem_of<DT>(vx[q], e) : 0.f;
        }
      mean = wave_sum(s) * inv_d;
    }
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const bool in = (lane + (int64_t)q * kWave) * VEC + e < a.d;
        const float c = in ? elem_of<DT>(vx[q], e) - mean : 0.f;
        ss += c * c;
      }
    }
    const float rstd = a.kind == 2 ? 1.f : 1.f / sqrtf(wave_sum(ss) * inv_d + a.eps);
    // Re-read the packed row rather than keeping kQ*VEC unpacked floats live
    // across the reductions (halves register pressure, doubles occupancy).
#pragma unroll
    for (int q = 0; q < kQ; ++q) asm volatile("" : "+v"(vx[q]));
#pragma unroll
    for (int q = 0; q < kQ; ++q)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const bool in = (lane + (int64_t)q * kWave) * VEC + e < a.d;
        const float gv = in ? elem_of<DT>(vg[q], e) : 0.f;
        dg[q][e] += (elem_of<DT>(vx[q], e) - mean) * rstd * gv;
        if constexpr (kBias) db[q][e] += gv;
      }
  }

  // Combine waves one at a time through LDS (one wave's sums fit), then wave 0
  // writes the workgroup's partial.
  const int64_t width = (1 + a.has_bias) * a.dp;
  for (int w = 1; w < kWaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int q = 0; q < kQ; ++q) {
        const int64_t c = lane + (int64_t)q * kWave;
        if (c < nchunk16)
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            lds[c * VEC + e] = dg[q][e];
            if constexpr (kBias) lds[a.dp + c * VEC + e] = db[q][e];
          }
      }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int q = 0; q < kQ; ++q) {
        const int64_t c = lane + (int64_t)q * kWave;
        if (c < nchunk16)
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            dg[q][e] += lds[c * VEC + e];
            if constexpr (kBias) db[q][e] += lds[a.dp + c * VEC + e];
          }
      }
    }
    __syncthreads();
  }
  if (wave == 0) {
    float* dst = a.partial + (b * a.chunks + chunk) * width;
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const int64_t c = lane + (int64_t)q * kWave;
      if (c < nchunk16)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          dst[c * VEC + e] = dg[q][e];
          if constexpr (kBias) dst[a.dp + c * VEC + e] = db[q][e];
        }
    }
  }
}

// The same per-chunk partials with the rows streamed into LDS: each wave owns
// a private ring of two slots (one token row of x and of g per slot) filled
// by non-temporal buffer loads with the LDS-direct bit, so the next row is in
// flight while the current one is reduced and no VGPRs hold data in flight.
// A slot holds the row's bytes as they are (instruction j of an operand
// carries 16-byte chunks 64j .. 64j+63), so lane l reads chunk l + 64q with
// one conflict-free 16-byte LDS read.  No barriers in the row loop: only
// wave w touches its slots.  Rows past the chunk and chunks past the width
// load zeros from no memory, so every row issues the same 2*kQ instructions
// and one vmcnt count holds.  At 8 KB rows the ring takes 128 KB (4 waves x
// 2 slots x 16 KB); three waves with three slots each measured 5% slower.
// acc + lo^2 + hi^2 of a packed pair of 16-bit values (v_dot2_f32_bf16 / _f16).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <int DT>
__device__ __forceinline__ float dot2_sq(uint32_t w, float acc) {
  if constexpr (DT == DA_BF16) {
    const bf16x2_t v = __builtin_bit_cast(bf16x2_t, w);
    return __builtin_amdgcn_fdot2_f32_bf16(v, v, acc, false);
  } else {
    const f16x2_t v = __builtin_bit_cast(f16x2_t, w);
    return __builtin_amdgcn_fdot2(v, v, acc, false);
  }
}

// Token rows per workgroup of the ring form: 64, or 32 / 16 when fewer
// workgroups would leave CUs idle (one long sample, a few short ones).
constexpr int kRingRowsMax = 64, kRingRowsMin = 16;
constexpr int kRingSlots = 2;
constexpr int ring_waves(int) { return 4; }

template <int DT, int kQ, bool kBias>
__global__ __launch_bounds__(ring_waves(kQ) * kWave, 1) void norm_grad_ring(NormArgs a) {
  static_assert(kQ <= 8, "ring slots are sized for at most 8 KB rows");
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int NW = ring_waves(kQ);
  constexpr int kRowBytes = kQ * kWave * 16;          // one operand's row, padded to kQ KB
  constexpr int kSlot = 2 * kRowBytes;                // x row, then g row
  __shared__ __attribute__((aligned(1024))) char ring[NW * kRingSlots * kSlot];
  // After the rows, the waves combine through the ring's first bytes.
  static_assert((kBias ? 2 : 1) * kQ * kWave * VEC * 4 <= NW * kRingSlots * kSlot, "combine buffer");
  float* const comb = (float*)ring;

  const int64_t b = blockIdx.y, chunk = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int uwave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nchunk16 = a.d / VEC;  // the host sends only widths of whole chunks here (dp == d)
  const float inv_d = 1.f / (float)a.d;
  const u32x4 rx = make_rsrc(a.x + b * a.x_bstride, (uint32_t)(a.tokens * a.x_tstride));
  const u32x4 rg = make_rsrc(a.g + b * a.g_bstride, (uint32_t)(a.tokens * a.g_tstride));
  const uint32_t xts = (uint32_t)a.x_tstride, gts = (uint32_t)a.g_tstride;
  const uint32_t lds_w = (uint32_t)(uintptr_t)(ring + uwave * kRingSlots * kSlot);
  const lds_char* const slot_ptr = (const lds_char*)(ring + uwave * kRingSlots * kSlot);

  const int64_t t_begin = chunk * a.ring_rows;
  const int64_t t_end = min(t_begin + a.ring_rows, a.tokens);
  const int nrows = (int)((t_end - t_begin - uwave + NW - 1) / NW);  // this wave's rows (may be <= 0)

  // Row i of this wave is token t_begin + uwave + NW*i, in slot i % 2.
  auto issue = [&](int i) __attribute__((always_inline)) {
    const bool live = i < nrows;
    const uint32_t t = (uint32_t)(t_begin + uwave + (int64_t)NW * i);
    const uint32_t lbase = lds_w + (uint32_t)((i % kRingSlots) * kSlot);
#pragma unroll
    for (int j = 0; j < kQ; ++j) {
      const bool in = live && lane + (int64_t)j * kWave < nchunk16;
      const uint32_t col = (uint32_t)((lane + j * kWave) * 16);
      dma16_nt(rx, lbase + (uint32_t)(j * kWave * 16), in ? t * xts + col : 0x80000000u);
    }
#pragma unroll
    for (int j = 0; j < kQ; ++j) {
      const bool in = live && lane + (int64_t)j * kWave < nchunk16;
      const uint32_t col = (uint32_t)((lane + j * kWave) * 16);
      dma16_nt(rg, lbase + (uint32_t)(kRowBytes + j * kWave * 16), in ? t * gts + col : 0x80000000u);
    }
  };

  float dg[kQ][VEC], db[kBias ? kQ : 1][VEC];
#pragma unroll
  for (int q = 0; q < kQ; ++q)
#pragma unroll
    for (int e = 0; e < VEC; ++e) dg[q][e] = 0.f;
#pragma unroll
  for (int q = 0; q < (kBias ? kQ : 1); ++q)
#pragma unroll
    for (int e = 0; e < VEC; ++e) db[q][e] = 0.f;

  issue(0);
  for (int i = 0; i < nrows; ++i) {
    // The slot row i + 1 fills held row i - 1, whose reads have returned
    // (lgkmcnt); then row i is awaited, row i + 1's 2*kQ instructions
    // staying in flight.
    __builtin_amdgcn_s_waitcnt(0xC07F);
    issue(i + 1);
    if constexpr (kQ == 1) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    else if constexpr (kQ == 2) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else if constexpr (kQ == 4) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    const lds_char* sx = slot_ptr + (i % kRingSlots) * kSlot;
    u32x4 vx[kQ], vg[kQ];
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      vx[q] = *(const __attribute__((address_space(3))) u32x4*)(sx + (lane + q * kWave) * 16);
      vg[q] = *(const __attribute__((address_space(3))) u32x4*)(sx + kRowBytes + (lane + q * kWave) * 16);
    }
    if (DT != DA_F32 && a.kind != 1) {
      // Zero mean (RMSNorm, or as given): the mean square comes from 16-bit
      // pairs through v_dot2 (both products exact in fp32), and the padding
      // lanes read zeros.
      float ss = 0.f;
      if (a.kind == 0) {
#pragma unroll
        for (int q = 0; q < kQ; ++q)
#pragma unroll
          for (int w = 0; w < 4; ++w) ss = dot2_sq<DT>(vx[q][w], ss);
      }
      const float rstd = a.kind == 2 ? 1.f : 1.f / sqrtf(wave_sum(ss) * inv_d + a.eps);
#pragma unroll
      for (int q = 0; q < kQ; ++q)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float gv = elem_of<DT>(vg[q], e);
          dg[q][e] += (elem_of<DT>(vx[q], e) * rstd) * gv;
          if constexpr (kBias) db[q][e] += gv;
        }
      continue;
    }
    float mean = 0.f;
    if (a.kind == 1) {
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < kQ; ++q)
#pragma unroll
        for (int e = 0; e < VEC; ++e) s += elem_of<DT>(vx[q], e);
      mean = wave_sum(s) * inv_d;
    }
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const bool in = lane + (int64_t)q * kWave < nchunk16;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float c = in ? elem_of<DT>(vx[q], e) - mean : 0.f;
        ss += c * c;
      }
    }
    const float rstd = a.kind == 2 ? 1.f : 1.f / sqrtf(wave_sum(ss) * inv_d + a.eps);
#pragma unroll
    for (int q = 0; q < kQ; ++q)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float gv = elem_of<DT>(vg[q], e);
        dg[q][e] += (elem_of<DT>(vx[q], e) - mean) * rstd * gv;
        if constexpr (kBias) db[q][e] += gv;
      }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the zero-fill loads past the last row
  __syncthreads();  // every wave is done with its slots before they hold the combine buffer

  // Combine the waves in order 0 + 1 + ... through LDS, then wave 0 writes.
  const int64_t width = (1 + a.has_bias) * a.dp;
  for (int w = 1; w < NW; ++w) {
    if (uwave == w) {
#pragma unroll
      for (int q = 0; q < kQ; ++q)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          comb[(q * kWave + lane) * VEC + e] = dg[q][e];
          if constexpr (kBias) comb[(kQ * kWave + q * kWave + lane) * VEC + e] = db[q][e];
        }
    }
    __syncthreads();
    if (uwave == 0) {
#pragma unroll
      for (int q = 0; q < kQ; ++q)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          dg[q][e] += comb[(q * kWave + lane) * VEC + e];
          if constexpr (kBias) db[q][e] += comb[(kQ * kWave + q * kWave + lane) * VEC + e];
        }
    }
    __syncthreads();
  }
  if (uwave == 0) {
    float* dst = a.partial + (b * a.chunks + chunk) * width;
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const int64_t c = lane + (int64_t)q * kWave;
      if (c < nchunk16) {
        *(f32x4*)(dst + c * VEC) = f32x4{dg[q][0], dg[q][1], dg[q][2], dg[q][3]};
        if constexpr (VEC == 8) *(f32x4*)(dst + c * VEC + 4) = f32x4{dg[q][4], dg[q][5], dg[q][6], dg[q][7]};
        if constexpr (kBias) {
          *(f32x4*)(dst + a.d + c * VEC) = f32x4{db[q][0], db[q][1], db[q][2], db[q][3]};
          if constexpr (VEC == 8)
            *(f32x4*)(dst + a.d + c * VEC + 4) = f32x4{db[q][4], db[q][5], db[q][6], db[q][7]};
        }
      }
    }
  }
}

// out[b, f] = sum over the sample's chunk partials in a fixed order: the
// chunks are split into NG consecutive groups, one per wave; within a group
// eight interleaved accumulators run in chunk order and are added in a fixed
// tree, and the group sums are added as (g0 + g1) + (g2 + g3) (NG = 4) or in
// group order (NG = 16, for 128 or more chunks per sample -- one long sample
// -- so that four times the loads are in flight).  The same order on every
// call with the same chunk count.  A lane owns four consecutive features
// (16-byte loads); a workgroup covers 64 feature quads of one sample.  The
// partials hold each block of d features at a pitch of dp (a multiple of 4):
// feature f of block k = f / dp lands at out index k * d + f % dp when
// f % dp < d.
template <int OT, int NG>
__global__ __launch_bounds__(NG * 64) void norm_grad_reduce(const float* __restrict__ partial, int64_t batch,
                                                            int64_t chunks, int64_t width, int64_t d, int64_t dp,
                                                            char* out, int64_t out_bstride) {
  __shared__ f32x4 red[NG - 1][64];
  const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int64_t f = ((int64_t)blockIdx.x * 64 + lane) * 4;
  const int64_t b = blockIdx.y;
  const int64_t per = (chunks + NG - 1) / NG;
  const int64_t c0 = min(chunks, grp * per), c1 = min(chunks, c0 + per);
  f32x4 acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (f < width) {
    const float* p = partial + b * chunks * width + f;
    int64_t c = c0;
    for (; c + 8 <= c1; c += 8)
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[u] += *(const f32x4*)(p + (c + u) * width);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (c + u < c1) acc[u] += *(const f32x4*)(p + (c + u) * width);
  }
  const f32x4 s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  if (grp > 0) red[grp - 1][lane] = s;
  __syncthreads();
  if (grp == 0 && f < width) {
    f32x4 t;
    if constexpr (NG == 4) {
      t = (s + red[0][lane]) + (red[1][lane] + red[2][lane]);
    } else {
      t = s;
#pragma unroll
      for (int w = 0; w < NG - 1; ++w) t += red[w][lane];
    }
    const int64_t k = f / dp, j = f - k * dp;  // dp % 4 == 0: the quad stays in one block
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (j + e < d) Elem<OT>::store(out, b * out_bstride + k * d + j + e, t[e]);
  }
}

// N consecutive outputs in the output dtype through 8- or 16-byte stores,
// each value rounded as Elem<OT>::store rounds it.  dst is aligned to
// min(N * bytes, 16).
template <int OT, int N>
__device__ __forceinline__ void store_chunk(char* dst, const float (&v)[N]) {
  if constexpr (Elem<OT>::kBytes == 2) {
    uint32_t w[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      uint16_t lo, hi;
      if constexpr (OT == DA_BF16) {
        lo = f32_to_bf16_bits(v[2 * i]);
        hi = f32_to_bf16_bits(v[2 * i + 1]);
      } else {
        lo = f32_to_f16_bits(v[2 * i]);
        hi = f32_to_f16_bits(v[2 * i + 1]);
      }
      w[i] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    if constexpr (N == 8) *(u32x4*)dst = u32x4{w[0], w[1], w[2], w[3]};
    else *(u32x2*)dst = u32x2{w[0], w[1]};
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 4) *(f32x4*)(dst + 4 * i) = f32x4{v[i], v[i + 1], v[i + 2], v[i + 3]};
  }
}

// x_hat rows for the preprocess API: one wave per row, same math as above.
template <int DT, int OT, int kQ>
__global__ __launch_bounds__(kThreads) void norm_xhat_rows(const char* x, int64_t rows, int64_t d,
                                                           int64_t x_rstride, int kind, float eps,
                                                           char* out, int64_t out_rstride) {
  constexpr int VEC = Elem<DT>::kVec;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t nchunk16 = (d + VEC - 1) / VEC;  // whole chunks are read; elements past d are masked
  const float inv_d = 1.f / (float)d;
  float xv[kQ][VEC];
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    const int64_t c = lane + (int64_t)q * kWave;
    const u32x4 v = c < nchunk16 ? ld16(x + row * x_rstride + c * 16) : u32x4{0, 0, 0, 0};
    unpack16<DT>(v, xv[q]);
  }
  float mean = 0.f;
  if (kind == 1) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < kQ; ++q)
#pragma unroll
      for (int e = 0; e < VEC; ++e) s += (lane + (int64_t)q * kWave) * VEC + e < d ? xv[q][e] : 0.f;
    mean = wave_sum(s) * inv_d;
  }
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const bool in = (lane + (int64_t)q * kWave) * VEC + e < d;
      const float c = in ? xv[q][e] - mean : 0.f;
      ss += c * c;
    }
  }
  const float rstd = kind == 2 ? 1.f : 1.f / sqrtf(wave_sum(ss) * inv_d + eps);
  constexpr int OS = Elem<OT>::kBytes;
  constexpr int kAlign = VEC * OS < 16 ? VEC * OS : 16;  // the widest store a chunk's outputs take
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    const int64_t c = lane + (int64_t)q * kWave;
    float y[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) y[e] = (xv[q][e] - mean) * rstd;
    char* dst = out + (row * out_rstride + c * VEC) * OS;
    if ((c + 1) * VEC <= d && ((uintptr_t)dst % kAlign) == 0) {
      store_chunk<OT, VEC>(dst, y);  // the chunk's outputs in whole 8- or 16-byte stores
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e)
        if (c * VEC + e < d) Elem<OT>::store(out, row * out_rstride + c * VEC + e, y[e]);
    }
  }
}

// Rows wider than the register forms hold (more than 16 chunks per lane): one
// wave per 32-row token chunk walks each row three times from L2 -- the sum,
// the squared deviations, then x_hat * g added into the chunk's partial row,
// which this wave alone owns (its first row writes it, later rows add), so no
// barrier and no zero fill.  Same fixed orders as the register forms.
template <int DT, bool kBias>
__global__ __launch_bounds__(kWave) void norm_grad_wide(NormArgs a) {
  constexpr int VEC = Elem<DT>::kVec;
  const int lane = threadIdx.x;
  const int64_t b = blockIdx.y, chunk = blockIdx.x;
  const int64_t nchunk16 = a.dp / VEC;
  const float inv_d = 1.f / (float)a.d;
  float* dst = a.partial + (b * a.chunks + chunk) * (1 + a.has_bias) * a.dp;
  const int64_t t_begin = chunk * kRowsPerWG;
  const int64_t t_end = min(t_begin + kRowsPerWG, a.tokens);
  for (int64_t t = t_begin; t < t_end; ++t) {
    const char* xr = a.x + b * a.x_bstride + t * a.x_tstride;
    const char* gr = a.g + b * a.g_bstride + t * a.g_tstride;
    float mean = 0.f;
    if (a.kind == 1) {
      float s = 0.f;
      for (int64_t c = lane; c < nchunk16; c += kWave) {
        const u32x4 v = ld16(xr + c * 16);
#pragma unroll
        for (int e = 0; e < VEC; ++e) s += c * VEC + e < a.d ? elem_of<DT>(v, e) : 0.f;
      }
      mean = wave_sum(s) * inv_d;
    }
    float ss = 0.f;
    for (int64_t c = lane; c < nchunk16; c += kWave) {
      const u32x4 v = ld16(xr + c * 16);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float dv = c * VEC + e < a.d ? elem_of<DT>(v, e) - mean : 0.f;
        ss += dv * dv;
      }
    }
    const float rstd = a.kind == 2 ? 1.f : 1.f / sqrtf(wave_sum(ss) * inv_d + a.eps);
    const bool first = t == t_begin;
    for (int64_t c = lane; c < nchunk16; c += kWave) {
      const u32x4 vx = ld16(xr + c * 16), vg = ld16(gr + c * 16);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const int64_t f = c * VEC + e;
        const float gv = f < a.d ? elem_of<DT>(vg, e) : 0.f;
        const float dg = (elem_of<DT>(vx, e) - mean) * rstd * gv;
        dst[f] = first ? dg : dst[f] + dg;
        if constexpr (kBias) dst[a.dp + f] = first ? gv : dst[a.dp + f] + gv;
      }
    }
  }
}

// x_hat of rows wider than the register form holds: one wave per row, three
// passes from L2.
template <int DT, int OT>
__global__ __launch_bounds__(kThreads) void norm_xhat_wide(const char* x, int64_t rows, int64_t d,
                                                           int64_t x_rstride, int kind, float eps,
                                                           char* out, int64_t out_rstride) {
  constexpr int VEC = Elem<DT>::kVec;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t nchunk16 = (d + VEC - 1) / VEC;
  const float inv_d = 1.f / (float)d;
  const char* xr = x + row * x_rstride;
  float mean = 0.f;
  if (kind == 1) {
    float s = 0.f;
    for (int64_t c = lane; c < nchunk16; c += kWave) {
      const u32x4 v = ld16(xr + c * 16);
#pragma unroll
      for (int e = 0; e < VEC; ++e) s += c * VEC + e < d ? elem_of<DT>(v, e) : 0.f;
    }
    mean = wave_sum(s) * inv_d;
  }
  float ss = 0.f;
  for (int64_t c = lane; c < nchunk16; c += kWave) {
    const u32x4 v = ld16(xr + c * 16);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float dv = c * VEC + e < d ? elem_of<DT>(v, e) - mean : 0.f;
      ss += dv * dv;
    }
  }
  const float rstd = kind == 2 ? 1.f : 1.f / sqrtf(wave_sum(ss) * inv_d + eps);
  for (int64_t c = lane; c < nchunk16; c += kWave) {
    const u32x4 v = ld16(xr + c * 16);
#pragma unroll
    for (int e = 0; e < VEC; ++e)
      if (c * VEC + e < d) Elem<OT>::store(out, row * out_rstride + c * VEC + e, (elem_of<DT>(v, e) - mean) * rstd);
  }
}

int pick_q(int64_t d, int64_t vec) {
  const int64_t per_lane = ((d + vec - 1) / vec + kWave - 1) / kWave;
  if (per_lane <= 1) return 1;
  if (per_lane <= 2) return 2;
  if (per_lane <= 4) return 4;
  if (per_lane <= 8) return 8;
  if (per_lane <= 16) return 16;
  return 0;  // the wide form
}

template <int DT, int OT>
int launch_grad(NormArgs& a, int q, void* out, int64_t out_bstride, hipStream_t st) {
  const int64_t width = (1 + a.has_bias) * a.dp;
  // The ring form addresses a sample's rows with 32-bit buffer offsets and
  // takes rows of whole 16-byte chunks.
  const int64_t max_ts = a.x_tstride > a.g_tstride ? a.x_tstride : a.g_tstride;
  if (q == 0) {
    dim3 grid((unsigned)a.chunks, (unsigned)a.batch);
    if (a.has_bias) norm_grad_wide<DT, true><<<grid, kWave, 0, st>>>(a);
    else norm_grad_wide<DT, false><<<grid, kWave, 0, st>>>(a);
  } else if (q <= 8 && a.tokens * max_ts < (1LL << 31) && a.dp == a.d) {
    // At 8 KB rows a workgroup's ring takes most of a CU's LDS: aim for one
    // workgroup per CU, else two.
    int64_t cus = 0;
    int rc = device_cu_count(&cus);
    if (rc) return rc;
    const int64_t want = cus * (q == 8 ? 1 : 2);
    a.ring_rows = kRingRowsMax;
    while (a.ring_rows > kRingRowsMin && a.batch * ((a.tokens + a.ring_rows - 1) / a.ring_rows) < want)
      a.ring_rows /= 2;
    a.chunks = (a.tokens + a.ring_rows - 1) / a.ring_rows;
    dim3 grid((unsigned)a.chunks, (unsigned)a.batch);
#define DA_NORM_RING(Q)                                       \
  if (a.has_bias)                                             \
    norm_grad_ring<DT, Q, true><<<grid, ring_waves(Q) * kWave, 0, st>>>(a); \
  else                                                                      \
    norm_grad_ring<DT, Q, false><<<grid, ring_waves(Q) * kWave, 0, st>>>(a)
    switch (q) {
      case 1: DA_NORM_RING(1); break;
      case 2: DA_NORM_RING(2); break;
      case 4: DA_NORM_RING(4); break;
      default: DA_NORM_RING(8); break;
    }
#undef DA_NORM_RING
  } else {
    const size_t lds = (size_t)width * sizeof(float);
    dim3 grid((unsigned)a.chunks, (unsigned)a.batch);
#define DA_NORM_Q(Q)                                              \
  if (a.has_bias)                                                 \
    norm_grad_chunks<DT, Q, true><<<grid, kThreads, lds, st>>>(a); \
  else                                                            \
    norm_grad_chunks<DT, Q, false><<<grid, kThreads, lds, st>>>(a)
    switch (q) {
      case 1: DA_NORM_Q(1); break;
      case 2: DA_NORM_Q(2); break;
      case 4: DA_NORM_Q(4); break;
      case 8: DA_NORM_Q(8); break;
      default: DA_NORM_Q(16); break;
    }
#undef DA_NORM_Q
  }
  int rc = check_launch("da_norm_weight_grad(chunks)");
  if (rc) return rc;
  dim3 g2((unsigned)((width / 4 + 63) / 64), (unsigned)a.batch);
  if (a.chunks >= 128)
    norm_grad_reduce<OT, 16><<<g2, 1024, 0, st>>>(a.partial, a.batch, a.chunks, width, a.d, a.dp, (char*)out,
                                                  out_bstride);
  else
    norm_grad_reduce<OT, 4><<<g2, 256, 0, st>>>(a.partial, a.batch, a.chunks, width, a.d, a.dp, (char*)out,
                                                out_bstride);
  return check_launch("da_norm_weight_grad(reduce)");
}

template <int DT, int OT>
int launch_xhat(const void* x, int64_t rows, int64_t d, int64_t x_rstride, int kind, float eps,
                void* out, int64_t out_rstride, int q, hipStream_t st) {
  const unsigned blocks = (unsigned)((rows + kWaves - 1) / kWaves);
  const int64_t xs = x_rstride * Elem<DT>::kBytes;
  if (q == 0) {
    norm_xhat_wide<DT, OT><<<blocks, kThreads, 0, st>>>((const char*)x, rows, d, xs, kind, eps, (char*)out,
                                                        out_rstride);
    return check_launch("da_norm_xhat");
  }
#define DA_XHAT_Q(Q)                                                                       \
  norm_xhat_rows<DT, OT, Q><<<blocks, kThreads, 0, st>>>((const char*)x, rows, d, xs, kind, \
                                                         eps, (char*)out, out_rstride)
  switch (q) {
    case 1: DA_XHAT_Q(1); break;
    case 2: DA_XHAT_Q(2); break;
    case 4: DA_XHAT_Q(4); break;
    case 8: DA_XHAT_Q(8); break;
    default: DA_XHAT_Q(16); break;
  }
#undef DA_XHAT_Q
  return check_launch("da_norm_xhat");
}

int check_common(const char* who, int dtype, int out_dtype, int64_t d, int kind, int* q) {
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype))
    return set_error(DA_ERR_INVALID, "%s: bad dtype", who);
  if (kind < 0 || kind > 2)
    return set_error(DA_ERR_INVALID, "%s: kind must be 0 (RMSNorm), 1 (LayerNorm) or 2 (normalised)", who);
  const int64_t vec = 16 / (int64_t)elem_bytes(dtype);
  if (d <= 0) return set_error(DA_ERR_INVALID, "%s: d=%lld must be positive", who, (long long)d);
  *q = pick_q(d, vec);
  return DA_OK;
}

}  // namespace
}  // namespace da

extern "C" {

int da_norm_weight_grad_workspace(int64_t batch, int64_t tokens, int64_t d, int has_bias,
                                  size_t* bytes) {
  if (batch < 0 || tokens < 0 || d < 0 || !bytes)
    return da::set_error(DA_ERR_INVALID, "da_norm_weight_grad_workspace: bad arguments");
  // chunks of the shortest token run any form gives a workgroup
  const int64_t chunks = (tokens + da::kRingRowsMin - 1) / da::kRingRowsMin;
  const int64_t dp = (d + 7) / 8 * 8;  // whole 16-byte chunks of the narrowest element (2 bytes)
  *bytes = (size_t)(batch * chunks * (1 + (has_bias ? 1 : 0)) * dp) * sizeof(float);
  return DA_OK;
}

int da_norm_weight_grad(const void* x, const void* g, int dtype, int64_t batch, int64_t tokens,
                        int64_t d, int64_t x_bstride, int64_t x_tstride, int64_t g_bstride,
                        int64_t g_tstride, int kind, float eps, int has_bias, void* out,
                        int out_dtype, int64_t out_bstride, void* workspace,
                        size_t workspace_bytes, void* stream) {
  using namespace da;
  int q;
  int rc = check_common("da_norm_weight_grad", dtype, out_dtype, d, kind, &q);
  if (rc) return rc;
  if (batch < 0 || tokens < 0) return set_error(DA_ERR_INVALID, "da_norm_weight_grad: negative size");
  if (batch == 0) return DA_OK;
  if (tokens == 0) return set_error(DA_ERR_INVALID, "da_norm_weight_grad: tokens must be >= 1");
  if (!x || !g || !out) return set_error(DA_ERR_INVALID, "da_norm_weight_grad: NULL pointer");
  const int64_t es = (int64_t)elem_bytes(dtype);
  if (((uintptr_t)x | (uintptr_t)g) & 15 ||
      ((x_bstride * es) | (x_tstride * es) | (g_bstride * es) | (g_tstride * es)) % 16)
    return set_error(DA_ERR_INVALID, "da_norm_weight_grad: rows must be 16-byte aligned");
  const int bias = has_bias ? 1 : 0;
  if (out_bstride < (1 + bias) * d)
    return set_error(DA_ERR_INVALID, "da_norm_weight_grad: out batch stride too small");
  size_t need = 0;
  da_norm_weight_grad_workspace(batch, tokens, d, bias, &need);
  if (!workspace || workspace_bytes < need)
    return set_error(DA_ERR_WORKSPACE, "da_norm_weight_grad: workspace needs %zu bytes", need);
  NormArgs a;
  a.x = (const char*)x;
  a.g = (const char*)g;
  a.batch = batch;
  a.tokens = tokens;
  a.d = d;
  a.dp = (d + 16 / es - 1) / (16 / es) * (16 / es);
  a.x_bstride = x_bstride * es;
  a.x_tstride = x_tstride * es;
  a.g_bstride = g_bstride * es;
  a.g_tstride = g_tstride * es;
  a.kind = kind;
  a.eps = eps;
  a.has_bias = bias;
  a.chunks = (tokens + kRowsPerWG - 1) / kRowsPerWG;
  a.ring_rows = 0;
  a.partial = (float*)workspace;
  hipStream_t st = (hipStream_t)stream;
#define DA_NG(DT)                                                                  \
  switch (out_dtype) {                                                             \
    case DA_F32: return launch_grad<DT, DA_F32>(a, q, out, out_bstride, st);       \
    case DA_BF16: return launch_grad<DT, DA_BF16>(a, q, out, out_bstride, st);     \
    default: return launch_grad<DT, DA_F16>(a, q, out, out_bstride, st);           \
  }
  switch (dtype) {
    case DA_BF16: DA_NG(DA_BF16)
    case DA_F16: DA_NG(DA_F16)
    default: DA_NG(DA_F32)
  }
#undef DA_NG
}

int da_norm_xhat(const void* x, int dtype, int64_t rows, int64_t d, int64_t x_rstride, int kind,
                 float eps, void* out, int out_dtype, int64_t out_rstride, void* stream) {
  using namespace da;
  int q;
  int rc = check_common("da_norm_xhat", dtype, out_dtype, d, kind, &q);
  if (rc) return rc;
  if (rows < 0) return set_error(DA_ERR_INVALID, "da_norm_xhat: negative rows");
  if (rows == 0) return DA_OK;
  if (!x || !out) return set_error(DA_ERR_INVALID, "da_norm_xhat: NULL pointer");
  const int64_t es = (int64_t)elem_bytes(dtype);
  if (((uintptr_t)x & 15) || (x_rstride * es) % 16)
    return set_error(DA_ERR_INVALID, "da_norm_xhat: rows must be 16-byte aligned");
  if (out_rstride < d) return set_error(DA_ERR_INVALID, "da_norm_xhat: out row stride too small");
  hipStream_t st = (hipStream_t)stream;
#define DA_XH(DT)                                                                                 \
  switch (out_dtype) {                                                                            \
    case DA_F32: return launch_xhat<DT, DA_F32>(x, rows, d, x_rstride, kind, eps, out, out_rstride, q, st);   \
    case DA_BF16: return launch_xhat<DT, DA_BF16>(x, rows, d, x_rstride, kind, eps, out, out_rstride, q, st); \
    default: return launch_xhat<DT, DA_F16>(x, rows, d, x_rstride, kind, eps, out, out_rstride, q, st);       \
  }
  switch (dtype) {
    case DA_BF16: DA_XH(DA_BF16)
    case DA_F16: DA_XH(DA_F16)
    default: DA_XH(DA_F32)
  }
#undef DA_XH
}

}  // extern "C"
