// K2c: per-sample weight gradient of a linear layer on gfx950 MFMA.
//
//   dW[b, o, k] = sum_t g[b, t, o] * a[b, t, k]          (b < B, o < D, k < K)
//   dW[b, o, K] = sum_t g[b, t, o]                        (only with has_bias)
//
// Follows materialize_factors for linear layers,
// dattri_llm/gradient/ops/materialize.py:114-116 (torch.bmm(g^T, a) flattened
// to (B, out*in), index o*K + i), with the bias folded as the ones column of
// preprocess.py:436-437 (so the layout is (B, D, K+1)).
//
// Both operands contract over the token axis, which is the slow (row) axis of
// the row-major captures.  Each stage therefore loads 8x8 (bf16/f16) or 4x4
// (fp32) blocks with 16-byte row loads, transposes them in registers and
// stores them into LDS token-contiguous, so the MFMA fragment reads are single
// 16-byte LDS reads.  Consecutive lanes take consecutive token blocks of one
// column block, so the 8 lanes the LDS serves together write one 128-byte row
// (all banks distinct); mapping them to consecutive column blocks instead puts
// their rows 8 apart and folds them onto two bank groups.  A workgroup owns a 128 (o) x 128 (k) output tile of one
// sample; the fp32 accumulators are converted to the output dtype and staged
// through LDS so the tile leaves as coalesced 16-byte row stores.
#include <atomic>

#include "common.h"

namespace da {
namespace {

constexpr int kBM = 128;                 // output rows (o) per tile
constexpr int kBN = 128;                 // output cols (k) per tile
constexpr int kRowBytes = 128;           // token bytes per LDS row and stage
constexpr int kLdsRow = kRowBytes + 16;  // padded LDS row
constexpr int kThreads = 256;
constexpr int kGroup = 8;
constexpr int kStageBytes = (kBM + kBN) * kLdsRow;

struct MatArgs {
  const char* a;
  const char* g;
  int64_t batch, tokens, k, d;               // k, d: element widths of a, g
  int64_t a_bstride, a_tstride;              // bytes
  int64_t g_bstride, g_tstride;              // bytes
  char* out;
  int64_t out_bstride, out_rstride;          // elements
  int64_t out_blk;                           // elements between 64-element output blocks
  int64_t tiles_m, tiles_n;                  // per sample
  int sym;                                   // a == g (a row Gram): only tiles on or above the diagonal
  int acc;                                   // add to the fp32 output instead of overwriting it
  int64_t rows_total;                        // sym with token splits: rows of all splits (sample b holds
                                             // rows b*tokens .. ; the last one may be short), else 0
  int64_t tile0, sym_count;                  // sym: triangle tiles tile0 .. tile0 + sym_count - 1 (row by row)
  int compact;                               // sym: tile t of split b lands at out + (b*sym_count + t) * 256^2
};

// Element offset (from the sample's base) of output (o, k): flat c = o*rstride + k
// stored in 64-element blocks out_blk apart (out_blk == 64: plain row-major).
__device__ __forceinline__ int64_t out_index(const MatArgs& m, int64_t o, int64_t k) {
  const int64_t c = o * m.out_rstride + k;
  return (c >> 6) * m.out_blk + (c & 63);
}

// Transpose a VEC x VEC block held as VEC rows of one 16-byte chunk each.
template <int DT>
__device__ __forceinline__ void transpose_block(const u32x4 (&in)[Elem<DT>::kVec],
                                                u32x4 (&out)[Elem<DT>::kVec]) {
  if constexpr (DT == DA_F32) {
#pragma unroll
    for (int c = 0; c < 4; ++c) out[c] = u32x4{in[0][c], in[1][c], in[2][c], in[3][c]};
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int w = c >> 1;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const uint32_t lo = in[2 * p][w], hi = in[2 * p + 1][w];
        out[c][p] = (c & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
      }
    }
  }
}

template <int DT, int OT, bool kAlignedOut>
__global__ __launch_bounds__(kThreads, 2) void materialize_tiles(MatArgs m) {
  constexpr int VEC = Elem<DT>::kVec;           // elements per 16-byte chunk
  constexpr int ES = Elem<DT>::kBytes;
  constexpr int TS = kRowBytes / ES;            // tokens per stage
  constexpr int BLK_T = TS / VEC;               // token blocks per stage
  constexpr int BLK_C = kBM / VEC;              // column blocks per operand tile
  constexpr int BLOCKS = BLK_T * BLK_C;         // blocks per operand per stage
  constexpr int PER_THREAD = BLOCKS / (kThreads / 2);
  static_assert(PER_THREAD >= 1 && BLOCKS % (kThreads / 2) == 0, "stage/block mismatch");

  __shared__ __attribute__((aligned(16))) char smem[2 * kStageBytes];

  const int64_t ntiles = (int64_t)gridDim.x;
  const int64_t logical = xcd_remap(blockIdx.x, ntiles);
  const int64_t per_sample = m.tiles_m * m.tiles_n;
  const int64_t b = logical / per_sample;
  const int64_t rem = logical - b * per_sample;
  // swizzle inside the sample: groups of kGroup row tiles sweep the columns
  const int64_t per_group = (int64_t)kGroup * m.tiles_n;
  const int64_t group = rem / per_group;
  const int64_t first = group * kGroup;
  const int64_t gsize = min(m.tiles_m - first, (int64_t)kGroup);
  const int64_t in_group = rem - group * per_group;
  const int64_t tm = first + in_group % gsize;
  const int64_t tn = in_group / gsize;
  const int64_t o0 = tm * kBM, k0 = tn * kBN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // This thread stages operand `side` (0: g -> rows o, 1: a -> rows k).
  const int side = tid / (kThreads / 2);
  const int tsub = tid % (kThreads / 2);
  const char* src = side == 0 ? m.g + b * m.g_bstride : m.a + b * m.a_bstride;
  const int64_t tstride = side == 0 ? m.g_tstride : m.a_tstride;
  const int64_t width = side == 0 ? m.d : m.k;
  const int64_t c0 = side == 0 ? o0 : k0;

  u32x4 blk[PER_THREAD][VEC];
  auto gload = [&](int st) {
#pragma unroll
    for (int q = 0; q < PER_THREAD; ++q) {
      const int bi = tsub + q * (kThreads / 2);
      const int bt = bi % BLK_T, bc = bi / BLK_T;
      const int64_t col = c0 + (int64_t)bc * VEC;
      const bool cin = col < width;
#pragma unroll
      for (int r = 0; r < VEC; ++r) {
        const int64_t t = (int64_t)st * TS + bt * VEC + r;
        blk[q][r] = (cin && t < m.tokens) ? ld16(src + t * tstride + col * ES) : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto lstore = [&](int buf) {
    char* base = smem + buf * kStageBytes + (side == 0 ? 0 : kBM * kLdsRow);
#pragma unroll
    for (int q = 0; q < PER_THREAD; ++q) {
      const int bi = tsub + q * (kThreads / 2);
      const int bt = bi % BLK_T, bc = bi / BLK_T;
      u32x4 tr[VEC];
      transpose_block<DT>(blk[q], tr);
#pragma unroll
      for (int c = 0; c < VEC; ++c) st16(base + (bc * VEC + c) * kLdsRow + bt * 16, tr[c]);
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) acc[x][y] = f32x16{};

  const int nst = (int)((m.tokens + TS - 1) / TS);
  gload(0);
  lstore(0);
  __syncthreads();
  const int frow = lane & 31, fhalf = lane >> 5;
  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    if (st + 1 < nst) gload(st + 1);
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
    if (st + 1 < nst) lstore(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: each wave stages its 64x64 output block (output dtype) in LDS,
  // then writes whole rows.  The loop above ended with a barrier, so the
  // stage buffers are free.
  constexpr int OS = Elem<OT>::kBytes;
  constexpr int ROWB = 64 * OS;                   // bytes of one staged row
  char* wbuf = smem + wave * (64 * ROWB);
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = 32 * x + acc_row(r, lane), col = 32 * y + acc_col(lane);
        Elem<OT>::store(wbuf, (int64_t)row * 64 + col, acc[x][y][r]);
      }
  __syncthreads();
  const int64_t orow0 = o0 + 64 * wm, ocol0 = k0 + 64 * wn;
  char* obase = m.out + (b * m.out_bstride) * OS;
  if constexpr (kAlignedOut) {
    constexpr int CH = ROWB / 16;                 // 16-byte chunks per row
    constexpr int ROWS_PER_PASS = 64 / CH;
#pragma unroll
    for (int pass = 0; pass < 64 / ROWS_PER_PASS; ++pass) {
      const int row = pass * ROWS_PER_PASS + lane / CH, ch = lane % CH;
      const int64_t orow = orow0 + row;
      const int64_t ocol = ocol0 + (int64_t)ch * (16 / OS);
      if (orow < m.d && ocol < m.k)
        st16(obase + out_index(m, orow, ocol) * OS, ld16(wbuf + row * ROWB + ch * 16));
    }
  } else {
    for (int e = lane; e < 64 * 64; e += 64) {
      const int row = e >> 6, col = e & 63;
      const int64_t orow = orow0 + row, ocol = ocol0 + col;
      if (orow < m.d && ocol < m.k) {
        if constexpr (OS == 4)
          ((uint32_t*)obase)[out_index(m, orow, ocol)] = ((const uint32_t*)wbuf)[e];
        else
          ((uint16_t*)obase)[out_index(m, orow, ocol)] = ((const uint16_t*)wbuf)[e];
      }
    }
  }
}

// Large-tile variant for the big layers: a 256 (o) x 256 (k) tile per
// workgroup, one wave per SIMD, each wave a 128 x 128 block (4 x 4 MFMA blocks,
// 256 fp32 accumulators).  Twice the MFMA work per LDS byte of the 128-tile
// kernel and four times the work per stage to hide the next stage's loads.
namespace big {
constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kStageBytes = (kBM + kBN) * kLdsRow;  // 73,728 B; two stages fit LDS
}  // namespace big

template <int DT, int OT>
__global__ __launch_bounds__(kThreads, 1) void materialize_tiles_big(MatArgs m) {
  constexpr int VEC = Elem<DT>::kVec;
  constexpr int ES = Elem<DT>::kBytes;
  constexpr int TS = kRowBytes / ES;           // tokens per stage
  constexpr int BLK_T = TS / VEC;              // token blocks per stage
  constexpr int BLK_C = big::kBM / VEC;        // column blocks per operand tile
  constexpr int BLOCKS = BLK_T * BLK_C;        // blocks per operand per stage
  constexpr int PER_THREAD = BLOCKS / (kThreads / 2);
  static_assert(PER_THREAD >= 1 && BLOCKS % (kThreads / 2) == 0, "stage/block mismatch");

  extern __shared__ __attribute__((aligned(16))) char smem[];  // 2 * big::kStageBytes

  const int64_t ntiles = (int64_t)gridDim.x;
  const int64_t logical = xcd_remap(blockIdx.x, ntiles);
  const int64_t per_sample = m.tiles_m * m.tiles_n;
  const int64_t b = logical / per_sample;
  const int64_t rem = logical - b * per_sample;
  const int64_t per_group = (int64_t)kGroup * m.tiles_n;
  const int64_t group = rem / per_group;
  const int64_t first = group * kGroup;
  const int64_t gsize = min(m.tiles_m - first, (int64_t)kGroup);
  const int64_t in_group = rem - group * per_group;
  const int64_t tm = first + in_group % gsize;
  const int64_t tn = in_group / gsize;
  const int64_t o0 = tm * big::kBM, k0 = tn * big::kBN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int side = tid / (kThreads / 2);
  const int tsub = tid % (kThreads / 2);
  const char* src = side == 0 ? m.g + b * m.g_bstride : m.a + b * m.a_bstride;
  const int64_t tstride = side == 0 ? m.g_tstride : m.a_tstride;
  const int64_t width = side == 0 ? m.d : m.k;
  const int64_t c0 = side == 0 ? o0 : k0;

  u32x4 blk[PER_THREAD][VEC];
  auto gload = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < PER_THREAD; ++q) {
      const int bi = tsub + q * (kThreads / 2);
      const int bt = bi % BLK_T, bc = bi / BLK_T;
      const int64_t col = c0 + (int64_t)bc * VEC;
      const bool cin = col < width;
#pragma unroll
      for (int r = 0; r < VEC; ++r) {
        const int64_t t = (int64_t)st * TS + bt * VEC + r;
        blk[q][r] = (cin && t < m.tokens) ? ld16(src + t * tstride + col * ES) : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto lstore = [&](int buf) __attribute__((always_inline)) {
    char* base = smem + buf * big::kStageBytes + (side == 0 ? 0 : big::kBM * kLdsRow);
#pragma unroll
    for (int q = 0; q < PER_THREAD; ++q) {
      const int bi = tsub + q * (kThreads / 2);
      const int bt = bi % BLK_T, bc = bi / BLK_T;
      u32x4 tr[VEC];
      transpose_block<DT>(blk[q], tr);
#pragma unroll
      for (int c = 0; c < VEC; ++c) st16(base + (bc * VEC + c) * kLdsRow + bt * 16, tr[c]);
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y) acc[x][y] = f32x16{};

  const int nst = (int)((m.tokens + TS - 1) / TS);
  gload(0);
  lstore(0);
  __syncthreads();
  const int frow = lane & 31, fhalf = lane >> 5;
  for (int st = 0; st < nst; ++st) {
    const int buf = st & 1;
    if (st + 1 < nst) gload(st + 1);
    const char* base = smem + buf * big::kStageBytes;
#pragma unroll
    for (int kg = 0; kg < kRowBytes / 32; ++kg) {
      u32x4 fa[4], fb[4];
#pragma unroll
      for (int x = 0; x < 4; ++x)
        fa[x] = ld16(base + (128 * wm + 32 * x + frow) * kLdsRow + 32 * kg + 16 * fhalf);
#pragma unroll
      for (int y = 0; y < 4; ++y)
        fb[y] = ld16(base + (big::kBM + 128 * wn + 32 * y + frow) * kLdsRow + 32 * kg + 16 * fhalf);
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y) Mfma32<DT>::mma(acc[x][y], fa[x], fb[y]);
    }
    if (st + 1 < nst) lstore(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: each wave stages its 128 x 128 block in LDS (output dtype), in
  // passes of kPassRows rows so fp32 fits, and writes whole 16-byte chunks.
  constexpr int OS = Elem<OT>::kBytes;
  constexpr int kPassRows = OS == 4 ? 64 : 128;
  constexpr int ROWB = 128 * OS;
  char* wbuf = smem + wave * (kPassRows * ROWB);
  const int64_t orow0 = o0 + 128 * wm, ocol0 = k0 + 128 * wn;
  char* obase = m.out + (b * m.out_bstride) * OS;
#pragma unroll
  for (int pass = 0; pass < 128 / kPassRows; ++pass) {
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      if ((32 * x) / kPassRows != pass) continue;
#pragma unroll
      for (int y = 0; y < 4; ++y)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = 32 * x + acc_row(r, lane) - pass * kPassRows, col = 32 * y + acc_col(lane);
          Elem<OT>::store(wbuf, (int64_t)row * 128 + col, acc[x][y][r]);
        }
    }
    __syncthreads();
    constexpr int CH = ROWB / 16;
    constexpr int RPP = 64 / CH;  // rows per 64-lane pass
    for (int rr = 0; rr < kPassRows; rr += RPP) {
      const int row = rr + lane / CH, ch = lane % CH;
      const int64_t orow = orow0 + pass * kPassRows + row;
      const int64_t ocol = ocol0 + (int64_t)ch * (16 / OS);
      if (orow < m.d && ocol < m.k)
        st16(obase + out_index(m, orow, ocol) * OS, ld16(wbuf + row * ROWB + ch * 16));
    }
    __syncthreads();
  }
}

// Transposing-read variant for 2-byte inputs (bf16 / f16), used for the large
// layers.  Operand tiles go from HBM to LDS untouched, by buffer loads with the
// LDS-direct bit (16 bytes per lane, nothing staged in VGPRs), and the MFMA
// fragments come out of LDS token-contiguous through ds_read_b64_tr_b16: within
// each 16-lane group, lane j addresses 4 consecutive columns of token row
// (r0 + j/4) and lane i receives tokens r0..r0+3 of column i.  Rows past the
// sample's last token and columns past the width read as zero through the
// buffer range check.  The ring holds four 32-token stages, three in flight
// while the fourth is multiplied (a fifth stage, all 160 KB of LDS, measured
// slower).
namespace trk {
constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kGroup = 4;                   // row tiles per column sweep (4 beat 8 and 16 on the C4 dW shapes)
constexpr int kTS = 32;                     // tokens per stage
constexpr int kRow = 512;                   // bytes per token row of a 256-column operand tile
constexpr int kOp = kTS * kRow;             // 16 KB per operand per stage
constexpr int kStage = 2 * kOp;             // g tile, then a tile
constexpr int kNBuf = 4;                    // ring of stages: 128 KB
constexpr int kDma = kTS * (kRow / 16) / (kWave * 4);  // DMA instructions per wave, operand and stage
constexpr uint32_t kOob = 0x80000000u;      // offset past every range: the load returns zeros
static_assert(kDma == 4, "the vmcnt wait assumes 8 DMA instructions per wave and stage");
// 16-byte chunk c of token row r is stored in slot c ^ swz(r).  One transposing
// read touches 8 token rows (r % 4 = 0..3, twice) x 64 bytes; the swizzle puts
// the four rows of each half in different 64-byte quarters of a 256-byte bank
// sweep.
__device__ __forceinline__ int swz(int r) { return (r & 3) << 2; }
}  // namespace trk

typedef short s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 tr_frag(const lds_char* p0, const lds_char* p1) {
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p0);
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p1);
  const u32x2 l = __builtin_bit_cast(u32x2, lo), h = __builtin_bit_cast(u32x2, hi);
  return u32x4{l[0], l[1], h[0], h[1]};
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Store 4 consecutive outputs in the output dtype (round to nearest even).
template <int OT>
__device__ __forceinline__ void store_run4(char* p, float a, float b, float c, float d) {
  if constexpr (OT == DA_F32) {
    *(f32x4*)p = f32x4{a, b, c, d};
  } else if constexpr (OT == DA_BF16) {
    *(u32x2*)p = u32x2{__builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2)),
                       __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{c, d}, bf16x2))};
  } else {
    *(u32x2*)p = u32x2{__builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2)),
                       __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{c, d}, f16x2))};
  }
}

template <int DT, int OT>
__global__ __launch_bounds__(kThreads, 1) void materialize_tiles_tr(MatArgs m) {
  static_assert(Elem<DT>::kBytes == 2, "transposing reads are 16-bit");
  __shared__ __attribute__((aligned(1024))) char smem[trk::kNBuf * trk::kStage];
  lds_char* const L = (lds_char*)smem;
  const uint32_t lds0 = (uint32_t)(uintptr_t)L;

  const int64_t ntiles = (int64_t)gridDim.x;
  const int64_t logical = xcd_remap(blockIdx.x, ntiles);
  int64_t b, tm, tn;
  int64_t sym_local = 0;
  if (m.sym) {
    // Sample b (a token split of the rows), then its tiles tile0 + .. of the
    // triangle tm <= tn, numbered row by row (tiles_m == tiles_n).
    b = logical / m.sym_count;
    sym_local = logical - b * m.sym_count;
    int64_t r = m.tile0 + sym_local;
    tm = 0;
    while (r >= m.tiles_n - tm) {
      r -= m.tiles_n - tm;
      ++tm;
    }
    tn = tm + r;
  } else {
    // When every sample's tile count divides by 8, XCD x takes the x-th
    // eighth of each sample in turn, so all XCDs stream one sample's factors
    // at a time (a working set the MALL keeps); otherwise XCD x takes the
    // x-th eighth of all tiles.  Within an XCD, the tiles running together
    // are consecutive in the grouped order below.
    const int64_t per_sample = m.tiles_m * m.tiles_n;
    int64_t rem;
    if (per_sample % kXcds == 0) {
      const int64_t chunk = per_sample / kXcds;
      const int64_t xcd = blockIdx.x % kXcds, local = blockIdx.x / kXcds;
      b = local / chunk;
      rem = xcd * chunk + local % chunk;
    } else {
      b = logical / per_sample;
      rem = logical - b * per_sample;
    }
    const int64_t per_group = (int64_t)trk::kGroup * m.tiles_n;
    const int64_t group = rem / per_group;
    const int64_t first = group * trk::kGroup;
    const int64_t gsize = min(m.tiles_m - first, (int64_t)trk::kGroup);
    const int64_t in_group = rem - group * per_group;
    tm = first + in_group % gsize;
    tn = in_group / gsize;
  }
  const int64_t o0 = tm * trk::kBM, k0 = tn * trk::kBN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int uwave = __builtin_amdgcn_readfirstlane(wave);  // wave-uniform, for M0

  // Buffer resources over the sample's token rows (the host guarantees
  // (tokens + kTS) * stride < 2^31, so no offset below wraps).
  // A token split's resources end at the last real row: the rows past it
  // (the short last split) read as zeros and touch no memory.
  const int64_t tok_b = m.rows_total > 0 ? min(m.tokens, m.rows_total - b * m.tokens) : m.tokens;
  const u32x4 rg = make_rsrc(m.g + b * m.g_bstride, (uint32_t)(tok_b * m.g_tstride));
  const u32x4 ra = make_rsrc(m.a + b * m.a_bstride, (uint32_t)(tok_b * m.a_tstride));
  const uint32_t gts = (uint32_t)m.g_tstride, ats = (uint32_t)m.a_tstride;

  const int nst = (int)((tok_b + trk::kTS - 1) / trk::kTS);
  // DMA: wave w fills token rows 8w .. 8w+7 of both operand tiles, two rows per
  // instruction; lane l takes row 8w + 2j + l/32 and slot l % 32.
  uint32_t goff[trk::kDma], aoff[trk::kDma];
#pragma unroll
  for (int j = 0; j < trk::kDma; ++j) {
    const int r = 8 * wave + 2 * j + (lane >> 5);
    const int c = (lane & 31) ^ trk::swz(r);
    const int64_t gc = o0 + 8 * c, ac = k0 + 8 * c;
    goff[j] = gc < m.d ? (uint32_t)(r * gts + gc * 2) : trk::kOob;
    aoff[j] = ac < m.k ? (uint32_t)(r * ats + ac * 2) : trk::kOob;
  }
  // One operand's 4 DMA instructions of stage st (side 0: g tile, 1: a tile);
  // j selects the instruction.  A stage past the last still issues them, with
  // an offset past the range (no memory is read; its ring slot, which no one
  // reads, is filled with zeros), so every stage slot issues the same 8
  // instructions per wave and the vmcnt wait below is one constant.
  auto dma_one = [&](int side, int st, int j) __attribute__((always_inline)) {
    const bool en = st < nst;
    const uint32_t lbase = lds0 + (uint32_t)((st % trk::kNBuf) * trk::kStage + side * trk::kOp +
                                             (8 * uwave + 2 * j) * trk::kRow);
    const uint32_t step = (uint32_t)st * (trk::kTS * (side == 0 ? gts : ats));
    const uint32_t off = (side == 0 ? goff[j] : aoff[j]) + step;
    dma16(side == 0 ? rg : ra, lbase, en ? off : trk::kOob);
  };
  auto issue = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < trk::kDma; ++j) dma_one(0, st, j);
#pragma unroll
    for (int j = 0; j < trk::kDma; ++j) dma_one(1, st, j);
  };

  // Fragment addresses: lane (q = lane/16, i = lane%16) reads token row
  // 16*kk + 8*(q/2) + 4*h + i/4 and columns W0 + 32f + 16*(q%2) + 4*(i%4) .. +3.
  const int q = lane >> 4, i16 = lane & 15;
  const int rsw = (i16 >> 2) << 2;  // swz() of that row: row % 4 == i16 / 4
  const int rowoff = (8 * (q >> 1) + (i16 >> 2)) * trk::kRow;
  int gfr[4], afr[4];
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int cg = (128 * wm + 32 * f) / 8 + 2 * (q & 1) + ((i16 & 3) >> 1);
    const int ca = (128 * wn + 32 * f) / 8 + 2 * (q & 1) + ((i16 & 3) >> 1);
    gfr[f] = rowoff + ((cg ^ rsw) << 4) + 8 * (i16 & 1);
    afr[f] = trk::kOp + rowoff + ((ca ^ rsw) << 4) + 8 * (i16 & 1);
  }

  f32x16 acc[4][4];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y) acc[x][y] = f32x16{};

  static_assert(trk::kTS == 32, "the loop below multiplies two 16-token slices per stage");
  u32x4 f0a[4], f0b[4], f1a[4], f1b[4];
  auto read = [&](const lds_char* sb, u32x4 (&fa)[4], u32x4 (&fb)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int f = 0; f < 4; ++f) fa[f] = tr_frag(sb + gfr[f], sb + gfr[f] + 4 * trk::kRow);
#pragma unroll
    for (int f = 0; f < 4; ++f) fb[f] = tr_frag(sb + afr[f], sb + afr[f] + 4 * trk::kRow);
  };
  // acc[x][y] holds the transposed 32x32 block: its MFMA rows are the k
  // columns (a tile) and its MFMA columns the o rows (g tile), so each lane ends
  // with 4 consecutive k of one o -- one short contiguous store per 4 values.
  auto mma = [&](const u32x4 (&fa)[4], const u32x4 (&fb)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
      for (int y = 0; y < 4; ++y) Mfma32<DT>::mma(acc[x][y], fb[y], fa[x]);
  };
  // Wait until this wave's loads of a stage are done -- the 8 * (kNBuf - 2)
  // instructions issued after them may still be in flight -- and its own LDS
  // reads have returned, then barrier: every wave's
  // part of the stage is visible and the buffer read before the barrier may be
  // refilled.  The LDS wait is the compiler's own s_waitcnt (lgkmcnt(0), all
  // other counters at their maximum) so it knows the fragments are complete.
  auto stage_sync = [&]() __attribute__((always_inline)) {
    static_assert(trk::kNBuf == 4, "vmcnt below is 8 * (kNBuf - 2)");
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("s_barrier" ::: "memory");
  };
  // Half a stage: the 16 MFMAs of one 16-token slice held in (ua, ub), the 16
  // transposing reads of the next slice into (na, nb), and one operand's 4 DMA
  // instructions of a later stage, interleaved one read per MFMA and one DMA
  // per 4 MFMAs.  Issuing a stage's loads in one burst fills the address
  // FIFO, and the stalled wave then cannot issue MFMAs either.
  auto half = [&](const u32x4 (&ua)[4], const u32x4 (&ub)[4], const lds_char* sb, u32x4 (&na)[4],
                  u32x4 (&nb)[4], int side, int dst) __attribute__((always_inline)) {
    s16x4 t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int fr = i >> 1;
      const int fo = fr < 4 ? gfr[fr] : afr[fr - 4];
      t[i] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(sb + fo + (i & 1) * 4 * trk::kRow));
      Mfma32<DT>::mma(acc[i >> 2][i & 3], ub[i & 3], ua[i >> 2]);
      if ((i & 3) == 2 && side >= 0) dma_one(side, dst, i >> 2);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const u32x2 lo = __builtin_bit_cast(u32x2, t[2 * f]), hi = __builtin_bit_cast(u32x2, t[2 * f + 1]);
      (f < 4 ? na[f] : nb[f - 4]) = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  };

  // Software pipeline over 16-token slices: the second slice of stage st is
  // multiplied after the barrier that opens stage st + 1 while the first slice
  // of st + 1 is read, so the MFMA pipe does not drain at barriers.  Stage
  // st + kNBuf - 1's a-tile loads go out in the first half of iteration st,
  // stage st + kNBuf's g-tile loads in the second half.
#pragma unroll
  for (int s = 0; s < trk::kNBuf - 1; ++s) issue(s);
  stage_sync();
#pragma unroll
  for (int j = 0; j < trk::kDma; ++j) dma_one(0, trk::kNBuf - 1, j);
  read(L, f0a, f0b);
  for (int st = 0; st + 1 < nst; ++st) {
    half(f0a, f0b, L + (st % trk::kNBuf) * trk::kStage + 16 * trk::kRow, f1a, f1b, 1, st + trk::kNBuf - 1);
    stage_sync();
    half(f1a, f1b, L + ((st + 1) % trk::kNBuf) * trk::kStage, f0a, f0b, 0, st + trk::kNBuf);
  }
  // Last stage (peeled, so no branch joins the loop's MFMA groups).
  half(f0a, f0b, L + ((nst - 1) % trk::kNBuf) * trk::kStage + 16 * trk::kRow, f1a, f1b, -1, 0);
  mma(f1a, f1b);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // Epilogue: lane l of acc[x][y] holds row o = 32x + l%32 and columns
  // k = 32y + 8q + 4*(l/32) + (0..3) in acc[x][y][4q .. 4q+3].  Per 32-row
  // group x, each wave converts in pairs (v_cvt_pk_*), writes its 32 x 128
  // block into its own padded LDS rows (one 8- or 16-byte write per run of 4),
  // and stores whole 16-byte chunks of each row.  No other wave touches that
  // LDS region, so only the loop's final barrier (ring reads done) is needed.
  // (Storing the runs of 4 straight to HBM puts the 32 rows of one
  // instruction a row stride apart; at 8 KB strides they serialize on one
  // memory channel.)
  constexpr int OS = Elem<OT>::kBytes;
  constexpr int ROWB = 128 * OS;           // bytes of one staged row
  constexpr int LROW = ROWB + 16;          // padded LDS row
  constexpr int CH = ROWB / 16;            // 16-byte chunks per row
  constexpr int RPI = kWave / CH;          // rows per store instruction
  static_assert(4 * 32 * LROW <= (int)sizeof(smem), "epilogue staging exceeds the ring");
  char* wbuf = smem + wave * (32 * LROW);
  const int h = lane >> 5, ol = lane & 31;
  const int64_t ocol0 = k0 + 128 * wn;
  char* obase = m.out + (b * m.out_bstride) * OS;
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
  for (int x = 0; x < 4; ++x) {
#pragma unroll
    for (int y = 0; y < 4; ++y)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x16& v = acc[x][y];
        store_run4<OT>(wbuf + ol * LROW + (32 * y + 8 * q + 4 * h) * OS, v[4 * q], v[4 * q + 1], v[4 * q + 2],
                       v[4 * q + 3]);
      }
#pragma unroll
    for (int rr = 0; rr < 32; rr += RPI) {
      const int row = rr + lane / CH, ch = lane % CH;
      const int64_t orow = o0 + 128 * wm + 32 * x + row;
      const int64_t ocol = ocol0 + (int64_t)ch * (16 / OS);
      u32x4 val = ld16(wbuf + row * LROW + ch * 16);
      if (orow < m.d && ocol < m.k) {
        char* dst = m.compact ? m.out + ((b * m.sym_count + sym_local) * (int64_t)(trk::kBM * trk::kBN) +
                                         (orow - o0) * trk::kBN + (ocol - k0)) * OS
                              : obase + out_index(m, orow, ocol) * OS;
        if constexpr (OT == DA_F32) {
          if (m.acc) {
            const f32x4 old = __builtin_bit_cast(f32x4, ld16(dst));
            val = __builtin_bit_cast(u32x4, __builtin_bit_cast(f32x4, val) + old);
          }
        }
        st16(dst, val);
      }
    }
  }
}

// The same 256 x 256 tile with two waves per SIMD (8 waves, 512 threads): wave
// w owns output rows 64 (w / 2) .. +64 and columns 128 (w % 2) .. +128 (2 x 4
// MFMA blocks, 128 fp32 accumulators, so two waves fit one SIMD's registers).
// While one wave of a SIMD waits at a barrier, on a load or on LDS, the other
// keeps the MFMA pipe busy.  Each 16-token slice costs 6 transposing fragment
// reads per 8 MFMAs (4 wave-blocks of 128 x 128 need 8 per 16); the LDS has
// the headroom.  The ring, its stages and the swizzle are the 4-wave kernel's;
// wave w loads token rows 4w .. 4w+3 of both operand tiles (2 DMA instructions
// per operand and stage).  Each output is the same MFMA chain over the same
// token order as in the 4-wave kernel, so the results are bit-identical; on
// the Llama-3-8B block's shapes (8 x 2048 tokens) it runs 7-11% faster
// (1230-1260 against 1130-1170 TFLOP/s on gate, down and q; a 5-stage ring
// and row-tile groups of 2 measured slower, groups of 8 the same).  Plain
// per-sample tiles only: the row-Gram triangle keeps the 4-wave kernel.
namespace tr8 {
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kDma = trk::kTS * (trk::kRow / 16) / (kWave * kWaves);  // per operand and stage
static_assert(kDma == 2, "the vmcnt wait assumes 4 DMA instructions per wave and stage");
}  // namespace tr8

template <int DT, int OT>
__global__ __launch_bounds__(tr8::kThreads, 1) void materialize_tiles_tr8(MatArgs m) {
  static_assert(Elem<DT>::kBytes == 2, "transposing reads are 16-bit");
  __shared__ __attribute__((aligned(1024))) char smem[trk::kNBuf * trk::kStage];
  lds_char* const L = (lds_char*)smem;
  const uint32_t lds0 = (uint32_t)(uintptr_t)L;

  // Tile order: the 4-wave kernel's (each XCD an eighth of every sample when
  // the sample's tile count divides by 8; groups of kGroup row tiles).
  const int64_t ntiles = (int64_t)gridDim.x;
  const int64_t logical = xcd_remap(blockIdx.x, ntiles);
  int64_t b, rem;
  const int64_t per_sample = m.tiles_m * m.tiles_n;
  if (per_sample % kXcds == 0) {
    const int64_t chunk = per_sample / kXcds;
    const int64_t xcd = blockIdx.x % kXcds, local = blockIdx.x / kXcds;
    b = local / chunk;
    rem = xcd * chunk + local % chunk;
  } else {
    b = logical / per_sample;
    rem = logical - b * per_sample;
  }
  const int64_t per_group = (int64_t)trk::kGroup * m.tiles_n;
  const int64_t group = rem / per_group;
  const int64_t first = group * trk::kGroup;
  const int64_t gsize = min(m.tiles_m - first, (int64_t)trk::kGroup);
  const int64_t in_group = rem - group * per_group;
  const int64_t tm = first + in_group % gsize, tn = in_group / gsize;
  const int64_t o0 = tm * trk::kBM, k0 = tn * trk::kBN;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;  // 64-row quarter of the g tile, 128-column half of the a tile
  const int uwave = __builtin_amdgcn_readfirstlane(wave);

  const u32x4 rg = make_rsrc(m.g + b * m.g_bstride, (uint32_t)(m.tokens * m.g_tstride));
  const u32x4 ra = make_rsrc(m.a + b * m.a_bstride, (uint32_t)(m.tokens * m.a_tstride));
  const uint32_t gts = (uint32_t)m.g_tstride, ats = (uint32_t)m.a_tstride;
  const int nst = (int)((m.tokens + trk::kTS - 1) / trk::kTS);

  // DMA: lane l of instruction j takes token row 4w + 2j + l/32, slot l % 32.
  uint32_t goff[tr8::kDma], aoff[tr8::kDma];
#pragma unroll
  for (int j = 0; j < tr8::kDma; ++j) {
    const int r = 4 * wave + 2 * j + (lane >> 5);
    const int c = (lane & 31) ^ trk::swz(r);
    const int64_t gc = o0 + 8 * c, ac = k0 + 8 * c;
    goff[j] = gc < m.d ? (uint32_t)(r * gts + gc * 2) : trk::kOob;
    aoff[j] = ac < m.k ? (uint32_t)(r * ats + ac * 2) : trk::kOob;
  }
  auto dma_one = [&](int side, int st, int j) __attribute__((always_inline)) {
    const bool en = st < nst;
    const uint32_t lbase = lds0 + (uint32_t)((st % trk::kNBuf) * trk::kStage + side * trk::kOp +
                                             (4 * uwave + 2 * j) * trk::kRow);
    const uint32_t step = (uint32_t)st * (trk::kTS * (side == 0 ? gts : ats));
    const uint32_t off = (side == 0 ? goff[j] : aoff[j]) + step;
    dma16(side == 0 ? rg : ra, lbase, en ? off : trk::kOob);
  };
  auto issue = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < tr8::kDma; ++j) dma_one(0, st, j);
#pragma unroll
    for (int j = 0; j < tr8::kDma; ++j) dma_one(1, st, j);
  };

  // Fragment addresses (the 4-wave kernel's lane layout): 2 g fragments (rows
  // 64 wm + 32 f) and 4 a fragments (columns 128 wn + 32 f).
  const int q = lane >> 4, i16 = lane & 15;
  const int rsw = (i16 >> 2) << 2;
  const int rowoff = (8 * (q >> 1) + (i16 >> 2)) * trk::kRow;
  int gfr[2], afr[4];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const int cg = (64 * wm + 32 * f) / 8 + 2 * (q & 1) + ((i16 & 3) >> 1);
    gfr[f] = rowoff + ((cg ^ rsw) << 4) + 8 * (i16 & 1);
  }
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int ca = (128 * wn + 32 * f) / 8 + 2 * (q & 1) + ((i16 & 3) >> 1);
    afr[f] = trk::kOp + rowoff + ((ca ^ rsw) << 4) + 8 * (i16 & 1);
  }

  f32x16 acc[2][4];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y) acc[x][y] = f32x16{};

  u32x4 f0a[2], f0b[4], f1a[2], f1b[4];
  auto read = [&](const lds_char* sb, u32x4 (&fa)[2], u32x4 (&fb)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int f = 0; f < 2; ++f) fa[f] = tr_frag(sb + gfr[f], sb + gfr[f] + 4 * trk::kRow);
#pragma unroll
    for (int f = 0; f < 4; ++f) fb[f] = tr_frag(sb + afr[f], sb + afr[f] + 4 * trk::kRow);
  };
  auto mma = [&](const u32x4 (&fa)[2], const u32x4 (&fb)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int y = 0; y < 4; ++y) Mfma32<DT>::mma(acc[x][y], fb[y], fa[x]);
  };
  // Wait until this wave's loads of the next stage are done (the 4 * (kNBuf -
  // 2) issued after them may still fly) and its LDS reads have returned, then
  // barrier.
  auto stage_sync = [&]() __attribute__((always_inline)) {
    static_assert(trk::kNBuf == 4, "vmcnt below is 4 * (kNBuf - 2)");
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("s_barrier" ::: "memory");
  };
  // Half a stage: the 8 MFMAs of one 16-token slice held in (ua, ub), the 12
  // transposing reads of the next slice into (na, nb), and one operand's 2 DMA
  // instructions of a later stage.  Reads are spread 3 per 2 MFMAs, DMA after
  // the 2nd and 6th MFMA.
  auto half = [&](const u32x4 (&ua)[2], const u32x4 (&ub)[4], const lds_char* sb, u32x4 (&na)[2],
                  u32x4 (&nb)[4], int side, int dst) __attribute__((always_inline)) {
    s16x4 t[12];
    auto rd = [&](int i) __attribute__((always_inline)) {
      const int fr = i >> 1;
      const int fo = fr < 2 ? gfr[fr] : afr[fr - 2];
      t[i] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(sb + fo + (i & 1) * 4 * trk::kRow));
    };
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      rd(i);
      if (i & 1) rd(8 + (i >> 1));
      Mfma32<DT>::mma(acc[i >> 2][i & 3], ub[i & 3], ua[i >> 2]);
      if ((i & 3) == 1 && side >= 0) dma_one(side, dst, i >> 2);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int f = 0; f < 6; ++f) {
      const u32x2 lo = __builtin_bit_cast(u32x2, t[2 * f]), hi = __builtin_bit_cast(u32x2, t[2 * f + 1]);
      (f < 2 ? na[f] : nb[f - 2]) = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
  };

#pragma unroll
  for (int s = 0; s < trk::kNBuf - 1; ++s) issue(s);
  stage_sync();
#pragma unroll
  for (int j = 0; j < tr8::kDma; ++j) dma_one(0, trk::kNBuf - 1, j);
  read(L, f0a, f0b);
  for (int st = 0; st + 1 < nst; ++st) {
    half(f0a, f0b, L + (st % trk::kNBuf) * trk::kStage + 16 * trk::kRow, f1a, f1b, 1, st + trk::kNBuf - 1);
    stage_sync();
    half(f1a, f1b, L + ((st + 1) % trk::kNBuf) * trk::kStage, f0a, f0b, 0, st + trk::kNBuf);
  }
  half(f0a, f0b, L + ((nst - 1) % trk::kNBuf) * trk::kStage + 16 * trk::kRow, f1a, f1b, -1, 0);
  mma(f1a, f1b);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue (the 4-wave kernel's, per 32-row group x of this wave's 64 rows):
  // lane l of acc[x][y] holds row o = 32x + l%32 and columns 32y + 8q + 4(l/32)
  // + (0..3) in acc[x][y][4q .. 4q+3].  A wave stages RG rows at a time in its
  // own padded LDS rows (16 when 8 waves' 32 fp32 rows would exceed the ring).
  constexpr int OS = Elem<OT>::kBytes;
  constexpr int ROWB = 128 * OS;
  constexpr int LROW = ROWB + 16;
  constexpr int CH = ROWB / 16;
  constexpr int RPI = kWave / CH;
  constexpr int RG = tr8::kWaves * 32 * LROW <= (int)sizeof(smem) ? 32 : 16;
  static_assert(tr8::kWaves * RG * LROW <= (int)sizeof(smem), "epilogue staging exceeds the ring");
  char* wbuf = smem + wave * (RG * LROW);
  const int h = lane >> 5, ol = lane & 31;
  const int64_t ocol0 = k0 + 128 * wn;
  char* obase = m.out + (b * m.out_bstride) * OS;
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
  for (int x = 0; x < 2; ++x) {
#pragma unroll
    for (int p = 0; p < 32 / RG; ++p) {
      if (ol / RG == p) {
#pragma unroll
        for (int y = 0; y < 4; ++y)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const f32x16& v = acc[x][y];
            store_run4<OT>(wbuf + (ol % RG) * LROW + (32 * y + 8 * q4 + 4 * h) * OS, v[4 * q4], v[4 * q4 + 1],
                           v[4 * q4 + 2], v[4 * q4 + 3]);
          }
      }
#pragma unroll
      for (int rr = 0; rr < RG; rr += RPI) {
        const int row = rr + lane / CH, ch = lane % CH;
        const int64_t orow = o0 + 64 * wm + 32 * x + p * RG + row;
        const int64_t ocol = ocol0 + (int64_t)ch * (16 / OS);
        u32x4 val = ld16(wbuf + row * LROW + ch * 16);
        if (orow < m.d && ocol < m.k) {
          char* dst = obase + out_index(m, orow, ocol) * OS;
          if constexpr (OT == DA_F32) {
            if (m.acc) {
              const f32x4 old = __builtin_bit_cast(f32x4, ld16(dst));
              val = __builtin_bit_cast(u32x4, __builtin_bit_cast(f32x4, val) + old);
            }
          }
          st16(dst, val);
        }
      }
    }
  }
}

// Narrow layers: one side at most 64 wide (LoRA adapters, small heads).  The
// wide-tile kernels pad such a side to their 128 or 256 rows and leave few
// tiles per sample (16 of 256 x 256 for 4096 -> 16), so the GPU idles and the
// bytes, which bound this shape, stream slowly.  Here a workgroup owns the
// whole narrow side (up to 64 columns) against 64 columns of the wide side:
// 64 tiles per sample at width 4096.  The tile's two 64-column operand slices
// go HBM -> LDS by buffer loads with the LDS-direct bit, 32 tokens per stage
// (8 KB), through a ring of four stages, three in flight, one DMA instruction
// per operand, wave and stage.  Wave w multiplies all (up to four) 16-row
// blocks of the narrow side against wide columns 16w .. 16w+15 with
// 16x16x32 MFMAs, fragments read with transposing LDS reads (16-byte chunk c
// of token row r stored at slot c ^ 2(r % 4), so the four rows of a read's
// 16-lane phase use distinct 32-byte bank groups).  The wide operand is read
// once (non-temporal); the narrow one, shared by the sample's tiles, through
// L2, each XCD owning a contiguous run of tiles.
namespace nw {
constexpr int kCols = 64;            // columns per operand and tile
constexpr int kTS = 32;              // tokens per stage
constexpr int kRow = kCols * 2;      // 128 bytes per token row and operand
constexpr int kSide = kTS * kRow;    // 4 KB
constexpr int kStage = 2 * kSide;    // narrow operand, then wide operand
constexpr int kNBuf = 4;             // three stages in flight (eight measured slower)
constexpr uint32_t kOob = 0x80000000u;
__device__ __forceinline__ int swz(int r) { return (r & 3) << 1; }
static_assert(kNBuf == 4, "the vmcnt wait below is 2 * (kNBuf - 2) = 4");
}  // namespace nw

template <int DT, int OT>
__global__ __launch_bounds__(256) void materialize_narrow(MatArgs m, int narrow_is_d) {
  static_assert(Elem<DT>::kBytes == 2, "transposing reads are 16-bit");
  __shared__ __attribute__((aligned(1024))) char smem[nw::kNBuf * nw::kStage];
  lds_char* const L = (lds_char*)smem;
  const uint32_t lds0 = (uint32_t)(uintptr_t)L;
  const int64_t logical = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t b = logical / m.tiles_n, tw = logical - b * m.tiles_n;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int uwave = __builtin_amdgcn_readfirstlane(wave);

  // the narrow operand (width N) and the wide one (width W) of sample b
  const char* xn = narrow_is_d ? m.g + b * m.g_bstride : m.a + b * m.a_bstride;
  const char* xw = narrow_is_d ? m.a + b * m.a_bstride : m.g + b * m.g_bstride;
  const uint32_t tsn = (uint32_t)(narrow_is_d ? m.g_tstride : m.a_tstride);
  const uint32_t tsw = (uint32_t)(narrow_is_d ? m.a_tstride : m.g_tstride);
  const int64_t n_cols = narrow_is_d ? m.d : m.k, w_cols = narrow_is_d ? m.k : m.d;
  const int64_t w0 = tw * nw::kCols;
  const u32x4 rn = uniform4(make_rsrc(xn, (uint32_t)(m.tokens * tsn)));
  const u32x4 rw = uniform4(make_rsrc(xw, (uint32_t)(m.tokens * tsw)));
  const int nst = (int)((m.tokens + nw::kTS - 1) / nw::kTS);

  // DMA: wave w loads token rows 8w .. 8w+7 of both operands; lane l takes
  // row 8w + l/8 and LDS slot l%8, which holds chunk (l%8) ^ swz(row).
  const int r = 8 * wave + (lane >> 3);
  const int c = (lane & 7) ^ nw::swz(r);
  const uint32_t offn = 8 * c < n_cols ? r * tsn + 16u * (uint32_t)c : nw::kOob;
  const uint32_t offw = w0 + 8 * c < w_cols ? r * tsw + (uint32_t)(w0 + 8 * c) * 2u : nw::kOob;
  auto issue = [&](int st) __attribute__((always_inline)) {
    const bool en = st < nst;
    const uint32_t base = lds0 + (uint32_t)((st % nw::kNBuf) * nw::kStage + 8 * uwave * nw::kRow);
    dma16(rn, base, en && offn != nw::kOob ? offn + (uint32_t)st * (nw::kTS * tsn) : nw::kOob);
    dma16_nt(rw, base + nw::kSide, en && offw != nw::kOob ? offw + (uint32_t)st * (nw::kTS * tsw) : nw::kOob);
  };

  // Fragment of the 16 columns c0 .. c0+15 of one operand over the stage's 32
  // tokens: lane l gets tokens 8(l/16) .. +7 of column c0 + l%16 (two
  // transposing reads of 4 tokens; lane j of a 16-lane phase addresses token
  // row t0 + j/4, columns c0 + 4(j%4) .. +3).
  const int g4 = lane >> 4, i16 = lane & 15;
  auto frag = [&](const lds_char* side, int c0) __attribute__((always_inline)) {
    u32x2 h[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int t = 8 * g4 + 4 * k + (i16 >> 2);
      const int col = c0 + 4 * (i16 & 3);
      const lds_char* p = side + t * nw::kRow + (((col >> 3) ^ nw::swz(t)) << 4) + (col & 7) * 2;
      h[k] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                           (__attribute__((address_space(3))) s16x4*)p));
    }
    return u32x4{h[0][0], h[0][1], h[1][0], h[1][1]};
  };

  const int nblk = (int)((n_cols + 15) / 16);  // 16-row blocks of the narrow side (<= 4)
  f32x4 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s0 = 0; s0 < nw::kNBuf - 1; ++s0) issue(s0);
  for (int st = 0; st < nst; ++st) {
    // this wave's loads of stage st are done (the two later stages' 4 may fly),
    // its LDS reads of stage st - 1 have returned; then every wave's
    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("s_barrier" ::: "memory");
    issue(st + nw::kNBuf - 1);  // into the slot stage st - 1 used
    const lds_char* sb = L + (st % nw::kNBuf) * nw::kStage;
    const u32x4 fw = frag(sb + nw::kSide, 16 * wave);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < nblk) Mfma16<DT>::mma(acc[j], frag(sb, 16 * j), fw);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the zero-fill loads past the last stage

  // lane l holds narrow rows 16j + 4(l/16) + e against wide column 16w + l%16
  const int64_t wc = w0 + 16 * wave + i16;
  if (wc >= w_cols) return;
  const int64_t base = b * m.out_bstride;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (j >= nblk) break;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t n = 16 * j + 4 * g4 + e;
      if (n < n_cols) {
        const int64_t o = narrow_is_d ? n : wc, k = narrow_is_d ? wc : n;
        Elem<OT>::store(m.out, base + out_index(m, o, k), acc[j][e]);
      }
    }
  }
}

// Row Gram with token splits: for the triangle tiles tile0 .. tile0 + count - 1
// (row by row over T tiles per side), out (+)= the sum over splits s, in order,
// of the compact partial tiles ws[s][t] (256 x 256 fp32 each).  Block (t, y):
// rows 4y .. 4y + 3 of tile t, one float4 per thread.
__global__ __launch_bounds__(256) void sum_split_tiles(const float* __restrict__ ws, int splits, int64_t count,
                                                       int64_t tile0, int64_t T, int64_t n, float* __restrict__ out,
                                                       int64_t ld, int acc) {
  const int64_t t = blockIdx.x;
  int64_t r = tile0 + t, tm = 0;
  while (r >= T - tm) {
    r -= T - tm;
    ++tm;
  }
  const int64_t tn = tm + r;
  const int row = (int)blockIdx.y * 4 + (int)(threadIdx.x >> 6), c4 = (int)(threadIdx.x & 63);
  const int64_t i = tm * trk::kBM + row, jc = tn * trk::kBN + 4 * c4;
  if (i >= n || jc >= n) return;  // n is a multiple of 8: the float4 lies inside
  const int64_t tile = (int64_t)trk::kBM * trk::kBN;
  const float* src = ws + t * tile + (int64_t)row * trk::kBN + 4 * c4;
  f32x4 v = *(const f32x4*)src;
  for (int s = 1; s < splits; ++s) v += *(const f32x4*)(src + (int64_t)s * count * tile);
  float* dst = out + i * ld + jc;
  if (acc) v += *(const f32x4*)dst;
  *(f32x4*)dst = v;
}

// Gradient-free rows: out[r] = 1 when some entry of row r compares unequal to
// zero, by its magnitude bits (-0.0 is zero; NaN, inf and subnormals are not),
// one workgroup per row reading it once in 16-byte chunks.
template <int ES>
__global__ __launch_bounds__(256) void nonzero_rows_kernel(const char* __restrict__ x, int64_t chunks,
                                                           int64_t stride_b, uint8_t* __restrict__ out) {
  const int64_t r = blockIdx.x;
  const u32x4* p = (const u32x4*)(x + r * stride_b);
  constexpr uint32_t kMag = ES == 4 ? 0x7fffffffu : 0x7fff7fffu;  // both halves of a 16-bit pair
  uint32_t any = 0;
  for (int64_t c = threadIdx.x; c < chunks; c += 256) {
    const u32x4 v = __builtin_nontemporal_load(p + c);
    any |= (v[0] & kMag) | (v[1] & kMag) | (v[2] & kMag) | (v[3] & kMag);
  }
  const int nz = __syncthreads_or(any != 0u);
  if (threadIdx.x == 0) out[r] = nz ? 1 : 0;
}

// Row Gram: copy the tiles above the diagonal (computed) to the ones below it.
// Block (I, J) of 64 x 64 outputs with tile(I) > tile(J) (256-output tiles,
// so a block lies in one tile pair) reads the transposed block (J, I) through
// LDS with 16-byte row accesses on both sides (n and ld are multiples of 4).
__global__ __launch_bounds__(256) void mirror_lower(float* __restrict__ out, int64_t n, int64_t ld) {
  __shared__ float t[64][65];
  const int64_t bi = blockIdx.y, bj = blockIdx.x;  // output block row, block column
  if ((bi * 64) / trk::kBM <= (bj * 64) / trk::kBN) return;  // uniform: on or above the diagonal tiles
  const int tid = threadIdx.x;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int idx = tid + 256 * k, r = idx >> 4, c4 = idx & 15;
    const int64_t sr = bj * 64 + r, sc = bi * 64 + 4 * c4;  // source (upper) row and first column
    const f32x4 v = (sr < n && sc < n) ? *(const f32x4*)(out + sr * ld + sc) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) t[r][4 * c4 + e] = v[e];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int idx = tid + 256 * k, r = idx >> 4, c4 = idx & 15;
    const int64_t dr = bi * 64 + r, dc = bj * 64 + 4 * c4;  // destination (lower) row and first column
    if (dr < n && dc < n)
      *(f32x4*)(out + dr * ld + dc) = f32x4{t[4 * c4][r], t[4 * c4 + 1][r], t[4 * c4 + 2][r], t[4 * c4 + 3][r]};
  }
}

// Bias column dW[b, o, K] = sum_t g[b, t, o]: one thread per (b, o).
template <int DT, int OT>
__global__ void bias_column(const char* g, int64_t batch, int64_t tokens, int64_t d,
                            int64_t g_bstride, int64_t g_tstride, char* out, int64_t out_bstride,
                            int64_t out_rstride, int64_t out_blk, int64_t kcol) {
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (o >= d) return;
  const char* src = g + b * g_bstride;
  float s = 0.f;
  for (int64_t t = 0; t < tokens; ++t) s += Elem<DT>::load(src + t * g_tstride, o);
  const int64_t c = o * out_rstride + kcol;
  Elem<OT>::store(out, b * out_bstride + (c >> 6) * out_blk + (c & 63), s);
}

template <int DT, int OT>
int launch(const MatArgs& m, int has_bias, hipStream_t st) {
  const int64_t ntiles = m.batch * m.tiles_m * m.tiles_n;
  if (ntiles > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "da_materialize_linear: too many tiles");
  // 16-byte output stores need whole output chunks inside every row.
  const bool aligned = (m.k % (16 / Elem<OT>::kBytes) == 0) &&
                       ((m.out_rstride * Elem<OT>::kBytes) % 16 == 0) &&
                       ((m.out_blk * Elem<OT>::kBytes) % 16 == 0) &&
                       ((m.out_bstride * Elem<OT>::kBytes) % 16 == 0) && (((uintptr_t)m.out & 15) == 0);
  const bool use_big = aligned && m.d >= big::kBM && m.k >= big::kBN && m.k % 8 == 0;
  // The transposing-read kernel addresses a sample's rows with 32-bit buffer
  // offsets and needs disjoint rows (a zero token stride would read as empty).
  const int64_t max_ts = m.g_tstride > m.a_tstride ? m.g_tstride : m.a_tstride;
  const bool use_tr = Elem<DT>::kBytes == 2 && use_big && (m.tokens + trk::kTS) * max_ts < (1LL << 31) &&
                      m.g_tstride >= m.d * 2 && m.a_tstride >= m.k * 2;
  // one side at most 64 wide: the narrow-layer kernel (rows addressed by
  // 32-bit buffer offsets, disjoint rows)
  const bool use_narrow = Elem<DT>::kBytes == 2 && (m.d <= nw::kCols || m.k <= nw::kCols) &&
                          (m.tokens + nw::kTS) * max_ts < (1LL << 31) && m.g_tstride >= m.d * 2 &&
                          m.a_tstride >= m.k * 2;
  if (use_narrow) {
    MatArgs mn = m;
    const int narrow_is_d = m.d <= nw::kCols ? 1 : 0;
    mn.tiles_m = 1;
    mn.tiles_n = ((narrow_is_d ? m.k : m.d) + nw::kCols - 1) / nw::kCols;
    const int64_t nt = m.batch * mn.tiles_n;
    if (nt > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "da_materialize_linear: too many tiles");
    if constexpr (Elem<DT>::kBytes == 2) materialize_narrow<DT, OT><<<(unsigned)nt, 256, 0, st>>>(mn, narrow_is_d);
    int rc = check_launch("da_materialize_linear(narrow)");
    if (rc) return rc;
  } else if (use_tr) {
    MatArgs mt = m;
    mt.tiles_m = (m.d + trk::kBM - 1) / trk::kBM;
    mt.tiles_n = (m.k + trk::kBN - 1) / trk::kBN;
    const int64_t nt = m.batch * mt.tiles_m * mt.tiles_n;
    if constexpr (Elem<DT>::kBytes == 2) materialize_tiles_tr8<DT, OT><<<(unsigned)nt, tr8::kThreads, 0, st>>>(mt);
    int rc = check_launch("da_materialize_linear(transposing reads)");
    if (rc) return rc;
  } else if (use_big) {
    MatArgs mb = m;
    mb.tiles_m = (m.d + big::kBM - 1) / big::kBM;
    mb.tiles_n = (m.k + big::kBN - 1) / big::kBN;
    const int64_t nb = m.batch * mb.tiles_m * mb.tiles_n;
    const size_t lds = 2 * (size_t)big::kStageBytes;
    // Idempotent, so racing first calls are harmless; per template instance.
    static std::atomic<bool> attr_set{false};
    if (!attr_set.load(std::memory_order_relaxed)) {
      if (hipFuncSetAttribute((const void*)materialize_tiles_big<DT, OT>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return set_error(DA_ERR_HIP, "da_materialize_linear: hipFuncSetAttribute failed");
      attr_set.store(true, std::memory_order_relaxed);
    }
    materialize_tiles_big<DT, OT><<<(unsigned)nb, kThreads, lds, st>>>(mb);
    int rc = check_launch("da_materialize_linear(big tiles)");
    if (rc) return rc;
  } else if (ntiles > 0) {
    if (aligned)
      materialize_tiles<DT, OT, true><<<(unsigned)ntiles, kThreads, 0, st>>>(m);
    else
      materialize_tiles<DT, OT, false><<<(unsigned)ntiles, kThreads, 0, st>>>(m);
    int rc = check_launch("da_materialize_linear(tiles)");
    if (rc) return rc;
  }
  if (has_bias) {
    dim3 grid((unsigned)((m.d + 255) / 256), (unsigned)m.batch);
    bias_column<DT, OT><<<grid, 256, 0, st>>>(m.g, m.batch, m.tokens, m.d, m.g_bstride, m.g_tstride,
                                              m.out, m.out_bstride, m.out_rstride, m.out_blk, m.k);
    return check_launch("da_materialize_linear(bias)");
  }
  return DA_OK;
}

}  // namespace
}  // namespace da

extern "C" int da_materialize_linear(const void* a, const void* g, int dtype, int64_t batch,
                                     int64_t tokens, int64_t K, int64_t D, int64_t a_bstride,
                                     int64_t a_tstride, int64_t g_bstride, int64_t g_tstride,
                                     int has_bias, void* out, int out_dtype, int64_t out_bstride,
                                     int64_t out_rstride, int64_t out_blk, void* stream) {
  using namespace da;
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype))
    return set_error(DA_ERR_INVALID, "da_materialize_linear: bad dtype");
  if (batch < 0 || tokens < 0 || K < 0 || D < 0)
    return set_error(DA_ERR_INVALID, "da_materialize_linear: negative size");
  if (batch == 0 || K == 0 || D == 0) return DA_OK;
  const int64_t es = (int64_t)elem_bytes(dtype);
  if ((K * es) % 16 || (D * es) % 16)
    return set_error(DA_ERR_INVALID, "da_materialize_linear: K and D must be multiples of %lld",
                     (long long)(16 / es));
  if (!a || !g || !out) return set_error(DA_ERR_INVALID, "da_materialize_linear: NULL pointer");
  if (((uintptr_t)a | (uintptr_t)g) & 15)
    return set_error(DA_ERR_INVALID, "da_materialize_linear: inputs must be 16-byte aligned");
  if (((a_bstride * es) | (a_tstride * es) | (g_bstride * es) | (g_tstride * es)) % 16)
    return set_error(DA_ERR_INVALID, "da_materialize_linear: strides must be multiples of 16 bytes");
  if (out_rstride < K + (has_bias ? 1 : 0))
    return set_error(DA_ERR_INVALID, "da_materialize_linear: out row stride too small");
  if (out_blk == 0) out_blk = 64;
  if (out_blk < 64) return set_error(DA_ERR_INVALID, "da_materialize_linear: out_blk must be 0 or >= 64");
  if (out_blk != 64 && ((out_rstride % 64) || out_bstride < 64))
    return set_error(DA_ERR_INVALID,
                     "da_materialize_linear: a blocked output needs a row stride multiple of 64 and "
                     "out_bstride >= 64");
  if (tokens == 0) return set_error(DA_ERR_INVALID, "da_materialize_linear: tokens must be >= 1");
  MatArgs m;
  m.a = (const char*)a;
  m.g = (const char*)g;
  m.batch = batch;
  m.tokens = tokens;
  m.k = K;
  m.d = D;
  m.a_bstride = a_bstride * es;
  m.a_tstride = a_tstride * es;
  m.g_bstride = g_bstride * es;
  m.g_tstride = g_tstride * es;
  m.out = (char*)out;
  m.out_bstride = out_bstride;
  m.out_rstride = out_rstride;
  m.out_blk = out_blk;
  m.tiles_m = (D + kBM - 1) / kBM;
  m.tiles_n = (K + kBN - 1) / kBN;
  m.sym = 0;
  m.acc = 0;
  m.rows_total = 0;
  m.tile0 = 0;
  m.sym_count = 0;
  m.compact = 0;
  hipStream_t st = (hipStream_t)stream;
#define DA_MAT_CASE(DT)                                                         \
  switch (out_dtype) {                                                          \
    case DA_F32: return launch<DT, DA_F32>(m, has_bias, st);                    \
    case DA_BF16: return launch<DT, DA_BF16>(m, has_bias, st);                  \
    default: return launch<DT, DA_F16>(m, has_bias, st);                        \
  }
  switch (dtype) {
    case DA_BF16: DA_MAT_CASE(DA_BF16)
    case DA_F16: DA_MAT_CASE(DA_F16)
    default: DA_MAT_CASE(DA_F32)
  }
#undef DA_MAT_CASE
}

namespace da {
namespace {

struct GramPlan {
  int64_t head;    // triangle tiles 0 .. head - 1 run over all rows, straight into out
  int splits;      // token splits of the remaining tiles (1: no split launch)
  int64_t chunk;   // rows per split
  size_t ws;       // workspace bytes: splits x (tiles - head) compact 256 x 256 fp32 partials
};

// Token splits of a row Gram.  Every tile runs over all the rows, so a triangle
// whose tile count is not a multiple of the CU count ends in a partly filled
// round (width 4096: 136 tiles in one round; width 14336: 1596 tiles, the
// seventh round a quarter full).  The tiles of the whole rounds (head) run as
// they are; the rest are cut into token splits that run side by side, and a
// second pass sums their partial tiles.  Time model in rows of one tile's
// work: a round over `chunk` rows costs `chunk`; the partials' HBM traffic,
// (S + 1) tiles of 256^2 fp32 per split tile at ~5 TB/s against a tile's ~29 ns
// per row on one CU, costs (S + 1) * tiles * 1.8.
GramPlan gram_plan(int64_t rows, int64_t width, int64_t sb, int64_t slots, size_t ws_limit) {
  const int64_t t = (width + trk::kBM - 1) / trk::kBM, nt = t * (t + 1) / 2;
  GramPlan g{nt, 1, rows, 0};
  const int64_t head = nt > slots ? nt / slots * slots : 0, tail = nt - head;
  if (tail == 0) return g;
  const int64_t lim32 = ((1LL << 31) - (1LL << 20)) / sb - trk::kTS;  // rows one buffer resource can span
  const size_t tile_bytes = (size_t)trk::kBM * trk::kBN * sizeof(float);
  // the cheapest split, kept when it beats one pass by 5%
  const double one_pass = (double)((nt + slots - 1) / slots) * (double)rows;
  double best = 0.95 * one_pass;
  for (int s = 2; s <= 64; ++s) {
    int64_t chunk = (rows + s - 1) / s;
    chunk = (chunk + trk::kTS - 1) / trk::kTS * trk::kTS;
    if (chunk < 8 * trk::kTS || chunk > lim32) continue;
    const int64_t sp = (rows + chunk - 1) / chunk;
    if ((size_t)(sp * tail) * tile_bytes > ws_limit || tail * sp > 0x7fffffffLL) continue;
    const double cost = (double)(head / slots) * (double)rows + (double)((tail * sp + slots - 1) / slots) * (double)chunk +
                        1.8 * (double)(sp + 1) * (double)tail;
    if (cost < best) {
      best = cost;
      g = GramPlan{head, (int)sp, chunk, (size_t)(sp * tail) * tile_bytes};
    }
  }
  return g;
}

}  // namespace
}  // namespace da

// Row Gram out (+)= x^T x of x (rows, width), fp32 out: the transposing-read
// dW kernel with every row as one token and both operands x, over the tiles on
// or above the diagonal, then the mirror.  Tiles run over all rows straight into
// out, in chunks of rows whose buffer offsets fit 32 bits, each adding to the
// output; with token splits (a workspace holding them), the tiles past the
// whole rounds run per split into compact partial tiles, which
// sum_split_tiles adds in split order.
extern "C" int da_row_gram_workspace(int64_t rows, int64_t width, int dtype, size_t* bytes) {
  using namespace da;
  if (!bytes) return set_error(DA_ERR_INVALID, "da_row_gram_workspace: bytes is NULL");
  if (dtype != DA_BF16 && dtype != DA_F16)
    return set_error(DA_ERR_UNSUPPORTED, "da_row_gram_workspace: bf16 or fp16 rows only");
  if (rows < 0 || width < 0) return set_error(DA_ERR_INVALID, "da_row_gram_workspace: negative size");
  *bytes = 0;
  if (rows == 0 || width == 0) return DA_OK;
  int64_t slots = 0;
  const int rc = device_cu_count(&slots);
  if (rc) return rc;
  *bytes = gram_plan(rows, width, width * 2, slots, (size_t)1 << 33).ws;
  return DA_OK;
}

extern "C" int da_row_gram(const void* x, int dtype, int64_t rows, int64_t width, int64_t x_stride, float* out,
                           int64_t ld_out, int accumulate, void* workspace, size_t workspace_bytes,
                           void* stream) {
  using namespace da;
  if (dtype != DA_BF16 && dtype != DA_F16)
    return set_error(DA_ERR_UNSUPPORTED, "da_row_gram: bf16 or fp16 rows only");
  if (rows < 0 || width < 0) return set_error(DA_ERR_INVALID, "da_row_gram: negative size");
  if (width == 0) return DA_OK;
  if (!out || (!x && rows > 0)) return set_error(DA_ERR_INVALID, "da_row_gram: NULL pointer");
  const int64_t es = 2;
  if ((width * es) % 16 || (x_stride * es) % 16 || x_stride < width || ((uintptr_t)x & 15))
    return set_error(DA_ERR_INVALID,
                     "da_row_gram: width and row stride must be multiples of 8 elements (stride >= width), "
                     "rows 16-byte aligned");
  if (ld_out < width || (ld_out * 4) % 16 || ((uintptr_t)out & 15))
    return set_error(DA_ERR_INVALID, "da_row_gram: out row stride must be >= width and a multiple of 4");
  if (workspace && ((uintptr_t)workspace & 15))
    return set_error(DA_ERR_INVALID, "da_row_gram: workspace must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (rows == 0) return accumulate ? DA_OK : zero_f32_2d(out, width, width, ld_out, st);
  const int64_t sb = x_stride * es;
  const int64_t chunk32 = ((1LL << 31) - (1LL << 20)) / sb - trk::kTS;
  if (chunk32 < trk::kTS) return set_error(DA_ERR_INVALID, "da_row_gram: rows too wide for 32-bit offsets");
  int64_t slots = 0;
  int rc = device_cu_count(&slots);
  if (rc) return rc;
  const GramPlan g = gram_plan(rows, width, sb, slots, workspace ? workspace_bytes : 0);
  MatArgs m;
  m.batch = 1;
  m.k = width;
  m.d = width;
  m.a_bstride = 0;
  m.g_bstride = 0;
  m.a_tstride = sb;
  m.g_tstride = sb;
  m.out = (char*)out;
  m.out_bstride = 0;
  m.out_rstride = ld_out;
  m.out_blk = 64;
  m.tiles_m = (width + trk::kBM - 1) / trk::kBM;
  m.tiles_n = (width + trk::kBN - 1) / trk::kBN;
  m.sym = 1;
  m.rows_total = 0;
  const int64_t nt = m.tiles_m * (m.tiles_m + 1) / 2;
  m.tile0 = 0;
  m.sym_count = nt;
  m.compact = 0;
  auto launch_tiles = [&](int64_t blocks) {
    if (dtype == DA_BF16)
      materialize_tiles_tr<DA_BF16, DA_F32><<<(unsigned)blocks, kThreads, 0, st>>>(m);
    else
      materialize_tiles_tr<DA_F16, DA_F32><<<(unsigned)blocks, kThreads, 0, st>>>(m);
    return check_launch("da_row_gram");
  };
  // head: tiles 0 .. head - 1 over all rows, into out (the whole triangle when
  // there are no splits)
  const int64_t head = g.splits > 1 ? g.head : nt;
  if (head > 0) {
    m.sym_count = head;
    for (int64_t r0 = 0; r0 < rows; r0 += chunk32) {
      m.a = (const char*)x + r0 * sb;
      m.g = m.a;
      m.tokens = rows - r0 < chunk32 ? rows - r0 : chunk32;
      m.acc = accumulate || r0 > 0;
      rc = launch_tiles(head);
      if (rc) return rc;
    }
  }
  if (g.splits > 1) {
    // tiles head .. nt - 1: split b = rows b*chunk .. of x, compact partial tiles
    const int64_t tail = nt - head;
    m.a = (const char*)x;
    m.g = m.a;
    m.batch = g.splits;
    m.tokens = g.chunk;
    m.rows_total = rows;
    m.a_bstride = g.chunk * sb;
    m.g_bstride = m.a_bstride;
    m.out = (char*)workspace;
    m.tile0 = head;
    m.sym_count = tail;
    m.compact = 1;
    m.acc = 0;
    rc = launch_tiles(tail * g.splits);
    if (rc) return rc;
    sum_split_tiles<<<dim3((unsigned)tail, trk::kBM / 4), 256, 0, st>>>(
        (const float*)workspace, g.splits, tail, head, m.tiles_m, width, out, ld_out, accumulate ? 1 : 0);
    rc = check_launch("da_row_gram(sum)");
    if (rc) return rc;
  }
  const int64_t nb = (width + 63) / 64;
  if (m.tiles_m > 1) {
    mirror_lower<<<dim3((unsigned)nb, (unsigned)nb), 256, 0, st>>>(out, width, ld_out);
    return check_launch("da_row_gram(mirror)");
  }
  return DA_OK;
}

// out[r] = (x[r, :] != 0).any() for the rows of x (rows, width) with row stride
// x_stride (elements): the gradient-free-row test of the K-FAC factors.
extern "C" int da_nonzero_rows(const void* x, int dtype, int64_t rows, int64_t width, int64_t x_stride,
                               uint8_t* out, void* stream) {
  using namespace da;
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "da_nonzero_rows: bad dtype %d", dtype);
  if (rows < 0 || width < 0) return set_error(DA_ERR_INVALID, "da_nonzero_rows: negative size");
  if (rows == 0) return DA_OK;
  if (!x || !out) return set_error(DA_ERR_INVALID, "da_nonzero_rows: NULL pointer");
  const int64_t es = (int64_t)elem_bytes(dtype);
  if ((width * es) % 16 || (x_stride * es) % 16 || x_stride < width || ((uintptr_t)x & 15))
    return set_error(DA_ERR_INVALID,
                     "da_nonzero_rows: rows must be 16-byte aligned, width and stride multiples of 16 bytes");
  if (rows > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "da_nonzero_rows: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const int64_t chunks = width * es / 16;
  if (es == 4)
    nonzero_rows_kernel<4><<<(unsigned)rows, 256, 0, st>>>((const char*)x, chunks, x_stride * es, out);
  else
    nonzero_rows_kernel<2><<<(unsigned)rows, 256, 0, st>>>((const char*)x, chunks, x_stride * es, out);
  return check_launch("da_nonzero_rows");
}
