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
// streaming both operands from HBM once.  Most launches take the streaming
// form below (an LDS ring per output tile).  The register-fed form here takes
// what the ring cannot address (k-blocked fp32 rows, rows past 2 GB): the
// flattened width of every layer is cut into chunks; a workgroup owns one
// chunk of one layer for a 16-row x 64-row (side-1 x side-2) output tile and
// runs 16x16 MFMAs straight from registers (every element is used by exactly
// one MFMA of the tile, so there is nothing to share through LDS).  In a 16x16 MFMA four lanes serve one
// row; they read 64 contiguous bytes of it per load instruction, and the same
// element-to-k assignment is used on both sides, so the sum is exact in any
// order.  The four waves split the chunk, combine through LDS and write one
// fp32 partial tile; a second kernel sums the partials in a fixed order.
#include <atomic>

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

// ---------------------------------------------------------------------------
// Streaming form: stream-K over 512-byte units of width through an LDS ring.
//
// The width of every layer is cut into units of 512 bytes (4 blocks of 128 B);
// the units of all layers form one sequence per output tile, and workgroup w
// of the tile's nwg owns units [w*U/nwg, (w+1)*U/nwg), accumulating across
// layer boundaries into one 16 x 64 partial (the score sums over layers).  A
// stage is one unit of the tile's 16 side-1 rows and 64 side-2 rows: 80 rows x
// 4 blocks, each DMA instruction 8 rows x one 128-byte block (with the
// k-blocked layout of the scoring loop, 1 KB contiguous), into a 4-deep ring.
// A side whose rows are read once per launch (the other side fits one tile)
// is loaded with the non-temporal hint: 6.18 -> 6.66 TB/s on the Llama-8B
// block's 8 x 64 score, where both sides are read once.  Rows read again by
// other tiles (a 4096 x 128 output re-reads each query row per 16-row tile)
// keep the default policy, which leaves them in L2.
// Rows past a side's end and bytes past a layer's width read as zero.  Wave w
// loads block w of every stage and multiplies it: 2 x 4 16x16 MFMA steps
// (one 16x16x32 MFMA for 2-byte rows, four 16x16x4 for fp32 rows: the lane's
// 16 bytes are four k-slots, paired the same way on both sides).  Each DMA
// instruction's buffer base is the unit's first block of its own 8 rows, so
// only 8 rows' offsets need fit the 32-bit per-lane offset.  LDS
// row r of a block holds logical 16-byte chunk c in slot c ^ ((r/2) % 8): the
// 16 rows of a fragment, 128 bytes apart, then hit 16 distinct bank groups.
// ---------------------------------------------------------------------------
namespace sr {
constexpr int kRows = kTileM + kTileN;   // 80 LDS rows per block
constexpr int kBlkB = 128;               // bytes per block
constexpr int kUnitB = 4 * kBlkB;        // 512 bytes of width per unit
constexpr int kStage = 4 * kRows * kBlkB;  // 40 KB
constexpr int kNBuf = 4;                 // three stages in flight
constexpr int kDma = kRows / 8;          // 10 instructions per wave and stage
constexpr uint32_t kOob = 0x80000000u;
static_assert(kNBuf * kStage <= 160 * 1024, "LDS");
static_assert(kDma == 10 && kNBuf == 4, "the vmcnt wait below is 10 * (kNBuf - 2) = 20");
}  // namespace sr

struct RingLayer {
  const char* m1;
  const char* m2;
  int64_t bytes;                 // row width in bytes
  int64_t ld1, ld2, blk1, blk2;  // row and 128-byte-block strides, bytes
  int64_t units, u0;             // units of this layer and its first unit in the sequence
};

struct RingArgs {
  RingLayer layers[kMaxLayers];
  int n_layers;
  int64_t units;          // units of all layers
  int64_t nwg;            // workgroups per output tile
  int64_t b1, b2, tiles_n;
  float* partial;         // [b1][b2][nwg]
  int nt1, nt2;           // side 1 / side 2 rows are read once (one tile across the other side):
                          // non-temporal loads
};

__device__ __forceinline__ int64_t ring_first(int64_t w, const RingArgs& a) { return w * a.units / a.nwg; }

template <int DT>
__global__ __launch_bounds__(kThreads, 1) void score_ring(RingArgs a) {
  __shared__ __attribute__((aligned(1024))) char smem[sr::kNBuf * sr::kStage];
  lds_char* const Ls = (lds_char*)smem;
  const uint32_t lds0 = (uint32_t)(uintptr_t)Ls;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int uwave = __builtin_amdgcn_readfirstlane(wave);
  const int64_t tile = blockIdx.x / a.nwg, w = blockIdx.x % a.nwg;
  const int64_t tm = tile / a.tiles_n, tn = tile % a.tiles_n;
  const int64_t ub = uniform64(ring_first(w, a));
  const int nloc = __builtin_amdgcn_readfirstlane((int)(ring_first(w + 1, a) - ub));

  // DMA instruction i of wave w: LDS rows 8i .. 8i+7 of block w (rows < 16:
  // side 1, row tm*16 + r; else side 2, row tn*64 + r - 16); lane l -> row
  // 8i + l/8, slot l%8 holding chunk (l%8) ^ ((row/2) % 8).
  bool rlive[sr::kDma];
  uint32_t cbo[sr::kDma];
#pragma unroll
  for (int i = 0; i < sr::kDma; ++i) {
    const int r = 8 * i + (lane >> 3);
    cbo[i] = 16u * (uint32_t)((lane & 7) ^ ((r >> 1) & 7));
    const int64_t row = i < 2 ? tm * kTileM + r : tn * kTileN + r - kTileM;  // row of its side
    rlive[i] = row < (i < 2 ? a.b1 : a.b2);
  }
  // issue cursor: layer il, unit iu of the layer, and the layer's per-lane offsets
  int il = 0;
  while (il + 1 < a.n_layers && a.layers[il + 1].u0 <= ub) ++il;
  int64_t iu = uniform64(ub - a.layers[il].u0);
  uint32_t roff[sr::kDma];
  uint32_t lbytes = 0;
  int64_t lunits = 0, blk1 = 0, blk2 = 0, ld1 = 0, ld2 = 0;
  const char* m1 = nullptr;  // the tile's first row of each side
  const char* m2 = nullptr;
  auto set_layer = [&]() __attribute__((always_inline)) {
    const RingLayer& Ly = a.layers[il];
    m1 = Ly.m1 + tm * kTileM * Ly.ld1;
    m2 = Ly.m2 + tn * kTileN * Ly.ld2;
    ld1 = Ly.ld1;
    ld2 = Ly.ld2;
    blk1 = Ly.blk1;
    blk2 = Ly.blk2;
    lbytes = (uint32_t)min(Ly.bytes, (int64_t)0x7fffffff);
    lunits = Ly.units;
#pragma unroll
    for (int i = 0; i < sr::kDma; ++i)
      roff[i] = rlive[i] ? (uint32_t)((lane >> 3) * (i < 2 ? Ly.ld1 : Ly.ld2) + uwave * (i < 2 ? Ly.blk1 : Ly.blk2)) + cbo[i]
                         : sr::kOob;
  };
  auto issue = [&](int slot, bool live, bool more) __attribute__((always_inline)) {
    // Each instruction's resource base is the unit's first block of its first
    // row, so per-lane offsets (row within the 8, block w, chunk) span 8 rows.
    const uint32_t kin = (uint32_t)iu * sr::kUnitB + (uint32_t)uwave * sr::kBlkB;  // byte of the layer row
    const uint32_t dst0 = lds0 + (uint32_t)(slot * sr::kStage + uwave * sr::kRows * sr::kBlkB);
#pragma unroll
    for (int i = 0; i < sr::kDma; ++i) {
      const u32x4 rs = uniform4(make_rsrc(i < 2 ? m1 + 8 * i * ld1 + iu * 4 * blk1 : m2 + 8 * (i - 2) * ld2 + iu * 4 * blk2,
                                          0x7fffffffu));
      const bool en = live & (roff[i] != sr::kOob) & (kin + cbo[i] < lbytes);
      if (i < 2 ? a.nt1 : a.nt2)
        dma16_nt(rs, dst0 + (uint32_t)(8 * i * sr::kBlkB), en ? roff[i] : sr::kOob);
      else
        dma16(rs, dst0 + (uint32_t)(8 * i * sr::kBlkB), en ? roff[i] : sr::kOob);
    }
    if (live && ++iu == lunits) {
      iu = 0;
      do {
        ++il;
      } while (il < a.n_layers && a.layers[il].units == 0);
      if (more) set_layer();
    }
  };

  set_layer();
  int ix = 0;
#pragma unroll
  for (int p = 0; p < sr::kNBuf - 1; ++p, ++ix) issue(p, ix < nloc, ix + 1 < nloc);

  const int r16 = lane & 15, q = lane >> 4;
  const int sw = (r16 >> 1) & 7;
  f32x4 acc[4] = {};
  int slot = 0;
  for (int x = 0; x < nloc; ++x, ++ix) {
    // this wave's loads of stage x done (the next stage's 10 may be in
    // flight), its LDS reads done; then every wave's block is visible and the
    // slot read one stage ago may be refilled
    asm volatile("s_waitcnt vmcnt(20) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(slot == 0 ? sr::kNBuf - 1 : slot - 1, ix < nloc, ix + 1 < nloc);
    const lds_char* bb = Ls + slot * sr::kStage + wave * sr::kRows * sr::kBlkB;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int so = (((4 * ks + q) ^ sw) << 4);
      const u32x4 va = *(const u32x4*)(bb + r16 * sr::kBlkB + so);
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const u32x4 vb = *(const u32x4*)(bb + (kTileM + 16 * cb + r16) * sr::kBlkB + so);
        Mfma16<DT>::mma(acc[cb], va, vb);
      }
    }
    slot = slot + 1 == sr::kNBuf ? 0 : slot + 1;
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  // the four waves' tiles through LDS, summed in wave order
  float* red = (float*)smem;
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[(wave * kTileM + acc16_row(e, lane)) * kTileN + 16 * cb + acc16_col(lane)] = acc[cb][e];
  __syncthreads();
  for (int x = tid; x < kTileM * kTileN; x += kThreads) {
    const int row = x / kTileN, col = x % kTileN;
    const float v = ((red[x] + red[kTileM * kTileN + x]) + red[2 * kTileM * kTileN + x]) + red[3 * kTileM * kTileN + x];
    const int64_t oi = tm * kTileM + row, oj = tn * kTileN + col;
    if (oi < a.b1 && oj < a.b2) a.partial[(oi * a.b2 + oj) * a.nwg + w] = v;
  }
}

// The same stream-K ring with a 64 x 64 output tile, for side 1 taller than
// one 16-row tile.  With 16-row tiles every tile stages the same side-2 rows
// again (64 train x 64 query rows: 4 tiles of 80 rows, 2.5 times the rows
// read from HBM, through the L2 -> LDS path, which caps the launch near 5 TB/s);
// here each unit's 128 rows are staged once.  A unit is 256 bytes of width (two
// 128-byte blocks), a stage one unit of the 128 rows (32 KB), four stages in
// the ring.  Wave w loads LDS rows 64 (w % 2) .. +63 of block w / 2 (side 1
// for w even, side 2 for w odd: 8 instructions of 8 rows) and multiplies
// output rows 32 (w % 2) .. +31 of block w / 2 against all 64 side-2 rows
// (2 x 4 16x16 MFMA steps per k-step, two k-steps per block); the two blocks'
// partial tiles are added in block order at the end.  Block rows keep the
// swizzle c ^ ((row/2) % 8).
namespace sr64 {
constexpr int kTM = 64, kTN = 64;
constexpr int kRows = kTM + kTN;            // 128 LDS rows per block
constexpr int kBlkB = 128;
constexpr int kUnitB = 2 * kBlkB;           // 256 bytes of width per unit
constexpr int kStage = 2 * kRows * kBlkB;   // 32 KB
constexpr int kNBuf = 4;                    // three stages in flight
constexpr int kDma = kRows / 2 / 8;         // 8 instructions per wave and stage
constexpr uint32_t kOob = 0x80000000u;
static_assert(kNBuf * kStage + 0 <= 160 * 1024, "LDS");
static_assert(kDma == 8 && kNBuf == 4, "the vmcnt wait below is 8 * (kNBuf - 2) = 16");
}  // namespace sr64

template <int DT>
__global__ __launch_bounds__(kThreads, 1) void score_ring64(RingArgs a) {
  __shared__ __attribute__((aligned(1024))) char smem[sr64::kNBuf * sr64::kStage];
  lds_char* const Ls = (lds_char*)smem;
  const uint32_t lds0 = (uint32_t)(uintptr_t)Ls;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int uwave = __builtin_amdgcn_readfirstlane(wave);
  const int bw = uwave >> 1, hw = uwave & 1;  // block and half of this wave (uniform)
  const int64_t tile = blockIdx.x / a.nwg, w = blockIdx.x % a.nwg;
  const int64_t tm = tile / a.tiles_n, tn = tile % a.tiles_n;
  const int64_t ub = uniform64(ring_first(w, a));
  const int nloc = __builtin_amdgcn_readfirstlane((int)(ring_first(w + 1, a) - ub));

  // DMA instruction i: LDS rows 64 hw + 8i .. +7 of block bw; lane l -> row
  // 64 hw + 8i + l/8 (side 1 row tm*64 + r, or side 2 row tn*64 + r - 64),
  // slot l%8 holding chunk (l%8) ^ ((row/2) % 8).
  bool rlive[sr64::kDma];
  uint32_t cbo[sr64::kDma];
#pragma unroll
  for (int i = 0; i < sr64::kDma; ++i) {
    const int r = 64 * hw + 8 * i + (lane >> 3);
    cbo[i] = 16u * (uint32_t)((lane & 7) ^ ((r >> 1) & 7));
    const int rl = r - 64 * hw;  // row within its side's tile
    const int64_t row = hw == 0 ? tm * sr64::kTM + rl : tn * sr64::kTN + rl;
    rlive[i] = row < (hw == 0 ? a.b1 : a.b2);
  }
  const bool nt = hw == 0 ? a.nt1 : a.nt2;  // uniform
  int il = 0;
  while (il + 1 < a.n_layers && a.layers[il + 1].u0 <= ub) ++il;
  int64_t iu = uniform64(ub - a.layers[il].u0);
  uint32_t roff[sr64::kDma];
  uint32_t lbytes = 0;
  int64_t lunits = 0, blk = 0, ld = 0;
  const char* mb = nullptr;  // this wave's side: the tile's first row
  auto set_layer = [&]() __attribute__((always_inline)) {
    const RingLayer& Ly = a.layers[il];
    ld = hw == 0 ? Ly.ld1 : Ly.ld2;
    blk = hw == 0 ? Ly.blk1 : Ly.blk2;
    mb = hw == 0 ? Ly.m1 + tm * sr64::kTM * Ly.ld1 : Ly.m2 + tn * sr64::kTN * Ly.ld2;
    lbytes = (uint32_t)min(Ly.bytes, (int64_t)0x7fffffff);
    lunits = Ly.units;
#pragma unroll
    for (int i = 0; i < sr64::kDma; ++i)
      roff[i] = rlive[i] ? (uint32_t)((lane >> 3) * ld + bw * blk) + cbo[i] : sr64::kOob;
  };
  auto issue = [&](int slot, bool live, bool more) __attribute__((always_inline)) {
    // instruction i's resource base: the unit's first block of row 8i (per-lane offsets span 8 rows)
    const uint32_t kin = (uint32_t)iu * sr64::kUnitB + (uint32_t)bw * sr64::kBlkB;
    const uint32_t dst0 = lds0 + (uint32_t)(slot * sr64::kStage + bw * sr64::kRows * sr64::kBlkB +
                                            64 * hw * sr64::kBlkB);
#pragma unroll
    for (int i = 0; i < sr64::kDma; ++i) {
      const u32x4 rs = uniform4(make_rsrc(mb + 8 * i * ld + iu * 2 * blk, 0x7fffffffu));
      const bool en = live & (roff[i] != sr64::kOob) & (kin + cbo[i] < lbytes);
      if (nt)
        dma16_nt(rs, dst0 + (uint32_t)(8 * i * sr64::kBlkB), en ? roff[i] : sr64::kOob);
      else
        dma16(rs, dst0 + (uint32_t)(8 * i * sr64::kBlkB), en ? roff[i] : sr64::kOob);
    }
    if (live && ++iu == lunits) {
      iu = 0;
      do {
        ++il;
      } while (il < a.n_layers && a.layers[il].units == 0);
      if (more) set_layer();
    }
  };

  set_layer();
  int ix = 0;
#pragma unroll
  for (int p = 0; p < sr64::kNBuf - 1; ++p, ++ix) issue(p, ix < nloc, ix + 1 < nloc);

  const int r16 = lane & 15, q = lane >> 4;
  const int sw = (r16 >> 1) & 7;
  f32x4 acc[2][4] = {};
  int slot = 0;
  for (int x = 0; x < nloc; ++x, ++ix) {
    asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(slot == 0 ? sr64::kNBuf - 1 : slot - 1, ix < nloc, ix + 1 < nloc);
    const lds_char* bb = Ls + slot * sr64::kStage + bw * sr64::kRows * sr64::kBlkB;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int so = (((4 * ks + q) ^ sw) << 4);
      u32x4 va[2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) va[rb] = *(const u32x4*)(bb + (32 * hw + 16 * rb + r16) * sr64::kBlkB + so);
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const u32x4 vb = *(const u32x4*)(bb + (sr64::kTM + 16 * cb + r16) * sr64::kBlkB + so);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) Mfma16<DT>::mma(acc[rb][cb], va[rb], vb);
      }
    }
    slot = slot + 1 == sr64::kNBuf ? 0 : slot + 1;
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  // the two blocks' partial tiles through LDS (64 x 64 fp32 each), summed in block order
  float* red = (float*)smem;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        red[(bw * sr64::kTM + 32 * hw + 16 * rb + acc16_row(e, lane)) * sr64::kTN + 16 * cb + acc16_col(lane)] =
            acc[rb][cb][e];
  __syncthreads();
  for (int x = tid; x < sr64::kTM * sr64::kTN; x += kThreads) {
    const int row = x / sr64::kTN, col = x % sr64::kTN;
    const float v = red[x] + red[sr64::kTM * sr64::kTN + x];
    const int64_t oi = tm * sr64::kTM + row, oj = tn * sr64::kTN + col;
    if (oi < a.b1 && oj < a.b2) a.partial[(oi * a.b2 + oj) * a.nwg + w] = v;
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

// Few partials per output (many output tiles, each with one or a few
// workgroups): one thread per output sums its partials in order.
constexpr int64_t kRowReduceMax = 32;
__global__ __launch_bounds__(256) void score_gemm_reduce_rows(const float* __restrict__ partial, int64_t n,
                                                              int64_t b1, int64_t b2, float* __restrict__ out,
                                                              int64_t ld_row, int64_t ld_col, int accumulate) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= b1 * b2) return;
  const float* p = partial + idx * n;
  float sum = 0.f;
  for (int64_t c = 0; c < n; ++c) sum += p[c];
  const int64_t i = idx / b2, j = idx - i * b2;
  float* o = out + i * ld_row + j * ld_col;
  *o = accumulate ? *o + sum : sum;
}

// Sum the n partials of every output into out.
int reduce_partials(const float* partial, int64_t n, int64_t b1, int64_t b2, float* out, int64_t ld_row,
                    int64_t ld_col, int accumulate, hipStream_t st) {
  const int64_t outs = b1 * b2;
  if (outs > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "da_score_gemm: too many outputs");
  if (n <= kRowReduceMax)
    score_gemm_reduce_rows<<<(unsigned)((outs + 255) / 256), 256, 0, st>>>(partial, n, b1, b2, out, ld_row,
                                                                            ld_col, accumulate);
  else
    score_gemm_reduce<<<(unsigned)outs, 256, 0, st>>>(partial, n, b1, b2, out, ld_row, ld_col, accumulate);
  return check_launch("da_score_gemm(reduce)");
}

// Stride between consecutive 128-byte blocks of a ring row, in bytes: a
// 64-element block of a 2-byte row is one 128-byte run at block stride blk
// (0: contiguous); 4-byte rows take the ring only when contiguous.
int64_t ring_block_stride(int64_t blk, int64_t es) { return es == 4 ? 128 : (blk ? blk : 64) * es; }

struct Plan {
  int64_t chunk_bytes, n_chunks;
  size_t ws;
  bool ring;              // streaming form (128-byte blocks at a fixed stride, offsets within 8 rows fit 32 bits)
  bool tall;              // its 64 x 64 tile (side 1 taller than one 16-row tile), else 16 x 64
  int64_t units, nwg;     // its units and workgroups per tile
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
  // Streaming form: rows whose 128-byte blocks sit a fixed stride apart --
  // every 2-byte layout (a 64-element block is one 128-byte run) and
  // contiguous 4-byte rows; the per-lane offsets within 8 rows and the row
  // widths fit 32 bits.
  const int64_t lim = (1LL << 31) - (1LL << 20);
  p->ring = (es == 2 || es == 4) && b1 > 0 && b2 > 0;
  p->tall = b1 > kTileM;
  const int64_t unit_b = p->tall ? sr64::kUnitB : sr::kUnitB;
  const int64_t tile_m = p->tall ? sr64::kTM : kTileM;
  int64_t units = 0;
  for (int l = 0; l < n_layers && p->ring; ++l) {
    const da_dense_layer& L = layers[l];
    const int64_t bytes = L.width * es, ld1 = L.ld1 * es, ld2 = L.ld2 * es;
    if (es == 4 && ((L.blk1 && L.blk1 != 64) || (L.blk2 && L.blk2 != 64))) p->ring = false;
    const int64_t bk1 = ring_block_stride(L.blk1, es), bk2 = ring_block_stride(L.blk2, es);
    if (bytes >= lim || 7 * ld1 + 4 * bk1 >= lim || 7 * ld2 + 4 * bk2 >= lim) p->ring = false;
    units += (bytes + unit_b - 1) / unit_b;
  }
  if (p->ring && units > 0) {
    int64_t slots = 0;
    const int rc = device_cu_count(&slots);
    if (rc) return rc;
    const int64_t tiles = ((b1 + tile_m - 1) / tile_m) * ((b2 + kTileN - 1) / kTileN);
    int64_t nwg = slots / tiles;
    // Workgroup w of every tile takes the same units at the same time; with
    // nwg a multiple of the 8 XCDs they also share an XCD (workgroups go to
    // the XCDs round-robin), so the rows the tiles have in common come from
    // that XCD's L2 once (3 tiles of 64 x 64 at 85 workgroups each read the
    // shared side three times).
    if (tiles > 1 && nwg > 8) nwg -= nwg % 8;
    if (nwg < 1) nwg = 1;
    if (nwg > units) nwg = units;
    p->units = units;
    p->nwg = nwg;
    if (tiles * nwg > 0x7fffffffLL || units / nwg > (1LL << 30)) p->ring = false;
    else p->ws = (size_t)(nwg * b1 * b2) * sizeof(float);
  } else {
    p->ring = false;
  }
  return DA_OK;
}

int run_plan(const Plan& p, int64_t b1, int64_t b2, const da_dense_layer* layers, int n_layers, int dtype,
             float* out, int64_t ld_row, int64_t ld_col, int accumulate, void* workspace,
             size_t workspace_bytes, hipStream_t st) {
  int rc = DA_OK;
  if (b1 == 0 || b2 == 0) return DA_OK;
  if (!out) return set_error(DA_ERR_INVALID, "da_score_gemm: out is NULL");
  if (p.n_chunks == 0) {
    if (accumulate) return DA_OK;
    if (ld_col != 1) return set_error(DA_ERR_INVALID, "da_score_gemm: empty product needs ld_col == 1");
    return zero_f32_2d(out, b1, b2, ld_row, st);
  }
  if (!workspace || workspace_bytes < p.ws)
    return set_error(DA_ERR_WORKSPACE, "da_score_gemm: workspace needs %zu bytes, got %zu", p.ws,
                     workspace_bytes);
  const int64_t es = (int64_t)elem_bytes(dtype);
  if (p.ring) {
    RingArgs r;
    r.n_layers = n_layers;
    int64_t u = 0;
    for (int l = 0; l < n_layers; ++l) {
      RingLayer& Ly = r.layers[l];
      Ly.m1 = (const char*)layers[l].m1;
      Ly.m2 = (const char*)layers[l].m2;
      Ly.bytes = layers[l].width * es;
      Ly.ld1 = layers[l].ld1 * es;
      Ly.ld2 = layers[l].ld2 * es;
      Ly.blk1 = ring_block_stride(layers[l].blk1, es);
      Ly.blk2 = ring_block_stride(layers[l].blk2, es);
      const int64_t unit_b = p.tall ? sr64::kUnitB : sr::kUnitB;
      Ly.units = (Ly.bytes + unit_b - 1) / unit_b;
      Ly.u0 = u;
      u += Ly.units;
    }
    const int64_t tile_m = p.tall ? sr64::kTM : kTileM;
    r.units = p.units;
    r.nwg = p.nwg;
    r.b1 = b1;
    r.b2 = b2;
    r.tiles_n = (b2 + kTileN - 1) / kTileN;
    r.partial = (float*)workspace;
    r.nt1 = r.tiles_n == 1;                     // side-1 rows meet one side-2 tile
    r.nt2 = (b1 + tile_m - 1) / tile_m == 1;    // side-2 rows meet one side-1 tile
    const int64_t tiles = ((b1 + tile_m - 1) / tile_m) * r.tiles_n;
    const unsigned grid = (unsigned)(tiles * p.nwg);
    if (p.tall) {
      switch (dtype) {
        case DA_BF16: score_ring64<DA_BF16><<<grid, kThreads, 0, st>>>(r); break;
        case DA_F16: score_ring64<DA_F16><<<grid, kThreads, 0, st>>>(r); break;
        default: score_ring64<DA_F32><<<grid, kThreads, 0, st>>>(r); break;
      }
    } else {
      switch (dtype) {
        case DA_BF16: score_ring<DA_BF16><<<grid, kThreads, 0, st>>>(r); break;
        case DA_F16: score_ring<DA_F16><<<grid, kThreads, 0, st>>>(r); break;
        default: score_ring<DA_F32><<<grid, kThreads, 0, st>>>(r); break;
      }
    }
    rc = check_launch("da_score_gemm(ring)");
    if (rc) return rc;
    return reduce_partials((const float*)workspace, p.nwg, b1, b2, out, ld_row, ld_col, accumulate, st);
  }
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
  return reduce_partials((const float*)workspace, p.n_chunks, b1, b2, out, ld_row, ld_col, accumulate, st);
}

// ---------------------------------------------------------------------------
// Per-row dot products of dense layers, summed over layers:
//
//   out[r] (+)= sum_L sum_c m1_L[r, c] * m2_L[r, c]     (m2_L = m1_L when NULL)
//
// -- the per-sample squared gradient norms of GradCos and the per-sample dots
// of two blocks, on the dense route.  HBM-bound: every weight is read once.
// The rows are walked block-major in stages of S consecutive 64-element blocks
// of R rows (R * S * C = kStage 16-byte chunks, kPer per thread), so in the
// k-blocked layout a stage reads S contiguous runs and in the row-major one R
// runs of S blocks.  Every layer starts a new stage (its blocks padded to whole
// stages), so the layer of a stage is uniform across the workgroup and its
// description comes through scalar loads.  A thread issues all its loads of a
// stage before the first product (chunks past the data read the layer's first
// chunk and are masked).  A workgroup owns one row tile and one range of stages
// and writes one fp32 partial per row; a second kernel adds a row's partials in
// range order (deterministic).
// ---------------------------------------------------------------------------
namespace rd {
constexpr int kThreads = 256;
constexpr int kPer = 8;                        // 16-byte chunks per thread and stage
constexpr int kStage = kThreads * kPer;        // chunks per stage
struct Layer {
  const char* m1;
  const char* m2;                              // == m1 for a squared norm
  int64_t ld1, blk1, ld2, blk2;                // bytes
  int64_t bytes;                               // row width in bytes
  int64_t stage0;                              // the layer's first stage
};
struct Args {
  Layer layers[kMaxLayers];
  int n_layers;
  int64_t rows;
  int64_t tile_rows, stage_blocks;             // R, S
  int64_t stages, ranges;                      // stages in all, stage ranges per row tile
  float* partial;                              // [rows][ranges]
};
}  // namespace rd

template <int DT>
__global__ __launch_bounds__(rd::kThreads) void row_dots_kernel(rd::Args a) {
  __shared__ float red[rd::kPer][rd::kThreads];
  constexpr int C = 4 * Elem<DT>::kBytes;      // 16-byte chunks per 64-element block
  constexpr int V = Elem<DT>::kVec;
  const int tid = threadIdx.x;
  const int R = (int)a.tile_rows, S = (int)a.stage_blocks;
  const int64_t rt = blockIdx.x / a.ranges, w = blockIdx.x % a.ranges;
  const int64_t st0 = w * a.stages / a.ranges, st1 = (w + 1) * a.stages / a.ranges;
  int row[rd::kPer], cb[rd::kPer], bo[rd::kPer];
  float acc[rd::kPer];
#pragma unroll
  for (int k = 0; k < rd::kPer; ++k) {
    const int q = tid + k * rd::kThreads;      // chunk q of a stage: block q / (R*C), row, chunk
    row[k] = (q % (R * C)) / C;
    cb[k] = q % C;
    bo[k] = q / (R * C);
    acc[k] = 0.f;
  }
  int l = 0;  // the stage's layer (uniform)
  for (int64_t st = st0; st < st1; ++st) {
    while (l + 1 < a.n_layers && st >= a.layers[l + 1].stage0) ++l;
    const rd::Layer& L = a.layers[l];
    const int64_t jb0 = (st - L.stage0) * S;
    u32x4 vx[rd::kPer], vy[rd::kPer];
    bool live[rd::kPer];
#pragma unroll
    for (int k = 0; k < rd::kPer; ++k) {
      const int64_t r = rt * R + row[k], jb = jb0 + bo[k];
      live[k] = r < a.rows && jb * 64 * Elem<DT>::kBytes + cb[k] * 16 < L.bytes;
      vx[k] = ld16(L.m1 + (live[k] ? r * L.ld1 + jb * L.blk1 + cb[k] * 16 : 0));
    }
    if (L.m2 != L.m1) {  // uniform
#pragma unroll
      for (int k = 0; k < rd::kPer; ++k) {
        const int64_t r = rt * R + row[k], jb = jb0 + bo[k];
        vy[k] = ld16(L.m2 + (live[k] ? r * L.ld2 + jb * L.blk2 + cb[k] * 16 : 0));
      }
    } else {
#pragma unroll
      for (int k = 0; k < rd::kPer; ++k) vy[k] = vx[k];
    }
#pragma unroll
    for (int k = 0; k < rd::kPer; ++k) {
      if (live[k]) {
        float x[V], y[V];
        unpack16<DT>(vx[k], x);
        unpack16<DT>(vy[k], y);
#pragma unroll
        for (int e = 0; e < V; ++e) acc[k] += x[e] * y[e];
      }
    }
  }
#pragma unroll
  for (int k = 0; k < rd::kPer; ++k) red[k][tid] = acc[k];
  __syncthreads();
  if (tid < R) {
    float sum = 0.f;
    for (int sb = 0; sb < S; ++sb)
      for (int c = 0; c < C; ++c) {
        const int q = (sb * R + tid) * C + c;
        sum += red[q / rd::kThreads][q % rd::kThreads];
      }
    const int64_t r = rt * R + tid;
    if (r < a.rows) a.partial[r * a.ranges + w] = sum;
  }
}

struct DotPlan {
  rd::Args args;
  int64_t row_tiles;
  size_t ws;
};

int row_dots_plan(int64_t rows, const da_dense_layer* layers, int n_layers, int dtype, DotPlan* p) {
  const char* who = "da_row_dots";
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "%s: bad dtype %d", who, dtype);
  if (rows < 0) return set_error(DA_ERR_INVALID, "%s: negative row count", who);
  if (n_layers < 0 || (n_layers > 0 && !layers)) return set_error(DA_ERR_INVALID, "%s: bad layer list", who);
  if (n_layers > kMaxLayers) return set_error(DA_ERR_INVALID, "%s: at most %d layers per call", who, kMaxLayers);
  const int64_t es = (int64_t)elem_bytes(dtype);
  const int64_t C = 4 * es;                       // chunks per block
  int64_t R = 1;
  while (R < rows && R * C < rd::kStage) R *= 2;  // rows per tile, a power of two with R * C <= kStage
  const int64_t S = rd::kStage / (R * C);         // blocks per stage
  rd::Args& a = p->args;
  a.n_layers = 0;
  int64_t stages = 0;
  for (int l = 0; l < n_layers; ++l) {
    const da_dense_layer& L = layers[l];
    const bool sq = L.m2 == nullptr;
    if (L.width < 0) return set_error(DA_ERR_INVALID, "%s: layer %d negative width", who, l);
    if (L.width == 0) continue;
    const int64_t blk1 = L.blk1 ? L.blk1 : 64, blk2 = sq ? blk1 : (L.blk2 ? L.blk2 : 64);
    const int64_t ld2 = sq ? L.ld1 : L.ld2;
    if ((L.width * es) % 16 || (L.ld1 * es) % 16 || (ld2 * es) % 16 || blk1 < 64 || blk2 < 64 ||
        (blk1 * es) % 16 || (blk2 * es) % 16)
      return set_error(DA_ERR_INVALID, "%s: layer %d width, strides and block strides must be 16-byte multiples "
                       "(block strides >= 64 elements)", who, l);
    if (!L.m1 || ((uintptr_t)L.m1 & 15) || (!sq && ((uintptr_t)L.m2 & 15)))
      return set_error(DA_ERR_INVALID, "%s: layer %d pointers NULL or misaligned", who, l);
    rd::Layer& D = a.layers[a.n_layers++];
    D.m1 = (const char*)L.m1;
    D.m2 = sq ? D.m1 : (const char*)L.m2;
    D.ld1 = L.ld1 * es;
    D.ld2 = ld2 * es;
    D.blk1 = blk1 * es;
    D.blk2 = blk2 * es;
    D.bytes = L.width * es;
    D.stage0 = stages;
    stages += ((L.width + 63) / 64 + S - 1) / S;  // the layer's blocks in whole stages
  }
  a.rows = rows;
  a.tile_rows = R;
  a.stage_blocks = S;
  a.stages = stages;
  p->row_tiles = rows > 0 ? (rows + R - 1) / R : 0;
  a.ranges = 1;
  p->ws = 0;
  if (rows == 0 || a.stages == 0) return DA_OK;
  int64_t cus = 0;
  const int rc = device_cu_count(&cus);
  if (rc) return rc;
  int64_t ranges = 4 * cus / p->row_tiles;         // ~4 workgroups per CU in all
  const int64_t most = a.stages / 8 > 0 ? a.stages / 8 : 1;  // at least 8 stages per workgroup
  if (ranges > most) ranges = most;
  if (ranges < 1) ranges = 1;
  a.ranges = ranges;
  if (p->row_tiles * ranges > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: problem too large", who);
  p->ws = (size_t)(rows * ranges) * sizeof(float);
  return DA_OK;
}

// The allocation-free entry point keeps its partials in this file-scope
// device array (one copy per GPU, alive until the process ends).  Host code
// must never pass `scratch` itself to a kernel: its name is a host-side
// stand-in, so kernels take the device address scratch_address() resolves.
constexpr size_t kScratchBytes = DA_SCORE_GEMM_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

// Device address of this GPU's scratch, resolved with the device current on
// its first use and cached per device (racing threads store the same value).
int scratch_address(float** ptr) {
  static std::atomic<float*> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(DA_ERR_HIP, "da_score_gemm_noalloc: hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(DA_ERR_UNSUPPORTED, "da_score_gemm_noalloc: device %d beyond the %d the library tracks", dev,
                     kMaxDevices);
  float* p = cache[dev].load(std::memory_order_acquire);
  if (!p) {
    void* addr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !addr)
      return set_error(DA_ERR_HIP, "da_score_gemm_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                       hipGetErrorString(e));
    p = (float*)addr;
    cache[dev].store(p, std::memory_order_release);
  }
  *ptr = p;
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
  da::Plan p;
  const int rc = da::make_plan(b1, b2, layers, n_layers, dtype, &p);
  if (rc) return rc;
  return da::run_plan(p, b1, b2, layers, n_layers, dtype, out, ld_row, ld_col, accumulate, workspace,
                      workspace_bytes, (hipStream_t)stream);
}

int da_score_gemm_noalloc(int64_t b1, int64_t b2, const da_dense_layer* layers, int n_layers, int dtype,
                          float* out, int64_t ld_row, int64_t ld_col, int accumulate, void* stream) {
  da::Plan p;
  int rc = da::make_plan(b1, b2, layers, n_layers, dtype, &p);
  if (rc) return rc;
  if (p.ws > da::kScratchBytes)
    return da::set_error(DA_ERR_WORKSPACE,
                         "da_score_gemm_noalloc: %lld x %lld outputs need %zu bytes of partials, more than the "
                         "%zu-byte scratch; call da_score_gemm with a workspace instead",
                         (long long)b1, (long long)b2, p.ws, da::kScratchBytes);
  float* ptr = nullptr;
  rc = da::scratch_address(&ptr);
  if (rc) return rc;
  return da::run_plan(p, b1, b2, layers, n_layers, dtype, out, ld_row, ld_col, accumulate, ptr, da::kScratchBytes,
                      (hipStream_t)stream);
}

int da_row_dots_workspace(int64_t rows, const da_dense_layer* layers, int n_layers, int dtype, size_t* bytes) {
  da::DotPlan p;
  const int rc = da::row_dots_plan(rows, layers, n_layers, dtype, &p);
  if (rc) return rc;
  if (!bytes) return da::set_error(DA_ERR_INVALID, "da_row_dots_workspace: bytes is NULL");
  *bytes = p.ws;
  return DA_OK;
}

int da_row_dots(int64_t rows, const da_dense_layer* layers, int n_layers, int dtype, float* out,
                int64_t out_stride, int accumulate, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace da;
  DotPlan p;
  int rc = row_dots_plan(rows, layers, n_layers, dtype, &p);
  if (rc) return rc;
  if (rows == 0) return DA_OK;
  if (!out || out_stride < 1) return set_error(DA_ERR_INVALID, "da_row_dots: out is NULL or out_stride < 1");
  hipStream_t st = (hipStream_t)stream;
  if (p.args.stages == 0) return accumulate ? DA_OK : zero_f32_2d(out, rows, 1, out_stride, st);
  if (!workspace || workspace_bytes < p.ws)
    return set_error(DA_ERR_WORKSPACE, "da_row_dots: workspace needs %zu bytes, got %zu", p.ws, workspace_bytes);
  p.args.partial = (float*)workspace;
  const unsigned grid = (unsigned)(p.row_tiles * p.args.ranges);
  switch (dtype) {
    case DA_BF16: row_dots_kernel<DA_BF16><<<grid, rd::kThreads, 0, st>>>(p.args); break;
    case DA_F16: row_dots_kernel<DA_F16><<<grid, rd::kThreads, 0, st>>>(p.args); break;
    default: row_dots_kernel<DA_F32><<<grid, rd::kThreads, 0, st>>>(p.args); break;
  }
  rc = check_launch("da_row_dots");
  if (rc) return rc;
  return reduce_partials((const float*)workspace, p.args.ranges, rows, 1, out, out_stride, 1, accumulate, st);
}

}  // extern "C"
