// K2: random projection of factor rows, and the fused capture-time projection
// + per-sample outer-product sum (LoGRA-style, double-sided).
//
//   project_rows:  out[r, c] = sum_j x[r, j] * P[j, c] (+ bias[c])
//     follows ProjectionMatrix.__call__, dattri_llm/gradient/ops/projection.py:363-370
//     (flat @ P, or addmm(bias_row, flat, P)).
//
//   project_outer: M[b, o, i] = sum_t (g[b,t,:] P_out)[o] * (a[b,t,:] P_in (+ bias_in))[i]
//     follows the capture path of hooks.py:631-648: project the activation with
//     proj_seed+1 and the gradient with proj_seed (projection.py:437-440,
//     :476-488), then materialize_factors(a_p, g_p, "nn.Linear"), i.e.
//     bmm(g_p^T, a_p) flattened to (B, k_g*k_a) (materialize.py:114-116).
//
// Both are bound by streaming the factor rows from HBM (the projected widths
// are <= 64, so every input byte meets at most 2*64 flops); each factor row is
// read once.
//
//   project_rows_stream  128-token chunks, factor and projection rows staged
//                        HBM -> LDS by buffer loads (da_project_rows).
//   project_pieces       stream-K over both sides of da_project_outer: equal
//                        ranges of 512-byte k-blocks per workgroup, fp32 partial
//                        projections ("pieces") at item boundaries;
//   outer_from_pieces    then sums each sample's pieces in a fixed order and
//                        contracts them on fp32 MFMAs.
//   project_tile / project_outer_kernel / project_rows_kernel: register-fed
//                        kernels for rows the buffer-offset paths cannot address.
#include "common.h"

namespace da {
namespace {

constexpr int kThreads = 256;
constexpr int kRows = 64;                 // rows per workgroup (4 waves x 16)
constexpr int kCols = 64;                 // projected columns per workgroup
constexpr int kStage = 256;               // bytes of feature width per stage
constexpr int kPtRow = kStage + 16;       // padded LDS row of P^T
constexpr int kPtBytes = kCols * kPtRow;  // one LDS stage of P^T

// acc[cb][e] += sum over the width of x[row(lane,e)] * pt[16*cb + col(lane)],
// rows = this wave's 16 rows.  xrow: this lane's row (nullptr = zero row).
template <int DT>
__device__ __forceinline__ void project_tile(const char* xrow, int64_t wbytes, const char* pt,
                                             int64_t pt_rstride, int ncols, char* lds,
                                             f32x4 (&acc)[4], int tid, int lane) {
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int q = lane >> 4, r = lane & 15;
  const int prow = tid >> 4, pch = tid & 15;  // P^T staging: 16 rows x 16 chunks per pass
  const int nk = (int)((wbytes + kStage - 1) / kStage);
  u32x4 xv[4], pv[4];

  auto load_x = [&](int kt) {
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int64_t off = (int64_t)kt * kStage + 64 * st + 16 * q;
      xv[st] = (xrow && off < wbytes) ? ld16(xrow + off) : u32x4{0, 0, 0, 0};
    }
  };
  auto load_p = [&](int kt) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int c = prow + 16 * p;
      const int64_t off = (int64_t)kt * kStage + 16 * pch;
      pv[p] = (c < ncols && off < wbytes) ? ld16(pt + c * pt_rstride + off) : u32x4{0, 0, 0, 0};
    }
  };
  auto store_p = [&](int buf) {
    char* base = lds + buf * kPtBytes;
#pragma unroll
    for (int p = 0; p < 4; ++p) st16(base + (prow + 16 * p) * kPtRow + 16 * pch, pv[p]);
  };

  load_p(0);
  store_p(0);
  load_x(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    u32x4 cur[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) cur[st] = xv[st];
    if (kt + 1 < nk) {
      load_x(kt + 1);
      load_p(kt + 1);
    }
    const char* base = lds + (kt & 1) * kPtBytes;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const u32x4 b = ld16(base + (16 * cb + r) * kPtRow + 64 * st + 16 * q);
        Mfma16<DT>::mma(acc[cb], cur[st], b);
      }
    if (kt + 1 < nk) store_p((kt + 1) & 1);
    __syncthreads();
  }
}

struct RowsArgs {
  const char* x;
  int64_t rows, wbytes, x_rstride;  // bytes
  const char* pt;
  int64_t pt_rstride;               // bytes
  int64_t k;
  const float* bias;                // k floats or nullptr
  char* out;
  int64_t out_rstride;              // elements
};

template <int DT, int OT>
__global__ __launch_bounds__(kThreads) void project_rows_kernel(RowsArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[2 * kPtBytes];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * kRows;
  const int64_t c0 = (int64_t)blockIdx.y * kCols;
  const int64_t row = r0 + 16 * wave + (lane & 15);
  const char* xrow = row < a.rows ? a.x + row * a.x_rstride : nullptr;
  const int ncols = (int)min((int64_t)kCols, a.k - c0);
  f32x4 acc[4];
  project_tile<DT>(xrow, a.wbytes, a.pt + c0 * a.pt_rstride, a.pt_rstride, ncols, lds, acc, tid, lane);
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t orow = r0 + 16 * wave + acc16_row(e, lane);
      const int64_t ocol = c0 + 16 * cb + acc16_col(lane);
      if (orow < a.rows && ocol < a.k)
        Elem<OT>::store(a.out, orow * a.out_rstride + ocol, acc[cb][e] + (a.bias ? a.bias[ocol] : 0.f));
    }
}

struct OuterArgs {
  const char* a;
  const char* g;
  int64_t batch, tokens;
  int64_t a_bstride, a_tstride, g_bstride, g_tstride;  // bytes
  int64_t abytes, gbytes;                              // row widths in bytes
  const char* pin_t;                                   // (ka, K) transposed P_in
  const char* pout_t;                                  // (kg, D) transposed P_out
  int64_t pin_rstride, pout_rstride;                   // bytes
  int ka, kg;
  const float* bias_in;                                // ka floats or nullptr
  int64_t chunks;                                      // 64-token chunks per sample
  float* partial;                                      // [batch][chunks][kg][ka]
};

template <int DT>
__global__ __launch_bounds__(kThreads) void project_outer_kernel(OuterArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[2 * kPtBytes];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.x / a.chunks, chunk = blockIdx.x % a.chunks;
  const int64_t t = chunk * kRows + 16 * wave + (lane & 15);
  const bool valid = t < a.tokens;
  const char* arow = valid ? a.a + b * a.a_bstride + t * a.a_tstride : nullptr;
  const char* grow = valid ? a.g + b * a.g_bstride + t * a.g_tstride : nullptr;

  f32x4 pa[4], pg[4];
  project_tile<DT>(arow, a.abytes, a.pin_t, a.pin_rstride, a.ka, lds, pa, tid, lane);
  project_tile<DT>(grow, a.gbytes, a.pout_t, a.pout_rstride, a.kg, lds, pg, tid, lane);

  // Park both projected chunks (tokens x 64, fp32) in LDS; the stage buffers
  // are free (project_tile ends with a barrier).
  float* ap = (float*)lds;        // [64 tokens][64]
  float* gp = ap + kRows * kCols;  // [64 tokens][64]
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tok = 16 * wave + acc16_row(e, lane);
      const int col = 16 * cb + acc16_col(lane);
      const bool tv = chunk * kRows + tok < a.tokens;
      const float bias = (a.bias_in && col < a.ka && tv) ? a.bias_in[col] : 0.f;
      ap[tok * kCols + col] = pa[cb][e] + bias;
      gp[tok * kCols + col] = pg[cb][e];
    }
  __syncthreads();
  // M[o][i] = sum_tok gp[tok][o] * ap[tok][i]: thread -> one o, 16 consecutive i.
  const int o = tid >> 2, i0 = (tid & 3) * 16;
  float m[16];
#pragma unroll
  for (int x = 0; x < 16; ++x) m[x] = 0.f;
  for (int tok = 0; tok < kRows; ++tok) {
    const float gv = gp[tok * kCols + o];
    const float* arow_l = ap + tok * kCols + i0;
#pragma unroll
    for (int x = 0; x < 16; ++x) m[x] += gv * arow_l[x];
  }
  if (o < a.kg) {
    float* dst = a.partial + ((b * a.chunks + chunk) * a.kg + o) * a.ka;
#pragma unroll
    for (int x = 0; x < 16; ++x)
      if (i0 + x < a.ka) dst[i0 + x] = m[x];
  }
}

// ---------------------------------------------------------------------------
// Streaming projection (the gfx950 path).
//
// project_rows_stream: out[b, t, c] = sum_j x[b, t, j] * P[j, c] (+ bias[c])
// for up to kMaxPGroups (x, P) pairs in one launch -- the activation and the
// gradient side of a fused capture share a launch, so the two row streams
// (of different widths) pack the GPU together, widest first.
//
// A workgroup owns a 128-token chunk of one sample of one group.  Factor rows
// and projection rows go HBM -> LDS by buffer loads with the LDS-direct bit
// (each instruction 4 rows x 256 contiguous bytes) through a ring of three
// 48 KB stages (128 factor rows + 64 projection rows, 256 bytes of width
// each), two stages in flight.  Each wave multiplies its 32 rows against the
// 64 projection rows with 16x16x32 MFMAs read from LDS; a 16-byte-chunk XOR
// swizzle by row (c ^ row % 16) keeps those reads conflict-free.  The chunk's
// results are staged through LDS and leave as 16-byte row stores.
// ---------------------------------------------------------------------------
namespace ps {
constexpr int kTok = 128;                // tokens per workgroup
constexpr int kRows = kTok + kCols;      // LDS rows per stage
constexpr int kSB = 128;                 // bytes of width per row and stage (two 64-byte k-steps)
constexpr int kStage = kRows * kSB;      // 24 KB
constexpr int kNBuf = 3;                 // two stages in flight, two workgroups per CU
constexpr int kDma = kRows * (kSB / 16) / (kWave * 4);  // 6 instructions per wave and stage
constexpr int kKs = kSB / 64;            // 16x16x32 k-steps per stage
constexpr uint32_t kOob = 0x80000000u;
constexpr int kMaxPGroups = 4;
static_assert(kDma == 6 && kNBuf == 3, "the vmcnt wait below is 6 * (kNBuf - 2) = 6");
static_assert(2 * kTok * 64 * 4 <= kNBuf * kStage, "output staging must fit the ring");
}  // namespace ps

struct PGroup {
  const char* x;                // factor rows: sample b, token t at x + b*bstride + t*tstride
  int64_t batch, tokens, bstride, tstride, wbytes;  // bytes
  const char* pt;               // (ncols, width) transposed projection, rows pt_rstride bytes apart
  int64_t pt_rstride;
  int ncols;                    // <= 64
  const float* bias;            // ncols floats or nullptr
  char* out;                    // out + (b*out_bstride + t*out_tstride + c) elements
  int64_t out_bstride, out_tstride;
  int64_t chunks;               // 128-token chunks per sample
  int64_t wg0;                  // first workgroup of this group
};

struct PGroupArgs {
  PGroup g[ps::kMaxPGroups];
  int n;
};

template <int DT, int OT>
__global__ __launch_bounds__(kThreads, 2) void project_rows_stream(PGroupArgs args) {
  __shared__ __attribute__((aligned(1024))) char smem[ps::kNBuf * ps::kStage];
  lds_char* const L = (lds_char*)smem;
  const uint32_t lds0 = (uint32_t)(uintptr_t)L;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int uwave = __builtin_amdgcn_readfirstlane(wave);
  // Dispatch order, not an XCD-contiguous remap: the widest group comes
  // first and every XCD should take its share of it.
  const int64_t wg = blockIdx.x;
  int gi = 0;
  while (gi + 1 < args.n && args.g[gi + 1].wg0 <= wg) ++gi;
  const PGroup& G = args.g[gi];
  const int64_t local = wg - G.wg0;
  const int64_t b = local / G.chunks, chunk = local % G.chunks;
  const int64_t tok0 = chunk * ps::kTok;
  const int nst = (int)((G.wbytes + ps::kSB - 1) / ps::kSB);
  const u32x4 rx = uniform4(make_rsrc(G.x + b * G.bstride, 0x7fffffffu));
  const u32x4 rp = uniform4(make_rsrc(G.pt, 0x7fffffffu));
  // DMA instruction j of this wave: rows 8*(6w + j) .. +7 (rows < 128 are
  // factor rows, then projection rows); lane l -> row 8*(6w+j) + l/8, slot l%8
  // holding logical chunk (l%8) ^ (row%8).
  uint32_t rof[ps::kDma], cb[ps::kDma];
#pragma unroll
  for (int j = 0; j < ps::kDma; ++j) {
    const int row = 8 * (ps::kDma * wave + j) + (lane >> 3);
    cb[j] = 16u * (uint32_t)((lane & 7) ^ (row & 7));
    const int64_t t = tok0 + row;
    const int c = row - ps::kTok;
    rof[j] = row < ps::kTok ? (t < G.tokens ? (uint32_t)(t * G.tstride) : ps::kOob)
                            : (c < G.ncols ? (uint32_t)(c * G.pt_rstride) : ps::kOob);
  }
  auto issue = [&](int st) __attribute__((always_inline)) {
    const uint32_t koff = (uint32_t)st * ps::kSB;
    const uint32_t base = lds0 + (uint32_t)((st % ps::kNBuf) * ps::kStage + ps::kDma * uwave * 8 * ps::kSB);
#pragma unroll
    for (int j = 0; j < ps::kDma; ++j) {
      const bool xrow = ps::kDma * uwave + j < ps::kTok / 8;  // uniform
      const uint32_t mx = xrow ? 0xffffffffu : 0u;
      u32x4 rs;
#pragma unroll
      for (int c = 0; c < 4; ++c) rs[c] = (rx[c] & mx) | (rp[c] & ~mx);
      const bool en = st < nst && rof[j] != ps::kOob && (int64_t)(koff + cb[j]) < G.wbytes;
      dma16(rs, base + (uint32_t)(j * 8 * ps::kSB), en ? rof[j] + koff + cb[j] : ps::kOob);
    }
  };

  // Fragments: factor rows 32w + 16rb + l%16, projection rows 128 + 16c + l%16;
  // k-step ks reads logical chunk 4ks + l/16 in slot (4ks + l/16) ^ (row%8),
  // row%8 = l%8: the 8 lanes one LDS cycle serves hit 8 distinct slots.
  const int r16 = lane & 15, q = lane >> 4;
  f32x4 acc[2][4];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[rb][c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s0 = 0; s0 < ps::kNBuf - 1; ++s0) issue(s0);
  for (int st = 0; st < nst; ++st) {
    // this wave's loads of stage st done (the later kNBuf - 2 stages, 24
    // instructions, may be in flight), its LDS reads done; then every wave's
    // part is visible and the buffer read one stage ago may be refilled
    asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(st + ps::kNBuf - 1);
    const lds_char* sb = L + (st % ps::kNBuf) * ps::kStage;
#pragma unroll
    for (int ks = 0; ks < ps::kKs; ++ks) {
      const int off = r16 * ps::kSB + (((4 * ks + q) ^ (r16 & 7)) << 4);
      u32x4 xf[2], pf[4];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) xf[rb] = *(const u32x4*)(sb + (32 * wave + 16 * rb) * ps::kSB + off);
#pragma unroll
      for (int c = 0; c < 4; ++c) pf[c] = *(const u32x4*)(sb + (ps::kTok + 16 * c) * ps::kSB + off);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int c = 0; c < 4; ++c) Mfma16<DT>::mma(acc[rb][c], xf[rb], pf[c]);
    }
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");

  // Stage the chunk (128 x 64, output dtype) in the ring, then 16-byte stores.
  constexpr int OS = Elem<OT>::kBytes;
  constexpr int ROWB = kCols * OS;
  char* obuf = smem;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tok = 32 * wave + 16 * rb + acc16_row(e, lane);
        const int col = 16 * c + acc16_col(lane);
        const float bias = (G.bias && col < G.ncols) ? G.bias[col] : 0.f;
        Elem<OT>::store(obuf, (int64_t)tok * kCols + col, acc[rb][c][e] + bias);
      }
  __syncthreads();
  constexpr int CH = ROWB / 16;
  const int64_t wcols = G.ncols;
  for (int idx = tid; idx < ps::kTok * CH; idx += kThreads) {
    const int tok = idx / CH, ch = idx % CH;
    const int64_t t = tok0 + tok;
    const int64_t c0 = (int64_t)ch * (16 / OS);
    if (t >= G.tokens || c0 >= wcols) continue;
    char* dst = G.out + (b * G.out_bstride + t * G.out_tstride + c0) * OS;
    const char* src = obuf + tok * ROWB + ch * 16;
    if (c0 + 16 / OS <= wcols && ((uintptr_t)dst & 15) == 0) {
      st16(dst, ld16(src));
    } else {
      for (int64_t c = c0; c < wcols && c < c0 + 16 / OS; ++c)
        for (int by = 0; by < OS; ++by) dst[(c - c0) * OS + by] = src[(c - c0) * OS + by];
    }
  }
}

// Stream-K capture projection.  The work of da_project_outer is the stage
// sequence (side, item, stage): side 0 = activations with P_in, side 1 =
// gradients with P_out; an item is one 128-token chunk of one sample; a stage
// is 128 bytes of feature width of the item's rows (plus the same bytes of the
// 64 P^T rows).  Workgroup w of nwg owns stages [w*total/nwg, (w+1)*total/nwg)
// and streams them through one DMA ring without draining it at item
// boundaries; at the end of each item (or of its range) it writes its fp32
// partial projection, a "piece", to slot item + w.  Along the stage sequence
// every new piece advances the item, the workgroup or both, so item + w is
// strictly increasing: slots are unique and < items + nwg.  The pieces of an
// item are those of workgroups sk_owner(first stage) .. sk_owner(last stage);
// outer_from_pieces sums them in that order, so the result does not depend on
// timing.
struct SkSide {
  const char* x;                // sample b, token t at x + b*bstride + t*tstride (bytes)
  int64_t bstride, tstride, wbytes;
  const char* pt;               // (ncols, width) transposed projection
  int64_t pt_rstride;
  int ncols, nst;               // projected width (<= 64), stages per item
  int64_t items, s0, i0;        // items of this side, its first stage, its first item
  const float* bias;            // ncols floats added to this side's projected rows, or nullptr
};

struct SkArgs {
  SkSide s[2];
  int64_t batch, tokens, chunks, total;  // samples, tokens per sample, 128-token chunks, stages of both sides
  int64_t nwg;
  float* pieces;                // (items of both sides + nwg) pieces of kPieceFloats
};

constexpr int kPieceFloats = ps::kTok * kCols;  // one piece: 128 tokens x 64 columns, MFMA layout

__device__ __forceinline__ int64_t sk_first(int64_t w, const SkArgs& a) { return w * a.total / a.nwg; }
// the workgroup whose range holds stage x
__device__ __forceinline__ int64_t sk_owner(int64_t x, const SkArgs& a) { return ((x + 1) * a.nwg - 1) / a.total; }

namespace sk {
constexpr int kKB = 512;                          // bytes of width per k-block
constexpr int kRG = 32;                           // factor rows per stage (a row group)
constexpr int kNRG = ps::kTok / kRG;              // 4 stages per k-block
constexpr int kFStage = kRG * kKB;                // 16 KB
constexpr int kNF = 6;                            // factor ring depth
constexpr int kPBlock = kCols * kKB;              // 32 KB of projection rows per k-block
constexpr int kLds = kNF * kFStage + 2 * kPBlock; // 160 KB: one workgroup per CU
constexpr int kFDma = kFStage / 1024 / 4;         // 4 instructions per wave and stage
constexpr int kPDma = kPBlock / 1024 / 4;         // 8 instructions per wave and k-block
constexpr int kKs = kKB / 64;                     // 8 MFMA k-steps per stage
static_assert(kFDma == 4 && kPDma == 8 && kNF == 6 && kNRG == 4,
              "the vmcnt waits below (12 and 24) assume these counts");
}  // namespace sk

// The stream-K unit is a k-block of an item: 512 bytes of width of its 128
// rows, read as four stages of one row group (32 rows) each, every DMA
// instruction two 512-byte runs.  Per side nst = ceil(width / 512) units per
// item.  The factor stages stream through a 6-deep ring; the unit's projection
// rows (64 x 512 B) are double-buffered and serve its four stages.  Wave w owns
// output columns 16w .. 16w+15 for all 128 tokens: per stage it runs 2 x 8
// MFMAs into the accumulators of that row group (static indices: the unit loop
// is unrolled over its four stages).
template <int DT>
__global__ __launch_bounds__(kThreads, 1) void project_pieces(SkArgs args) {
  __shared__ __attribute__((aligned(1024))) char smem[sk::kLds];
  lds_char* const L = (lds_char*)smem;
  const uint32_t lds0 = (uint32_t)(uintptr_t)L;
  const uint32_t ldsp = lds0 + sk::kNF * sk::kFStage;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int uwave = __builtin_amdgcn_readfirstlane(wave);
  const int64_t w = blockIdx.x;
  const int64_t ub = uniform64(sk_first(w, args));
  const int nu = __builtin_amdgcn_readfirstlane((int)(sk_first(w + 1, args) - ub));  // units of this workgroup
  const int nstage = sk::kNRG * nu;

  // Lane roles.  Factor instruction j of wave w: stage rows 8w + 2j + l/32;
  // projection instruction j: projection rows 16w + 2j + l/32.  Lane l writes
  // slot l%32 of its 512-byte LDS row, holding logical chunk (l%32) ^ (row%16):
  // a 16-byte read serves 16 lanes (256 bytes of banks) per cycle, and the 16
  // rows of a fragment, 512 bytes apart, then hit 16 distinct bank groups.
  uint32_t fcb[sk::kFDma], pcb[sk::kPDma];
  int frow[sk::kFDma], prow[sk::kPDma];
#pragma unroll
  for (int j = 0; j < sk::kFDma; ++j) {
    frow[j] = 8 * wave + 2 * j + (lane >> 5);
    fcb[j] = 16u * (uint32_t)((lane & 31) ^ (frow[j] & 15));
  }
#pragma unroll
  for (int j = 0; j < sk::kPDma; ++j) {
    prow[j] = 16 * wave + 2 * j + (lane >> 5);
    pcb[j] = 16u * (uint32_t)((lane & 31) ^ (prow[j] & 15));
  }

  // Factor cursor: side is, item ii, unit iu, row group ir, and its item's state.
  int is = ub >= args.s[1].s0 ? 1 : 0;
  int64_t ii = uniform64((ub - args.s[is].s0) / args.s[is].nst);
  int iu = __builtin_amdgcn_readfirstlane((int)(ub - args.s[is].s0 - ii * args.s[is].nst)), ir = 0;
  const int xs0 = is, xu0 = iu;
  const int64_t xi0 = ii;
  u32x4 rx;
  uint32_t fwb = 0, ftst = 0;
  int64_t fnv = 0, fitems = 0;
  int fnu = 0;
  auto set_item = [&]() __attribute__((always_inline)) {
    const SkSide& S = args.s[is];
    const int64_t b = uniform64(ii / args.chunks), t0 = (ii - b * args.chunks) * ps::kTok;
    rx = uniform4(make_rsrc(S.x + b * S.bstride + t0 * S.tstride, 0x7fffffffu));
    fwb = (uint32_t)S.wbytes;
    ftst = (uint32_t)S.tstride;
    fnv = args.tokens - t0;  // valid rows of this chunk (may exceed 128)
    fnu = S.nst;
    fitems = S.items;
  };
  auto issue_f = [&](uint32_t dst0, bool live, bool more) __attribute__((always_inline)) {
    const uint32_t koff = (uint32_t)iu * sk::kKB;
#pragma unroll
    for (int j = 0; j < sk::kFDma; ++j) {
      const int row = 32 * ir + frow[j];
      const bool en = live & (row < fnv) & (koff + fcb[j] < fwb);
      dma16_nt(rx, dst0 + (uint32_t)((8 * uwave + 2 * j) * sk::kKB),
               en ? (uint32_t)row * ftst + koff + fcb[j] : ps::kOob);
    }
    if (live && ++ir == sk::kNRG) {
      ir = 0;
      if (++iu == fnu) {
        iu = 0;
        if (++ii == fitems) {
          ii = 0;
          ++is;
        }
        if (more) set_item();
      }
    }
  };

  // Projection cursor: side pside, item pitem, unit pu (one issue per unit).
  int pside = xs0, pu = xu0, pnu = 0, pcols = 0;
  int64_t pitem = xi0, pitems = 0;
  u32x4 rp;
  uint32_t pwb = 0, prs = 0;
  auto set_side = [&]() __attribute__((always_inline)) {
    const SkSide& S = args.s[pside];
    rp = uniform4(make_rsrc(S.pt, 0x7fffffffu));
    pwb = (uint32_t)S.wbytes;
    prs = (uint32_t)S.pt_rstride;
    pnu = S.nst;
    pitems = S.items;
    pcols = S.ncols;
  };
  auto issue_p = [&](uint32_t dst0) __attribute__((always_inline)) {
    const bool live = pside < 2;  // uniform; past the last side: zero fill
    const uint32_t koff = (uint32_t)pu * sk::kKB;
#pragma unroll
    for (int j = 0; j < sk::kPDma; ++j) {
      const bool en = live & (prow[j] < pcols) & (koff + pcb[j] < pwb);
      dma16(rp, dst0 + (uint32_t)((16 * uwave + 2 * j) * sk::kKB),
            en ? (uint32_t)prow[j] * prs + koff + pcb[j] : ps::kOob);
    }
    if (live && ++pu == pnu) {
      pu = 0;
      if (++pitem == pitems) {
        pitem = 0;
        if (++pside < 2) set_side();
      }
    }
  };

  set_item();
  set_side();
  issue_p(ldsp);
  issue_p(ldsp + sk::kPBlock);
  int ix = 0;  // next factor stage to issue, relative to the first
#pragma unroll
  for (int p = 0; p < sk::kNF - 1; ++p, ++ix) issue_f(lds0 + p * sk::kFStage, ix < nstage, ix + 1 < nstage);

  const int r16 = lane & 15, q = lane >> 4;
  f32x4 acc[8];  // row block tb = 2 * row group + rb: tokens 16tb .., columns 16w ..
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  int fslot = 0, islot = sk::kNF - 1, pslot = 0;
  // One unit.  Waits: this wave's loads of the stage (and, at row group 0, of
  // the unit's projection rows) must be done; later loads and piece stores may
  // be pending (loads complete in order).  At row group 0 the projection load
  // was issued one unit earlier, after the stage's own loads: 12 may stay
  // pending.  At row groups 1-3 of every unit but the first, the projection
  // load of this unit's row group 0 lies between the stage's loads and now:
  // 24 may stay pending.  Then every wave's part is visible and the slots read
  // before may be refilled.
  u32x4 pf[sk::kKs];
  auto unit = [&](auto firstc) __attribute__((always_inline)) {
    constexpr bool kFirst = decltype(firstc)::value;
    const lds_char* pb = L + sk::kNF * sk::kFStage + (16 * wave + r16) * sk::kKB;
#pragma unroll
    for (int r = 0; r < sk::kNRG; ++r) {
      if (r == 0 || kFirst)
        asm volatile("s_waitcnt vmcnt(12) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(24) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      issue_f(lds0 + islot * sk::kFStage, ix < nstage, ix + 1 < nstage);
      ++ix;
      islot = islot + 1 == sk::kNF ? 0 : islot + 1;
      if (r == 0 && !kFirst) {
        pslot ^= 1;                                // this unit's projection rows
        issue_p(ldsp + (pslot ^ 1) * sk::kPBlock);  // the next unit's, into the freed buffer
      }
      if (r == 0) {  // this wave's projection fragments of the unit, kept for its four stages
        const lds_char* pbs = pb + pslot * sk::kPBlock;
#pragma unroll
        for (int ks = 0; ks < sk::kKs; ++ks) pf[ks] = *(const u32x4*)(pbs + (((4 * ks + q) ^ r16) << 4));
      }
      const lds_char* fb = L + fslot * sk::kFStage;
#pragma unroll
      for (int ks = 0; ks < sk::kKs; ++ks) {
        const int sw = ((4 * ks + q) ^ r16) << 4;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
          const u32x4 xf = *(const u32x4*)(fb + (16 * rb + r16) * sk::kKB + sw);
          Mfma16<DT>::mma(acc[2 * r + rb], xf, pf[ks]);
        }
      }
      fslot = fslot + 1 == sk::kNF ? 0 : fslot + 1;
    }
  };

  int xs = xs0, xu = xu0, u = 0;
  int64_t xi = xi0;
  while (u < nu) {
    const int seg_end = min(nu, u + (args.s[xs].nst - xu));
    if (u == 0) {
      unit(std::true_type{});
      ++u;
    }
    for (; u < seg_end; ++u) unit(std::false_type{});
    // piece of item (xs, xi): lane-major MFMA layout, blocks (column block w, row block tb) of 64 x 16 B
    f32x4* dst = (f32x4*)(args.pieces + (args.s[xs].i0 + xi + w) * kPieceFloats) + wave * 8 * 64 + lane;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      dst[t * 64] = acc[t];
      acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    xu = 0;
    if (++xi == args.s[xs].items) {
      xi = 0;
      ++xs;
    }
  }
  // the zero-filling DMAs past the range still write this workgroup's LDS
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// M[b, o*ka + i] = sum over chunks and tokens of gp[t, o] * ap[t, i], where
// ap / gp are the summed pieces (plus the bias row on the activation side,
// on valid tokens only).  Four workgroups per sample, one per 16-row block ob
// of M; workgroup id 32q + 8ob + x takes sample 8q + x, so the four share an
// XCD (ids are dealt to the 8 XCDs round robin) and its L2 copy of the
// activation pieces.  Wave w contracts its 32 tokens of each chunk with fp32
// 16x16x4 MFMAs straight from the piece layout: lane l holds tokens
// 4*(l/16) + r (r = 0..3) of column l%16 of each 16x16 block, so step r pairs
// MFMA k-slot l/16 with token 4*(l/16) + r on both operands.  The four waves'
// sums are added in wave order.
template <int OT>
__global__ __launch_bounds__(kThreads) void outer_from_pieces(SkArgs args, int ka, int kg, char* out,
                                                              int64_t out_bstride, int64_t nb, int64_t tokens,
                                                              int flat) {
  __shared__ f32x4 red[4][4][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t id = blockIdx.x;
  const int64_t b = 8 * (id >> 5) + (id & 7);
  const int ob = (int)((id >> 3) & 3);
  if (b >= nb || 16 * ob >= kg) return;  // uniform
  const SkSide& SA = args.s[0];
  const SkSide& SG = args.s[1];
  f32x4 m[4];
#pragma unroll
  for (int ib = 0; ib < 4; ++ib) m[ib] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Sample b's rows in the items' row space (128 rows per item): its own
  // chunks, or, with short samples packed (flat), rows b*T .. of one run.
  const int64_t r0 = flat ? b * tokens : b * args.chunks * ps::kTok;
  const int64_t il0 = r0 / ps::kTok, il1 = (r0 + tokens - 1) / ps::kTok;
  for (int64_t il = il0; il <= il1; ++il) {
    // the item's rows [lo, hi) are this sample's
    const int64_t lo = max(r0, il * ps::kTok) - il * ps::kTok;
    const int64_t hi = min(r0 + tokens, (il + 1) * ps::kTok) - il * ps::kTok;
    const int64_t fa = SA.s0 + il * SA.nst, fg = SG.s0 + il * SG.nst;
    const int64_t a0 = sk_owner(fa, args), a1 = sk_owner(fa + SA.nst - 1, args);
    const int64_t g0 = sk_owner(fg, args), g1 = sk_owner(fg + SG.nst - 1, args);
    auto piece = [&](const SkSide& S, int64_t wq) __attribute__((always_inline)) {
      return (const f32x4*)(args.pieces + (S.i0 + il + wq) * kPieceFloats) + 2 * wave * 64 + lane;
    };
    f32x4 va[2][4], vg[2];  // activation: rb x column block; gradient: rb (column block ob)
    {
      const f32x4* pa = piece(SA, a0);
      const f32x4* pg = piece(SG, g0);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        vg[rb] = pg[(ob * 8 + rb) * 64];
#pragma unroll
        for (int c = 0; c < 4; ++c) va[rb][c] = pa[(c * 8 + rb) * 64];
      }
    }
    for (int64_t wq = a0 + 1; wq <= a1; ++wq) {
      const f32x4* pa = piece(SA, wq);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int c = 0; c < 4; ++c) va[rb][c] += pa[(c * 8 + rb) * 64];
    }
    for (int64_t wq = g0 + 1; wq <= g1; ++wq) {
      const f32x4* pg = piece(SG, wq);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) vg[rb] += pg[(ob * 8 + rb) * 64];
    }
    // rows outside [lo, hi): past the sample's last token (zero pieces) or
    // another sample's (packed items) -- out of both products
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = 32 * wave + 16 * rb + 4 * (lane >> 4) + r;
        if (row < lo || row >= hi) {
          vg[rb][r] = 0.f;
#pragma unroll
          for (int c = 0; c < 4; ++c) va[rb][c][r] = 0.f;
        }
      }
    if (SA.bias) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int col = 16 * c + (lane & 15);
        const float bv = col < SA.ncols ? SA.bias[col] : 0.f;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t row = 32 * wave + 16 * rb + 4 * (lane >> 4) + r;
            if (row >= lo && row < hi) va[rb][c][r] += bv;
          }
      }
    }
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int ib = 0; ib < 4; ++ib)
          m[ib] = __builtin_amdgcn_mfma_f32_16x16x4f32(vg[rb][r], va[rb][ib][r], m[ib], 0, 0, 0);
  }
#pragma unroll
  for (int ib = 0; ib < 4; ++ib) red[wave][ib][lane] = m[ib];
  __syncthreads();
  const int ib = tid >> 6, ln = tid & 63;
  const f32x4 sum = red[0][ib][ln] + red[1][ib][ln] + red[2][ib][ln] + red[3][ib][ln];
  const int i = 16 * ib + (ln & 15);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int o = 16 * ob + 4 * (ln >> 4) + r;
    if (o < kg && i < ka) Elem<OT>::store(out, b * out_bstride + (int64_t)o * ka + i, sum[r]);
  }
}

// The streaming kernel addresses a sample's rows and the projection rows with
// 32-bit buffer offsets.
bool stream_fits(int64_t tokens, int64_t tstride_b, int64_t wbytes, int64_t pt_rstride_b) {
  const int64_t lim = (1LL << 31) - (1LL << 20);
  return tstride_b >= 0 && tokens * tstride_b + wbytes < lim && kCols * pt_rstride_b + wbytes < lim;
}

// The stream-K kernel addresses one 128-token chunk and the projection rows
// with 32-bit buffer offsets.
bool sk_fits(int64_t tstride_b, int64_t wbytes, int64_t pt_rstride_b) {
  const int64_t lim = (1LL << 31) - (1LL << 20);
  return tstride_b >= 0 && ps::kTok * tstride_b + wbytes < lim && kCols * pt_rstride_b + wbytes < lim;
}

template <int OT>
__global__ void project_outer_reduce(const float* __restrict__ partial, int64_t batch, int64_t chunks,
                                     int64_t width, char* out, int64_t out_bstride) {
  const int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (f >= width) return;
  float s = 0.f;
  for (int64_t c = 0; c < chunks; ++c) s += partial[(b * chunks + c) * width + f];
  Elem<OT>::store(out, b * out_bstride + f, s);
}

int check_rows(const void* p, int64_t rstride_bytes, const char* who, const char* what) {
  if (((uintptr_t)p & 15) || (rstride_bytes % 16))
    return set_error(DA_ERR_INVALID, "%s: %s rows must be 16-byte aligned", who, what);
  return DA_OK;
}

}  // namespace
// ---------------------------------------------------------------------------
// Coordinate subset ("mask" projection) of per-sample linear weight gradients,
// gathered from the factors without forming the gradient:
//   out[b, k] = sum_t g[b, t, rows[k]] * A[b, t, cols[k]]
// with A's column K the implicit ones column of a bias.  One thread per
// coordinate and sample; a token row of g and of a is a few tens of KB, so the
// scattered reads of one workgroup's 256 coordinates hit the caches.
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void gather_entries_kernel(const char* a, const char* g, int64_t tokens,
                                                             int64_t K, int64_t D, int64_t a_bs, int64_t a_ts,
                                                             int64_t g_bs, int64_t g_ts, int has_bias,
                                                             const int64_t* rows, const int64_t* cols, int64_t n,
                                                             float* out, int64_t out_ld) {
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (k >= n) return;
  const int64_t r = rows[k], c = cols[k];
  float acc = 0.f;
  // indices outside the layer contribute nothing (the host draws them in range)
  if (r >= 0 && r < D && c >= 0 && c < K + has_bias) {
    const char* gp = g + b * g_bs + r * Elem<DT>::kBytes;
    const char* ap = a + b * a_bs + c * Elem<DT>::kBytes;
    const bool ones = c == K;
    for (int64_t t = 0; t < tokens; ++t) {
      const float gv = Elem<DT>::load(gp + t * g_ts, 0);
      acc += ones ? gv : gv * Elem<DT>::load(ap + t * a_ts, 0);
    }
  }
  out[b * out_ld + k] = acc;
}

}  // namespace da

extern "C" {

int da_project_rows(const void* x, int dtype, int64_t rows, int64_t d, int64_t x_rstride,
                    const void* pt, int64_t k, int64_t pt_rstride, const float* bias, void* out,
                    int out_dtype, int64_t out_rstride, void* stream) {
  using namespace da;
  const char* who = "da_project_rows";
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return set_error(DA_ERR_INVALID, "%s: bad dtype", who);
  if (rows < 0 || d < 0 || k < 0) return set_error(DA_ERR_INVALID, "%s: negative size", who);
  if (rows == 0 || k == 0) return DA_OK;
  if (!x || !pt || !out) return set_error(DA_ERR_INVALID, "%s: NULL pointer", who);
  const int64_t es = (int64_t)elem_bytes(dtype);
  if ((d * es) % 16) return set_error(DA_ERR_INVALID, "%s: d must be a multiple of %lld", who, (long long)(16 / es));
  if (out_rstride < k) return set_error(DA_ERR_INVALID, "%s: out row stride < k", who);
  int rc = check_rows(x, x_rstride * es, who, "x");
  if (rc) return rc;
  rc = check_rows(pt, pt_rstride * es, who, "P^T");
  if (rc) return rc;
  RowsArgs a;
  a.x = (const char*)x;
  a.rows = rows;
  a.wbytes = d * es;
  a.x_rstride = x_rstride * es;
  a.pt = (const char*)pt;
  a.pt_rstride = pt_rstride * es;
  a.k = k;
  a.bias = bias;
  a.out = (char*)out;
  a.out_rstride = out_rstride;
  hipStream_t st = (hipStream_t)stream;
  if (k <= kCols && stream_fits(rows, a.x_rstride, a.wbytes, a.pt_rstride)) {
    PGroupArgs pa;
    pa.n = 1;
    PGroup& G = pa.g[0];
    G.x = a.x;
    G.batch = 1;
    G.tokens = rows;
    G.bstride = 0;
    G.tstride = a.x_rstride;
    G.wbytes = a.wbytes;
    G.pt = a.pt;
    G.pt_rstride = a.pt_rstride;
    G.ncols = (int)k;
    G.bias = bias;
    G.out = (char*)out;
    G.out_bstride = 0;
    G.out_tstride = out_rstride;
    G.chunks = (rows + ps::kTok - 1) / ps::kTok;
    G.wg0 = 0;
    if (G.chunks > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: problem too large", who);
    const unsigned blocks = (unsigned)G.chunks;
#define DA_PRS(DT)                                                                            \
    switch (out_dtype) {                                                                      \
      case DA_F32: project_rows_stream<DT, DA_F32><<<blocks, kThreads, 0, st>>>(pa); break;   \
      case DA_BF16: project_rows_stream<DT, DA_BF16><<<blocks, kThreads, 0, st>>>(pa); break; \
      default: project_rows_stream<DT, DA_F16><<<blocks, kThreads, 0, st>>>(pa); break;       \
    }
    switch (dtype) {
      case DA_BF16: DA_PRS(DA_BF16) break;
      case DA_F16: DA_PRS(DA_F16) break;
      default: DA_PRS(DA_F32) break;
    }
#undef DA_PRS
    return check_launch(who);
  }
  const int64_t gx = (rows + kRows - 1) / kRows, gy = (k + kCols - 1) / kCols;
  if (gx > 0x7fffffffLL || gy > 65535) return set_error(DA_ERR_INVALID, "%s: problem too large", who);
  dim3 grid((unsigned)gx, (unsigned)gy);
#define DA_PR(DT)                                                                           \
  switch (out_dtype) {                                                                      \
    case DA_F32: project_rows_kernel<DT, DA_F32><<<grid, kThreads, 0, st>>>(a); break;      \
    case DA_BF16: project_rows_kernel<DT, DA_BF16><<<grid, kThreads, 0, st>>>(a); break;    \
    default: project_rows_kernel<DT, DA_F16><<<grid, kThreads, 0, st>>>(a); break;          \
  }
  switch (dtype) {
    case DA_BF16: DA_PR(DA_BF16) break;
    case DA_F16: DA_PR(DA_F16) break;
    default: DA_PR(DA_F32) break;
  }
#undef DA_PR
  return check_launch(who);
}

int da_project_outer_workspace(int64_t batch, int64_t tokens, int64_t ka, int64_t kg, size_t* bytes) {
  if (batch < 0 || tokens < 0 || ka < 0 || kg < 0 || !bytes)
    return da::set_error(DA_ERR_INVALID, "da_project_outer_workspace: bad arguments");
  const int64_t chunks = (tokens + da::kRows - 1) / da::kRows;
  const size_t partials = (size_t)(batch * chunks * ka * kg) * sizeof(float);
  // the stream-K path keeps one fp32 piece per (item, workgroup) boundary
  int64_t slots = 0;
  const int rc = da::device_cu_count(&slots);
  if (rc) return rc;
  const int64_t items = 2 * batch * ((tokens + da::ps::kTok - 1) / da::ps::kTok);
  const size_t pieces = (size_t)(items + slots) * da::kPieceFloats * sizeof(float);
  *bytes = partials > pieces ? partials : pieces;
  return DA_OK;
}

int da_project_outer(const void* a, const void* g, int dtype, int64_t batch, int64_t tokens, int64_t K,
                     int64_t D, int64_t a_bstride, int64_t a_tstride, int64_t g_bstride,
                     int64_t g_tstride, const void* pin_t, int64_t ka, int64_t pin_rstride,
                     const float* bias_in, const void* pout_t, int64_t kg, int64_t pout_rstride,
                     void* out, int out_dtype, int64_t out_bstride, void* workspace,
                     size_t workspace_bytes, void* stream) {
  using namespace da;
  const char* who = "da_project_outer";
  if (!valid_dtype(dtype) || !valid_dtype(out_dtype)) return set_error(DA_ERR_INVALID, "%s: bad dtype", who);
  if (batch < 0 || tokens < 0 || K < 0 || D < 0 || ka < 0 || kg < 0)
    return set_error(DA_ERR_INVALID, "%s: negative size", who);
  if (ka > kCols || kg > kCols)
    return set_error(DA_ERR_UNSUPPORTED, "%s: projected widths above %d (got %lld, %lld)", who, kCols,
                     (long long)ka, (long long)kg);
  if (batch == 0 || ka == 0 || kg == 0) return DA_OK;
  if (tokens == 0) return set_error(DA_ERR_INVALID, "%s: tokens must be >= 1", who);
  if (!a || !g || !pin_t || !pout_t || !out) return set_error(DA_ERR_INVALID, "%s: NULL pointer", who);
  const int64_t es = (int64_t)elem_bytes(dtype);
  if ((K * es) % 16 || (D * es) % 16)
    return set_error(DA_ERR_INVALID, "%s: K and D must be multiples of %lld", who, (long long)(16 / es));
  if (((a_bstride * es) | (a_tstride * es) | (g_bstride * es) | (g_tstride * es)) % 16 ||
      (((uintptr_t)a | (uintptr_t)g) & 15))
    return set_error(DA_ERR_INVALID, "%s: factor rows must be 16-byte aligned", who);
  int rc = check_rows(pin_t, pin_rstride * es, who, "P_in^T");
  if (rc) return rc;
  rc = check_rows(pout_t, pout_rstride * es, who, "P_out^T");
  if (rc) return rc;
  if (out_bstride < ka * kg) return set_error(DA_ERR_INVALID, "%s: out batch stride < kg*ka", who);
  size_t need = 0;
  da_project_outer_workspace(batch, tokens, ka, kg, &need);
  if (!workspace || workspace_bytes < need)
    return set_error(DA_ERR_WORKSPACE, "%s: workspace needs %zu bytes", who, need);
  OuterArgs o;
  o.a = (const char*)a;
  o.g = (const char*)g;
  o.batch = batch;
  o.tokens = tokens;
  o.a_bstride = a_bstride * es;
  o.a_tstride = a_tstride * es;
  o.g_bstride = g_bstride * es;
  o.g_tstride = g_tstride * es;
  o.abytes = K * es;
  o.gbytes = D * es;
  o.pin_t = (const char*)pin_t;
  o.pout_t = (const char*)pout_t;
  o.pin_rstride = pin_rstride * es;
  o.pout_rstride = pout_rstride * es;
  o.ka = (int)ka;
  o.kg = (int)kg;
  o.bias_in = bias_in;
  o.chunks = (tokens + kRows - 1) / kRows;
  o.partial = (float*)workspace;
  hipStream_t st = (hipStream_t)stream;
  const bool stream_ok = sk_fits(o.a_tstride, o.abytes, o.pin_rstride) && sk_fits(o.g_tstride, o.gbytes, o.pout_rstride);
  if (stream_ok) {
    // Stream-K projection of both sides into fp32 pieces, then the per-sample
    // contraction.
    // Samples whose rows lie at one stride (batch stride = tokens x token
    // stride on both sides) are packed: the items run over the B*T rows as
    // one sample, so an item's 128 rows may hold several samples, and a
    // sample's last rows share an item with the next sample's first instead
    // of with zero rows.
    const bool flat = batch > 1 && tokens % ps::kTok != 0 && o.a_bstride == tokens * o.a_tstride &&
                      o.g_bstride == tokens * o.g_tstride;
    SkArgs sk;
    sk.batch = flat ? 1 : batch;
    sk.tokens = flat ? batch * tokens : tokens;
    sk.chunks = (sk.tokens + ps::kTok - 1) / ps::kTok;
    sk.pieces = (float*)workspace;
    int64_t s0 = 0;
    for (int side = 0; side < 2; ++side) {
      SkSide& S = sk.s[side];
      const bool act = side == 0;
      S.x = act ? o.a : o.g;
      S.bstride = act ? o.a_bstride : o.g_bstride;
      S.tstride = act ? o.a_tstride : o.g_tstride;
      S.wbytes = act ? o.abytes : o.gbytes;
      S.pt = act ? o.pin_t : o.pout_t;
      S.pt_rstride = act ? o.pin_rstride : o.pout_rstride;
      S.ncols = act ? o.ka : o.kg;
      S.nst = (int)((S.wbytes + sk::kKB - 1) / sk::kKB);  // stream-K units (k-blocks) per item
      S.items = sk.batch * sk.chunks;
      S.s0 = s0;
      S.i0 = side * S.items;
      S.bias = act ? bias_in : nullptr;
      if (S.nst == 0) return set_error(DA_ERR_INVALID, "%s: K and D must be >= 1", who);
      s0 += S.items * S.nst;
    }
    sk.total = s0;
    int64_t slots = 0;
    rc = device_cu_count(&slots);
    if (rc) return rc;
    sk.nwg = slots < sk.total ? slots : sk.total;
    if (sk.total / sk.nwg > (1LL << 30) || batch > (1LL << 28))
      return set_error(DA_ERR_INVALID, "%s: problem too large", who);
    const unsigned blocks = (unsigned)sk.nwg;
    switch (dtype) {
      case DA_BF16: project_pieces<DA_BF16><<<blocks, kThreads, 0, st>>>(sk); break;
      case DA_F16: project_pieces<DA_F16><<<blocks, kThreads, 0, st>>>(sk); break;
      default: project_pieces<DA_F32><<<blocks, kThreads, 0, st>>>(sk); break;
    }
    rc = check_launch("da_project_outer(projection)");
    if (rc) return rc;
    const unsigned ob_blocks = (unsigned)(32 * ((batch + 7) / 8));  // 4 row blocks x 8 samples per 32 ids
    switch (out_dtype) {
      case DA_F32: outer_from_pieces<DA_F32><<<ob_blocks, kThreads, 0, st>>>(sk, o.ka, o.kg, (char*)out, out_bstride, batch, tokens, flat ? 1 : 0); break;
      case DA_BF16: outer_from_pieces<DA_BF16><<<ob_blocks, kThreads, 0, st>>>(sk, o.ka, o.kg, (char*)out, out_bstride, batch, tokens, flat ? 1 : 0); break;
      default: outer_from_pieces<DA_F16><<<ob_blocks, kThreads, 0, st>>>(sk, o.ka, o.kg, (char*)out, out_bstride, batch, tokens, flat ? 1 : 0); break;
    }
    return check_launch("da_project_outer(outer)");
  } else {
    const int64_t blocks = batch * o.chunks;
    if (blocks > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: problem too large", who);
    switch (dtype) {
      case DA_BF16: project_outer_kernel<DA_BF16><<<(unsigned)blocks, kThreads, 0, st>>>(o); break;
      case DA_F16: project_outer_kernel<DA_F16><<<(unsigned)blocks, kThreads, 0, st>>>(o); break;
      default: project_outer_kernel<DA_F32><<<(unsigned)blocks, kThreads, 0, st>>>(o); break;
    }
  }
  rc = check_launch("da_project_outer(chunks)");
  if (rc) return rc;
  const int64_t width = ka * kg;
  dim3 g2((unsigned)((width + 255) / 256), (unsigned)batch);
  switch (out_dtype) {
    case DA_F32: project_outer_reduce<DA_F32><<<g2, 256, 0, st>>>(o.partial, batch, o.chunks, width, (char*)out, out_bstride); break;
    case DA_BF16: project_outer_reduce<DA_BF16><<<g2, 256, 0, st>>>(o.partial, batch, o.chunks, width, (char*)out, out_bstride); break;
    default: project_outer_reduce<DA_F16><<<g2, 256, 0, st>>>(o.partial, batch, o.chunks, width, (char*)out, out_bstride); break;
  }
  return check_launch("da_project_outer(reduce)");
}

int da_gather_entries(const void* a, const void* g, int dtype, int64_t batch, int64_t tokens, int64_t K, int64_t D,
                      int64_t a_bstride, int64_t a_tstride, int64_t g_bstride, int64_t g_tstride, int has_bias,
                      const int64_t* rows, const int64_t* cols, int64_t n, float* out, int64_t out_ld,
                      void* stream) {
  using namespace da;
  const char* who = "da_gather_entries";
  if (!valid_dtype(dtype)) return set_error(DA_ERR_INVALID, "%s: bad dtype %d", who, dtype);
  if (batch < 0 || tokens < 0 || K < 0 || D < 0 || n < 0) return set_error(DA_ERR_INVALID, "%s: negative size", who);
  if (batch == 0 || n == 0) return DA_OK;
  if (!a || !g || !rows || !cols || !out) return set_error(DA_ERR_INVALID, "%s: NULL pointer", who);
  if (out_ld < n) return set_error(DA_ERR_INVALID, "%s: out_ld < n", who);
  if (batch > 65535) return set_error(DA_ERR_INVALID, "%s: at most 65535 samples per call", who);
  if ((n + 255) / 256 > 0x7fffffffLL) return set_error(DA_ERR_INVALID, "%s: too many coordinates", who);
  const int64_t es = (int64_t)elem_bytes(dtype);
  dim3 grid((unsigned)((n + 255) / 256), (unsigned)batch);
  hipStream_t st = (hipStream_t)stream;
#define DA_GATHER(DT)                                                                                        \
  gather_entries_kernel<DT><<<grid, 256, 0, st>>>((const char*)a, (const char*)g, tokens, K, D, a_bstride * es,  \
                                                  a_tstride * es, g_bstride * es, g_tstride * es, has_bias ? 1 : 0, \
                                                  rows, cols, n, out, out_ld)
  switch (dtype) {
    case DA_BF16: DA_GATHER(DA_BF16); break;
    case DA_F16: DA_GATHER(DA_F16); break;
    default: DA_GATHER(DA_F32); break;
  }
#undef DA_GATHER
  return check_launch(who);
}

}  // extern "C"
