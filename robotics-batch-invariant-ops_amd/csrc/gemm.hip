// Persistent fixed-schedule GEMM / batched GEMM entry points.
#include <stdlib.h>

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "gemm.h"
#include "gemm_big.h"
#include "gemm_skinny.h"
#include "gemm_stream.h"

namespace biops {

// ------------------------------------------------------------------ tile menu ----
// Every entry computes each output element with the same MFMA sequence (see gemm_core.h); the
// entries differ in block tile, wavefront layout and LDS ring depth only.
template <int ID> struct Cfg;
#define BIOPS_CFG(ID, BM_, BN_, WGM_, WGN_, ST_, PERCU_, PP_, LW_)                   \
  template <> struct Cfg<ID> {                                                    \
    static constexpr int bm = BM_, bn = BN_, wgm = WGM_, wgn = WGN_, stages = ST_;   \
    static constexpr int loaders = LW_;                                           \
    static constexpr int threads = 64 * (WGM_ * WGN_ + LW_), per_cu = PERCU_;     \
    static constexpr int waves_per_eu = ((WGM_ * WGN_ + LW_) * PERCU_ + 3) / 4;   \
    static constexpr bool pingpong = PP_;                                         \
    static constexpr bool persist = BM_ * BN_ < 256 * 256;                       \
  };
//         id   BM   BN  WGM WGN stages  workgroups/CU  ping-pong  loader waves
BIOPS_CFG(0, 256, 256, 2, 4, 2, 1, true, 0)
BIOPS_CFG(1, 256, 128, 2, 2, 3, 1, false, 0)
BIOPS_CFG(2, 128, 128, 2, 2, 2, 2, false, 0)
BIOPS_CFG(3, 128, 64, 2, 2, 4, 1, false, 0)
BIOPS_CFG(4, 64, 64, 2, 2, 4, 2, false, 0)
BIOPS_CFG(5, 32, 64, 1, 2, 4, 2, false, 0)
BIOPS_CFG(6, 32, 32, 1, 1, 4, 4, false, 0)
// 7: 32x64 tiles (one gate/up pair of 32 columns) on one computing wavefront plus three that only
// load, into a 12-stage ring: the SwiGLU expert GEMM of few-token MoE calls, a latency-bound
// weight stream (each wavefront keeps at most 63 loads in flight)
BIOPS_CFG(7, 32, 64, 1, 1, 12, 1, false, 3)
BIOPS_CFG(8, 128, 128, 2, 2, 4, 1, false, 0)
BIOPS_CFG(9, 128, 256, 2, 2, 3, 1, false, 0)
BIOPS_CFG(10, 256, 128, 4, 2, 3, 1, false, 0)
BIOPS_CFG(11, 128, 256, 2, 4, 3, 1, false, 0)
#undef BIOPS_CFG
constexpr int kNumCfg = 12;
// Entry 12: the skinny tile (gemm_skinny.h), one 32-row block (64, 32, 16 or 8 columns) per
// workgroup with loader wavefronts.  Needs the direct-load conditions and a plain / bias epilogue; elsewhere it falls
// back to the automatic choice.
constexpr int kSkinnyCfg = kNumCfg;
// Entries 13-19: the four-wavefront schedule (gemm_big.h), one wavefront per SIMD with the
// accumulators in the accumulation registers and a ring as deep as the LDS holds, on blocks of
// 256x256 (entry 13), 256x128, 128x256, 128x128, 128x64, 64x128 and 64x64.  16-bit operands,
// direct-load conditions and a plain / bias epilogue; elsewhere they fall back to the
// automatic choice.  The tile cost model weighs them against entries 0-11 from K = 1024 on.
constexpr int kBigCfg = kNumCfg + 1;
constexpr int kNumBig = 7;
static const int kBigBM[kNumBig] = {256, 256, 128, 128, 128, 64, 64};
static const int kBigBN[kNumBig] = {256, 128, 256, 128, 64, 128, 64};
// Throughput of each block in the tile cost model (TFLOP/s-equivalent, as kCfgRate).  The
// 64x128 block is rated above the 128x64 one: measured on MI355X it was 3-7 % faster on every
// shape where both fill the same rounds (M=1024, N=2048, K=8192: 47.4 against 51.3 us; M=256,
// N=8192, K=2048: 15.7 against 16.4 us).  The 64x64 block (rate unused) stays out of the
// cost model; it takes the long-K shapes of up to four 32x32 tiles per compute unit instead
// of entry 6 (below).
static const double kBigRate[kNumBig] = {1150, 1050, 1050, 850, 700, 720, 480};
constexpr int kBigAutoCount = kNumBig - 1;  // blocks the automatic choice weighs
// With a 16-bit N-major B (transposing LDS reads) each block is costed at this share of its
// rate: the time of the same problem with B K-major over its time N-major, measured on MI355X
// (bf16; M x N x K = 4096^3, 4096 x 8192 x 2048, 2048 x 2048 x 8192, 1024 x 2048 x 8192,
// 2048 x 6144 x 4096, 1024 x 4096 x 4096, 512 x 8192 x 2048; the 256x256 block 0.86-0.96,
// 0.96 on the shapes it wins).
static const double kBigNmajorShare[kNumBig] = {0.93, 0.91, 0.87, 0.87, 0.88, 0.79, 0.86};
constexpr int kBigEnd = kBigCfg + kNumBig;
// Entries 20-22: the weight-streaming tile (gemm_stream.h), one m-tile of 16 (entry 20), 32
// (entry 21) or 64 (entry 22) rows x 64 output columns per workgroup (128 for a plain
// epilogue on 64-row m-tiles).  Grouped rows with a 16-bit N-major B only (the MoE
// expert GEMMs); elsewhere they fall back to the automatic choice.
constexpr int kStreamCfg = kBigEnd;
constexpr int kNumStream = 3;
constexpr int kStreamBM[kNumStream] = {16, 32, 64};
static_assert(kMinGroupedTileRows == 16, "grouped tables are sized for the 16-row stream entry");
constexpr int kMenuSize = kStreamCfg + kNumStream;

// One persistent workgroup walks tiles t = slot, slot + G, ... over all batch elements.
// Epilogues: plain C = round(acc (+ bias[n])) (bias added in fp32 before the single rounding);
// Tile t of a launch -> batch indices and the tile's first row / column.  Tiles are numbered
// batch-major; inside one GEMM, 8 tile-rows form a group walked column by column.
struct TileOrigin {
  uint32_t b1, b2;
  int64_t m0, m_end, n0;
};
template <bool GRP = false>
__device__ __forceinline__ TileOrigin tile_origin(const BmmArgs& args, uint32_t t, int BM, int cols) {
  const uint32_t tiles_n = (uint32_t)args.tiles_n;
  if constexpr (GRP) {
    // Grouped rows: m-tile list from the device table, same 8-row-group walk.
    const uint32_t tiles_m = (uint32_t)args.grp[0];
    const uint32_t per_group = 8u * tiles_n;
    const uint32_t group = t / per_group;
    const uint32_t first = group * 8u;
    const uint32_t gsize = tiles_m - first < 8u ? tiles_m - first : 8u;
    const uint32_t in_group = t - group * per_group;
    const uint32_t tn = in_group / gsize;
    const uint32_t tm = first + (in_group - tn * gsize);
    const int32_t* e = args.grp + kGrpHeader + kGrpStride * tm;
    TileOrigin o;
    o.b1 = (uint32_t)e[0];
    o.b2 = 0;
    o.m0 = e[1];
    o.m_end = e[2];
    o.n0 = (int64_t)tn * cols;
    return o;
  }
  const uint32_t tiles_m = (uint32_t)args.tiles_m;
  const uint32_t tpb = tiles_m * tiles_n;
  const uint32_t nb2 = (uint32_t)args.nb2;
  const uint32_t b = t / tpb;
  const uint32_t in_b = t - b * tpb;
  const uint32_t per_group = 8u * tiles_n;
  const uint32_t group = in_b / per_group;
  const uint32_t first = group * 8u;
  const uint32_t gsize = tiles_m - first < 8u ? tiles_m - first : 8u;
  const uint32_t in_group = in_b - group * per_group;
  const uint32_t tn = in_group / gsize;
  const uint32_t tm = first + (in_group - tn * gsize);
  TileOrigin o;
  o.b1 = b / nb2;
  o.b2 = b - o.b1 * nb2;
  o.m0 = (int64_t)tm * BM;
  o.m_end = args.M;
  o.n0 = (int64_t)tn * cols;
  return o;
}

// SwiGLU C = round(round(silu(round(g))) * round(u)) -- the roundings of F.silu(gate) * up
// applied to rounded bmm outputs -- where gate and up accumulators of one output sit in
// adjacent 32-column MFMA blocks of the same wavefront.
template <typename T, int CFG, bool BKM, bool DIRECT, int EPI, bool GRP>
__device__ __forceinline__ void bmm_tile(const BmmArgs& args, uint32_t t, char* smem) {
  using C = Cfg<CFG>;
  using Tile = GemmTile<T, C::bm, C::bn, C::wgm, C::wgn, (DIRECT ? C::stages : 2), BKM, DIRECT, C::loaders>;
  constexpr int BM = C::bm, BN = C::bn;
  constexpr int kCols = EPI == kEpiSwiglu ? BN / 2 : BN;
  typename Tile::Acc acc[Tile::FM][Tile::FN];

  const TileOrigin o = tile_origin<GRP>(args, t, BM, kCols);
  const uint32_t b1 = o.b1, b2 = o.b2, gB = (uint32_t)args.gB;
  const int64_t m0 = o.m0, n0 = o.n0;

  const T* A = reinterpret_cast<const T*>(args.A) + b1 * args.sA1 + b2 * args.sA2 + m0 * args.lda;
  const int64_t boff = b1 * args.sB1 + (b2 / gB) * args.sB2 + (BKM ? n0 * args.ldb : n0);
  BSource<T> src;
  src.p0 = reinterpret_cast<const T*>(args.B) + boff;
  src.p1 = EPI == kEpiSwiglu ? reinterpret_cast<const T*>(args.B2) + boff : src.p0;
  src.ld = args.ldb;
  src.ncols = args.N - n0;
  src.swiglu = EPI == kEpiSwiglu;
  src.vec_ok = args.b_vec != 0;
  const int64_t rows = o.m_end - m0;
  const int64_t cols = args.N - n0;

  auto run = [&](const auto& as) {
    if constexpr (C::pingpong && DIRECT) Tile::mainloop_pingpong(smem, acc, as, src, args.K);
    else Tile::mainloop(smem, acc, as, args.a_vec != 0, src, args.K);
  };
  if constexpr (GRP) {
    if (args.a_rows)  // rows come through the table (grouped launches have no A batch strides)
      run(Tile::a_table(reinterpret_cast<const T*>(args.A), args.lda, rows, args.a_rows + m0));
    else
      run(typename Tile::ARows{A, args.lda, rows});
  } else {
    run(typename Tile::ARows{A, args.lda, rows});
  }

  T* Cp = reinterpret_cast<T*>(args.C) + b1 * args.sC1 + b2 * args.sC2 + m0 * args.ldc + n0;
  const T* bias = (EPI != kEpiSwiglu && args.bias) ? reinterpret_cast<const T*>(args.bias) + n0 : nullptr;
  Tile::template epilogue<EPI == kEpiSwiglu>(smem, acc, Cp, args.ldc, rows < BM ? (int)rows : BM,
                                             cols < kCols ? (int)cols : kCols, bias, args.c_vec != 0);
}

// Persistent entries walk tiles t = slot, slot + G, ... (slot = XCD-aware rank of the
// workgroup); the large-tile entries run one tile per workgroup (grid = tiles, same XCD-aware
// order), which keeps their register budget for the accumulators.
// GRP (grouped rows): the tile count is only known on the device.  XCD x (workgroups g with
// g % 8 == x) takes the x-th eighth of the tiles, so the work stays balanced however far the
// launch's worst-case size overshoots (the launcher makes G a multiple of 8).
template <typename T, int CFG, bool BKM, bool DIRECT, int EPI, bool GRP>
__global__ __launch_bounds__(Cfg<CFG>::threads)
__attribute__((amdgpu_waves_per_eu(Cfg<CFG>::waves_per_eu, Cfg<CFG>::waves_per_eu)))
void bmm_kernel(BmmArgs args) {
  using C = Cfg<CFG>;
  using Tile = GemmTile<T, C::bm, C::bn, C::wgm, C::wgn, (DIRECT ? C::stages : 2), BKM, DIRECT, C::loaders>;
  __shared__ __attribute__((aligned(16))) char smem[Tile::SMEM_BYTES];
  const uint32_t G = gridDim.x;
  if constexpr (GRP) {
    const uint32_t total = (uint32_t)args.grp[0] * (uint32_t)args.tiles_n;
    const uint32_t per = (total + 7u) / 8u;
    const uint32_t x = blockIdx.x % 8u, stride = G / 8u;
    if constexpr (C::persist) {
      for (uint32_t i = blockIdx.x / 8u; i < per; i += stride) {
        const uint32_t t = x * per + i;
        if (t >= total) break;
        bmm_tile<T, CFG, BKM, DIRECT, EPI, true>(args, t, smem);
      }
    } else {
      // One tile per workgroup: the launch covers the worst case, so G / 8 >= per.
      const uint32_t i = blockIdx.x / 8u, t = x * per + i;
      if (i < per && t < total) bmm_tile<T, CFG, BKM, DIRECT, EPI, true>(args, t, smem);
    }
  } else {
    const uint32_t total = (uint32_t)args.total;
    if constexpr (C::persist) {
      for (uint32_t t = (uint32_t)xcd_slot(blockIdx.x, G); t < total; t += G)
        bmm_tile<T, CFG, BKM, DIRECT, EPI, false>(args, t, smem);
    } else {
      const uint32_t t = (uint32_t)xcd_slot(blockIdx.x, G);
      if (t < total) bmm_tile<T, CFG, BKM, DIRECT, EPI, false>(args, t, smem);
    }
  }
}

// Computing wavefront w < CW of a skinny block stores its part straight from the accumulators
// with the rounding of the LDS-staged epilogue: round(acc (+ bias[n])).
template <typename S, typename T>
__device__ __forceinline__ void skinny_store(const BmmArgs& args, const TileOrigin& o, int rows, int cols,
                                             const typename S::Acc& acc) {
  const int w = threadIdx.x >> 6;
  if (w >= S::CW) return;
  const int wr = w / S::CWC, wc = w % S::CWC;
  const int64_t n0 = o.n0 + S::WC * wc;
  T* Cp = reinterpret_cast<T*>(args.C) + o.b1 * args.sC1 + o.b2 * args.sC2 + (o.m0 + S::WR * wr) * args.ldc + n0;
  const T* bias = args.bias ? reinterpret_cast<const T*>(args.bias) + n0 : nullptr;
  const int wrows = rows - S::WR * wr, wcols = cols - S::WC * wc;
  S::Math::store(acc, Cp, args.ldc, wrows < S::WR ? wrows : S::WR, wcols < S::WC ? wcols : S::WC, bias);
}

// One 32 x BC (or 64 x BC) block per workgroup.
template <typename T, int AR, int BC>
__global__ __launch_bounds__(512) void skinny_kernel(BmmArgs args) {
  using S = SkinnyTile<T, AR, BC>;
  static_assert(S::THREADS == 512, "launch bounds");
  __shared__ __attribute__((aligned(16))) char smem[S::LDS_BYTES];
  const uint32_t t = (uint32_t)xcd_slot(blockIdx.x, gridDim.x);
  if (t >= (uint32_t)args.total) return;
  constexpr int BH = AR > 32 ? 64 : 32;  // block rows
  const TileOrigin o = tile_origin(args, t, BH, BC);
  const T* A = reinterpret_cast<const T*>(args.A) + o.b1 * args.sA1 + o.b2 * args.sA2 + o.m0 * args.lda;
  const T* B = reinterpret_cast<const T*>(args.B) + o.b1 * args.sB1 +
               (o.b2 / (uint32_t)args.gB) * args.sB2 + o.n0 * args.ldb;
  const int64_t rows64 = o.m_end - o.m0, cols64 = args.N - o.n0;
  const int rows = rows64 < BH ? (int)rows64 : BH;
  const int cols = cols64 < BC ? (int)cols64 : BC;
  const typename S::Acc acc = S::run(smem, A, args.lda, rows, B, args.ldb, cols, args.K / S::BK);
  skinny_store<S, T>(args, o, rows, cols, acc);
}

// The same blocks on the loader-split schedule (SkinnyTile::run_deep): CW computing and DL
// loader wavefronts, K a whole number of 8-step stages (checked by the launcher).
template <typename T, int AR, int BC>
__global__ __launch_bounds__((SkinnyTile<T, AR, BC>::DTHREADS)) void skinny_deep_kernel(BmmArgs args) {
  using S = SkinnyTile<T, AR, BC>;
  static_assert(S::DEEP && AR <= 32, "loader-split blocks of 32 rows");
  __shared__ __attribute__((aligned(16))) char smem[S::DLDS_BYTES];
  const uint32_t t = (uint32_t)xcd_slot(blockIdx.x, gridDim.x);
  if (t >= (uint32_t)args.total) return;
  const TileOrigin o = tile_origin(args, t, 32, BC);
  const T* A = reinterpret_cast<const T*>(args.A) + o.b1 * args.sA1 + o.b2 * args.sA2 + o.m0 * args.lda;
  const T* B = reinterpret_cast<const T*>(args.B) + o.b1 * args.sB1 +
               (o.b2 / (uint32_t)args.gB) * args.sB2 + o.n0 * args.ldb;
  const int64_t rows64 = o.m_end - o.m0, cols64 = args.N - o.n0;
  const int rows = rows64 < 32 ? (int)rows64 : 32;
  const int cols = cols64 < BC ? (int)cols64 : BC;
  const typename S::Acc acc = S::run_deep(smem, A, args.lda, rows, B, args.ldb, cols, args.K / S::BK);
  skinny_store<S, T>(args, o, rows, cols, acc);
}

template <typename T, int BM, int BN, int SB, bool BKM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void big_kernel(BmmArgs args) {
  using Tile = BigTile<T, BM, BN, SB, BKM>;
  __shared__ __attribute__((aligned(16))) char smem[Tile::SMEM_BYTES];
  const uint32_t t = (uint32_t)xcd_slot(blockIdx.x, gridDim.x);
  if (t >= (uint32_t)args.total) return;
  const TileOrigin o = tile_origin(args, t, BM, BN);
  const T* A = reinterpret_cast<const T*>(args.A) + o.b1 * args.sA1 + o.b2 * args.sA2 + o.m0 * args.lda;
  // B K-major: column n at row n (stride ldb); N-major: column n at element n of each K row
  const T* B = reinterpret_cast<const T*>(args.B) + o.b1 * args.sB1 +
               (o.b2 / (uint32_t)args.gB) * args.sB2 + (BKM ? o.n0 * args.ldb : o.n0);
  const int64_t rows64 = o.m_end - o.m0, cols64 = args.N - o.n0;
  const int rows = rows64 < BM ? (int)rows64 : BM;
  const int cols = cols64 < BN ? (int)cols64 : BN;
  typename Tile::Acc acc[Tile::FM][Tile::FN];
  Tile::mainloop(smem, acc, A, args.lda, rows, B, args.ldb, cols, args.K);
  T* Cp = reinterpret_cast<T*>(args.C) + o.b1 * args.sC1 + o.b2 * args.sC2 + o.m0 * args.ldc + o.n0;
  const T* bias = args.bias ? reinterpret_cast<const T*>(args.bias) + o.n0 : nullptr;
  Tile::epilogue(acc, Cp, args.ldc, rows, cols, bias, args.nt_store != 0);
}

// -------------------------------------------------------------- tile selection ----
// Measured full-chip throughput of each entry on large bf16 problems (TFLOP/s, MI355X).  A
// compute unit works through ceil(tiles / CUs) tiles, each costing BM x BN / throughput (two
// resident workgroups share the unit, so they do not finish sooner), and the entry with the
// smallest estimate is launched.
static const double kCfgRate[kNumCfg] = {950, 750, 820, 450, 520, 330, 400, 180, 570, 670, 900, 900};
// With a 16-bit N-major B on the direct path the fragments come through the transposing LDS
// reads, and each entry is costed at this share of its K-major rate.  The shares were measured
// on MI355X (M = 4096 x N = 8192 / 2048 x K = 2048 / 8192 and 2048 x 1536 x 2048) while the
// compiler still drained the global->LDS loads before those reads; re-measured without that
// drain the large entries keep 0.94-1.0, but the older shares pick the faster entries for the
// MoE expert GEMMs (4096 tokens: 553 us per call against 598 us), so they are kept.  An fp32
// N-major B on the direct path (one 4-byte LDS read per fragment value) is costed at the
// K-major rate: it measured within 1 % of K-major on every entry (2048 x 4096 x 4096).
static const double kCfgNmajorShare[kNumCfg] = {0.97, 0.78, 0.86, 0.60, 0.72, 0.60, 0.55, 0.60, 0.73, 0.78, 0.80, 0.83};
static const int kCfgBM[kNumCfg] = {256, 256, 128, 128, 64, 32, 32, 32, 128, 128, 256, 128};
static const int kCfgBN[kNumCfg] = {256, 128, 128, 64, 64, 64, 32, 64, 128, 256, 128, 256};

// Forced tile entry (-1: automatic).  Initialised from BIOPS_GEMM_CFG, settable through
// biops_set_gemm_tile; every entry yields the same bits, so forcing one only changes speed.
static std::atomic<int> g_forced_cfg{-2};

static int forced_cfg() {
  int v = g_forced_cfg.load(std::memory_order_relaxed);
  if (v == -2) {
    const char* e = getenv("BIOPS_GEMM_CFG");
    v = e ? atoi(e) : -1;
    int expected = -2;
    g_forced_cfg.compare_exchange_strong(expected, v);
    v = g_forced_cfg.load(std::memory_order_relaxed);
  }
  return v;
}

// The skinny entry (one workgroup per compute unit, one 32x32 block each) wins when all its
// blocks run in one round: measured on MI355X at K = 2048 / 8192 it takes 0.6-0.75x the time
// of the best table entry for up to one block per compute unit and loses beyond (every extra
// round re-streams the weights).

// Entries with a kernel for this dtype / epilogue / row mode: no fp32 kernel for 0, 7 and 9;
// the SwiGLU epilogue needs wave tiles of whole 64-column gate/up pairs and is built for 0, 1,
// 2 and 7; grouped rows are built for a short menu (each entry is a separate kernel).
static bool grouped_cfg(int c, bool swiglu) {
  return swiglu ? (c == 0 || c == 2 || c == 7) : (c == 0 || c == 2 || c == 4 || c == 6 || c == 11);
}
static bool cfg_ok(int dtype, int c, bool swiglu, bool grouped) {
  if (c < 0 || c >= kNumCfg) return false;
  if (dtype == BIOPS_F32 && (c == 0 || c == 9)) return false;
  if (grouped && !grouped_cfg(c, swiglu)) return false;
  return !swiglu || c <= 2 || c == 7;
}

static int pick_cfg(int dtype, const BmmArgs& a, int epi, bool skinny_ok, bool nmajor16) {
  const bool swiglu = epi == kEpiSwiglu;
  const bool grouped = a.grp != nullptr;
  const int forced = forced_cfg();
  if (forced == kSkinnyCfg && skinny_ok) return forced;
  // Four-wave entries: the skinny conditions (direct loads, K-major B, plain rows, no SwiGLU),
  // or the same with a 16-bit N-major B; 32-bit output offsets inside a 256-row tile.
  const bool big_ok = (skinny_ok || (nmajor16 && !swiglu && !grouped)) && dtype != BIOPS_F32 &&
                      a.ldc < (int64_t(1) << 23);
  if (forced >= kBigCfg && forced < kBigEnd && big_ok) return forced;
  // The weight-streaming entries: grouped rows, 16-bit N-major B on the direct path.
  const bool stream_ok = grouped && nmajor16;
  if (forced >= kStreamCfg && forced < kMenuSize && stream_ok) return forced;
  if (cfg_ok(dtype, forced, swiglu, grouped)) return forced;
  const int cus = device_cus();
  const int64_t batch = a.nb1 * a.nb2;
  // Grouped rows: groups of the mean size.
  const int64_t groups = std::max<int64_t>(1, std::min(a.grp_groups, a.grp_rows));
  const int64_t mean = a.grp_rows / groups;
  int best = 2;
  double best_cost = 1e300;
  for (int c = 0; c < kNumCfg; ++c) {
    if (!cfg_ok(dtype, c, swiglu, grouped)) continue;
    const int64_t cols = swiglu ? kCfgBN[c] / 2 : kCfgBN[c];
    // grouped: a group of the mean size spans mean / BM tiles plus, on average, half a tile of
    // its last partial m-tile (and at least one tile)
    const double per_group = std::max((double)cdiv(mean, kCfgBM[c]), (double)mean / kCfgBM[c] + 0.5);
    const int64_t mt = grouped ? (int64_t)(groups * per_group + 0.5) : batch * cdiv(a.M, kCfgBM[c]);
    const int64_t tiles = mt * cdiv(a.N, cols);
    const double rate = kCfgRate[c] * (nmajor16 ? kCfgNmajorShare[c] : 1.0);
    const double cost = (double)cdiv(tiles, cus) * kCfgBM[c] * kCfgBN[c] / rate;
    if (cost < best_cost) { best_cost = cost; best = c; }
  }
  // Long K with up to four 32x32 tiles per compute unit: four resident one-wavefront
  // workgroups keep more of the operand stream in flight than one 64x64 workgroup, despite
  // twice the bytes (MI355X, M = 512, N = 2048, K = 8192: 39.1 us against 45.8 us; M = 128,
  // N = 8192, K = 2048: 12.9 against 15.0 us; with more tiles than that the 64x64 entry wins:
  // 54.6 against 78.2 us at M = 1024, N = 2048, K = 8192).
  const bool prefer32 = a.K >= 2048 && !grouped && !swiglu && batch * cdiv(a.M, 32) * cdiv(a.N, 32) <= 4 * cus;
  // The four-wave entries (13-19) join the same cost model from K = 1024 on, at their own
  // rates.  Measured on MI355X (bf16, one box, against the best of entries 0-12, us):
  // 3072 x 4096 x 2048 52.3 / 70.1 (256x256, 192 tiles), 2048 x 6144 x 4096 101.8 / 130.6
  // (256x256), 4096 x 6144 x 4096 184.7 / 200.9 (256x128, three rounds), 4096 x 2048 x 8192
  // 120.2 / 127.0 (256x128), 2048 x 2048 x 8192 71.8 / 80.0 (128x128), 1024 x 2048 x 8192
  // 50.7 / 54.8 (128x64), 512 x 8192 x 2048 22.9 / 26.7 (128x128), 2048 x 2048 x 1024
  // 14.2 / 16.9 (128x128), 1024 x 4096 x 4096 38.8 / 45.1 (128x128).
  if (big_ok && a.K >= 1024)
    for (int i = 0; i < kBigAutoCount; ++i) {
      const int64_t tiles = batch * cdiv(a.M, kBigBM[i]) * cdiv(a.N, kBigBN[i]);
      const double rate = kBigRate[i] * (nmajor16 ? kBigNmajorShare[i] : 1.0);
      const double cost = (double)cdiv(tiles, cus) * kBigBM[i] * kBigBN[i] / rate;
      if (cost < best_cost) { best_cost = cost; best = kBigCfg + i; }
    }
  // There the four-wave 64x64 block (4-stage ring), where it applies, beat both (MI355X, all
  // entries forced on one box: M = 512, N = 2048, K = 8192: 34.5 against 37.1 us for entry 6;
  // M = 256: 33.3 against 34.5; M = 128, N = 8192, K = 2048: 11.6 against 12.4; M = 64: 10.9
  // against 11.4).
  if ((best == 4 || best == 6) && prefer32) best = (big_ok && !nmajor16) ? kBigCfg + 6 : 6;
  // The skinny entry: 32-column (or narrower) blocks in one round, or, with at least two row
  // blocks and K >= 1024, 64-column blocks in one round (MI355X, bf16, same-box A/B against the
  // automatic choice before them, same bits: 256 x 2048 x 8192 33.7 -> 26.8 us, 128 x 4096 x
  // 4096 18.3 -> 15.6 us, 512 x 1024 x 4096 18.3 -> 15.5 us, 96 x 5000 x 2048 11.6 -> 10.1 us,
  // 512 x 1024 x 1024 7.9 -> 7.3 us; with one row block or K = 512 they lost: 32 x 16384 x
  // 2048 13.0 -> 14.0 us, 64 x 8192 x 512 6.0 -> 6.3 us), or, for 16-bit types, 64-row blocks
  // of 32 or 64 columns in one round with 2 to 8 of them down M (512 x 2048 x 8192 38.4 ->
  // 33.0 us, 300 x 3000 x 2048 11.7 -> 10.3 us, 128 x 8192 x 2048 12.7 -> 12.2 us; 16 down M
  // lost: 1024 x 1024 x 4096 19.0 -> 19.8 us).
  const int64_t row_blocks = batch * cdiv(a.M, 32), row_blocks64 = batch * cdiv(a.M, 64);
  if (skinny_ok && (row_blocks * cdiv(a.N, 32) <= cus ||
                    (row_blocks >= 2 && a.K >= 1024 && row_blocks * cdiv(a.N, 64) <= cus) ||
                    (dtype != BIOPS_F32 && row_blocks64 >= 2 && row_blocks64 <= 8 && a.K >= 1024 &&
                     row_blocks64 * cdiv(a.N, 64) <= cus)))
    best = kSkinnyCfg;
  // Grouped rows of at most 56 rows per group on average with a 16-bit N-major B (the MoE
  // expert GEMMs of calls up to about 7E/k tokens): the weight-streaming entries.  MI355X, C5
  // shapes (E = 64, D = 2048, I = 768, top-8), per sparse MoE call against the best table entry:
  // 1 token 47.1 us (16 rows) against 62.8 (entry 7); 2 tokens 56.3 against 74.5 (entry 2);
  // 32 tokens 154.6 (32 rows) against 171.4; 128 tokens 130.5 (32 rows) against 160.9; 256
  // tokens (32 rows per group) 160.1 (64 rows) against 170.8.  With the 128-column plain
  // blocks of 64-row m-tiles (same box): 384 tokens 167.3-173.0 against 173.8 (entry 2), 448
  // tokens 170.5 against 176.3; at 512 tokens entry 2 wins, 176.7 against 184.7.
  if (stream_ok && mean <= 56)
    best = mean <= 2 ? kStreamCfg : mean <= 16 ? kStreamCfg + 1 : kStreamCfg + 2;
  return best;
}

template <typename T, int AR, int BC>
static int launch_skinny_block(const BmmArgs& a0, hipStream_t stream) {
  BmmArgs a = a0;
  a.tiles_m = cdiv(a.M, AR > 32 ? 64 : 32);
  a.tiles_n = cdiv(a.N, BC);
  a.total = a.nb1 * a.nb2 * a.tiles_m * a.tiles_n;
  if (a.total == 0) return BIOPS_OK;
  if (a.total >= (int64_t(1) << 31) - 8) return fail(BIOPS_ERR_SIZE, "too many GEMM tiles");
  // a whole number of workgroups per XCD, so that xcd_slot keeps neighbouring blocks (which
  // share A rows and B columns) on one XCD; the extra workgroups exit at once
  const int64_t grid = (a.total + 7) & ~int64_t(7);
  using S = SkinnyTile<T, AR, BC>;
  if constexpr (S::DEEP) {
    const int64_t kt = a.K / S::BK;
    if (kt % S::UD == 0) {
      hipLaunchKernelGGL((skinny_deep_kernel<T, AR, BC>), dim3((unsigned)grid), dim3(S::DTHREADS), 0, stream, a);
      return check_launch("skinny_deep_kernel");
    }
  }
  hipLaunchKernelGGL((skinny_kernel<T, AR, BC>), dim3((unsigned)grid), dim3(S::THREADS), 0, stream, a);
  return check_launch("skinny_kernel");
}

// Block width: the narrowest of 8 / 16 / 32 / 64 columns whose blocks still fit one round on the
// compute units (N = 2048: 8 columns at M <= 32, 16 columns at M = 64, 64 columns at M = 256).
// Measured on MI355X, N = 2048, K = 8192: M = 64 takes 15.5 us at 16 columns against 19.8 us
// at 32.
template <typename T, int AR>
static int launch_skinny_rows(const BmmArgs& a, hipStream_t stream) {
  const int64_t cus = device_cus();
  const int64_t row_blocks = a.nb1 * a.nb2 * cdiv(a.M, 32);
  if (row_blocks * cdiv(a.N, 8) <= cus) return launch_skinny_block<T, AR, 8>(a, stream);
  if (row_blocks * cdiv(a.N, 16) <= cus) return launch_skinny_block<T, AR, 16>(a, stream);
  if (row_blocks * cdiv(a.N, 32) <= cus) return launch_skinny_block<T, AR, 32>(a, stream);
  return launch_skinny_block<T, AR, 64>(a, stream);
}

// Grouped rows, 16-bit N-major B: one m-tile x 64 (WIDE: 128) output columns per workgroup.  Like the
// one-tile-per-workgroup grouped entries, XCD x (workgroups g with g % 8 == x) takes the x-th
// eighth of the tiles; the tiles are numbered column-block-major, so the m-tiles of one group
// and column block (the same weights) fall on one XCD and its L2.
template <typename T, int BM, bool SWIGLU, bool WIDE>
__global__ __launch_bounds__((StreamTile<T, BM, SWIGLU, WIDE>::THREADS)) void stream_kernel(BmmArgs args) {
  using S = StreamTile<T, BM, SWIGLU, WIDE>;
  __shared__ __attribute__((aligned(16))) char smem[S::LDS_BYTES];
  const uint32_t J = (uint32_t)args.grp[0];
  const uint32_t total = J * (uint32_t)args.tiles_n;
  const uint32_t per = (total + 7u) / 8u;
  const uint32_t i = blockIdx.x / 8u, x = blockIdx.x % 8u;
  const uint32_t t = x * per + i;
  if (i >= per || t >= total) return;
  const uint32_t tn = t / J, tm = t - tn * J;
  const int32_t* e = args.grp + kGrpHeader + kGrpStride * tm;
  const int64_t m0 = e[1], rows = e[2] - e[1];
  const int64_t n0 = (int64_t)tn * S::BLOCK_OUT;
  const int64_t boff = (int64_t)e[0] * args.sB1 + n0;
  typename S::Sources src;
  src.A = reinterpret_cast<const T*>(args.A);
  src.lda = args.lda;
  src.a_rows = args.a_rows;
  src.m0 = m0;
  src.rows = rows < BM ? (int)rows : BM;
  src.bg = reinterpret_cast<const T*>(args.B) + boff;
  src.bu = reinterpret_cast<const T*>(SWIGLU ? args.B2 : args.B) + boff + (WIDE ? S::OUT : 0);
  src.ldb = args.ldb;
  src.ncols = args.N - n0;
  src.K = args.K;
  const typename S::Acc acc = S::run(smem, src);
  S::store(acc, reinterpret_cast<T*>(args.C) + m0 * args.ldc + n0, args.ldc, src.rows, src.ncols);
}

template <typename T, int BM, bool SWIGLU>
static int launch_stream(const BmmArgs& a0, hipStream_t stream) {
  constexpr bool WIDE = !SWIGLU && BM == 64;  // 128-column plain blocks
  using S = StreamTile<T, BM, SWIGLU, WIDE>;
  BmmArgs a = a0;
  a.tiles_m = cdiv(a.grp_rows, BM) + std::min(a.grp_groups, a.grp_rows);
  a.tiles_n = cdiv(a.N, S::BLOCK_OUT);
  a.total = a.tiles_m * a.tiles_n;
  if (a.total == 0) return BIOPS_OK;
  if (a.total >= (int64_t(1) << 31) - 8) return fail(BIOPS_ERR_SIZE, "too many GEMM tiles");
  const int64_t grid = (a.total + 7) & ~int64_t(7);
  hipLaunchKernelGGL((stream_kernel<T, BM, SWIGLU, WIDE>), dim3((unsigned)grid), dim3(S::THREADS), 0, stream, a);
  return check_launch("stream_kernel");
}

template <typename T, int BM, int BN, int SB, bool BKM>
static int launch_big(const BmmArgs& a0, hipStream_t stream) {
  BmmArgs a = a0;
  a.tiles_m = cdiv(a.M, BM);
  a.tiles_n = cdiv(a.N, BN);
  a.total = a.nb1 * a.nb2 * a.tiles_m * a.tiles_n;
  if (a.total == 0) return BIOPS_OK;
  if (a.total >= (int64_t(1) << 31) - 8) return fail(BIOPS_ERR_SIZE, "too many GEMM tiles");
  const int cus = device_cus();
  if (cus <= 0) return fail(BIOPS_ERR_HIP, "no HIP device");
  a.nt_store = a.total <= cus ? 1 : 0;  // one round: non-temporal output stores (gemm_big.h)
  const int64_t grid = (a.total + 7) & ~int64_t(7);  // whole workgroups per XCD (xcd_slot)
  hipLaunchKernelGGL((big_kernel<T, BM, BN, SB, BKM>), dim3((unsigned)grid), dim3(256), 0, stream, a);
  return check_launch("big_kernel");
}

// A rows loaded per stage: the fewest of 8 / 16 / 32 that hold a block's rows.
template <typename T>
static int launch_skinny(const BmmArgs& a, hipStream_t stream) {
  if (a.M <= 8) return launch_skinny_rows<T, 8>(a, stream);
  if (a.M <= 16) return launch_skinny_rows<T, 16>(a, stream);
  // 64-row blocks (16-bit types) where 32-row blocks of up to 64 columns take more than one
  // round and 64-row ones fit it (pick_cfg's rule)
  if constexpr (sizeof(T) == 2) {
    const int64_t cus = device_cus(), batch = a.nb1 * a.nb2;
    if (batch * cdiv(a.M, 32) * cdiv(a.N, 64) > cus && batch * cdiv(a.M, 64) * cdiv(a.N, 64) <= cus) {
      if (batch * cdiv(a.M, 64) * cdiv(a.N, 32) <= cus) return launch_skinny_block<T, 64, 32>(a, stream);
      return launch_skinny_block<T, 64, 64>(a, stream);
    }
  }
  return launch_skinny_rows<T, 32>(a, stream);
}

template <typename T, int CFG, bool BKM, bool DIRECT, int EPI, bool GRP>
static int launch_cfg(const BmmArgs& a0, hipStream_t stream) {
  using C = Cfg<CFG>;
  BmmArgs a = a0;
  constexpr int64_t kCols = EPI == kEpiSwiglu ? C::bn / 2 : C::bn;
  constexpr bool grouped = GRP;
  a.tiles_m = grouped ? cdiv(a.grp_rows, C::bm) + std::min(a.grp_groups, a.grp_rows) : cdiv(a.M, C::bm);
  a.tiles_n = cdiv(a.N, kCols);
  a.total = (grouped ? 1 : a.nb1 * a.nb2) * a.tiles_m * a.tiles_n;
  if (a.total == 0) return BIOPS_OK;
  if (a.total >= (int64_t(1) << 31) - 8) return fail(BIOPS_ERR_SIZE, "too many GEMM tiles");
  const int cus = device_cus();
  if (cus <= 0) return fail(BIOPS_ERR_HIP, "no HIP device");
  int64_t grid = C::persist ? (int64_t)cus * C::per_cu : a.total;
  if (a.total < grid) grid = a.total;
  // whole workgroups per XCD: the grouped walk deals tiles by XCD, and xcd_slot keeps
  // neighbouring tiles on one XCD only then; the extra workgroups find no tile
  grid = (grid + 7) & ~int64_t(7);
  hipLaunchKernelGGL((bmm_kernel<T, CFG, BKM, DIRECT, EPI, GRP>), dim3((unsigned)grid), dim3(C::threads),
                     0, stream, a);
  return check_launch("bmm_kernel");
}

template <typename T, int CFG, int EPI, bool GRP = false>
static int launch_layout(const BmmArgs& a, bool b_kmajor, bool direct, hipStream_t s) {
  if (!b_kmajor) {
    if (direct) return launch_cfg<T, CFG, false, true, EPI, GRP>(a, s);
    return launch_cfg<T, CFG, false, false, EPI, GRP>(a, s);
  }
  if (direct) return launch_cfg<T, CFG, true, true, EPI, GRP>(a, s);
  return launch_cfg<T, CFG, true, false, EPI, GRP>(a, s);
}

template <typename T, int EPI>
static int launch_grouped_typed(const BmmArgs& a, bool b_kmajor, bool direct, int cfg, hipStream_t s) {
  constexpr bool kPlain = EPI != kEpiSwiglu;
  switch (cfg) {
    case 0: if constexpr (sizeof(T) == 2) return launch_layout<T, 0, EPI, true>(a, b_kmajor, direct, s); break;
    case 2: return launch_layout<T, 2, EPI, true>(a, b_kmajor, direct, s);
    case 4: if constexpr (kPlain) return launch_layout<T, 4, EPI, true>(a, b_kmajor, direct, s); break;
    case 6: if constexpr (kPlain) return launch_layout<T, 6, EPI, true>(a, b_kmajor, direct, s); break;
    case 7: if constexpr (!kPlain) return launch_layout<T, 7, EPI, true>(a, b_kmajor, direct, s); break;
    case 11: if constexpr (kPlain) return launch_layout<T, 11, EPI, true>(a, b_kmajor, direct, s); break;
    case kStreamCfg:
      if constexpr (sizeof(T) == 2) return launch_stream<T, 16, !kPlain>(a, s);
      break;
    case kStreamCfg + 1:
      if constexpr (sizeof(T) == 2) return launch_stream<T, 32, !kPlain>(a, s);
      break;
    case kStreamCfg + 2:
      if constexpr (sizeof(T) == 2) return launch_stream<T, 64, !kPlain>(a, s);
      break;
    default: break;
  }
  return fail(BIOPS_ERR_ARG, "no grouped kernel for tile config %d", cfg);
}

template <typename T, int EPI>
static int launch_typed(const BmmArgs& a, bool b_kmajor, bool direct, int cfg, hipStream_t s) {
  if constexpr (EPI == kEpiSwiglu) {
    switch (cfg) {
      case 0: if constexpr (sizeof(T) == 2) return launch_layout<T, 0, EPI>(a, b_kmajor, direct, s); break;
      case 1: return launch_layout<T, 1, EPI>(a, b_kmajor, direct, s);
      case 2: return launch_layout<T, 2, EPI>(a, b_kmajor, direct, s);
      case 7: return launch_layout<T, 7, EPI>(a, b_kmajor, direct, s);
      default: break;
    }
    return fail(BIOPS_ERR_ARG, "no SwiGLU kernel for tile config %d", cfg);
  } else {
    switch (cfg) {
      case 0: if constexpr (sizeof(T) == 2) return launch_layout<T, 0, EPI>(a, b_kmajor, direct, s); break;
      case 1: return launch_layout<T, 1, EPI>(a, b_kmajor, direct, s);
      case 2: return launch_layout<T, 2, EPI>(a, b_kmajor, direct, s);
      case 3: return launch_layout<T, 3, EPI>(a, b_kmajor, direct, s);
      case 4: return launch_layout<T, 4, EPI>(a, b_kmajor, direct, s);
      case 5: return launch_layout<T, 5, EPI>(a, b_kmajor, direct, s);
      case 6: return launch_layout<T, 6, EPI>(a, b_kmajor, direct, s);
      case 7: return launch_layout<T, 7, EPI>(a, b_kmajor, direct, s);
      case 8: return launch_layout<T, 8, EPI>(a, b_kmajor, direct, s);
      case 9: if constexpr (sizeof(T) == 2) return launch_layout<T, 9, EPI>(a, b_kmajor, direct, s); break;
      case 10: return launch_layout<T, 10, EPI>(a, b_kmajor, direct, s);
      case 11: return launch_layout<T, 11, EPI>(a, b_kmajor, direct, s);
      case kSkinnyCfg: return launch_skinny<T>(a, s);
      case kBigCfg:
        if constexpr (sizeof(T) == 2)
          return b_kmajor ? launch_big<T, 256, 256, 128, true>(a, s) : launch_big<T, 256, 256, 128, false>(a, s);
        break;
      case kBigCfg + 1:
        if constexpr (sizeof(T) == 2)
          return b_kmajor ? launch_big<T, 256, 128, 128, true>(a, s) : launch_big<T, 256, 128, 128, false>(a, s);
        break;
      case kBigCfg + 2:
        if constexpr (sizeof(T) == 2)
          return b_kmajor ? launch_big<T, 128, 256, 128, true>(a, s) : launch_big<T, 128, 256, 128, false>(a, s);
        break;
      case kBigCfg + 3:
        if constexpr (sizeof(T) == 2)
          return b_kmajor ? launch_big<T, 128, 128, 128, true>(a, s) : launch_big<T, 128, 128, 128, false>(a, s);
        break;
      case kBigCfg + 4:
        if constexpr (sizeof(T) == 2)
          return b_kmajor ? launch_big<T, 128, 64, 128, true>(a, s) : launch_big<T, 128, 64, 128, false>(a, s);
        break;
      case kBigCfg + 5:
        if constexpr (sizeof(T) == 2)
          return b_kmajor ? launch_big<T, 64, 128, 128, true>(a, s) : launch_big<T, 64, 128, 128, false>(a, s);
        break;
      case kBigCfg + 6:
        if constexpr (sizeof(T) == 2)
          return b_kmajor ? launch_big<T, 64, 64, 128, true>(a, s) : launch_big<T, 64, 64, 128, false>(a, s);
        break;
      default: break;
    }
    return fail(BIOPS_ERR_ARG, "no kernel for tile config %d", cfg);
  }
}

// BIOPS_GEMM_NO_DIRECT (any value) forces the register load path (read once per process).
static bool direct_disabled() {
  static const bool off = getenv("BIOPS_GEMM_NO_DIRECT") != nullptr;
  return off;
}

static bool aligned16(const void* p, int64_t ld, int elt) {
  return (reinterpret_cast<uintptr_t>(p) % 16 == 0) && ((ld * elt) % 16 == 0);
}

// Operand alignment flags and the direct-load condition; returns the tile entry to launch.
static int prepare_bmm(int dtype, BmmArgs& a, int epi, bool b_kmajor, bool& direct) {
  const int elt = dtype_bytes(dtype);
  a.a_vec = aligned16(a.A, a.lda, elt) && (a.sA1 * elt) % 16 == 0 && (a.sA2 * elt) % 16 == 0;
  bool bv = aligned16(a.B, a.ldb, elt) && (a.sB1 * elt) % 16 == 0 && (a.sB2 * elt) % 16 == 0;
  if (epi == kEpiSwiglu) bv = bv && aligned16(a.B2, a.ldb, elt);
  a.b_vec = bv;
  a.c_vec = aligned16(a.C, a.ldc, elt) && (a.sC1 * elt) % 16 == 0 && (a.sC2 * elt) % 16 == 0;
  if (a.gB <= 0) a.gB = 1;
  if (a.nb2 <= 0) a.nb2 = 1;
  // Direct global->LDS loads need whole 16-byte chunks: aligned operands, K a multiple of the
  // 128-byte step, and B K-major or N-major with N a multiple of 16 / elt.
  direct = a.a_vec && a.b_vec && ((a.K * elt) % kKBytes == 0) && (b_kmajor || (a.N * elt) % 16 == 0) &&
           !direct_disabled();
  // Grouped rows run on the table entries only (the skinny and large-tile kernels take a fixed
  // tile count from the host); those two read K-major B only.
  const bool skinny_ok = direct && b_kmajor && epi != kEpiSwiglu && a.grp == nullptr;
  return pick_cfg(dtype, a, epi, skinny_ok, direct && !b_kmajor && elt == 2);
}

int grouped_tile_rows(int dtype, BmmArgs a, int epi, bool b_kmajor) {
  if (dtype_bytes(dtype) == 0) return 0;
  bool direct;
  const int cfg = prepare_bmm(dtype, a, epi, b_kmajor, direct);
  if (cfg >= kStreamCfg && cfg < kMenuSize) return kStreamBM[cfg - kStreamCfg];
  return cfg >= 0 && cfg < kNumCfg ? kCfgBM[cfg] : 0;
}

// Tails pay off only when the groups span two m-tiles or more on average: each tail streams its
// group's whole B once more.  MI355X, C5 shapes (E = 64, D = 2048, I = 768, top-8), per sparse
// MoE call, same box, with tails against without: 4096 tokens (512 rows per expert, 256-row
// m-tiles) 471.3 against 496.3 us, 2048 tokens 323.1 against 319.7; without this condition
// 1024 tokens took 264.4 against 234.0 and 512 tokens 199.5 against 181.4.
int grouped_tail_rows(int dtype, BmmArgs a, int epi, bool b_kmajor) {
  if (dtype_bytes(dtype) != 2 || b_kmajor || a.grp == nullptr) return 0;
  bool direct;
  const int cfg = prepare_bmm(dtype, a, epi, b_kmajor, direct);
  if (!direct || cfg < 0 || cfg >= kNumCfg || kCfgBM[cfg] < 128) return 0;
  const int64_t groups = std::max<int64_t>(1, std::min(a.grp_groups, a.grp_rows));
  if (a.grp_rows / groups < 2 * kCfgBM[cfg]) return 0;
  return kStreamBM[kNumStream - 1];
}

int launch_grouped_tail(int dtype, BmmArgs a, int epi, hipStream_t stream) {
  constexpr int BM = kStreamBM[kNumStream - 1];
  a.nb1 = a.nb2 = a.gB = 1;
  a.sA1 = a.sA2 = a.sB2 = a.sC1 = a.sC2 = 0;
  switch (dtype) {
    case BIOPS_F16:
      return epi == kEpiSwiglu ? launch_stream<f16_t, BM, true>(a, stream) : launch_stream<f16_t, BM, false>(a, stream);
    case BIOPS_BF16:
      return epi == kEpiSwiglu ? launch_stream<bf16_t, BM, true>(a, stream) : launch_stream<bf16_t, BM, false>(a, stream);
    default:
      return fail(BIOPS_ERR_DTYPE, "no weight-streaming tile for dtype %d", dtype);
  }
}

int launch_bmm(int dtype, BmmArgs a, int epi, bool b_kmajor, hipStream_t stream) {
  bool direct;
  const int cfg = prepare_bmm(dtype, a, epi, b_kmajor, direct);
  if (a.grp) {
    a.nb1 = a.nb2 = a.gB = 1;
    a.sA1 = a.sA2 = a.sB2 = a.sC1 = a.sC2 = 0;
    switch (dtype) {
      case BIOPS_F32:
        return epi == kEpiSwiglu ? launch_grouped_typed<float, kEpiSwiglu>(a, b_kmajor, direct, cfg, stream)
                                 : launch_grouped_typed<float, kEpiPlain>(a, b_kmajor, direct, cfg, stream);
      case BIOPS_F16:
        return epi == kEpiSwiglu ? launch_grouped_typed<f16_t, kEpiSwiglu>(a, b_kmajor, direct, cfg, stream)
                                 : launch_grouped_typed<f16_t, kEpiPlain>(a, b_kmajor, direct, cfg, stream);
      case BIOPS_BF16:
        return epi == kEpiSwiglu ? launch_grouped_typed<bf16_t, kEpiSwiglu>(a, b_kmajor, direct, cfg, stream)
                                 : launch_grouped_typed<bf16_t, kEpiPlain>(a, b_kmajor, direct, cfg, stream);
      default:
        return fail(BIOPS_ERR_DTYPE, "unsupported GEMM dtype %d", dtype);
    }
  }
  switch (dtype) {
    case BIOPS_F32:
      return epi == kEpiSwiglu ? launch_typed<float, kEpiSwiglu>(a, b_kmajor, direct, cfg, stream)
                               : launch_typed<float, kEpiPlain>(a, b_kmajor, direct, cfg, stream);
    case BIOPS_F16:
      return epi == kEpiSwiglu ? launch_typed<f16_t, kEpiSwiglu>(a, b_kmajor, direct, cfg, stream)
                               : launch_typed<f16_t, kEpiPlain>(a, b_kmajor, direct, cfg, stream);
    case BIOPS_BF16:
      return epi == kEpiSwiglu ? launch_typed<bf16_t, kEpiSwiglu>(a, b_kmajor, direct, cfg, stream)
                               : launch_typed<bf16_t, kEpiPlain>(a, b_kmajor, direct, cfg, stream);
    default:
      return fail(BIOPS_ERR_DTYPE, "unsupported GEMM dtype %d", dtype);
  }
}

// ------------------------------------------------------------- grouped (varlen) ----
// Index of the plan item whose first tile (plan column `col`) is the last one <= t.
__device__ __forceinline__ int64_t plan_find(const int64_t* plan, int64_t items, int col, int64_t t) {
  int64_t lo = 0, hi = items - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (plan[kPlanHeader + kPlanStride * mid + col] <= t) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

template <typename T, int MODE>
__global__ __launch_bounds__(256) void grouped_kernel(GroupedArgs a) {
  constexpr int BM = kVarlenBM, BN = kVarlenBN;
  constexpr bool BKM = MODE == kGroupQK;  // K^T is K-major, V is N-major
  using Tile = GemmTile<T, BM, BN, 2, 2, 2, BKM, false>;
  __shared__ __attribute__((aligned(16))) char smem[Tile::SMEM_BYTES];
  typename Tile::Acc acc[Tile::FM][Tile::FN];
  constexpr int elt = sizeof(T);
  auto al = [](const void* p, int64_t off_elems) {
    return ((reinterpret_cast<uintptr_t>(p) + (uintptr_t)off_elems * elt) % 16) == 0;
  };

  const int64_t G = gridDim.x;
  const int col = MODE == kGroupQK ? 5 : 6;
  for (int64_t t = xcd_slot(blockIdx.x, G); t < a.total_tiles; t += G) {
    const int64_t it = plan_find(a.plan, a.items, col, t);
    const int64_t* p = a.plan + kPlanHeader + kPlanStride * it;
    const int64_t q0 = p[0], ql = p[1], k0 = p[2], kl = p[3], soff = p[4];
    const int64_t M = ql, N = MODE == kGroupQK ? kl : a.dv, K = MODE == kGroupQK ? a.d : kl;
    const int64_t tm_n = cdiv(M, BM), tn_n = cdiv(N, BN);
    const int64_t local = t - p[col];
    const int64_t h = local / (tm_n * tn_n);
    int64_t tm, tn;
    tile_coords(local - h * tm_n * tn_n, tm_n, tn_n, tm, tn);
    const int64_t hk = h / a.group;
    const int64_t m0 = tm * BM, n0 = tn * BN;
    const int64_t lds = varlen_score_ld(kl);  // padded score row pitch
    const int64_t s_head = soff + h * ql * lds;

    const T* A;
    int64_t lda;
    bool avec;
    BSource<T> src;
    T* C;
    int64_t ldc;
    if constexpr (MODE == kGroupQK) {
      const int64_t aoff = (q0 + m0) * a.sq_t + h * a.sq_h;
      A = reinterpret_cast<const T*>(a.q) + aoff;
      lda = a.sq_t;
      avec = al(a.q, aoff) && (lda * elt) % 16 == 0;
      const int64_t boff = (k0 + n0) * a.sk_t + hk * a.sk_h;
      src.p0 = reinterpret_cast<const T*>(a.k) + boff;
      src.ld = a.sk_t;
      src.vec_ok = al(a.k, boff) && (a.sk_t * elt) % 16 == 0;
      const int64_t coff = s_head + m0 * lds + n0;
      C = reinterpret_cast<T*>(a.s) + coff;
      ldc = lds;
    } else {
      const int64_t aoff = s_head + m0 * lds;
      A = reinterpret_cast<const T*>(a.s) + aoff;
      lda = lds;
      avec = al(a.s, aoff) && (lda * elt) % 16 == 0;
      const int64_t boff = k0 * a.sv_t + hk * a.sv_h + n0;
      src.p0 = reinterpret_cast<const T*>(a.v) + boff;
      src.ld = a.sv_t;
      src.vec_ok = al(a.v, boff) && (a.sv_t * elt) % 16 == 0;
      C = reinterpret_cast<T*>(a.out) + (q0 + m0) * a.so_t + h * a.so_h + n0;
      ldc = a.so_t;
    }
    src.p1 = src.p0;
    src.ncols = N - n0;
    src.swiglu = false;
    const int64_t rows = M - m0, cols = N - n0;

    Tile::mainloop(smem, acc, typename Tile::ARows{A, lda, rows}, avec, src, K);
    const bool cvec = al(C, 0) && (ldc * elt) % 16 == 0;
    Tile::template epilogue<false>(smem, acc, C, ldc, rows < BM ? (int)rows : BM,
                                   cols < BN ? (int)cols : BN, nullptr, cvec);
  }
}

template <typename T>
static int launch_grouped_t(const GroupedArgs& a, int mode, hipStream_t s) {
  if (a.total_tiles <= 0) return BIOPS_OK;
  const int cus = device_cus();
  if (cus <= 0) return fail(BIOPS_ERR_HIP, "no HIP device");
  int64_t grid = (int64_t)cus * 2;
  if (a.total_tiles < grid) grid = a.total_tiles;
  if (mode == kGroupQK)
    hipLaunchKernelGGL((grouped_kernel<T, kGroupQK>), dim3((unsigned)grid), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((grouped_kernel<T, kGroupPV>), dim3((unsigned)grid), dim3(256), 0, s, a);
  return check_launch("grouped_kernel");
}

int launch_grouped(int dtype, const GroupedArgs& a, int mode, hipStream_t stream) {
  switch (dtype) {
    case BIOPS_F32: return launch_grouped_t<float>(a, mode, stream);
    case BIOPS_F16: return launch_grouped_t<f16_t>(a, mode, stream);
    case BIOPS_BF16: return launch_grouped_t<bf16_t>(a, mode, stream);
    default: return fail(BIOPS_ERR_DTYPE, "unsupported dtype %d", dtype);
  }
}

bool b_layout(int64_t K, int64_t N, int64_t sBk, int64_t sBn, bool& kmajor, int64_t& ldb) {
  if (sBk == 1 || K <= 1) { kmajor = true; ldb = sBn; return true; }
  if (sBn == 1 || N <= 1) { kmajor = false; ldb = sBk; return true; }
  return false;
}

}  // namespace biops

using namespace biops;

extern "C" int biops_bmm(int dtype, int64_t nb1, int64_t nb2, int64_t M, int64_t N, int64_t K,
                         const void* A, int64_t sA1, int64_t sA2, int64_t sAm, int64_t sAk,
                         const void* B, int64_t sB1, int64_t sB2, int64_t gB, int64_t sBk,
                         int64_t sBn, void* C, int64_t sC1, int64_t sC2, int64_t sCm, int64_t sCn,
                         void* stream) {
  if (!is_float_dtype(dtype)) return fail(BIOPS_ERR_DTYPE, "unsupported dtype %d", dtype);
  if (nb1 < 0 || nb2 < 0 || M < 0 || N < 0 || K < 0) return fail(BIOPS_ERR_ARG, "negative size");
  if (gB < 1 || (nb2 > 0 && nb2 % gB != 0))
    return fail(BIOPS_ERR_ARG, "group %lld must divide the inner batch %lld", (long long)gB,
                (long long)nb2);
  if (nb1 == 0 || nb2 == 0 || M == 0 || N == 0) return BIOPS_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(BIOPS_ERR_ARG, "null operand");
  if (sAk != 1 && K > 1) return fail(BIOPS_ERR_LAYOUT, "A must be contiguous in K");
  if (sCn != 1 && N > 1) return fail(BIOPS_ERR_LAYOUT, "C must be contiguous in N");
  bool kmajor;
  int64_t ldb;
  if (!b_layout(K, N, sBk, sBn, kmajor, ldb))
    return fail(BIOPS_ERR_LAYOUT, "B needs a unit stride in K or in N");
  BmmArgs a{};
  a.A = A; a.B = B; a.B2 = nullptr; a.C = C; a.bias = nullptr;
  a.M = M; a.N = N; a.K = K;
  a.lda = sAm; a.ldb = ldb; a.ldc = sCm;
  a.nb1 = nb1; a.nb2 = nb2; a.gB = gB;
  a.sA1 = sA1; a.sA2 = sA2; a.sB1 = sB1; a.sB2 = sB2; a.sC1 = sC1; a.sC2 = sC2;
  return launch_bmm(dtype, a, kEpiPlain, kmajor, (hipStream_t)stream);
}

extern "C" int biops_gemm(int dtype, int64_t M, int64_t N, int64_t K, const void* A, int64_t sAm,
                          int64_t sAk, const void* B, int64_t sBk, int64_t sBn, const void* bias,
                          void* C, int64_t sCm, int64_t sCn, void* stream) {
  if (!is_float_dtype(dtype)) return fail(BIOPS_ERR_DTYPE, "unsupported dtype %d", dtype);
  if (M < 0 || N < 0 || K < 0) return fail(BIOPS_ERR_ARG, "negative size");
  if (M == 0 || N == 0) return BIOPS_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(BIOPS_ERR_ARG, "null operand");
  if (sAk != 1 && K > 1) return fail(BIOPS_ERR_LAYOUT, "A must be contiguous in K");
  if (sCn != 1 && N > 1) return fail(BIOPS_ERR_LAYOUT, "C must be contiguous in N");
  bool kmajor;
  int64_t ldb;
  if (!b_layout(K, N, sBk, sBn, kmajor, ldb))
    return fail(BIOPS_ERR_LAYOUT, "B needs a unit stride in K or in N");
  BmmArgs a{};
  a.A = A; a.B = B; a.B2 = nullptr; a.C = C; a.bias = bias;
  a.M = M; a.N = N; a.K = K;
  a.lda = sAm; a.ldb = ldb; a.ldc = sCm;
  a.nb1 = 1; a.nb2 = 1; a.gB = 1;
  return launch_bmm(dtype, a, bias ? kEpiBias : kEpiPlain, kmajor, (hipStream_t)stream);
}

// ------------------------------------------------------------------ K padding ----
// dst [rows_out, cols_out] = src [rows, cols] zero-extended; one 16-byte output chunk per thread
// and iteration.  Whole chunks of a 16-byte aligned source are read with one load, others
// element by element (a row of odd length is not 16-byte aligned after the first).
struct PadArgs {
  const void* src;
  void* dst;
  int64_t rows, cols, ld, rows_out, cols_out;
  int64_t batches, sbatch;  // source matrices and their stride (elements); destinations follow each other
  int32_t vec;              // src, ld and sbatch 16-byte aligned
};

template <int E>
__global__ __launch_bounds__(256) void pad_rows_kernel(PadArgs a) {
  using W = typename std::conditional<E == 2, uint16_t, uint32_t>::type;
  constexpr int V = 16 / E;
  const int64_t cpr = a.cols_out / V;
  const int64_t per = a.rows_out * cpr;  // chunks of one destination matrix
  const int64_t total = a.batches * per;
  const W* src = reinterpret_cast<const W*>(a.src);
  W* dst = reinterpret_cast<W*>(a.dst);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t b = i / per, j = i - b * per;
    const int64_t r = j / cpr, k0 = (j - r * cpr) * V;
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (r < a.rows && k0 < a.cols) {
      const W* s = src + b * a.sbatch + r * a.ld + k0;
      if (a.vec && k0 + V <= a.cols) {
        v = *reinterpret_cast<const u32x4_t*>(s);
      } else {
        W e[V];
#pragma unroll
        for (int j = 0; j < V; ++j) e[j] = k0 + j < a.cols ? s[j] : W(0);
        v = __builtin_bit_cast(u32x4_t, e);
      }
    }
    *reinterpret_cast<u32x4_t*>(dst + i * V) = v;
  }
}

static int pad_rows(int dtype, int64_t rows, int64_t cols, const void* src, int64_t ld_src, int64_t rows_out,
                    int64_t cols_out, void* dst, hipStream_t stream, int64_t batches = 1, int64_t sbatch = 0) {
  const int elt = dtype_bytes(dtype);
  if (!is_float_dtype(dtype)) return fail(BIOPS_ERR_DTYPE, "unsupported dtype %d", dtype);
  if (rows < 0 || cols < 0 || rows_out < rows || cols_out < cols)
    return fail(BIOPS_ERR_ARG, "padded shape [%lld, %lld] smaller than [%lld, %lld]", (long long)rows_out,
                (long long)cols_out, (long long)rows, (long long)cols);
  if ((cols_out * elt) % 16 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0)
    return fail(BIOPS_ERR_LAYOUT, "padded rows must be whole 16-byte chunks on a 16-byte aligned base");
  if (rows > 1 && ld_src < cols) return fail(BIOPS_ERR_LAYOUT, "source rows overlap");
  if (rows_out == 0 || cols_out == 0) return BIOPS_OK;
  if (!dst || (rows > 0 && cols > 0 && !src)) return fail(BIOPS_ERR_ARG, "null operand");
  PadArgs a{src, dst, rows, cols, ld_src, rows_out, cols_out, batches, sbatch, 0};
  a.vec = reinterpret_cast<uintptr_t>(src) % 16 == 0 && (ld_src * elt) % 16 == 0 && (sbatch * elt) % 16 == 0;
  const int64_t chunks = batches * rows_out * (cols_out * elt / 16);
  const int64_t blocks = std::min<int64_t>(cdiv(chunks, 256), 8192);
  if (elt == 2)
    hipLaunchKernelGGL(pad_rows_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(pad_rows_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return check_launch("pad_rows_kernel");
}

extern "C" int biops_pad_rows(int dtype, int64_t rows, int64_t cols, const void* src, int64_t ld_src,
                              int64_t rows_out, int64_t cols_out, void* dst, void* stream) {
  return pad_rows(dtype, rows, cols, src, ld_src, rows_out, cols_out, dst, (hipStream_t)stream);
}

// Padded operands of biops_gemm_padded: A [M, Kp] at the workspace base, B [N, Kp] (K-major) or
// [Kp, Np] (row-major, Np the row length rounded up to whole 16-byte chunks) 256 bytes further
// on; Kp = K rounded up to a whole number of 128-byte steps.
struct PadLayout {
  int64_t kp, np, a_bytes, bytes;
};
static PadLayout pad_layout(int elt, int64_t M, int64_t N, int64_t K, bool kmajor) {
  PadLayout p;
  const int64_t step = kKBytes / elt;
  p.kp = cdiv(K, step) * step;
  p.np = kmajor ? N : cdiv(N * elt, 16) * 16 / elt;
  p.a_bytes = cdiv(M * p.kp * elt, 256) * 256;
  p.bytes = p.a_bytes + (kmajor ? N * p.kp : p.kp * p.np) * elt;
  return p;
}

extern "C" int64_t biops_gemm_padded_workspace_size(int dtype, int64_t M, int64_t N, int64_t K, int64_t sBk,
                                                     int64_t sBn) {
  bool kmajor;
  int64_t ldb;
  const int elt = dtype_bytes(dtype);
  if (!is_float_dtype(dtype) || M < 0 || N < 0 || K < 0 || !b_layout(K, N, sBk, sBn, kmajor, ldb)) return -1;
  return pad_layout(elt, M, N, K, kmajor).bytes;
}

extern "C" int biops_gemm_padded(int dtype, int64_t M, int64_t N, int64_t K, const void* A, int64_t sAm,
                                 int64_t sAk, const void* B, int64_t sBk, int64_t sBn, const void* bias,
                                 void* C, int64_t sCm, int64_t sCn, void* workspace, int64_t workspace_bytes,
                                 void* stream) {
  if (!is_float_dtype(dtype)) return fail(BIOPS_ERR_DTYPE, "unsupported dtype %d", dtype);
  if (M < 0 || N < 0 || K < 0) return fail(BIOPS_ERR_ARG, "negative size");
  if (M == 0 || N == 0) return BIOPS_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(BIOPS_ERR_ARG, "null operand");
  if (sAk != 1 && K > 1) return fail(BIOPS_ERR_LAYOUT, "A must be contiguous in K");
  if (sCn != 1 && N > 1) return fail(BIOPS_ERR_LAYOUT, "C must be contiguous in N");
  bool kmajor;
  int64_t ldb;
  if (!b_layout(K, N, sBk, sBn, kmajor, ldb)) return fail(BIOPS_ERR_LAYOUT, "B needs a unit stride in K or in N");
  const int elt = dtype_bytes(dtype);
  const PadLayout p = pad_layout(elt, M, N, K, kmajor);
  if (workspace_bytes < p.bytes)
    return fail(BIOPS_ERR_SIZE, "workspace %lld < %lld bytes", (long long)workspace_bytes, (long long)p.bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return fail(BIOPS_ERR_LAYOUT, "workspace must be 256-byte aligned");
  char* ap = static_cast<char*>(workspace);
  char* bp = ap + p.a_bytes;
  const hipStream_t s = (hipStream_t)stream;
  int rc = pad_rows(dtype, M, K, A, sAm, M, p.kp, ap, s);
  if (rc != BIOPS_OK) return rc;
  rc = kmajor ? pad_rows(dtype, N, K, B, ldb, N, p.kp, bp, s) : pad_rows(dtype, K, N, B, ldb, p.kp, p.np, bp, s);
  if (rc != BIOPS_OK) return rc;
  BmmArgs a{};
  a.A = ap; a.B = bp; a.B2 = nullptr; a.C = C; a.bias = bias;
  a.M = M; a.N = N; a.K = p.kp;
  a.lda = p.kp; a.ldb = kmajor ? p.kp : p.np; a.ldc = sCm;
  a.nb1 = 1; a.nb2 = 1; a.gB = 1;
  return launch_bmm(dtype, a, bias ? kEpiBias : kEpiPlain, kmajor, s);
}

// biops_bmm_padded: one padded copy per distinct batch matrix (a stride-0 operand is copied once).
static PadLayout pad_layout_batched(int elt, int64_t na, int64_t nb, int64_t M, int64_t N, int64_t K, bool kmajor) {
  PadLayout p = pad_layout(elt, M, N, K, kmajor);
  p.a_bytes = cdiv(na * M * p.kp * elt, 256) * 256;
  p.bytes = p.a_bytes + nb * (kmajor ? N * p.kp : p.kp * p.np) * elt;
  return p;
}

extern "C" int64_t biops_bmm_padded_workspace_size(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
                                                    int64_t sA, int64_t sB, int64_t sBk, int64_t sBn) {
  bool kmajor;
  int64_t ldb;
  const int elt = dtype_bytes(dtype);
  if (!is_float_dtype(dtype) || batch < 0 || M < 0 || N < 0 || K < 0 || !b_layout(K, N, sBk, sBn, kmajor, ldb))
    return -1;
  return pad_layout_batched(elt, sA == 0 ? 1 : batch, sB == 0 ? 1 : batch, M, N, K, kmajor).bytes;
}

extern "C" int biops_bmm_padded(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K, const void* A, int64_t sA,
                                int64_t sAm, int64_t sAk, const void* B, int64_t sB, int64_t sBk, int64_t sBn,
                                void* C, int64_t sC, int64_t sCm, int64_t sCn, void* workspace,
                                int64_t workspace_bytes, void* stream) {
  if (!is_float_dtype(dtype)) return fail(BIOPS_ERR_DTYPE, "unsupported dtype %d", dtype);
  if (batch < 0 || M < 0 || N < 0 || K < 0) return fail(BIOPS_ERR_ARG, "negative size");
  if (batch == 0 || M == 0 || N == 0) return BIOPS_OK;
  if (!C || (K > 0 && (!A || !B))) return fail(BIOPS_ERR_ARG, "null operand");
  if (sAk != 1 && K > 1) return fail(BIOPS_ERR_LAYOUT, "A must be contiguous in K");
  if (sCn != 1 && N > 1) return fail(BIOPS_ERR_LAYOUT, "C must be contiguous in N");
  bool kmajor;
  int64_t ldb;
  if (!b_layout(K, N, sBk, sBn, kmajor, ldb)) return fail(BIOPS_ERR_LAYOUT, "B needs a unit stride in K or in N");
  const int elt = dtype_bytes(dtype);
  const int64_t na = sA == 0 ? 1 : batch, nb = sB == 0 ? 1 : batch;
  const PadLayout p = pad_layout_batched(elt, na, nb, M, N, K, kmajor);
  if (workspace_bytes < p.bytes)
    return fail(BIOPS_ERR_SIZE, "workspace %lld < %lld bytes", (long long)workspace_bytes, (long long)p.bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return fail(BIOPS_ERR_LAYOUT, "workspace must be 256-byte aligned");
  char* ap = static_cast<char*>(workspace);
  char* bp = ap + p.a_bytes;
  const hipStream_t s = (hipStream_t)stream;
  int rc = pad_rows(dtype, M, K, A, sAm, M, p.kp, ap, s, na, sA);
  if (rc != BIOPS_OK) return rc;
  rc = kmajor ? pad_rows(dtype, N, K, B, ldb, N, p.kp, bp, s, nb, sB) : pad_rows(dtype, K, N, B, ldb, p.kp, p.np, bp, s, nb, sB);
  if (rc != BIOPS_OK) return rc;
  BmmArgs a{};
  a.A = ap; a.B = bp; a.B2 = nullptr; a.C = C; a.bias = nullptr;
  a.M = M; a.N = N; a.K = p.kp;
  a.lda = p.kp; a.ldb = kmajor ? p.kp : p.np; a.ldc = sCm;
  a.nb1 = batch; a.nb2 = 1; a.gB = 1;
  a.sA1 = na == 1 ? 0 : M * p.kp;
  a.sB1 = nb == 1 ? 0 : (kmajor ? N * p.kp : p.kp * p.np);
  a.sC1 = sC;
  return launch_bmm(dtype, a, kEpiPlain, kmajor, s);
}

extern "C" int biops_gemm_tile_count(void) { return kMenuSize; }

extern "C" int biops_set_gemm_tile(int cfg) {
  if (cfg < -1 || cfg >= kMenuSize) return fail(BIOPS_ERR_ARG, "tile entry %d outside [-1, %d)", cfg, kMenuSize);
  g_forced_cfg.store(cfg, std::memory_order_relaxed);
  return BIOPS_OK;
}
