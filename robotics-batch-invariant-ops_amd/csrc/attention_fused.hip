// Fused attention for 16-bit inputs: no score matrix in memory.
//
// One workgroup (four wavefronts) owns a tile of 128 query rows of one (batch, head) -- or of
// one (sequence, head) of a packed varlen batch -- and walks the key/value rows in fixed blocks
// of 64, in order, twice:
//   pass 1: S = Q K^T for the block, the reference's transform (below), then the running row
//           maximum m and the row sum l of exp(s - m) (rescaled when m grows);
//   pass 2: S again, P = round(exp(s - m) * (1 / l)), O += P V.
// The transform and the roundings are the eager composite's (batch_invariant_ops.py:1194-1212):
//   s = round(round(S) * scale); causal / boolean mask -> -inf; additive mask -> round(s + mask);
// P is normalised and rounded to the input dtype before it meets V; a row with no visible key
// gives zeros.  S itself is produced by the same MFMA sequence as the GEMM path (128-byte steps
// of the head dimension, chunk pairs in order), so its bits equal the materialised S.  The row
// sum is accumulated per lane in block order and combined across the two half-wavefronts, so it
// may differ from the row kernel's sum in the last fp32 bits.
//
// Batch invariance: a tile's arithmetic depends only on its own sequence (query rows, keys,
// values, mask) and on the head dimension; the block order and the MFMA sequence are fixed.
//
// Register layout (wavefront w owns query rows 32w .. 32w+31 of the tile).  The scores are
// computed transposed, S^T = K Q^T, with K as the MFMA A operand and Q as B, so that lane L holds
// query row L % 32 and keys 8j + 4(L/32) + i (j, i = 0..3) of each 32-key block.  Those eight
// keys per 16-key chunk are exactly one A-operand fragment of the P V product (with the key order
// inside the chunk permuted the same way for P and for V), so P goes from the accumulators to
// the next MFMA without passing through LDS.  V fragments come from LDS with the transposing
// 64-bit read.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <vector>

#include "gemm.h"
#include "rowops.h"

namespace biops {

struct FusedArgs {
  const void* q; const void* k; const void* v; void* out;
  const void* mask;
  const int64_t* plan;   // varlen work list (VARLEN kernels)
  const int64_t* order;  // varlen tile order: (item << 32) | query tile, longest key range first
  int64_t hq, group, hkv, lq, lk, d, dv;
  // element strides: batch (unused for varlen), head, row (token)
  int64_t sqB, sqH, sqL, skB, skH, skL, svB, svH, svL, soB, soH, soL;
  int64_t mB, mH, mI, mJ;
  int64_t items, tiles;
  float scale;
  int causal;
  int pow2;  // the scale is 2^k, -8 <= k <= 0 (bf16 kernels without an additive mask)
};

constexpr int kFusedBM = 128;  // query rows per workgroup
constexpr int kFusedBN = 64;   // keys per block
// The varlen kernels take their tiles from the work list's PV tile prefix (one tile per head
// and 128 query rows when dv <= 128).
static_assert(kFusedBM == kVarlenBM && kVarlenBN >= 128, "fused tiles follow the varlen plan");

template <typename T, int DP, int DVP>
struct FusedTile {
  static constexpr int THREADS = 256;
  static constexpr int KCH = DP / 8;   // 16-byte chunks per K row
  static constexpr int VCH = DVP / 8;  // 16-byte chunks per V row
  static constexpr int K_BYTES = kFusedBN * DP * 2;
  static constexpr int V_BYTES = kFusedBN * DVP * 2;
  static constexpr int LDS_BYTES = 2 * (K_BYTES + V_BYTES);
  static constexpr int K_LOADS = kFusedBN * KCH / THREADS;
  static constexpr int V_LOADS = kFusedBN * VCH / THREADS;
  static constexpr int QF = DP / 16;   // MFMAs per 32x32 score block
  static constexpr int OF = DVP / 32;  // 32-column output blocks
  static_assert(K_LOADS >= 1 && V_LOADS >= 1, "block loads");

  // K rows: 16-byte chunk c of row r at slot c ^ swz(r); 16 consecutive rows reading the same
  // chunk hit 16 distinct 16-byte bank slots.
  __device__ static __forceinline__ int k_off(int r, int c) {
    if constexpr (KCH == 16) return r * (DP * 2) + ((c ^ (r & 15)) << 4);
    else return r * (DP * 2) + ((c ^ ((r >> 1) & 7)) << 4);
  }
  // V rows: the layout of the GEMM's N-major operand stage (transposing reads, 4 rows at once).
  __device__ static __forceinline__ int v_off(int r, int col) { return lds_off_n<VCH>(r, col); }
};

// Per-tile geometry, decoded from the tile index.
struct FusedGeom {
  const char* q;  // first query row of the tile, this head
  const char* k;  // first key row of the sequence, this kv head
  const char* v;
  char* out;      // first output row of the tile, this head
  int64_t b, h;   // batch (0 for varlen) and query head
  int64_t qrows;  // valid query rows in the tile
  int64_t i0;     // index of the tile's first row inside its sequence
  int64_t ql, kl; // sequence lengths
};

// Tile order (workgroup w takes tile w; the dispatcher deals workgroups to the 8 XCDs in turn,
// so XCD x runs tiles x, x + 8, ...).  Causal tiles differ in cost by up to the number of query
// tiles, so the order is longest key range first, which keeps long tiles out of the launch's
// tail:
//   dense: (batch, head) pairs in chunks of kFusedChunk; inside a chunk, query tiles from the
//          last (longest causal key range) to the first, all pairs of the chunk per level.  When
//          the chunk holds a multiple of 8 pairs, XCD x takes pairs x*n/8 .. (x+1)*n/8 - 1 of it
//          at every level, so a head's key/value rows stay in one XCD's L2;
//   varlen: the host sorts (sequence, query tile) entries by key range
//          (biops_varlen_fused_order); the heads of an entry are consecutive tiles, and in
//          every chunk of kFusedChunk tiles XCD x takes the x-th eighth, so an entry's heads
//          share one XCD's L2.
constexpr int64_t kFusedChunk = 64;

template <typename T, bool VARLEN>
__device__ __forceinline__ bool fused_geom(const FusedArgs& a, int64_t t, FusedGeom& g) {
  constexpr int E = sizeof(T);
  int64_t h, qt, qstart = 0, kstart = 0, b = 0;
  if constexpr (VARLEN) {
    // Workgroup t runs XCD t % 8; in every chunk of kFusedChunk tiles (a multiple of 8), XCD x
    // takes tiles x n/8 .. (x+1) n/8 - 1, the heads of one or a few consecutive entries, so a
    // sequence's key/value rows are fetched into one XCD's L2 rather than into all eight.
    {
      const int64_t first = t / kFusedChunk * kFusedChunk;
      const int64_t n = a.tiles - first < kFusedChunk ? a.tiles - first : kFusedChunk;
      const int64_t j = t - first;
      if ((n & 7) == 0) t = first + (j & 7) * (n >> 3) + (j >> 3);
    }
    const int64_t e = a.order[t / a.hq];
    const int64_t item = e >> 32;
    qt = e & 0xffffffffLL;
    if (item < 0 || item >= a.items) return false;
    const int64_t* p = a.plan + kPlanHeader + kPlanStride * item;
    g.ql = p[1];
    g.kl = p[3];
    qstart = p[0];
    kstart = p[2];
    if (qt >= cdiv(g.ql, kFusedBM)) return false;
    h = t % a.hq;
  } else {
    g.ql = a.lq;
    g.kl = a.lk;
    const int64_t qtiles = cdiv(a.lq, kFusedBM);
    const int64_t pairs = a.tiles / qtiles;
    const int64_t chunk = t / (kFusedChunk * qtiles);
    const int64_t first = chunk * kFusedChunk;
    const int64_t n = pairs - first < kFusedChunk ? pairs - first : kFusedChunk;
    const int64_t r = t - chunk * kFusedChunk * qtiles;
    const int64_t j = r % n;
    qt = qtiles - 1 - r / n;
    // pair index: (batch, kv head, head in group), heads sharing a key/value head adjacent
    int64_t pair = first + ((n & 7) == 0 ? (j & 7) * (n >> 3) + (j >> 3) : j);
    const int64_t gi = pair % a.group;
    pair /= a.group;
    const int64_t hk = pair % a.hkv;
    b = pair / a.hkv;
    h = hk * a.group + gi;
  }
  const int64_t hk = h / a.group;
  g.i0 = qt * kFusedBM;
  g.qrows = g.ql - g.i0 < kFusedBM ? g.ql - g.i0 : kFusedBM;
  g.q = reinterpret_cast<const char*>(a.q) + E * (b * a.sqB + h * a.sqH + (qstart + g.i0) * a.sqL);
  g.k = reinterpret_cast<const char*>(a.k) + E * (b * a.skB + hk * a.skH + kstart * a.skL);
  g.v = reinterpret_cast<const char*>(a.v) + E * (b * a.svB + hk * a.svH + kstart * a.svL);
  g.out = reinterpret_cast<char*>(a.out) + E * (b * a.soB + h * a.soH + (qstart + g.i0) * a.soL);
  g.b = b;
  g.h = h;
  return true;
}

// Round two fp32 values to T (and back to fp32): one conversion each (for bf16, the pair
// conversion with +0 in the low half).
template <typename T>
__device__ __forceinline__ void round2(float& x0, float& x1) {
  x0 = Num<T>::round(x0);
  x1 = Num<T>::round(x1);
}

// First MFMA of a chain: the accumulator input is the constant zero.
template <typename T>
__device__ __forceinline__ f32x16_t mfma_first(const u32x4_t& a, const u32x4_t& b) {
  const f32x16_t z = {};
  if constexpr (std::is_same<T, bf16_t>::value)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), z, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), z, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
  if constexpr (std::is_same<T, bf16_t>::value) return f32x2_to_bf16x2_bits(x, y);
  else return (uint32_t)Num<T>::to_bits(x) | ((uint32_t)Num<T>::to_bits(y) << 16);
}

// MASK: 0 none, 1 boolean (bytes, nonzero = keep), 2 additive (T).  Wavefronts per SIMD: three
// with head sizes up to 64 (154-167 registers, 32 KiB of K/V blocks per workgroup; C4's varlen
// call, MI355X, same-box A/B: 157.7 -> 138.1 us, same bits), two up to 128 (the mixed 64 / 128
// heads spill at three), and with a 256-wide head (Q fragments and O accumulators twice as
// large, 128 KiB of K/V blocks) one with the full register file.
template <int DP, int DVP>
constexpr int fused_waves_per_eu() { return DP > 128 || DVP > 128 ? 1 : (DP <= 64 && DVP <= 64 ? 3 : 2); }

// P2: the scale is a power of two 2^k (-8 <= k <= 0), bf16 inputs, no additive mask.  Then
// round(round(S) * scale) = round(S) * scale exactly whenever the product is a normal number (a
// bf16 significand survives the power of two, and bf16 has fp32's exponent range), so the kernel
// keeps the scores in units of round(S) and folds the scale into the base change of the
// exponentials: scale * log2(e) is exact too, and so are the products with it.  Only a product
// below 2^-126 in magnitude (a bf16 denormal) skips its rounding.
template <typename T, int DP, int DVP, int MASK, bool VARLEN, bool P2>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(fused_waves_per_eu<DP, DVP>(),
                                                                     fused_waves_per_eu<DP, DVP>() < 2 ? 2 : fused_waves_per_eu<DP, DVP>())))
void fused_attn_kernel(FusedArgs a) {
  static_assert(!P2 || (MASK != 2 && std::is_same<T, bf16_t>::value), "power-of-two scale path");
  using F = FusedTile<T, DP, DVP>;
  __shared__ __attribute__((aligned(16))) char smem[F::LDS_BYTES];
  const int64_t t = blockIdx.x;
  if (t >= a.tiles) return;
  FusedGeom g;
  if (!fused_geom<T, VARLEN>(a, t, g)) return;

  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63, hf = lane >> 5, l32 = lane & 31;
  constexpr int E = sizeof(T);
  const u32x4_t zero4 = {0u, 0u, 0u, 0u};
  const int ql = (int)g.ql, kl = (int)g.kl, qrows = (int)g.qrows, i0 = (int)g.i0;
  const int shift = a.causal == BIOPS_CAUSAL_BOTTOM_RIGHT ? kl - ql : 0;

  // Key limit of tile-local row r: keys n >= lim(r) are masked out (sequence end, causal
  // alignment).  Limits grow with the row.
  auto row_lim = [&](int r) -> int {
    if (a.causal == BIOPS_CAUSAL_NONE) return kl;
    const int c = i0 + r + shift + 1;
    return c < 0 ? 0 : (c > kl ? kl : c);
  };
  // Query row of this lane (column of S^T); rows past the tile's end see no key.
  const int rloc = 32 * w + l32;
  const bool row_ok = rloc < qrows;
  const int lim = row_ok ? row_lim(rloc) : 0;
  const int tile_lim = qrows > 0 ? row_lim(qrows - 1) : 0;
  const int wrows = qrows - 32 * w;
  // keys this wavefront needs (wave-uniform), and key blocks of the workgroup
  const int wave_lim = wrows > 0 ? row_lim(32 * w + (wrows < 32 ? wrows : 32) - 1) : 0;
  const int nblk = (tile_lim + kFusedBN - 1) / kFusedBN;

  const char* mrow = nullptr;
  if constexpr (MASK != 0) {
    if (row_ok) {
      constexpr int ME = MASK == 1 ? 1 : E;  // mask strides count mask elements
      mrow = reinterpret_cast<const char*>(a.mask) + ME * (g.b * a.mB + g.h * a.mH + (int64_t)(i0 + rloc) * a.mI);
    }
  }

  // Q fragments (B operand of S^T = K Q^T): lane holds row l32, head-dim chunk 2cc + hf.
  u32x4_t qf[F::QF];
#pragma unroll
  for (int cc = 0; cc < F::QF; ++cc) {
    const int d0 = 16 * cc + 8 * hf;
    qf[cc] = (row_ok && d0 < a.d) ? *reinterpret_cast<const u32x4_t*>(g.q + E * (rloc * a.sqL + d0)) : zero4;
  }

  char* const kbuf0 = smem;
  char* const vbuf0 = smem + 2 * F::K_BYTES;

  // Block loads through registers: thread chunk s = tid + 256p is row s / CH, chunk s % CH.
  // Each thread keeps the byte offset of its chunks inside a block (head-dim chunks past the
  // problem point at chunk 0) and a validity flag.
  uint32_t koff[F::K_LOADS], voff[F::V_LOADS];
  bool kdv[F::K_LOADS], vdv[F::V_LOADS];
  int krow[F::K_LOADS], vrow_[F::V_LOADS];
#pragma unroll
  for (int p = 0; p < F::K_LOADS; ++p) {
    const int s = tid + F::THREADS * p;
    krow[p] = s / F::KCH;
    const int c = s % F::KCH;
    kdv[p] = 8 * c < a.d;
    koff[p] = (uint32_t)(E * (krow[p] * a.skL + (kdv[p] ? 8 * c : 0)));
  }
#pragma unroll
  for (int p = 0; p < F::V_LOADS; ++p) {
    const int s = tid + F::THREADS * p;
    vrow_[p] = s / F::VCH;
    const int c = s % F::VCH;
    vdv[p] = 8 * c < a.dv;
    voff[p] = (uint32_t)(E * (vrow_[p] * a.svL + (vdv[p] ? 8 * c : 0)));
  }
  u32x4_t kr[F::K_LOADS];
  u32x4_t vr[F::V_LOADS];
  // Rows of block blk: a whole block with the full head dimension reads in place; otherwise
  // rows n >= kl and chunks past the head dimension are zeros (read from a valid address).
  const bool kfull = a.d == DP, vfull = a.dv == DVP;
  auto load_k = [&](int blk) {
    const int n0 = blk * kFusedBN;
    const char* base = g.k + (int64_t)E * n0 * a.skL;
    if (n0 + kFusedBN <= kl && kfull) {
#pragma unroll
      for (int p = 0; p < F::K_LOADS; ++p) kr[p] = *reinterpret_cast<const u32x4_t*>(base + koff[p]);
    } else {
#pragma unroll
      for (int p = 0; p < F::K_LOADS; ++p) {
        const bool in = n0 + krow[p] < kl;
        const int64_t off = in ? (int64_t)koff[p] : -(int64_t)E * n0 * a.skL;  // row 0 of the sequence
        const u32x4_t x = *reinterpret_cast<const u32x4_t*>(base + off);
        kr[p] = (kdv[p] && in) ? x : zero4;
      }
    }
  };
  auto store_k = [&](int buf) {
#pragma unroll
    for (int p = 0; p < F::K_LOADS; ++p) {
      const int s = tid + F::THREADS * p;
      *reinterpret_cast<u32x4_t*>(kbuf0 + buf * F::K_BYTES + F::k_off(s / F::KCH, s % F::KCH)) = kr[p];
    }
  };
  auto load_v = [&](int blk) {
    const int n0 = blk * kFusedBN;
    const char* base = g.v + (int64_t)E * n0 * a.svL;
    if (n0 + kFusedBN <= kl && vfull) {
#pragma unroll
      for (int p = 0; p < F::V_LOADS; ++p) vr[p] = *reinterpret_cast<const u32x4_t*>(base + voff[p]);
    } else {
#pragma unroll
      for (int p = 0; p < F::V_LOADS; ++p) {
        const bool in = n0 + vrow_[p] < kl;
        const int64_t off = in ? (int64_t)voff[p] : -(int64_t)E * n0 * a.svL;
        const u32x4_t x = *reinterpret_cast<const u32x4_t*>(base + off);
        vr[p] = (vdv[p] && in) ? x : zero4;
      }
    }
  };
  auto store_v = [&](int buf) {
#pragma unroll
    for (int p = 0; p < F::V_LOADS; ++p) {
      const int s = tid + F::THREADS * p;
      *reinterpret_cast<u32x4_t*>(vbuf0 + buf * F::V_BYTES + F::v_off(s / F::VCH, 8 * (s % F::VCH))) = vr[p];
    }
  };

  // Smallest key limit among the wavefront's rows: key half-blocks below it need no limit test.
  const int wave_min_lim = wrows > 0 ? row_lim(32 * w) : 0;

  // Scores of keys 32 hb .. 32 hb + 31 of a block: acc[r] is key 64 blk + 32 hb + 8(r/4) +
  // 4 hf + r%4 of this lane's row.  s_mfma produces the raw fp32 S (one MFMA chain over the
  // head dimension); transform applies the reference's roundings and masks in place.
  // The K fragments of a chain are read from LDS before its first MFMA (a scheduling barrier
  // keeps the compiler from sinking each read next to its MFMA, which would expose one LDS
  // latency per MFMA).
  auto s_frags = [&](int buf, int hb, u32x4_t (&kf)[F::QF]) {
    const char* kb = kbuf0 + buf * F::K_BYTES;
#pragma unroll
    for (int cc = 0; cc < F::QF; ++cc)
      kf[cc] = *reinterpret_cast<const u32x4_t*>(kb + F::k_off(32 * hb + l32, 2 * cc + hf));
  };
  auto s_chain = [&](const u32x4_t (&kf)[F::QF], f32x16_t& acc) {
    acc = mfma_first<T>(kf[0], qf[0]);
#pragma unroll
    for (int cc = 1; cc < F::QF; ++cc) Mfma<T>::step(acc, kf[cc], qf[cc]);
  };
  // (Masked kernels leave the reads to the compiler: their mask words leave no registers for
  // the fragments.)
  auto s_mfma = [&](int buf, int hb, f32x16_t& acc) {
    if constexpr (MASK == 0) {
      u32x4_t kf[F::QF];
      s_frags(buf, hb, kf);
      __builtin_amdgcn_sched_barrier(0);
      s_chain(kf, acc);
    } else {
      const char* kb = kbuf0 + buf * F::K_BYTES;
      acc = mfma_first<T>(*reinterpret_cast<const u32x4_t*>(kb + F::k_off(32 * hb + l32, hf)), qf[0]);
#pragma unroll
      for (int cc = 1; cc < F::QF; ++cc)
        Mfma<T>::step(acc, *reinterpret_cast<const u32x4_t*>(kb + F::k_off(32 * hb + l32, 2 * cc + hf)), qf[cc]);
    }
  };
  // both halves of a block: all reads first
  auto s_mfma2 = [&](int buf, f32x16_t& acc0, f32x16_t& acc1) {
    if constexpr (MASK != 0) {
      s_mfma(buf, 0, acc0);
      s_mfma(buf, 1, acc1);
    } else {
      u32x4_t kf0[F::QF], kf1[F::QF];
      s_frags(buf, 0, kf0);
      s_frags(buf, 1, kf1);
      __builtin_amdgcn_sched_barrier(0);
      s_chain(kf0, acc0);
      s_chain(kf1, acc1);
    }
  };
  // Raw mask words of the 16 keys of a half-block: MASK 1 -> mw[j] holds the four bytes of keys
  // nb + 8j .. + 3; MASK 2 -> mw[2j], mw[2j+1] their four 16-bit values.  The launcher
  // guarantees contiguous, aligned mask rows and lk % 4 == 0, so a group of four keys starting
  // below the limit lies inside the row; groups at or past the limit read as 0 (they are
  // masked out by the limit test anyway).
  constexpr int MW = MASK == 2 ? 8 : 4;
  auto mask_words = [&](int blk, int hb, uint32_t (&mw)[MW]) {
    if constexpr (MASK != 0) {
      const int nb = blk * kFusedBN + 32 * hb + 4 * hf;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n0 = nb + 8 * j;
        const bool in = n0 < lim;
        if constexpr (MASK == 1) {
          mw[j] = in ? *reinterpret_cast<const uint32_t*>(mrow + n0) : 0u;
        } else {
          const u32x2_t x = in ? *reinterpret_cast<const u32x2_t*>(mrow + E * n0) : u32x2_t{0u, 0u};
          mw[2 * j] = x[0];
          mw[2 * j + 1] = x[1];
        }
      }
    }
  };
  // Keys 8(r/4) + r%4 (relative to nb) at or past rel = lim - nb are masked out; OPEN skips the
  // test (every key of the half-block is visible to every row of the wavefront).
  auto transform = [&](auto open, int blk, int hb, f32x16_t& acc, const uint32_t (&mw)[MW]) {
    const int rel = lim - (blk * kFusedBN + 32 * hb + 4 * hf);
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      float s0 = acc[r], s1 = acc[r + 1];
      round2<T>(s0, s1);
      if constexpr (!P2) {
        s0 *= a.scale;
        s1 *= a.scale;
        round2<T>(s0, s1);
      }
      if constexpr (!decltype(open)::value) {
        const int o = 8 * (r >> 2) + (r & 3);
        s0 = o < rel ? s0 : -INFINITY;
        s1 = o + 1 < rel ? s1 : -INFINITY;
      }
      if constexpr (MASK == 1) {
        const uint32_t wj = mw[r >> 2];
        s0 = (wj >> (8 * (r & 3))) & 0xffu ? s0 : -INFINITY;
        s1 = (wj >> (8 * ((r + 1) & 3))) & 0xffu ? s1 : -INFINITY;
      } else if constexpr (MASK == 2) {
        const uint32_t wj = mw[2 * (r >> 2) + ((r & 3) >> 1)];  // keys r, r + 1 share a word
        s0 += Num<T>::from_bits(wj & 0xffffu);
        s1 += Num<T>::from_bits(wj >> 16);
        round2<T>(s0, s1);
      }
      acc[r] = s0;
      acc[r + 1] = s1;
    }
  };
  // A half-block's state of the wavefront: skipped (no row sees a key), open or limited.
  auto half_open = [&](int blk, int hb) { return blk * kFusedBN + 32 * hb + 32 <= wave_min_lim; };
  auto half_live = [&](int blk, int hb) { return blk * kFusedBN + 32 * hb < wave_lim; };

  // ---------------------------------------------------------------- pass 1: m, l ----
  // Running maximum m (shared by both half-wavefronts of a row) and this half's sum l of
  // exp(s - m), rescaled when m grows; 32-key steps in order.
  float m = -INFINITY, l = 0.f;
  // base change of the exponentials (scores in units of round(S) under P2)
  const float kexp = P2 ? a.scale * kLog2e : kLog2e;
  auto stats = [&](const f32x16_t& sc) {
    float bm = sc[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) bm = fmaxf(bm, sc[r]);
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    // m = -inf until a visible key appears: the shift stays 0 and every term is exp(-inf) = 0
    const float mn = fmaxf(m, bm);
    const float sh = (mn == -INFINITY ? 0.f : mn) * kexp;
    const float corr = __builtin_amdgcn_exp2f(__builtin_fmaf(m, kexp, -sh));
    float part = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) part += __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], kexp, -sh));
    l = __builtin_fmaf(l, corr, part);
    m = mn;
  };
  if (nblk > 0) {
    load_k(0);
    store_k(0);
    __syncthreads();
  }
  for (int blk = 0; blk < nblk; ++blk) {
    if (blk + 1 < nblk) load_k(blk + 1);
    const int buf = blk & 1;
    if (half_open(blk, 1)) {
      // both halves open: the second S chain overlaps the first half's vector work
      uint32_t mw0[MW], mw1[MW];
      mask_words(blk, 0, mw0);
      mask_words(blk, 1, mw1);
      f32x16_t s0, s1;
      s_mfma2(buf, s0, s1);
      transform(std::true_type{}, blk, 0, s0, mw0);
      stats(s0);
      transform(std::true_type{}, blk, 1, s1, mw1);
      stats(s1);
    } else {
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        if (half_live(blk, hb)) {
          uint32_t mw[MW];
          mask_words(blk, hb, mw);
          f32x16_t sc;
          s_mfma(buf, hb, sc);
          if (half_open(blk, hb)) transform(std::true_type{}, blk, hb, sc, mw);
          else transform(std::false_type{}, blk, hb, sc, mw);
          stats(sc);
        }
      }
    }
    if (blk + 1 < nblk) store_k((blk + 1) & 1);
    __syncthreads();
  }
  const float lt = l + __shfl_xor(l, 32, 64);
  const bool dead = (m == -INFINITY) || (lt == 0.f);
  const float inv = dead ? 0.f : 1.0f / lt;
  const float shl2e = (m == -INFINITY ? 0.f : m) * kexp;

  // ---------------------------------------------------------------- pass 2: P V ----
  f32x16_t oacc[F::OF];
#pragma unroll
  for (int e = 0; e < F::OF; ++e)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[e][r] = 0.f;
  if (nblk > 0) {
    load_k(0);
    load_v(0);
    store_k(0);
    store_v(0);
    __syncthreads();
  }
  // V fragment source (transposing read): lane s of a 16-lane group points at row k0 + s/4,
  // column n0 + 4(s%4), and receives rows k0..k0+3 of column n0 + s.
  const int vrow = 4 * hf + ((lane & 15) >> 2);
  const int vcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  // P = round(exp(s - m) / l) of a half-block's two 16-key chunks, each straight into PV MFMAs.
  auto pv = [&](const f32x16_t& sc, int hb, const char* vb) {
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
      // 16-key chunk c = 2 hb + c2: this lane's keys 16c + 4hf + (0..3) and + 8
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[8 * c2 + e], kexp, -shl2e)) * inv;
      const u32x4_t pa = {pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3]), pack2<T>(p[4], p[5]),
                          pack2<T>(p[6], p[7])};
      const int row = 16 * (2 * hb + c2) + vrow;
#pragma unroll
      for (int e = 0; e < F::OF; ++e) {
        const u32x2_t lo = lds_read_tr16(vb + F::v_off(row, 32 * e + vcol));
        const u32x2_t hi = lds_read_tr16(vb + F::v_off(row + 8, 32 * e + vcol));
        const u32x4_t vf = {lo[0], lo[1], hi[0], hi[1]};
        Mfma<T>::step(oacc[e], pa, vf);
      }
    }
  };
  for (int blk = 0; blk < nblk; ++blk) {
    if (blk + 1 < nblk) {
      load_k(blk + 1);
      load_v(blk + 1);
    }
    const int buf = blk & 1;
    const char* vb = vbuf0 + buf * F::V_BYTES;
    if (half_open(blk, 1)) {
      uint32_t mw0[MW], mw1[MW];
      mask_words(blk, 0, mw0);
      mask_words(blk, 1, mw1);
      f32x16_t s0, s1;
      s_mfma(buf, 0, s0);
      s_mfma(buf, 1, s1);
      transform(std::true_type{}, blk, 0, s0, mw0);
      pv(s0, 0, vb);
      transform(std::true_type{}, blk, 1, s1, mw1);
      pv(s1, 1, vb);
    } else {
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        if (half_live(blk, hb)) {
          uint32_t mw[MW];
          mask_words(blk, hb, mw);
          f32x16_t sc;
          s_mfma(buf, hb, sc);
          if (half_open(blk, hb)) transform(std::true_type{}, blk, hb, sc, mw);
          else transform(std::false_type{}, blk, hb, sc, mw);
          pv(sc, hb, vb);
        }
      }
    }
    if (blk + 1 < nblk) {
      store_k((blk + 1) & 1);
      store_v((blk + 1) & 1);
    }
    __syncthreads();
  }

  // O rows 32w + 8(r/4) + 4hf + r%4, column 32e + l32.
#pragma unroll
  for (int e = 0; e < F::OF; ++e) {
    const int col = 32 * e + l32;
    if (col >= a.dv) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int orow = 32 * w + 8 * (r >> 2) + 4 * hf + (r & 3);
      if (orow < qrows) Num<T>::store(reinterpret_cast<T*>(g.out + E * (orow * a.soL)) + col, oacc[e][r]);
    }
  }
}

template <typename T, int DP, int DVP, int MASK, bool VARLEN>
static int launch_fused_t(const FusedArgs& a, hipStream_t s) {
  if (a.tiles > 0x7fffffffLL) return fail(BIOPS_ERR_SIZE, "too many attention tiles");
  constexpr bool kP2 = MASK != 2 && std::is_same<T, bf16_t>::value;
  if (kP2 && a.pow2)
    hipLaunchKernelGGL((fused_attn_kernel<T, DP, DVP, MASK, VARLEN, kP2>), dim3((unsigned)a.tiles), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((fused_attn_kernel<T, DP, DVP, MASK, VARLEN, false>), dim3((unsigned)a.tiles), dim3(256), 0, s, a);
  return check_launch("fused_attn_kernel");
}

template <typename T, int MASK, bool VARLEN>
static int launch_fused_d(const FusedArgs& a, hipStream_t s) {
  if constexpr (!VARLEN) {  // 256-wide heads: dense SDPA only (the varlen plan has 128-wide PV tiles)
    if (a.d > 128) {
      if (a.dv <= 128) return launch_fused_t<T, 256, 128, MASK, false>(a, s);
      return launch_fused_t<T, 256, 256, MASK, false>(a, s);
    }
    if (a.dv > 128) return launch_fused_t<T, 128, 256, MASK, false>(a, s);
  }
  if (a.d <= 64) {
    if (a.dv <= 64) return launch_fused_t<T, 64, 64, MASK, VARLEN>(a, s);
    return launch_fused_t<T, 64, 128, MASK, VARLEN>(a, s);
  }
  if (a.dv <= 64) return launch_fused_t<T, 128, 64, MASK, VARLEN>(a, s);
  return launch_fused_t<T, 128, 128, MASK, VARLEN>(a, s);
}

template <int MASK, bool VARLEN>
static int launch_fused(int dtype, const FusedArgs& a, hipStream_t s) {
  if (dtype == BIOPS_F16) return launch_fused_d<f16_t, MASK, VARLEN>(a, s);
  return launch_fused_d<bf16_t, MASK, VARLEN>(a, s);
}

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
// scale = 2^k with -8 <= k <= 0 (the fused kernels' exact power-of-two path); the environment
// variable BIOPS_ATTN_GENERIC_SCALE=1 turns the path off (tests compare the two).
static int pow2_scale(float scale) {
  int e = 0;
  if (!(scale > 0.f) || std::frexp(scale, &e) != 0.5f || e - 1 < -8 || e - 1 > 0) return 0;
  const char* env = std::getenv("BIOPS_ATTN_GENERIC_SCALE");
  return (env && env[0] == '1') ? 0 : 1;
}
static bool mult8(int64_t x) { return (x & 7) == 0; }
// Byte offsets inside one key block (64 rows) are 32-bit.
static bool block_fits(int64_t row_stride) { return row_stride >= 0 && 2 * kFusedBN * row_stride < (int64_t(1) << 31); }

}  // namespace biops

using namespace biops;

extern "C" int biops_attention_fused_supported(int dtype, int64_t d, int64_t dv) {
  return (dtype == BIOPS_BF16 || dtype == BIOPS_F16) && d >= 1 && d <= 256 && dv >= 1 &&
         dv <= 256 && mult8(d) && mult8(dv);
}

extern "C" int biops_varlen_fused_supported(int dtype, int64_t d, int64_t dv) {
  return biops_attention_fused_supported(dtype, d, dv) && d <= 128 && dv <= 128;
}

extern "C" int biops_attention_fused_mask_ok(const void* mask, int mask_dtype, int64_t lk, int64_t mB,
                                             int64_t mH, int64_t mI, int64_t mJ) {
  const int64_t align = mask_dtype == BIOPS_BOOL ? 4 : 8;  // bytes of four mask elements
  return mask != nullptr && mJ == 1 && lk % 4 == 0 && (reinterpret_cast<uintptr_t>(mask) % align) == 0 &&
         ((mB | mH | mI) & 3) == 0;
}

extern "C" int biops_sdpa_fused(int dtype, int64_t batch, int64_t hq, int64_t hkv, int64_t lq,
                                int64_t lk, int64_t d, int64_t dv, const void* q, int64_t sqB,
                                int64_t sqH, int64_t sqL, const void* k, int64_t skB, int64_t skH,
                                int64_t skL, const void* v, int64_t svB, int64_t svH, int64_t svL,
                                const void* mask, int mask_dtype, int64_t mB, int64_t mH, int64_t mI,
                                int64_t mJ, int causal, float scale, void* out, void* stream) {
  if (!biops_attention_fused_supported(dtype, d, dv))
    return fail(BIOPS_ERR_DTYPE, "fused attention takes bf16/fp16 with head dims <= 256, multiples of 8");
  if (batch < 0 || hq < 0 || hkv <= 0 || lq < 0 || lk < 0) return fail(BIOPS_ERR_ARG, "invalid attention sizes");
  if (hq % hkv != 0) return fail(BIOPS_ERR_ARG, "query heads must be a multiple of kv heads");
  if (mask && causal != BIOPS_CAUSAL_NONE) return fail(BIOPS_ERR_ARG, "mask and causal are exclusive");
  if (mask && mask_dtype != BIOPS_BOOL && mask_dtype != dtype)
    return fail(BIOPS_ERR_DTYPE, "mask dtype must be bool or the score dtype");
  if (batch == 0 || hq == 0 || lq == 0) return BIOPS_OK;
  if (mask && !biops_attention_fused_mask_ok(mask, mask_dtype, lk, mB, mH, mI, mJ))
    return fail(BIOPS_ERR_LAYOUT, "fused attention needs a mask with contiguous, aligned rows and keys % 4 == 0");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !mult8(sqB) || !mult8(sqH) || !mult8(sqL) ||
      !mult8(skB) || !mult8(skH) || !mult8(skL) || !mult8(svB) || !mult8(svH) || !mult8(svL))
    return fail(BIOPS_ERR_LAYOUT, "fused attention needs 16-byte aligned rows (strides multiples of 8)");
  if (!block_fits(skL) || !block_fits(svL) || !block_fits(sqL) || lq >= (int64_t(1) << 31) || lk >= (int64_t(1) << 31))
    return fail(BIOPS_ERR_LAYOUT, "fused attention row strides or lengths too large");
  FusedArgs a{};
  a.q = q; a.k = k; a.v = v; a.out = out; a.mask = mask; a.plan = nullptr; a.order = nullptr;
  a.hq = hq; a.group = hq / hkv; a.hkv = hkv; a.lq = lq; a.lk = lk; a.d = d; a.dv = dv;
  a.sqB = sqB; a.sqH = sqH; a.sqL = sqL; a.skB = skB; a.skH = skH; a.skL = skL;
  a.svB = svB; a.svH = svH; a.svL = svL;
  a.soB = hq * lq * dv; a.soH = lq * dv; a.soL = dv;
  a.mB = mB; a.mH = mH; a.mI = mI; a.mJ = mJ;
  a.tiles = batch * hq * cdiv(lq, kFusedBM);
  a.scale = scale;
  a.causal = causal;
  a.pow2 = pow2_scale(scale);
  hipStream_t s = (hipStream_t)stream;
  if (!mask) return launch_fused<0, false>(dtype, a, s);
  if (mask_dtype == BIOPS_BOOL) return launch_fused<1, false>(dtype, a, s);
  return launch_fused<2, false>(dtype, a, s);
}

extern "C" int64_t biops_varlen_fused_order(const int64_t* plan, int causal, int64_t* order) {
  if (!plan || !order || plan[0] < 0 || plan[5] < 0) {
    set_error("invalid varlen plan or order buffer");
    return -1;
  }
  struct Entry { int64_t keys, code; };
  std::vector<Entry> list;
  list.reserve((size_t)plan[5]);
  for (int64_t i = 0; i < plan[0]; ++i) {
    const int64_t* p = plan + kPlanHeader + kPlanStride * i;
    const int64_t ql = p[1], kl = p[3];
    const int64_t shift = causal == BIOPS_CAUSAL_BOTTOM_RIGHT ? kl - ql : 0;
    const int64_t qtiles = cdiv(ql, kFusedBM);
    for (int64_t qt = 0; qt < qtiles; ++qt) {
      int64_t keys = kl;
      if (causal != BIOPS_CAUSAL_NONE) {  // keys of the tile's last row (row_lim in the kernel)
        const int64_t last = (ql < (qt + 1) * kFusedBM ? ql : (qt + 1) * kFusedBM) - 1;
        keys = last + shift + 1;
        keys = keys < 0 ? 0 : (keys > kl ? kl : keys);
      }
      list.push_back({keys, (i << 32) | qt});
    }
  }
  if ((int64_t)list.size() != plan[5]) {
    set_error("varlen plan's query-tile count (word 5) does not match its items");
    return -1;
  }
  std::stable_sort(list.begin(), list.end(), [](const Entry& x, const Entry& y) { return x.keys > y.keys; });
  for (size_t k = 0; k < list.size(); ++k) order[k] = list[k].code;
  return (int64_t)list.size();
}

extern "C" int biops_varlen_sdpa_fused(int dtype, int64_t hq, int64_t hkv, int64_t d, int64_t dv,
                                       const void* q, int64_t sq_t, int64_t sq_h, const void* k,
                                       int64_t sk_t, int64_t sk_h, const void* v, int64_t sv_t,
                                       int64_t sv_h, void* out, int64_t so_t, int64_t so_h,
                                       const int64_t* dplan, const int64_t* hplan,
                                       const int64_t* dorder, int causal, float scale, void* stream) {
  if (!biops_varlen_fused_supported(dtype, d, dv))
    return fail(BIOPS_ERR_DTYPE, "fused varlen attention takes bf16/fp16 with head dims <= 128, multiples of 8");
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0) return fail(BIOPS_ERR_ARG, "invalid varlen head configuration");
  if (!dplan || !hplan || !dorder) return fail(BIOPS_ERR_ARG, "null plan or tile order");
  const int64_t items = hplan[0];
  if (items == 0) return BIOPS_OK;
  if (hplan[5] <= 0 || hplan[5] * hq != hplan[2])
    return fail(BIOPS_ERR_ARG, "plan without its query-tile count (word 5)");
  for (int64_t i = 0; i < items; ++i) {  // sequence lengths are 32-bit inside the kernel
    const int64_t* p = hplan + kPlanHeader + kPlanStride * i;
    if (p[1] >= (int64_t(1) << 31) || p[3] >= (int64_t(1) << 31))
      return fail(BIOPS_ERR_LAYOUT, "fused attention sequence longer than 2^31 tokens");
  }
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !mult8(sq_t) || !mult8(sq_h) ||
      !mult8(sk_t) || !mult8(sk_h) || !mult8(sv_t) || !mult8(sv_h))
    return fail(BIOPS_ERR_LAYOUT, "fused attention needs 16-byte aligned rows (strides multiples of 8)");
  if (!block_fits(sk_t) || !block_fits(sv_t) || !block_fits(sq_t))
    return fail(BIOPS_ERR_LAYOUT, "fused attention row strides too large");
  FusedArgs a{};
  a.q = q; a.k = k; a.v = v; a.out = out; a.mask = nullptr; a.plan = dplan; a.order = dorder;
  a.hq = hq; a.group = hq / hkv; a.hkv = hkv; a.d = d; a.dv = dv;
  a.sqL = sq_t; a.sqH = sq_h; a.skL = sk_t; a.skH = sk_h; a.svL = sv_t; a.svH = sv_h;
  a.soL = so_t; a.soH = so_h;
  a.items = items;
  a.tiles = hplan[5] * hq;  // one tile per head and 128-row query tile
  a.scale = scale;
  a.causal = causal;
  a.pow2 = pow2_scale(scale);
  return launch_fused<0, true>(dtype, a, (hipStream_t)stream);
}

// Zeros of rows t < rows, heads h < hq of a [rows, hq, dv] output of 2-byte elements with byte
// strides st_bytes, sh_bytes (unit stride inside a row); one thread per element.
__global__ __launch_bounds__(256) void zero_rows_kernel(char* out, int64_t rows, int64_t hq, int64_t st_bytes,
                                                        int64_t sh_bytes, int64_t row_bytes) {
  const int64_t per = row_bytes / 2;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * hq * per) return;
  const int64_t e = i % per, rh = i / per;
  *reinterpret_cast<uint16_t*>(out + (rh / hq) * st_bytes + (rh % hq) * sh_bytes + 2 * e) = 0;
}

extern "C" int biops_varlen_sdpa_fused_planned(int dtype, int64_t hq, int64_t hkv, int64_t d, int64_t dv,
                                               const void* q, int64_t sq_t, int64_t sq_h, const void* k,
                                               int64_t sk_t, int64_t sk_h, const void* v, int64_t sv_t,
                                               int64_t sv_h, void* out, int64_t so_t, int64_t so_h,
                                               int64_t total_q, int64_t total_kv, int64_t nseq, const int64_t* cu_q,
                                               const int64_t* cu_kv, int64_t* host_buf, int64_t host_words,
                                               int64_t* dev_buf, int causal, float scale, void* stream) {
  if (!biops_varlen_fused_supported(dtype, d, dv))
    return fail(BIOPS_ERR_DTYPE, "fused varlen attention takes bf16/fp16 with head dims <= 128, multiples of 8");
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0) return fail(BIOPS_ERR_ARG, "invalid varlen head configuration");
  if (total_q < 0 || total_kv < 0 || nseq < 0 || !cu_q || !cu_kv || !host_buf || !dev_buf || !out)
    return fail(BIOPS_ERR_ARG, "invalid varlen arguments");
  // the offsets' own rules (batch_invariant_ops.py:1264-1269); the planner rejects decreasing ones
  if (cu_q[0] != 0 || cu_kv[0] != 0) return fail(BIOPS_ERR_ARG, "cumulative sequence lengths must start at zero");
  if (cu_q[nseq] > total_q || cu_kv[nseq] > total_kv)
    return fail(BIOPS_ERR_ARG, "cumulative sequence lengths exceed packed tensor size");
  const int64_t words = biops_varlen_plan_len(nseq);
  if (words > host_words) return fail(BIOPS_ERR_SIZE, "work-list buffer of %lld words < %lld",
                                      (long long)host_words, (long long)words);
  if (biops_varlen_plan(nseq, cu_q, cu_kv, hq, dv, dtype, host_buf) < 0) return BIOPS_ERR_ARG;  // message set
  hipStream_t s = (hipStream_t)stream;
  // the kernel writes the rows of every sequence with keys; the rest (uncovered rows, sequences
  // without keys) read zero
  if (host_buf[3] != hq * total_q && total_q > 0 && dv > 0) {
    const int64_t n = total_q * hq * dv;  // 2-byte elements
    if (cdiv(n, 256) > 0x7fffffffLL) return fail(BIOPS_ERR_SIZE, "varlen output too large");
    hipLaunchKernelGGL(zero_rows_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, s, (char*)out, total_q, hq,
                       (int64_t)2 * so_t, (int64_t)2 * so_h, (int64_t)2 * dv);
    const int rc = check_launch("zero_rows_kernel");
    if (rc != BIOPS_OK) return rc;
  }
  if (host_buf[0] == 0) return BIOPS_OK;
  if (words + host_buf[5] > host_words) return fail(BIOPS_ERR_SIZE, "work-list buffer of %lld words < %lld",
                                                    (long long)host_words, (long long)(words + host_buf[5]));
  const int64_t n = biops_varlen_fused_order(host_buf, causal, host_buf + words);
  if (n < 0) return BIOPS_ERR_ARG;  // message set
  if (hipMemcpyAsync(dev_buf, host_buf, sizeof(int64_t) * (size_t)(words + n), hipMemcpyHostToDevice, s) != hipSuccess)
    return fail(BIOPS_ERR_HIP, "work-list upload failed");
  return biops_varlen_sdpa_fused(dtype, hq, hkv, d, dv, q, sq_t, sq_h, k, sk_t, sk_h, v, sv_t, sv_h, out, so_t, so_h,
                                 dev_buf, host_buf, dev_buf + words, causal, scale, stream);
}
