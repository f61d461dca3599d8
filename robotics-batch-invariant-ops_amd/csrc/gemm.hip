// Persistent fixed-schedule GEMM / batched GEMM entry points.
#include "gemm.h"

namespace biops {

// One persistent workgroup walks tiles t = slot, slot + G, ... over all batch elements.
// Epilogues: plain C = round(acc); bias C = round(acc + bias[n]) (bias added in fp32 before the
// single rounding); SwiGLU C = round(round(silu(round(g))) * round(u)) -- the roundings of
// F.silu(gate) * up applied to rounded bmm outputs -- where gate and up accumulators of one
// output sit in adjacent 32-column MFMA blocks of the same wavefront.
template <typename T, int BM, int BN, bool BKM, int EPI>
__global__ __launch_bounds__(kGemmThreads) void bmm_kernel(BmmArgs args) {
  using Tile = GemmTile<T, BM, BN, BKM>;
  __shared__ __attribute__((aligned(16))) char smem[Tile::LDS_BYTES];
  f32x16_t acc[Tile::FM][Tile::FN];

  const int64_t G = gridDim.x;
  const int64_t slot = xcd_slot(blockIdx.x, G);
  constexpr int64_t kCols = EPI == kEpiSwiglu ? BN / 2 : BN;
  const int64_t tpb = args.tiles_m * args.tiles_n;
  for (int64_t t = slot; t < args.total; t += G) {
    const int64_t b = t / tpb;
    int64_t tm, tn;
    tile_coords(t - b * tpb, args.tiles_m, args.tiles_n, tm, tn);
    const int64_t b1 = b / args.nb2;
    const int64_t b2 = b - b1 * args.nb2;
    const int64_t m0 = tm * BM, n0 = tn * kCols;

    const T* A = reinterpret_cast<const T*>(args.A) + b1 * args.sA1 + b2 * args.sA2 + m0 * args.lda;
    const int64_t boff = b1 * args.sB1 + (b2 / args.gB) * args.sB2 + (BKM ? n0 * args.ldb : n0);
    BSource<T> src;
    src.p0 = reinterpret_cast<const T*>(args.B) + boff;
    src.p1 = EPI == kEpiSwiglu ? reinterpret_cast<const T*>(args.B2) + boff : src.p0;
    src.ld = args.ldb;
    src.ncols = args.N - n0;
    src.swiglu = EPI == kEpiSwiglu;
    src.vec_ok = args.b_vec != 0;
    const int64_t rows = args.M - m0;
    const int64_t cols = args.N - n0;

    Tile::mainloop(smem, acc, A, args.lda, rows, args.a_vec != 0, src, args.K);

    T* C = reinterpret_cast<T*>(args.C) + b1 * args.sC1 + b2 * args.sC2 + m0 * args.ldc + n0;
    if constexpr (EPI == kEpiSwiglu) {
#pragma unroll
      for (int i = 0; i < Tile::FM; ++i)
#pragma unroll
        for (int j = 0; j < Tile::FN; j += 2) {
          const int c = Tile::acc_col(j);              // gate column in tile space
          const int col = ((c >> 6) << 5) + (c & 31);  // output column
          if (col >= cols) continue;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = Tile::acc_row(i, r);
            if (row < rows) {
              const float g = Num<T>::round(acc[i][j][r]);
              const float u = Num<T>::round(acc[i][j + 1][r]);
              const float s = Num<T>::round(g / (1.0f + expf(-g)));
              Num<T>::store(C + (int64_t)row * args.ldc + col, s * u);
            }
          }
        }
    } else {
      const T* bias = reinterpret_cast<const T*>(args.bias) + n0;
#pragma unroll
      for (int i = 0; i < Tile::FM; ++i)
#pragma unroll
        for (int j = 0; j < Tile::FN; ++j) {
          const int col = Tile::acc_col(j);
          if (col >= cols) continue;
          const float bv = EPI == kEpiBias ? Num<T>::load(bias + col) : 0.f;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = Tile::acc_row(i, r);
            if (row < rows) {
              float v = acc[i][j][r];
              if (EPI == kEpiBias) v += bv;
              Num<T>::store(C + (int64_t)row * args.ldc + col, v);
            }
          }
        }
    }
    // The next tile's prologue rewrites LDS stage 0: every wavefront finished reading LDS in
    // the last main-loop iteration, which ended with a barrier.
  }
}

// -------------------------------------------------------------- tile selection ----
// The block tile depends only on (dtype, N, K) and the epilogue, never on M or the batch.
struct TileChoice { int bm, bn; };

static TileChoice choose_tile(int dtype, int64_t N, int64_t K, int epi) {
  (void)dtype; (void)N; (void)K; (void)epi;
  return {128, 128};
}

template <typename T, int BM, int BN, bool BKM, int EPI>
static int launch_cfg(const BmmArgs& a0, hipStream_t stream) {
  using Tile = GemmTile<T, BM, BN, BKM>;
  BmmArgs a = a0;
  constexpr int64_t kCols = EPI == kEpiSwiglu ? BN / 2 : BN;
  a.tiles_m = cdiv(a.M, BM);
  a.tiles_n = cdiv(a.N, kCols);
  a.total = a.nb1 * a.nb2 * a.tiles_m * a.tiles_n;
  if (a.total == 0) return BIOPS_OK;
  const int cus = device_cus();
  if (cus <= 0) return fail(BIOPS_ERR_HIP, "no HIP device");
  const int per_cu = Tile::LDS_BYTES * 2 <= 160 * 1024 ? 2 : 1;
  int64_t grid = (int64_t)cus * per_cu;
  if (a.total < grid) grid = a.total;
  hipLaunchKernelGGL((bmm_kernel<T, BM, BN, BKM, EPI>), dim3((unsigned)grid), dim3(kGemmThreads),
                     0, stream, a);
  return check_launch("bmm_kernel");
}

template <typename T, int EPI>
static int launch_typed(const BmmArgs& a, bool b_kmajor, TileChoice tc, hipStream_t stream) {
  if (tc.bm == 128 && tc.bn == 128)
    return b_kmajor ? launch_cfg<T, 128, 128, true, EPI>(a, stream)
                    : launch_cfg<T, 128, 128, false, EPI>(a, stream);
  return fail(BIOPS_ERR_ARG, "no kernel for tile %dx%d", tc.bm, tc.bn);
}

template <int EPI>
static int launch_epi(int dtype, const BmmArgs& a, bool b_kmajor, TileChoice tc, hipStream_t s) {
  switch (dtype) {
    case BIOPS_F32: return launch_typed<float, EPI>(a, b_kmajor, tc, s);
    case BIOPS_F16: return launch_typed<f16_t, EPI>(a, b_kmajor, tc, s);
    case BIOPS_BF16: return launch_typed<bf16_t, EPI>(a, b_kmajor, tc, s);
    default: return fail(BIOPS_ERR_DTYPE, "unsupported GEMM dtype %d", dtype);
  }
}

static bool aligned16(const void* p, int64_t ld, int elt) {
  return (reinterpret_cast<uintptr_t>(p) % 16 == 0) && ((ld * elt) % 16 == 0);
}

int launch_bmm(int dtype, BmmArgs a, int epi, bool b_kmajor, hipStream_t stream) {
  const int elt = dtype_bytes(dtype);
  a.a_vec = aligned16(a.A, a.lda, elt) && (a.sA1 * elt) % 16 == 0 && (a.sA2 * elt) % 16 == 0;
  bool bv = aligned16(a.B, a.ldb, elt) && (a.sB1 * elt) % 16 == 0 && (a.sB2 * elt) % 16 == 0;
  if (epi == kEpiSwiglu) bv = bv && aligned16(a.B2, a.ldb, elt);
  a.b_vec = bv;
  if (a.gB <= 0) a.gB = 1;
  if (a.nb2 <= 0) a.nb2 = 1;
  const TileChoice tc = choose_tile(dtype, a.N, a.K, epi);
  switch (epi) {
    case kEpiBias: return launch_epi<kEpiBias>(dtype, a, b_kmajor, tc, stream);
    case kEpiSwiglu: return launch_epi<kEpiSwiglu>(dtype, a, b_kmajor, tc, stream);
    default: return launch_epi<kEpiPlain>(dtype, a, b_kmajor, tc, stream);
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
__global__ __launch_bounds__(kGemmThreads) void grouped_kernel(GroupedArgs a) {
  constexpr int BM = kVarlenBM, BN = kVarlenBN;
  constexpr bool BKM = MODE == kGroupQK;  // K^T is K-major, V is N-major
  using Tile = GemmTile<T, BM, BN, BKM>;
  __shared__ __attribute__((aligned(16))) char smem[Tile::LDS_BYTES];
  f32x16_t acc[Tile::FM][Tile::FN];
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

    Tile::mainloop(smem, acc, A, lda, rows, avec, src, K);

#pragma unroll
    for (int i = 0; i < Tile::FM; ++i)
#pragma unroll
      for (int j = 0; j < Tile::FN; ++j) {
        const int c = Tile::acc_col(j);
        if (c >= cols) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = Tile::acc_row(i, r);
          if (row < rows) Num<T>::store(C + (int64_t)row * ldc + c, acc[i][j][r]);
        }
      }
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
    hipLaunchKernelGGL((grouped_kernel<T, kGroupQK>), dim3((unsigned)grid), dim3(kGemmThreads), 0, s, a);
  else
    hipLaunchKernelGGL((grouped_kernel<T, kGroupPV>), dim3((unsigned)grid), dim3(kGemmThreads), 0, s, a);
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
