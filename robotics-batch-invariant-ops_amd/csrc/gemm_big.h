// Four-wavefront GEMM schedule (long K): BM x BN block on four wavefronts (2 x 2), each owning a
// (BM/2) x (BN/2) wave tile whose fp32 accumulators live in the accumulation registers (one
// wavefront per SIMD, 16 independent 32x32 accumulators at 256 x 256, one at 64 x 64).  Blocks
// from 256 x 256 down to 64 x 64; the ring takes as many stages as 160 KiB of LDS holds (2 at
// 256 x 256, 10 at 64 x 64), except that K-major 128 x 128 blocks keep 3 and 128 x 64 / 64 x 128
// / 64 x 64 blocks 4 (fewer in flight measured faster: same-box A/B in alternating order,
// 128 x 128 at M = 2048, N = 2048, K = 8192 63.8 -> 62.4 us, 512 x 8192 x 2048 22.0 -> 21.2 us;
// 64 x 128 at 256 x 8192 x 2048 16.0 -> 15.2 us, 1024 x 2048 x 8192 43.8 -> 43.3 us; 128 x 64
// at 512 x 8192 x 2048 28.2 -> 27.3 us; 64 x 64 at 128 x 8192 x 2048 12.1 -> 11.2 us; two stages
// are slower everywhere).
//
// Same arithmetic as every other tile entry (gemm_core.h): 128-byte K steps in order, chunk
// pairs q = 0..3 in order inside a step.  A stage of the LDS ring holds one K step (SB = 128
// bytes per row; 64 KiB at 256 x 256).  Measured on MI355X (bf16, M = 4096, N = 8192,
// K = 2048): half-step stages (deeper ring, 64-byte requests) and register-staged loads were
// both slower than this schedule.
//
// Stage h (ring slot h % STAGES) holds P = 4 chunk pairs.  Per stage, per wavefront:
//   group p (p = 0 .. P-2): the MFMAs of pair p, interleaved with the LDS reads of pair p+1;
//   group P-1: wait for stage h+1 and barrier (publishes h+1; all of stage h has been read),
//   read pair 0 of stage h+1, then the MFMAs of pair P-1 with the global->LDS loads that
//   refill slot h with stage h+STAGES interleaved (one per MFMA at 256 x 256, several per MFMA
//   in the smaller blocks).
// The compiler waits for all outstanding LDS reads before an MFMA that needs one (the global
// -> LDS loads make its LDS counter out of order), so each group starts with one wait and its
// MFMAs only read fragments loaded during the previous group.
// K-major blocks from 128 x 128 up take two pairs per group instead (group A: pairs 0, 1 with
// the reads of pairs 2, 3; group B: wait, barrier, the reads of pairs 0, 1 of stage h+1, pairs
// 2, 3 with the refill, part of it after pair 2's reads where MFMAs of pair 2 remain there),
// so that a read has two pairs of MFMAs to land, not one.  Measured on
// MI355X (same-box A/B, the two kernels timed in alternating order, bitwise-identical outputs):
// 256 x 256 at M = 4096, N = 8192, K = 2048 114.5 -> 113.0 us and K = 8192 378.2 -> 373.8 us;
// 256 x 128 at 4096 x 2048 x 8192 110.1 -> 107.5 us; 128 x 128 at 2048 x 2048 x 8192
// 63.8 -> 62.6 us; 128 x 256 at 2048 x 8192 x 2048 70.1 -> 69.0 us.
//
// LDS stage layout: A rows (BM x 128 bytes) then B columns (BN x 128 bytes).  A 16-byte read
// serves 16 lanes per clock from a 256-byte window, so 16 consecutive rows reading the same
// chunk must land in 16 distinct 16-byte slots: chunk c of row r sits at slot c ^ ((r >> 1) & 7).
#pragma once

#include "gemm_core.h"

namespace biops {

// BKM: B K-major (an nn.Linear weight, [N, K] rows); otherwise N-major (row-major [K, N], N a
// multiple of 8): a stage then holds 64 K rows of BN columns in the N-major layout of the table
// entries (lds_off_n) and the B fragments come through the transposing LDS reads.
template <typename T, int BM, int BN, int SB, bool BKM = true>
struct BigTile {
  static_assert(sizeof(T) == 2, "16-bit operands");
  static_assert(BKM || BN >= 64, "N-major stage rows of at least 8 chunks");
  static_assert(SB == 128, "whole K step per stage");
  static constexpr int THREADS = 256;
  static constexpr int WM = BM / 2, WN = BN / 2;
  static constexpr int FM = WM / 32, FN = WN / 32;
  static constexpr int NM = FM * FN;              // MFMAs per chunk pair
  static constexpr int VEC = 8;
  static constexpr int CPR = SB / 16;             // 16-byte chunks per row of a stage
  static constexpr int P = CPR / 2;               // chunk pairs per stage
  static constexpr int STAGE_ELEMS = SB / 2;      // K elements per stage
  static constexpr int LDS_A = BM * SB;
  static constexpr int LDS_STAGE = (BM + BN) * SB;
  static constexpr int LDS_MAX = 160 * 1024;
  static constexpr int MAX_STAGES = LDS_MAX / LDS_STAGE;
  static constexpr int STAGES = !BKM ? MAX_STAGES
                                : BM * BN == 128 * 128 ? 3
                                : BM * BN == 128 * 64 || BM * BN == 64 * 64 ? 4
                                : MAX_STAGES;
  static constexpr int RING = STAGES * LDS_STAGE;
  static constexpr int SMEM_BYTES = RING;
  static constexpr int A_LOADS = BM * CPR / THREADS;  // 16-byte chunks per thread per stage
  static constexpr int B_LOADS = BN * CPR / THREADS;
  static constexpr int LOADS = A_LOADS + B_LOADS;
  static constexpr int CPR_N = BN / 8;            // 16-byte chunks per K row of an N-major stage
  static_assert(STAGES >= 2, "ring");
  static_assert((STAGES - 1) * LOADS < 64, "vmcnt range");
  static_assert(SMEM_BYTES <= LDS_MAX, "LDS");
  typedef f32x16_t Acc;

  struct Frags {
    u32x4_t a[FM];
    u32x4_t b[FN];
    u32x2_t lo[FN], hi[FN];  // N-major: the two transposing-read halves of b
  };

  __device__ static __forceinline__ int off(int r, int c) { return (r << 7) + ((c ^ ((r >> 1) & 7)) << 4); }

  template <int N>
  __device__ static __forceinline__ void wait_loads() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  }
  // Through the builtins rather than inline assembly: the compiler then knows that every LDS
  // read has landed at the barrier.  With the wait hidden in assembly it still counted the
  // previous group's reads as pending and, once a global->LDS load had been issued after the
  // barrier, waited for all LDS reads (the next stage's fragments included) before the second
  // MFMA of the group.  Measured on MI355X (bf16, bitwise-identical outputs), together with the
  // front-loaded reads of interleave(): 128x64 blocks at M=1024, N=2048, K=8192 53 -> 47 us,
  // 128x128 at 2048x2048x8192 75 -> 68 us, 256x128 at 4096x2048x8192 -3 %, 256x256 -1.5 %.
  __device__ static __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");  // no memory access moves across the barrier (compiler fence)
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0), vmcnt unchanged
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }

  // Chunk pair p of the stage at `stage` for this wavefront's blocks.
  __device__ static __forceinline__ void read_frags(const char* stage, int p, Frags& f) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int wm = w >> 1, wn = w & 1;
    const int lr = lane & 31, c = 2 * p + (lane >> 5);
#pragma unroll
    for (int i = 0; i < FM; ++i)
      f.a[i] = *reinterpret_cast<const u32x4_t*>(stage + off(wm * WM + i * 32 + lr, c));
    if constexpr (BKM) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
        f.b[j] = *reinterpret_cast<const u32x4_t*>(stage + LDS_A + off(wn * WN + j * 32 + lr, c));
    } else {
      // lane group g = lane / 16: columns 16 (g & 1) .. +15 of a 32-column block, K half g >> 1
      // (the K values of chunk 2p + (lane >> 5), as on the K-major side); the reads are inline
      // assembly, so that the compiler does not drain the global->LDS loads in flight before
      // them, and ready() waits for them.
      const int g = lane >> 4, s = lane & 15;
      const int k = 16 * p + 8 * (g >> 1) + (s >> 2);
      const int cb = 16 * (g & 1) + 4 * (s & 3);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const char* base = stage + LDS_A;
        const int col = wn * WN + j * 32 + cb;
        f.lo[j] = lds_read_tr16_asm(base + lds_off_n<CPR_N>(k, col));
        f.hi[j] = lds_read_tr16_asm(base + lds_off_n<CPR_N>(k + 4, col));
      }
    }
  }
  // N-major: wait for the transposing reads of f and assemble the B fragments (no-op K-major).
  __device__ static __forceinline__ void ready(Frags& f) {
    if constexpr (!BKM) {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        lds_wait_anchor(f.lo[j], f.hi[j]);
        f.b[j] = u32x4_t{f.lo[j][0], f.lo[j][1], f.hi[j][0], f.hi[j][1]};
      }
    }
  }

  __device__ static __forceinline__ void mfmas(Acc (&acc)[FM][FN], const Frags& f) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) Mfma<T>::step(acc[i][j], f.a[i], f.b[j]);
  }

  // Interleave the group's MFMAs with its LDS reads: two reads after each of the group's first
  // MFMAs, then the remaining MFMAs, so that the reads have most of the group to land before
  // the next group waits for them (one read per two MFMAs left the last reads two MFMAs before
  // that wait).
  __device__ static __forceinline__ void interleave() {
    if constexpr (!BKM) return;  // inline-assembly reads are not scheduling units
    constexpr int NR = FM + FN;
    constexpr int NG = (NR + 1) / 2;  // MFMAs followed by reads; NG <= NM for FM, FN >= 1
#pragma unroll
    for (int i = 0; i < NR / 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
    }
    if constexpr (NR % 2 != 0) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (NM > NG) __builtin_amdgcn_sched_group_barrier(0x008, NM - NG, 0);
  }

  // Direct-load sources of this thread.  Slot s = t + 256p of a stage is row s / 8 of the A
  // rows (p < A_LOADS) or of the B columns, i.e. row r0 + 32p (r0 = t / 8), holding logical
  // chunk (t % 8) ^ ((r0 >> 1) & 7) -- the same chunk for every p, 32 being a multiple of 16.
  // Rows past the valid ones re-load the last valid row (their products are never stored).
  // N-major B: slot s = t + 256 q of the B part is K row s / CPR_N, physical chunk
  // t % CPR_N, i.e. K row k0 + (256 / CPR_N) q (k0 = t / CPR_N) holding logical chunk
  // (t % CPR_N) ^ swz(k0) -- the same for every q (256 / CPR_N is a multiple of the swizzle's
  // period); chunks past the tile's valid columns re-load its last whole chunk (N is a
  // multiple of 8; their products are never stored).
  struct Src {
    const T* a;
    const T* b;
    int64_t lda, ldb;
    int rows, cols, r0;
  };
  __device__ static __forceinline__ Src make_src(const T* A, int64_t lda, int rows, const T* B, int64_t ldb,
                                                 int cols) {
    const int t = threadIdx.x;
    const int r0 = t >> 3;
    const int c = (t & 7) ^ ((r0 >> 1) & 7);
    if constexpr (BKM) {
      return Src{A + c * VEC, B + c * VEC, lda, ldb, rows, cols, r0};
    } else {
      const int k0 = t / CPR_N;
      int col = VEC * ((t % CPR_N) ^ nmajor_swz<CPR_N>(k0));
      if (col >= cols) col = cols - VEC;
      return Src{A + c * VEC, B + (int64_t)k0 * ldb + col, lda, ldb, rows, cols, r0};
    }
  }
  // Load p of this thread for the stage at K element k into ring slot `slot`.
  __device__ static __forceinline__ void issue_one(char* smem, const Src& src, int slot, int64_t k, int p) {
    // Wave-uniform by construction; read from lane 0 so that the LDS destination (M0) is scalar
    // arithmetic instead of a vector value moved to a scalar register for every load (128x64
    // blocks at M=1024, N=2048, K=8192: 47.7 -> 44.6 us in a same-box A/B, same bits).
    const int wbase = __builtin_amdgcn_readfirstlane(threadIdx.x & ~63);
    const T* ptr;  // this load's 16 source bytes
    if (p < A_LOADS) {
      const int r = src.r0 + 32 * p;
      ptr = src.a + (int64_t)(r < src.rows ? r : src.rows - 1) * src.lda + k;
    } else if constexpr (BKM) {
      const int r = src.r0 + 32 * (p - A_LOADS);
      ptr = src.b + (int64_t)(r < src.cols ? r : src.cols - 1) * src.ldb + k;
    } else {
      ptr = src.b + (k + (int64_t)(THREADS / CPR_N) * (p - A_LOADS)) * src.ldb;  // K rows from k
    }
    __builtin_amdgcn_global_load_lds((global_cvoid_t*)ptr,
                                     (lds_void_t*)(smem + slot * LDS_STAGE + (THREADS * p + wbase) * 16), 16, 0, 0);
  }
  // The MFMAs of one pair with loads [P0, P1) of a stage interleaved: MFMA q is followed by
  // loads P0 + [q * n / NM, (q + 1) * n / NM), n = P1 - P0.  A burst of loads ahead of the
  // MFMAs (each load sets M0 and its address first) leaves the MFMA pipe idle: interleaving
  // measured -4 % at 256 x 256, M = 4096, N = 8192, K = 2048 and 8192.
  template <int P0, int P1>
  __device__ static __forceinline__ void mfmas_loads(Acc (&acc)[FM][FN], const Frags& f, char* smem,
                                                     const Src& src, int slot, int64_t k) {
    constexpr int n = P1 - P0;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        Mfma<T>::step(acc[i][j], f.a[i], f.b[j]);
        const int q = i * FN + j;
#pragma unroll
        for (int p = P0 + q * n / NM; p < P0 + (q + 1) * n / NM; ++p) issue_one(smem, src, slot, k, p);
      }
    sched_loads<0, n>();
  }
  // Schedule of NMF MFMAs, each followed by its share of n loads.
  template <int Q, int n, int NMF = NM>
  __device__ static __forceinline__ void sched_loads() {
    if constexpr (Q < NMF) {
      constexpr int c = (Q + 1) * n / NMF - Q * n / NMF;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                    // MFMA
      if constexpr (c > 0) __builtin_amdgcn_sched_group_barrier(0x020, c, 0);  // VMEM
      sched_loads<Q + 1, n, NMF>();
    }
  }

  // Two pairs per group when a group's reads fit after the first pair's first MFMAs (two reads
  // after each).
  static constexpr bool TWO_PAIR = BKM && (FM + FN) <= NM;
  // Refill loads of a stage that go with the MFMAs of pair 2 after its reads (FM + FN MFMAs
  // carry the reads): one per remaining MFMA, at most half the loads; the rest go with pair 3.
  // Measured on MI355X (same-box A/B, alternating order, bitwise-equal outputs): 256 x 256 (8
  // of 16 loads) at M = 4096, N = 8192, K = 2048 121.5 -> 119.0 us, 8192^3 845.5 -> 818.6 us;
  // 256 x 128 (2 of 12) at 4096 x 2048 x 8192 122.2 -> 120.4 us.  128 x 128 blocks have no MFMA
  // of pair 2 left after its reads and keep every load with pair 3 (all 8 after pair 2's
  // MFMAs measured slower there: 2048 x 2048 x 8192 69.4 -> 71.6 us).
  static constexpr int LOADS_P2 = NM - (FM + FN) < LOADS / 2 ? NM - (FM + FN) : LOADS / 2;
  struct Frags2 {
    Frags f[2];
  };
  __device__ static __forceinline__ void read2(const char* stage, int p0, Frags2& g) {
    read_frags(stage, p0, g.f[0]);
    read_frags(stage, p0 + 1, g.f[1]);
  }
  // The 2 (FM + FN) reads of a group, two after each of its first MFMAs, then the rest of the
  // MFMAS MFMAs this pattern covers.
  template <int MFMAS>
  __device__ static __forceinline__ void interleave2() {
    constexpr int NR = 2 * (FM + FN);
    static_assert(NR / 2 <= MFMAS, "reads after the MFMAs");
#pragma unroll
    for (int i = 0; i < NR / 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
    }
    if constexpr (MFMAS > NR / 2) __builtin_amdgcn_sched_group_barrier(0x008, MFMAS - NR / 2, 0);
  }
  __device__ static __forceinline__ void mainloop_two_pair(char* smem, Acc (&acc)[FM][FN], const Src& src,
                                                           int64_t H) {
    auto stage_k = [&](int64_t h) { return (h < H ? h : H - 1) * STAGE_ELEMS; };
    Frags2 F[2];
    read2(smem, 0, F[0]);
    int cur = 0;
    for (int64_t h = 0; h < H; ++h) {
      const char* st = smem + cur * LDS_STAGE;
      const int nxt = cur + 1 == STAGES ? 0 : cur + 1;
      // group A: pairs 0, 1 (read during the previous group B) with the reads of pairs 2, 3
      read2(st, 2, F[1]);
      mfmas(acc, F[0].f[0]);
      mfmas(acc, F[0].f[1]);
      interleave2<2 * NM>();
      __builtin_amdgcn_sched_barrier(0);
      // group B: stage h+1 landed and published (all of stage h has been read), its pairs 0, 1
      // read, then pairs 2, 3 with the refill of slot h by stage h+STAGES
      wait_loads<(STAGES - 2) * LOADS>();
      lds_barrier();
      read2(smem + nxt * LDS_STAGE, 0, F[0]);
      mfmas(acc, F[1].f[0]);
#pragma unroll
      for (int p = 0; p < LOADS_P2; ++p) issue_one(smem, src, cur, stage_k(h + STAGES), p);
      interleave2<FM + FN>();
      sched_loads<0, LOADS_P2, NM - (FM + FN)>();
      __builtin_amdgcn_sched_barrier(0);
      mfmas_loads<LOADS_P2, LOADS>(acc, F[1].f[1], smem, src, cur, stage_k(h + STAGES));
      __builtin_amdgcn_sched_barrier(0);
      cur = nxt;
    }
    wait_loads<0>();
    lds_barrier();  // the ring is idle
  }

  // Full K loop of one tile into acc (zeroed here).  A: tile rows (rows valid), B: tile
  // columns (cols valid; K-major rows, or N-major from the tile's first column), K a whole
  // number of 128-byte steps.
  __device__ static __forceinline__ void mainloop(char* smem, Acc (&acc)[FM][FN], const T* A, int64_t lda,
                                                  int rows, const T* B, int64_t ldb, int cols, int64_t K) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    const int64_t H = K / STAGE_ELEMS;  // stages
    if (H == 0) return;
    const Src src = make_src(A, lda, rows, B, ldb, cols);
    // Stages past the end re-load the last one (into a slot nobody reads again), so every
    // iteration issues the same loads and the vmcnt waits are constants.
    auto stage_k = [&](int64_t h) { return (h < H ? h : H - 1) * STAGE_ELEMS; };
#pragma unroll
    for (int s = 0; s < STAGES; ++s)
#pragma unroll
      for (int p = 0; p < LOADS; ++p) issue_one(smem, src, s, stage_k(s), p);
    wait_loads<(STAGES - 1) * LOADS>();  // stage 0 landed
    lds_barrier();
    if constexpr (TWO_PAIR) {
      mainloop_two_pair(smem, acc, src, H);
      return;
    }
    Frags f[2];
    read_frags(smem, 0, f[0]);
    int cur = 0;  // ring slot of stage h
    for (int64_t h = 0; h < H; ++h) {
      const char* st = smem + cur * LDS_STAGE;
      const int nxt = cur + 1 == STAGES ? 0 : cur + 1;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        Frags& use = f[p & 1];
        Frags& next = f[(p + 1) & 1];
        ready(use);
        if (p + 1 < P) {
          read_frags(st, p + 1, next);
          mfmas(acc, use);
          interleave();
          __builtin_amdgcn_sched_barrier(0);
        } else {
          // Stage h+1 landed once the STAGES-2 stages issued after it remain in flight.  The
          // barrier publishes it; every wavefront has read all of stage h, whose slot takes
          // stage h+STAGES.  The next stage's first fragments are read before the loads are
          // issued (a read after a global->LDS load may not move above it).
          wait_loads<(STAGES - 2) * LOADS>();
          lds_barrier();
          read_frags(smem + nxt * LDS_STAGE, 0, next);
          mfmas_loads<0, LOADS>(acc, use, smem, src, cur, stage_k(h + STAGES));
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      cur = nxt;
    }
    wait_loads<0>();
    lds_barrier();  // the ring is idle
  }

  __device__ static __forceinline__ int acc_row(int i, int r) {
    const int lane = threadIdx.x & 63;
    const int wm = (threadIdx.x >> 6) >> 1;
    return wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
  }
  __device__ static __forceinline__ int acc_col(int j) {
    const int lane = threadIdx.x & 63;
    const int wn = (threadIdx.x >> 6) & 1;
    return wn * WN + j * 32 + (lane & 31);
  }

  // round(acc (+ bias[col])) stored straight from the accumulators, one 16-bit store per value
  // (measured on MI355X against staging the tile through LDS for 16-byte stores: -7 us per
  // launch at M = 4096, N = 8192, K = 128 and -4 us at K = 2048, the LDS writes of 256 values
  // per lane being the slower part).  Offsets inside the tile are 32-bit (the launcher
  // requires BM * ldc < 2^31); the opaque copy of ldc keeps the compiler from holding all
  // row offsets in registers.  A whole tile stores without per-value bounds checks: the 256
  // branches of the checked form cost 6-8 us per launch at M = 4096, N = 8192 (MI355X).
  // NT: non-temporal stores (whole tiles of a launch that fills one round of the compute units;
  // see epilogue()).
  template <bool CHECKED, bool NT = false>
  __device__ static __forceinline__ void store_tile(Acc (&acc)[FM][FN], T* C, int ldc32, int rows, int cols,
                                                    const T* bias) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = acc_col(j);
        const bool col_ok = !CHECKED || col < cols;
        const float bv = (bias && col_ok) ? Num<T>::load(bias + col) : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = acc_row(i, r);
          if (!CHECKED || (col_ok && row < rows)) {
            const float v = bias ? acc[i][j][r] + bv : acc[i][j][r];
            T* p = C + (uint32_t)(row * ldc32 + col);
            if constexpr (NT)
              __builtin_nontemporal_store(Num<T>::to_bits(v), reinterpret_cast<uint16_t*>(p));
            else
              Num<T>::store(p, v);
          }
        }
      }
  }
  // With `nt` (set by the launcher when the launch's tiles fit one round of the compute units)
  // whole tiles store non-temporally.  Measured on MI355X (bf16, same-box A/B, same bits):
  // one-round launches 512 / 1024 / 2048 x 8192 x 2048 25.2 -> 23.9, 39.3 -> 37.3,
  // 62.6 -> 60.8 us and 2048 x 2048 x 8192 70.2 -> 68.9 us; launches of several rounds slower
  // (4096 x 8192 x 2048 120.2 -> 126.9 us), so they keep ordinary stores.
  __device__ static __forceinline__ void epilogue(Acc (&acc)[FM][FN], T* C, int64_t ldc, int rows, int cols,
                                                  const T* bias, bool nt) {
    int ldc32 = (int)ldc;
    asm volatile("" : "+s"(ldc32));
    if (rows == BM && cols == BN) {
      if (nt)
        store_tile<false, true>(acc, C, ldc32, rows, cols, bias);
      else
        store_tile<false>(acc, C, ldc32, rows, cols, bias);
    } else {
      store_tile<true>(acc, C, ldc32, rows, cols, bias);
    }
  }
};

}  // namespace biops
