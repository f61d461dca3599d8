// Weight-streaming tile for grouped GEMMs whose groups have few rows and whose B is a 16-bit
// N-major matrix per group (the expert GEMMs of few-token MoE calls: at one token a route's
// gate/up GEMM is one x row against 2048 x 1536 weights).
//
// Such a launch reads each expert's weights once and does next to no arithmetic, so its time
// is the weight stream.  On MI355X that stream is bounded by the number of distinct memory
// segments, not by the loads in flight: reading 8 experts' [2048, 1536] weights with blocks
// of 32 gate + 32 up columns (64-byte row segments) takes 14.7 us whatever the load depth, with
// 64 + 64 columns (128-byte segments) 8.9 us (13.6 us from HBM with a cold MALL).  This tile
// therefore owns 64 output columns of one m-tile: in SwiGLU mode 64 gate and 64 up columns,
// whole 128-byte segments of every K row.
//
// Arithmetic: v_mfma_f32_16x16x32 on 16-row x 16-column blocks, quad q' of a 128-byte K step
// feeding chunks 4q'..4q'+3 (the chain of the skinny entry, gemm_skinny.h, whose bits equal
// those of the two 32x32x16 pair steps of every other entry), K in order, no split.  Plain:
// four wavefronts, wavefront w owns output columns 16w..16w+15.  Plain WIDE (the launcher
// takes it for 64-row m-tiles): eight wavefronts over 128 output columns in two 64-column
// halves, loaded and read as the SwiGLU mode's gate and up halves; half the workgroups, and
// each A row read by half as many (MI355X, same-box A/B, same bits, per C5 MoE call: 256
// tokens, the down GEMM on 64-row m-tiles, 155.0 -> 140.6 us, 4096 tokens (its tails)
// 478.1 -> 469.4 us; with 32-row m-tiles it measured slower, 32 tokens 123.9 -> 127.1 us,
// with 16-row ones even at one to four tokens).  SwiGLU: eight wavefronts,
// wavefront w owns the gate (w < 4) or up (w >= 4) columns 16(w%4)..+15, which halves each
// wavefront's work per stage (one-token gate/up GEMM of 8 experts: 14.7 -> 11.8 us); after the
// K loop the up wavefronts pass their accumulators through LDS to the gate wavefront of the
// same columns.  The store rounds straight from the accumulators as the LDS-staged epilogues do.
//
// Operands go global -> LDS by global_load_lds_dwordx4 into a ring of 128-element K stages;
// all wavefronts load and compute (64-element stages and a 3-stage ring were measured slower
// for the gate/up GEMM: 16.6 and 16.5 us against 15.4 us before the batched reads).  A stage
// holds BM rows of A (K-major, 256 bytes each, chunk c of row r in slot c ^ (r & 15)) and 128 K
// rows of B (N-major, the block's chunks of 8 columns, gate then up, chunk pairs swizzled by K
// row), read back with ds_read_b128 (A) and the transposing ds_read_b64_tr_b16 (B).
//
// Requirements (checked by the launcher): 16-bit types, grouped rows, N-major B with 16-byte
// aligned rows and N a multiple of 8, K a multiple of 64.
#pragma once

#include "gemm_core.h"
#include "gemm_skinny.h"

namespace biops {

template <typename T, int BM, bool SWIGLU, bool WIDE = false>
struct StreamTile {
  static_assert(sizeof(T) == 2, "16-bit operands");
  static_assert(BM == 16 || BM == 32 || BM == 64, "m-tile rows");
  static_assert(!(SWIGLU && WIDE), "one mode");
  static constexpr bool TWO = SWIGLU || WIDE;             // two 64-column halves of B per block
  static constexpr int THREADS = TWO ? 512 : 256;
  static constexpr int OUT = 64;                          // output columns of a half
  static constexpr int BLOCK_OUT = WIDE ? 2 * OUT : OUT;  // output columns of a block
  static constexpr int CPR = (TWO ? 2 : 1) * OUT / 8;     // 16-byte chunks of a B K row (8 / 16)
  static constexpr int SK = 128;                          // K elements of a stage
  static constexpr int STEPS = SK / 64;                   // 128-byte K steps of a stage
  static constexpr int RB = BM / 16;                      // 16-row MFMA blocks
  static constexpr int A_ROW = SK * 2;                    // bytes of one A row in a stage
  // A slots of a stage; with fewer slots than threads the other threads load a copy of them
  // into a spare area, so that every thread issues the same loads (constant vmcnt waits).
  static constexpr int A_SLOTS = BM * (A_ROW / 16);
  static constexpr int A_SPARE = A_SLOTS < THREADS ? (THREADS - A_SLOTS) * 16 : 0;
  static constexpr int LDS_A = BM * A_ROW + A_SPARE;
  static constexpr int LDS_B = SK * CPR * 16;
  static constexpr int LDS_STAGE = LDS_A + LDS_B;
  // SwiGLU: as deep as 160 KiB allows (4 stages; 3 with 64-row m-tiles).  Plain: at most 4
  // stages within 80 KiB, so that two workgroups share a compute unit (the down GEMM of 64
  // one-row groups, K = 768, took 48.5 us with an 8-stage ring and 31.0 us with 4, of 8 groups
  // 6.4 and 5.6 us, MI355X); with 64-row m-tiles, whose stages are twice as large, 4 stages in
  // 160 KiB.
  static constexpr int STAGES_FIT = (TWO || BM == 64 ? 160 * 1024 : 80 * 1024) / LDS_STAGE;
  static constexpr int STAGES = STAGES_FIT < (TWO ? 8 : 4) ? STAGES_FIT : (TWO ? 8 : 4);
  static constexpr int LDS_BYTES = STAGES * LDS_STAGE;
  static constexpr int A_LOADS = A_SLOTS < THREADS ? 1 : A_SLOTS / THREADS;  // per thread and stage
  static constexpr int B_LOADS = SK * CPR / THREADS;
  static constexpr int LOADS = A_LOADS + B_LOADS;
  static_assert((A_SLOTS < THREADS || A_LOADS * THREADS == A_SLOTS) && B_LOADS * THREADS == SK * CPR,
                "load split");
  static_assert(STAGES >= 3 && (STAGES - 1) * LOADS < 64, "ring depth and vmcnt range");

  // Chunk-pair swizzle of B K row k: the 16 rows one transposing read covers (k0 + 8g + i,
  // g, i = 0..3) land on distinct 32-byte bank slots up to a factor two.
  __device__ static __forceinline__ int bswz(int k) {
    if constexpr (CPR == 16) return 2 * ((k & 3) | (((k >> 3) & 1) << 2));
    else return 2 * (((k >> 1) & 1) | (((k >> 3) & 1) << 1));
  }
  __device__ static __forceinline__ int a_off(int r, int c) { return r * A_ROW + ((c ^ (r & 15)) << 4); }
  __device__ static __forceinline__ int b_off(int k, int col) {
    return LDS_A + k * (CPR * 16) + ((((col >> 3) ^ bswz(k))) << 4) + ((col & 7) << 1);
  }

  template <int N>
  __device__ static __forceinline__ void wait_loads() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  }
  __device__ static __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0), vmcnt unchanged
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }

  struct Acc {
    f32x4_t g[RB];  // plain: the output; SwiGLU: gate
    f32x4_t u[RB];  // SwiGLU: up
  };

  // Operand sources of one block.  a_row(r): A row of m-tile row r (r < rows); B: gate / plain
  // columns at bg + n, up columns at bu + n (N-major, K row k at + k * ldb), n < ncols; WIDE:
  // the block's columns OUT + n at bu + n (bu = bg + OUT), valid for n < ncols - OUT.
  struct Sources {
    const T* A;
    int64_t lda;
    const int32_t* a_rows;  // row table (nullptr: row m0 + r)
    int64_t m0;
    int rows;
    const T* bg;
    const T* bu;
    int64_t ldb;
    int64_t ncols;  // valid columns from the block origin
    int64_t K;
  };

  // The block over K (a multiple of 64).  Every wavefront returns its accumulators (SwiGLU:
  // the gate wavefronts return gate and up of their columns).
  __device__ static __forceinline__ Acc run(char* smem, const Sources& S) {
    Acc acc;
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      acc.g[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      acc.u[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    const int64_t KT = S.K / 64;  // 128-byte K steps
    if (KT == 0) return acc;
    const int64_t NS = (KT + STEPS - 1) / STEPS;
    const int t = threadIdx.x;
    const int wbase = __builtin_amdgcn_readfirstlane(t & ~63);  // wave-uniform LDS offsets

    // This thread's sources at K = 0.  A slot s = (t + THREADS p) % A_SLOTS: row s / 16, slot
    // s % 16 holding logical chunk (s % 16) ^ (row & 15).  B slot s = t + THREADS p: K row
    // s / CPR, slot s % CPR holding logical chunk (s % CPR) ^ bswz(row); chunks past the last
    // column re-load the last whole chunk (never stored).
    const T* asrc[A_LOADS];
    int acol[A_LOADS];
#pragma unroll
    for (int p = 0; p < A_LOADS; ++p) {
      const int s = (t + THREADS * p) % A_SLOTS;
      const int r = s >> 4;
      const int c = (s & 15) ^ (r & 15);
      const int rr = r < S.rows ? r : S.rows - 1;
      const int64_t row = S.a_rows ? (int64_t)S.a_rows[S.m0 + rr] : S.m0 + rr;
      asrc[p] = S.A + row * S.lda;
      acol[p] = c * 8;
    }
    const T* bsrc[B_LOADS];
    int brow[B_LOADS];
#pragma unroll
    for (int p = 0; p < B_LOADS; ++p) {
      const int s = t + THREADS * p;
      const int k = s / CPR;
      const int c = (s % CPR) ^ bswz(k);
      const bool hi = TWO && c >= 8;
      const T* base = hi ? S.bu : S.bg;
      int64_t nc = S.ncols;
      if (WIDE && hi) {
        nc = S.ncols - OUT;  // the upper half's valid columns
        if (nc < 8) {        // none: any whole chunk of the lower half (never stored)
          base = S.bg;
          nc = S.ncols;
        }
      }
      int64_t col = (int64_t)(hi ? c - 8 : c) * 8;
      if (col + 8 > nc) col = nc - 8;
      bsrc[p] = base + col;
      brow[p] = k;
    }
    auto issue = [&](int64_t st) {
      char* buf = smem + (int)(st % STAGES) * LDS_STAGE;
      const int64_t k0 = st * SK;
#pragma unroll
      for (int p = 0; p < A_LOADS; ++p) {
        int64_t k = k0 + acol[p];
        if (k + 8 > S.K) k = S.K - 8;  // past the end: any whole chunk (never read)
        __builtin_amdgcn_global_load_lds((global_cvoid_t*)(asrc[p] + k),
                                         (lds_void_t*)(buf + (THREADS * p + wbase) * 16), 16, 0, 0);
      }
#pragma unroll
      for (int p = 0; p < B_LOADS; ++p) {
        int64_t k = k0 + brow[p];
        if (k >= S.K) k = S.K - 1;
        __builtin_amdgcn_global_load_lds((global_cvoid_t*)(bsrc[p] + k * S.ldb),
                                         (lds_void_t*)(buf + LDS_A + (THREADS * p + wbase) * 16), 16, 0, 0);
      }
    };

    const int lane = t & 63, w = t >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    // Output column block jb of this wavefront, and the B part it reads (SwiGLU: 0 gate, 1 up).
    const int jb = TWO ? (w & 3) : w, part = TWO ? (w >> 2) : 0;
    // Transposing reads: source lane lr points at K row 8 lg + lr / 4 (+ 4 for the upper half),
    // column 4 (lr % 4) of the wavefront's 16-column block.
    const int tr_k = 8 * lg + (lr >> 2), tr_c = OUT * part + 16 * jb + 4 * (lr & 3);
    // All fragment reads of a stage go out before one wait, then its MFMAs in K order (one
    // read latency per stage instead of one per K chunk: 15.4 -> 14.7 us for the one-token
    // gate/up GEMM of 8 experts).  The accumulator is acc.g in every wavefront.
    constexpr int KC = 2 * STEPS;  // 32-element K chunks of a stage
    auto compute = [&](const char* stage, int nsteps) {
      u32x4_t a[KC][RB];
      u32x2_t blo[KC], bhi[KC];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
        for (int i = 0; i < RB; ++i)
          a[kc][i] = *reinterpret_cast<const u32x4_t*>(stage + a_off(16 * i + lr, 4 * kc + lg));
        blo[kc] = lds_read_tr16_asm(stage + b_off(32 * kc + tr_k, tr_c));
        bhi[kc] = lds_read_tr16_asm(stage + b_off(32 * kc + tr_k + 4, tr_c));
      }
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) lds_wait_anchor(blo[kc], bhi[kc]);
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        if (kc >= 2 * nsteps) break;
        const u32x4_t bf = u32x4_t{blo[kc][0], blo[kc][1], bhi[kc][0], bhi[kc][1]};
#pragma unroll
        for (int i = 0; i < RB; ++i) Mfma16<T>::step(acc.g[i], a[kc][i], bf);
      }
    };

    constexpr int AHEAD = STAGES - 1;
#pragma unroll
    for (int s = 0; s < AHEAD; ++s)
      if (s < NS) issue(s);
    for (int64_t s = 0; s < NS; ++s) {
      // stage s landed once at most min(AHEAD - 1, NS - 1 - s) later stages remain in flight
      if (NS - 1 - s >= AHEAD - 1) wait_loads<(AHEAD - 1) * LOADS>();
      else wait_loads<0>();
      // Publishes stage s; every wavefront is done reading stage s - 1, whose slot is refilled.
      lds_barrier();
      if (s + AHEAD < NS) issue(s + AHEAD);
      const int64_t left = KT - s * STEPS;
      compute(smem + (int)(s % STAGES) * LDS_STAGE, left < STEPS ? (int)left : STEPS);
    }
    wait_loads<0>();
    if constexpr (SWIGLU) {
      // The up wavefronts hand their accumulators to the gate wavefront of the same columns
      // (acc.u there).  The ring is free: every load has landed and every read is done.
      lds_barrier();
      float* x = reinterpret_cast<float*>(smem);
      if (part == 1) {
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) x[((jb * RB + i) * 4 + r) * 64 + lane] = acc.g[i][r];
      }
      lds_barrier();
      if (part == 0) {
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc.u[i][r] = x[((jb * RB + i) * 4 + r) * 64 + lane];
      }
    }
    return acc;
  }

  // round(acc) (plain) or round(swiglu_value(gate, up)) (the gate wavefronts) of this lane's
  // outputs: row 16 i + 4 (lane / 16) + r, column 16 (w % 4) + lane % 16 of the block.
  __device__ static __forceinline__ void store(const Acc& acc, T* C, int64_t ldc, int rows, int64_t cols) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (SWIGLU && w >= 4) return;
    const int col = (WIDE ? OUT * (w >> 2) : 0) + 16 * (w & 3) + (lane & 15);
    if (col >= cols) return;
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * i + 4 * (lane >> 4) + r;
        if (row >= rows) continue;
        const float v = SWIGLU ? swiglu_value<T>(acc.g[i][r], acc.u[i][r]) : acc.g[i][r];
        Num<T>::store(C + (int64_t)row * ldc + col, v);
      }
  }
};

}  // namespace biops
