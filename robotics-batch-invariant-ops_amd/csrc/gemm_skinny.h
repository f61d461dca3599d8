// Skinny GEMM tile for problems with few rows (decode-size linears): one 32 x BC (or, 16-bit
// types, 64 x BC) block per workgroup, used when all blocks of a launch fit one round on the
// compute units.
//
// One workgroup owns one 32 x BC output block (BC = 64, 32, 16 or 8 columns; 64 x 32 and
// 64 x 64 blocks load AR = 64 rows).  Up to eight of its wavefronts compute it, each a 16- or
// 32-row by 8- to 32-column part, over K steps of 128 bytes in order, with the arithmetic of
// SkinnyMath below (bits equal to those of every other tile entry).  What differs is how
// operands arrive: eight
// wavefronts share the 1 KiB global->LDS load instructions of a stage (4 or 8 K steps, 512 or
// 1024 bytes of every row) round-robin, into a ring of 2-4 stages (up to the 160 KiB of a
// compute unit), and one barrier per stage publishes it.  On MI355X a compute unit's load rate
// grows with the bytes per row per stage and with the number of issuing wavefronts (4 KiB
// per-step stages on one wavefront: ~37 GB/s; 8-step stages on 8 wavefronts: ~2x), but not
// with the bytes in flight past a few stages.  With few rows a block's time is the serial K
// chain of its accumulator and the bytes it streams; the ring keeps the stream ahead of the
// chain.
//
// Only AR A rows are loaded (AR = 8, 16 or 32 for 32-row blocks, the rows a block can hold);
// MFMA rows past AR read loaded rows again (row r reads row r mod AR) and, like rows past M,
// are never stored.
// Likewise only BC B columns are loaded and MFMA column c reads column c mod BC.  An MFMA output
// element depends on its own A row and B column only, so the BC stored columns carry the bits
// of a full 32-column block; narrow blocks spread a few-column-block problem (N = 2048: 64
// blocks of 32) over every compute unit, each streaming BC/32 of the weight bytes.
//
// Requirements (checked by the launcher): K-major B, 16-byte aligned A and B rows, K a whole
// number of 128-byte steps, plain or bias epilogue.
#pragma once

#include "gemm_core.h"

namespace biops {

// Arithmetic of one skinny block.  16-bit types: v_mfma_f32_16x16x32_{bf16,f16} on 16-row x
// 16-column sub-blocks; quad q' = 0, 1 of a K step feeds chunks 4q'..4q'+3 (lane group g = l/16
// holding chunk 4q'+g) to one instruction.  On MI355X one such instruction gives the bits of
// the two v_mfma_f32_32x32x16 of chunk pairs (4q', 4q'+1) and (4q'+2, 4q'+3) that every other
// tile entry issues: a standalone comparison of both chains over 9.4 M dot products of length
// 4096 (bf16 and fp16; normal, wide-exponent, cancelling, subnormal, infinite, NaN and
// overflowing operands) found no differing bit, and the tile-menu tests compare the entries
// bit for bit.  The 16x16x32 chain is half as long and each link about half as slow, which is
// what bounds a one-row block with long K.  fp32 keeps the 32x32x2 MFMAs of GemmTile.
template <typename T> struct Mfma16;
template <> struct Mfma16<bf16_t> {
  __device__ static __forceinline__ void step(f32x4_t& acc, const u32x4_t& a, const u32x4_t& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
  }
};
template <> struct Mfma16<f16_t> {
  __device__ static __forceinline__ void step(f32x4_t& acc, const u32x4_t& a, const u32x4_t& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), acc, 0, 0, 0);
  }
};

template <typename T, int AR, int BC, bool NARROW = (sizeof(T) == 2)>
struct SkinnyMath;

template <typename T, int AR, int BC>
struct SkinnyMath<T, AR, BC, true> {
  static constexpr int RB = AR > 16 ? 2 : 1;  // 16-row sub-blocks
  static constexpr int CB = BC > 16 ? 2 : 1;  // 16-column sub-blocks
  struct Acc {
    f32x4_t c[RB][CB];
  };
  struct Frags {
    u32x4_t a[2][RB];
    u32x4_t b[2][CB];
  };
  __device__ static __forceinline__ void zero(Acc& acc) {
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int j = 0; j < CB; ++j) acc.c[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  // Lane l reads row / column 16 i + l % 16 (modulo the rows / columns loaded), chunk
  // 4 q' + l / 16.
  __device__ static __forceinline__ void load(const char* kstep, int lds_a, Frags& f) {
    const int lane = threadIdx.x & 63;
    const int lr = lane & 15, lg = lane >> 4;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
#pragma unroll
      for (int i = 0; i < RB; ++i)
        f.a[q][i] = *reinterpret_cast<const u32x4_t*>(kstep + lds_off((16 * i + lr) & (AR - 1), 4 * q + lg));
#pragma unroll
      for (int j = 0; j < CB; ++j)
        f.b[q][j] = *reinterpret_cast<const u32x4_t*>(kstep + lds_a + lds_off((16 * j + lr) & (BC - 1), 4 * q + lg));
    }
  }
  // MFMA number n of a K step (n = 0 .. COUNT-1, quad-major), so that a caller can place other
  // instructions after the first one.
  static constexpr int COUNT = 2 * RB * CB;
  __device__ static __forceinline__ void one(Acc& acc, const Frags& f, int n) {
    const int q = n / (RB * CB), i = (n / CB) % RB, j = n % CB;
    Mfma16<T>::step(acc.c[i][j], f.a[q][i], f.b[q][j]);
  }
  // round(acc (+ bias[n])) of this lane's outputs: row 16 i + 4 (l / 16) + r, column
  // 16 j + l % 16.
  __device__ static __forceinline__ void store(const Acc& acc, T* C, int64_t ldc, int rows, int cols, const T* bias) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      const int col = 16 * j + (lane & 15);
      if (col >= cols) continue;
      const float bv = bias ? Num<T>::load(bias + col) : 0.f;
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * i + 4 * (lane >> 4) + r;
          if (row < rows) Num<T>::store(C + (int64_t)row * ldc + col, bias ? acc.c[i][j][r] + bv : acc.c[i][j][r]);
        }
    }
  }
};

// fp32: the 32x32 block of GemmTile's MFMA sequence (chunk pairs q = 0..3, four 32x32x2 MFMAs
// each).
template <typename T, int AR, int BC>
struct SkinnyMath<T, AR, BC, false> {
  struct Acc {
    f32x16_t c;
  };
  struct Frags {
    u32x4_t a[4];
    u32x4_t b[4];
  };
  __device__ static __forceinline__ void zero(Acc& acc) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc.c[r] = 0.f;
  }
  __device__ static __forceinline__ void load(const char* kstep, int lds_a, Frags& f) {
    const int lane = threadIdx.x & 63;
    const int lr = lane & 31, lb = lane >> 5;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f.a[q] = *reinterpret_cast<const u32x4_t*>(kstep + lds_off(lr & (AR - 1), 2 * q + lb));
      f.b[q] = *reinterpret_cast<const u32x4_t*>(kstep + lds_a + lds_off(lr & (BC - 1), 2 * q + lb));
    }
  }
  static constexpr int COUNT = 4;
  __device__ static __forceinline__ void one(Acc& acc, const Frags& f, int n) { Mfma<T>::step(acc.c, f.a[n], f.b[n]); }
  // Row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
  __device__ static __forceinline__ void store(const Acc& acc, T* C, int64_t ldc, int rows, int cols, const T* bias) {
    const int lane = threadIdx.x & 63;
    const int col = lane & 31;
    if (col >= cols) return;
    const float bv = bias ? Num<T>::load(bias + col) : 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (row < rows) Num<T>::store(C + (int64_t)row * ldc + col, bias ? acc.c[r] + bv : acc.c[r]);
    }
  }
};

template <typename T, int AR, int BC>
struct SkinnyTile {
  static_assert(AR == 8 || AR == 16 || AR == 32 || AR == 64, "A rows per K step");
  static_assert(BC == 8 || BC == 16 || BC == 32 || BC == 64, "B columns per K step");
  static constexpr int WAVES = 8;
  // The block's MFMA chains are split over CW computing wavefronts of WR rows x WC columns
  // (whole 16-row / 16-column sub-blocks, so that the lds_off swizzle of a wavefront's rows and
  // columns is that of rows / columns 0..15); all eight wavefronts load.  16-bit types: 16
  // columns per wavefront from 32-column blocks on, and 16 rows for 32-row blocks of at most 32
  // columns; fp32 keeps whole 32x32 blocks (32 columns each for 64-column blocks).  Measured on
  // MI355X (bf16, same-box A/B, same bits; one computing wavefront per 32 columns before):
  // 128 x 2048 x 8192 (32 x 32 blocks, 4 wavefronts) 20.3 -> 14.8 us, 32 x 2048 x 8192 (32 x 8,
  // 2) 12.9 -> 11.5 us, 64 x 2048 x 8192 (32 x 16, 2) 12.8 -> 11.6 us, 32 x 8192 x 2048 (32 x 32)
  // 8.3 -> 6.8 us, 256 x 2048 x 8192 (32 x 64, 4) 27.2 -> 24.8 us (25.9 with 8 of 16 x 16).
  static constexpr int WC = sizeof(T) == 2 ? (BC >= 32 ? 16 : BC) : (BC > 32 ? 32 : BC);
  static constexpr int WR = AR > 32 ? 32 : (sizeof(T) == 2 && AR == 32 && BC <= 32 ? 16 : AR);
  static constexpr int CWC = BC / WC;
  static constexpr int CW = (AR / WR) * CWC;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int VEC = 16 / (int)sizeof(T);
  static constexpr int BK = kKBytes / (int)sizeof(T);
  static constexpr int IPK = AR / 8 + BC / 8;             // 1 KiB load instructions per K step
  static constexpr int LDS_A = AR * kKBytes;             // A rows of one K step
  static constexpr int LDS_KSTEP = LDS_A + BC * kKBytes;  // one K step: A rows, then B columns
  // K steps per stage: 4 for the blocks of at least 48 rows + columns whose 4-step stage deals
  // evenly over the wavefronts (32 x 32, 32 x 16, 16 x 32), 8 for the others.  Ring: as deep as
  // 160 KiB allows, at most 4 stages, 2 for 8 x 32 blocks.  Fewer bytes in flight measured
  // faster on MI355X (bf16, same-box A/B in alternating order, same bits): M = 64, N = 2048,
  // K = 8192 (32 x 16) 15.0 -> 12.6 us with 4-step stages (4 of 24 KiB instead of 3 of 48);
  // M = 16 / 32, N = 8192, K = 2048 (16 x 32 / 32 x 32) 7.6 -> 6.6 / 9.3 -> 8.8 us; one to eight
  // rows, N = 8192, K = 2048 (8 x 32) 6.7-7.1 -> 6.4-6.8 us with 2 stages instead of 4; 3, 6 and
  // 8 stages were slower, and so were deeper rings of the narrow blocks (N = 2048, K = 8192,
  // one row, 8-column blocks: 13.8 us at 8 stages, 13.3 us at 4, against 12.5 us for the bare
  // chain of 512 dependent MFMAs).
  static constexpr int U = (IPK * 4) % WAVES == 0 && AR + BC >= 48 ? 4 : 8;
  static constexpr int LDS_STAGE = U * LDS_KSTEP;
  static constexpr int MAX_STAGES = AR == 8 && BC == 32 ? 2 : 4;
  static constexpr int STAGES_FIT = (160 * 1024) / LDS_STAGE;
  static constexpr int STAGES = STAGES_FIT < MAX_STAGES ? STAGES_FIT : MAX_STAGES;
  static constexpr int LDS_BYTES = STAGES * LDS_STAGE;
  static constexpr int LOADS = U * IPK / WAVES;           // per wavefront per stage
  static_assert(U * IPK % WAVES == 0, "uniform loads per wavefront");
  static_assert(STAGES >= 2 && STAGES * LOADS < 64, "ring depth and vmcnt range");
  static_assert(U % 4 == 0, "stages start on fragment set 0");

  template <int N>
  __device__ static __forceinline__ void wait_loads() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  }
  // Through the builtins, so the compiler knows every LDS read has landed (see GemmTile).
  __device__ static __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");  // no memory access moves across the barrier (compiler fence)
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0), vmcnt unchanged
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }

  using Math = SkinnyMath<T, WR, WC>;
  using Acc = typename Math::Acc;
  using Frags = typename Math::Frags;
  // Computing wavefront w reads rows WR (w / CWC) .. + WR-1 and columns WC (w % CWC) .. + WC-1
  // (the lds_off swizzle of a row or column only depends on its index modulo 16).
  __device__ static __forceinline__ void load_frags(const char* kstep, Frags& f) {
    const int w = CW > 1 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;
    const int aofs = (w / CWC) * WR * kKBytes, bofs = (w % CWC) * WC * kKBytes;
    Math::load(kstep + aofs, LDS_A + bofs - aofs, f);
  }
  __device__ static __forceinline__ void mfma(Acc& acc, const Frags& f) {
#pragma unroll
    for (int n = 0; n < Math::COUNT; ++n) Math::one(acc, f, n);
  }
  // Two consecutive K steps (their fragments read together).
  struct Frags2 {
    Frags s[2];
  };
  // K steps j, j+1 on `f` while the fragments of the two steps at `next` are read into `g`.
  // With an LDS DMA in flight the compiler waits for every outstanding LDS read before an
  // MFMA that needs one, so the reads go out right after the first MFMA and have the other
  // MFMAs of the two steps to land before the next pair's wait.  The scheduling barriers keep
  // the compiler from sinking each read next to its consumer.
  __device__ static __forceinline__ void step2(Acc& acc, const Frags2& f, const char* next, Frags2& g) {
    Math::one(acc, f.s[0], 0);
    __builtin_amdgcn_sched_barrier(0);
    load_frags(next, g.s[0]);
    load_frags(next + LDS_KSTEP, g.s[1]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int n = 1; n < Math::COUNT; ++n) Math::one(acc, f.s[0], n);
    mfma(acc, f.s[1]);
    __builtin_amdgcn_sched_barrier(0);
  }

  // The 32 x BC block at (A, B) with `rows` / `cols` valid rows and columns (>= 1) over KT K
  // steps.  Stage s holds K steps s*U .. s*U+U-1 (the last stage may hold fewer).  The U*IPK
  // 1 KiB load instructions of a stage (K step u, part p: A rows 8p..8p+7 or B columns) are
  // dealt round-robin to the 8 wavefronts.  Returns the accumulator of its part of the block
  // in computing wavefront w < CW (the other wavefronts return zeros once their last load is
  // issued; the kernel only lets the computing wavefronts continue).
  __device__ static __forceinline__ Acc run(char* smem, const T* A, int64_t lda, int rows,
                                            const T* B, int64_t ldb, int cols, int64_t KT) {
    Acc acc;
    Math::zero(acc);
    if (KT == 0) return acc;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar LDS offsets
    const int lane = threadIdx.x & 63;
    // This thread's load i of a stage: instruction w + WAVES*i = (K step u, part p).  Lane l
    // writes slot l of the part's 64 slots: row 8*part + l/8, holding logical chunk
    // (l%8) ^ ((row>>1)&7) (the lds_off swizzle).
    const T* src[LOADS];
    int ku[LOADS];   // K step inside the stage
    int dst[LOADS];  // byte offset of the part inside a stage (wave-uniform)
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int ins = w + WAVES * i;
      const int u = ins / IPK, p = ins % IPK;
      const bool is_a = p < AR / 8;
      const int part = is_a ? p : p - AR / 8;
      const int r = 8 * part + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      src[i] = is_a ? A + (int64_t)(r < rows ? r : rows - 1) * lda + c * VEC
                    : B + (int64_t)(r < cols ? r : cols - 1) * ldb + c * VEC;
      ku[i] = u;
      dst[i] = u * LDS_KSTEP + (is_a ? 0 : LDS_A) + part * 64 * 16;
    }
    const int64_t NS = (KT + U - 1) / U;  // stages
    // Loads of stage `stage`; K steps past the end re-load the last one (into slots nobody
    // reads), so every stage issues the same loads and the vmcnt waits are constants.
    auto issue = [&](int64_t stage) {
      char* buf = smem + (int)(stage % STAGES) * LDS_STAGE;
#pragma unroll
      for (int i = 0; i < LOADS; ++i) {
        const int64_t k = stage * U + ku[i];
        __builtin_amdgcn_global_load_lds((global_cvoid_t*)(src[i] + (k < KT ? k : KT - 1) * BK),
                                         (lds_void_t*)(buf + dst[i]), 16, 0, 0);
      }
    };

#pragma unroll
    for (int s = 0; s < STAGES; ++s) issue(s);
    wait_loads<(STAGES - 1) * LOADS>();  // stage 0 landed
    lds_barrier();
    // Stages 0 .. NS-2 are full (U steps) and each ends with the barrier that publishes the next
    // stage; the last stage (1..U steps) has none.  The computing and the loader wavefronts run
    // separate branch-free loops that meet at the same barriers.
    if (w >= CW) {
      for (int64_t s = 0; s + 1 < NS; ++s) {
        wait_loads<(STAGES - 2) * LOADS>();  // stage s+1 landed
        lds_barrier();
        issue(s + STAGES);
      }
      wait_loads<0>();
      return acc;
    }
    // Two fragment sets of two K steps each, used alternately (steps 2d, 2d+1 of a stage read
    // set d&1 while the next pair lands in the other): copying fragments between registers
    // would stall on the MFMAs still reading them.  U is a multiple of 4, so every stage
    // starts on set 0.
    Frags2 F[2];
    load_frags(smem, F[0].s[0]);
    load_frags(smem + LDS_KSTEP, F[0].s[1]);
    for (int64_t s = 0; s + 1 < NS; ++s) {
      const char* cur = smem + (int)(s % STAGES) * LDS_STAGE;
#pragma unroll
      for (int d = 0; d + 1 < U / 2; ++d) step2(acc, F[d & 1], cur + (2 * d + 2) * LDS_KSTEP, F[(d + 1) & 1]);
      // Stage s+1 landed once the loads of the STAGES-2 later stages remain in flight.
      wait_loads<(STAGES - 2) * LOADS>();
      // Publishes stage s+1.  Every fragment of stage s is in registers (the last pair's were
      // read before this barrier), so stage s is refilled.
      lds_barrier();
      issue(s + STAGES);
      step2(acc, F[(U / 2 - 1) & 1], smem + (int)((s + 1) % STAGES) * LDS_STAGE, F[0]);
    }
    {
      // last stage: 1..U steps, fragments read one step ahead (set 0 holds steps 0 and 1)
      const int64_t s = NS - 1;
      const char* cur = smem + (int)(s % STAGES) * LDS_STAGE;
      const int nk = (int)(KT - s * U);
      mfma(acc, F[0].s[0]);
      if (nk > 1) mfma(acc, F[0].s[1]);
#pragma unroll
      for (int j = 2; j < U; ++j) {
        if (j < nk) {
          Frags g;
          load_frags(cur + j * LDS_KSTEP, g);
          mfma(acc, g);
        }
      }
    }
    wait_loads<0>();
    return acc;
  }

  // ---- Loader-split schedule with fragments read three pairs ahead ----
  // For blocks whose computing wavefronts each hold one 16 x 16 accumulator (16-bit types, at
  // most 16 rows and 16 columns per wavefront) the time of run() is the computing wavefronts'
  // chain: every pair of K steps waited for the LDS reads issued during the pair before it.
  // A global->LDS load in flight makes the compiler wait for every outstanding LDS read
  // (lgkmcnt(0)) before a fragment is used, so reads issued further ahead would be waited for
  // just as early.  Here DL loader wavefronts (after the CW computing ones) issue every load,
  // and the computing wavefronts, with no such load on their path, read the fragments of pair
  // p + 3 while pair p runs (four register sets) and the compiler waits for each set alone.
  // Stages hold UD = 8 K steps in a ring of DSTAGES = 4 slots; barrier t (t = 1 .. NS-1),
  // which the computing wavefronts reach at pair 1 of stage t-1, publishes stage t and refills
  // the slot of stage t-2, whose fragments are all in registers by then, so it needs no LDS
  // wait.  The MFMAs run in run()'s order (K step pairs in order, quads in order), so the bits
  // are those of every other entry.  Measured on MI355X (bf16, same-box A/B against run(),
  // launches back to back, weights in the last-level cache): one row, N = 8192, K = 2048 (8 x 32
  // blocks) 6.3 -> 5.7 us; N = 2048, K = 8192 (8 x 8 blocks) 7.8 -> 6.6 us, M = 32 (32 x 8)
  // 11.6 -> 10.4 us.  Blocks whose 8-step stages leave room for only three slots (16 x 32,
  // 32 x 16, 32 x 32) keep run(): with three slots (one stage in flight) M = 16, N = 8192,
  // K = 2048 took 6.2 -> 7.1 us and M = 64, N = 2048, K = 8192 11.5 -> 16.1 us, and with 4-step
  // stages in rings of five or six slots 6.3 -> 6.8, 11.7 -> 12.6 and, for 32 x 32 blocks,
  // M = 32, N = 8192 6.9 -> 7.8 us and M = 128, N = 2048, K = 8192 14.1 -> 16.5 us.  K that is
  // not a whole number of stages keeps run() as well.  Filling all four slots up front (the
  // last stage of a K = 2048 block then issued with the others) measured slower: one row,
  // N = 8192, K = 2048 5.6 -> 5.7 us, M = 8, N = 4096, K = 1024 4.2 -> 4.5 us.
  static constexpr int DL = 8;                     // loader wavefronts
  static constexpr int DTHREADS = 64 * (CW + DL);
  static constexpr int UD = 8;                     // K steps per stage
  static constexpr int PPS = UD / 2;               // K step pairs per stage
  static constexpr int DSETS = 4;                  // fragment sets (pairs) in registers
  static constexpr int DA = DSETS - 1;             // read-ahead, in pairs
  static constexpr int DSTAGE_BYTES = UD * LDS_KSTEP;
  static constexpr int DSTAGES = 4;
  static constexpr int DLDS_BYTES = DSTAGES * DSTAGE_BYTES;
  static constexpr int DLOADS = UD * IPK / DL;     // loads per loader wavefront per stage
  static constexpr bool DEEP = sizeof(T) == 2 && Math::COUNT == 2 && DLDS_BYTES <= 160 * 1024;
  static_assert(!DEEP || (PPS == DSETS && UD * IPK % DL == 0 && (DSTAGES - 1) * DLOADS < 64 &&
                          DTHREADS <= 1024), "deep schedule");

  __device__ static __forceinline__ void barrier_only() {
    asm volatile("" ::: "memory");  // compiler fence
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  __device__ static __forceinline__ void read_pair(const char* p, Frags2& g) {
    load_frags(p, g.s[0]);
    load_frags(p + LDS_KSTEP, g.s[1]);
  }
  // Pair f with the reads of the pair at `next` into g (g was last read by the previous pair's
  // MFMAs).  The reads are unconditional, so that the compiler's count of outstanding reads is
  // the same on every path; past the last stage they read ring bytes that nothing uses.
  __device__ static __forceinline__ void deep_pair(Acc& acc, const Frags2& f, const char* next, Frags2& g) {
    Math::one(acc, f.s[0], 0);
    __builtin_amdgcn_sched_barrier(0);
    read_pair(next, g);
    __builtin_amdgcn_sched_barrier(0);
    Math::one(acc, f.s[0], 1);
    mfma(acc, f.s[1]);
    __builtin_amdgcn_sched_barrier(0);
  }

  // The block of run() on DTHREADS threads, KT a positive multiple of UD.  Returns the
  // accumulator of computing wavefront w < CW (loader wavefronts return zeros).
  __device__ static __forceinline__ Acc run_deep(char* smem, const T* A, int64_t lda, int rows,
                                                 const T* B, int64_t ldb, int cols, int64_t KT) {
    Acc acc;
    Math::zero(acc);
    if constexpr (DEEP) {
      const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
      const int64_t NS = KT / UD;
      if (w >= CW) {
        // Loader li issues instructions li + DL*i of a stage (K step u, part p: A rows 8p..8p+7
        // or B columns, as in run()).
        const int li = w - CW;
        const int lane = threadIdx.x & 63;
        const T* src[DLOADS];
        int ku[DLOADS];
        int dst[DLOADS];
#pragma unroll
        for (int i = 0; i < DLOADS; ++i) {
          const int ins = li + DL * i;
          const int u = ins / IPK, p = ins % IPK;
          const bool is_a = p < AR / 8;
          const int part = is_a ? p : p - AR / 8;
          const int r = 8 * part + (lane >> 3);
          const int c = (lane & 7) ^ ((r >> 1) & 7);
          src[i] = is_a ? A + (int64_t)(r < rows ? r : rows - 1) * lda + c * VEC
                        : B + (int64_t)(r < cols ? r : cols - 1) * ldb + c * VEC;
          ku[i] = u;
          dst[i] = u * LDS_KSTEP + (is_a ? 0 : LDS_A) + part * 64 * 16;
        }
        auto issue = [&](int64_t stage) {  // stage < NS
          char* buf = smem + (int)(stage % DSTAGES) * DSTAGE_BYTES;
#pragma unroll
          for (int i = 0; i < DLOADS; ++i)
            __builtin_amdgcn_global_load_lds((global_cvoid_t*)(src[i] + (stage * UD + ku[i]) * BK),
                                             (lds_void_t*)(buf + dst[i]), 16, 0, 0);
        };
#pragma unroll
        for (int s = 0; s < DSTAGES - 1; ++s)
          if (s < NS) issue(s);
        if (NS >= DSTAGES - 1)
          wait_loads<(DSTAGES - 2) * DLOADS>();  // stage 0 landed
        else
          wait_loads<0>();
        barrier_only();  // publishes stage 0
        for (int64_t t = 1; t < NS; ++t) {
          // issued so far: stages 0 .. min(t + DSTAGES - 3, NS - 1)
          if (t + DSTAGES - 3 < NS)
            wait_loads<(DSTAGES - 3) * DLOADS>();  // stage t landed
          else
            wait_loads<0>();
          barrier_only();
          if (t + DSTAGES - 2 < NS) issue(t + DSTAGES - 2);  // into the slot of stage t-2
        }
        wait_loads<0>();
        return acc;
      }
      // Nothing of this wavefront is outstanding, but the compiler may join this path with the
      // loaders' (their loads still counted as pending), which would make it wait for every LDS
      // read at the loop head; the explicit wait gives the loop a clean count.  (With the one
      // drain per stage that this and the read order below remove, the shapes above measured
      // the same: their time is the chain of dependent MFMAs, about 30 cycles a link.)
      __builtin_amdgcn_s_waitcnt(0);
      barrier_only();  // stage 0 published
      // Pairs 0 .. DA-1 read in order (the scheduling barriers keep the compiler from reversing
      // them), so that on entry, as on every later pass, the set of the loop's first pair is
      // the oldest of the outstanding reads and its wait leaves the younger ones in flight.
      Frags2 F[DSETS];
#pragma unroll
      for (int i = 0; i < DA; ++i) {
        read_pair(smem + 2 * i * LDS_KSTEP, F[i]);
        __builtin_amdgcn_sched_barrier(0);
      }
      for (int64_t s = 0; s < NS; ++s) {
        const char* cur = smem + (int)(s % DSTAGES) * DSTAGE_BYTES;
        const char* nxt = smem + (int)((s + 1) % DSTAGES) * DSTAGE_BYTES;
#pragma unroll
        for (int d = 0; d < PPS; ++d) {
          // the reads of this pair reach stage s+1 from pair PPS - DA on
          if (d == PPS - DA && s + 1 < NS) barrier_only();
          const int rp = d + DA;
          const char* next = rp < PPS ? cur + rp * 2 * LDS_KSTEP : nxt + (rp - PPS) * 2 * LDS_KSTEP;
          deep_pair(acc, F[d], next, F[(d + DA) % DSETS]);
        }
      }
    }
    return acc;
  }
};

}  // namespace biops
