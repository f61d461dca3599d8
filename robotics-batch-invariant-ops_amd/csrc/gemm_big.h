// Large-tile GEMM schedule (M >= ~1024): BM x BN block on four wavefronts (2 x 2), each owning
// a (BM/2) x (BN/2) wave tile whose fp32 accumulators live in the accumulation registers (one
// wavefront per SIMD, 16 independent 32x32 accumulators at 256 x 256).
//
// Same arithmetic as every other tile entry (gemm_core.h): 128-byte K steps in order, chunk
// pairs q = 0..3 in order inside a step.  A stage of the LDS ring holds SB bytes of K per row
// (SB = 128: one K step, two stages of 64 KiB at 256 x 256).  Measured on MI355X (bf16,
// M = 4096, N = 8192, K = 2048): half-step stages (deeper ring, 64-byte requests) and
// register-staged loads were both slower than this schedule.
//
// Stage h (ring slot h % STAGES) holds P = SB / 32 chunk pairs.  Per stage, per wavefront:
//   group p (p = 0 .. P-1): the MFMAs of pair p, interleaved with the LDS reads of the next
//   pair (pair p+1, or pair 0 of stage h+1 for the last group);
//   between groups P-2 and P-1: wait for stage h+1, barrier (publishes h+1; all of stage h
//   has been read), refill slot h with stage h+STAGES.
// The compiler waits for all outstanding LDS reads before an MFMA that needs one (the global
// -> LDS loads make its LDS counter out of order), so each group starts with one wait and its
// MFMAs only read fragments loaded during the previous group.
//
// LDS stage layout: A rows (BM x SB bytes) then B columns (BN x SB bytes).  A 16-byte read
// serves 16 lanes per clock from a 256-byte window, so 16 consecutive rows reading the same
// chunk must land in 16 distinct 16-byte slots: chunk c of row r sits at slot c ^ ((r >> 1) & 7)
// (c ^ ((r >> 2) & 3) for 64-byte rows).
#pragma once

#include "gemm_core.h"

namespace biops {

template <typename T, int BM, int BN, int SB>
struct BigTile {
  static_assert(sizeof(T) == 2, "16-bit operands");
  static_assert(SB == 64 || SB == 128, "stage = half or whole K step");
  static constexpr int THREADS = 256;
  static constexpr int WM = BM / 2, WN = BN / 2;
  static constexpr int FM = WM / 32, FN = WN / 32;
  static constexpr int VEC = 8;
  static constexpr int CPR = SB / 16;             // 16-byte chunks per row of a stage
  static constexpr int P = CPR / 2;               // chunk pairs per stage
  static constexpr int STAGE_ELEMS = SB / 2;      // K elements per stage
  static constexpr int LDS_A = BM * SB;
  static constexpr int LDS_STAGE = (BM + BN) * SB;
  static constexpr int LDS_MAX = 160 * 1024;
  static constexpr int STAGES = LDS_MAX / LDS_STAGE;
  static constexpr int RING = STAGES * LDS_STAGE;
  static constexpr int SMEM_BYTES = RING;
  static constexpr int A_LOADS = BM * CPR / THREADS;  // 16-byte chunks per thread per stage
  static constexpr int B_LOADS = BN * CPR / THREADS;
  static constexpr int LOADS = A_LOADS + B_LOADS;
  static_assert(STAGES >= 2, "ring");
  static_assert((STAGES - 1) * LOADS < 64, "vmcnt range");
  static_assert(SMEM_BYTES <= LDS_MAX, "LDS");
  typedef f32x16_t Acc;

  struct Frags {
    u32x4_t a[FM];
    u32x4_t b[FN];
  };

  __device__ static __forceinline__ int off(int r, int c) {
    if constexpr (SB == 128) return (r << 7) + ((c ^ ((r >> 1) & 7)) << 4);
    else return (r << 6) + ((c ^ ((r >> 2) & 3)) << 4);
  }

  template <int N>
  __device__ static __forceinline__ void wait_loads() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  }
  __device__ static __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
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
#pragma unroll
    for (int j = 0; j < FN; ++j)
      f.b[j] = *reinterpret_cast<const u32x4_t*>(stage + LDS_A + off(wn * WN + j * 32 + lr, c));
  }

  __device__ static __forceinline__ void mfmas(Acc (&acc)[FM][FN], const Frags& f) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) Mfma<T>::step(acc[i][j], f.a[i], f.b[j]);
  }

  // Interleave the group's MFMAs with its LDS reads (and global->LDS loads, `nv` of them).
  template <int NV>
  __device__ static __forceinline__ void interleave() {
    constexpr int NM = FM * FN, NR = FM + FN;
    constexpr int MPR = NM / NR > 0 ? NM / NR : 1;  // MFMAs per read
    constexpr int VPR = (NV + NR - 1) / NR;         // loads per read
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, MPR, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);    // DS read
      if constexpr (NV > 0) __builtin_amdgcn_sched_group_barrier(0x020, VPR, 0);  // VMEM read
    }
  }

  // Full K loop of one tile into acc (zeroed here).  A: tile rows (rows valid), B: tile
  // columns, K-major (cols valid), K a whole number of 128-byte steps.
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
    const int t = threadIdx.x;
    const int wbase = t & ~63;
    // Source of this thread's chunk p of every stage (slot s = t + 256p: row s/CPR, slot s%CPR
    // holding logical chunk (slot) ^ swizzle(row)).
    const T* src[LOADS];
#pragma unroll
    for (int p = 0; p < LOADS; ++p) {
      const int s = t + THREADS * p;
      const int sl = p < A_LOADS ? s : s - BM * CPR;
      const int r = sl / CPR;
      const int pos = sl % CPR;
      const int c = (off(r, pos) >> 4) & (CPR - 1);  // off() is an involution on the slot
      if (p < A_LOADS) src[p] = A + (int64_t)(r < rows ? r : rows - 1) * lda + c * VEC;
      else src[p] = B + (int64_t)(r < cols ? r : cols - 1) * ldb + c * VEC;
    }
    // Loads of stage h into ring slot `slot`; stages past the end re-load the last one (into a
    // slot nobody reads again), so every iteration issues the same loads and the vmcnt waits
    // are constants.
    auto issue = [&](int slot, int64_t h) {
      char* st = smem + slot * LDS_STAGE;
      const int64_t k = (h < H ? h : H - 1) * STAGE_ELEMS;
#pragma unroll
      for (int p = 0; p < LOADS; ++p)
        __builtin_amdgcn_global_load_lds((global_cvoid_t*)(src[p] + k),
                                         (lds_void_t*)(st + (THREADS * p + wbase) * 16), 16, 0, 0);
    };

#pragma unroll
    for (int s = 0; s < STAGES; ++s) issue(s, s);
    wait_loads<(STAGES - 1) * LOADS>();  // stage 0 landed
    lds_barrier();
    Frags f[2];
    read_frags(smem, 0, f[0]);
    int cur = 0;  // ring slot of stage h
    for (int64_t h = 0; h < H; ++h) {
      const char* st = smem + cur * LDS_STAGE;
      const int nxt = cur + 1 == STAGES ? 0 : cur + 1;
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const Frags& use = f[p & 1];
        Frags& next = f[(p + 1) & 1];
        if (p + 1 < P) {
          read_frags(st, p + 1, next);
          mfmas(acc, use);
          interleave<0>();
          __builtin_amdgcn_sched_barrier(0);
        } else {
          // Stage h+1 landed once the STAGES-2 stages issued after it remain in flight.  The
          // barrier publishes it; every wavefront has read all of stage h, which takes stage
          // h+STAGES.
          wait_loads<(STAGES - 2) * LOADS>();
          lds_barrier();
          issue(cur, h + STAGES);
          read_frags(smem + nxt * LDS_STAGE, 0, next);
          mfmas(acc, use);
          interleave<LOADS>();
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
  // row offsets in registers.
  __device__ static __forceinline__ void epilogue(Acc (&acc)[FM][FN], T* C, int64_t ldc, int rows, int cols,
                                                  const T* bias) {
    int ldc32 = (int)ldc;
    asm volatile("" : "+s"(ldc32));
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = acc_col(j);
        const bool col_ok = col < cols;
        const float bv = (bias && col_ok) ? Num<T>::load(bias + col) : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = acc_row(i, r);
          if (col_ok && row < rows)
            Num<T>::store(C + (uint32_t)(row * ldc32 + col), bias ? acc[i][j][r] + bv : acc[i][j][r]);
        }
      }
  }
};

}  // namespace biops
