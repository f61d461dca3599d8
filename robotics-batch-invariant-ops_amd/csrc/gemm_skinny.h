// Skinny GEMM tile for problems with few rows (decode-size linears): one 32x32 block per
// workgroup, used when all blocks of a launch fit one round on the compute units.
//
// One workgroup owns one 32x32 output block.  Wavefront 0 computes it with exactly the MFMA
// sequence of GemmTile (K steps of 128 bytes in order; inside a step chunk pairs q = 0..3, lane
// half h holding chunk 2q+h), so its bits equal those of every other tile entry.  What differs
// is how operands arrive: every wavefront of the workgroup -- AR/8 for the A rows and 4 for the
// 32 B columns -- issues one 16-byte global->LDS chunk load per K step into a ring of 4-6
// stages of 4 K steps (about 120 KiB).  A stage brings 512 contiguous bytes of every row, and
// one barrier per stage (not per K step) publishes it: on MI355X the per-step wait + barrier
// of a 4 KiB step caps a compute unit near 37 GB/s, four-step stages reach ~55 GB/s.  With
// few rows a block's time is the serial K chain of its accumulator and the weight bytes it
// streams; the ring keeps the stream ahead of the chain.
//
// Only AR A rows are loaded (AR = 8, 16 or 32, the rows a block can hold); MFMA rows past AR
// read loaded rows again (row r reads row r mod AR) and, like rows past M, are never stored.
//
// Requirements (checked by the launcher): K-major B, 16-byte aligned A and B rows, K a whole
// number of 128-byte steps, plain or bias epilogue.
#pragma once

#include "gemm_core.h"

namespace biops {

template <typename T, int AR>
struct SkinnyTile {
  static_assert(AR == 8 || AR == 16 || AR == 32, "A rows per K step");
  static constexpr int NA = AR / 8;       // wavefronts loading A (8 rows x 8 chunks each)
  static constexpr int NB = 4;            // wavefronts loading B (32 columns)
  static constexpr int WAVES = NA + NB;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int VEC = 16 / (int)sizeof(T);
  static constexpr int BK = kKBytes / (int)sizeof(T);
  static constexpr int LDS_A = AR * kKBytes;             // A rows of one K step
  static constexpr int LDS_KSTEP = LDS_A + 32 * kKBytes;  // one K step: A rows, then B columns
  static constexpr int U = 4;                             // K steps per stage (even)
  static constexpr int LDS_STAGE = U * LDS_KSTEP;
  static constexpr int STAGES = (128 * 1024) / LDS_STAGE;  // 6 / 5 / 4 for AR = 8 / 16 / 32
  static constexpr int LDS_BYTES = STAGES * LDS_STAGE;
  static_assert(STAGES >= 3 && (STAGES - 1) * U < 64, "ring depth and vmcnt range");
  static_assert(U % 2 == 0, "stages start on fragment set 0");

  template <int N>
  __device__ static __forceinline__ void wait_loads() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  }
  __device__ static __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }

  // Fragments of one K step for wavefront 0: a[q], b[q] feed MFMA step q.
  struct Frags {
    u32x4_t a[4];
    u32x4_t b[4];
  };
  __device__ static __forceinline__ void load_frags(const char* kstep, Frags& f) {
    const int lane = threadIdx.x & 63;
    const int lr = lane & 31, lb = lane >> 5;
    const int ar = lr & (AR - 1);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f.a[q] = *reinterpret_cast<const u32x4_t*>(kstep + lds_off(ar, 2 * q + lb));
      f.b[q] = *reinterpret_cast<const u32x4_t*>(kstep + LDS_A + lds_off(lr, 2 * q + lb));
    }
  }
  __device__ static __forceinline__ void mfma(f32x16_t& acc, const Frags& f) {
#pragma unroll
    for (int q = 0; q < 4; ++q) Mfma<T>::step(acc, f.a[q], f.b[q]);
  }
  // One K step on `f` while the next step's fragments are read into `g`.  The reads go out
  // right after the first MFMA (the wave issues them while that MFMA occupies the pipe) and
  // have the other three MFMAs to land before the next step needs them.  The scheduling
  // barriers keep the compiler from sinking each read next to its consumer.
  __device__ static __forceinline__ void step(f32x16_t& acc, const Frags& f, const char* next, Frags& g) {
    Mfma<T>::step(acc, f.a[0], f.b[0]);
    __builtin_amdgcn_sched_barrier(0);
    load_frags(next, g);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 1; q < 4; ++q) Mfma<T>::step(acc, f.a[q], f.b[q]);
    __builtin_amdgcn_sched_barrier(0);
  }

  // The 32x32 block at (A, B) with `rows` / `cols` valid rows and columns (>= 1) over KT K
  // steps.  Stage s holds K steps s*U .. s*U+U-1 (the last stage may hold fewer); each
  // wavefront issues one chunk load per K step of a stage.  Returns the accumulator in
  // wavefront 0 (other wavefronts return zeros once their last load is issued; the kernel
  // only lets wavefront 0 continue).
  __device__ static __forceinline__ f32x16_t run(char* smem, const T* A, int64_t lda, int rows,
                                                 const T* B, int64_t ldb, int cols, int64_t KT) {
    f32x16_t acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    if (KT == 0) return acc;
    const int w = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    // This thread's chunk of every K step: slot s = 64*wave + lane of the A or B region, row
    // s/8 at LDS slot s%8, holding logical chunk (s%8) ^ ((row>>1)&7) (the lds_off swizzle).
    const T* src;
    int dst;  // byte offset of this wavefront's 64 slots inside a K step
    {
      const int j = w < NA ? w : w - NA;
      const int s = 64 * j + lane;
      const int r = s >> 3;
      const int c = (s & 7) ^ ((r >> 1) & 7);
      if (w < NA) {
        src = A + (int64_t)(r < rows ? r : rows - 1) * lda + c * VEC;
        dst = 64 * 16 * j;
      } else {
        src = B + (int64_t)(r < cols ? r : cols - 1) * ldb + c * VEC;
        dst = LDS_A + 64 * 16 * j;
      }
    }
    const int64_t NS = (KT + U - 1) / U;  // stages
    auto issue = [&](int64_t stage) {
      char* buf = smem + (int)(stage % STAGES) * LDS_STAGE + dst;
      const int64_t k0 = stage * U;
      if (k0 + U <= KT) {
#pragma unroll
        for (int u = 0; u < U; ++u)
          __builtin_amdgcn_global_load_lds((global_cvoid_t*)(src + (k0 + u) * BK),
                                           (lds_void_t*)(buf + u * LDS_KSTEP), 16, 0, 0);
      } else {
        for (int64_t k = k0; k < KT; ++k)
          __builtin_amdgcn_global_load_lds((global_cvoid_t*)(src + k * BK),
                                           (lds_void_t*)(buf + (int)(k - k0) * LDS_KSTEP), 16, 0, 0);
      }
    };

    for (int64_t s = 0; s < NS && s < STAGES; ++s) issue(s);
    // Stage 0 landed once the loads of stages 1 .. STAGES-1 are all that remain in flight
    // (exact while those are full stages; otherwise wait for everything).
    if (NS > STAGES) wait_loads<(STAGES - 1) * U>();
    else wait_loads<0>();
    lds_barrier();
    // Stages 0 .. NS-2 are full (U steps) and each ends with the barrier that publishes the next
    // stage; the last stage (1..U steps) has none.  Wavefront 0 and the loader wavefronts run
    // separate branch-free loops that meet at the same barriers.
    if (w != 0) {
      for (int64_t s = 0; s + 1 < NS; ++s) {
        if (s + STAGES < NS) wait_loads<(STAGES - 2) * U>();
        else wait_loads<0>();
        lds_barrier();
        if (s + STAGES < NS) issue(s + STAGES);
      }
      return acc;
    }
    // Two fragment sets used alternately (K step j of a stage reads set j&1 while the next
    // step's fragments land in the other): copying fragments between registers would stall on
    // the MFMAs still reading them.  U is even, so every stage starts on set 0.
    Frags F[2];
    load_frags(smem, F[0]);
    for (int64_t s = 0; s + 1 < NS; ++s) {
      const char* cur = smem + (int)(s % STAGES) * LDS_STAGE;
#pragma unroll
      for (int j = 0; j + 1 < U; ++j) step(acc, F[j & 1], cur + (j + 1) * LDS_KSTEP, F[(j + 1) & 1]);
      // Stage s+1 landed once the loads of stages s+2 .. s+STAGES-1 remain in flight.
      if (s + STAGES < NS) wait_loads<(STAGES - 2) * U>();
      else wait_loads<0>();
      // Publishes stage s+1.  Every fragment of stage s is in registers (the last step's were
      // read before this barrier), so stage s is refilled.
      lds_barrier();
      if (s + STAGES < NS) issue(s + STAGES);
      step(acc, F[(U - 1) & 1], smem + (int)((s + 1) % STAGES) * LDS_STAGE, F[0]);
    }
    {
      const int64_t s = NS - 1;
      const char* cur = smem + (int)(s % STAGES) * LDS_STAGE;
      const int nk = (int)(KT - s * U);
#pragma unroll
      for (int j = 0; j < U; ++j) {
        if (j < nk) {
          if (j + 1 < nk) load_frags(cur + (j + 1) * LDS_KSTEP, F[(j + 1) & 1]);
          mfma(acc, F[j & 1]);
        }
      }
    }
    return acc;
  }
};

}  // namespace biops
