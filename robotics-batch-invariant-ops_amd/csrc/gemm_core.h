// Fixed-schedule MFMA GEMM tiles for gfx950 (CDNA4), shared by GEMM, BMM, grouped GEMM
// (varlen attention) and the MoE expert GEMMs.
//
// Batch-invariance rule: every output element C[m,n] is produced by the same sequence of MFMA
// instructions over the same K chunks, in the same order, whatever M, the batch size, the block
// tile or the load path:
//   * K is consumed in fixed steps of 128 bytes (64 bf16/fp16 or 32 fp32 elements), in order;
//   * inside a step, 16-byte chunks are paired (2q, 2q+1), q = 0..3 in order, and each pair feeds
//     one v_mfma_f32_32x32x16_{bf16,f16} (lane half 0 holds chunk 2q, half 1 chunk 2q+1);
//     fp32 feeds the pair element by element (s = 0..3) to four v_mfma_f32_32x32x2_f32 (the
//     skinny entry feeds 16-bit chunk quads to v_mfma_f32_16x16x32, which returns the bits of
//     the two pair steps; gemm_skinny.h);
//   * out-of-range K is zero in both operands; rows / columns outside the problem never reach
//     the output;
//   * there is no split-K: one workgroup owns the whole K loop of its tile.
// The block tile (BM x BN), the wavefront layout and the load path (direct-to-LDS or through
// registers) only decide which elements share a workgroup and how operands reach LDS, never
// the arithmetic of an element, so they may be chosen per problem shape.
#pragma once

#include "biops_common.h"

namespace biops {

constexpr int kKBytes = 128;  // bytes of K per main-loop step

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void global_cvoid_t;

// One 32x32 output block, one chunk pair of the step (32 x 32 fp32 accumulators: 16 per lane).
template <typename T> struct Mfma;
template <> struct Mfma<bf16_t> {
  __device__ static __forceinline__ void step(f32x16_t& acc, const u32x4_t& a, const u32x4_t& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), acc, 0, 0, 0);
  }
};
template <> struct Mfma<f16_t> {
  __device__ static __forceinline__ void step(f32x16_t& acc, const u32x4_t& a, const u32x4_t& b) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), acc, 0, 0, 0);
  }
};
template <> struct Mfma<float> {
  __device__ static __forceinline__ void step(f32x16_t& acc, const u32x4_t& a, const u32x4_t& b) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a[s]), __uint_as_float(b[s]), acc,
                                                 0, 0, 0);
  }
};

// Raw bits of element e of a 16-byte chunk, and packing of elementwise loads.
template <typename T> struct Bits;
template <> struct Bits<float> {
  __device__ static __forceinline__ uint32_t get(const float* p) { return __float_as_uint(*p); }
  __device__ static __forceinline__ void put(u32x4_t& v, int e, uint32_t b) { v[e] = b; }
};
template <typename T16> struct Bits16 {
  __device__ static __forceinline__ uint32_t get(const T16* p) { return p->bits; }
  __device__ static __forceinline__ void put(u32x4_t& v, int e, uint32_t b) {
    const int d = e >> 1;
    if (e & 1) v[d] = (v[d] & 0x0000ffffu) | (b << 16);
    else v[d] = (v[d] & 0xffff0000u) | b;
  }
};
template <> struct Bits<bf16_t> : Bits16<bf16_t> {};
template <> struct Bits<f16_t> : Bits16<f16_t> {};

// Load one 16-byte chunk of `valid` (<= VEC) consecutive elements, zero beyond.
template <typename T>
__device__ __forceinline__ u32x4_t load_chunk(const T* p, int valid, bool vec_ok) {
  constexpr int VEC = 16 / sizeof(T);
  if (vec_ok && valid >= VEC) return *reinterpret_cast<const u32x4_t*>(p);
  u32x4_t v = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < VEC; ++e)
    if (e < valid) Bits<T>::put(v, e, Bits<T>::get(p + e));
  return v;
}

// Where the B operand of one tile comes from.  Logical tile column c (0..BN-1) maps to
// problem column n0 + c, or, in SwiGLU mode, to column n0/2 + (c/64)*32 + c%32 of the gate
// matrix (c/32 even) or the up matrix (c/32 odd), so that one wavefront holds gate and up
// accumulators of the same output element in adjacent 32x32 blocks.
template <typename T>
struct BSource {
  const T* p0;      // gate / plain B
  const T* p1;      // up (SwiGLU) or unused
  int64_t ld;       // K-major: stride between columns; N-major: stride between K rows
  int64_t ncols;    // valid problem columns counted from the tile origin (per source)
  bool swiglu;
  bool vec_ok;
  __device__ __forceinline__ const T* col_base(int c, int64_t& local) const {
    if (!swiglu) { local = c; return p0; }
    local = (int64_t)((c >> 6) << 5) + (c & 31);
    return ((c >> 5) & 1) ? p1 : p0;
  }
};

// SwiGLU output of one element from its gate and up accumulators, before the rounding of the
// store: round(silu(round(g))) * round(u) (the product of two rounded 16-bit values is exact in
// fp32).  Every kernel with the SwiGLU epilogue calls this one function.
template <typename T>
__device__ __forceinline__ float swiglu_value(float g_acc, float u_acc) {
  const float g = Num<T>::round(g_acc);
  const float u = Num<T>::round(u_acc);
  return Num<T>::round(g / (1.0f + expf(-g))) * u;
}

// LDS tile layout: rows of 128 bytes (one K step), unpadded; 16-byte chunk c of row r lives in
// slot c ^ ((r >> 1) & 7).  Sixteen consecutive rows reading the same chunk hit 16 distinct
// (half-row, slot) bank groups, so the MFMA operand reads (ds_read_b128) are conflict-free.
__device__ __forceinline__ int lds_off(int r, int c) { return (r << 7) + ((c ^ ((r >> 1) & 7)) << 4); }

// N-major B stage (16-bit types): K row k of the step holds the tile's CPR = BN/8 chunks of 8
// columns, chunk c at slot c ^ swz(k).  The MFMA fragments are read with the transposing
// 64-bit LDS read: within each 16-lane group, result lane i gets element i % 4 of the 64-bit
// words of source lanes 4j + i / 4 (j = 0..3), so source lane s pointing at row k0 + s / 4,
// column n0 + 4 (s % 4) hands lane i the K values k0..k0+3 of column n0 + i.  A half wavefront
// reads rows k0..k0+3 x 4 chunks; swz spreads them over 16 distinct 16-byte bank slots.
template <int CPR>
__device__ __forceinline__ int nmajor_swz(int k) {
  if constexpr (CPR >= 16) return (k & 3) << 2;
  else if constexpr (CPR == 8) return ((k >> 1) & 1) << 2;
  else return 0;
}
template <int CPR>
__device__ __forceinline__ int lds_off_n(int k, int col) {
  return k * CPR * 16 + ((((col >> 3) ^ nmajor_swz<CPR>(k))) << 4) + ((col & 7) << 1);
}
// N-major B stage (fp32): K row k holds the tile's CPR = BN/4 chunks of 4 columns, chunk c at
// slot c ^ swz32(k).  Each fragment value is one 4-byte read: lanes 0-31 read 32 consecutive
// columns of row k, lanes 32-63 the same columns of row k + 4, and swz32 puts those two rows in
// opposite 128-byte halves of the banks (for CPR >= 16: rows of 256 bytes or more).
template <int CPR>
__device__ __forceinline__ int nmajor32_swz(int k) {
  if constexpr (CPR >= 16) return ((k >> 2) & 1) << 3;
  else return 0;
}
template <int CPR>
__device__ __forceinline__ int lds_off_n32(int k, int col) {
  return k * CPR * 16 + ((((col >> 2) ^ nmajor32_swz<CPR>(k))) << 4) + ((col & 3) << 2);
}
typedef short tr16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) tr16x4_t lds_tr16x4_t;
__device__ __forceinline__ u32x2_t lds_read_tr16(const char* p) {
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_tr16x4_t*)p));
}
// The same read as inline assembly, for schedules with global->LDS (DMA) loads in flight: for
// the builtin the compiler puts a full `s_waitcnt vmcnt(0)` before every transposing read (it
// cannot rule out that the read aliases a pending DMA write), which drains the whole prefetch
// ring at every K step.  Those schedules order their reads after the DMA of the same stage by
// their own waits and barriers.  The compiler does not track the result either: the caller
// waits with lds_wait_anchor before anything reads it.
__device__ __forceinline__ u32x2_t lds_read_tr16_asm(const char* p) {
  u32x2_t r;
  const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"(a) : "memory");
  return r;
}
// Waits for every outstanding LDS operation of the wavefront; x and y count as produced here,
// so no copy of a lds_read_tr16_asm result can be placed before the wait.
__device__ __forceinline__ void lds_wait_anchor(u32x2_t& x, u32x2_t& y) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(x), "+v"(y));
}

// Block tile BM x BN computed by WGM x WGN wavefronts (each WM x WN = FM x FN 32x32 blocks);
// LW further wavefronts only issue loads (more bytes in flight per workgroup: a wavefront keeps at
// most 63 vector-memory operations outstanding).  STAGES LDS buffers form a ring.  DIRECT: operands go global -> LDS by global_load_lds_dwordx4
// (16-byte aligned rows, K a multiple of the step; B K-major, or N-major with whole 16-byte
// chunks of columns); otherwise through registers.
template <typename T, int BM, int BN, int WGM, int WGN, int STAGES, bool B_KMAJOR, bool DIRECT, int LW = 0>
struct GemmTile {
  static constexpr int THREADS = 64 * (WGM * WGN + LW);
  // This wavefront computes (wave-uniform; always true without loader wavefronts).
  __device__ static __forceinline__ bool computes() { return LW == 0 || (int)(threadIdx.x >> 6) < WGM * WGN; }
  static constexpr int VEC = 16 / (int)sizeof(T);
  static constexpr int BK = kKBytes / (int)sizeof(T);
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int FM = WM / 32, FN = WN / 32;
  typedef f32x16_t Acc;
  static constexpr int LDS_A = BM * kKBytes, LDS_B = BN * kKBytes;
  static constexpr int LDS_STAGE = LDS_A + LDS_B;
  static constexpr int LDS_BYTES = STAGES * LDS_STAGE;
  // shared memory of a kernel using this tile: the LDS ring, or the staged output tile
  static constexpr int EPI_BYTES = BM * BN * (int)sizeof(T);
  static constexpr int SMEM_BYTES = LDS_BYTES > EPI_BYTES ? LDS_BYTES : EPI_BYTES;
  // 16-byte chunk slots of one stage, and per-thread counts (last round may be partial)
  static constexpr int A_SLOTS = BM * 8, B_SLOTS = BN * 8;
  static constexpr int A_LOADS = (A_SLOTS + THREADS - 1) / THREADS;
  static constexpr int B_LOADS = (B_SLOTS + THREADS - 1) / THREADS;
  // N-major B (register path): blocks of 4 K-rows x one 16-byte chunk of columns
  static constexpr int BN_BLOCKS = (BK / 4) * (BN / VEC);
  static constexpr int BN_LOADS = (BN_BLOCKS + THREADS - 1) / THREADS;
  static constexpr int B_REGS = B_KMAJOR ? B_LOADS : 4 * BN_LOADS;
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be a multiple of 32");
  static constexpr int CPR_N = BN / VEC;  // chunks per K row of an N-major B stage
  // slot of chunk c in K row k of an N-major B stage (an involution on 0 .. CPR_N - 1)
  __device__ static __forceinline__ int nmajor_slot(int k, int c) {
    if constexpr (sizeof(T) == 4) return c ^ nmajor32_swz<CPR_N>(k);
    else return c ^ nmajor_swz<CPR_N>(k);
  }
  static_assert(!DIRECT || (A_SLOTS % THREADS == 0 && B_SLOTS % THREADS == 0), "direct split");
  static_assert(STAGES >= 2, "at least two stages");
  static constexpr int LOADS_PER_STAGE = A_LOADS + B_LOADS;  // direct path, per thread

  struct Regs {
    u32x4_t a[A_LOADS];
    u32x4_t b[B_REGS];
  };

  // ---------------------------------------------------------------- register path ----
  // Where the tile's A rows come from.  ARows: row r (clamped to rows - 1 for the direct
  // loads) at A + r * lda, addresses formed per call.  ATable: row r at A + idx[r] * lda (a
  // row table, grouped launches), with this thread's direct-load sources read from the table
  // once per tile.  at(p) is the source of direct-load slot s = t + THREADS*p at K = 0: row s/8,
  // logical chunk (s%8) ^ ((row>>1)&7).
  __device__ static __forceinline__ int slot_row(int p) { return (threadIdx.x + THREADS * p) >> 3; }
  __device__ static __forceinline__ int slot_chunk(int p) {
    const int s = threadIdx.x + THREADS * p;
    return (s & 7) ^ (((s >> 3) >> 1) & 7);
  }
  struct ARows {
    const T* A;
    int64_t lda, rows;
    __device__ __forceinline__ const T* row_ptr(int64_t r) const { return A + r * lda; }
    __device__ __forceinline__ const T* at(int p) const {
      const int r = slot_row(p);
      return row_ptr(r < rows ? r : rows - 1) + slot_chunk(p) * VEC;
    }
  };
  static constexpr int A_DIRECT = A_SLOTS / THREADS > 0 ? A_SLOTS / THREADS : 1;
  struct ATable {
    const T* A;
    int64_t lda, rows;
    const int32_t* idx;
    const T* src[A_DIRECT];
    __device__ __forceinline__ const T* row_ptr(int64_t r) const { return A + (int64_t)idx[r] * lda; }
    __device__ __forceinline__ const T* at(int p) const { return src[p]; }
  };
  __device__ static __forceinline__ ATable a_table(const T* A, int64_t lda, int64_t rows, const int32_t* idx) {
    ATable a{A, lda, rows, idx, {}};
#pragma unroll
    for (int p = 0; p < A_DIRECT; ++p) {
      const int r = slot_row(p);
      a.src[p] = a.row_ptr(r < rows ? r : rows - 1) + slot_chunk(p) * VEC;
    }
    return a;
  }

  template <class AS>
  __device__ static __forceinline__ void reg_load_a(Regs& R, const AS& as, int64_t k0, int64_t K, bool vec_ok) {
    const int t = threadIdx.x;
    const int c = t & 7;
    const int64_t kk = k0 + c * VEC;
    const int valid = (int)(K - kk < VEC ? (K - kk < 0 ? 0 : K - kk) : VEC);
#pragma unroll
    for (int p = 0; p < A_LOADS; ++p) {
      const int s = t + THREADS * p;
      const int r = s >> 3;
      if (s < A_SLOTS && r < as.rows) R.a[p] = load_chunk<T>(as.row_ptr(r) + kk, valid, vec_ok);
      else R.a[p] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }

  __device__ static __forceinline__ void reg_load_b(Regs& R, const BSource<T>& B, int64_t k0, int64_t K) {
    const int t = threadIdx.x;
    if constexpr (B_KMAJOR) {
      const int c = t & 7;
      const int64_t kk = k0 + c * VEC;
      const int valid = (int)(K - kk < VEC ? (K - kk < 0 ? 0 : K - kk) : VEC);
#pragma unroll
      for (int p = 0; p < B_LOADS; ++p) {
        const int s = t + THREADS * p;
        const int r = s >> 3;
        int64_t local;
        const T* base = B.col_base(r, local);
        if (s < B_SLOTS && local < B.ncols) R.b[p] = load_chunk<T>(base + local * B.ld + kk, valid, B.vec_ok);
        else R.b[p] = u32x4_t{0u, 0u, 0u, 0u};
      }
    } else {
      constexpr int CHUNKS = BN / VEC;
#pragma unroll
      for (int p = 0; p < BN_LOADS; ++p) {
        const int blk = t + THREADS * p;
        const int nc = blk % CHUNKS;
        const int kg = blk / CHUNKS;
        int64_t local;
        const T* base = B.col_base(nc * VEC, local);
        const int64_t nrem = B.ncols - local;
        const int valid = (int)(nrem < VEC ? (nrem < 0 ? 0 : nrem) : VEC);
#pragma unroll
        for (int kr = 0; kr < 4; ++kr) {
          const int64_t k = k0 + 4 * kg + kr;
          if (blk < BN_BLOCKS && k < K) R.b[4 * p + kr] = load_chunk<T>(base + k * B.ld + local, valid, B.vec_ok);
          else R.b[4 * p + kr] = u32x4_t{0u, 0u, 0u, 0u};
        }
      }
    }
  }

  __device__ static __forceinline__ void reg_store(char* stage, const Regs& R) {
    const int t = threadIdx.x;
    char* As = stage;
    char* Bs = stage + LDS_A;
    const int c = t & 7;
#pragma unroll
    for (int p = 0; p < A_LOADS; ++p) {
      const int s = t + THREADS * p;
      if (s < A_SLOTS) *reinterpret_cast<u32x4_t*>(As + lds_off(s >> 3, c)) = R.a[p];
    }
    if constexpr (B_KMAJOR) {
#pragma unroll
      for (int p = 0; p < B_LOADS; ++p) {
        const int s = t + THREADS * p;
        if (s < B_SLOTS) *reinterpret_cast<u32x4_t*>(Bs + lds_off(s >> 3, c)) = R.b[p];
      }
    } else {
      constexpr int CHUNKS = BN / VEC;
#pragma unroll
      for (int p = 0; p < BN_LOADS; ++p) {
        const int blk = t + THREADS * p;
        if (blk >= BN_BLOCKS) continue;
        const int nc = blk % CHUNKS;
        const int kg = blk / CHUNKS;  // K rows 4kg .. 4kg+3 of the step
        const u32x4_t* in = &R.b[4 * p];
        if constexpr (sizeof(T) == 4) {
          // 4 K-rows x 4 columns of fp32: column j gets {in[0][j], .., in[3][j]} = chunk kg.
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            u32x4_t o = {in[0][j], in[1][j], in[2][j], in[3][j]};
            *reinterpret_cast<u32x4_t*>(Bs + lds_off(nc * 4 + j, kg)) = o;
          }
        } else {
          // 4 K-rows x 8 columns of 16-bit values: column j gets 4 halves = half of chunk kg/2.
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int d = j >> 1;
            uint32_t lo, hi;
            if (j & 1) {
              lo = (in[0][d] >> 16) | (in[1][d] & 0xffff0000u);
              hi = (in[2][d] >> 16) | (in[3][d] & 0xffff0000u);
            } else {
              lo = (in[0][d] & 0x0000ffffu) | (in[1][d] << 16);
              hi = (in[2][d] & 0x0000ffffu) | (in[3][d] << 16);
            }
            u32x2_t o = {lo, hi};
            *reinterpret_cast<u32x2_t*>(Bs + lds_off(nc * 8 + j, kg >> 1) + (kg & 1) * 8) = o;
          }
        }
      }
    }
  }

  // ------------------------------------------------------------------ direct path ----
  // Slot s of the stage (s = THREADS*p + thread) is written by lane s%64 of instruction p at
  // LDS byte 16*s (row s/8, slot s%8); that slot holds logical chunk (s%8) ^ ((row>>1)&7), so
  // the lane fetches exactly that chunk.  Rows past the problem are clamped to its last row
  // (their products are never stored).
  template <class AS>
  __device__ static __forceinline__ void direct_load(char* stage, const AS& as, const BSource<T>& B,
                                                     int64_t k0) {
    const int t = threadIdx.x;
    const int wbase = __builtin_amdgcn_readfirstlane(t & ~63);  // wave-uniform: scalar LDS offsets
#pragma unroll
    for (int p = 0; p < A_SLOTS / THREADS; ++p) {
      const T* src = as.at(p) + k0;
      __builtin_amdgcn_global_load_lds((global_cvoid_t*)src,
                                       (lds_void_t*)(stage + (THREADS * p + wbase) * 16), 16, 0, 0);
    }
    char* Bs = stage + LDS_A;
    if constexpr (B_KMAJOR) {
#pragma unroll
      for (int p = 0; p < B_SLOTS / THREADS; ++p) {
        const int s = t + THREADS * p;
        const int r = s >> 3;
        const int c = (s & 7) ^ ((r >> 1) & 7);
        int64_t local;
        const T* base = B.col_base(r, local);
        if (local >= B.ncols) local = B.ncols - 1;
        const T* src = base + local * B.ld + k0 + c * VEC;
        __builtin_amdgcn_global_load_lds((global_cvoid_t*)src,
                                         (lds_void_t*)(Bs + (THREADS * p + wbase) * 16), 16, 0, 0);
      }
    } else {
      // Slot s: K row s / CPR_N, slot s % CPR_N holding chunk nmajor_slot(row, slot) of VEC
      // columns; chunks past the last column re-load the last whole chunk (never stored).
#pragma unroll
      for (int p = 0; p < B_SLOTS / THREADS; ++p) {
        const int s = t + THREADS * p;
        const int k = s / CPR_N;
        const int c = nmajor_slot(k, s % CPR_N);
        int64_t local;
        const T* base = B.col_base(c * VEC, local);
        if (local >= B.ncols) local = B.ncols - VEC;
        const T* src = base + (k0 + k) * B.ld + local;
        __builtin_amdgcn_global_load_lds((global_cvoid_t*)src,
                                         (lds_void_t*)(Bs + (THREADS * p + wbase) * 16), 16, 0, 0);
      }
    }
  }

  // ---------------------------------------------------------------------- compute ----
  __device__ static __forceinline__ void load_frags(const char* stage, int q, u32x4_t (&a)[FM], u32x4_t (&b)[FN]) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int wm = w / WGN, wn = w % WGN;
    const int lr = lane & 31, lb = lane >> 5;
#pragma unroll
    for (int i = 0; i < FM; ++i)
      a[i] = *reinterpret_cast<const u32x4_t*>(stage + lds_off(wm * WM + i * 32 + lr, 2 * q + lb));
    if constexpr (B_KMAJOR || !DIRECT) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
        b[j] = *reinterpret_cast<const u32x4_t*>(stage + LDS_A + lds_off(wn * WN + j * 32 + lr, 2 * q + lb));
    } else if constexpr (sizeof(T) == 4) {
      // fp32 N-major: value e of the fragment is K row 8q + 4lb + e (the K index the K-major
      // chunk 2q + lb holds in element e) of column wn*WN + 32j + lr
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          b[j][e] = *reinterpret_cast<const uint32_t*>(
              stage + LDS_A + lds_off_n32<CPR_N>(8 * q + 4 * lb + e, wn * WN + j * 32 + lr));
    } else {
      (void)wn;
      TrHalves h;
      issue_tr(stage, q, h);
      finish_tr(h, b);
    }
  }
  // N-major B fragments of MFMA step q through the transposing reads (inline assembly), and the
  // wait that makes them usable.
  struct TrHalves {
    u32x2_t lo[FN], hi[FN];
  };
  // Lane group g = lane / 16 holds columns 16 (g & 1) .. +15 of the block, K half g >> 1.
  __device__ static __forceinline__ void issue_tr(const char* stage, int q, TrHalves& h) {
    const int lane = threadIdx.x & 63;
    const int wn = (threadIdx.x >> 6) % WGN;
    const int g = lane >> 4, s = lane & 15;
    const int k = 16 * q + 8 * (g >> 1) + (s >> 2);
    const int cb = 16 * (g & 1) + 4 * (s & 3);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const char* base = stage + LDS_A;
      const int col = wn * WN + j * 32 + cb;
      h.lo[j] = lds_read_tr16_asm(base + lds_off_n<CPR_N>(k, col));
      h.hi[j] = lds_read_tr16_asm(base + lds_off_n<CPR_N>(k + 4, col));
    }
  }
  __device__ static __forceinline__ void finish_tr(TrHalves& h, u32x4_t (&b)[FN]) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      lds_wait_anchor(h.lo[j], h.hi[j]);
      b[j] = u32x4_t{h.lo[j][0], h.lo[j][1], h.hi[j][0], h.hi[j][1]};
    }
  }

  // K group g (0, 1) of a step = MFMA steps q = 2g, 2g+1 (64 bytes of K).
  struct Frags {
    u32x4_t a[2][FM];
    u32x4_t b[2][FN];
  };
  __device__ static __forceinline__ void load_group(const char* stage, int g, Frags& f) {
    if constexpr (DIRECT && !B_KMAJOR && sizeof(T) == 2) {
      // both steps' reads go out before the one wait
      const int lane = threadIdx.x & 63;
      const int wm = (threadIdx.x >> 6) / WGN;
      const int lr = lane & 31, lb = lane >> 5;
      TrHalves h0, h1;
#pragma unroll
      for (int i = 0; i < FM; ++i)
        f.a[0][i] = *reinterpret_cast<const u32x4_t*>(stage + lds_off(wm * WM + i * 32 + lr, 4 * g + lb));
      issue_tr(stage, 2 * g, h0);
#pragma unroll
      for (int i = 0; i < FM; ++i)
        f.a[1][i] = *reinterpret_cast<const u32x4_t*>(stage + lds_off(wm * WM + i * 32 + lr, 4 * g + 2 + lb));
      issue_tr(stage, 2 * g + 1, h1);
      finish_tr(h0, f.b[0]);
      finish_tr(h1, f.b[1]);
    } else {
      load_frags(stage, 2 * g, f.a[0], f.b[0]);
      load_frags(stage, 2 * g + 1, f.a[1], f.b[1]);
    }
  }
  __device__ static __forceinline__ void mfma_group(Acc (&acc)[FM][FN], const Frags& f) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) Mfma<T>::step(acc[i][j], f.a[h][i], f.b[h][j]);
  }

  // One K step (groups 0 then 1).  Small wave tiles read both groups' fragments before the
  // MFMAs (two buffers); large ones read one group at a time to save registers.
  static constexpr bool FRAG_DB = FM + FN <= 4;
  __device__ static __forceinline__ void compute(const char* stage, Acc (&acc)[FM][FN]) {
    if constexpr (FRAG_DB) {
      Frags f0, f1;
      load_group(stage, 0, f0);
      load_group(stage, 1, f1);
      mfma_group(acc, f0);
      mfma_group(acc, f1);
    } else {
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        Frags f;
        load_group(stage, g, f);
        mfma_group(acc, f);
        // keep the next group's fragment reads behind these MFMAs (one live fragment set)
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // Workgroup barrier that orders this thread's LDS reads/writes only: in-flight global loads
  // (the prefetch of later stages) keep running across it, which a fenced __syncthreads()
  // would drain.  Completion of the direct-to-LDS loads is tracked separately (wait_loads).
  // Written with the builtins so that the compiler knows every LDS read has landed here; with
  // the wait inside inline assembly it kept the reads pending and, once a global->LDS load was
  // issued after the barrier, waited for all LDS reads (those just issued included) before the
  // next MFMA that used an older fragment.
  __device__ static __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");  // no memory access moves across the barrier (compiler fence)
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0), vmcnt unchanged
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  // The barrier between the two MFMA groups of the pipelined schedule.  The reads it could
  // leave in flight were issued a whole MFMA group earlier, so it waits for them too (see
  // lds_barrier): the fragments the next group uses then count as landed for the compiler.
  __device__ static __forceinline__ void raw_barrier() { lds_barrier(); }

  // Waits until at most `n` direct loads of this thread are still in flight.
  template <int N>
  __device__ static __forceinline__ void wait_loads() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    // s_waitcnt: vmcnt[3:0] | expcnt[6:4]=7 | lgkmcnt[11:8]=15 | vmcnt[5:4] at [15:14]
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  }

  // Full K loop of one tile into acc (zeroed here).  The caller guarantees that no wavefront
  // reads the LDS ring on entry (a barrier separates consecutive tiles).
  template <class AS>
  __device__ static __forceinline__ void mainloop(char* smem, Acc (&acc)[FM][FN], const AS& as, bool a_vec,
                                                  const BSource<T>& B, int64_t K) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    const int64_t KT = cdiv(K, BK);
    if (KT == 0) return;
    if constexpr (DIRECT && STAGES >= 3) {
      // Software-pipelined schedule: the fragments of K group 1 of tile kt and of group 0 of
      // tile kt+1 are read from LDS while the MFMAs of the previous group run; the barrier
      // that publishes tile kt+1 sits between the two MFMA groups of tile kt.
      (void)a_vec;
      constexpr int AHEAD = STAGES - 1;  // tiles loaded ahead of the one being computed
#pragma unroll
      for (int s = 0; s < AHEAD; ++s)
        if (s < KT) direct_load(smem + s * LDS_STAGE, as, B, (int64_t)s * BK);
      if (KT - 1 >= AHEAD - 1) wait_loads<(AHEAD - 1) * LOADS_PER_STAGE>();
      else wait_loads<0>();
      lds_barrier();
      Frags f0, f1;
      const bool cw = computes();
      if (cw) load_group(smem, 0, f0);
      int cur = 0;      // stage of tile kt
      int nxt = AHEAD;  // stage of tile kt + AHEAD (== stage of tile kt - 1)
      for (int64_t kt = 0; kt < KT; ++kt) {
        const int cstage = cur;
        cur = cur + 1 == STAGES ? 0 : cur + 1;
        if (cw) {
          load_group(smem + cstage * LDS_STAGE, 1, f1);
          mfma_group(acc, f0);
        }
        if (kt + 1 < KT) {
          // tile kt+1 landed once at most min(AHEAD-2, KT-2-kt) later tiles remain in flight
          if (KT - 2 - kt >= AHEAD - 2) wait_loads<(AHEAD - 2) * LOADS_PER_STAGE>();
          else wait_loads<0>();
          // Publishes tile kt+1.  Every wave passed the MFMAs of tile kt-1 (which consumed all
          // reads of its stage), so that stage may now be refilled.
          raw_barrier();
          if (kt + AHEAD < KT)
            direct_load(smem + nxt * LDS_STAGE, as, B, (kt + AHEAD) * BK);
          if (cw) load_group(smem + cur * LDS_STAGE, 0, f0);
        }
        if (cw) mfma_group(acc, f1);
        nxt = nxt + 1 == STAGES ? 0 : nxt + 1;
      }
      lds_barrier();
    } else if constexpr (DIRECT) {
      (void)a_vec;
      constexpr int AHEAD = STAGES - 1;  // tiles in flight beyond the one being computed
#pragma unroll
      for (int s = 0; s < AHEAD; ++s)
        if (s < KT) direct_load(smem + s * LDS_STAGE, as, B, (int64_t)s * BK);
      int cur = 0;            // stage of tile kt
      int nxt = AHEAD;        // stage of tile kt + AHEAD (== stage of tile kt - 1)
      for (int64_t kt = 0; kt < KT; ++kt) {
        // tile kt landed once at most min(AHEAD-1, KT-1-kt) later tiles remain in flight
        if (KT - 1 - kt >= AHEAD - 1) wait_loads<(AHEAD - 1) * LOADS_PER_STAGE>();
        else wait_loads<0>();
        lds_barrier();  // tile kt visible to all; every wave is done with tile kt - 1
        if (kt + AHEAD < KT)
          direct_load(smem + nxt * LDS_STAGE, as, B, (kt + AHEAD) * BK);
        if (computes()) compute(smem + cur * LDS_STAGE, acc);
        cur = cur + 1 == STAGES ? 0 : cur + 1;
        nxt = nxt + 1 == STAGES ? 0 : nxt + 1;
      }
      lds_barrier();
    } else {
      Regs R;
      reg_load_a(R, as, 0, K, a_vec);
      reg_load_b(R, B, 0, K);
      reg_store(smem, R);
      lds_barrier();
      for (int64_t kt = 0; kt < KT; ++kt) {
        const int cur = (int)(kt & 1);
        const bool more = kt + 1 < KT;
        if (more) {
          reg_load_a(R, as, (kt + 1) * BK, K, a_vec);
          reg_load_b(R, B, (kt + 1) * BK, K);
        }
        if (computes()) compute(smem + cur * LDS_STAGE, acc);
        if (more) reg_store(smem + (cur ^ 1) * LDS_STAGE, R);
        lds_barrier();
      }
    }
  }

  // Epilogue.  The rounded tile is staged in LDS (row-major, 16-byte chunk k of row r stored
  // at chunk position k ^ (r & 7), masked to the chunks of a row) and written to C with
  // 16-byte stores.  SWIGLU: gate / up accumulators of one output sit in
  // blocks (i, j) / (i, j+1) of the same lane; the stored value is
  // round(round(silu(round(g))) * round(u)) and the tile is BN/2 wide.  Otherwise the value is
  // round(acc + bias[col]) (bias may be null: no add).  Ends with a barrier, so the LDS ring
  // is free for the next tile.
  template <bool SWIGLU>
  __device__ static __forceinline__ void epilogue(char* smem, Acc (&acc)[FM][FN], T* C,
                                                  int64_t ldc, int rows, int cols, const T* bias,
                                                  bool c_vec) {
    constexpr int OUTW = SWIGLU ? BN / 2 : BN;
    constexpr int PITCH = OUTW * (int)sizeof(T);
    constexpr int SWZ = OUTW / VEC >= 8 ? 7 : OUTW / VEC - 1;  // chunk swizzle stays inside the row
    static_assert(BM * PITCH <= SMEM_BYTES, "epilogue tile must fit the shared memory");
    if (computes()) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; j += (SWIGLU ? 2 : 1)) {
        const int c = acc_col(j);
        const int col = SWIGLU ? ((c >> 6) << 5) + (c & 31) : c;
        const float bv = (!SWIGLU && bias && col < cols) ? Num<T>::load(bias + col) : 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v;
          if constexpr (SWIGLU) {
            v = swiglu_value<T>(acc[i][j][r], acc[i][j + 1][r]);
          } else {
            v = bias ? acc[i][j][r] + bv : acc[i][j][r];
          }
          const int row = acc_row(i, r);
          const int pos = (((col / VEC) ^ (row & SWZ)) * VEC) + (col % VEC);
          Num<T>::store(reinterpret_cast<T*>(smem + row * PITCH) + pos, v);
        }
      }
    }
    lds_barrier();
    constexpr int CH = OUTW / VEC;
    for (int id = threadIdx.x; id < BM * CH; id += THREADS) {
      const int r = id / CH;
      const int c0 = (id - r * CH) * VEC;
      if (r >= rows || c0 >= cols) continue;
      const char* src = smem + r * PITCH + (((c0 / VEC) ^ (r & SWZ)) * 16);
      T* dst = C + (int64_t)r * ldc + c0;
      if (c_vec && c0 + VEC <= cols) {
        *reinterpret_cast<u32x4_t*>(dst) = *reinterpret_cast<const u32x4_t*>(src);
      } else {
        for (int e = 0; e < VEC && c0 + e < cols; ++e) dst[e] = reinterpret_cast<const T*>(src)[e];
      }
    }
    lds_barrier();
  }

  // Ping-pong schedule for 8 wavefronts (2 per SIMD) and a 2-stage ring: waves 0-3 (group 0)
  // and 4-7 (group 1) alternate between a load phase (the fragments of one K group, LDS ->
  // registers) and a compute phase (that group's MFMAs), group 1 one phase behind, so on every
  // SIMD one wave feeds the MFMA pipe while the other reads LDS.  With half step j = 2k + q
  // (tile k, K group q = 64 bytes of K), global phases separated by workgroup barriers are
  //   P(2j) = group 0 loads j, group 1 computes j-1;  P(2j+1) = group 0 computes j, group 1 loads j.
  // Tile k+1 goes into the other stage from P(4k) on (group 0 slots at its load of half step
  // 2k, group 1 slots at its compute of half step 2k-1) and is waited for at the end of
  // P(4k+3).  Same MFMA order per element as every other schedule.
  template <class AS>
  __device__ static __forceinline__ void mainloop_pingpong(char* smem, Acc (&acc)[FM][FN], const AS& as,
                                                           const BSource<T>& B, int64_t K) {
    static_assert(DIRECT && STAGES == 2 && THREADS == 512 && WGM == 2, "8 waves, 2 stages");
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    const int64_t KT = cdiv(K, BK);
    if (KT == 0) return;
    const bool lag = threadIdx.x >= 256;  // group 1
    direct_load(smem, as, B, 0);
    wait_loads<0>();
    lds_barrier();  // tile 0 visible
    if (lag) {
      if (KT > 1) direct_load(smem + LDS_STAGE, as, B, BK);
      lds_barrier();  // group 1 starts one phase behind
    }
    for (int64_t kt = 0; kt < KT; ++kt) {
      const char* st = smem + (int)(kt & 1) * LDS_STAGE;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        Frags f;
        // load phase
        if (!lag && q == 0 && kt + 1 < KT)
          direct_load(smem + (int)((kt + 1) & 1) * LDS_STAGE, as, B, (kt + 1) * BK);
        load_group(st, q, f);
        if (lag && q == 1) wait_loads<0>();  // group 1's slots of tile kt+1
        lds_barrier();
        // compute phase
        if (lag && q == 1 && kt + 2 < KT)
          direct_load(smem + (int)(kt & 1) * LDS_STAGE, as, B, (kt + 2) * BK);
        __builtin_amdgcn_s_setprio(1);
        mfma_group(acc, f);
        __builtin_amdgcn_s_setprio(0);
        if (!lag && q == 1) wait_loads<0>();  // group 0's slots of tile kt+1
        lds_barrier();
      }
    }
    if (!lag) lds_barrier();  // pairs with group 1's extra barrier
  }

  // Tile-local coordinates of accumulator register r (0..15) of block (i, j) for this lane:
  // the 32x32 MFMA result holds row 8*(r/4) + 4*(lane/32) + r%4, column lane%32 of its block.
  __device__ static __forceinline__ int acc_row(int i, int r) {
    const int lane = threadIdx.x & 63;
    const int wm = (threadIdx.x >> 6) / WGN;
    return wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
  }
  __device__ static __forceinline__ int acc_col(int j) {
    const int lane = threadIdx.x & 63;
    const int wn = (threadIdx.x >> 6) % WGN;
    return wn * WN + j * 32 + (lane & 31);
  }
};

// Persistent walk: workgroup g of G visits tiles g', g'+G, ... where g' spreads consecutive
// tiles over the workgroups of one XCD (workgroups are dispatched round-robin over 8 XCDs),
// so that neighbouring tiles -- which share A rows or B columns -- meet in the same L2.
__device__ __forceinline__ int64_t xcd_slot(int64_t g, int64_t G) {
  if (G % 8 != 0) return g;
  return (g % 8) * (G / 8) + g / 8;
}

// Grouped tile order inside one GEMM: 8 tile-rows form a group walked column by column.
__device__ __forceinline__ void tile_coords(int64_t t, int64_t tiles_m, int64_t tiles_n,
                                            int64_t& tm, int64_t& tn) {
  constexpr int64_t G = 8;
  const int64_t per_group = G * tiles_n;
  const int64_t group = t / per_group;
  const int64_t first = group * G;
  const int64_t gsize = (tiles_m - first) < G ? (tiles_m - first) : G;
  const int64_t in_group = t % per_group;
  tm = first + in_group % gsize;
  tn = in_group / gsize;
}

}  // namespace biops
