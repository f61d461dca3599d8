// Fixed-schedule MFMA GEMM tile for gfx950 (CDNA4), shared by GEMM, BMM, grouped GEMM
// (varlen attention) and the MoE expert GEMMs.
//
// Batch-invariance rule: every output element C[m,n] is produced by the same sequence of MFMA
// instructions over the same K chunks, in the same order, whatever M, the batch size or the
// tile the element falls in:
//   * K is consumed in fixed steps of 128 bytes (64 bf16/fp16 or 32 fp32 elements), in order;
//   * inside a step, 16-byte chunks are paired (2q, 2q+1) and fed to one MFMA per pair
//     (bf16/fp16: v_mfma_f32_32x32x16_{bf16,f16}); fp32 feeds the chunk pair element by element
//     to four v_mfma_f32_32x32x2_f32;
//   * out-of-range K is zero-filled in both operands, out-of-range rows/columns are zero-filled
//     and never stored;
//   * there is no split-K: one workgroup owns the whole K loop of its tile.
// The block tile (BM x BN) only decides which elements share a workgroup, not how any element
// is computed, so it may be chosen from (dtype, N, K) without breaking invariance.
#pragma once

#include "biops_common.h"

namespace biops {

constexpr int kGemmThreads = 256;  // 4 wavefronts in a 2 x 2 arrangement
constexpr int kKBytes = 128;       // bytes of K per main-loop step
constexpr int kLdsRow = 144;       // LDS row pitch: 128 B of K + 16 B pad (conflict-free b128 reads)

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

// Load one 16-byte chunk of `count_valid` (<= VEC) consecutive elements, zero beyond.
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
// accumulators of the same output element.
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

template <typename T, int BM, int BN, bool B_KMAJOR>
struct GemmTile {
  static constexpr int VEC = 16 / (int)sizeof(T);
  static constexpr int BK = kKBytes / (int)sizeof(T);
  static constexpr int WM = BM / 2, WN = BN / 2;
  static constexpr int FM = WM / 32, FN = WN / 32;
  static constexpr int LDS_A = BM * kLdsRow, LDS_B = BN * kLdsRow;
  static constexpr int LDS_STAGE = LDS_A + LDS_B;
  static constexpr int LDS_BYTES = 2 * LDS_STAGE;
  static constexpr int A_LOADS = BM / 32;  // 16-byte chunks per thread for the A tile
  // B tile, K-major: BN rows of 8 chunks.  N-major: blocks of 4 K-rows x one 16-byte chunk.
  static constexpr int B_LOADS_K = BN / 32;
  static constexpr int B_BLOCKS_N = (BK / 4) * (BN / VEC) / kGemmThreads;
  static_assert(BM % 64 == 0 && BN % 64 == 0, "tile must be a multiple of 64");
  static_assert((BK / 4) * (BN / VEC) % kGemmThreads == 0, "N-major B tile split");

  struct Regs {
    u32x4_t a[A_LOADS];
    u32x4_t b[B_KMAJOR ? B_LOADS_K : 4 * B_BLOCKS_N];
  };

  // A tile: rows [0, rows) valid (row r at A + r*lda), K columns [k0, K).
  __device__ static __forceinline__ void load_a(Regs& R, const T* A, int64_t lda, int64_t rows,
                                                int64_t k0, int64_t K, bool vec_ok) {
    const int t = threadIdx.x;
    const int c = t & 7;
    const int64_t kk = k0 + c * VEC;
    const int valid = (int)(K - kk < VEC ? (K - kk < 0 ? 0 : K - kk) : VEC);
#pragma unroll
    for (int p = 0; p < A_LOADS; ++p) {
      const int r = (t >> 3) + 32 * p;
      if (r < rows) R.a[p] = load_chunk<T>(A + (int64_t)r * lda + kk, valid, vec_ok);
      else R.a[p] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }

  __device__ static __forceinline__ void load_b(Regs& R, const BSource<T>& B, int64_t k0, int64_t K) {
    const int t = threadIdx.x;
    if constexpr (B_KMAJOR) {
      const int c = t & 7;
      const int64_t kk = k0 + c * VEC;
      const int valid = (int)(K - kk < VEC ? (K - kk < 0 ? 0 : K - kk) : VEC);
#pragma unroll
      for (int p = 0; p < B_LOADS_K; ++p) {
        const int r = (t >> 3) + 32 * p;
        int64_t local;
        const T* base = B.col_base(r, local);
        if (local < B.ncols) R.b[p] = load_chunk<T>(base + local * B.ld + kk, valid, B.vec_ok);
        else R.b[p] = u32x4_t{0u, 0u, 0u, 0u};
      }
    } else {
      constexpr int CHUNKS = BN / VEC;
#pragma unroll
      for (int p = 0; p < B_BLOCKS_N; ++p) {
        const int blk = t + kGemmThreads * p;
        const int nc = blk % CHUNKS;
        const int kg = blk / CHUNKS;
        int64_t local;
        const T* base = B.col_base(nc * VEC, local);
        const int64_t nrem = B.ncols - local;
        const int valid = (int)(nrem < VEC ? (nrem < 0 ? 0 : nrem) : VEC);
#pragma unroll
        for (int kr = 0; kr < 4; ++kr) {
          const int64_t k = k0 + 4 * kg + kr;
          if (k < K) R.b[4 * p + kr] = load_chunk<T>(base + k * B.ld + local, valid, B.vec_ok);
          else R.b[4 * p + kr] = u32x4_t{0u, 0u, 0u, 0u};
        }
      }
    }
  }

  __device__ static __forceinline__ void store_lds(char* stage, const Regs& R) {
    const int t = threadIdx.x;
    char* As = stage;
    char* Bs = stage + LDS_A;
    {
      const int c = t & 7;
#pragma unroll
      for (int p = 0; p < A_LOADS; ++p) {
        const int r = (t >> 3) + 32 * p;
        *reinterpret_cast<u32x4_t*>(As + r * kLdsRow + c * 16) = R.a[p];
      }
    }
    if constexpr (B_KMAJOR) {
      const int c = t & 7;
#pragma unroll
      for (int p = 0; p < B_LOADS_K; ++p) {
        const int r = (t >> 3) + 32 * p;
        *reinterpret_cast<u32x4_t*>(Bs + r * kLdsRow + c * 16) = R.b[p];
      }
    } else {
      constexpr int CHUNKS = BN / VEC;
#pragma unroll
      for (int p = 0; p < B_BLOCKS_N; ++p) {
        const int blk = t + kGemmThreads * p;
        const int nc = blk % CHUNKS;
        const int kg = blk / CHUNKS;
        const u32x4_t* in = &R.b[4 * p];
        if constexpr (sizeof(T) == 4) {
          // 4 K-rows x 4 columns of fp32: column j gets {in[0][j], .., in[3][j]}.
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            u32x4_t o = {in[0][j], in[1][j], in[2][j], in[3][j]};
            *reinterpret_cast<u32x4_t*>(Bs + (nc * 4 + j) * kLdsRow + kg * 16) = o;
          }
        } else {
          // 4 K-rows x 8 columns of 16-bit values: column j gets 4 halves (8 bytes).
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
            *reinterpret_cast<u32x2_t*>(Bs + (nc * 8 + j) * kLdsRow + kg * 8) = o;
          }
        }
      }
    }
  }

  __device__ static __forceinline__ void compute(const char* stage, f32x16_t (&acc)[FM][FN]) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int wm = w >> 1, wn = w & 1;
    const int lr = lane & 31, lb = lane >> 5;
    const char* As = stage + (wm * WM + lr) * kLdsRow + lb * 16;
    const char* Bs = stage + LDS_A + (wn * WN + lr) * kLdsRow + lb * 16;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      u32x4_t a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        a[i] = *reinterpret_cast<const u32x4_t*>(As + i * 32 * kLdsRow + q * 32);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        b[j] = *reinterpret_cast<const u32x4_t*>(Bs + j * 32 * kLdsRow + q * 32);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) Mfma<T>::step(acc[i][j], a[i], b[j]);
    }
  }

  // Full K loop of one tile into acc (zeroed here).  The caller guarantees that the LDS is not
  // being read by another wavefront on entry (a barrier separates consecutive tiles).
  __device__ static __forceinline__ void mainloop(char* smem, f32x16_t (&acc)[FM][FN],
                                                  const T* A, int64_t lda, int64_t rows, bool a_vec,
                                                  const BSource<T>& B, int64_t K) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    const int64_t KT = cdiv(K, BK);
    if (KT == 0) return;
    Regs R;
    load_a(R, A, lda, rows, 0, K, a_vec);
    load_b(R, B, 0, K);
    store_lds(smem, R);
    __syncthreads();
    for (int64_t kt = 0; kt < KT; ++kt) {
      const int cur = (int)(kt & 1);
      const bool more = kt + 1 < KT;
      if (more) {
        load_a(R, A, lda, rows, (kt + 1) * BK, K, a_vec);
        load_b(R, B, (kt + 1) * BK, K);
      }
      compute(smem + cur * LDS_STAGE, acc);
      if (more) store_lds(smem + (cur ^ 1) * LDS_STAGE, R);
      __syncthreads();
    }
  }

  // Tile-local coordinates of accumulator register r of block (i, j) for this lane.
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
