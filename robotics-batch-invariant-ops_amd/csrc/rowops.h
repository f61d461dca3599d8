// Row-reduction building blocks shared by softmax, attention and the mean / L2 reductions.
//
// Reduction tree (the batch-invariance contract of every row operation here): a row of C
// elements is cut into 16-byte chunks of VEC input elements; lane L of the wavefront owning the
// row takes chunks L, L+64, L+128, ... and adds their elements in increasing column order into
// one fp32 partial; the 64 partials are then combined by the xor butterfly (offsets 32, 16, 8,
// 4, 2, 1).  Because fp32 addition is commutative, every lane ends with the same bits, and the
// tree depends only on C and VEC (the input element size) -- not on the number of rows, the
// row's position, or whether the row was read once (kept in registers) or several times.
#pragma once

#include <type_traits>

#include "biops_common.h"

namespace biops {

constexpr int kRowWaves = 4;      // rows (wavefronts) per 256-thread workgroup
constexpr int kRowRegChunks = 4;  // chunks per lane kept in registers (one HBM read when it fits)

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Chunk of VEC consecutive elements starting at column c0 of a contiguous row of `cols`
// elements, as fp32; elements past the row end read as `fill`.
template <typename T>
__device__ __forceinline__ void load_row_chunk(const T* row, int64_t cols, int64_t c0, bool vec_ok,
                                               float fill, float (&v)[16 / sizeof(T)]) {
  constexpr int VEC = 16 / sizeof(T);
  if (vec_ok && c0 + VEC <= cols) {
    const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(row + c0);
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(raw[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = Num<T>::from_bits((raw[e >> 1] >> (16 * (e & 1))) & 0xffffu);
    }
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] = (c0 + e < cols) ? Num<T>::load(row + c0 + e) : fill;
  }
}

// Store N fp32 values at columns c0 .. c0+N-1 of a contiguous row (columns >= cols skipped).
// vec_ok promises the row start is 16-byte aligned.  NT marks the vector stores non-temporal
// (streaming outputs nobody reads back soon: measured 6-10 % faster for the softmax rows).
template <typename V>
__device__ __forceinline__ void vstore(V* p, const V& v, bool nt) {
  if (nt) __builtin_nontemporal_store(v, p);
  else *p = v;
}
template <typename T, int N, bool NT = false>
__device__ __forceinline__ void store_row_chunk(T* row, int64_t cols, int64_t c0, bool vec_ok,
                                                const float (&v)[N]) {
  if (vec_ok && c0 + N <= cols) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int h = 0; h < N / 4; ++h) {
        f32x4_t o = {v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
        vstore(reinterpret_cast<f32x4_t*>(row + c0 + 4 * h), o, NT);
      }
      return;
    } else {
      uint32_t w[N / 2];
#pragma unroll
      for (int d = 0; d < N / 2; ++d) {
        if constexpr (std::is_same<T, bf16_t>::value)
          w[d] = f32x2_to_bf16x2_bits(v[2 * d], v[2 * d + 1]);
        else
          w[d] = (uint32_t)Num<T>::to_bits(v[2 * d]) | ((uint32_t)Num<T>::to_bits(v[2 * d + 1]) << 16);
      }
      if constexpr (N == 8) {
        u32x4_t o = {w[0], w[1], w[2], w[3]};
        vstore(reinterpret_cast<u32x4_t*>(row + c0), o, NT);
      } else {
        u32x2_t o = {w[0], w[1]};
        vstore(reinterpret_cast<u32x2_t*>(row + c0), o, NT);
      }
      return;
    }
  }
#pragma unroll
  for (int e = 0; e < N; ++e)
    if (c0 + e < cols) Num<T>::store(row + c0 + e, v[e]);
}

// exp(x - shift) for the softmax family: the accurate libm expf when the result is stored as
// fp32; when it is rounded to 16 bits anyway, the hardware exp2 of fma(x, log2 e, -shift log2 e)
// (`shl2e` = shift * log2 e, computed once per row).
constexpr float kLog2e = 1.4426950408889634f;
template <typename Tout>
__device__ __forceinline__ float soft_exp(float x, float shift, float shl2e) {
  if constexpr (sizeof(Tout) == 4) return expf(x - shift);
  else return __builtin_amdgcn_exp2f(__builtin_fmaf(x, kLog2e, -shl2e));
}

// ------------------------------------------------------------------ softmax rows ----
// Row transform applied while loading scores (attention only): scale with the rounding of the
// score dtype, then causal / boolean masking to -inf or an additive mask with rounding.
struct AttnRow {
  float scale;
  int64_t col_limit;   // columns >= col_limit are causally masked (cols when not causal)
  const void* mask;    // row base of the mask (nullptr: none)
  int64_t mask_stride; // element stride between mask columns
  int mask_kind;       // 0 none, 1 bool, 2 additive (same dtype as the scores)
};

enum { kSoftmax = 0, kLogSoftmax = 1, kAttn = 2 };

template <typename Tin, int MODE>
__device__ __forceinline__ void transform_chunk(const AttnRow& ar, int64_t c0, int64_t cols,
                                                float (&v)[16 / sizeof(Tin)]) {
  if constexpr (MODE == kAttn) {
    constexpr int VEC = 16 / sizeof(Tin);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const int64_t c = c0 + e;
      if (c >= cols) { v[e] = -INFINITY; continue; }
      float s = Num<Tin>::round(v[e] * ar.scale);
      if (c >= ar.col_limit) {
        s = -INFINITY;
      } else if (ar.mask_kind == 1) {
        if (!reinterpret_cast<const uint8_t*>(ar.mask)[c * ar.mask_stride]) s = -INFINITY;
      } else if (ar.mask_kind == 2) {
        s = Num<Tin>::round(s + Num<Tin>::load(reinterpret_cast<const Tin*>(ar.mask) + c * ar.mask_stride));
      }
      v[e] = s;
    }
  }
}

// Softmax / log-softmax of one row by one wavefront.  Reference semantics
// (batch_invariant_ops.py:1074-1114, 974-1034): m = max; softmax = exp(x-m)/sum exp(x-m), with
// an all -inf row giving 0; log_softmax = x - m - log(sum exp(x-m)).
template <typename Tin, typename Tout, int MODE>
__device__ __forceinline__ void softmax_row(const Tin* in, Tout* out, int64_t cols, bool vin,
                                            bool vout, const AttnRow& ar) {
  constexpr int VEC = 16 / sizeof(Tin);
  const int lane = threadIdx.x & 63;
  const int64_t nchunks = cdiv(cols, VEC);
  const bool fits = nchunks <= 64 * kRowRegChunks;
  float cache[kRowRegChunks][VEC];

  float mx = -INFINITY;
  if (fits) {
#pragma unroll
    for (int j = 0; j < kRowRegChunks; ++j) {
      const int64_t ci = lane + 64 * j;
      if (ci < nchunks) {
        load_row_chunk<Tin>(in, cols, ci * VEC, vin, -INFINITY, cache[j]);
        transform_chunk<Tin, MODE>(ar, ci * VEC, cols, cache[j]);
#pragma unroll
        for (int e = 0; e < VEC; ++e) mx = fmaxf(mx, cache[j][e]);
      }
    }
  } else {
    for (int64_t ci = lane; ci < nchunks; ci += 64) {
      float v[VEC];
      load_row_chunk<Tin>(in, cols, ci * VEC, vin, -INFINITY, v);
      transform_chunk<Tin, MODE>(ar, ci * VEC, cols, v);
#pragma unroll
      for (int e = 0; e < VEC; ++e) mx = fmaxf(mx, v[e]);
    }
  }
  mx = wave_max(mx);
  const bool all_neg_inf = (mx == -INFINITY);
  const float shift = (MODE == kLogSoftmax || !all_neg_inf) ? mx : 0.f;
  const float shl2e = shift * kLog2e;

  float sum = 0.f;
  if (fits) {
#pragma unroll
    for (int j = 0; j < kRowRegChunks; ++j) {
      const int64_t ci = lane + 64 * j;
      if (ci < nchunks) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float ex = (MODE != kLogSoftmax && all_neg_inf) ? 0.f : soft_exp<Tout>(cache[j][e], shift, shl2e);
          if (MODE != kLogSoftmax) cache[j][e] = ex;
          if (ci * VEC + e < cols) sum += ex;
        }
      }
    }
  } else {
    for (int64_t ci = lane; ci < nchunks; ci += 64) {
      float v[VEC];
      load_row_chunk<Tin>(in, cols, ci * VEC, vin, -INFINITY, v);
      transform_chunk<Tin, MODE>(ar, ci * VEC, cols, v);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float ex = (MODE != kLogSoftmax && all_neg_inf) ? 0.f : soft_exp<Tout>(v[e], shift, shl2e);
        if (ci * VEC + e < cols) sum += ex;
      }
    }
  }
  sum = wave_sum(sum);

  if (MODE == kLogSoftmax) {
    const float lse = logf(sum);
    auto emit = [&](int64_t ci, float (&v)[VEC]) {
      float o[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = v[e] - mx - lse;
      store_row_chunk<Tout, VEC>(out, cols, ci * VEC, vout, o);
    };
    if (fits) {
#pragma unroll
      for (int j = 0; j < kRowRegChunks; ++j) {
        const int64_t ci = lane + 64 * j;
        if (ci < nchunks) emit(ci, cache[j]);
      }
    } else {
      for (int64_t ci = lane; ci < nchunks; ci += 64) {
        float v[VEC];
        load_row_chunk<Tin>(in, cols, ci * VEC, vin, -INFINITY, v);
        emit(ci, v);
      }
    }
  } else {
    const bool zero = (sum == 0.f);
    const float inv = zero ? 0.f : 1.0f / sum;
    if (fits) {
#pragma unroll
      for (int j = 0; j < kRowRegChunks; ++j) {
        const int64_t ci = lane + 64 * j;
        if (ci < nchunks) {
          float o[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) o[e] = zero ? 0.f : cache[j][e] * inv;
          store_row_chunk<Tout, VEC>(out, cols, ci * VEC, vout, o);
        }
      }
    } else {
      for (int64_t ci = lane; ci < nchunks; ci += 64) {
        float v[VEC];
        load_row_chunk<Tin>(in, cols, ci * VEC, vin, -INFINITY, v);
        transform_chunk<Tin, MODE>(ar, ci * VEC, cols, v);
        float o[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          o[e] = zero ? 0.f : (all_neg_inf ? 0.f : soft_exp<Tout>(v[e], shift, shl2e)) * inv;
        store_row_chunk<Tout, VEC>(out, cols, ci * VEC, vout, o);
      }
    }
  }
}

// Softmax / log-softmax of R rows (row r at in + r*ld_in) by one wavefront when a row has at
// most 64*NC chunks (NC <= kRowRegChunks): the loads of all R rows are issued before the first
// reduction, so a wavefront keeps R*NC chunks per lane in flight.  Per row, the arithmetic and
// reduction order are those of softmax_row.  Rows r >= nrows are skipped.
template <typename Tin, typename Tout, int MODE, int R, int NC>
__device__ __forceinline__ void softmax_rows_fit(const Tin* in, int64_t ld_in, Tout* out, int64_t ld_out,
                                                 int nrows, int64_t cols, bool vin, bool vout) {
  static_assert(MODE != kAttn, "plain rows only");
  static_assert(NC <= kRowRegChunks, "register cache");
  constexpr int VEC = 16 / sizeof(Tin);
  const int lane = threadIdx.x & 63;
  const int64_t nchunks = cdiv(cols, VEC);
  float cache[R][NC][VEC];
  // rows past nrows are treated as all -inf and never stored
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int64_t ci = lane + 64 * j;
      if (r < nrows && ci < nchunks) {
        load_row_chunk<Tin>(in + r * ld_in, cols, ci * VEC, vin, -INFINITY, cache[r][j]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) cache[r][j][e] = -INFINITY;
      }
    }
  }
  // The butterflies of the R rows run step by step together (independent shuffles overlap).
  float mx[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    mx[r] = -INFINITY;
#pragma unroll
    for (int j = 0; j < NC; ++j)
#pragma unroll
      for (int e = 0; e < VEC; ++e) mx[r] = fmaxf(mx[r], cache[r][j][e]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
    for (int r = 0; r < R; ++r) mx[r] = fmaxf(mx[r], __shfl_xor(mx[r], off, 64));
  float sum[R];
  bool neg_inf[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    neg_inf[r] = (mx[r] == -INFINITY);
    const float shift = (MODE == kLogSoftmax || !neg_inf[r]) ? mx[r] : 0.f;
    const float shl2e = shift * kLog2e;
    sum[r] = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int64_t ci = lane + 64 * j;
      if (ci < nchunks) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float ex = (MODE != kLogSoftmax && neg_inf[r]) ? 0.f : soft_exp<Tout>(cache[r][j][e], shift, shl2e);
          if (MODE != kLogSoftmax) cache[r][j][e] = ex;
          if (ci * VEC + e < cols) sum[r] += ex;
        }
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
    for (int r = 0; r < R; ++r) sum[r] += __shfl_xor(sum[r], off, 64);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (r >= nrows) continue;
    Tout* orow = out + r * ld_out;
    if (MODE == kLogSoftmax) {
      const float lse = logf(sum[r]);
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int64_t ci = lane + 64 * j;
        if (ci < nchunks) {
          float o[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) o[e] = cache[r][j][e] - mx[r] - lse;
          store_row_chunk<Tout, VEC, true>(orow, cols, ci * VEC, vout, o);
        }
      }
    } else {
      const bool zero = (sum[r] == 0.f);
      const float inv = zero ? 0.f : 1.0f / sum[r];
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int64_t ci = lane + 64 * j;
        if (ci < nchunks) {
          float o[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) o[e] = zero ? 0.f : cache[r][j][e] * inv;
          store_row_chunk<Tout, VEC, true>(orow, cols, ci * VEC, vout, o);
        }
      }
    }
  }
}

}  // namespace biops
