// Softmax / log-softmax and mean / L2-norm reductions.
#include <type_traits>

#include "rowops.h"

namespace biops {

// ------------------------------------------------------------------ softmax ----
struct SoftmaxArgs {
  const void* in;
  void* out;
  int64_t rows, cols, ld_in, ld_out;
  int32_t vin, vout;
};

// One wavefront per row for long rows.  Rows of at most 64*NC chunks (NC = 1, 2, 4 per lane):
// fit_rows<NC>() rows per wavefront, whose loads are all issued before the first reduction,
// with non-temporal output stores.  Same arithmetic per row either way.
template <typename Tin, typename Tout, int MODE>
__global__ __launch_bounds__(256) void softmax_kernel(SoftmaxArgs a) {
  const int64_t r = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  if (r >= a.rows) return;
  AttnRow ar{1.f, a.cols, nullptr, 0, 0};
  softmax_row<Tin, Tout, MODE>(reinterpret_cast<const Tin*>(a.in) + r * a.ld_in,
                               reinterpret_cast<Tout*>(a.out) + r * a.ld_out, a.cols, a.vin != 0,
                               a.vout != 0, ar);
}

// Rows per wavefront R for rows of NC chunks per lane: two rows of one chunk, else one row
// (measured on 512 MiB of bf16 rows: more rows per wavefront left fewer wavefronts in flight).
template <int NC>
constexpr int fit_rows() { return NC == 1 ? 2 : 1; }

template <typename Tin, typename Tout, int MODE, int NC>
__global__ __launch_bounds__(256) void softmax_fit_kernel(SoftmaxArgs a) {
  constexpr int R = fit_rows<NC>();
  const int64_t r = ((int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6)) * R;
  if (r >= a.rows) return;
  const int n = a.rows - r < R ? (int)(a.rows - r) : R;
  softmax_rows_fit<Tin, Tout, MODE, R, NC>(reinterpret_cast<const Tin*>(a.in) + r * a.ld_in, a.ld_in,
                                           reinterpret_cast<Tout*>(a.out) + r * a.ld_out, a.ld_out, n,
                                           a.cols, a.vin != 0, a.vout != 0);
}

template <typename Tin, typename Tout, int NC>
static int launch_softmax_fit(const SoftmaxArgs& a, int is_log, hipStream_t s) {
  const int64_t blocks = cdiv(a.rows, kRowWaves * fit_rows<NC>());
  if (blocks > 0x7fffffffLL) return fail(BIOPS_ERR_ARG, "too many rows");
  if (is_log)
    hipLaunchKernelGGL((softmax_fit_kernel<Tin, Tout, kLogSoftmax, NC>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((softmax_fit_kernel<Tin, Tout, kSoftmax, NC>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_launch("softmax_fit_kernel");
}

template <typename Tin, typename Tout>
static int launch_softmax(const SoftmaxArgs& a, int is_log, hipStream_t s) {
  constexpr int VEC = 16 / (int)sizeof(Tin);
  const int64_t nchunks = cdiv(a.cols, VEC);
  if (nchunks <= 64) return launch_softmax_fit<Tin, Tout, 1>(a, is_log, s);
  if (nchunks <= 128) return launch_softmax_fit<Tin, Tout, 2>(a, is_log, s);
  if (nchunks <= 256) return launch_softmax_fit<Tin, Tout, 4>(a, is_log, s);
  const int64_t blocks = cdiv(a.rows, kRowWaves);
  if (blocks > 0x7fffffffLL) return fail(BIOPS_ERR_ARG, "too many rows");
  if (is_log)
    hipLaunchKernelGGL((softmax_kernel<Tin, Tout, kLogSoftmax>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((softmax_kernel<Tin, Tout, kSoftmax>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_launch("softmax_kernel");
}

// ------------------------------------------------------------------ reductions ----
// Contiguous rows (K == 1).  Rows of up to kWaveRowMax elements: one wavefront per row with the
// tree described in rowops.h.  Longer rows: one 256-thread workgroup per row -- lane L of 256
// takes chunks L, L+256, ...; each wavefront butterflies its 64 partials and the four wavefront
// sums are added as (w0 + w1) + (w2 + w3).  The choice depends on N only; rows of up to 512
// aligned 16-byte chunks go to reduce_rows_fit, which gives reduce_rows_wave's bits.
constexpr int64_t kWaveRowMax = 65536;

struct ReduceArgs {
  const void* in;
  void* out;
  int64_t M, N, K, sM, sN, sK;
  int32_t vin;   // contiguous rows are 16-byte aligned
  int32_t kvec;  // K > 1: k contiguous and every (m, n) row start 16-byte aligned
};

template <int OP>
__device__ __forceinline__ float reduce_add(float acc, float x) {
  // L2: acc + x * x with one rounding (a fused multiply-add), written out so that the compiler's
  // contraction choices (which product to fuse next to a known-zero accumulator) cannot differ
  // between the kernels below
  return OP == BIOPS_REDUCE_L2 ? __builtin_fmaf(x, x, acc) : acc + x;
}
template <int OP>
__device__ __forceinline__ float reduce_final(float s, int64_t n) {
  return OP == BIOPS_REDUCE_L2 ? sqrtf(s) : s / (float)n;
}

template <typename Tin, typename Tout, int OP>
__global__ __launch_bounds__(256) void reduce_rows_wave(ReduceArgs a) {
  constexpr int VEC = 16 / sizeof(Tin);
  const int64_t r = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  if (r >= a.M) return;
  const int lane = threadIdx.x & 63;
  const Tin* row = reinterpret_cast<const Tin*>(a.in) + r * a.sM;
  const int64_t nchunks = cdiv(a.N, VEC);
  float acc = 0.f;
  for (int64_t ci = lane; ci < nchunks; ci += 64) {
    float v[VEC];
    load_row_chunk<Tin>(row, a.N, ci * VEC, a.vin != 0, 0.f, v);
#pragma unroll
    for (int e = 0; e < VEC; ++e)
      if (ci * VEC + e < a.N) acc = reduce_add<OP>(acc, v[e]);
  }
  acc = wave_sum(acc);
  if (lane == 0) Num<Tout>::store(reinterpret_cast<Tout*>(a.out) + r, reduce_final<OP>(acc, a.N));
}

// reduce_rows_wave for rows of whole 16-byte chunks, at most 64 NC of them: the NC loads of a
// lane are issued together, then added in the same order as reduce_rows_wave adds them (chunk
// lane, lane + 64, ..., elements in order), so the bits are the same.  Measured on MI355X
// ([8192, 2048] bf16, inputs streamed from HBM): 9.0 -> 7.4 us per call; two, four or eight rows
// per wavefront, or workgroups of 2 to 16 wavefronts, measured no faster.
template <typename Tin, typename Tout, int OP, int NC>
__global__ __launch_bounds__(256) void reduce_rows_fit(ReduceArgs a) {
  constexpr int VEC = 16 / sizeof(Tin);
  const int64_t r = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  if (r >= a.M) return;
  const int lane = threadIdx.x & 63;
  const Tin* row = reinterpret_cast<const Tin*>(a.in) + r * a.sM;
  const int nchunks = (int)(a.N / VEC);
  u32x4_t raw[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int ci = lane + 64 * j;
    raw[j] = ci < nchunks ? *reinterpret_cast<const u32x4_t*>(row + (int64_t)ci * VEC) : u32x4_t{0u, 0u, 0u, 0u};
  }
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    if (lane + 64 * j < nchunks) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float x;
        if constexpr (sizeof(Tin) == 4) x = __uint_as_float(raw[j][e]);
        else x = Num<Tin>::from_bits((raw[j][e >> 1] >> (16 * (e & 1))) & 0xffffu);
        acc = reduce_add<OP>(acc, x);
      }
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) Num<Tout>::store(reinterpret_cast<Tout*>(a.out) + r, reduce_final<OP>(acc, a.N));
}

template <typename Tin, typename Tout, int OP>
__global__ __launch_bounds__(256) void reduce_rows_block(ReduceArgs a) {
  constexpr int VEC = 16 / sizeof(Tin);
  __shared__ float part[4];
  const int64_t r = blockIdx.x;
  const int t = threadIdx.x;
  const Tin* row = reinterpret_cast<const Tin*>(a.in) + r * a.sM;
  const int64_t nchunks = cdiv(a.N, VEC);
  float acc = 0.f;
  for (int64_t ci = t; ci < nchunks; ci += 256) {
    float v[VEC];
    load_row_chunk<Tin>(row, a.N, ci * VEC, a.vin != 0, 0.f, v);
#pragma unroll
    for (int e = 0; e < VEC; ++e)
      if (ci * VEC + e < a.N) acc = reduce_add<OP>(acc, v[e]);
  }
  acc = wave_sum(acc);
  if ((t & 63) == 0) part[t >> 6] = acc;
  __syncthreads();
  if (t == 0) {
    const float s = (part[0] + part[1]) + (part[2] + part[3]);
    Num<Tout>::store(reinterpret_cast<Tout*>(a.out) + r, reduce_final<OP>(s, a.N));
  }
}

// Strided reduction (K > 1): a workgroup owns 64*VK consecutive k of one m (VK consecutive k
// per lane: 16 bytes when the k run is contiguous and aligned, else 1); wavefront w adds the
// elements n = w, w+4, w+8, ... of each of its columns in increasing n, and the four partials
// are added as (p0 + p1) + (p2 + p3).  Depends on N only (VK only decides how columns are
// grouped into loads).  The loads of kUnroll consecutive n of a wavefront are issued before
// their additions, which still happen in increasing n.
constexpr int kStridedUnroll = 8;

template <typename Tin, int VK>
__device__ __forceinline__ void load_k_run(const Tin* p, int64_t sK, int valid, float (&v)[VK]) {
  if constexpr (VK > 1) {
    if (valid >= VK) {
      const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(p);
      if constexpr (sizeof(Tin) == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(raw[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = Num<Tin>::from_bits((raw[e >> 1] >> (16 * (e & 1))) & 0xffffu);
      }
      return;
    }
  }
#pragma unroll
  for (int e = 0; e < VK; ++e) v[e] = e < valid ? Num<Tin>::load(p + e * sK) : 0.f;
}

template <typename Tin, typename Tout, int OP, int VK>
__global__ __launch_bounds__(256) void reduce_strided(ReduceArgs a) {
  __shared__ float part[4][64 * VK];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t kblocks = cdiv(a.K, 64 * VK);
  const int64_t m = blockIdx.x / kblocks;
  const int64_t k0 = (blockIdx.x - m * kblocks) * 64 * VK + (int64_t)lane * VK;
  const int valid = k0 < a.K ? (int)(a.K - k0 < VK ? a.K - k0 : VK) : 0;
  float acc[VK];
#pragma unroll
  for (int e = 0; e < VK; ++e) acc[e] = 0.f;
  // Lanes with a whole k run take a branch-free loop (its loads stay in flight together); the
  // lanes of a partial run (last workgroup of a row only) take the element-wise one.
  auto run = [&](auto whole) {
    constexpr bool WHOLE = decltype(whole)::value;
    const int nv = WHOLE ? VK : valid;
    const Tin* base = reinterpret_cast<const Tin*>(a.in) + m * a.sM + k0 * a.sK;
    int64_t n = w;
    for (; n + 4 * (kStridedUnroll - 1) < a.N; n += 4 * kStridedUnroll) {
      float v[kStridedUnroll][VK];
#pragma unroll
      for (int u = 0; u < kStridedUnroll; ++u) load_k_run<Tin, VK>(base + (n + 4 * u) * a.sN, a.sK, nv, v[u]);
#pragma unroll
      for (int u = 0; u < kStridedUnroll; ++u)
#pragma unroll
        for (int e = 0; e < VK; ++e) acc[e] = reduce_add<OP>(acc[e], v[u][e]);
    }
    for (; n < a.N; n += 4) {
      float v[VK];
      load_k_run<Tin, VK>(base + n * a.sN, a.sK, nv, v);
#pragma unroll
      for (int e = 0; e < VK; ++e) acc[e] = reduce_add<OP>(acc[e], v[e]);
    }
  };
  if (valid == VK) run(std::true_type{});
  else if (valid > 0) run(std::false_type{});
#pragma unroll
  for (int e = 0; e < VK; ++e) part[w][lane * VK + e] = acc[e];
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int e = 0; e < VK; ++e) {
      if (e < valid) {
        const int i = lane * VK + e;
        const float s = (part[0][i] + part[1][i]) + (part[2][i] + part[3][i]);
        Num<Tout>::store(reinterpret_cast<Tout*>(a.out) + m * a.K + k0 + e, reduce_final<OP>(s, a.N));
      }
    }
  }
}

template <typename Tin, typename Tout, int OP>
static int launch_reduce(const ReduceArgs& a, hipStream_t s) {
  if (a.K == 1) {
    constexpr int VEC = 16 / (int)sizeof(Tin);
    const int64_t blocks = cdiv(a.M, kRowWaves);
    const int64_t nc = cdiv(cdiv(a.N, VEC), 64);  // chunks per lane
    if (a.vin && a.N % VEC == 0 && nc <= 8) {
      if (nc <= 1) hipLaunchKernelGGL((reduce_rows_fit<Tin, Tout, OP, 1>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      else if (nc <= 2) hipLaunchKernelGGL((reduce_rows_fit<Tin, Tout, OP, 2>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      else if (nc <= 4) hipLaunchKernelGGL((reduce_rows_fit<Tin, Tout, OP, 4>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      else hipLaunchKernelGGL((reduce_rows_fit<Tin, Tout, OP, 8>), dim3((unsigned)blocks), dim3(256), 0, s, a);
    } else if (a.N <= kWaveRowMax) {
      hipLaunchKernelGGL((reduce_rows_wave<Tin, Tout, OP>), dim3((unsigned)blocks), dim3(256), 0, s, a);
    } else {
      hipLaunchKernelGGL((reduce_rows_block<Tin, Tout, OP>), dim3((unsigned)a.M), dim3(256), 0, s, a);
    }
  } else if (a.kvec) {
    constexpr int VK = 16 / (int)sizeof(Tin);
    const int64_t blocks = a.M * cdiv(a.K, 64 * VK);
    if (blocks > 0x7fffffffLL) return fail(BIOPS_ERR_ARG, "reduction too large");
    hipLaunchKernelGGL((reduce_strided<Tin, Tout, OP, VK>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  } else {
    const int64_t blocks = a.M * cdiv(a.K, 64);
    if (blocks > 0x7fffffffLL) return fail(BIOPS_ERR_ARG, "reduction too large");
    hipLaunchKernelGGL((reduce_strided<Tin, Tout, OP, 1>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  }
  return check_launch("reduce");
}

template <typename Tin, typename Tout>
static int launch_reduce_op(int op, const ReduceArgs& a, hipStream_t s) {
  if (op == BIOPS_REDUCE_L2) return launch_reduce<Tin, Tout, BIOPS_REDUCE_L2>(a, s);
  return launch_reduce<Tin, Tout, BIOPS_REDUCE_MEAN>(a, s);
}

}  // namespace biops

using namespace biops;

#define BIOPS_DISPATCH_IN_OUT(din, dout, FN, ...)                                              \
  do {                                                                                        \
    switch ((din) * 3 + (dout)) {                                                              \
      case BIOPS_F32 * 3 + BIOPS_F32: return FN<float, float>(__VA_ARGS__);                   \
      case BIOPS_F32 * 3 + BIOPS_F16: return FN<float, f16_t>(__VA_ARGS__);                   \
      case BIOPS_F32 * 3 + BIOPS_BF16: return FN<float, bf16_t>(__VA_ARGS__);                 \
      case BIOPS_F16 * 3 + BIOPS_F32: return FN<f16_t, float>(__VA_ARGS__);                   \
      case BIOPS_F16 * 3 + BIOPS_F16: return FN<f16_t, f16_t>(__VA_ARGS__);                   \
      case BIOPS_F16 * 3 + BIOPS_BF16: return FN<f16_t, bf16_t>(__VA_ARGS__);                 \
      case BIOPS_BF16 * 3 + BIOPS_F32: return FN<bf16_t, float>(__VA_ARGS__);                 \
      case BIOPS_BF16 * 3 + BIOPS_F16: return FN<bf16_t, f16_t>(__VA_ARGS__);                 \
      case BIOPS_BF16 * 3 + BIOPS_BF16: return FN<bf16_t, bf16_t>(__VA_ARGS__);               \
    }                                                                                         \
  } while (0)

extern "C" int biops_softmax(int dtype_in, int dtype_out, int64_t rows, int64_t cols,
                             const void* in, int64_t ld_in, void* out, int64_t ld_out, int is_log,
                             void* stream) {
  if (!is_float_dtype(dtype_in) || !is_float_dtype(dtype_out))
    return fail(BIOPS_ERR_DTYPE, "unsupported softmax dtype %d -> %d", dtype_in, dtype_out);
  if (rows < 0 || cols < 0) return fail(BIOPS_ERR_ARG, "negative size");
  if (rows == 0 || cols == 0) return BIOPS_OK;
  if (!in || !out) return fail(BIOPS_ERR_ARG, "null pointer");
  SoftmaxArgs a{in, out, rows, cols, ld_in, ld_out, 0, 0};
  a.vin = (reinterpret_cast<uintptr_t>(in) % 16 == 0) && ((ld_in * dtype_bytes(dtype_in)) % 16 == 0);
  a.vout = (reinterpret_cast<uintptr_t>(out) % 16 == 0) && ((ld_out * dtype_bytes(dtype_out)) % 16 == 0);
  BIOPS_DISPATCH_IN_OUT(dtype_in, dtype_out, launch_softmax, a, is_log, (hipStream_t)stream);
  return fail(BIOPS_ERR_DTYPE, "unsupported softmax dtype");
}

extern "C" int biops_reduce(int op, int dtype_in, int dtype_out, int64_t M, int64_t N, int64_t K,
                            const void* in, int64_t sM, int64_t sN, int64_t sK, void* out,
                            void* stream) {
  if (op != BIOPS_REDUCE_MEAN && op != BIOPS_REDUCE_L2) return fail(BIOPS_ERR_ARG, "bad op %d", op);
  if (!is_float_dtype(dtype_in) || !is_float_dtype(dtype_out))
    return fail(BIOPS_ERR_DTYPE, "unsupported reduce dtype %d -> %d", dtype_in, dtype_out);
  if (M < 0 || N < 0 || K < 0) return fail(BIOPS_ERR_ARG, "negative size");
  if (M == 0 || K == 0) return BIOPS_OK;
  if (!in || !out) return fail(BIOPS_ERR_ARG, "null pointer");
  if (K == 1 && sN != 1 && N > 1) return fail(BIOPS_ERR_LAYOUT, "rows must be contiguous when K == 1");
  ReduceArgs a{in, out, M, N, K, sM, sN, sK, 0, 0};
  const int elt = dtype_bytes(dtype_in);
  a.vin = (reinterpret_cast<uintptr_t>(in) % 16 == 0) && ((sM * elt) % 16 == 0);
  a.kvec = K > 1 && sK == 1 && a.vin && ((sN * elt) % 16 == 0);
  if (M > 0x7fffffffLL) return fail(BIOPS_ERR_ARG, "too many rows");
  if (op == BIOPS_REDUCE_L2) {
    BIOPS_DISPATCH_IN_OUT(dtype_in, dtype_out, launch_reduce_op, BIOPS_REDUCE_L2, a, (hipStream_t)stream);
  } else {
    BIOPS_DISPATCH_IN_OUT(dtype_in, dtype_out, launch_reduce_op, BIOPS_REDUCE_MEAN, a, (hipStream_t)stream);
  }
  return fail(BIOPS_ERR_DTYPE, "unsupported reduce dtype");
}
