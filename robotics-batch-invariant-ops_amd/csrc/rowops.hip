// Softmax / log-softmax and mean / L2-norm reductions.
#include "rowops.h"

namespace biops {

// ------------------------------------------------------------------ softmax ----
struct SoftmaxArgs {
  const void* in;
  void* out;
  int64_t rows, cols, ld_in, ld_out;
  int32_t vin, vout;
};

template <typename Tin, typename Tout, int MODE>
__global__ __launch_bounds__(256) void softmax_kernel(SoftmaxArgs a) {
  const int64_t r = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  if (r >= a.rows) return;
  AttnRow ar{1.f, a.cols, nullptr, 0, 0};
  softmax_row<Tin, Tout, MODE>(reinterpret_cast<const Tin*>(a.in) + r * a.ld_in,
                               reinterpret_cast<Tout*>(a.out) + r * a.ld_out, a.cols, a.vin != 0,
                               a.vout != 0, ar);
}

template <typename Tin, typename Tout>
static int launch_softmax(const SoftmaxArgs& a, int is_log, hipStream_t s) {
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
// sums are added as (w0 + w1) + (w2 + w3).  The choice depends on N only.
constexpr int64_t kWaveRowMax = 65536;

struct ReduceArgs {
  const void* in;
  void* out;
  int64_t M, N, K, sM, sN, sK;
  int32_t vin;
};

template <int OP>
__device__ __forceinline__ float reduce_term(float x) { return OP == BIOPS_REDUCE_L2 ? x * x : x; }
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
      if (ci * VEC + e < a.N) acc += reduce_term<OP>(v[e]);
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
      if (ci * VEC + e < a.N) acc += reduce_term<OP>(v[e]);
  }
  acc = wave_sum(acc);
  if ((t & 63) == 0) part[t >> 6] = acc;
  __syncthreads();
  if (t == 0) {
    const float s = (part[0] + part[1]) + (part[2] + part[3]);
    Num<Tout>::store(reinterpret_cast<Tout*>(a.out) + r, reduce_final<OP>(s, a.N));
  }
}

// Strided reduction (K > 1): a workgroup owns 64 consecutive k of one m; wavefront w adds the
// elements n = w, w+4, w+8, ... in increasing n, and the four partials are added as
// (p0 + p1) + (p2 + p3).  Depends on N only.
template <typename Tin, typename Tout, int OP>
__global__ __launch_bounds__(256) void reduce_strided(ReduceArgs a) {
  __shared__ float part[4][64];
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t kblocks = cdiv(a.K, 64);
  const int64_t m = blockIdx.x / kblocks;
  const int64_t k = (blockIdx.x - m * kblocks) * 64 + lane;
  float acc = 0.f;
  if (k < a.K) {
    const Tin* base = reinterpret_cast<const Tin*>(a.in) + m * a.sM + k * a.sK;
    for (int64_t n = w; n < a.N; n += 4) acc += reduce_term<OP>(Num<Tin>::load(base + n * a.sN));
  }
  part[w][lane] = acc;
  __syncthreads();
  if (w == 0 && k < a.K) {
    const float s = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
    Num<Tout>::store(reinterpret_cast<Tout*>(a.out) + m * a.K + k, reduce_final<OP>(s, a.N));
  }
}

template <typename Tin, typename Tout, int OP>
static int launch_reduce(const ReduceArgs& a, hipStream_t s) {
  if (a.K == 1) {
    if (a.N <= kWaveRowMax) {
      const int64_t blocks = cdiv(a.M, kRowWaves);
      hipLaunchKernelGGL((reduce_rows_wave<Tin, Tout, OP>), dim3((unsigned)blocks), dim3(256), 0, s, a);
    } else {
      hipLaunchKernelGGL((reduce_rows_block<Tin, Tout, OP>), dim3((unsigned)a.M), dim3(256), 0, s, a);
    }
  } else {
    const int64_t blocks = a.M * cdiv(a.K, 64);
    if (blocks > 0x7fffffffLL) return fail(BIOPS_ERR_ARG, "reduction too large");
    hipLaunchKernelGGL((reduce_strided<Tin, Tout, OP>), dim3((unsigned)blocks), dim3(256), 0, s, a);
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
  ReduceArgs a{in, out, M, N, K, sM, sN, sK, 0};
  a.vin = (reinterpret_cast<uintptr_t>(in) % 16 == 0) && ((sM * dtype_bytes(dtype_in)) % 16 == 0);
  if (M > 0x7fffffffLL) return fail(BIOPS_ERR_ARG, "too many rows");
  if (op == BIOPS_REDUCE_L2) {
    BIOPS_DISPATCH_IN_OUT(dtype_in, dtype_out, launch_reduce_op, BIOPS_REDUCE_L2, a, (hipStream_t)stream);
  } else {
    BIOPS_DISPATCH_IN_OUT(dtype_in, dtype_out, launch_reduce_op, BIOPS_REDUCE_MEAN, a, (hipStream_t)stream);
  }
  return fail(BIOPS_ERR_DTYPE, "unsupported reduce dtype");
}
