// Convolution family (aten::convolution) on the fixed-schedule GEMM.
//
//   depthwise 1-D (groups == C_in == C_out, one input channel per group): one thread per output,
//     fp32 accumulation over the taps in order (zero for taps in the padding), bias added to the
//     accumulator, one rounding;
//   regular 1-D / 2-D / 3-D (any groups, stride, padding, dilation): patches of every output
//     position (im2col, K ordered channel, kd, kh, kw and zero-padded to whole 128-byte GEMM
//     steps), then out[b, g*Og + o, l] = W_g[o, :] . patches[b, g, l, :] as one batched GEMM
//     (weights as A, patches as K-major B, so C lands in [B, C_out, spatial] order), then
//     round(out + bias[c]);
//   transposed with stride == kernel, no padding / dilation (every output position gets one
//     contribution): Y[b, g, (o, kidx), l] = W_g^T[(o, kidx), :] . x[b, g*Cg .. , l] as one
//     batched GEMM with the input as N-major B, then each Y element moves to its output position
//     with round(y + bias[c]).
// The zero K padding does not change any bit: the GEMM treats K beyond the problem as zero in
// both operands, step by step.  Every output element's arithmetic depends on the weight shape
// and the convolution parameters only, never on the batch size.
#include <algorithm>

#include "gemm.h"

namespace biops {

constexpr int kConvThreads = 256;

struct ConvShape {
  int64_t B, Cin, Cout, G, Cg, Og;
  int64_t in[3], out[3], k[3], s[3], p[3], d[3];
  int64_t Lin, Lout, kvol, Kc, Kp;
  bool transposed, depthwise1d;
};

// Leading spatial dims of 1-D / 2-D problems become size-1 dims (kernel 1, stride 1, no padding).
static int conv_shape(int dtype, int nd, int transposed, int64_t batch, int64_t cin, const int64_t* in_size,
                      int64_t cout, const int64_t* ksize, const int64_t* stride, const int64_t* padding,
                      const int64_t* dilation, int64_t groups, ConvShape& c) {
  if (!is_float_dtype(dtype)) return fail(BIOPS_ERR_DTYPE, "unsupported convolution dtype %d", dtype);
  if (nd < 1 || nd > 3) return fail(BIOPS_ERR_ARG, "convolution rank %d", nd);
  if (!in_size || !ksize || !stride || !padding || !dilation) return fail(BIOPS_ERR_ARG, "null size array");
  if (batch < 0 || cin <= 0 || cout < 0 || groups <= 0 || cin % groups != 0 || cout % groups != 0)
    return fail(BIOPS_ERR_ARG, "invalid channel / group sizes");
  c.B = batch; c.Cin = cin; c.Cout = cout; c.G = groups;
  c.Cg = cin / groups; c.Og = cout / groups;
  c.transposed = transposed != 0;
  const int off = 3 - nd;
  for (int i = 0; i < 3; ++i) {
    const bool lead = i < off;
    c.in[i] = lead ? 1 : in_size[i - off];
    c.k[i] = lead ? 1 : ksize[i - off];
    c.s[i] = lead ? 1 : stride[i - off];
    c.p[i] = lead ? 0 : padding[i - off];
    c.d[i] = lead ? 1 : dilation[i - off];
    if (c.in[i] < 0 || c.k[i] <= 0 || c.s[i] <= 0 || c.p[i] < 0 || c.d[i] <= 0)
      return fail(BIOPS_ERR_ARG, "invalid convolution sizes");
    if (c.transposed) {
      if (c.s[i] != c.k[i] || c.p[i] != 0 || c.d[i] != 1)
        return fail(BIOPS_ERR_ARG, "transposed convolution needs stride == kernel, no padding or dilation");
      c.out[i] = c.in[i] * c.k[i];
    } else {
      const int64_t span = c.in[i] + 2 * c.p[i] - c.d[i] * (c.k[i] - 1) - 1;
      c.out[i] = span < 0 ? 0 : span / c.s[i] + 1;
    }
  }
  c.Lin = c.in[0] * c.in[1] * c.in[2];
  c.Lout = c.out[0] * c.out[1] * c.out[2];
  c.kvol = c.k[0] * c.k[1] * c.k[2];
  // GEMM K: channels x taps (regular) or input channels (transposed), padded to whole steps.
  const int64_t step = kKBytes / dtype_bytes(dtype);
  c.Kc = c.transposed ? c.Cg : c.Cg * c.kvol;
  c.Kp = cdiv(c.Kc, step) * step;
  c.depthwise1d = nd == 1 && !c.transposed && c.G == c.Cin && c.Cout == c.Cin && c.Cg == 1;
  if (c.transposed && c.Og * c.kvol >= (int64_t(1) << 31)) return fail(BIOPS_ERR_SIZE, "kernel too large");
  return BIOPS_OK;
}

// Workspace: regular -- padded weights [C_out, Kp] then patches [B, G, Lout, Kp];
// transposed -- transposed weights [G, Og*kvol, Kp] then Y [B, G, Og*kvol, Lin].
struct ConvWorkspace {
  int64_t weights, scratch, total;
};
static ConvWorkspace conv_workspace(const ConvShape& c, int elt) {
  auto al = [](int64_t b) { return (b + 255) & ~int64_t(255); };
  ConvWorkspace w{0, 0, 0};
  if (c.depthwise1d) return w;
  if (c.transposed) {
    const int64_t n = c.Og * c.kvol;
    w.scratch = al(c.G * n * c.Kp * elt);
    w.total = w.scratch + al(c.B * c.G * n * c.Lin * elt);
  } else {
    w.scratch = al(c.Cout * c.Kp * elt);
    w.total = w.scratch + al(c.B * c.G * c.Lout * c.Kp * elt);
  }
  return w;
}

// ------------------------------------------------------------------ kernels ----
struct DepthwiseArgs {
  const void* x; const void* w; const void* bias; void* out;
  int64_t total, C, Lin, Lout, K, stride, pad, dil;
  int64_t sxb, sxc, sxl, swc, swk;
};

// acc = sum over taps k of x[l*stride - pad + k*dil] * w[k] (0 outside the input), then + bias.
template <typename T>
__global__ __launch_bounds__(kConvThreads) void conv_depthwise1d_kernel(DepthwiseArgs a) {
  const T* x = reinterpret_cast<const T*>(a.x);
  const T* w = reinterpret_cast<const T*>(a.w);
  T* out = reinterpret_cast<T*>(a.out);
  for (int64_t e = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; e < a.total;
       e += (int64_t)gridDim.x * kConvThreads) {
    const int64_t l = e % a.Lout;
    const int64_t bc = e / a.Lout;
    const int64_t c = bc % a.C, b = bc / a.C;
    const T* xr = x + b * a.sxb + c * a.sxc;
    float acc = 0.f;
    for (int64_t k = 0; k < a.K; ++k) {
      const int64_t i = l * a.stride - a.pad + k * a.dil;
      const float v = (i >= 0 && i < a.Lin) ? Num<T>::load(xr + i * a.sxl) : 0.f;
      acc = fmaf(v, Num<T>::load(w + c * a.swc + k * a.swk), acc);
    }
    if (a.bias) acc += Num<T>::load(reinterpret_cast<const T*>(a.bias) + c);
    Num<T>::store(out + e, acc);
  }
}

struct Im2colArgs {
  const void* x; void* patches;
  int64_t sx[5];  // element strides of (b, c, d, h, w)
  int64_t G, Cg, Lout, Kc, Kp, total;  // total = B * G * Lout * Kp / VEC chunks
  int32_t in[3], out[3], k[3], s[3], p[3], d[3];
};

// One 16-byte chunk of a patch row per thread: patches[(b*G + g)*Lout + l][k .. k+VEC).
template <typename T>
__global__ __launch_bounds__(kConvThreads) void conv_im2col_kernel(Im2colArgs a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  const T* x = reinterpret_cast<const T*>(a.x);
  const int64_t kch = a.Kp / VEC;
  const int32_t kvol = a.k[0] * a.k[1] * a.k[2];
  for (int64_t e = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; e < a.total;
       e += (int64_t)gridDim.x * kConvThreads) {
    const int64_t k0 = (e % kch) * VEC;
    const int64_t row = e / kch;
    const int64_t l = row % a.Lout;
    const int64_t bg = row / a.Lout;
    const int64_t g = bg % a.G, b = bg / a.G;
    const int32_t ow = (int32_t)(l % a.out[2]);
    const int32_t oh = (int32_t)((l / a.out[2]) % a.out[1]);
    const int32_t od = (int32_t)(l / ((int64_t)a.out[2] * a.out[1]));
    const T* xb = x + b * a.sx[0] + g * a.Cg * a.sx[1];
    u32x4_t v = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int64_t k = k0 + j;
      uint32_t bits = 0;
      if (k < a.Kc) {
        const int32_t c = (int32_t)(k / kvol);
        const int32_t r = (int32_t)(k - (int64_t)c * kvol);
        const int32_t kw = r % a.k[2], kh = (r / a.k[2]) % a.k[1], kd = r / (a.k[2] * a.k[1]);
        const int32_t id = od * a.s[0] - a.p[0] + kd * a.d[0];
        const int32_t ih = oh * a.s[1] - a.p[1] + kh * a.d[1];
        const int32_t iw = ow * a.s[2] - a.p[2] + kw * a.d[2];
        if (id >= 0 && id < a.in[0] && ih >= 0 && ih < a.in[1] && iw >= 0 && iw < a.in[2]) {
          const T* src = xb + c * a.sx[1] + id * a.sx[2] + ih * a.sx[3] + iw * a.sx[4];
          if constexpr (sizeof(T) == 4) bits = __float_as_uint(*reinterpret_cast<const float*>(src));
          else bits = reinterpret_cast<const uint16_t*>(src)[0];
        }
      }
      if constexpr (sizeof(T) == 4) v[j] = bits;
      else v[j >> 1] |= bits << (16 * (j & 1));
    }
    *reinterpret_cast<u32x4_t*>(reinterpret_cast<T*>(a.patches) + row * a.Kp + k0) = v;
  }
}

struct WeightPrepArgs {
  const void* w; void* dst;
  int64_t rows, Kc, Kp, total;  // total = rows * Kp
  int64_t G, Cg, N;             // transposed: w is [G*Cg, N], dst [G, N, Kp] (row = g*N + n)
  int32_t transpose;
};

// dst[row, k] = weight element (k < Kc) or 0: regular -- w[row, k]; transposed -- w[g*Cg + k, n].
template <typename T>
__global__ __launch_bounds__(kConvThreads) void conv_weight_kernel(WeightPrepArgs a) {
  const T* w = reinterpret_cast<const T*>(a.w);
  T* dst = reinterpret_cast<T*>(a.dst);
  for (int64_t e = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; e < a.total;
       e += (int64_t)gridDim.x * kConvThreads) {
    const int64_t k = e % a.Kp, row = e / a.Kp;
    T v{};
    if (k < a.Kc) {
      if (a.transpose) {
        const int64_t g = row / a.N, n = row % a.N;
        v = w[(g * a.Cg + k) * a.N + n];
      } else {
        v = w[row * a.Kc + k];
      }
    }
    dst[e] = v;
  }
}

struct ChannelBiasArgs {
  void* out; const void* bias;
  int64_t C, L, total;
};

// out[b, c, l] = round(out[b, c, l] + bias[c]), the rounded GEMM output plus the bias.
template <typename T>
__global__ __launch_bounds__(kConvThreads) void conv_bias_kernel(ChannelBiasArgs a) {
  T* out = reinterpret_cast<T*>(a.out);
  const T* bias = reinterpret_cast<const T*>(a.bias);
  for (int64_t e = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; e < a.total;
       e += (int64_t)gridDim.x * kConvThreads) {
    const int64_t c = (e / a.L) % a.C;
    Num<T>::store(out + e, Num<T>::load(out + e) + Num<T>::load(bias + c));
  }
}

struct ScatterArgs {
  const void* y; const void* bias; void* out;
  int64_t G, Og, Cout, N, Lin, total;
  int32_t in[3], k[3], out_sz[3];
};

// out[b, c, od, oh, ow] = Y[b, g, (o, kd, kh, kw), (id, ih, iw)] (+ bias[c], rounded), with
// c = g*Og + o, od = id*kd_size + kd, ...
template <typename T>
__global__ __launch_bounds__(kConvThreads) void conv_scatter_kernel(ScatterArgs a) {
  const T* y = reinterpret_cast<const T*>(a.y);
  T* out = reinterpret_cast<T*>(a.out);
  const int64_t Lout = (int64_t)a.out_sz[0] * a.out_sz[1] * a.out_sz[2];
  for (int64_t e = (int64_t)blockIdx.x * kConvThreads + threadIdx.x; e < a.total;
       e += (int64_t)gridDim.x * kConvThreads) {
    const int64_t sp = e % Lout;
    const int64_t bc = e / Lout;
    const int64_t c = bc % a.Cout, b = bc / a.Cout;
    const int64_t g = c / a.Og, o = c % a.Og;
    const int32_t ow = (int32_t)(sp % a.out_sz[2]);
    const int32_t oh = (int32_t)((sp / a.out_sz[2]) % a.out_sz[1]);
    const int32_t od = (int32_t)(sp / ((int64_t)a.out_sz[2] * a.out_sz[1]));
    const int32_t kd = od % a.k[0], kh = oh % a.k[1], kw = ow % a.k[2];
    const int64_t l = ((int64_t)(od / a.k[0]) * a.in[1] + oh / a.k[1]) * a.in[2] + ow / a.k[2];
    const int64_t n = o * ((int64_t)a.k[0] * a.k[1] * a.k[2]) + ((int64_t)kd * a.k[1] + kh) * a.k[2] + kw;
    const float v = Num<T>::load(y + ((b * a.G + g) * a.N + n) * a.Lin + l);
    if (a.bias) Num<T>::store(out + e, v + Num<T>::load(reinterpret_cast<const T*>(a.bias) + c));
    else Num<T>::store(out + e, v);
  }
}

static unsigned elementwise_grid(int64_t total) {
  const int64_t blocks = cdiv(total, kConvThreads);
  return (unsigned)std::min<int64_t>(blocks, 65536);
}

// Launch KERNEL<T> for the dtype over `total` elements (grid-stride loops).
#define BIOPS_CONV_LAUNCH(KERNEL, DTYPE, ARGS, TOTAL, STREAM)                                     \
  [&]() -> int {                                                                                \
    if ((TOTAL) <= 0) return BIOPS_OK;                                                          \
    const dim3 grid_(elementwise_grid(TOTAL)), block_(kConvThreads);                            \
    switch (DTYPE) {                                                                            \
      case BIOPS_F32: hipLaunchKernelGGL(KERNEL<float>, grid_, block_, 0, STREAM, ARGS); break;  \
      case BIOPS_F16: hipLaunchKernelGGL(KERNEL<f16_t>, grid_, block_, 0, STREAM, ARGS); break;  \
      default: hipLaunchKernelGGL(KERNEL<bf16_t>, grid_, block_, 0, STREAM, ARGS); break;        \
    }                                                                                           \
    return check_launch(#KERNEL);                                                               \
  }()

}  // namespace biops

using namespace biops;

extern "C" int64_t biops_conv_workspace_size(int dtype, int nd, int transposed, int64_t batch, int64_t cin,
                                             const int64_t* in_size, int64_t cout, const int64_t* ksize,
                                             const int64_t* stride, const int64_t* padding,
                                             const int64_t* dilation, int64_t groups) {
  ConvShape c;
  if (conv_shape(dtype, nd, transposed, batch, cin, in_size, cout, ksize, stride, padding, dilation, groups, c) !=
      BIOPS_OK)
    return -1;
  return conv_workspace(c, dtype_bytes(dtype)).total;
}

extern "C" int biops_conv(int dtype, int nd, int transposed, int64_t batch, int64_t cin, const int64_t* in_size,
                          int64_t cout, const int64_t* ksize, const int64_t* stride, const int64_t* padding,
                          const int64_t* dilation, int64_t groups, const void* x, const int64_t* x_strides,
                          const void* w, const void* bias, void* out, void* workspace, int64_t workspace_bytes,
                          void* stream) {
  ConvShape c;
  int rc = conv_shape(dtype, nd, transposed, batch, cin, in_size, cout, ksize, stride, padding, dilation, groups, c);
  if (rc != BIOPS_OK) return rc;
  if (!x_strides) return fail(BIOPS_ERR_ARG, "null input strides");
  if (c.B == 0 || c.Cout == 0 || c.Lout == 0) return BIOPS_OK;
  const int elt = dtype_bytes(dtype);
  const ConvWorkspace ws = conv_workspace(c, elt);
  if (workspace_bytes < ws.total)
    return fail(BIOPS_ERR_SIZE, "workspace %lld < %lld bytes", (long long)workspace_bytes, (long long)ws.total);
  if (ws.total > 0 && reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return fail(BIOPS_ERR_LAYOUT, "workspace must be 256-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  // input strides as (b, c, d, h, w); absent leading spatial dims have extent 1 and get the
  // stride a contiguous layout would give them (never used in an address)
  int64_t sx[5];
  sx[0] = x_strides[0];
  sx[1] = x_strides[1];
  for (int i = 2; i >= 0; --i)
    sx[2 + i] = i >= 3 - nd ? x_strides[2 + i - (3 - nd)] : sx[3 + i] * c.in[i + 1];
  char* wsp = reinterpret_cast<char*>(workspace);

  if (c.depthwise1d) {
    DepthwiseArgs a{x, w, bias, out, c.B * c.Cout * c.Lout, c.Cout, c.in[2], c.out[2], c.k[2], c.s[2], c.p[2],
                    c.d[2], sx[0], sx[1], sx[4], c.kvol, 1};
    return BIOPS_CONV_LAUNCH(conv_depthwise1d_kernel, dtype, a, a.total, s);
  }
  for (int i = 0; i < 3; ++i)
    if (c.in[i] >= (int64_t(1) << 31) || c.out[i] >= (int64_t(1) << 31))
      return fail(BIOPS_ERR_SIZE, "spatial extent too large");

  if (!c.transposed) {
    // weights [C_out, Kc] -> [C_out, Kp]
    WeightPrepArgs wp{w, wsp, c.Cout, c.Kc, c.Kp, c.Cout * c.Kp, c.G, c.Cg, 0, 0};
    if ((rc = BIOPS_CONV_LAUNCH(conv_weight_kernel, dtype, wp, wp.total, s)) != BIOPS_OK)
      return rc;
    Im2colArgs ia{};
    ia.x = x;
    ia.patches = wsp + ws.scratch;
    for (int i = 0; i < 5; ++i) ia.sx[i] = sx[i];
    ia.G = c.G; ia.Cg = c.Cg; ia.Lout = c.Lout; ia.Kc = c.Kc; ia.Kp = c.Kp;
    ia.total = c.B * c.G * c.Lout * (c.Kp / (16 / elt));
    for (int i = 0; i < 3; ++i) {
      ia.in[i] = (int32_t)c.in[i]; ia.out[i] = (int32_t)c.out[i]; ia.k[i] = (int32_t)c.k[i];
      ia.s[i] = (int32_t)c.s[i]; ia.p[i] = (int32_t)c.p[i]; ia.d[i] = (int32_t)c.d[i];
    }
    if ((rc = BIOPS_CONV_LAUNCH(conv_im2col_kernel, dtype, ia, ia.total, s)) != BIOPS_OK)
      return rc;
    BmmArgs g{};
    g.A = wsp; g.lda = c.Kp; g.sA1 = 0; g.sA2 = c.Og * c.Kp;
    g.B = wsp + ws.scratch; g.ldb = c.Kp; g.sB1 = c.G * c.Lout * c.Kp; g.sB2 = c.Lout * c.Kp; g.gB = 1;
    g.C = out; g.ldc = c.Lout; g.sC1 = c.Cout * c.Lout; g.sC2 = c.Og * c.Lout;
    g.M = c.Og; g.N = c.Lout; g.K = c.Kp;
    g.nb1 = c.B; g.nb2 = c.G;
    if ((rc = launch_bmm(dtype, g, kEpiPlain, true, s)) != BIOPS_OK) return rc;
    if (bias) {
      ChannelBiasArgs ba{out, bias, c.Cout, c.Lout, c.B * c.Cout * c.Lout};
      return BIOPS_CONV_LAUNCH(conv_bias_kernel, dtype, ba, ba.total, s);
    }
    return BIOPS_OK;
  }

  // transposed: the GEMM reads the input as N-major B, so its spatial dims must be contiguous
  if (sx[4] != 1 || sx[3] != c.in[2] || sx[2] != c.in[1] * c.in[2])
    return fail(BIOPS_ERR_LAYOUT, "transposed convolution needs contiguous spatial input dims");
  const int64_t n = c.Og * c.kvol;
  WeightPrepArgs wp{w, wsp, c.G * n, c.Kc, c.Kp, c.G * n * c.Kp, c.G, c.Cg, n, 1};
  if ((rc = BIOPS_CONV_LAUNCH(conv_weight_kernel, dtype, wp, wp.total, s)) != BIOPS_OK)
    return rc;
  void* y = wsp + ws.scratch;
  BmmArgs g{};
  g.A = wsp; g.lda = c.Kp; g.sA1 = 0; g.sA2 = n * c.Kp;
  g.B = x; g.ldb = sx[1]; g.sB1 = sx[0]; g.sB2 = c.Cg * sx[1]; g.gB = 1;
  g.C = y; g.ldc = c.Lin; g.sC1 = c.G * n * c.Lin; g.sC2 = n * c.Lin;
  g.M = n; g.N = c.Lin; g.K = c.Cg;
  g.nb1 = c.B; g.nb2 = c.G;
  if ((rc = launch_bmm(dtype, g, kEpiPlain, false, s)) != BIOPS_OK) return rc;
  ScatterArgs sa{};
  sa.y = y; sa.bias = bias; sa.out = out;
  sa.G = c.G; sa.Og = c.Og; sa.Cout = c.Cout; sa.N = n; sa.Lin = c.Lin;
  sa.total = c.B * c.Cout * c.Lout;
  for (int i = 0; i < 3; ++i) {
    sa.in[i] = (int32_t)c.in[i]; sa.k[i] = (int32_t)c.k[i]; sa.out_sz[i] = (int32_t)c.out[i];
  }
  return BIOPS_CONV_LAUNCH(conv_scatter_kernel, dtype, sa, sa.total, s);
}
