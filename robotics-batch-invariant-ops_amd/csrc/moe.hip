// Deterministic token-choice top-k SwiGLU mixture of experts (dense expert evaluation).
//   act[e] = SwiGLU(x . gate_e^T, x . up_e^T)   one fused GEMM launch over all experts
//   y[e]   = act[e] . down_e^T                  one GEMM launch over all experts
//   out[t] = fixed left-to-right sum over the top-k slots of round(y[sel[t,s], t] * round(w[t,s]))
// No atomics anywhere: every output element is written by exactly one thread.
#include "gemm.h"

namespace biops {

struct CombineArgs {
  const void* y;          // [E, T, D]
  const void* w;          // [T, k]
  const int64_t* sel;     // [T, k]
  void* out;              // [T, D]
  int32_t* bad;           // optional error flag
  int64_t T, D, E, k;
  int w_dtype;
  int32_t vec;
};

template <typename T>
__device__ __forceinline__ float load_weight(const void* w, int wdt, int64_t idx) {
  switch (wdt) {
    case BIOPS_F32: return Num<T>::round(reinterpret_cast<const float*>(w)[idx]);
    case BIOPS_F16: return Num<T>::round(Num<f16_t>::load(reinterpret_cast<const f16_t*>(w) + idx));
    default: return Num<T>::round(Num<bf16_t>::load(reinterpret_cast<const bf16_t*>(w) + idx));
  }
}

// One workgroup per token; each thread owns 4 consecutive hidden columns per pass.
template <typename T>
__global__ __launch_bounds__(256) void moe_combine_kernel(CombineArgs a) {
  const int64_t t = blockIdx.x;
  bool ok = true;
  for (int64_t s = 0; s < a.k; ++s) {
    const int64_t e = a.sel[t * a.k + s];
    ok = ok && e >= 0 && e < a.E;
  }
  if (!ok && threadIdx.x == 0 && a.bad) *a.bad = 1;
  T* out = reinterpret_cast<T*>(a.out) + t * a.D;
  for (int64_t d0 = (int64_t)threadIdx.x * 4; d0 < a.D; d0 += 256 * 4) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    if (ok) {
      for (int64_t s = 0; s < a.k; ++s) {
        const int64_t e = a.sel[t * a.k + s];
        const float w = load_weight<T>(a.w, a.w_dtype, t * a.k + s);
        const T* y = reinterpret_cast<const T*>(a.y) + (e * a.T + t) * a.D;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (d0 + c < a.D) {
            const float r = Num<T>::round(Num<T>::load(y + d0 + c) * w);
            acc[c] = (s == 0) ? r : Num<T>::round(acc[c] + r);
          }
        }
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (d0 + c < a.D) Num<T>::store(out + d0 + c, acc[c]);
  }
}

static bool weight_layout(int64_t sE, int64_t sRow, int64_t sK, int64_t rows, int64_t K, bool& kmajor,
                          int64_t& ld) {
  (void)sE;
  return b_layout(K, rows, sK, sRow, kmajor, ld);
}

}  // namespace biops

using namespace biops;

extern "C" int64_t biops_moe_workspace_size(int dtype, int64_t tokens, int64_t experts,
                                            int64_t hidden, int64_t inter) {
  const int elt = dtype_bytes(dtype);
  if (elt == 0 || tokens < 0 || experts < 0 || hidden < 0 || inter < 0) return -1;
  const int64_t act = experts * tokens * inter;
  const int64_t act_pad = (act + 63) & ~int64_t(63);
  return (act_pad + experts * tokens * hidden) * elt;
}

extern "C" int biops_moe(int dtype, int64_t tokens, int64_t experts, int64_t hidden, int64_t inter,
                         int64_t top_k, const void* x, int64_t sx, const void* gate, int64_t sgE,
                         int64_t sgI, int64_t sgD, const void* up, int64_t suE, int64_t suI,
                         int64_t suD, const void* down, int64_t sdE, int64_t sdD, int64_t sdI,
                         const void* weights, int w_dtype, const int64_t* sel, void* out,
                         int32_t* bad_index, void* workspace, int64_t workspace_bytes,
                         void* stream) {
  if (!is_float_dtype(dtype) || !is_float_dtype(w_dtype))
    return fail(BIOPS_ERR_DTYPE, "unsupported MoE dtype");
  if (tokens < 0 || experts <= 0 || hidden < 0 || inter < 0 || top_k < 0)
    return fail(BIOPS_ERR_ARG, "invalid MoE sizes");
  if (tokens == 0 || hidden == 0) return BIOPS_OK;
  if (sgE != suE || sgI != suI || sgD != suD)
    return fail(BIOPS_ERR_LAYOUT, "gate and up weights must share strides");
  const int64_t need = biops_moe_workspace_size(dtype, tokens, experts, hidden, inter);
  if (workspace_bytes < need) return fail(BIOPS_ERR_SIZE, "workspace %lld < %lld bytes",
                                          (long long)workspace_bytes, (long long)need);
  const int elt = dtype_bytes(dtype);
  hipStream_t s = (hipStream_t)stream;
  char* ws = reinterpret_cast<char*>(workspace);
  const int64_t act_elems = (experts * tokens * inter + 63) & ~int64_t(63);
  void* act = ws;
  void* y = ws + act_elems * elt;
  int rc;

  if (top_k > 0) {
    // act[e, t, i] for every expert: B = gate_e / up_e viewed as [I, D] (column i, K = d).
    bool kmaj;
    int64_t ldb;
    if (!weight_layout(sgE, sgI, sgD, inter, hidden, kmaj, ldb))
      return fail(BIOPS_ERR_LAYOUT, "gate/up weights need a unit stride");
    BmmArgs g{};
    g.A = x; g.B = gate; g.B2 = up; g.C = act;
    g.M = tokens; g.N = inter; g.K = hidden;
    g.lda = sx; g.ldb = ldb; g.ldc = inter;
    g.nb1 = experts; g.nb2 = 1; g.gB = 1;
    g.sA1 = 0; g.sB1 = sgE; g.sC1 = tokens * inter;
    if ((rc = launch_bmm(dtype, g, kEpiSwiglu, kmaj, s)) != BIOPS_OK) return rc;

    // y[e, t, d] = act[e, t, :] . down_e[d, :]
    if (!weight_layout(sdE, sdD, sdI, hidden, inter, kmaj, ldb))
      return fail(BIOPS_ERR_LAYOUT, "down weights need a unit stride");
    BmmArgs dn{};
    dn.A = act; dn.B = down; dn.C = y;
    dn.M = tokens; dn.N = hidden; dn.K = inter;
    dn.lda = inter; dn.ldb = ldb; dn.ldc = hidden;
    dn.nb1 = experts; dn.nb2 = 1; dn.gB = 1;
    dn.sA1 = tokens * inter; dn.sB1 = sdE; dn.sC1 = tokens * hidden;
    if ((rc = launch_bmm(dtype, dn, kEpiPlain, kmaj, s)) != BIOPS_OK) return rc;
  }

  CombineArgs c{y, weights, sel, out, bad_index, tokens, hidden, experts, top_k, w_dtype, 0};
  if (tokens > 0x7fffffffLL) return fail(BIOPS_ERR_ARG, "too many tokens");
  switch (dtype) {
    case BIOPS_F32: hipLaunchKernelGGL(moe_combine_kernel<float>, dim3((unsigned)tokens), dim3(256), 0, s, c); break;
    case BIOPS_F16: hipLaunchKernelGGL(moe_combine_kernel<f16_t>, dim3((unsigned)tokens), dim3(256), 0, s, c); break;
    default: hipLaunchKernelGGL(moe_combine_kernel<bf16_t>, dim3((unsigned)tokens), dim3(256), 0, s, c); break;
  }
  return check_launch("moe_combine_kernel");
}
