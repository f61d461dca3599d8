// Eager attention (materialised scores) and packed variable-length attention:
//   S = Q K^T (fixed-schedule GEMM, rounded to the input dtype)
//   P = softmax(round(S * scale) masked)          (one wavefront per row, fused transform)
//   O = P V   (fixed-schedule GEMM)
// Scores and probabilities share one caller-provided workspace (softmax runs in place).
#include "gemm.h"
#include "rowops.h"

namespace biops {

// ------------------------------------------------------------- attention softmax ----
struct AttnSoftmaxArgs {
  void* s;
  int64_t rows, lq, lk, hq, ld;  // score rows = batch*hq*lq, row pitch ld
  float scale;
  int causal;
  const void* mask;
  int mask_kind;  // 0 none, 1 bool, 2 additive
  int64_t mB, mH, mI, mJ;
};

template <typename T>
__global__ __launch_bounds__(256) void attn_softmax_kernel(AttnSoftmaxArgs a) {
  const int64_t r = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  if (r >= a.rows) return;
  const int64_t i = r % a.lq;
  const int64_t bh = r / a.lq;
  const int64_t h = bh % a.hq;
  const int64_t b = bh / a.hq;
  AttnRow ar;
  ar.scale = a.scale;
  ar.col_limit = a.lk;
  if (a.causal != BIOPS_CAUSAL_NONE) {
    const int64_t shift = a.causal == BIOPS_CAUSAL_BOTTOM_RIGHT ? a.lk - a.lq : 0;
    int64_t lim = i + shift + 1;
    ar.col_limit = lim < 0 ? 0 : (lim > a.lk ? a.lk : lim);
  }
  ar.mask_kind = a.mask_kind;
  ar.mask_stride = a.mJ;
  ar.mask = nullptr;
  if (a.mask_kind == 1)
    ar.mask = reinterpret_cast<const uint8_t*>(a.mask) + b * a.mB + h * a.mH + i * a.mI;
  else if (a.mask_kind == 2)
    ar.mask = reinterpret_cast<const T*>(a.mask) + b * a.mB + h * a.mH + i * a.mI;
  T* row = reinterpret_cast<T*>(a.s) + r * a.ld;
  const bool v = (reinterpret_cast<uintptr_t>(a.s) % 16 == 0) && ((a.ld * sizeof(T)) % 16 == 0);
  softmax_row<T, T, kAttn>(row, row, a.lk, v, v, ar);
}

struct VarlenSoftmaxArgs {
  void* s;
  const int64_t* plan;
  int64_t items, rows, hq;
  float scale;
  int causal;
};

template <typename T>
__global__ __launch_bounds__(256) void varlen_softmax_kernel(VarlenSoftmaxArgs a) {
  const int64_t r = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
  if (r >= a.rows) return;
  int64_t lo = 0, hi = a.items - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (a.plan[kPlanHeader + kPlanStride * mid + 7] <= r) lo = mid;
    else hi = mid - 1;
  }
  const int64_t* p = a.plan + kPlanHeader + kPlanStride * lo;
  const int64_t ql = p[1], kl = p[3], soff = p[4];
  const int64_t local = r - p[7];
  const int64_t h = local / ql, i = local - h * ql;
  const int64_t lds = varlen_score_ld(kl);
  AttnRow ar;
  ar.scale = a.scale;
  ar.col_limit = kl;
  if (a.causal != BIOPS_CAUSAL_NONE) {
    const int64_t shift = a.causal == BIOPS_CAUSAL_BOTTOM_RIGHT ? kl - ql : 0;
    const int64_t lim = i + shift + 1;
    ar.col_limit = lim < 0 ? 0 : (lim > kl ? kl : lim);
  }
  ar.mask = nullptr;
  ar.mask_kind = 0;
  ar.mask_stride = 0;
  T* row = reinterpret_cast<T*>(a.s) + soff + (h * ql + i) * lds;
  const bool v = (reinterpret_cast<uintptr_t>(row) % 16) == 0;
  softmax_row<T, T, kAttn>(row, row, kl, v, v, ar);
}

}  // namespace biops

using namespace biops;

extern "C" int64_t biops_sdpa_workspace_size(int dtype, int64_t batch, int64_t hq, int64_t lq,
                                             int64_t lk) {
  const int elt = dtype_bytes(dtype);
  if (elt == 0 || batch < 0 || hq < 0 || lq < 0 || lk < 0) return -1;
  return batch * hq * lq * varlen_score_ld(lk) * elt;
}

extern "C" int biops_sdpa(int dtype, int64_t batch, int64_t hq, int64_t hkv, int64_t lq, int64_t lk,
                          int64_t d, int64_t dv, const void* q, int64_t sqB, int64_t sqH,
                          int64_t sqL, const void* k, int64_t skB, int64_t skH, int64_t skL,
                          const void* v, int64_t svB, int64_t svH, int64_t svL, const void* mask,
                          int mask_dtype, int64_t mB, int64_t mH, int64_t mI, int64_t mJ, int causal,
                          float scale, void* out, void* workspace, int64_t workspace_bytes,
                          void* stream) {
  if (!is_float_dtype(dtype)) return fail(BIOPS_ERR_DTYPE, "unsupported dtype %d", dtype);
  if (batch < 0 || hq < 0 || hkv <= 0 || lq < 0 || lk < 0 || d < 0 || dv < 0)
    return fail(BIOPS_ERR_ARG, "invalid attention sizes");
  if (hq % hkv != 0) return fail(BIOPS_ERR_ARG, "query heads must be a multiple of kv heads");
  if (mask && causal != BIOPS_CAUSAL_NONE) return fail(BIOPS_ERR_ARG, "mask and causal are exclusive");
  if (mask && mask_dtype != BIOPS_BOOL && mask_dtype != dtype)
    return fail(BIOPS_ERR_DTYPE, "mask dtype must be bool or the score dtype");
  if (batch == 0 || hq == 0 || lq == 0 || dv == 0) return BIOPS_OK;
  const int64_t need = biops_sdpa_workspace_size(dtype, batch, hq, lq, lk);
  if (workspace_bytes < need) return fail(BIOPS_ERR_SIZE, "workspace %lld < %lld bytes",
                                          (long long)workspace_bytes, (long long)need);
  hipStream_t s = (hipStream_t)stream;
  const int64_t group = hq / hkv;
  const int64_t ld = varlen_score_ld(lk);
  int rc;
  if (lk > 0) {
    // S[b,h] = Q[b,h] . K[b,h/group]^T  (K^T is K-major: column j of K^T is row j of K)
    BmmArgs a{};
    a.A = q; a.B = k; a.C = workspace;
    a.M = lq; a.N = lk; a.K = d;
    a.lda = sqL; a.ldb = skL; a.ldc = ld;
    a.nb1 = batch; a.nb2 = hq; a.gB = group;
    a.sA1 = sqB; a.sA2 = sqH; a.sB1 = skB; a.sB2 = skH; a.sC1 = hq * lq * ld; a.sC2 = lq * ld;
    if ((rc = launch_bmm(dtype, a, kEpiPlain, true, s)) != BIOPS_OK) return rc;

    AttnSoftmaxArgs sm{};
    sm.s = workspace; sm.rows = batch * hq * lq; sm.lq = lq; sm.lk = lk; sm.hq = hq; sm.ld = ld;
    sm.scale = scale; sm.causal = causal; sm.mask = mask;
    sm.mask_kind = mask ? (mask_dtype == BIOPS_BOOL ? 1 : 2) : 0;
    sm.mB = mB; sm.mH = mH; sm.mI = mI; sm.mJ = mJ;
    const int64_t blocks = cdiv(sm.rows, kRowWaves);
    if (blocks > 0x7fffffffLL) return fail(BIOPS_ERR_ARG, "too many score rows");
    switch (dtype) {
      case BIOPS_F32: hipLaunchKernelGGL(attn_softmax_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, s, sm); break;
      case BIOPS_F16: hipLaunchKernelGGL(attn_softmax_kernel<f16_t>, dim3((unsigned)blocks), dim3(256), 0, s, sm); break;
      default: hipLaunchKernelGGL(attn_softmax_kernel<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, s, sm); break;
    }
    if ((rc = check_launch("attn_softmax_kernel")) != BIOPS_OK) return rc;
  }
  // O[b,h] = P[b,h] . V[b,h/group]  (V rows are N-major); lk == 0 gives zeros (K loop empty).
  BmmArgs o{};
  o.A = workspace; o.B = v; o.C = out;
  o.M = lq; o.N = dv; o.K = lk;
  o.lda = ld; o.ldb = svL; o.ldc = dv;
  o.nb1 = batch; o.nb2 = hq; o.gB = group;
  o.sA1 = hq * lq * ld; o.sA2 = lq * ld; o.sB1 = svB; o.sB2 = svH; o.sC1 = hq * lq * dv; o.sC2 = lq * dv;
  return launch_bmm(dtype, o, kEpiPlain, false, s);
}

extern "C" int64_t biops_varlen_plan_len(int64_t nseq) {
  return nseq < 0 ? -1 : kPlanHeader + kPlanStride * nseq;
}

extern "C" int64_t biops_varlen_plan(int64_t nseq, const int64_t* cu_q, const int64_t* cu_kv,
                                     int64_t hq, int64_t dv, int dtype, int64_t* plan) {
  const int elt = dtype_bytes(dtype);
  if (nseq < 0 || hq <= 0 || dv < 0 || elt == 0 || !cu_q || !cu_kv || !plan) {
    set_error("invalid varlen plan arguments");
    return -1;
  }
  int64_t items = 0, qk = 0, pv = 0, rows = 0, selems = 0, qtiles = 0;
  for (int64_t s = 0; s < nseq; ++s) {
    const int64_t q0 = cu_q[s], ql = cu_q[s + 1] - cu_q[s];
    const int64_t k0 = cu_kv[s], kl = cu_kv[s + 1] - cu_kv[s];
    if (ql < 0 || kl < 0) {
      set_error("cumulative sequence lengths must be nondecreasing");
      return -1;
    }
    if (ql == 0 || kl == 0) continue;
    int64_t* p = plan + kPlanHeader + kPlanStride * items;
    p[0] = q0; p[1] = ql; p[2] = k0; p[3] = kl; p[4] = selems;
    p[5] = qk; p[6] = pv; p[7] = rows;
    qk += hq * cdiv(ql, kVarlenBM) * cdiv(kl, kVarlenBN);
    pv += hq * cdiv(ql, kVarlenBM) * cdiv(dv, kVarlenBN);
    rows += hq * ql;
    selems += hq * ql * varlen_score_ld(kl);
    qtiles += cdiv(ql, kVarlenBM);
    ++items;
  }
  plan[0] = items; plan[1] = qk; plan[2] = pv; plan[3] = rows; plan[4] = selems;
  plan[5] = qtiles;
  plan[6] = plan[7] = 0;
  return selems * elt;
}

extern "C" int biops_varlen_sdpa(int dtype, int64_t hq, int64_t hkv, int64_t d, int64_t dv,
                                 const void* q, int64_t sq_t, int64_t sq_h, const void* k,
                                 int64_t sk_t, int64_t sk_h, const void* v, int64_t sv_t,
                                 int64_t sv_h, void* out, int64_t so_t, int64_t so_h,
                                 const int64_t* dplan, const int64_t* hplan, int causal, float scale,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
  if (!is_float_dtype(dtype)) return fail(BIOPS_ERR_DTYPE, "unsupported dtype %d", dtype);
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0 || d < 0 || dv < 0)
    return fail(BIOPS_ERR_ARG, "invalid varlen head configuration");
  if (!dplan || !hplan) return fail(BIOPS_ERR_ARG, "null plan");
  const int64_t items = hplan[0];
  if (items == 0 || dv == 0) return BIOPS_OK;
  const int64_t need = hplan[4] * dtype_bytes(dtype);
  if (workspace_bytes < need) return fail(BIOPS_ERR_SIZE, "workspace %lld < %lld bytes",
                                          (long long)workspace_bytes, (long long)need);
  hipStream_t s = (hipStream_t)stream;
  GroupedArgs g{};
  g.q = q; g.k = k; g.v = v; g.s = workspace; g.out = out; g.plan = dplan;
  g.items = items; g.heads = hq; g.group = hq / hkv; g.d = d; g.dv = dv;
  g.sq_t = sq_t; g.sq_h = sq_h; g.sk_t = sk_t; g.sk_h = sk_h; g.sv_t = sv_t; g.sv_h = sv_h;
  g.so_t = so_t; g.so_h = so_h;
  int rc;
  g.total_tiles = hplan[1];
  if ((rc = launch_grouped(dtype, g, kGroupQK, s)) != BIOPS_OK) return rc;

  VarlenSoftmaxArgs sm{workspace, dplan, items, hplan[3], hq, scale, causal};
  const int64_t blocks = cdiv(sm.rows, kRowWaves);
  if (blocks > 0x7fffffffLL) return fail(BIOPS_ERR_ARG, "too many score rows");
  switch (dtype) {
    case BIOPS_F32: hipLaunchKernelGGL(varlen_softmax_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, s, sm); break;
    case BIOPS_F16: hipLaunchKernelGGL(varlen_softmax_kernel<f16_t>, dim3((unsigned)blocks), dim3(256), 0, s, sm); break;
    default: hipLaunchKernelGGL(varlen_softmax_kernel<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, s, sm); break;
  }
  if ((rc = check_launch("varlen_softmax_kernel")) != BIOPS_OK) return rc;

  g.total_tiles = hplan[2];
  return launch_grouped(dtype, g, kGroupPV, s);
}
