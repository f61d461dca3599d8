"""Float64 CPU restatement of the reference operators (test infrastructure only).

Each function follows the cited lines of yiannisha/robotics-batch-invariant-ops:
``batch_invariant_ops/batch_invariant_ops.py`` (BIO) and ``batch_invariant_ops/moe.py`` (MOE).
Arithmetic is float64 with explicit roundings to the working dtype exactly where the reference
materialises a tensor of that dtype (GEMM outputs, the scaled / masked scores, softmax outputs,
the SwiGLU intermediates, the weighted routes and every partial slot sum).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

__all__ = [
    "rnd",
    "matmul",
    "bmm",
    "linear",
    "softmax",
    "log_softmax",
    "mean_dim",
    "mean_dims",
    "vector_norm",
    "sdpa",
    "sdpa_abs",
    "varlen_sdpa",
    "varlen_sdpa_abs",
    "moe",
    "moe_abs",
    "conv",
    "conv_abs",
    "gemm_abs",
    "gamma",
]

_INT_DTYPES = (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8)


def rnd(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Round a float64 tensor to ``dtype`` (round to nearest even), returned as float64."""
    return x.to(dtype).double()


def gamma(k: int, dtype: torch.dtype = torch.float32) -> float:
    """Higham's gamma_k = k u / (1 - k u) for the accumulation precision (fp32 here)."""
    u = 2.0**-24
    ku = k * u
    return ku / (1.0 - ku) if ku < 1 else math.inf


def gemm_abs(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """|A| @ |B| in float64: scales the dot-product error bound of every output element."""
    return a.double().abs() @ b.double().abs()


# ---------------------------------------------------------------------------- GEMM ----
def matmul(a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """C = A @ B (+ bias) rounded once to A's dtype; the bias joins the wide accumulator before
    the rounding (BIO 113-139 accumulate + 134-137 bias epilogue, 271-343 wrapper)."""
    out = a.double() @ b.double()
    if bias is not None:
        out = out + bias.double()
    return out.to(a.dtype)


def bmm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Per-batch C[i] = A[i] @ B[i], one rounding (BIO 142-229, 346-431)."""
    return (a.double() @ b.double()).to(a.dtype)


def linear(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """Leading dims flatten into GEMM rows; B = W^T (BIO 1608-1616)."""
    flat = x.reshape(-1, x.shape[-1])
    return matmul(flat, w.t(), bias).reshape(*x.shape[:-1], w.shape[0])


# ---------------------------------------------------------------- row reductions ----
def softmax(x: torch.Tensor, dim: int = -1, dtype: torch.dtype | None = None) -> torch.Tensor:
    """exp(x - max) / sum; a row whose max is -inf gives 0, not NaN (BIO 1093-1114)."""
    x64 = x.double()
    m = x64.amax(dim=dim, keepdim=True) if x64.numel() else x64
    all_neg_inf = m == -math.inf
    shifted = torch.where(all_neg_inf, torch.full_like(x64, -math.inf), x64 - m)
    e = torch.exp(shifted)
    s = e.sum(dim=dim, keepdim=True)
    out = torch.where(s == 0, torch.zeros_like(e), e / s)
    return out.to(dtype or x.dtype)


def log_softmax(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """x - max - log(sum exp(x - max)) (BIO 994-1034)."""
    x64 = x.double()
    m = x64.amax(dim=dim, keepdim=True)
    lse = torch.log(torch.exp(x64 - m).sum(dim=dim, keepdim=True))
    return (x64 - m - lse).to(x.dtype)


def mean_dim(x: torch.Tensor, dim: int, keepdim: bool = False, dtype: torch.dtype | None = None):
    """Mean over one dim; integer inputs produce fp32; the input is cast to the output dtype
    first (BIO 1411-1427); the sum is exact here (the kernels accumulate in fp32)."""
    if dtype is None:
        dtype = torch.float32 if x.dtype in _INT_DTYPES else x.dtype
    x = x.to(dtype)
    return x.double().mean(dim=dim, keepdim=keepdim).to(dtype)


def mean_dims(x: torch.Tensor, dims, keepdim: bool = False, dtype: torch.dtype | None = None):
    """Mean over several dims (all when empty) in the input (or given) dtype."""
    if dtype is not None:
        x = x.to(dtype)
    if not dims:
        dims = list(range(x.ndim))
    out_dtype = torch.float32 if x.dtype in _INT_DTYPES else x.dtype
    return x.to(out_dtype).double().mean(dim=tuple(dims), keepdim=keepdim).to(out_dtype)


def vector_norm(x: torch.Tensor, dim=None, keepdim: bool = False, dtype: torch.dtype | None = None):
    """sqrt(sum x^2) with the output in the (optionally cast) input dtype (BIO 1525-1597)."""
    if dtype is not None:
        x = x.to(dtype)
    dims = tuple(range(x.ndim)) if dim is None else ((dim,) if isinstance(dim, int) else tuple(dim))
    out = torch.sqrt((x.double() ** 2).sum(dim=dims, keepdim=keepdim))
    return out.to(x.dtype)


# ---------------------------------------------------------------------- attention ----
def _scalar_to_opmath(scale: float) -> float:
    """Python scalars multiply low-precision tensors in fp32 (the tensor op's compute type)."""
    return float(torch.tensor(scale, dtype=torch.float32))


def _sdpa_probs(q, k, v, attn_mask=None, is_causal=False, scale=None, enable_gqa=False):
    """The probabilities P (rounded to q.dtype, held in float64) and the GQA-expanded V of
    ``sdpa``; the roundings are listed there."""
    dt = q.dtype
    if enable_gqa:
        rep = q.shape[-3] // k.shape[-3]
        k = k.repeat_interleave(rep, dim=-3)
        v = v.repeat_interleave(rep, dim=-3)
    d = q.shape[-1]
    s = rnd(q.double() @ k.double().transpose(-1, -2), dt)
    sc = _scalar_to_opmath(scale if scale is not None else 1.0 / math.sqrt(d))
    s = rnd(s * sc, dt)
    lq, lk = q.shape[-2], k.shape[-2]
    if is_causal:
        keep = torch.ones(lq, lk, dtype=torch.bool).tril()
        s = s.masked_fill(~keep, -math.inf)
    elif attn_mask is not None:
        if attn_mask.dtype == torch.bool:
            s = s.masked_fill(~attn_mask, -math.inf)
        else:
            res_dtype = torch.promote_types(dt, attn_mask.dtype)
            s = rnd(s + attn_mask.double(), res_dtype)
    return softmax(s, dim=-1, dtype=dt).double(), v


def sdpa(q, k, v, attn_mask=None, is_causal=False, scale=None, enable_gqa=False):
    """Eager attention with the reference's roundings (BIO 1148-1213):
    S = round(Q K^T); S = round(S * scale); causal top-left / bool mask -> -inf, additive mask
    -> round(S + mask); P = softmax(S) in q.dtype; O = round(P V)."""
    p, v = _sdpa_probs(q, k, v, attn_mask, is_causal, scale, enable_gqa)
    return rnd(p @ v.double(), q.dtype).to(q.dtype)


def sdpa_abs(q, k, v, attn_mask=None, is_causal=False, scale=None, enable_gqa=False):
    """P |V| in float64 with the P of ``sdpa``: the per-element scale of the output's error
    bound (one ulp of a probability moves an output by at most that ulp times P |V|)."""
    p, v = _sdpa_probs(q, k, v, attn_mask, is_causal, scale, enable_gqa)
    return p @ v.double().abs()


def _varlen(q, k, v, cu_q, cu_kv, is_causal, causal_type, scale, per_sequence):
    """Packed varlen attention (BIO 1216-1344): each sequence alone through ``per_sequence``
    (``sdpa`` or ``sdpa_abs``); rows outside every sequence and sequences with empty key
    ranges are zero; BottomRight causal keeps j <= i + (kv - q), TopLeft / None keeps j <= i."""
    cu_q = [int(x) for x in cu_q]
    cu_kv = [int(x) for x in cu_kv]
    out = None
    name = getattr(causal_type, "name", None)
    if name is None and causal_type is not None:
        name = str(causal_type).rsplit(".", 1)[-1]
    for q0, q1, k0, k1 in zip(cu_q[:-1], cu_q[1:], cu_kv[:-1], cu_kv[1:]):
        ql, kl = q1 - q0, k1 - k0
        if ql == 0 or kl == 0:
            continue
        qi = q[:, q0:q1].transpose(1, 2)
        ki = k[:, k0:k1].transpose(1, 2)
        vi = v[:, k0:k1].transpose(1, 2)
        mask = None
        causal = is_causal
        if is_causal and ql != kl:
            qi_idx = torch.arange(ql)[:, None]
            ki_idx = torch.arange(kl)[None, :]
            shift = kl - ql if name == "BottomRight" else 0
            mask = ki_idx <= qi_idx + shift
            causal = False
        o = per_sequence(qi, ki, vi, attn_mask=mask, is_causal=causal, scale=scale,
                         enable_gqa=qi.shape[-3] != ki.shape[-3])
        if out is None:
            out = torch.zeros((1, q.shape[1], q.shape[2], v.shape[3]), dtype=o.dtype)
        out[:, q0:q1] = o.transpose(1, 2)
    if out is None:
        out = torch.zeros((1, q.shape[1], q.shape[2], v.shape[3]), dtype=v.dtype)
    return out


def varlen_sdpa(q, k, v, cu_q, cu_kv, *, is_causal=False, causal_type=None, scale=None):
    """Packed varlen attention with the rules of ``_varlen``, in the input dtype."""
    return _varlen(q, k, v, cu_q, cu_kv, is_causal, causal_type, scale, sdpa).to(v.dtype)


def varlen_sdpa_abs(q, k, v, cu_q, cu_kv, *, is_causal=False, causal_type=None, scale=None):
    """P |V| per packed output element (float64; zero where the output is zero)."""
    return _varlen(q, k, v, cu_q, cu_kv, is_causal, causal_type, scale, sdpa_abs).double()


# ---------------------------------------------------------------------------- MoE ----
def _moe_routes(hidden, routing_weights, selected, gate, up, down):
    """The weighted routes round(y[sel] * round(w)) of every slot, in slot order (MOE 75-87):
    g = round(x gate_e^T), u = round(x up_e^T), a = round(round(silu(g)) * u),
    y = round(a down_e^T)."""
    dt = hidden.dtype
    x = hidden.double()
    T, k = selected.shape
    g = rnd(torch.einsum("td,eid->eti", x, gate.double()), dt)
    u = rnd(torch.einsum("td,eid->eti", x, up.double()), dt)
    a = rnd(rnd(g / (1.0 + torch.exp(-g)), dt) * u, dt)
    y = rnd(torch.einsum("eti,edi->etd", a, down.double()), dt)
    w = rnd(routing_weights.double(), dt)
    t_idx = torch.arange(T)
    return [rnd(y[selected[:, s], t_idx] * w[:, s : s + 1], dt) for s in range(k)]


def moe(hidden, routing_weights, selected, gate, up, down):
    """Dense top-k SwiGLU MoE with the reference's roundings (MOE 75-91): the routes of
    ``_moe_routes`` summed left to right over the slots with a rounding after every add."""
    dt = hidden.dtype
    T, k = selected.shape
    D = hidden.shape[1]
    if T == 0:
        return hidden.new_empty((0, D))
    if k == 0:
        return hidden.new_zeros((T, D))
    out = None
    for route in _moe_routes(hidden, routing_weights, selected, gate, up, down):
        out = route if out is None else rnd(out + route, dt)
    return out.to(dt)


def moe_abs(hidden, routing_weights, selected, gate, up, down):
    """sum over the slots of |round(w) y| (float64): the per-element scale of the output's error
    bound (one ulp of a route or of a partial sum is at most one ulp of this sum)."""
    T, k = selected.shape
    out = torch.zeros(T, hidden.shape[1], dtype=torch.float64)
    for route in _moe_routes(hidden, routing_weights, selected, gate, up, down) if T and k else ():
        out = out + route.abs()
    return out


# -------------------------------------------------------------------- convolution ----
def _conv_f64(x, w, stride, padding, dilation, transposed, output_padding, groups):
    nd = x.ndim - 2
    if transposed:
        f = {1: F.conv_transpose1d, 2: F.conv_transpose2d, 3: F.conv_transpose3d}[nd]
        return f(x, w, None, stride, padding, output_padding, groups, dilation)
    f = {1: F.conv1d, 2: F.conv2d, 3: F.conv3d}[nd]
    return f(x, w, None, stride, padding, dilation, groups)


def conv(x, w, bias, stride, padding, dilation, transposed, output_padding, groups):
    """aten::convolution with the reference's roundings (BIO 434-971).  Depthwise 1-D
    (groups == C_in == C_out, one channel per group, BIO 531): the taps and the bias summed in
    the wide accumulator, one rounding (BIO 435-494).  Every other form goes through bmm_persistent
    (one rounding of the patch dot products) and then adds the bias as a separate tensor op, which
    rounds again (BIO 590-595, 675-680, 775-780, 818-826, 898-906)."""
    dt = x.dtype
    nd = x.ndim - 2
    acc = _conv_f64(x.double(), w.double(), stride, padding, dilation, transposed, output_padding, groups)
    shape = (1, -1) + (1,) * nd
    depthwise = nd == 1 and not transposed and groups == x.shape[1] == w.shape[0] and w.shape[1] == 1
    if depthwise:
        out = acc if bias is None else acc + bias.double().reshape(shape)
        return out.to(dt)
    out = rnd(acc, dt)
    if bias is not None:
        out = rnd(out + bias.double().reshape(shape), dt)
    return out.to(dt)


def conv_abs(x, w, stride, padding, dilation, transposed, output_padding, groups):
    """The convolution of |x| and |w| in float64: scales each output's dot-product error bound."""
    return _conv_f64(x.double().abs(), w.double().abs(), stride, padding, dilation, transposed,
                     output_padding, groups)
