"""Tolerances for comparing the HIP kernels with the float64 CPU oracle.

GEMM-shaped results (one rounding after an fp32 accumulation of K products):
    |gpu - oracle| <= r_out * |oracle| + gamma_K * (1 + r_out) * (|A| @ |B|)      (elementwise)
The kernel rounds its fp32 sum s' (|s' - s| <= gamma_K |A||B|, gamma_K = K 2^-24 / (1 - K 2^-24))
and the oracle rounds the exact sum s; two roundings of values that close differ by at most
|s' - s| plus one ulp of the output, and one ulp is at most r_out * |oracle| with
r_out = 2^-7 (bf16), 2^-10 (fp16).  For fp32 outputs r_out = 1e-5 (the north-star rtol; the
output rounding itself is 2^-24).

Composite ops (attention, MoE) round several times; each extra rounding of an intermediate can
move the result by one more ulp of that intermediate, so their bound is n_roundings ulps of
the output dtype relative to the natural output scale (documented per test).
"""

from __future__ import annotations

import torch

ULP = {torch.float32: 2.0**-23, torch.float16: 2.0**-10, torch.bfloat16: 2.0**-7}


def gamma(k: int) -> float:
    ku = k * 2.0**-24
    return ku / (1.0 - ku)


def assert_gemm_close(actual: torch.Tensor, expected: torch.Tensor, abs_product: torch.Tensor, k: int):
    """Elementwise GEMM bound; ``abs_product`` = |A| @ |B| (+|bias|) in float64."""
    dtype = actual.dtype
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    r_out = 1e-5 if dtype == torch.float32 else ULP[dtype]
    bound = r_out * e.abs() + gamma(k) * (1 + r_out) * abs_product.double().cpu()
    err = (a - e).abs()
    bad = ~(err <= bound)
    assert not bool(bad.any()), (
        f"{int(bad.sum())} of {bad.numel()} elements outside the GEMM bound; "
        f"max err {float(err.max()):.3e}, at a bound of {float(bound.flatten()[int(err.flatten().argmax())]):.3e}"
    )


def assert_close_scaled(actual, expected, *, rel: float, abs_scale: float, what: str = ""):
    """|a - e| <= rel * |e| + abs_scale elementwise (NaN positions must agree)."""
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    nan_a, nan_e = torch.isnan(a), torch.isnan(e)
    assert torch.equal(nan_a, nan_e), f"{what}: NaN pattern differs"
    a = torch.where(nan_a, torch.zeros_like(a), a)
    e = torch.where(nan_e, torch.zeros_like(e), e)
    inf = torch.isinf(e)
    assert torch.equal(a[inf], e[inf]), f"{what}: infinities differ"
    err = (a - e).abs()
    err = torch.where(inf, torch.zeros_like(err), err)
    bound = rel * e.abs() + abs_scale
    bound = torch.where(inf, torch.ones_like(bound), bound)
    bad = ~(err <= bound)
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {bad.numel()} outside rel {rel:g} + abs {abs_scale:g}; "
        f"max err {float(err.max()):.3e}"
    )


def assert_first_sample_equal(alone: torch.Tensor, batched: torch.Tensor) -> None:
    """Bitwise equality of sample 0 (test_batch_invariance.py:35-39 semantics)."""
    assert torch.equal(alone, batched[:1]), (
        f"first sample changed: max diff {(alone.float() - batched[:1].float()).abs().max().item()}"
    )


def assert_bitwise(a: torch.Tensor, b: torch.Tensor, what: str = "") -> None:
    """Same bits (also for NaN / -0): compares the raw storage."""
    assert a.shape == b.shape and a.dtype == b.dtype, f"{what}: {a.shape}/{a.dtype} vs {b.shape}/{b.dtype}"
    ia = a.contiguous().view(torch.int16 if a.element_size() == 2 else torch.int32)
    ib = b.contiguous().view(torch.int16 if b.element_size() == 2 else torch.int32)
    diff = int((ia != ib).sum())
    assert diff == 0, f"{what}: {diff} elements differ bitwise"


# Share of elements that must carry the oracle's exact bits in a composite op's 16-bit output.
# The kernels round where the oracle rounds, so only elements whose fp32 sums straddle a
# rounding boundary may differ (fp32 emulations on the CPU: over 99.8 % equal in bf16, over 98 %
# in fp16).  One dropped intermediate rounding, a reordered slot sum or a wrong GQA head map
# leaves under 60 % equal (the same emulations), so these shares catch such mistakes where an
# error bound alone cannot.
MIN_EXACT = {torch.bfloat16: 0.97, torch.float16: 0.95, torch.float32: 0.0}


def assert_composite_close(actual, expected, scale, *, n: int = 2, min_exact: float | None = None,
                           what: str = ""):
    """Composite ops (attention, MoE) against the float64 oracle, in two parts.

    * Every element: |a - e| <= r * (|e| + n * scale).  ``scale`` is the oracle's per-element
      magnitude of the summed terms (P |V| for attention, sum_s |round(w_s) y_s| for MoE); an
      intermediate that lands one ulp (r) away moves the output by at most r times that
      magnitude, and the final rounding adds one ulp of the output.  r is the output dtype's ulp
      (2^-7 bf16, 2^-10 fp16) or the north-star rtol 1e-5 for fp32.
    * The share of elements bitwise equal to the oracle is at least ``min_exact`` (default
      ``MIN_EXACT`` by dtype).
    """
    dtype = actual.dtype
    r = 1e-5 if dtype == torch.float32 else ULP[dtype]
    a = actual.detach().double().cpu()
    e = expected.detach().double().cpu()
    s = scale.detach().double().cpu()
    nan_a, nan_e = torch.isnan(a), torch.isnan(e)
    assert torch.equal(nan_a, nan_e), f"{what}: NaN pattern differs"
    a = torch.where(nan_a, torch.zeros_like(a), a)
    e = torch.where(nan_e, torch.zeros_like(e), e)
    err = (a - e).abs()
    bound = r * (e.abs() + n * s)
    bad = ~(err <= bound)
    worst = int((err - bound).flatten().argmax()) if err.numel() else 0
    assert not bool(bad.any()), (
        f"{what}: {int(bad.sum())} of {bad.numel()} elements outside the per-element bound; worst err "
        f"{float(err.flatten()[worst]):.3e} at a bound of {float(bound.flatten()[worst]):.3e}"
    )
    if min_exact is None:
        min_exact = MIN_EXACT[dtype]
    exact = float((a == e).double().mean()) if a.numel() else 1.0
    print(f"[parity] {what}: {exact:.4f} of {a.numel()} elements bitwise equal", flush=True)
    assert exact >= min_exact, (
        f"{what}: only {exact:.4f} of the elements carry the oracle's bits (at least {min_exact} expected)")
