"""The five BASELINE configs at their own sizes on the GPU.

Each test checks (1) bitwise batch invariance the way the config states it and (2) parity of
the HIP path with the float64 oracle on sampled rows, heads, sequences or tokens.  Inputs are
made on the CPU from the configs' seeds (2/20, 3/30, 4, 5) so the oracle sees the same values.
Tolerances:

* GEMM-shaped outputs: ``assert_gemm_close`` -- one ulp of the output (rtol 1e-5 for fp32)
  plus gamma_K |A||B| (tests/_tol.py).
* fp32 row reductions (mean of squares): rtol 1e-5 (the north-star fp32 tolerance).
* bf16 row reductions: one bf16 ulp of the result plus gamma_N times the mean of |x|.
* attention and MoE (tests/_parity.py): every element within one bf16 ulp times
  (|out| + n * its own magnitude of terms) -- P |V| for attention (n = 2), the sum of the
  weighted routes' magnitudes for MoE (n = 2 + top_k) -- and at least 97 % of the elements
  carrying the oracle's exact bits.  The kernels round where the reference does, so dropping
  one intermediate rounding, reordering the slot sum or mapping query heads to the wrong KV
  head would leave well under 60 % of the bits equal.

The reference's own versions of these checks: README.md:62-76 (C1) and
test_batch_invariance.py:512-780 (C3-C5).
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from batch_invariant_ops import (
    deterministic_token_choice_moe,
    linear_batch_invariant,
    matmul_persistent,
    scaled_dot_product_attention_batch_invariant as sdpa,
    set_batch_invariant_mode,
    varlen_scaled_dot_product_attention_batch_invariant as varlen,
)
from batch_invariant_ops.moe import _moe

from _parity import check_moe, check_sdpa, check_varlen
from _tol import ULP, assert_bitwise, assert_close_scaled, assert_gemm_close, gamma

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def say(msg: str) -> None:
    print(f"[configs] {msg}", flush=True)


@pytest.fixture
def path_env(monkeypatch):
    """Select the fused ('fused') or the materialised-score ('materialized') attention path."""

    def select(path):
        if path == "materialized":
            monkeypatch.setenv("BIOPS_ATTENTION_MATERIALIZE", "1")
        else:
            monkeypatch.delenv("BIOPS_ATTENTION_MATERIALIZE", raising=False)

    return select


# ------------------------------------------------------------------------------ C1 ----
def test_c1_readme_linspace_fp32_mm():
    """README.md:62-76: mm(A[:1], B) must equal mm(A, B)[:1]; also parity of sampled rows."""
    say("C1 fp32 mm 2048x4096 . 4096x4096")
    a = torch.linspace(-100, 100, 2048 * 4096).reshape(2048, 4096)
    b = torch.linspace(-100, 100, 4096 * 4096).reshape(4096, 4096)
    ag, bg = a.cuda(), b.cuda()
    full = matmul_persistent(ag, bg)
    assert_bitwise(matmul_persistent(ag[:1], bg), full[:1], "C1 M=1 vs M=2048")
    with set_batch_invariant_mode():
        assert_bitwise(torch.mm(ag[:1], bg), full[:1], "C1 torch.mm under the mode")
        assert_bitwise(torch.mm(ag[:7], bg), full[:7], "C1 M=7")
    rows = [0, 1, 31, 32, 1023, 2047]
    sub = a[rows]
    assert_gemm_close(full[rows], oracle.matmul(sub, b), oracle.gemm_abs(sub, b), 4096)


# ------------------------------------------------------------------------------ C2 ----
@pytest.fixture(scope="module")
def c2_inputs():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(32, 256, 2048, generator=g).to(BF16)
    g = torch.Generator().manual_seed(20)
    w1 = (torch.randn(8192, 2048, generator=g) * 0.02).to(BF16)
    b1 = (torch.randn(8192, generator=g) * 0.02).to(BF16)
    w2 = (torch.randn(2048, 8192, generator=g) * 0.02).to(BF16)
    return x, w1, b1, w2


def _c2_stack(x, w1, b1, w2, rw):
    """Two linears, HF-style RMSNorm (x.float().pow(2).mean(-1)), then mean and L2 norm."""
    h = F.linear(x, w1, b1)
    y = F.linear(h, w2)
    var = y.float().pow(2).mean(-1, keepdim=True)
    yn = (y.float() * torch.rsqrt(var + 1e-6)).to(BF16) * rw
    return {"h": h, "y": y, "var": var, "yn": yn, "mean": yn.mean(-1),
            "norm": torch.linalg.vector_norm(yn, dim=-1)}


def test_c2_stack_batch_invariant_and_matches_oracle(c2_inputs):
    x, w1, b1, w2 = c2_inputs
    xg, w1g, b1g, w2g = (t.cuda() for t in c2_inputs)
    rw = torch.ones(2048, dtype=BF16, device="cuda")
    say("C2 stack B in (1, 8, 32)")
    with set_batch_invariant_mode():
        outs = {b: _c2_stack(xg[:b], w1g, b1g, w2g, rw) for b in (1, 8, 32)}
    for b in (1, 8):
        for name in outs[32]:
            assert_bitwise(outs[b][name], outs[32][name][:b], f"C2 {name} B={b} vs B=32")

    o = {name: t[0].cpu() for name, t in outs[1].items()}
    # each stage against the oracle applied to the GPU's own previous stage
    ref_h = oracle.linear(x[0], w1, b1)
    assert_gemm_close(o["h"], ref_h, oracle.gemm_abs(x[0], w1.t()) + b1.double().abs(), 2048)
    ref_y = oracle.linear(o["h"], w2)
    assert_gemm_close(o["y"], ref_y, oracle.gemm_abs(o["h"], w2.t()), 8192)
    ref_var = oracle.mean_dim(o["y"].float().pow(2), -1, keepdim=True)
    assert_close_scaled(o["var"], ref_var, rel=1e-5, abs_scale=0.0, what="C2 mean(y^2)")
    ref_yn = (o["y"].double() * torch.rsqrt(o["var"].double() + 1e-6)).to(BF16)
    assert_close_scaled(o["yn"], ref_yn, rel=2 * ULP[BF16], abs_scale=0.0, what="C2 RMSNorm")
    yn = o["yn"]
    slack = gamma(2048) * float(yn.double().abs().mean())
    assert_close_scaled(o["mean"], oracle.mean_dim(yn, -1), rel=ULP[BF16], abs_scale=slack, what="C2 mean")
    assert_close_scaled(o["norm"], oracle.vector_norm(yn, dim=-1), rel=ULP[BF16], abs_scale=0.0,
                        what="C2 vector_norm")


# ------------------------------------------------------------- metric GEMM, every M ----
# Row counts on both sides of every change of the automatic tile choice for the two metric
# shapes: the skinny entry (<= one 32x32 block per compute unit: M <= 32 at N = 8192, M <= 128
# at N = 2048), the 32x32 four-per-unit preference, the four-wave blocks and the round counts.
TRANSITION_M = (1, 2, 3, 7, 8, 9, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257,
                511, 512, 513, 767, 768, 1023, 1024, 1025, 1536, 2047, 2048, 2049, 3072, 4095, 4096,
                4097, 6144, 8191)


@pytest.mark.parametrize(("n", "k", "with_bias"), ((8192, 2048, True), (2048, 8192, False)))
def test_metric_gemm_rows_identical_across_tile_choices(n, k, with_bias):
    g = torch.Generator().manual_seed(2900 + n)
    x = torch.randn(8192, k, generator=g).to(BF16).cuda()
    w = (torch.randn(n, k, generator=g) * 0.02).to(BF16).cuda()
    bias = (torch.randn(n, generator=g) * 0.02).to(BF16).cuda() if with_bias else None
    full = linear_batch_invariant(x, w, bias)
    for m in TRANSITION_M:
        assert_bitwise(linear_batch_invariant(x[:m], w, bias), full[:m], f"N={n} K={k} M={m}")
    # a sample at another row offset (other tile position, other workgroup)
    assert_bitwise(linear_batch_invariant(x[4000:4033], w, bias), full[4000:4033], "rows 4000..4032")
    rows = [0, 4095, 8191]
    xs = x[rows].cpu()
    ref = oracle.linear(xs, w.cpu(), None if bias is None else bias.cpu())
    absprod = oracle.gemm_abs(xs, w.cpu().t()) + (0 if bias is None else bias.cpu().double().abs())
    assert_gemm_close(full[rows], ref, absprod, k)


# ------------------------------------------------------------------------------ C3 ----
@pytest.fixture(scope="module")
def c3_inputs():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(16, 16, 1024, 128, generator=g).to(BF16)
    k = torch.randn(16, 4, 1024, 128, generator=g).to(BF16)
    v = torch.randn(16, 4, 1024, 128, generator=g).to(BF16)
    g = torch.Generator().manual_seed(30)
    mask = torch.rand(16, 1, 1024, 1024, generator=g) * -10
    mask[torch.rand(16, 1, 1024, 1024, generator=g) < 0.1] = -math.inf
    mask = mask.to(BF16)
    return q, k, v, mask


@pytest.mark.parametrize("path", ("fused", "materialized"))
@pytest.mark.parametrize("variant", ("causal", "mask"))
def test_c3_sdpa_at_size(c3_inputs, variant, path, path_env):
    q, k, v, mask = c3_inputs
    qg, kg, vg, mg = (t.cuda() for t in c3_inputs)
    path_env(path)
    say(f"C3 {variant} {path} B in (1, 4, 16)")

    def run(b):
        kw = {"is_causal": True} if variant == "causal" else {"attn_mask": mg[:b]}
        return sdpa(qg[:b], kg[:b], vg[:b], enable_gqa=True, scale=1 / math.sqrt(128), **kw)

    o16 = run(16)
    assert_bitwise(run(1), o16[:1], f"C3 {variant} B=1 vs B=16")
    assert_bitwise(run(4), o16[:4], f"C3 {variant} B=4 vs B=16")
    # oracle on the first and the last sample, one query head of each KV group; heads 1, 6, 11
    # and 14 read KV heads h // 4 = 0, 1, 2, 3, which h % 4 = 1, 2, 3, 2 would not
    for b in (0, 15):
        for h in (1, 6, 11, 14):
            kv = h // 4
            kw = {"is_causal": True} if variant == "causal" else {"attn_mask": mask[b : b + 1]}
            check_sdpa(o16[b : b + 1, h : h + 1], q[b : b + 1, h : h + 1], k[b : b + 1, kv : kv + 1],
                       v[b : b + 1, kv : kv + 1], scale=1 / math.sqrt(128), what=f"C3 {variant} {path} b={b} h={h}",
                       **kw)


# ------------------------------------------------------------------------------ C4 ----
@pytest.fixture(scope="module")
def c4_inputs():
    g = torch.Generator().manual_seed(4)
    lengths = torch.randint(64, 2049, (32,), generator=g)
    total = int(lengths.sum())
    q = torch.randn(1, total, 8, 64, generator=g).to(BF16)
    k = torch.randn(1, total, 2, 64, generator=g).to(BF16)
    v = torch.randn(1, total, 2, 64, generator=g).to(BF16)
    cu = torch.zeros(33, dtype=torch.int32)
    cu[1:] = torch.cumsum(lengths, 0)
    return q, k, v, cu


@pytest.mark.parametrize("path", ("fused", "materialized"))
def test_c4_varlen_at_size(c4_inputs, path, path_env):
    q, k, v, cu = c4_inputs
    qg, kg, vg, cug = q.cuda(), k.cuda(), v.cuda(), cu.cuda()
    path_env(path)
    say(f"C4 varlen {path}: 32 sequences, {q.shape[1]} tokens")
    packed = varlen(qg, kg, vg, cug, cug, is_causal=True, causal_type="BottomRight")
    for s in range(32):
        s0, s1 = int(cu[s]), int(cu[s + 1])
        one = torch.tensor([0, s1 - s0], dtype=torch.int32, device="cuda")
        alone = varlen(qg[:, s0:s1], kg[:, s0:s1], vg[:, s0:s1], one, one, is_causal=True,
                       causal_type="BottomRight")
        assert_bitwise(alone, packed[:, s0:s1], f"C4 sequence {s} alone vs packed")
    for s in (0, 13, 31):
        s0, s1 = int(cu[s]), int(cu[s + 1])
        one = torch.tensor([0, s1 - s0], dtype=torch.int32)
        check_varlen(packed[:, s0:s1], q[:, s0:s1], k[:, s0:s1], v[:, s0:s1], one, one, is_causal=True,
                     causal_type="BottomRight", what=f"C4 {path} sequence {s} ({s1 - s0} tokens)")


# ------------------------------------------------------------------------------ C5 ----
@pytest.fixture(scope="module")
def c5_inputs():
    g = torch.Generator().manual_seed(5)
    hidden = torch.randn(4096, 2048, generator=g).to(BF16)
    gate_up = (torch.randn(64, 2048, 1536, generator=g) * 0.02).to(BF16)
    down = (torch.randn(64, 768, 2048, generator=g) * 0.02).to(BF16)
    probs = torch.softmax(torch.randn(4096, 64, generator=g), -1)
    weights, selected = torch.topk(probs, 8, dim=-1)
    return hidden, gate_up, down, weights, selected


def _expert_views(gate_up, down):
    """C5's fused weights as the reference's [E, I, D] gate / up (gate first) and [E, D, I] down."""
    return gate_up[..., :768].transpose(1, 2), gate_up[..., 768:].transpose(1, 2), down.transpose(1, 2)


def test_c5_moe_at_size(c5_inputs):
    hidden, gate_up, down, weights, selected = c5_inputs
    gate, up, dn = _expert_views(gate_up.cuda(), down.cuda())
    x, w, sel = hidden.cuda(), weights.cuda(), selected.cuda()
    say("C5 MoE T=4096 in batches of 4096 / 256 / 1")
    full = deterministic_token_choice_moe(x, w, sel, gate, up, dn)
    by_256 = torch.cat([deterministic_token_choice_moe(x[t : t + 256], w[t : t + 256], sel[t : t + 256],
                                                       gate, up, dn) for t in range(0, 4096, 256)])
    assert_bitwise(by_256, full, "C5 batches of 256 vs 4096")
    by_1 = torch.cat([deterministic_token_choice_moe(x[t : t + 1], w[t : t + 1], sel[t : t + 1], gate, up, dn)
                      for t in range(4096)])
    assert_bitwise(by_1, full, "C5 batches of 1 vs 4096")
    say("C5 sparse vs dense evaluation")
    assert_bitwise(_moe(x, w, sel, gate, up, dn, sparse=False), full, "C5 dense vs sparse")

    # oracle on sampled tokens, restricted to the experts they select
    tokens = sorted({0, 1, 255, 256, 2049, 4095, *range(7, 4096, 157)})
    sel_t = selected[tokens]
    used = torch.unique(sel_t)
    g_cpu, u_cpu, d_cpu = _expert_views(gate_up[used], down[used])
    check_moe(full[tokens], hidden[tokens], weights[tokens], torch.searchsorted(used, sel_t), g_cpu, u_cpu,
              d_cpu, what="C5 sampled tokens")
