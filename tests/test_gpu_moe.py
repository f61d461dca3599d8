"""Deterministic token-choice MoE on the GPU (reference tests test_batch_invariance.py:745-780).

Parity: the MoE rounds gate, up, silu(gate), the SwiGLU product, the down projection, each
weighted route and each partial slot sum, where the reference does.  Random inputs are checked
per element (one ulp of the output dtype times |out| + (2 + top_k) times the token's sum of
route magnitudes) and by the share of elements carrying the oracle's exact bits
(tests/_parity.py); the known-answer cases (tests/_moe_known.py) pin each rounding and the slot
order exactly, on the dense and the sparse evaluation and on every token alone.
"""

import pytest
import torch
import torch.nn.functional as F

import oracle
from batch_invariant_ops import deterministic_token_choice_moe as moe

from batch_invariant_ops.moe import _IndexWatch, _moe, check_moe_indices

from _moe_known import CASES, known_answer_problem, midpoint_margin, silu_sweep_problem
from _parity import check_moe
from _tol import ULP, assert_bitwise, assert_close_scaled

pytestmark = pytest.mark.gpu


def randn(*shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def routing(tokens, experts, k, seed):
    g = torch.Generator().manual_seed(seed)
    selected = torch.stack([torch.randperm(experts, generator=g)[:k] for _ in range(tokens)])
    weights = torch.rand(tokens, k, generator=g)
    return weights, selected


def test_moe_matches_route_by_route_loop():
    """Brute-force route loop of the reference test (float32, test_batch_invariance.py:757-766)."""
    hidden = randn(7, 12, seed=7400)
    gate = randn(5, 16, 12, seed=7401)
    up = randn(5, 16, 12, seed=7402)
    down = randn(5, 12, 16, seed=7403)
    g = torch.Generator().manual_seed(7404)
    selected = torch.randint(0, 5, (7, 3), generator=g)
    weights = torch.rand(7, 3, generator=g)
    args = [t.cuda() for t in (hidden, weights, selected, gate, up, down)]
    actual = moe(*args)
    assert_bitwise(actual, moe(*args), "repeat call")
    expected = torch.zeros(7, 12, dtype=torch.float64)
    for t in range(7):
        for s in range(3):
            e = selected[t, s]
            h = hidden[t].double()
            inter = F.silu(gate[e].double() @ h) * (up[e].double() @ h)
            expected[t] += (down[e].double() @ inter) * weights[t, s].double()
    assert_close_scaled(actual, expected, rel=2e-5, abs_scale=2e-5, what="route loop")


@pytest.mark.parametrize("dtype", (torch.float32, torch.bfloat16, torch.float16))
def test_moe_matches_oracle(dtype):
    T, E, D, I, k = 37, 6, 64, 80, 3
    hidden = randn(T, D, seed=7410, dtype=dtype)
    gate = randn(E, I, D, seed=7411, dtype=dtype, scale=0.2)
    up = randn(E, I, D, seed=7412, dtype=dtype, scale=0.2)
    down = randn(E, D, I, seed=7413, dtype=dtype, scale=0.2)
    w, sel = routing(T, E, k, 7414)
    out = moe(*(t.cuda() for t in (hidden, w, sel, gate, up, down)))
    check_moe(out, hidden, w, sel, gate, up, down, what=f"moe {dtype}")


def test_moe_is_batch_invariant():
    hidden = randn(11, 64, seed=7425).cuda()
    gate = randn(7, 80, 64, seed=7426).cuda()
    up = randn(7, 80, 64, seed=7427).cuda()
    down = randn(7, 64, 80, seed=7428).cuda()
    g = torch.Generator().manual_seed(7429)
    selected = torch.randint(0, 7, (11, 4), generator=g).cuda()
    weights = torch.rand(11, 4, generator=g).cuda()
    alone = moe(hidden[:1], weights[:1], selected[:1], gate, up, down)
    together = moe(hidden, weights, selected, gate, up, down)
    assert_bitwise(alone, together[:1], "token 0")
    mid = moe(hidden[5:8], weights[5:8], selected[5:8], gate, up, down)
    assert_bitwise(mid, together[5:8], "tokens 5..7")


def test_moe_fused_gate_up_layout():
    """gate/up given as transposed halves of a fused [E, D, 2I] tensor (N-major operands)."""
    T, E, D, I, k = 9, 4, 48, 40, 2
    hidden = randn(T, D, seed=7440, dtype=torch.bfloat16)
    gu = randn(E, D, 2 * I, seed=7441, dtype=torch.bfloat16, scale=0.1)
    dn = randn(E, I, D, seed=7442, dtype=torch.bfloat16, scale=0.1)
    w, sel = routing(T, E, k, 7443)
    gate, up, down = gu[..., :I].transpose(1, 2), gu[..., I:].transpose(1, 2), dn.transpose(1, 2)
    out = moe(hidden.cuda(), w.cuda(), sel.cuda(), gate.cuda(), up.cuda(), down.cuda())
    contiguous = moe(hidden.cuda(), w.cuda(), sel.cuda(), gate.contiguous().cuda(), up.contiguous().cuda(),
                     down.contiguous().cuda())
    assert_bitwise(out, contiguous, "strided vs contiguous weights")
    check_moe(out, hidden, w, sel, gate, up, down, what="fused gate_up layout")


def test_moe_edge_cases(monkeypatch):
    hidden = randn(3, 8, seed=7450).cuda()
    gate = randn(2, 4, 8, seed=7451).cuda()
    down = randn(2, 8, 4, seed=7452).cuda()
    empty = moe(hidden[:0], torch.zeros(0, 2, device="cuda"), torch.zeros(0, 2, dtype=torch.int64, device="cuda"),
                gate, gate, down)
    assert empty.shape == (0, 8)
    zero_k = moe(hidden, torch.zeros(3, 0, device="cuda"), torch.zeros(3, 0, dtype=torch.int64, device="cuda"),
                 gate, gate, down)
    assert torch.count_nonzero(zero_k) == 0 and zero_k.shape == (3, 8)
    with pytest.raises(ValueError):
        moe(hidden, torch.zeros(3, 2, device="cuda"), torch.zeros(3, 1, dtype=torch.int64, device="cuda"),
            gate, gate, down)
    bad_sel = torch.full((3, 1), 5, dtype=torch.int64, device="cuda")
    # default: no host synchronisation; the tokens with an invalid expert give zero rows
    monkeypatch.delenv("BIOPS_MOE_CHECK_INDICES", raising=False)
    quiet = moe(hidden, torch.ones(3, 1, device="cuda"), bad_sel, gate, gate, down)
    assert torch.count_nonzero(quiet) == 0
    monkeypatch.setenv("BIOPS_MOE_CHECK_INDICES", "1")
    with pytest.raises(RuntimeError, match="outside"):
        moe(hidden, torch.ones(3, 1, device="cuda"), bad_sel, gate, gate, down)
    check_moe_indices()  # the report above cleared the flag


@pytest.mark.parametrize("sparse", (False, True), ids=("dense", "sparse"))
def test_moe_reports_out_of_range_indices_without_waiting(monkeypatch, sparse):
    """The reference rejects out-of-range expert indices (moe.py:66-73).  Here the call itself
    does not wait: the kernels set a device flag, an asynchronous copy brings it to the host,
    and the next call after the copy has landed raises RuntimeError (so does
    check_moe_indices(), which waits).  One report clears the flag."""
    monkeypatch.delenv("BIOPS_MOE_CHECK_INDICES", raising=False)
    monkeypatch.setattr(_IndexWatch, "PERIOD", 0.0)
    hidden = randn(4, 16, seed=7460).cuda()
    gate = randn(3, 8, 16, seed=7461).cuda()
    down = randn(3, 16, 8, seed=7462).cuda()
    w = torch.ones(4, 2, device="cuda")
    good = torch.tensor([[0, 1], [2, 0], [1, 2], [0, 2]], device="cuda")
    bad = good.clone()
    bad[2, 1] = 3
    ref = _moe(hidden, w, good, gate, gate, down, sparse=sparse)
    check_moe_indices()
    out = _moe(hidden, w, bad, gate, gate, down, sparse=sparse)  # returns without raising
    assert torch.count_nonzero(out[2]) == 0
    assert_bitwise(out[[0, 1, 3]], ref[[0, 1, 3]], "valid tokens of the bad call")
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="outside"):
        _moe(hidden, w, good, gate, gate, down, sparse=sparse)
    assert_bitwise(_moe(hidden, w, good, gate, gate, down, sparse=sparse), ref, "after the report")
    check_moe_indices()
    _moe(hidden, w, bad, gate, gate, down, sparse=sparse)
    with pytest.raises(RuntimeError, match="outside"):
        check_moe_indices()
    check_moe_indices()


@pytest.mark.parametrize("sparse", (False, True), ids=("dense", "sparse"))
def test_moe_known_answers(sparse):
    """Each token is one case of tests/_moe_known.py: the silu rounding, the silu*up rounding,
    the routing weight's rounding, the weighted route's rounding and the left-to-right slot sum
    each decide its output bits.  Checked exactly, for the whole batch and for every token alone
    (the few-token calls run other GEMM tile entries and the one-workgroup route packing)."""
    hidden, weights, selected, gate, up, down, expected = known_answer_problem()
    args = [t.cuda() for t in (hidden, weights, selected, gate, up, down)]
    out = _moe(*args, sparse=sparse)
    for t, (name, _, value, mistake) in enumerate(CASES):
        got = out[t, 0].item()
        assert got == value, f"token {t} ({name}): {got}, expected {value} ({mistake} would be the mistake)"
    assert_bitwise(out, expected.cuda(), "known answers")
    for t in range(len(CASES)):
        alone = _moe(*(a[t : t + 1] for a in args[:3]), *args[3:], sparse=sparse)
        assert_bitwise(alone, expected[t : t + 1].cuda(), f"token {t} alone ({CASES[t][0]})")


@pytest.mark.parametrize("u", (1.5, -1.75))
def test_moe_swiglu_epilogue_over_every_bf16_gate_value(u):
    """round(round(silu(g)) * u) for every bf16 g with 2^-4 <= |g| < 8 (1792 tokens): the dense
    and the sparse evaluation both give the oracle's bits, except where silu(g) lies within
    10^-5 of its magnitude of a bf16 rounding midpoint (an fp32 silu may land on either side;
    there one ulp is allowed)."""
    problem, g = silu_sweep_problem(u)
    ref = oracle.moe(*problem)[:, 0].double()
    silu = g.double() / (1 + torch.exp(-g.double()))
    tight = midpoint_margin(silu) < 1e-5
    args = [t.cuda() for t in problem]
    for sparse in (False, True):
        got = _moe(*args, sparse=sparse)[:, 0].cpu().double()
        assert torch.count_nonzero(_moe(*args, sparse=sparse)[:, 1:]) == 0
        exact = got == ref
        assert bool(exact[~tight].all()), (
            f"sparse={sparse}: {int((~exact[~tight]).sum())} of {int((~tight).sum())} tokens differ, first at "
            f"g = {float(g[~tight][~exact[~tight]][0])}")
        assert bool(((got - ref).abs() <= ULP[torch.bfloat16] * ref.abs())[tight].all())
