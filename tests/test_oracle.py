"""Pins for the CPU oracle (CPU only).

The reference commits no golden vectors for this path (its tests compare live against stock
CUDA torch), so every oracle function is pinned here against facts that do not restate it:
exact integer-valued products, identity / permutation matrices, the README linspace closed form,
constant-row and two-element closed forms, structural invariants (uniform attention averages V,
causal prefixes, GQA head mapping) and rounding-order cases built so that a plausible mistake
(bias added after the rounding, a transposed operand, a different slot order, a missing max
shift, the wrong GQA mapping) gives a different answer.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

BF16 = torch.bfloat16


def ints(*shape, lo, hi, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, shape, generator=g)


# ------------------------------------------------------------------------------ GEMM ----
@pytest.mark.parametrize("dtype", (torch.float32, torch.float16, BF16))
def test_matmul_integer_valued_is_exact(dtype):
    a = ints(9, 16, lo=-2, hi=2, seed=1)
    b = ints(16, 7, lo=-2, hi=2, seed=2)
    exact = torch.from_numpy(a.numpy().astype(np.int64) @ b.numpy().astype(np.int64))
    out = oracle.matmul(a.to(dtype), b.to(dtype))
    assert out.dtype == dtype
    assert torch.equal(out.to(torch.int64), exact)


def test_matmul_bias_joins_before_the_rounding():
    # x = 1 + 2^-9 (rounds to 1 in bf16), bias = 3 * 2^-10: rounding once gives 1 + 2^-7,
    # adding the bias to the already rounded product would give 1.
    a = torch.tensor([[1.0, 2.0**-9]], dtype=BF16)
    b = torch.tensor([[1.0], [1.0]], dtype=BF16)
    bias = torch.tensor([3 * 2.0**-10], dtype=BF16)
    assert oracle.matmul(a, b, bias).item() == 1 + 2.0**-7
    assert oracle.matmul(a, b).item() == 1.0


def test_matmul_identity_and_permutation():
    g = torch.Generator().manual_seed(3)
    a = torch.randn(6, 5, generator=g)
    assert torch.equal(oracle.matmul(a, torch.eye(5)), a)
    perm = torch.tensor([3, 0, 5, 1, 4, 2])
    p = torch.eye(6)[perm]
    assert torch.equal(oracle.matmul(p, a), a[perm])


def test_matmul_readme_linspace_closed_form():
    # README.md:62-76 check at a small size: A = linspace(-100, 100, D*D), B likewise.
    d = 16
    a = torch.linspace(-100, 100, d * d).reshape(d, d)
    b = torch.linspace(-100, 100, d * d).reshape(d, d)
    out = oracle.matmul(a, b).double()
    step = 200.0 / (d * d - 1)
    i = torch.arange(d, dtype=torch.float64)[:, None, None]
    k = torch.arange(d, dtype=torch.float64)[None, :, None]
    j = torch.arange(d, dtype=torch.float64)[None, None, :]
    closed = ((-100 + step * (i * d + k)) * (-100 + step * (k * d + j))).sum(1)
    assert torch.allclose(out, closed, rtol=1e-6, atol=1e-3)
    # a transposed operand gives a different closed form
    assert not torch.allclose(oracle.matmul(a, b.t().contiguous()).double(), closed, rtol=1e-3)


def test_bmm_and_linear_integer_valued():
    a = ints(3, 4, 8, lo=-3, hi=3, seed=4)
    b = ints(3, 8, 5, lo=-3, hi=3, seed=5)
    exact = np.einsum("bik,bkj->bij", a.numpy().astype(np.int64), b.numpy().astype(np.int64))
    assert np.array_equal(oracle.bmm(a.float(), b.float()).numpy().astype(np.int64), exact)
    x = ints(2, 3, 8, lo=-3, hi=3, seed=6)
    w = ints(5, 8, lo=-3, hi=3, seed=7)
    bias = ints(5, lo=-3, hi=3, seed=8)
    exact = np.einsum("btk,nk->btn", x.numpy().astype(np.int64), w.numpy().astype(np.int64)) + bias.numpy()
    out = oracle.linear(x.float(), w.float(), bias.float())
    assert out.shape == (2, 3, 5)
    assert np.array_equal(out.numpy().astype(np.int64), exact)


# ------------------------------------------------------------------------- softmax ----
@pytest.mark.parametrize("n", (1, 2, 64, 1024, 4096))
def test_softmax_constant_row_is_exact_power_of_two(n):
    out = oracle.softmax(torch.full((3, n), 0.37), dim=-1)
    assert torch.equal(out, torch.full((3, n), 1.0 / n))


def test_softmax_two_element_closed_form_and_shift_invariance():
    x = torch.tensor([[0.0, math.log(3.0)]], dtype=torch.float64)
    assert torch.allclose(oracle.softmax(x), torch.tensor([[0.25, 0.75]], dtype=torch.float64), atol=1e-15)
    # without the max shift exp(1000) overflows; the oracle must not
    shifted = oracle.softmax((x + 1000.0).float())
    assert torch.allclose(shifted.double(), torch.tensor([[0.25, 0.75]], dtype=torch.float64), atol=1e-4)
    lsm = oracle.log_softmax(x + 1000.0)
    assert torch.allclose(lsm, torch.log(torch.tensor([[0.25, 0.75]], dtype=torch.float64)), atol=1e-12)


def test_softmax_neg_inf_rules():
    x = torch.tensor([[-math.inf, -math.inf, -math.inf], [-math.inf, 2.0, -math.inf]])
    out = oracle.softmax(x)
    assert torch.equal(out, torch.tensor([[0.0, 0.0, 0.0], [0.0, 1.0, 0.0]]))
    assert torch.isnan(torch.softmax(x, -1)[0]).all()  # stock CPU differs: NaN


def test_softmax_rows_sum_to_one_and_dim_and_dtype():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(4, 7, 33, generator=g) * 4
    for dim in (0, 1, 2):
        s = oracle.softmax(x, dim=dim).double().sum(dim)
        assert torch.allclose(s, torch.ones_like(s), atol=1e-6)
    assert oracle.softmax(x.to(BF16), dtype=torch.float32).dtype == torch.float32
    lsm = oracle.log_softmax(x.double(), dim=1)
    assert torch.allclose(torch.exp(lsm), oracle.softmax(x.double(), dim=1), atol=1e-12)


# ---------------------------------------------------------------------- reductions ----
def test_mean_closed_forms():
    n = 1000
    x = torch.arange(n, dtype=torch.float32).repeat(3, 1)
    assert torch.equal(oracle.mean_dim(x, 1), torch.full((3,), (n - 1) / 2))
    assert torch.equal(oracle.mean_dim(torch.full((2, 5, 3), 0.75, dtype=BF16), 1), torch.full((2, 3), 0.75, dtype=BF16))
    ints_in = torch.arange(24, dtype=torch.int32).reshape(4, 6)
    out = oracle.mean_dim(ints_in, 1, keepdim=True)
    assert out.dtype == torch.float32 and out.shape == (4, 1)
    assert torch.equal(out[:, 0], torch.tensor([2.5, 8.5, 14.5, 20.5]))
    y = torch.arange(2 * 3 * 4, dtype=torch.float32).reshape(2, 3, 4)
    assert torch.equal(oracle.mean_dims(y, (0, 2)), torch.tensor([7.5, 11.5, 15.5]))
    assert oracle.mean_dims(y, []).item() == 11.5


def test_vector_norm_closed_forms():
    assert oracle.vector_norm(torch.ones(64 * 64)).item() == 64.0
    assert oracle.vector_norm(torch.tensor([[3.0, 4.0]]), dim=1).item() == 5.0
    x = torch.tensor([[3.0, 0.0], [4.0, 12.0]], dtype=BF16)
    out = oracle.vector_norm(x, dim=0, keepdim=True)
    assert out.dtype == BF16 and out.shape == (1, 2)
    assert torch.equal(out, torch.tensor([[5.0, 12.0]], dtype=BF16))
    assert oracle.vector_norm(torch.ones(2, 3, 4), dim=(1, 2)).tolist() == [float(torch.tensor(math.sqrt(12)))] * 2
    assert oracle.vector_norm(torch.ones(3, dtype=BF16), dtype=torch.float32).dtype == torch.float32


# ----------------------------------------------------------------------- attention ----
def test_sdpa_uniform_attention_averages_values():
    g = torch.Generator().manual_seed(10)
    q = torch.zeros(1, 2, 5, 8)
    k = torch.randn(1, 2, 5, 8, generator=g)
    v = torch.randn(1, 2, 5, 3, generator=g)
    out = oracle.sdpa(q, k, v)
    assert torch.allclose(out, v.mean(-2, keepdim=True).expand_as(out), atol=1e-6)
    causal = oracle.sdpa(q, k, v, is_causal=True)
    prefix = torch.cumsum(v, -2) / torch.arange(1, 6).reshape(1, 1, 5, 1)
    assert torch.allclose(causal, prefix, atol=1e-6)


def test_sdpa_gqa_maps_query_head_to_kv_head_floor_division():
    q = torch.zeros(1, 4, 3, 2)
    k = torch.zeros(1, 2, 3, 2)
    v = torch.stack([torch.full((3, 1), 1.0), torch.full((3, 1), 2.0)]).unsqueeze(0)
    out = oracle.sdpa(q, k, v, enable_gqa=True)
    assert out[0, :, 0, 0].tolist() == [1.0, 1.0, 2.0, 2.0]  # h // 2, not h % 2


def test_sdpa_masks_and_scale():
    q = torch.tensor([[[[1.0, 0.0]]]])
    k = torch.tensor([[[[2.0, 0.0], [0.0, 0.0]]]])
    v = torch.tensor([[[[1.0], [0.0]]]])
    # scores (2, 0) scaled by 1/sqrt(2): weight of key 0 = sigmoid(sqrt 2)
    out = oracle.sdpa(q, k, v)
    s = float(torch.tensor(1 / math.sqrt(2), dtype=torch.float32))
    assert abs(out.item() - 1 / (1 + math.exp(-2 * s))) < 1e-7
    assert abs(oracle.sdpa(q, k, v, scale=0.5).item() - 1 / (1 + math.exp(-1.0))) < 1e-7
    keep = torch.tensor([[[[False, True]]]])
    assert oracle.sdpa(q, k, v, attn_mask=keep).item() == 0.0
    neg = torch.where(keep, 0.0, -math.inf)
    assert oracle.sdpa(q, k, v, attn_mask=neg).item() == 0.0
    none = torch.zeros(1, 1, 1, 2, dtype=torch.bool)
    assert oracle.sdpa(q, k, v, attn_mask=none).item() == 0.0  # fully masked row -> 0
    # a constant additive mask shifts both scores: same weights up to the rounding of S + 5
    assert abs(oracle.sdpa(q, k, v, attn_mask=torch.full((1, 1, 1, 2), 5.0)).item() - out.item()) < 1e-6


def _bf16(rows):
    return torch.tensor(rows, dtype=torch.float64).to(BF16)


@pytest.mark.parametrize("case", ("score", "scaled_score", "masked_score"))
def test_sdpa_rounds_each_bf16_intermediate(case):
    """Each case has two keys whose exact logits differ but whose bf16-rounded logits are equal,
    with values 1 and 0: with the rounding the output is exactly 0.5; dropping that one rounding
    gives about 0.67-0.73.
    score:        q.k = 257 and 256; 257 rounds to 256 (ties to even, spacing 2 above 256).
    scaled_score: q.k = 200 and 199 (exact); times 1/sqrt(2) = 141.42 and 140.71, both 141.
    masked_score: q.k = 256 for both keys; key 0 gets +1 from the additive mask, 257 -> 256."""
    v = _bf16([[[[1.0], [0.0]]]])
    if case == "score":
        q, k, kw = _bf16([[[[16.0, 1.0]]]]), _bf16([[[[16.0, 1.0], [16.0, 0.0]]]]), {"scale": 1.0}
    elif case == "scaled_score":
        q, k, kw = _bf16([[[[1.0, 1.0]]]]), _bf16([[[[100.0, 100.0], [100.0, 99.0]]]]), {"scale": 2**-0.5}
    else:
        q, k = _bf16([[[[16.0, 0.0]]]]), _bf16([[[[16.0, 0.0], [16.0, 0.0]]]])
        kw = {"scale": 1.0, "attn_mask": _bf16([[[[1.0, 0.0]]]])}
    assert oracle.sdpa(q, k, v, **kw).item() == 0.5
    # the same logits without bf16 roundings (fp64 inputs keep every intermediate exact)
    unrounded = oracle.sdpa(q.double(), k.double(), v.double(), **{
        key: (val.double() if isinstance(val, torch.Tensor) else val) for key, val in kw.items()})
    assert 0.6 < unrounded.item() < 0.75


def test_sdpa_abs_closed_forms():
    """P |V|: uniform attention gives the mean of |V| (the prefix means under causal); a
    one-hot attention row (one key far above the others) gives that key's |V| row."""
    g = torch.Generator().manual_seed(12)
    q = torch.zeros(1, 1, 4, 8)
    k = torch.randn(1, 1, 4, 8, generator=g)
    v = torch.randn(1, 1, 4, 3, generator=g)
    assert torch.allclose(oracle.sdpa_abs(q, k, v), v.abs().double().mean(-2, keepdim=True).expand(1, 1, 4, 3))
    prefix = torch.cumsum(v.abs().double(), -2) / torch.arange(1, 5).reshape(1, 1, 4, 1)
    assert torch.allclose(oracle.sdpa_abs(q, k, v, is_causal=True), prefix)
    q1 = torch.tensor([[[[100.0, 0.0]]]])
    k1 = torch.tensor([[[[1.0, 0.0], [-1.0, 0.0], [0.0, 0.0]]]])
    v1 = torch.tensor([[[[-2.0, 3.0], [5.0, 7.0], [1.0, 1.0]]]])
    assert oracle.sdpa_abs(q1, k1, v1, scale=1.0)[0, 0, 0].tolist() == [2.0, 3.0]
    # varlen: per sequence, zero outside every sequence
    vv = torch.arange(6, dtype=torch.float32).reshape(1, 6, 1, 1) - 2.5
    qq, kk = torch.zeros(1, 6, 1, 2), torch.zeros(1, 6, 1, 2)
    cu = torch.tensor([0, 2, 5])
    out = oracle.varlen_sdpa_abs(qq, kk, vv, cu, cu)
    # sequence 0: mean |-2.5|, |-1.5|; sequence 1: mean of 0.5, 0.5, 1.5 (P = 1/3 in fp32)
    assert out[0, :, 0, 0].tolist() == pytest.approx([2.0, 2.0, 5 / 6, 5 / 6, 5 / 6, 0.0], rel=1e-7)


def test_varlen_alignment_rules_and_zero_rows():
    # two sequences: (q 2, kv 4) and (q 3, kv 3); Q = 0 -> outputs are means of visible V rows
    q = torch.zeros(1, 6, 1, 4)
    k = torch.zeros(1, 7, 1, 4)
    v = torch.arange(7, dtype=torch.float32).reshape(1, 7, 1, 1)
    cq = torch.tensor([0, 2, 5])
    ck = torch.tensor([0, 4, 7])
    br = oracle.varlen_sdpa(q, k, v, cq, ck, is_causal=True, causal_type="BottomRight")
    tl = oracle.varlen_sdpa(q, k, v, cq, ck, is_causal=True, causal_type="TopLeft")
    full = oracle.varlen_sdpa(q, k, v, cq, ck)
    # bottom-right: row i of seq 0 sees keys 0..i+2; top-left: keys 0..i
    assert br[0, :2, 0, 0].tolist() == [1.0, 1.5]
    assert tl[0, :2, 0, 0].tolist() == [0.0, 0.5]
    assert full[0, :2, 0, 0].tolist() == [1.5, 1.5]
    # equal lengths: both alignments agree (keys 4..6)
    assert br[0, 2:5, 0, 0].tolist() == tl[0, 2:5, 0, 0].tolist() == [4.0, 4.5, 5.0]
    assert br[0, 5].abs().sum() == 0  # row outside every sequence
    empty_kv = oracle.varlen_sdpa(q[:, :2], k[:, :0], v[:, :0], torch.tensor([0, 2]), torch.tensor([0, 0]))
    assert torch.count_nonzero(empty_kv) == 0


# ------------------------------------------------------------------------------ MoE ----
def test_moe_matches_route_by_route_loop():
    """The reference test's brute force (test_batch_invariance.py:757-766), float64."""
    g = torch.Generator().manual_seed(11)
    hidden = torch.randn(7, 12, generator=g, dtype=torch.float64)
    gate = torch.randn(5, 16, 12, generator=g, dtype=torch.float64)
    up = torch.randn(5, 16, 12, generator=g, dtype=torch.float64)
    down = torch.randn(5, 12, 16, generator=g, dtype=torch.float64)
    sel = torch.randint(0, 5, (7, 3), generator=g)
    w = torch.rand(7, 3, generator=g, dtype=torch.float64)
    out = oracle.moe(hidden, w, sel, gate, up, down)
    expected = torch.zeros(7, 12, dtype=torch.float64)
    for t in range(7):
        for s in range(3):
            e = sel[t, s]
            inter = F.silu(gate[e] @ hidden[t]) * (up[e] @ hidden[t])
            expected[t] += (down[e] @ inter) * w[t, s]
    assert torch.allclose(out, expected, rtol=1e-12, atol=1e-12)


def test_moe_slot_sum_is_left_to_right_with_rounding():
    # y = 1 for every expert (silu(16) = 16 in bf16, up = 1/16, down = 1); routes 1, r, r with
    # r = 3 * 2^-10: left to right, 1 + r rounds back to 1 twice; r + r first would give 1 + 2^-7.
    hidden = torch.ones(1, 1, dtype=BF16)
    gate = torch.full((3, 1, 1), 16.0, dtype=BF16)
    up = torch.full((3, 1, 1), 1 / 16, dtype=BF16)
    down = torch.ones(3, 1, 1, dtype=BF16)
    r = 3 * 2.0**-10
    w = torch.tensor([[1.0, r, r]])
    sel = torch.tensor([[0, 1, 2]])
    assert oracle.moe(hidden, w, sel, gate, up, down).item() == 1.0
    w2 = torch.tensor([[r, r, 1.0]])
    assert oracle.moe(hidden, w2, sel, gate, up, down).item() == 1 + 2.0**-7


def _bf16_scalar(x):
    return torch.tensor(x, dtype=torch.float64).to(BF16).item()


def _known_case_scalar(slots, drop=None):
    """One known-answer case in Python scalars, each rounding explicit (moe.py:75-91); ``drop``
    removes one of them or reverses the slot order."""
    rb = _bf16_scalar
    routes = []
    for g, u, c, w in slots:
        s = g / (1.0 + math.exp(-g))
        s = s if drop == "silu rounding" else rb(s)
        a = s * u if drop == "silu*up rounding" else rb(s * u)
        y = rb(a * c)
        w = w if drop == "routing weight rounding" else rb(w)
        routes.append(y * w if drop == "weighted route rounding" else rb(y * w))
    if drop == "slot order":
        routes = routes[::-1]
    out = routes[0]
    for r in routes[1:]:
        out = rb(out + r)
    return rb(out)


def test_moe_known_answers():
    """Each case isolates one rounding of the reference's route evaluation or its slot order:
    the oracle gives the expected bits, and the named mistake gives the other value."""
    from _moe_known import CASES, known_answer_problem

    hidden, weights, selected, gate, up, down, expected = known_answer_problem()
    out = oracle.moe(hidden, weights, selected, gate, up, down)
    assert torch.equal(out, expected)
    for name, slots, value, mistake in CASES:
        assert _known_case_scalar(slots) == value, name
        assert _known_case_scalar(slots, drop=name) == mistake != value, name


def test_moe_abs_is_the_sum_of_route_magnitudes():
    from _moe_known import CASES, known_answer_problem

    args = known_answer_problem()[:6]
    scale = oracle.moe_abs(*args)
    for t, (_, slots, _, _) in enumerate(CASES):
        mags = [abs(_known_case_scalar([slot])) for slot in slots]
        assert scale[t, 0].item() == pytest.approx(sum(mags), rel=0, abs=0)
        assert torch.count_nonzero(scale[t, 1:]) == 0


def test_moe_edge_shapes():
    hidden = torch.ones(3, 4)
    gate = torch.ones(2, 5, 4)
    down = torch.ones(2, 4, 5)
    assert oracle.moe(hidden[:0], torch.zeros(0, 1), torch.zeros(0, 1, dtype=torch.long), gate, gate, down).shape == (0, 4)
    z = oracle.moe(hidden, torch.zeros(3, 0), torch.zeros(3, 0, dtype=torch.long), gate, gate, down)
    assert z.shape == (3, 4) and torch.count_nonzero(z) == 0


# ----------------------------------------------------------------------- convolution ----
def _conv_loop(x, w, stride, padding, dilation, groups):
    """Regular N-d convolution straight from its definition (python loops, float64)."""
    nd = x.ndim - 2
    B, C = x.shape[:2]
    O, Cg = w.shape[:2]
    k = w.shape[2:]
    out_size = [(x.shape[2 + i] + 2 * padding[i] - dilation[i] * (k[i] - 1) - 1) // stride[i] + 1 for i in range(nd)]
    out = torch.zeros(B, O, *out_size, dtype=torch.float64)
    Og = O // groups
    for b in range(B):
        for o in range(O):
            g = o // Og
            for pos in np.ndindex(*out_size):
                acc = 0.0
                for c in range(Cg):
                    for tap in np.ndindex(*k):
                        src = [pos[i] * stride[i] - padding[i] + tap[i] * dilation[i] for i in range(nd)]
                        if all(0 <= src[i] < x.shape[2 + i] for i in range(nd)):
                            acc += float(x[(b, g * Cg + c, *src)]) * float(w[(o, c, *tap)])
                out[(b, o, *pos)] = acc
    return out


def _conv_transpose_loop(x, w, groups):
    """Non-overlapping transposed convolution (stride == kernel) from its definition."""
    nd = x.ndim - 2
    B, C = x.shape[:2]
    Og = w.shape[1]
    k = w.shape[2:]
    Cg = C // groups
    out = torch.zeros(B, Og * groups, *[x.shape[2 + i] * k[i] for i in range(nd)], dtype=torch.float64)
    for b in range(B):
        for c in range(C):
            g = c // Cg
            for pos in np.ndindex(*x.shape[2:]):
                for o in range(Og):
                    for tap in np.ndindex(*k):
                        dst = [pos[i] * k[i] + tap[i] for i in range(nd)]
                        out[(b, g * Og + o, *dst)] += float(x[(b, c, *pos)]) * float(w[(c, o, *tap)])
    return out


@pytest.mark.parametrize(("xs", "ws", "stride", "padding", "dilation", "groups"), (
    ((2, 4, 9), (6, 2, 3), (2,), (3,), (2,), 2),
    ((2, 4, 6, 5), (6, 2, 3, 2), (2, 1), (1, 0), (2, 1), 2),
    ((1, 3, 4, 5, 4), (2, 3, 2, 3, 2), (1, 2, 1), (1, 0, 1), (1, 1, 2), 1),
    ((2, 4, 7), (4, 1, 3), (1,), (1,), (1,), 4),  # depthwise 1-D
))
def test_conv_integer_valued_matches_definition(xs, ws, stride, padding, dilation, groups):
    """Integer operands: every sum is exact in float64 and bf16-representable (|sum| < 256), so
    the oracle must reproduce the loop bit for bit, bias included."""
    x = ints(*xs, lo=-3, hi=3, seed=9100).to(BF16)
    w = ints(*ws, lo=-2, hi=2, seed=9101).to(BF16)
    bias = ints(ws[0], lo=-4, hi=4, seed=9102).to(BF16)
    loop = _conv_loop(x.double(), w.double(), stride, padding, dilation, groups)
    assert loop.abs().max() < 200
    out = oracle.conv(x, w, bias, stride, padding, dilation, False, (0,) * len(stride), groups)
    assert torch.equal(out.double(), loop + bias.double().reshape(1, -1, *([1] * len(stride))))


@pytest.mark.parametrize(("xs", "ws", "groups"), (((2, 4, 2, 3), (4, 3, 2, 2), 2), ((1, 2, 2, 1, 2), (2, 2, 3, 1, 2), 1)))
def test_conv_transpose_integer_valued_matches_definition(xs, ws, groups):
    x = ints(*xs, lo=-3, hi=3, seed=9110).to(BF16)
    w = ints(*ws, lo=-2, hi=2, seed=9111).to(BF16)
    nd = len(xs) - 2
    k = tuple(ws[2:])
    bias = ints(ws[1] * groups, lo=-4, hi=4, seed=9112).to(BF16)
    loop = _conv_transpose_loop(x.double(), w.double(), groups)
    out = oracle.conv(x, w, bias, k, (0,) * nd, (1,) * nd, True, (0,) * nd, groups)
    assert torch.equal(out.double(), loop + bias.double().reshape(1, -1, *([1] * nd)))


def test_conv_bias_rounding_follows_the_path():
    """Depthwise 1-D rounds once after the bias; every other form rounds the dot product and then
    the sum with the bias.  With dot = 1 + 2^-8 and bias = 2^-8 (bf16): one rounding gives
    1 + 2^-7, two give round(1 + 2^-8) = 1 (tie to even), then 1 + 2^-8 -> 1."""
    x = torch.tensor([[[1.0, 2.0**-8]]]).to(BF16)  # one channel, two taps
    w = torch.tensor([[[1.0, 1.0]]]).to(BF16)
    b = torch.tensor([2.0**-8]).to(BF16)
    depthwise = oracle.conv(x, w, b, (1,), (0,), (1,), False, (0,), 1)  # groups == C == O == 1
    assert depthwise.item() == 1 + 2.0**-7
    x2 = x.expand(1, 2, 2).contiguous()
    w2 = torch.tensor([[[1.0, 1.0], [0.0, 0.0]]]).to(BF16)  # one output over two channels
    regular = oracle.conv(x2, w2, b, (1,), (0,), (1,), False, (0,), 1)
    assert regular.item() == 1.0


def test_conv_delta_kernel_copies_and_shifts():
    x = torch.randn(2, 3, 6, 7, generator=torch.Generator().manual_seed(9120))
    w = torch.zeros(3, 1, 3, 3)
    w[:, 0, 2, 0] = 1.0  # tap (2, 0) of every channel
    out = oracle.conv(x, w, None, (1, 1), (1, 1), (1, 1), False, (0, 0), 3)
    # output (h, w) reads input (h + 1, w - 1)
    assert torch.equal(out[:, :, :5, 1:], x[:, :, 1:, :6])
    assert torch.count_nonzero(out[:, :, 5, :]) == 0 and torch.count_nonzero(out[:, :, :, 0]) == 0
