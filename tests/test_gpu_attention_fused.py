"""Fused attention (no score matrix in memory) on the GPU: parity with the CPU oracle, with the
materialised-score path, and bitwise batch invariance (reference tests
test_batch_invariance.py:512-742 for the operator semantics).

The fused kernel takes bf16 / fp16 calls with head sizes <= 256 (varlen: <= 128) that are
multiples of 8; the
shapes below cover partial query tiles (rows not a multiple of 128), partial key blocks (keys not
a multiple of 64), head-dim padding (72 -> 128, 40 -> 64), grouped-query heads, both causal
alignments, boolean and additive masks and fully masked rows.

Parity: as for the materialised path (tests/_parity.py), a per-element bound of one ulp of the
output dtype times (|O| + 2 (P |V|)) and a share of outputs carrying the oracle's exact bits.
Against the materialised path the only difference is the fp32 order of the softmax row sum,
which can move a probability across a rounding boundary of the input dtype: the same bound
applies, and over 90 % of the outputs are bitwise equal.
"""

import math

import pytest
import torch

import oracle
from batch_invariant_ops import (
    scaled_dot_product_attention_batch_invariant as sdpa,
    varlen_scaled_dot_product_attention_batch_invariant as varlen,
)
from batch_invariant_ops import _native as nat

from _parity import check_sdpa, check_sdpa_against, check_varlen
from _tol import ULP, assert_bitwise, assert_close_scaled, assert_composite_close, assert_first_sample_equal

pytestmark = pytest.mark.gpu
DTYPES16 = (torch.bfloat16, torch.float16)


def randn(*shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


@pytest.fixture
def materialized(monkeypatch):
    """Run a callable with the materialised-score path selected."""

    def run(fn, *args, **kwargs):
        monkeypatch.setenv("BIOPS_ATTENTION_MATERIALIZE", "1")
        try:
            return fn(*args, **kwargs)
        finally:
            monkeypatch.delenv("BIOPS_ATTENTION_MATERIALIZE")

    return run


def test_fused_envelope():
    lib = nat.load()
    assert lib.biops_attention_fused_supported(nat.BF16, 128, 128) == 1
    assert lib.biops_attention_fused_supported(nat.F16, 8, 64) == 1
    assert lib.biops_attention_fused_supported(nat.F32, 64, 64) == 0
    assert lib.biops_attention_fused_supported(nat.BF16, 65, 64) == 0
    assert lib.biops_attention_fused_supported(nat.BF16, 256, 256) == 1
    assert lib.biops_attention_fused_supported(nat.BF16, 264, 64) == 0
    assert lib.biops_attention_fused_supported(nat.BF16, 64, 0) == 0
    assert lib.biops_varlen_fused_supported(nat.BF16, 128, 128) == 1
    assert lib.biops_varlen_fused_supported(nat.BF16, 136, 64) == 0


SHAPES = (
    # B, Hq, Hkv, Lq, Lk, D, Dv
    (2, 4, 4, 200, 333, 64, 64),
    (1, 2, 2, 128, 128, 128, 128),
    (2, 8, 2, 77, 190, 72, 40),
    (1, 4, 1, 1, 300, 128, 64),
    (3, 2, 2, 257, 65, 32, 128),
    (1, 2, 2, 64, 1, 8, 8),
    (2, 8, 1, 300, 257, 256, 256),   # 256-wide heads (one wavefront per SIMD)
    (1, 4, 2, 129, 64, 200, 136),
    (1, 2, 2, 65, 130, 96, 256),
)


@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("causal", (False, True))
@pytest.mark.parametrize("shape", SHAPES)
def test_fused_sdpa_matches_oracle_and_materialized(dtype, causal, shape, materialized):
    B, Hq, Hkv, Lq, Lk, D, Dv = shape
    seed = 8000 + 10 * SHAPES.index(shape) + (5 if causal else 0)
    q = randn(B, Hq, Lq, D, seed=seed, dtype=dtype)
    k = randn(B, Hkv, Lk, D, seed=seed + 1, dtype=dtype)
    v = randn(B, Hkv, Lk, Dv, seed=seed + 2, dtype=dtype)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    kw = dict(is_causal=causal, enable_gqa=Hq != Hkv)
    out = sdpa(qd, kd, vd, **kw)
    check_sdpa(out, q, k, v, what=f"fused vs oracle {shape}", **kw)
    mat = materialized(sdpa, qd, kd, vd, **kw)
    check_sdpa(mat, q, k, v, what=f"materialised vs oracle {shape}", **kw)
    check_sdpa_against(out, mat, q, k, v, min_exact=0.9, what="fused vs materialised", **kw)


@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("batch_size", (2, 5))
@pytest.mark.parametrize("causal", (False, True))
def test_fused_sdpa_is_batch_invariant(dtype, batch_size, causal):
    q = randn(batch_size, 8, 300, 128, seed=8100 + batch_size, dtype=dtype).cuda()
    k = randn(batch_size, 2, 300, 128, seed=8110 + batch_size, dtype=dtype).cuda()
    v = randn(batch_size, 2, 300, 128, seed=8120 + batch_size, dtype=dtype).cuda()
    full = sdpa(q, k, v, is_causal=causal, enable_gqa=True)
    assert_first_sample_equal(sdpa(q[:1], k[:1], v[:1], is_causal=causal, enable_gqa=True), full)
    # a middle sample alone, too
    j = batch_size // 2
    assert_bitwise(sdpa(q[j:j + 1], k[j:j + 1], v[j:j + 1], is_causal=causal, enable_gqa=True),
                   full[j:j + 1], "middle sample")


@pytest.mark.parametrize("mask_kind", ("boolean", "additive"))
@pytest.mark.parametrize("dtype", DTYPES16)
@pytest.mark.parametrize("lk", (172, 170))  # 170 keys: not a multiple of 4, materialised path
def test_fused_sdpa_masks(mask_kind, dtype, lk, materialized):
    q = randn(2, 4, 150, 64, seed=8200, dtype=dtype)
    k = randn(2, 4, lk, 64, seed=8201, dtype=dtype)
    v = randn(2, 4, lk, 64, seed=8202, dtype=dtype)
    g = torch.Generator().manual_seed(8203)
    keep = torch.rand(2, 1, 150, lk, generator=g) > 0.2
    keep[:, :, 7] = False  # fully masked rows -> 0
    if mask_kind == "boolean":
        mask = keep
    else:
        mask = (torch.rand(2, 1, 150, lk, generator=g) * -10).to(dtype)
        mask[~keep] = -math.inf
    assert nat.load().biops_attention_fused_mask_ok(
        mask.cuda().data_ptr(), nat.BOOL if mask_kind == "boolean" else nat.dtype_code(dtype), lk,
        0, 0, lk, 1) == (lk % 4 == 0)
    out = sdpa(q.cuda(), k.cuda(), v.cuda(), attn_mask=mask.cuda())
    check_sdpa(out, q, k, v, attn_mask=mask, what=f"{mask_kind} mask, {lk} keys")
    assert torch.count_nonzero(out[:, :, 7]) == 0
    mat = materialized(sdpa, q.cuda(), k.cuda(), v.cuda(), attn_mask=mask.cuda())
    check_sdpa_against(out, mat, q, k, v, attn_mask=mask, min_exact=0.9, what="fused vs materialised")
    # per-sample mask: batch invariance holds with the sample's own mask
    alone = sdpa(q[:1].cuda(), k[:1].cuda(), v[:1].cuda(), attn_mask=mask[:1].cuda())
    assert_first_sample_equal(alone, out)


def test_fused_sdpa_per_head_mask_and_gqa_equals_repeat():
    dtype = torch.bfloat16
    q = randn(1, 8, 96, 64, seed=8250, dtype=dtype).cuda()
    k = randn(1, 2, 96, 64, seed=8251, dtype=dtype).cuda()
    v = randn(1, 2, 96, 64, seed=8252, dtype=dtype).cuda()
    g = torch.Generator().manual_seed(8253)
    mask = (torch.rand(1, 8, 96, 96, generator=g) > 0.3).cuda()
    out = sdpa(q, k, v, attn_mask=mask, enable_gqa=True)
    rep = sdpa(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1), attn_mask=mask)
    assert_bitwise(out, rep, "gqa vs repeat_interleave")
    check_sdpa(out, q, k, v, attn_mask=mask, enable_gqa=True, what="per-head mask, gqa")


def test_fused_sdpa_empty_keys_give_zero():
    q = randn(1, 2, 10, 16, seed=8260, dtype=torch.bfloat16).cuda()
    k = torch.empty(1, 2, 0, 16, dtype=torch.bfloat16, device="cuda")
    v = torch.empty(1, 2, 0, 16, dtype=torch.bfloat16, device="cuda")
    out = sdpa(q, k, v)
    assert out.shape == (1, 2, 10, 16) and torch.count_nonzero(out) == 0


def _offsets(lengths):
    out = [0]
    for n in lengths:
        out.append(out[-1] + n)
    return torch.tensor(out, dtype=torch.int32)


@pytest.mark.parametrize("causal_type", (None, "TopLeft", "BottomRight"))
@pytest.mark.parametrize("dtype", DTYPES16)
def test_fused_varlen_matches_oracle(causal_type, dtype, materialized):
    ql, kl = (130, 3, 200, 64, 1), (100, 70, 200, 129, 5)
    q = randn(1, sum(ql) + 4, 8, 64, seed=8300, dtype=dtype)
    k = randn(1, sum(kl), 2, 64, seed=8301, dtype=dtype)
    v = randn(1, sum(kl), 2, 64, seed=8302, dtype=dtype)
    cq, ck = _offsets(ql), _offsets(kl)
    kw = dict(is_causal=causal_type is not None, causal_type=causal_type)
    out = varlen(q.cuda(), k.cuda(), v.cuda(), cq.cuda(), ck.cuda(), **kw)
    check_varlen(out, q, k, v, cq, ck, what=f"fused varlen {causal_type} {dtype}", **kw)
    assert torch.count_nonzero(out[:, sum(ql):]) == 0  # rows outside every sequence
    mat = materialized(varlen, q.cuda(), k.cuda(), v.cuda(), cq.cuda(), ck.cuda(), **kw)
    check_varlen(mat, q, k, v, cq, ck, what=f"materialised varlen {causal_type} {dtype}", **kw)
    assert_composite_close(out, mat, oracle.varlen_sdpa_abs(q, k, v, cq, ck, **kw), min_exact=0.9,
                           what="fused vs materialised")


def test_fused_varlen_sequence_alone_equals_packed():
    lengths = (300, 64, 1, 129, 513)
    q = randn(1, sum(lengths), 8, 64, seed=8350, dtype=torch.bfloat16).cuda()
    k = randn(1, sum(lengths), 2, 64, seed=8351, dtype=torch.bfloat16).cuda()
    v = randn(1, sum(lengths), 2, 64, seed=8352, dtype=torch.bfloat16).cuda()
    cu = _offsets(lengths)
    packed = varlen(q, k, v, cu.cuda(), cu.cuda(), is_causal=True, causal_type="BottomRight")
    for s in range(len(lengths)):
        s0, s1 = int(cu[s]), int(cu[s + 1])
        one = torch.tensor([0, s1 - s0], dtype=torch.int32, device="cuda")
        alone = varlen(q[:, s0:s1], k[:, s0:s1], v[:, s0:s1], one, one, is_causal=True,
                       causal_type="BottomRight")
        assert_bitwise(alone, packed[:, s0:s1], f"sequence {s}")


@pytest.mark.parametrize("causal_type", (None, "TopLeft"))
def test_fused_varlen_sequence_without_keys_between_others(causal_type):
    """A sequence with queries but no keys inside the pack reads zero (the reference skips it,
    batch_invariant_ops.py:1296-1299); its neighbours match the oracle."""
    ql, kl = (40, 7, 90), (30, 0, 90)
    q = randn(1, sum(ql) + 3, 4, 32, seed=8360, dtype=torch.bfloat16)
    k = randn(1, sum(kl), 2, 32, seed=8361, dtype=torch.bfloat16)
    v = randn(1, sum(kl), 2, 32, seed=8362, dtype=torch.bfloat16)
    cq, ck = _offsets(ql), _offsets(kl)
    kw = dict(is_causal=causal_type is not None, causal_type=causal_type)
    out = varlen(q.cuda(), k.cuda(), v.cuda(), cq.cuda(), ck.cuda(), **kw)
    assert torch.count_nonzero(out[:, 40:47]) == 0
    assert torch.count_nonzero(out[:, sum(ql):]) == 0
    check_varlen(out, q, k, v, cq, ck, what=f"sequence without keys, {causal_type}", **kw)


def test_fused_varlen_bottom_right_with_short_keys_zeroes_early_rows():
    """q_len > kv_len with bottom-right alignment: the first q_len - kv_len rows see no key."""
    ql, kl = (40,), (10,)
    q = randn(1, 40, 2, 32, seed=8370, dtype=torch.bfloat16)
    k = randn(1, 10, 2, 32, seed=8371, dtype=torch.bfloat16)
    v = randn(1, 10, 2, 32, seed=8372, dtype=torch.bfloat16)
    cq, ck = _offsets(ql), _offsets(kl)
    out = varlen(q.cuda(), k.cuda(), v.cuda(), cq.cuda(), ck.cuda(), is_causal=True, causal_type="BottomRight")
    assert torch.count_nonzero(out[:, :30]) == 0
    assert torch.count_nonzero(out[:, 30:]) > 0
    check_varlen(out, q, k, v, cq, ck, is_causal=True, causal_type="BottomRight", what="short keys")


def test_fused_sdpa_uniform_attention_averages_values():
    """Q = 0 gives the mean of V over the visible keys (causal: prefix means) -- a closed form."""
    dtype = torch.bfloat16
    q = torch.zeros(1, 1, 100, 64, dtype=dtype)
    k = randn(1, 1, 100, 64, seed=8380, dtype=dtype)
    v = randn(1, 1, 100, 64, seed=8381, dtype=dtype)
    out = sdpa(q.cuda(), k.cuda(), v.cuda(), is_causal=True).cpu().double()
    vd = v.double()
    prefix = vd.cumsum(2) / torch.arange(1, 101, dtype=torch.float64).view(1, 1, 100, 1)
    # P = round(1/n) for every visible key: the output is sum(round(1/n) * v), within 4 ulps
    assert_close_scaled(out, prefix, rel=4 * ULP[dtype], abs_scale=4 * ULP[dtype] * float(vd.abs().max()))


POW2_CASES = {
    # name: (B, Hq, Hkv, L, D, explicit scale, mask kind)
    "d64_causal": (2, 4, 2, 300, 64, None, "causal"),
    "d64_boolean_mask": (2, 4, 4, 190, 64, None, "boolean"),
    "d256": (1, 2, 1, 200, 256, None, "causal"),
    "d16": (1, 2, 2, 129, 16, None, None),
    "scale_half": (1, 2, 2, 150, 128, 0.5, "causal"),
    "scale_one": (1, 2, 2, 150, 128, 1.0, None),
    "scale_2^-8": (1, 2, 2, 150, 128, 2.0 ** -8, "causal"),
}


@pytest.mark.parametrize("case", sorted(POW2_CASES))
def test_power_of_two_scale_path_equals_generic_path(case, monkeypatch):
    """bf16 attention with a scale 2^k (-8 <= k <= 0) and no additive mask takes the fused
    kernels' power-of-two path (scores kept in units of round(S), the scale folded into the
    exponentials' base change); for scores of normal magnitude its bits equal the generic path's
    (round(round(S) * scale) per score), selected with BIOPS_ATTN_GENERIC_SCALE=1."""
    B, Hq, Hkv, L, D, scale, kind = POW2_CASES[case]
    dtype = torch.bfloat16
    seed = 8500 + sorted(POW2_CASES).index(case) * 10
    q = randn(B, Hq, L, D, seed=seed, dtype=dtype, scale=2.0).cuda()
    k = randn(B, Hkv, L, D, seed=seed + 1, dtype=dtype).cuda()
    v = randn(B, Hkv, L, D, seed=seed + 2, dtype=dtype).cuda()
    kw = dict(scale=scale, enable_gqa=Hq != Hkv)
    if kind == "causal":
        kw["is_causal"] = True
    elif kind == "boolean":
        g = torch.Generator().manual_seed(seed + 3)
        kw["attn_mask"] = (torch.rand(B, 1, L, L, generator=g) > 0.25).cuda()
    fast = sdpa(q, k, v, **kw)
    monkeypatch.setenv("BIOPS_ATTN_GENERIC_SCALE", "1")
    generic = sdpa(q, k, v, **kw)
    assert_bitwise(fast, generic, f"{case}: power-of-two path vs generic path")
    check_sdpa(fast, q, k, v, what=f"{case} vs oracle", **kw)


def test_power_of_two_scale_path_varlen(monkeypatch):
    lengths = (300, 64, 1, 129, 513, 77)
    dtype = torch.bfloat16
    q = randn(1, sum(lengths), 8, 64, seed=8600, dtype=dtype, scale=2.0).cuda()
    k = randn(1, sum(lengths), 2, 64, seed=8601, dtype=dtype).cuda()
    v = randn(1, sum(lengths), 2, 64, seed=8602, dtype=dtype).cuda()
    cu = _offsets(lengths).cuda()
    for causal_type in (None, "BottomRight"):
        kw = dict(is_causal=causal_type is not None, causal_type=causal_type)
        monkeypatch.delenv("BIOPS_ATTN_GENERIC_SCALE", raising=False)
        fast = varlen(q, k, v, cu, cu, **kw)
        monkeypatch.setenv("BIOPS_ATTN_GENERIC_SCALE", "1")
        generic = varlen(q, k, v, cu, cu, **kw)
        assert_bitwise(fast, generic, f"varlen {causal_type}: power-of-two path vs generic path")
