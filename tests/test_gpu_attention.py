"""Eager and packed-varlen attention on the GPU (reference tests test_batch_invariance.py:512-742).

Parity (composite, tests/_parity.py): each output element is within one ulp of the output
dtype times (|O| + 2 (P |V|)) of the oracle, P |V| being that element's own magnitude of terms,
and in 16-bit dtypes almost every element carries the oracle's exact bits (the kernels round S,
S*scale, S+mask, P and O where the oracle does).
"""

import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from batch_invariant_ops import (
    scaled_dot_product_attention_batch_invariant as sdpa,
    set_batch_invariant_mode,
    varlen_scaled_dot_product_attention_batch_invariant as varlen,
)

from _parity import check_sdpa, check_varlen
from _tol import assert_bitwise, assert_first_sample_equal

pytestmark = pytest.mark.gpu
DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def randn(*shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch_size", (2, 3, 5, 17))
def test_sdpa_is_batch_invariant(dtype, batch_size):
    target = randn(1, 16, 256, 72, seed=7100 + batch_size, dtype=dtype)
    companions = randn(batch_size - 1, 16, 256, 72, seed=7200 + batch_size, dtype=dtype)
    q = torch.cat((target, companions)).cuda()
    k = randn(*q.shape, seed=7300 + batch_size, dtype=dtype).cuda()
    v = randn(*q.shape, seed=7400 + batch_size, dtype=dtype).cuda()
    assert_first_sample_equal(sdpa(q[:1], k[:1], v[:1]), sdpa(q, k, v))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("causal", (False, True))
def test_sdpa_matches_oracle(dtype, causal):
    q = randn(2, 8, 33, 65, seed=7200, dtype=dtype)
    k = randn(2, 8, 47, 65, seed=7201, dtype=dtype)
    v = randn(2, 8, 47, 39, seed=7202, dtype=dtype)
    out = sdpa(q.cuda(), k.cuda(), v.cuda(), is_causal=causal)
    check_sdpa(out, q, k, v, is_causal=causal, what=f"sdpa {dtype} causal={causal}")


@pytest.mark.parametrize("mask_kind", ("boolean", "additive"))
@pytest.mark.parametrize("dtype", DTYPES)
def test_sdpa_matches_oracle_with_mask(mask_kind, dtype):
    q = randn(2, 4, 17, 32, seed=7250, dtype=dtype)
    k = randn(2, 4, 23, 32, seed=7251, dtype=dtype)
    v = randn(2, 4, 23, 24, seed=7252, dtype=dtype)
    g = torch.Generator().manual_seed(7253)
    keep = torch.rand(2, 1, 17, 23, generator=g) > 0.2
    keep[:, :, -1] = False  # fully masked rows -> 0
    if mask_kind == "boolean":
        mask = keep
    else:
        mask = torch.where(keep, torch.tensor(0.0), torch.tensor(-math.inf)).to(dtype)
    out = sdpa(q.cuda(), k.cuda(), v.cuda(), attn_mask=mask.cuda())
    check_sdpa(out, q, k, v, attn_mask=mask, what=f"sdpa {mask_kind} mask {dtype}")
    assert torch.count_nonzero(out[:, :, -1]) == 0


def test_sdpa_additive_float_mask_values():
    q = randn(2, 4, 40, 32, seed=7260, dtype=torch.bfloat16)
    k = randn(2, 4, 50, 32, seed=7261, dtype=torch.bfloat16)
    v = randn(2, 4, 50, 32, seed=7262, dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(7263)
    mask = (torch.rand(2, 1, 40, 50, generator=g) * -10).to(torch.bfloat16)
    mask[torch.rand(2, 1, 40, 50, generator=g) < 0.1] = -math.inf
    out = sdpa(q.cuda(), k.cuda(), v.cuda(), attn_mask=mask.cuda())
    check_sdpa(out, q, k, v, attn_mask=mask, what="additive mask values")


def test_sdpa_promoting_mask_dtype():
    """A float32 additive mask on bf16 scores promotes the masked scores (reference glue)."""
    q = randn(1, 2, 9, 16, seed=7270, dtype=torch.bfloat16)
    k = randn(1, 2, 11, 16, seed=7271, dtype=torch.bfloat16)
    v = randn(1, 2, 11, 8, seed=7272, dtype=torch.bfloat16)
    mask = randn(1, 1, 9, 11, seed=7273)
    out = sdpa(q.cuda(), k.cuda(), v.cuda(), attn_mask=mask.cuda())
    check_sdpa(out, q, k, v, attn_mask=mask, what="fp32 mask on bf16 scores")


@pytest.mark.parametrize("dtype", DTYPES)
def test_sdpa_matches_oracle_with_grouped_query_attention(dtype):
    q = randn(2, 8, 17, 32, seed=7275, dtype=dtype)
    k = randn(2, 2, 23, 32, seed=7276, dtype=dtype)
    v = randn(2, 2, 23, 24, seed=7277, dtype=dtype)
    out = sdpa(q.cuda(), k.cuda(), v.cuda(), enable_gqa=True)
    check_sdpa(out, q, k, v, enable_gqa=True, what=f"gqa {dtype}")
    # GQA by head indexing equals explicit head repetition bit for bit
    rep = sdpa(q.cuda(), k.repeat_interleave(4, 1).cuda(), v.repeat_interleave(4, 1).cuda())
    assert_bitwise(out, rep, "gqa vs repeat_interleave")


def test_sdpa_custom_scale_and_rank3():
    q = randn(6, 20, 16, seed=7280)
    k = randn(6, 30, 16, seed=7281)
    v = randn(6, 30, 16, seed=7282)
    out = sdpa(q.cuda(), k.cuda(), v.cuda(), scale=0.3)
    check_sdpa(out, q, k, v, scale=0.3, what="fp32 rank 3, scale 0.3")


def test_sdpa_rejects_dropout_and_mask_with_causal():
    q = torch.zeros(1, 1, 2, 4, device="cuda")
    with pytest.raises(ValueError):
        sdpa(q, q, q, dropout_p=0.1)
    with pytest.raises(ValueError):
        sdpa(q, q, q, attn_mask=torch.ones(2, 2, dtype=torch.bool, device="cuda"), is_causal=True)


def test_mode_overrides_scaled_dot_product_attention():
    q = randn(3, 16, 256, 72, seed=7300, dtype=torch.bfloat16).cuda()
    k = randn(3, 16, 256, 72, seed=7301, dtype=torch.bfloat16).cuda()
    v = randn(3, 16, 256, 72, seed=7302, dtype=torch.bfloat16).cuda()
    with set_batch_invariant_mode():
        alone = F.scaled_dot_product_attention(q[:1], k[:1], v[:1])
        batched = F.scaled_dot_product_attention(q, k, v)
    assert_first_sample_equal(alone, batched)
    assert_bitwise(batched, sdpa(q, k, v), "mode vs direct call")


def _offsets(lengths):
    out = [0]
    for n in lengths:
        out.append(out[-1] + n)
    return torch.tensor(out, dtype=torch.int32)


@pytest.mark.parametrize("causal_type", (None, "TopLeft", "BottomRight"))
def test_varlen_matches_oracle(causal_type):
    ql, kl = (5, 3, 7), (7, 4, 5)
    q = randn(1, sum(ql), 4, 32, seed=7350, dtype=torch.bfloat16)
    k = randn(1, sum(kl), 2, 32, seed=7351, dtype=torch.bfloat16)
    v = randn(1, sum(kl), 2, 24, seed=7352, dtype=torch.bfloat16)
    cq, ck = _offsets(ql), _offsets(kl)
    out = varlen(q.cuda(), k.cuda(), v.cuda(), cq.cuda(), ck.cuda(), is_causal=causal_type is not None,
                 causal_type=causal_type)
    check_varlen(out, q, k, v, cq, ck, is_causal=causal_type is not None, causal_type=causal_type,
                 what=f"varlen {causal_type}")


def test_varlen_is_batch_invariant_for_duplicate_and_unrelated_packs():
    ql, kl = (33, 17, 33), (47, 23, 47)
    q = randn(1, sum(ql), 8, 64, seed=7375, dtype=torch.bfloat16).cuda()
    k = randn(1, sum(kl), 8, 64, seed=7376, dtype=torch.bfloat16).cuda()
    v = randn(1, sum(kl), 8, 64, seed=7377, dtype=torch.bfloat16).cuda()
    alone = varlen(q[:, :33], k[:, :47], v[:, :47], _offsets(ql[:1]).cuda(), _offsets(kl[:1]).cuda(),
                   is_causal=True, causal_type="BottomRight")
    packed = varlen(q, k, v, _offsets(ql).cuda(), _offsets(kl).cuda(), is_causal=True, causal_type="BottomRight")
    assert_bitwise(alone, packed[:, :33], "first sequence")
    # the third sequence (same geometry as the first, different data) alone
    third = varlen(q[:, 50:], k[:, 70:], v[:, 70:], _offsets(ql[2:]).cuda(), _offsets(kl[2:]).cuda(),
                   is_causal=True, causal_type="BottomRight")
    assert_bitwise(third, packed[:, 50:], "third sequence")


def test_varlen_leaves_uncovered_padding_rows_zero():
    q = randn(1, 11, 2, 16, seed=7390, dtype=torch.float16).cuda()
    k = randn(1, 11, 2, 16, seed=7391, dtype=torch.float16).cuda()
    v = randn(1, 11, 2, 16, seed=7392, dtype=torch.float16).cuda()
    cu = torch.tensor([0, 5, 9], dtype=torch.int32, device="cuda")
    out = varlen(q, k, v, cu, cu)
    assert torch.count_nonzero(out[:, :9]) > 0
    assert torch.count_nonzero(out[:, 9:]) == 0


def test_varlen_empty_kv_range_is_zero():
    q = randn(1, 2, 2, 16, seed=7395, dtype=torch.float16).cuda()
    k = torch.empty(1, 0, 2, 16, device="cuda", dtype=torch.float16)
    out = varlen(q, k, torch.empty_like(k), torch.tensor([0, 2], dtype=torch.int32, device="cuda"),
                 torch.tensor([0, 0], dtype=torch.int32, device="cuda"))
    assert torch.count_nonzero(out) == 0


def test_varlen_rejects_bad_offsets():
    q = torch.zeros(1, 4, 2, 8, device="cuda")
    with pytest.raises(ValueError):
        varlen(q, q, q, torch.tensor([1, 4], device="cuda"), torch.tensor([0, 4], device="cuda"))
    with pytest.raises(ValueError):
        varlen(q, q, q, torch.tensor([0, 5], device="cuda"), torch.tensor([0, 4], device="cuda"))
    with pytest.raises(ValueError):
        varlen(q, q, q, torch.tensor([0, 3, 2], device="cuda"), torch.tensor([0, 2, 4], device="cuda"))
    with pytest.raises(ValueError):
        varlen(q, q[:, :3], q[:, :3], torch.tensor([0, 4], device="cuda"), torch.tensor([0, 3], device="cuda"),
               is_causal=True, causal_type="DontCare")


@pytest.mark.parametrize("path", ("fused", "materialized"))
@pytest.mark.parametrize("case", ("score", "scaled_score", "masked_score"))
def test_sdpa_rounds_each_bf16_intermediate(case, path, monkeypatch):
    """The kernels round S, S*scale and S+mask to bf16 like the reference composite: keys whose
    exact logits differ but round to the same bf16 value get equal weight, so the output is
    exactly 0.5 (0.67-0.73 without that rounding).  Head size 8 and four keys (two copies of
    each) so that the fused kernel takes the call too."""
    if path == "materialized":
        monkeypatch.setenv("BIOPS_ATTENTION_MATERIALIZE", "1")
    else:
        monkeypatch.delenv("BIOPS_ATTENTION_MATERIALIZE", raising=False)

    def t(rows):
        x = torch.zeros(1, 1, len(rows), 8, dtype=torch.float64)
        x[0, 0, :, : len(rows[0])] = torch.tensor(rows, dtype=torch.float64)
        return x.to(torch.bfloat16).cuda()

    v = t([[1.0], [0.0], [1.0], [0.0]])
    if case == "score":
        q, k, kw = t([[16.0, 1.0]]), t([[16.0, 1.0], [16.0, 0.0]] * 2), {"scale": 1.0}
    elif case == "scaled_score":
        q, k, kw = t([[1.0, 1.0]]), t([[100.0, 100.0], [100.0, 99.0]] * 2), {"scale": 2**-0.5}
    else:
        q, k = t([[16.0]]), t([[16.0]] * 4)
        mask = torch.tensor([[[[1.0, 0.0, 1.0, 0.0]]]]).to(torch.bfloat16).cuda()
        kw = {"scale": 1.0, "attn_mask": mask}
    out = sdpa(q, k, v, **kw)
    assert out[0, 0, 0, 0].item() == 0.5, f"{case} on the {path} path gave {out[0, 0, 0, 0].item()}"
    ref = oracle.sdpa(q.cpu(), k.cpu(), v.cpu(), **{key: (val.cpu() if isinstance(val, torch.Tensor) else val)
                                                     for key, val in kw.items()})
    assert_bitwise(out, ref.cuda(), case)
