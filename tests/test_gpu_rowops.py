"""Softmax, log-softmax, mean and vector norm on the GPU: bitwise batch invariance and parity
with the oracle (reference tests test_batch_invariance.py:452-509)."""

import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from batch_invariant_ops import (
    linalg_vector_norm_batch_invariant,
    mean_dim,
    set_batch_invariant_mode,
    softmax,
)

from _tol import assert_bitwise, assert_close_scaled, assert_first_sample_equal

pytestmark = pytest.mark.gpu
DTYPES = (torch.float32, torch.float16, torch.bfloat16)
# one rounding of the output after fp32 math (exp / log / sqrt add a few fp32 ulps)
REL = {torch.float32: 1e-5, torch.float16: 2.0**-10, torch.bfloat16: 2.0**-7}


def randn(*shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch_size", (2, 5, 17))
@pytest.mark.parametrize("dim", (-1, 1))
def test_mode_softmax_is_batch_invariant(dtype, batch_size, dim):
    x = randn(batch_size, 7, 145, seed=7025 + batch_size, dtype=dtype).cuda()
    with set_batch_invariant_mode():
        assert_first_sample_equal(torch.softmax(x[:1], dim=dim), torch.softmax(x, dim=dim))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dim", (-1, 1))
def test_mode_softmax_and_log_softmax_match_oracle(dtype, dim):
    x = randn(3, 7, 145, seed=7040 + dim, dtype=dtype)
    with set_batch_invariant_mode():
        sm = torch.softmax(x.cuda(), dim=dim)
        lsm = torch.log_softmax(x.cuda(), dim=dim)
    assert sm.dtype == dtype and lsm.dtype == dtype
    assert_close_scaled(sm, oracle.softmax(x, dim), rel=REL[dtype], abs_scale=1e-7, what="softmax")
    assert_close_scaled(lsm, oracle.log_softmax(x, dim), rel=REL[dtype], abs_scale=REL[dtype] * 8, what="log_softmax")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("cols", (1, 7, 64, 1000, 1024, 2048, 2049, 4100, 70000))
def test_softmax_row_lengths(dtype, cols):
    """Register-resident rows and re-read rows (beyond 256 chunks per lane group) alike."""
    x = randn(6, cols, seed=7100 + cols, dtype=dtype, scale=3.0)
    out = softmax(x.cuda(), dim=-1)
    assert_close_scaled(out, oracle.softmax(x), rel=REL[dtype], abs_scale=1e-7, what=f"cols={cols}")
    # the same row alone
    assert_bitwise(softmax(x[3:4].cuda(), dim=-1), out[3:4], "row 3 alone")


@pytest.mark.parametrize("dtype", DTYPES)
def test_softmax_all_neg_inf_row_is_zero(dtype):
    x = randn(4, 300, seed=7150, dtype=dtype)
    x[1] = -math.inf
    x[2, :299] = -math.inf
    out = softmax(x.cuda(), dim=-1).cpu()
    assert torch.count_nonzero(out[1]) == 0
    assert out[2, 299].item() == 1.0 and torch.count_nonzero(out[2, :299]) == 0
    assert_close_scaled(out, oracle.softmax(x), rel=REL[dtype], abs_scale=1e-7, what="-inf rows")


def test_softmax_output_dtype_and_half_to_float():
    x = randn(5, 33, seed=7160, dtype=torch.float16)
    out = softmax(x.cuda(), dim=-1, dtype=torch.float32)
    assert out.dtype == torch.float32
    assert_close_scaled(out, oracle.softmax(x, dtype=torch.float32), rel=1e-5, abs_scale=1e-7)
    with set_batch_invariant_mode():
        out2 = torch.softmax(x.cuda(), dim=-1, dtype=torch.float32)
    assert out2.dtype == torch.float32
    assert_close_scaled(out2, oracle.softmax(x, dtype=torch.float32), rel=1e-5, abs_scale=1e-7)


def test_softmax_rejects_integer_input():
    with pytest.raises(ValueError):
        softmax(torch.ones(3, 4, dtype=torch.int32, device="cuda"))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dims", ((1,), (1, 3), None))
@pytest.mark.parametrize("keepdim", (False, True))
def test_vector_norm_matches_oracle(dtype, dims, keepdim):
    x = randn(3, 17, 5, 11, seed=7050, dtype=dtype)
    out = linalg_vector_norm_batch_invariant(x.cuda(), dim=dims, keepdim=keepdim)
    ref = oracle.vector_norm(x, dim=dims, keepdim=keepdim)
    assert out.shape == ref.shape and out.dtype == ref.dtype
    assert_close_scaled(out, ref, rel=REL[dtype], abs_scale=0, what="vector_norm")


@pytest.mark.parametrize("composition", ("duplicate", "unrelated"))
def test_normalize_is_batch_invariant(composition):
    target = randn(1, 1024, 4, 33, 40, seed=7075, dtype=torch.bfloat16).cuda()
    if composition == "duplicate":
        inputs = target.repeat(2, 1, 1, 1, 1)
    else:
        inputs = torch.cat((target, randn(1, 1024, 4, 33, 40, seed=7076, dtype=torch.bfloat16).cuda()))
    with set_batch_invariant_mode():
        alone = F.normalize(target, dim=1)
        batched = F.normalize(inputs, dim=1)
    assert_first_sample_equal(alone, batched)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("shape", "dim"), (((4, 256, 2048), -1), ((3, 70, 9), 1), ((2, 5, 100000), -1), ((6, 3), 0)))
@pytest.mark.parametrize("keepdim", (False, True))
def test_mean_dim_matches_oracle(dtype, shape, dim, keepdim):
    x = randn(*shape, seed=7300 + shape[-1], dtype=dtype)
    out = mean_dim(x.cuda(), dim, keepdim=keepdim)
    ref = oracle.mean_dim(x, dim, keepdim=keepdim)
    assert out.shape == ref.shape and out.dtype == ref.dtype
    n = shape[dim]
    # fp32 accumulation of n terms: gamma_n * mean(|x|) on top of one output rounding
    abs_scale = (n * 2.0**-24) * float(x.double().abs().mean())
    assert_close_scaled(out, ref, rel=REL[dtype], abs_scale=abs_scale, what="mean")


def test_mean_integer_input_gives_float32():
    x = torch.arange(24, dtype=torch.int32).reshape(4, 6)
    out = mean_dim(x.cuda(), 1)
    assert out.dtype == torch.float32
    assert torch.equal(out.cpu(), oracle.mean_dim(x, 1))


@pytest.mark.parametrize("batch_size", (2, 8, 32))
def test_mode_mean_and_rmsnorm_are_batch_invariant(batch_size):
    x = randn(batch_size, 256, 2048, seed=7400, dtype=torch.bfloat16).cuda()
    with set_batch_invariant_mode():
        a = x[:1].float().pow(2).mean(-1, keepdim=True)
        b = x.float().pow(2).mean(-1, keepdim=True)
        c = x[:1].mean(-1)
        d = x.mean(-1)
        e = torch.linalg.vector_norm(x[:1], dim=-1)
        f = torch.linalg.vector_norm(x, dim=-1)
        g = x[:1].mean(dim=(1, 2))
        h = x.mean(dim=(1, 2))
    assert_first_sample_equal(a, b)
    assert_first_sample_equal(c, d)
    assert_first_sample_equal(e, f)
    assert_first_sample_equal(g, h)


def test_mode_multi_dim_mean_matches_oracle():
    x = randn(3, 5, 7, 11, seed=7450)
    with set_batch_invariant_mode():
        out = x.cuda().mean(dim=(1, 3), keepdim=True)
        out_all = x.cuda().mean(dim=[])
    assert_close_scaled(out, oracle.mean_dims(x, (1, 3), keepdim=True), rel=1e-5, abs_scale=1e-7)
    assert_close_scaled(out_all, oracle.mean_dims(x, []), rel=1e-5, abs_scale=1e-7)
