"""Randomised shapes across the GEMM, row-reduction and attention entry points: for every drawn
problem, bitwise batch invariance (a row / sample computed alone equals the same row inside the
batch) and agreement with the CPU oracle within the bounds of tests/_tol.py.

Shapes are drawn with a fixed seed (deterministic test) from ranges that cross the tile and
block boundaries of every kernel: rows and columns not multiples of 32/64/128, K not a multiple
of the 128-byte step, head sizes on and off the fused-attention envelope."""

import random

import pytest
import torch

import oracle
from batch_invariant_ops import (
    bmm_persistent,
    linalg_vector_norm_batch_invariant,
    linear_batch_invariant,
    mean_dim,
    scaled_dot_product_attention_batch_invariant as sdpa,
    softmax,
)

from _parity import check_sdpa
from _tol import ULP, assert_bitwise, assert_close_scaled, assert_gemm_close

pytestmark = pytest.mark.gpu
DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def randn(*shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def _cases(n, seed):
    rng = random.Random(seed)
    return [rng.randrange(1 << 30) for _ in range(n)]


@pytest.mark.parametrize("case", _cases(24, 11))
def test_random_linear(case):
    rng = random.Random(case)
    dtype = rng.choice(DTYPES)
    m = rng.choice((1, 2, 3, 7, 31, 33, 65, 130, 257, 600))
    k = rng.choice((8, 24, 64, 100, 136, 512, 777, 2048))
    n = rng.choice((8, 16, 40, 96, 200, 513, 1024))
    if dtype == torch.float32 and k % 4:
        k += 4 - k % 4
    x = randn(m, k, seed=case, dtype=dtype)
    w = randn(n, k, seed=case + 1, dtype=dtype) * 0.1
    bias = randn(n, seed=case + 2, dtype=dtype) if rng.random() < 0.5 else None
    full = linear_batch_invariant(x.cuda(), w.cuda(), None if bias is None else bias.cuda())
    i = rng.randrange(m)
    one = linear_batch_invariant(x[i : i + 1].cuda(), w.cuda(), None if bias is None else bias.cuda())
    assert_bitwise(one, full[i : i + 1], f"row {i} of {m}x{n}x{k} {dtype}")
    ref = oracle.linear(x, w, bias)
    absprod = oracle.gemm_abs(x, w.t()) + (0 if bias is None else bias.double().abs())
    assert_gemm_close(full, ref, absprod, k)


@pytest.mark.parametrize("case", _cases(12, 12))
def test_random_bmm(case):
    rng = random.Random(case)
    dtype = rng.choice(DTYPES)
    b, m, k, n = rng.choice((1, 3, 9)), rng.choice((1, 17, 64, 100)), rng.choice((16, 72, 300)), rng.choice((8, 33, 128))
    a = randn(b, m, k, seed=case, dtype=dtype)
    bb = randn(b, k, n, seed=case + 1, dtype=dtype)
    full = bmm_persistent(a.cuda(), bb.cuda())
    j = rng.randrange(b)
    assert_bitwise(bmm_persistent(a[j : j + 1].cuda(), bb[j : j + 1].cuda()), full[j : j + 1], "batch element")
    assert_gemm_close(full, oracle.bmm(a, bb), torch.bmm(a.double().abs(), bb.double().abs()), k)


@pytest.mark.parametrize("case", _cases(16, 13))
def test_random_row_reductions(case):
    rng = random.Random(case)
    dtype = rng.choice(DTYPES)
    rows, cols = rng.choice((1, 5, 64, 300)), rng.choice((1, 7, 64, 513, 1024, 3000))
    x = randn(rows, cols, seed=case, dtype=dtype)
    xd = x.cuda()
    i = rng.randrange(rows)
    s = softmax(xd, -1)
    assert_bitwise(softmax(xd[i : i + 1], -1), s[i : i + 1], "softmax row")
    assert_close_scaled(s, oracle.softmax(x, -1), rel=2 * ULP[dtype] if dtype != torch.float32 else 1e-5,
                        abs_scale=1e-6, what="softmax")
    mn = mean_dim(xd, -1)
    assert_bitwise(mean_dim(xd[i : i + 1], -1), mn[i : i + 1], "mean row")
    ref = oracle.mean_dim(x, -1).double()
    tol = (cols * 2.0**-24 + (ULP[dtype] if dtype != torch.float32 else 1e-5)) * x.double().abs().mean(-1)
    assert bool(((mn.cpu().double() - ref).abs() <= tol + 1e-30).all()), "mean"
    nr = linalg_vector_norm_batch_invariant(xd, dim=-1)
    assert_bitwise(linalg_vector_norm_batch_invariant(xd[i : i + 1], dim=-1), nr[i : i + 1], "norm row")
    refn = oracle.vector_norm(x, dim=-1).double()
    tol = (cols * 2.0**-24 + (ULP[dtype] if dtype != torch.float32 else 1e-5)) * refn.abs()
    assert bool(((nr.cpu().double() - refn).abs() <= tol + 1e-30).all()), "norm"


@pytest.mark.parametrize("case", _cases(16, 14))
def test_random_sdpa(case):
    rng = random.Random(case)
    dtype = rng.choice(DTYPES)
    b = rng.choice((1, 2, 3))
    hkv = rng.choice((1, 2))
    hq = hkv * rng.choice((1, 2, 4))
    lq, lk = rng.choice((1, 9, 64, 130, 257)), rng.choice((1, 31, 64, 200, 300))
    d, dv = rng.choice((8, 40, 64, 72, 128, 136)), rng.choice((8, 24, 64, 128))
    causal = rng.random() < 0.5
    q = randn(b, hq, lq, d, seed=case, dtype=dtype)
    k = randn(b, hkv, lk, d, seed=case + 1, dtype=dtype)
    v = randn(b, hkv, lk, dv, seed=case + 2, dtype=dtype)
    kw = dict(is_causal=causal, enable_gqa=hq != hkv)
    out = sdpa(q.cuda(), k.cuda(), v.cuda(), **kw)
    j = rng.randrange(b)
    alone = sdpa(q[j : j + 1].cuda(), k[j : j + 1].cuda(), v[j : j + 1].cuda(), **kw)
    assert_bitwise(alone, out[j : j + 1], f"sample {j} of {b} ({hq}/{hkv} heads, {lq}x{lk}, d {d}/{dv}, {dtype})")
    # few elements per case: the share of exact bits is left to the larger tests
    check_sdpa(out, q, k, v, min_exact=0.0 if out.numel() < 4096 else None, what=f"sdpa case {case}", **kw)
