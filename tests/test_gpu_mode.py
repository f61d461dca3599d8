"""set_batch_invariant_mode on the GPU: the aten overrides route to the HIP kernels
(reference tests test_batch_invariance.py:407-449, 577-586, 783-792)."""

import pytest
import torch
import torch.nn.functional as F

from batch_invariant_ops import (
    bmm_persistent,
    is_batch_invariant_mode_enabled,
    linear_batch_invariant,
    matmul_persistent,
    set_batch_invariant_mode,
)

from _tol import assert_bitwise, assert_first_sample_equal

pytestmark = pytest.mark.gpu


def randn(*shape, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).cuda()


def test_mode_overrides_matmul_family():
    q = randn(5, 19, 23, seed=7000)
    k = randn(5, 23, 17, seed=7001)
    x = randn(5, 37, 257, seed=7002)
    w = randn(91, 257, seed=7003)
    b = randn(91, seed=7004)
    a2 = randn(40, 257, seed=7005)
    with set_batch_invariant_mode():
        assert_first_sample_equal(q[:1] @ k[:1], q @ k)
        assert_first_sample_equal(F.linear(x[:1], w, b), F.linear(x, w, b))
        mm = torch.mm(a2, w.t())
        addmm = torch.addmm(b, a2, w.t())
        bmm = torch.bmm(q, k)
        lin = F.linear(x, w, b)
    assert_bitwise(mm, matmul_persistent(a2, w.t()), "aten::mm")
    assert_bitwise(addmm, matmul_persistent(a2, w.t(), b), "aten::addmm")
    assert_bitwise(bmm, bmm_persistent(q, k), "aten::bmm")
    assert_bitwise(lin, linear_batch_invariant(x, w, b), "aten::linear")


def test_mode_addmm_with_scalars():
    a = randn(8, 16, seed=7010)
    b = randn(16, 4, seed=7011)
    c = randn(8, 4, seed=7012)
    with set_batch_invariant_mode():
        out = torch.addmm(c, a, b, beta=0.5, alpha=2.0)
    ref = 0.5 * c + 2.0 * matmul_persistent(a, b)
    torch.testing.assert_close(out, ref)


def test_mode_context_is_exception_safe_and_reentrant():
    assert not is_batch_invariant_mode_enabled()
    with pytest.raises(RuntimeError, match="sentinel"):
        with set_batch_invariant_mode():
            assert is_batch_invariant_mode_enabled()
            with set_batch_invariant_mode():
                assert is_batch_invariant_mode_enabled()
            assert is_batch_invariant_mode_enabled()
            raise RuntimeError("sentinel")
    assert not is_batch_invariant_mode_enabled()
