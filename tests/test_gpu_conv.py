"""Convolution family on the GPU (reference tests test_batch_invariance.py:175-450).

Parity bound per output (dot product of K = channels x taps, then the bias):
  regular / transposed: the GEMM rounding is within r_out |d| + gamma_K (1 + r_out) (|x| * |w|) of
  the oracle's rounded dot product d, and the bias add rounds once more: one more ulp of the
  result, so |gpu - oracle| <= r_out (|out| + |d|) + gamma_K (1 + r_out) (|x| * |w|);
  depthwise 1-D: one rounding of the fp32 sum of K taps and the bias:
  r_out |out| + gamma_{K+1} ((|x| * |w|) + |bias|).
r_out = 2^-7 (bf16), 2^-10 (fp16), 1e-5 (fp32, the north-star rtol).
"""

import pytest
import torch
import torch.nn.functional as F

import oracle
from batch_invariant_ops import (
    conv1d_batch_invariant,
    conv2d_batch_invariant,
    conv3d_batch_invariant,
    conv_transpose2d_batch_invariant,
    conv_transpose3d_batch_invariant,
    set_batch_invariant_mode,
)

from _tol import ULP, assert_bitwise, assert_first_sample_equal, gamma

pytestmark = pytest.mark.gpu
DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def randn(*shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def assert_conv_close(actual, x, w, bias, stride, padding, dilation, transposed, groups):
    dtype = actual.dtype
    nd = x.ndim - 2
    op = (0,) * nd
    xc, wc = x.cpu(), w.cpu()
    bc = None if bias is None else bias.cpu()
    expected = oracle.conv(xc, wc, bc, stride, padding, dilation, transposed, op, groups).double()
    absprod = oracle.conv_abs(xc, wc, stride, padding, dilation, transposed, op, groups)
    r_out = 1e-5 if dtype == torch.float32 else ULP[dtype]
    depthwise = nd == 1 and not transposed and groups == x.shape[1] == w.shape[0] and w.shape[1] == 1
    K = x.shape[1] // groups if transposed else w.shape[1] * int(torch.tensor(w.shape[2:]).prod())
    shape = (1, -1) + (1,) * nd
    babs = torch.zeros(1, dtype=torch.float64) if bc is None else bc.double().abs().reshape(shape)
    if depthwise:
        bound = r_out * expected.abs() + gamma(K + 1) * (absprod + babs)
    else:
        dot = oracle.conv(xc, wc, None, stride, padding, dilation, transposed, op, groups).double()
        bound = r_out * (expected.abs() + dot.abs()) + gamma(K) * (1 + r_out) * absprod
    err = (actual.double().cpu() - expected).abs()
    bad = ~(err <= bound)
    assert not bool(bad.any()), f"{int(bad.sum())} of {bad.numel()} outside the bound; max err {float(err.max()):.3e}"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("composition", ("duplicate", "unrelated"))
@pytest.mark.parametrize("batch_size", (2, 5, 17, 32))
def test_siglip_patch_conv_is_batch_invariant(dtype, composition, batch_size):
    target = randn(1, 3, 28, 28, seed=5000 + batch_size, dtype=dtype)
    if composition == "duplicate":
        inputs = target.expand(batch_size, -1, -1, -1).contiguous()
    else:
        inputs = torch.cat((target, randn(batch_size - 1, 3, 28, 28, seed=5100 + batch_size, dtype=dtype)))
    weight = randn(32, 3, 14, 14, seed=5200, dtype=dtype).cuda()
    bias = randn(32, seed=5201, dtype=dtype).cuda()
    args = (weight, bias, (14, 14), (0, 0), (1, 1), False, (0, 0), 1)
    alone = conv2d_batch_invariant(target.cuda(), *args)
    batched = conv2d_batch_invariant(inputs.cuda(), *args)
    assert_first_sample_equal(alone, batched)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch_size", (2, 5, 17))
def test_depthwise_conv1d_is_batch_invariant(dtype, batch_size):
    inputs = randn(batch_size, 32, 73, seed=5800 + batch_size, dtype=dtype).cuda()
    weight = randn(32, 1, 4, seed=5850, dtype=dtype).cuda()
    bias = randn(32, seed=5851, dtype=dtype).cuda()
    args = (weight, bias, (1,), (3,), (1,), False, (0,), 32)
    assert_first_sample_equal(conv1d_batch_invariant(inputs[:1], *args), conv1d_batch_invariant(inputs, *args))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("shape", "weight_shape", "stride", "padding", "dilation", "groups"), (
    ((3, 4, 19), (7, 4, 3), (1,), (0,), (1,), 1),
    ((2, 8, 23), (12, 2, 4), (2,), (3,), (2,), 4),
    ((2, 16, 31), (16, 1, 4), (1,), (3,), (1,), 16),
))
def test_conv1d_matches_oracle(dtype, shape, weight_shape, stride, padding, dilation, groups):
    x = randn(*shape, seed=5900, dtype=dtype).cuda()
    w = randn(*weight_shape, seed=5901, dtype=dtype).cuda()
    b = randn(weight_shape[0], seed=5902, dtype=dtype).cuda()
    out = conv1d_batch_invariant(x, w, b, stride, padding, dilation, False, (0,), groups)
    assert out.shape == F.conv1d(x.cpu().float(), w.cpu().float(), None, stride, padding, dilation, groups).shape
    assert_conv_close(out, x, w, b, stride, padding, dilation, False, groups)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("shape", "weight_shape", "stride", "padding", "dilation", "groups"), (
    ((3, 4, 13, 11), (7, 4, 3, 3), (1, 1), (0, 0), (1, 1), 1),
    ((2, 4, 13, 11), (6, 2, 3, 2), (2, 1), (1, 0), (2, 1), 2),
    ((2, 4, 9, 9), (4, 1, 3, 3), (1, 1), (1, 1), (1, 1), 4),
    ((2, 64, 16, 16), (128, 64, 3, 3), (1, 1), (1, 1), (1, 1), 1),  # K = 576: direct GEMM loads
))
def test_conv2d_matches_oracle(dtype, shape, weight_shape, stride, padding, dilation, groups):
    x = randn(*shape, seed=6000, dtype=dtype).cuda()
    w = randn(*weight_shape, seed=6001, dtype=dtype, scale=0.2).cuda()
    b = randn(weight_shape[0], seed=6002, dtype=dtype).cuda()
    out = conv2d_batch_invariant(x, w, b, stride, padding, dilation, False, (0, 0), groups)
    assert_conv_close(out, x, w, b, stride, padding, dilation, False, groups)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("shape", "weight_shape", "stride", "padding", "dilation", "groups"), (
    ((3, 3, 2, 16, 16), (12, 3, 2, 16, 16), (2, 16, 16), (0, 0, 0), (1, 1, 1), 1),
    ((2, 4, 7, 9, 8), (6, 2, 3, 2, 2), (2, 1, 2), (1, 0, 1), (2, 1, 1), 2),
))
def test_conv3d_matches_oracle(dtype, shape, weight_shape, stride, padding, dilation, groups):
    x = randn(*shape, seed=6500, dtype=dtype).cuda()
    w = randn(*weight_shape, seed=6501, dtype=dtype, scale=0.2).cuda()
    b = randn(weight_shape[0], seed=6502, dtype=dtype).cuda()
    out = conv3d_batch_invariant(x, w, b, stride, padding, dilation, False, (0, 0, 0), groups)
    assert_conv_close(out, x, w, b, stride, padding, dilation, False, groups)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch_size", (2, 5, 17))
def test_qwen_patch_conv3d_is_batch_invariant(dtype, batch_size):
    inputs = randn(batch_size, 3, 2, 16, 16, seed=6700 + batch_size, dtype=dtype).cuda()
    weight = randn(12, 3, 2, 16, 16, seed=6750, dtype=dtype).cuda()
    bias = randn(12, seed=6751, dtype=dtype).cuda()
    args = (weight, bias, (2, 16, 16), (0, 0, 0), (1, 1, 1), False, (0, 0, 0), 1)
    assert_first_sample_equal(conv3d_batch_invariant(inputs[:1], *args), conv3d_batch_invariant(inputs, *args))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("groups", (1, 2))
def test_nonoverlapping_conv_transpose3d_matches_oracle(dtype, groups):
    x = randn(2, 4, 2, 3, 3, seed=6760 + groups, dtype=dtype).cuda()
    w = randn(4, 6 // groups, 2, 2, 2, seed=6761, dtype=dtype).cuda()
    b = randn(6, seed=6762, dtype=dtype).cuda()
    out = conv_transpose3d_batch_invariant(x, w, b, stride=(2, 2, 2), padding=(0, 0, 0), dilation=(1, 1, 1),
                                           output_padding=(0, 0, 0), groups=groups)
    assert_conv_close(out, x, w, b, (2, 2, 2), (0, 0, 0), (1, 1, 1), True, groups)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("groups", (1, 2))
def test_nonoverlapping_conv_transpose2d_matches_oracle(dtype, groups):
    x = randn(2, 4, 3, 3, seed=6730 + groups, dtype=dtype).cuda()
    w = randn(4, 6 // groups, 2, 2, seed=6731, dtype=dtype).cuda()
    b = randn(6, seed=6732, dtype=dtype).cuda()
    out = conv_transpose2d_batch_invariant(x, w, b, stride=(2, 2), padding=(0, 0), dilation=(1, 1),
                                           output_padding=(0, 0), groups=groups)
    assert_conv_close(out, x, w, b, (2, 2), (0, 0), (1, 1), True, groups)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_conv_transpose2d_wide_channels(dtype):
    """128 input channels and 8-aligned spatial runs: the N-major direct GEMM path."""
    x = randn(3, 128, 4, 8, seed=6740, dtype=dtype).cuda()
    w = randn(128, 16, 4, 4, seed=6741, dtype=dtype, scale=0.1).cuda()
    b = randn(16, seed=6742, dtype=dtype).cuda()
    out = conv_transpose2d_batch_invariant(x, w, b, (4, 4), (0, 0), (1, 1), (0, 0), 1)
    assert_conv_close(out, x, w, b, (4, 4), (0, 0), (1, 1), True, 1)
    assert_first_sample_equal(conv_transpose2d_batch_invariant(x[:1], w, b, (4, 4), (0, 0), (1, 1), (0, 0), 1), out)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch_size", (2, 5, 17))
def test_nonoverlapping_conv_transpose2d_is_batch_invariant(dtype, batch_size):
    inputs = randn(batch_size, 8, 3, 3, seed=6775 + batch_size, dtype=dtype).cuda()
    weight = randn(8, 6, 4, 4, seed=6790, dtype=dtype).cuda()
    bias = randn(6, seed=6791, dtype=dtype).cuda()
    args = (weight, bias, (4, 4), (0, 0), (1, 1), (0, 0), 1)
    assert_first_sample_equal(conv_transpose2d_batch_invariant(inputs[:1], *args),
                              conv_transpose2d_batch_invariant(inputs, *args))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch_size", (2, 5, 17))
def test_nonoverlapping_conv_transpose3d_is_batch_invariant(dtype, batch_size):
    inputs = randn(batch_size, 8, 2, 3, 3, seed=6800 + batch_size, dtype=dtype).cuda()
    weight = randn(8, 6, 4, 1, 1, seed=6820, dtype=dtype).cuda()
    bias = randn(6, seed=6821, dtype=dtype).cuda()
    args = (weight, bias, (4, 1, 1), (0, 0, 0), (1, 1, 1), (0, 0, 0), 1)
    assert_first_sample_equal(conv_transpose3d_batch_invariant(inputs[:1], *args),
                              conv_transpose3d_batch_invariant(inputs, *args))


def test_mode_overrides_convolution_family():
    """F.conv* under the mode route through aten::convolution to these kernels (reference
    test_mode_overrides_matmul_and_convolution_family, test_batch_invariance.py:407-449)."""
    image = randn(5, 3, 28, 28, seed=7000).cuda()
    weight = randn(8, 3, 14, 14, seed=7001).cuda()
    signal = randn(5, 8, 19, seed=7002).cuda()
    signal_weight = randn(8, 1, 4, seed=7003).cuda()
    video = randn(5, 3, 2, 16, 16, seed=7004).cuda()
    video_weight = randn(8, 3, 2, 16, 16, seed=7005).cuda()
    latent = randn(5, 8, 2, 3, 3, seed=7006).cuda()
    transpose_weight = randn(8, 6, 4, 1, 1, seed=7007).cuda()
    image_latent = randn(5, 8, 3, 3, seed=7008).cuda()
    image_transpose_weight = randn(8, 6, 4, 4, seed=7009).cuda()
    with set_batch_invariant_mode():
        c1 = F.conv1d(signal, signal_weight, padding=3, groups=8)
        assert_first_sample_equal(F.conv1d(signal[:1], signal_weight, padding=3, groups=8), c1)
        c2 = F.conv2d(image, weight, stride=14)
        assert_first_sample_equal(F.conv2d(image[:1], weight, stride=14), c2)
        c3 = F.conv3d(video, video_weight, stride=(2, 16, 16))
        assert_first_sample_equal(F.conv3d(video[:1], video_weight, stride=(2, 16, 16)), c3)
        t3 = F.conv_transpose3d(latent, transpose_weight, stride=(4, 1, 1))
        assert_first_sample_equal(F.conv_transpose3d(latent[:1], transpose_weight, stride=(4, 1, 1)), t3)
        t2 = F.conv_transpose2d(image_latent, image_transpose_weight, stride=4)
        assert_first_sample_equal(F.conv_transpose2d(image_latent[:1], image_transpose_weight, stride=4), t2)
    # the mode calls are the library's kernels
    assert_bitwise(c1, conv1d_batch_invariant(signal, signal_weight, None, (1,), (3,), (1,), False, (0,), 8))
    assert_bitwise(c2, conv2d_batch_invariant(image, weight, None, (14, 14), (0, 0), (1, 1), False, (0, 0), 1))
    assert_bitwise(t2, conv_transpose2d_batch_invariant(image_latent, image_transpose_weight, None, (4, 4),
                                                        (0, 0), (1, 1), (0, 0), 1))


def test_conv_strided_input_and_edge_cases():
    x = randn(4, 6, 20, 18, seed=7100, dtype=torch.bfloat16).cuda()
    view = x[:, ::2, 1:17, ::2]  # non-contiguous input
    w = randn(5, 3, 3, 3, seed=7101, dtype=torch.bfloat16).cuda()
    out = conv2d_batch_invariant(view, w, None, (1, 1), (1, 1), (1, 1), False, (0, 0), 1)
    assert_bitwise(out, conv2d_batch_invariant(view.contiguous(), w, None, (1, 1), (1, 1), (1, 1), False, (0, 0), 1))
    assert_conv_close(out, view, w, None, (1, 1), (1, 1), (1, 1), False, 1)
    empty = conv2d_batch_invariant(x[:0, :3], w, None, (1, 1), (0, 0), (1, 1), False, (0, 0), 1)
    assert empty.shape == (0, 5, 18, 16)
    with pytest.raises(AssertionError, match="transposed convolution is not supported"):
        conv2d_batch_invariant(x, w, None, (1, 1), (0, 0), (1, 1), True, (0, 0), 2)
    with pytest.raises(AssertionError, match="Incompatible channel dimensions"):
        conv2d_batch_invariant(x, w, None, (1, 1), (0, 0), (1, 1), False, (0, 0), 1)
    tw = randn(6, 2, 3, 3, seed=7102, dtype=torch.bfloat16).cuda()
    with pytest.raises(AssertionError, match="non-overlapping"):
        conv_transpose2d_batch_invariant(x, tw, None, (2, 2), (0, 0), (1, 1), (0, 0), 1)
