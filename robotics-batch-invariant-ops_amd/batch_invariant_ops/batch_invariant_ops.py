"""Batch-invariant operators for PyTorch-ROCm on AMD Instinct MI355X (gfx950).

Same Python API as the reference package ``batch_invariant_ops``
(yiannisha/robotics-batch-invariant-ops, batch_invariant_ops/batch_invariant_ops.py): launch
wrappers (``matmul_persistent``, ``bmm_persistent``, ``softmax``, ``log_softmax``, ``mean_dim``,
``linalg_vector_norm_batch_invariant``), attention composites, the aten signature shims and the
``set_batch_invariant_mode`` registration.  Every numeric op runs in the hand-written HIP kernels
of ``libbiops.so`` (see ``_native``); Python only canonicalises layouts, allocates outputs and
workspaces and validates arguments.  There is no CPU path.
"""

from __future__ import annotations

import contextlib
import ctypes
import math
import threading
from collections import namedtuple
from typing import Any

import torch

from . import _native as nat

__all__ = [
    "set_batch_invariant_mode",
    "is_batch_invariant_mode_enabled",
    "disable_batch_invariant_mode",
    "enable_batch_invariant_mode",
    "matmul_persistent",
    "bmm_persistent",
    "linear_batch_invariant",
    "conv1d_batch_invariant",
    "conv2d_batch_invariant",
    "conv3d_batch_invariant",
    "conv_transpose2d_batch_invariant",
    "conv_transpose3d_batch_invariant",
    "scaled_dot_product_attention_batch_invariant",
    "varlen_scaled_dot_product_attention_batch_invariant",
    "linalg_vector_norm_batch_invariant",
    "softmax",
    "log_softmax",
    "mean_dim",
    "get_batch_invariant_attention_block_size",
    "AttentionBlockSize",
    "get_compute_units",
]

_FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


# ----------------------------------------------------------------- device query ----
def get_compute_units() -> int:
    """Compute units of the current GPU (MI355X: 256).

    Mirrors ``get_compute_units`` (batch_invariant_ops.py:232-253), including its CPU answer
    (the torch thread count) when no GPU is present.  The value sizes the persistent grids;
    it never changes the arithmetic of an output element.
    """
    if not torch.cuda.is_available():
        print("No CUDA or XPU device available. Using CPU.")
        return torch.get_num_threads()
    lib = nat.load()
    n = lib.biops_compute_units()
    if n <= 0:
        raise RuntimeError(f"biops_compute_units failed: {lib.biops_last_error().decode()}")
    return n


def _current_accelerator_type() -> str:
    """Accelerator type, as ``_current_accelerator_type`` (batch_invariant_ops.py:256-268)."""
    accelerator = getattr(torch, "accelerator", None)
    if accelerator is not None:
        current = accelerator.current_accelerator()
        if current is not None:
            return current.type
    return "cuda" if torch.cuda.is_available() else "cpu"


# ------------------------------------------------------------------------- GEMM ----
def _k_contiguous(x: torch.Tensor, k_dim: int) -> torch.Tensor:
    return x if x.stride(k_dim) == 1 or x.shape[k_dim] <= 1 else x.contiguous()


def _b_operand(b: torch.Tensor) -> torch.Tensor:
    """B[..., K, N] with a unit stride in K (W^T of nn.Linear) or in N (row-major)."""
    k, n = b.shape[-2], b.shape[-1]
    if b.stride(-2) == 1 or b.stride(-1) == 1 or k <= 1 or n <= 1:
        return b
    return b.contiguous()


# Products whose operands cannot take the direct global->LDS loads (K not a whole number of
# 128-byte steps, or rows not 16-byte aligned) run through biops_gemm_padded / biops_bmm_padded,
# on zero-padded copies, when they have at least _PAD_MIN_WORK multiply-adds and rows of at
# least _PAD_MIN_K_BYTES (_PAD_MIN_MISALIGNED_K_BYTES when misaligned rows leave the register
# path element-by-element loads); the others keep the register load path of biops_gemm /
# biops_bmm.  Both give the same bits: out-of-range K is zero in both operands on every load
# path.  MI355X, bf16, per call (register path -> padded): 2048 x 2048 x 2050 357 -> 42 us,
# 512 x 512 x 500 50 -> 21 us, 300 x 700 x 5000 77 -> 28 us, 1 x 4096 x 4000 57 -> 27 us,
# bmm 16 x 1024 x 2050 x 256 229 -> 73 us; the register path was as fast or faster with
# aligned rows at K = 1000 (256 x 1024 x 1000 18 against 21 us) and with misaligned rows at
# K = 100 (bmm 64 x 256 x 100 x 256 16.6 against 19.2 us).
_PAD_MIN_WORK = 1 << 23
_PAD_MIN_K_BYTES = 4000
_PAD_MIN_MISALIGNED_K_BYTES = 512


def _aligned16(t: torch.Tensor, ld: int) -> bool:
    return t.data_ptr() % 16 == 0 and (ld * t.element_size()) % 16 == 0


def _padded_workspace(a: torch.Tensor, b: torch.Tensor, M: int, N: int, K: int, batch: int = 0) -> int:
    """Workspace bytes of biops_gemm_padded for A [M, K] and B [K, N] (unit stride in K or N),
    or of biops_bmm_padded (``batch`` > 0) for A [batch, M, K] and B [batch, K, N]; 0 when the
    product should run on the operands as they are."""
    elt = a.element_size()
    step = 128 // elt
    kmajor = b.stride(-2) == 1 or K <= 1
    if not kmajor and b.stride(-1) != 1 and N > 1:
        return 0
    ldb = b.stride(-1) if kmajor else b.stride(-2)
    aligned = (_aligned16(a, a.stride(-2)) and _aligned16(b, ldb) and (kmajor or (N * elt) % 16 == 0)
               and (not batch or (a.stride(0) * elt) % 16 == 0 and (b.stride(0) * elt) % 16 == 0))
    if aligned and K % step == 0:
        return 0
    if max(batch, 1) * M * N * K < _PAD_MIN_WORK:
        return 0
    if K * elt < (_PAD_MIN_K_BYTES if aligned else _PAD_MIN_MISALIGNED_K_BYTES):
        return 0
    kp = -(-K // step) * step
    np_ = N if kmajor else -(-N * elt // 16) * 16 // elt
    na = 1 if not batch or a.stride(0) == 0 else batch
    nb = 1 if not batch or b.stride(0) == 0 else batch
    return -(-na * M * kp * elt // 256) * 256 + nb * (N * kp if kmajor else kp * np_) * elt


def matmul_persistent(a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None = None):
    """C = A @ B (+ bias) with a fixed tile, K order and MFMA instruction, fp32 accumulation.

    Reference: matmul_persistent (batch_invariant_ops.py:271-343) and its kernel (60-139):
    the bias is added to the fp32 accumulator before the single rounding to ``a.dtype``.
    """
    assert a.shape[1] == b.shape[0], "Incompatible dimensions"
    assert a.dtype == b.dtype, "Incompatible dtypes"
    assert (
        bias is None or bias.dim() == 1
    ), "Currently assuming bias is 1D, let Horace know if you run into this"
    nat.require_gpu_tensors(a, b, bias)
    code = nat.dtype_code(a.dtype)
    M, K = a.shape
    N = b.shape[1]
    c = torch.empty((M, N), device=a.device, dtype=a.dtype)
    if M == 0 or N == 0:
        return c
    a = _k_contiguous(a, 1)
    b = _b_operand(b)
    bias_ptr = None
    if bias is not None:
        if bias.numel() == 1 and N != 1:
            bias = bias.expand(N)
        assert bias.shape[0] == N, "bias length must equal the number of output columns"
        bias = bias.to(a.dtype).contiguous()
        bias_ptr = bias.data_ptr()
    stream = nat.stream_of(c)
    ws_bytes = _padded_workspace(a, b, M, N, K) if K > 0 else 0
    if ws_bytes:
        ws = torch.empty(ws_bytes, device=a.device, dtype=torch.uint8)
        if ws.data_ptr() % 256 == 0:
            rc = _fast_fn("biops_gemm_padded")(
                code, M, N, K, a.data_ptr(), a.stride(0), a.stride(1), b.data_ptr(), b.stride(0), b.stride(1),
                bias_ptr, c.data_ptr(), c.stride(0), c.stride(1), ws.data_ptr(), ws_bytes, stream)
            nat.check(rc, "biops_gemm_padded")
            return c
    nat.call(
        "biops_gemm",
        code, M, N, K,
        a.data_ptr(), a.stride(0), a.stride(1),
        b.data_ptr(), b.stride(0), b.stride(1),
        bias_ptr,
        c.data_ptr(), c.stride(0), c.stride(1),
        stream,
    )
    return c


def bmm_persistent(a: torch.Tensor, b: torch.Tensor):
    """Batch-invariant ``torch.bmm``: every batch element is an independent fixed-schedule GEMM.

    Reference: bmm_persistent (batch_invariant_ops.py:346-431).  Stride-0 (expanded) and
    transposed operands are read in place; batches beyond the 65 535 grid limit are walked by
    the persistent grid.
    """
    assert a.ndim == b.ndim == 3, "bmm expects two rank-3 tensors"
    assert a.shape[0] == b.shape[0] and a.shape[2] == b.shape[1], "Incompatible dimensions"
    assert a.dtype == b.dtype, "Incompatible dtypes"
    assert a.dtype in set(_FLOAT_DTYPES), f"unsupported dtype: {a.dtype}"
    nat.require_gpu_tensors(a, b)
    batch, m, k = a.shape
    n = b.shape[2]
    c = torch.empty((batch, m, n), device=a.device, dtype=a.dtype)
    if batch == 0 or m == 0 or n == 0:
        return c
    a = _k_contiguous(a, 2)
    b = _b_operand(b)
    stream = nat.stream_of(c)
    ws_bytes = _padded_workspace(a, b, m, n, k, batch) if k > 0 else 0
    if ws_bytes:
        ws = torch.empty(ws_bytes, device=a.device, dtype=torch.uint8)
        if ws.data_ptr() % 256 == 0:
            nat.call(
                "biops_bmm_padded",
                nat.dtype_code(a.dtype), batch, m, n, k,
                a.data_ptr(), a.stride(0), a.stride(1), a.stride(2),
                b.data_ptr(), b.stride(0), b.stride(1), b.stride(2),
                c.data_ptr(), c.stride(0), c.stride(1), c.stride(2),
                ws.data_ptr(), ws_bytes, stream,
            )
            return c
    nat.call(
        "biops_bmm",
        nat.dtype_code(a.dtype), batch, 1, m, n, k,
        a.data_ptr(), a.stride(0), 0, a.stride(1), a.stride(2),
        b.data_ptr(), b.stride(0), 0, 1, b.stride(1), b.stride(2),
        c.data_ptr(), c.stride(0), 0, c.stride(1), c.stride(2),
        stream,
    )
    return c


def mm_batch_invariant(a, b):
    """``aten::mm`` override (batch_invariant_ops.py:1600-1601)."""
    return matmul_persistent(a, b)


def addmm_batch_invariant(bias, a, b, *, beta=1, alpha=1):
    """``aten::addmm`` override (batch_invariant_ops.py:1604-1605).

    The common case (beta = alpha = 1, 1-D or [1, N] bias) is one fused kernel; other scalings
    and a full [M, N] bias are applied to the invariant product with elementwise ops.
    """
    if beta == 1 and alpha == 1 and (bias.dim() == 1 or (bias.dim() == 2 and bias.shape[0] == 1)):
        return matmul_persistent(a, b, bias=bias.reshape(-1))
    product = matmul_persistent(a, b)
    if alpha != 1:
        product = product * alpha
    if beta == 0:
        return product
    return product + (bias if beta == 1 else bias * beta)


def _linear_direct(input, weight, bias):
    """``linear`` for the common layout -- contiguous input, weight rows of unit stride, a
    matching 1-D bias -- straight into ``biops_gemm`` without intermediate views (the decode
    loop of a policy is bound by per-call host time at small batch).  Returns None when the
    arguments need the general path."""
    if not (input.is_cuda and weight.is_cuda and weight.dim() == 2 and input.dim() >= 1):
        return None
    dtype = input.dtype
    code = nat.DIRECT_DTYPES.get(dtype)
    if code is None or weight.dtype != dtype or not input.is_contiguous() or weight.stride(1) != 1:
        return None
    n, k = weight.shape
    shape = input.shape
    if shape[-1] != k or k == 0 or n == 0:
        return None
    elt = input.element_size()
    if (k * elt) % 128:
        # K not a whole number of 128-byte steps: products that repay the padded copies take the
        # general path (biops_gemm_padded), the others the register loads here
        m = input.numel() // k
        aligned = (input.data_ptr() | weight.data_ptr()) % 16 == 0 and (k * elt) % 16 == 0 and \
            (weight.stride(0) * elt) % 16 == 0
        if m * n * k >= _PAD_MIN_WORK and k * elt >= (_PAD_MIN_K_BYTES if aligned else _PAD_MIN_MISALIGNED_K_BYTES):
            return None
    bias_ptr = None
    if bias is not None:
        if not (bias.is_cuda and bias.dim() == 1 and bias.dtype == dtype and bias.shape[0] == n
                and bias.stride(0) == 1):
            return None
        bias_ptr = bias.data_ptr()
    m = input.numel() // k
    out = torch.empty((*shape[:-1], n), device=input.device, dtype=dtype)
    if m:
        rc = _gemm_fn()(code, m, n, k, input.data_ptr(), k, 1, weight.data_ptr(), 1, weight.stride(0),
                        bias_ptr, out.data_ptr(), n, 1, nat.stream_of(out))
        if rc:
            nat.check(rc, "biops_gemm")
    return out


_gemm = None


def _gemm_fn():
    global _gemm
    if _gemm is None:
        _gemm = nat.fast_function("biops_gemm")
    return _gemm


def linear_batch_invariant(input, weight, bias=None):
    """Batch-invariant ``aten::linear`` for arbitrary leading dimensions.

    Reference: linear_batch_invariant (batch_invariant_ops.py:1608-1616): leading dims flatten
    into GEMM rows; ``weight.T`` is read in place (unit stride in K).
    """
    out = _linear_direct(input, weight, bias)
    if out is not None:
        return out
    assert input.ndim >= 1, "linear input must have at least one dimension"
    assert weight.ndim == 2, "linear weight must be a matrix"
    assert input.shape[-1] == weight.shape[-1], "Incompatible dimensions"
    output_shape = (*input.shape[:-1], weight.shape[0])
    flattened = input.reshape(-1, input.shape[-1])
    output = matmul_persistent(flattened, weight.transpose(0, 1), bias=bias)
    return output.reshape(output_shape)


def bmm_batch_invariant(a, b):
    """``aten::bmm`` override (batch_invariant_ops.py:1619-1620)."""
    return bmm_persistent(a, b)


# --------------------------------------------------------------- row reductions ----
_fast_fns = {}


def _fast_fn(name):
    """nat.fast_function(name), looked up once."""
    fn = _fast_fns.get(name)
    if fn is None:
        fn = _fast_fns[name] = nat.fast_function(name)
    return fn


def _last_dim_fast(input, dim) -> int:
    """Row length when ``input`` is a contiguous CUDA tensor of a kernel dtype reduced over its
    last dimension with rows to reduce, else 0.  The common RMSNorm / pooling / attention
    calls take this path straight into the library (per-call host time is what bounds them at
    model shapes)."""
    if not input.is_cuda or input.dtype not in nat.DIRECT_DTYPES or not input.is_contiguous():
        return 0
    nd = input.dim()
    if nd == 0 or (dim != -1 and dim != nd - 1):
        return 0
    n = input.shape[-1]
    return n if n > 0 and input.numel() > 0 else 0


def _reduce_last_fast(op, input, n, keepdim):
    """biops_reduce over the last dimension of a contiguous tensor (see _last_dim_fast)."""
    shape = input.shape
    out = torch.empty((*shape[:-1], 1) if keepdim else shape[:-1], dtype=input.dtype, device=input.device)
    code = nat.DIRECT_DTYPES[input.dtype]
    rc = _fast_fn("biops_reduce")(op, code, code, input.numel() // n, n, 1, input.data_ptr(), n, 1, 1,
                                 out.data_ptr(), nat.stream_of(out))
    if rc:
        nat.check(rc, "biops_reduce")
    return out


def _rows_last(input: torch.Tensor, dim: int) -> tuple[torch.Tensor, int]:
    """``input`` with ``dim`` moved last and rows contiguous, plus the normalised dim."""
    dim %= input.ndim
    moved = input.movedim(dim, -1)
    if not moved.is_contiguous():
        moved = moved.contiguous()
    return moved, dim


def _softmax_impl(input, dim, out_dtype, is_log):
    n = _last_dim_fast(input, dim)
    if n and out_dtype in nat.DIRECT_DTYPES:
        out = torch.empty(input.shape, dtype=out_dtype, device=input.device)
        rc = _fast_fn("biops_softmax")(nat.DIRECT_DTYPES[input.dtype], nat.DIRECT_DTYPES[out_dtype],
                                      input.numel() // n, n, input.data_ptr(), n, out.data_ptr(), n,
                                      int(is_log), nat.stream_of(out))
        if rc:
            nat.check(rc, "biops_softmax")
        return out
    nat.require_gpu_tensors(input)
    if input.ndim == 0:
        return _softmax_impl(input.reshape(1), 0, out_dtype, is_log).reshape(())
    moved, dim = _rows_last(input, dim)
    out = torch.empty(moved.shape, dtype=out_dtype, device=input.device)
    cols = moved.shape[-1] if moved.ndim else 1
    rows = moved.numel() // cols if cols else 0
    if rows and cols:
        nat.call(
            "biops_softmax",
            nat.dtype_code(input.dtype), nat.dtype_code(out_dtype), rows, cols,
            moved.data_ptr(), cols, out.data_ptr(), cols, int(is_log),
            nat.stream_of(out),
        )
    return out.movedim(-1, dim)


def softmax(input: torch.Tensor, dim: int = -1, *, dtype: torch.dtype | None = None) -> torch.Tensor:
    """Batch-invariant softmax along any dimension (one wavefront per row, fixed tree).

    Reference: softmax/_softmax_kernel (batch_invariant_ops.py:1074-1145).  An all -inf row
    gives 0 (not NaN); ``dtype`` sets the output dtype.
    """
    if input.dtype not in _FLOAT_DTYPES:
        raise ValueError(f"unsupported softmax dtype: {input.dtype}")
    if dtype not in {None, *_FLOAT_DTYPES}:
        raise ValueError(f"unsupported softmax output dtype: {dtype}")
    return _softmax_impl(input, dim, dtype or input.dtype, False)


def log_softmax(input: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """Batch-invariant log-softmax along any dimension.

    Reference: log_softmax/_log_softmax_kernel (batch_invariant_ops.py:974-1071).
    """
    if input.dtype not in _FLOAT_DTYPES:
        raise ValueError(f"unsupported log_softmax dtype: {input.dtype}")
    return _softmax_impl(input, dim, input.dtype, True)


def _softmax_batch_invariant(input, dim, _half_to_float):
    """``aten::_softmax`` override (batch_invariant_ops.py:1628-1630); half_to_float gives fp32."""
    return softmax(input, dim=dim, dtype=torch.float32 if _half_to_float else None)


def _log_softmax_batch_invariant(input, dim, _half_to_float):
    """``aten::_log_softmax`` override (batch_invariant_ops.py:1623-1625)."""
    if _half_to_float:
        return log_softmax(input.float(), dim=dim)
    return log_softmax(input, dim=dim)


_INT_DTYPES = (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8)


def _reduce(op, x3: torch.Tensor, out: torch.Tensor, M: int, N: int, K: int) -> None:
    if K == 1 and N > 1 and x3.stride(1) != 1:
        x3 = x3.contiguous()
    nat.call(
        "biops_reduce",
        op, nat.dtype_code(x3.dtype), nat.dtype_code(out.dtype), M, N, K,
        x3.data_ptr(), x3.stride(0), x3.stride(1), x3.stride(2),
        out.data_ptr(), nat.stream_of(out),
    )


def mean_dim(
    input: torch.Tensor, dim: int, keepdim: bool = False, dtype: torch.dtype | None = None
) -> torch.Tensor:
    """Mean over one dimension with a fixed fp32 reduction tree per output element.

    Reference: mean_dim/mean_kernel (batch_invariant_ops.py:1347-1482): the input is viewed as
    (M, N, K) with N reduced; integer inputs produce fp32.  Partial sums are fp32 for every
    input dtype.
    """
    if dtype is None or dtype == input.dtype:
        n = _last_dim_fast(input, dim)
        if n:
            return _reduce_last_fast(nat.REDUCE_MEAN, input, n, keepdim)
    assert input.is_cuda, "Input must be a CUDA tensor"
    assert -input.ndim <= dim < input.ndim, f"Invalid dimension {dim} for tensor with {input.ndim} dimensions"
    if dim < 0:
        dim += input.ndim
    if dtype is None:
        dtype = torch.float32 if input.dtype in _INT_DTYPES else input.dtype
    if input.dtype != dtype:
        input = input.to(dtype)
    if dtype not in _FLOAT_DTYPES:
        raise TypeError(f"batch-invariant mean does not support {dtype}")
    shape = list(input.shape)
    M = math.prod(shape[:dim])
    N = shape[dim]
    K = math.prod(shape[dim + 1 :])
    output_shape = shape.copy()
    if keepdim:
        output_shape[dim] = 1
    else:
        del output_shape[dim]
    output = torch.empty(output_shape, dtype=dtype, device=input.device)
    if M * K == 0:
        return output
    _reduce(nat.REDUCE_MEAN, input.reshape(M, N, K), output, M, N, K)
    return output


def mean_batch_invariant(input, dim, keepdim=False, dtype: torch.dtype | None = None):
    """``aten::mean.dim`` override (batch_invariant_ops.py:1633-1651).

    One dimension: ``mean_dim``.  Several (or none = all): the reduced dimensions are moved
    last and flattened into one contiguous row per output, reduced by the same fixed tree
    (the reference falls back to a stock ``torch.sum`` there).  ``dtype`` is honoured as in
    ``torch.mean`` (the input is cast first).
    """
    if (dtype is None or dtype == input.dtype) and dim is not None and len(dim) == 1:
        n = _last_dim_fast(input, dim[0])
        if n:
            return _reduce_last_fast(nat.REDUCE_MEAN, input, n, keepdim)
    nat.require_gpu_tensors(input)
    if dtype is not None and input.dtype != dtype:
        input = input.to(dtype)
    if dim is None or len(dim) == 0:
        dim = list(range(input.ndim))
    dims = sorted({d % input.ndim for d in dim}) if input.ndim else []
    if len(dims) == 1:
        return mean_dim(input, dims[0], keepdim=keepdim)
    out_dtype = torch.float32 if input.dtype in _INT_DTYPES else input.dtype
    if input.dtype != out_dtype:
        input = input.to(out_dtype)
    if out_dtype not in _FLOAT_DTYPES:
        raise TypeError(f"batch-invariant mean does not support {out_dtype}")
    kept = [d for d in range(input.ndim) if d not in dims]
    kept_shape = [input.shape[d] for d in kept]
    R = math.prod(input.shape[d] for d in dims)
    M = math.prod(kept_shape)
    rows = input.permute(*kept, *dims).reshape(M, R, 1)
    output = torch.empty(kept_shape, dtype=out_dtype, device=input.device)
    if M > 0:
        _reduce(nat.REDUCE_MEAN, rows, output, M, R, 1)
    if keepdim:
        for d in dims:
            output = output.unsqueeze(d)
    return output


def linalg_vector_norm_batch_invariant(
    input: torch.Tensor,
    ord: float = 2,
    dim: int | list[int] | tuple[int, ...] | None = None,
    keepdim: bool = False,
    *,
    dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """Euclidean norm sqrt(sum x^2) with fp32 accumulation and a fixed tree per output.

    Reference: linalg_vector_norm_batch_invariant/_vector_norm_kernel
    (batch_invariant_ops.py:1485-1597): a contiguous single-dimension reduction keeps the
    (M, N, K) layout; anything else is permuted to one contiguous row per output.
    """
    if dtype is None and (ord == 2 or ord == 2.0):
        d0 = dim if isinstance(dim, int) else (dim[0] if dim is not None and len(dim) == 1 else None)
        n = _last_dim_fast(input, d0) if d0 is not None else 0
        if n:
            return _reduce_last_fast(nat.REDUCE_L2, input, n, keepdim)
    assert input.is_cuda, "input must be a CUDA tensor"
    assert input.is_floating_point(), "only real floating-point inputs are supported"
    assert float(ord) == 2.0, f"only the Euclidean norm is supported, got ord={ord!r}"
    if dtype is not None:
        assert dtype in {torch.float16, torch.bfloat16, torch.float32, torch.float64}, f"unsupported dtype: {dtype}"
        assert dtype != torch.float64, "float64 is not supported by the HIP kernel"
        input = input.to(dtype)
    assert input.dtype != torch.float64, "float64 is not supported by the HIP kernel"
    if dim is None:
        dimensions = tuple(range(input.ndim))
    elif isinstance(dim, int):
        dimensions = (dim,)
    else:
        dimensions = tuple(dim)
    dimensions = tuple(d % input.ndim for d in dimensions) if input.ndim else ()
    assert len(set(dimensions)) == len(dimensions), "duplicate dimensions are not allowed"
    retained = tuple(d for d in range(input.ndim) if d not in dimensions)
    retained_shape = tuple(input.shape[d] for d in retained)
    if len(dimensions) == 1 and input.is_contiguous():
        d0 = dimensions[0]
        M = math.prod(input.shape[:d0])
        R = input.shape[d0]
        K = math.prod(input.shape[d0 + 1 :])
        kernel_input = input.reshape(M, R, K)
    else:
        R = math.prod(input.shape[d] for d in dimensions)
        M = math.prod(retained_shape)
        K = 1
        kernel_input = input.permute(*retained, *dimensions).contiguous().reshape(M, R, K)
    output = torch.empty(M * K, device=input.device, dtype=input.dtype)
    if M * K > 0:
        _reduce(nat.REDUCE_L2, kernel_input, output, M, R, K)
    output = output.reshape(retained_shape)
    if keepdim:
        for d in sorted(dimensions):
            output = output.unsqueeze(d)
    return output


# -------------------------------------------------------------------- attention ----
def _fused_attention_ok(dtype, d, dv, *tensors, varlen=False):
    """True when the fused attention kernel takes this call: bf16/fp16, head sizes multiples of
    8 up to 256 (128 for varlen), 16-byte aligned rows.  ``BIOPS_ATTENTION_MATERIALIZE=1``
    selects the materialised-score path (same operator, row sums in the row kernel's order)."""
    if dtype not in (torch.bfloat16, torch.float16) or nat.env_flag("BIOPS_ATTENTION_MATERIALIZE", False):
        return False
    lib = nat.load()
    supported = lib.biops_varlen_fused_supported if varlen else lib.biops_attention_fused_supported
    if not supported(nat.dtype_code(dtype), d, dv):
        return False
    for t in tensors:
        if t.data_ptr() % 16 or any(st % 8 for st in t.stride()[:-1]):
            return False
    return True


def _sdpa_glue(q4, k4, v4, group, mask4, scale, out_dtype):
    """Eager SDPA for mask dtypes the fused softmax does not take (type promotion): the GEMMs
    and the softmax are the library kernels, the masking is the reference's elementwise glue
    (batch_invariant_ops.py:1194-1212)."""
    B, Hq, Lq, D = q4.shape
    Lk = k4.shape[2]
    if group > 1:
        k4 = k4.repeat_interleave(group, dim=1)
        v4 = v4.repeat_interleave(group, dim=1)
    scores = bmm_persistent(q4.reshape(B * Hq, Lq, D), k4.reshape(B * Hq, Lk, D).transpose(1, 2))
    scores = (scores * scale).reshape(B, Hq, Lq, Lk)
    scores = scores + mask4
    probabilities = softmax(scores, dim=-1, dtype=out_dtype)
    return bmm_persistent(probabilities.reshape(B * Hq, Lq, Lk), v4.reshape(B * Hq, Lk, v4.shape[-1]))


def scaled_dot_product_attention_batch_invariant(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attn_mask: torch.Tensor | None = None,
    dropout_p: float = 0.0,
    is_causal: bool = False,
    *,
    scale: float | None = None,
    enable_gqa: bool = False,
) -> torch.Tensor:
    """Eager SDPA from the fixed-schedule GEMM and softmax kernels.

    Reference: scaled_dot_product_attention_batch_invariant (batch_invariant_ops.py:1148-1213):
    S = round(Q K^T); S = round(S * scale); causal (top-left) / boolean mask -> -inf, additive
    mask -> round(S + mask); P = softmax(S) in ``query.dtype``; O = P V.  Scale and masking are
    fused into the softmax kernel; grouped-query heads index the shared key/value head instead
    of copying it.
    """
    if dropout_p != 0.0:
        raise ValueError("batch-invariant SDPA only supports dropout_p=0")
    if query.ndim < 3 or key.ndim != query.ndim or value.ndim != query.ndim:
        raise ValueError("query, key, and value must have matching rank >= 3")
    if query.dtype != key.dtype or query.dtype != value.dtype:
        raise ValueError("query, key, and value must have the same dtype")
    if query.dtype not in _FLOAT_DTYPES:
        raise ValueError(f"unsupported varlen attention dtype: {query.dtype}")
    group = 1
    if enable_gqa:
        if query.shape[-3] % key.shape[-3] or key.shape[-3] != value.shape[-3]:
            raise ValueError("invalid grouped-query attention head counts")
        group = query.shape[-3] // key.shape[-3]
    kv_heads_expected = query.shape[-3] // group
    if (
        query.shape[:-3] != key.shape[:-3]
        or query.shape[:-3] != value.shape[:-3]
        or key.shape[-3] != kv_heads_expected
        or value.shape[-3] != kv_heads_expected
    ):
        raise ValueError("leading query, key, and value dimensions must match")
    if query.shape[-1] != key.shape[-1] or key.shape[-2] != value.shape[-2]:
        raise ValueError("incompatible attention dimensions")
    if is_causal and attn_mask is not None:
        raise ValueError("attn_mask and is_causal cannot both be set")
    nat.require_gpu_tensors(query, key, value, attn_mask)

    leading = query.shape[:-2]
    Lq, Lk = query.shape[-2], key.shape[-2]
    D, Dv = query.shape[-1], value.shape[-1]
    Hq = query.shape[-3]
    Hkv = Hq // group
    B = math.prod(query.shape[:-3])
    scale_value = scale if scale is not None else 1.0 / math.sqrt(D)

    def as4(x, h, length, width):
        x = x.reshape(B, h, length, width)
        return x if x.stride(-1) == 1 or width <= 1 else x.contiguous()

    q4 = as4(query, Hq, Lq, D)
    k4 = as4(key, Hkv, Lk, D)
    v4 = as4(value, Hkv, Lk, Dv)

    mask4 = None
    mask_code = 0
    if attn_mask is not None:
        mask4 = attn_mask.expand(*leading, Lq, Lk).reshape(B, Hq, Lq, Lk)
        if attn_mask.dtype == torch.bool:
            mask_code = nat.BOOL
        elif attn_mask.dtype == query.dtype:
            mask_code = nat.dtype_code(query.dtype)
        else:
            out = _sdpa_glue(q4, k4, v4, group, mask4, scale_value, query.dtype)
            return out.reshape(*leading, Lq, Dv)

    out = torch.empty((B, Hq, Lq, Dv), dtype=query.dtype, device=query.device)
    if out.numel() == 0:
        return out.reshape(*leading, Lq, Dv)
    causal_code = nat.CAUSAL_TOP_LEFT if is_causal else nat.CAUSAL_NONE
    fused = _fused_attention_ok(query.dtype, D, Dv, q4, k4, v4)
    if fused and mask4 is not None:
        fused = bool(nat.load().biops_attention_fused_mask_ok(mask4.data_ptr(), mask_code, Lk, *mask4.stride()))
    if fused:
        rc = _fast_fn("biops_sdpa_fused")(
            nat.dtype_code(query.dtype), B, Hq, Hkv, Lq, Lk, D, Dv,
            q4.data_ptr(), q4.stride(0), q4.stride(1), q4.stride(2),
            k4.data_ptr(), k4.stride(0), k4.stride(1), k4.stride(2),
            v4.data_ptr(), v4.stride(0), v4.stride(1), v4.stride(2),
            mask4.data_ptr() if mask4 is not None else None, mask_code,
            *(mask4.stride() if mask4 is not None else (0, 0, 0, 0)),
            causal_code, float(scale_value), out.data_ptr(), nat.stream_of(out),
        )
        nat.check(rc, "biops_sdpa_fused")
        return out.reshape(*leading, Lq, Dv)
    ws_bytes = nat.load().biops_sdpa_workspace_size(nat.dtype_code(query.dtype), B, Hq, Lq, Lk)
    workspace = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=query.device)
    nat.call(
        "biops_sdpa",
        nat.dtype_code(query.dtype), B, Hq, Hkv, Lq, Lk, D, Dv,
        q4.data_ptr(), q4.stride(0), q4.stride(1), q4.stride(2),
        k4.data_ptr(), k4.stride(0), k4.stride(1), k4.stride(2),
        v4.data_ptr(), v4.stride(0), v4.stride(1), v4.stride(2),
        mask4.data_ptr() if mask4 is not None else None, mask_code,
        *(mask4.stride() if mask4 is not None else (0, 0, 0, 0)),
        causal_code, float(scale_value),
        out.data_ptr(), workspace.data_ptr(), workspace.numel(),
        nat.stream_of(out),
    )
    return out.reshape(*leading, Lq, Dv)


def _offsets_on_host(cu_q, cu_kv):
    """Both offset lists as host int64 arrays: one blocking device-to-host copy (the reference
    synchronises here too, batch_invariant_ops.py:1264-1265), shared when the query and key
    offsets are the same tensor, as in self-attention over a packed batch."""
    import numpy as np

    host_q = np.ascontiguousarray(cu_q.detach().cpu().numpy(), dtype=np.int64)
    if cu_kv is cu_q:
        return host_q, host_q
    return host_q, np.ascontiguousarray(cu_kv.detach().cpu().numpy(), dtype=np.int64)


class _VarlenStaging:
    """Pinned host buffer + device buffer pairs for the varlen work list, a ring of up to
    ``RING`` pairs per (device, stream), reused across calls.  The event recorded after each
    call's upload keeps a pair's host buffer untouched until that copy has run: a call takes
    the least recently used pair whose event has completed, and waits on an event only when
    every pair of the ring is still in flight.  A lock covers the choice, the write, the
    upload and the launch."""

    RING = 4
    _cache: dict = {}
    _lock = threading.Lock()
    _h2d = None  # the fast-call module's host-to-device copy, False without the module

    def __init__(self, words, device):
        self.host = torch.empty(words, dtype=torch.int64, pin_memory=True)
        self.dev = torch.empty(words, dtype=torch.int64, device=device)
        self.view = self.host.numpy()
        self.event = torch.cuda.Event()

    @classmethod
    def get(cls, device, stream, words):
        ring = cls._cache.setdefault((device.index, stream), [])  # least recently used first
        idle = None
        for i, st in enumerate(ring):
            if st.event.query():  # the last upload from this host buffer has run
                if st.view.size >= words:
                    ring.append(ring.pop(i))
                    return st
                idle = i if idle is None else idle
        if len(ring) < cls.RING:
            ring.append(cls(max(words, 4096), device))
            return ring[-1]
        i = 0 if idle is None else idle
        ring[i].event.synchronize()
        if ring[i].view.size < words:
            # a grown pair replaces the old one (the device buffer goes back to torch's stream-
            # ordered allocator; the work queued on it runs first)
            ring[i] = cls(max(words, 2 * ring[i].view.size), device)
        ring.append(ring.pop(i))
        return ring[-1]

    def upload(self, used, stream):
        """The first ``used`` words of the host buffer to the device buffer, on ``stream``,
        then the event that guards the host buffer."""
        copy = nat.fast_copy_h2d() if _VarlenStaging._h2d is None else _VarlenStaging._h2d
        if copy:
            _VarlenStaging._h2d = copy
            rc = copy(self.dev.data_ptr(), self.host.data_ptr(), 8 * used, stream)
            if rc != 0:
                raise RuntimeError(f"hipMemcpyAsync of the varlen work list failed ({rc})")
        else:
            _VarlenStaging._h2d = False
            self.dev[:used].copy_(self.host[:used], non_blocking=True)
        self.event.record()


def _varlen_plan(cu_q, cu_kv, heads, value_dim, dtype, out):
    """The work list of biops_varlen_plan in ``out`` (int64 numpy array).  Returns (plan words,
    workspace bytes)."""
    nseq = len(cu_q) - 1
    words = int(nat.load().biops_varlen_plan_len(nseq))
    ws_bytes = _fast_fn("biops_varlen_plan")(nseq, cu_q.ctypes.data, cu_kv.ctypes.data, heads, value_dim,
                                             nat.dtype_code(dtype), out.ctypes.data)
    if ws_bytes < 0:
        raise ValueError(nat.last_error())
    return words, ws_bytes


def _varlen_words(nseq, total_q, fused):
    """Upper bound of the plan (and, for the fused kernel, tile order) words: at most
    total_q / 128 + nseq query tiles (each sequence adds at most one partial tile)."""
    return 8 + 8 * nseq + (total_q // 128 + nseq if fused else 0)


def varlen_scaled_dot_product_attention_batch_invariant(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    cumulative_seqlen_q: torch.Tensor,
    cumulative_seqlen_kv: torch.Tensor,
    *,
    is_causal: bool = False,
    causal_type: Any | None = None,
    scale: float | None = None,
) -> torch.Tensor:
    """Attention over sequence-packed inputs ``[1, total_tokens, heads, head_dim]``.

    Reference: varlen_scaled_dot_product_attention_batch_invariant
    (batch_invariant_ops.py:1216-1344).  Every (sequence, head) pair is an independent GEMM /
    softmax / GEMM problem in one grouped launch per stage, so a sequence's bits never depend
    on the rest of the pack.  Rows outside every sequence, and sequences with an empty key
    range, stay zero.  ``causal_type`` accepts enum-like values named ``TopLeft``,
    ``BottomRight`` or ``DontCare`` (the latter only for equal query / key lengths).
    """
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        raise ValueError("varlen attention expects rank-4 query, key, and value")
    if query.shape[0] != 1 or key.shape[0] != 1 or value.shape[0] != 1:
        raise ValueError("varlen attention expects sequence-packed batch size 1")
    if query.dtype != key.dtype or query.dtype != value.dtype:
        raise ValueError("query, key, and value must have the same dtype")
    if key.shape[1] != value.shape[1] or key.shape[2] != value.shape[2]:
        raise ValueError("key and value token and head dimensions must match")
    if query.shape[3] != key.shape[3]:
        raise ValueError("query and key head dimensions must match")
    if key.shape[2] == 0 or query.shape[2] % key.shape[2]:
        raise ValueError("query heads must be divisible by key/value heads")
    if cumulative_seqlen_q.ndim != 1 or cumulative_seqlen_kv.ndim != 1:
        raise ValueError("cumulative sequence lengths must be rank 1")
    integer_dtypes = {torch.int32, torch.int64}
    if cumulative_seqlen_q.dtype not in integer_dtypes or cumulative_seqlen_kv.dtype not in integer_dtypes:
        raise ValueError("cumulative sequence lengths must use int32 or int64")
    if cumulative_seqlen_q.numel() != cumulative_seqlen_kv.numel():
        raise ValueError("query and KV cumulative sequence counts must match")
    if query.dtype not in _FLOAT_DTYPES:
        raise ValueError(f"unsupported varlen attention dtype: {query.dtype}")

    nat.require_gpu_tensors(query, key, value)
    causal_name = getattr(causal_type, "name", None)
    if causal_name is None and causal_type is not None:
        causal_name = str(causal_type).rsplit(".", 1)[-1]
    heads, kv_heads = query.shape[2], key.shape[2]
    head_dim, value_dim = query.shape[3], value.shape[3]
    out_shape = (1, query.shape[1], heads, value_dim)

    # Everything that does not depend on the offsets' values happens before the host waits for
    # them (below), while the GPU still runs earlier work.
    def tokens_heads(x):
        return x if x.stride(3) == 1 or x.shape[3] <= 1 else x.contiguous()

    q, k, v = tokens_heads(query), tokens_heads(key), tokens_heads(value)
    fused = _fused_attention_ok(query.dtype, head_dim, value_dim, q, k, v, varlen=True)
    if is_causal:
        causal = nat.CAUSAL_BOTTOM_RIGHT if causal_name == "BottomRight" else nat.CAUSAL_TOP_LEFT
    else:
        causal = nat.CAUSAL_NONE
    scale_value = float(scale if scale is not None else 1.0 / math.sqrt(head_dim))
    output = torch.empty(out_shape, dtype=value.dtype, device=value.device)
    stream = nat.stream_of(output)

    cu_q, cu_kv = _offsets_on_host(cumulative_seqlen_q, cumulative_seqlen_kv)
    if cu_q.size == 0 or cu_q[0] != 0 or cu_kv[0] != 0:
        raise ValueError("cumulative sequence lengths must start at zero")
    if cu_q[-1] > query.shape[1] or cu_kv[-1] > key.shape[1]:
        raise ValueError("cumulative sequence lengths exceed packed tensor size")
    if is_causal and causal_name not in {"BottomRight", "TopLeft", None}:
        q_lens, kv_lens = cu_q[1:] - cu_q[:-1], cu_kv[1:] - cu_kv[:-1]
        if ((q_lens > 0) & (kv_lens > 0) & (q_lens != kv_lens)).any():
            raise ValueError(f"causal type {causal_name!r} requires equal query and KV lengths")
    if cu_q.size <= 1 or math.prod(out_shape) == 0:
        # still reject decreasing offsets, as the planner does
        if cu_q.size > 1 and ((cu_q[1:] < cu_q[:-1]).any() or (cu_kv[1:] < cu_kv[:-1]).any()):
            raise ValueError("cumulative sequence lengths must be nondecreasing")
        return output.zero_()

    nseq = cu_q.size - 1
    if fused:
        # one library call plans the work list and tile order into the pinned buffer, zeroes the
        # rows no sequence writes, uploads the list and launches the fused kernel
        with _VarlenStaging._lock:
            st = _VarlenStaging.get(output.device, stream, _varlen_words(nseq, int(cu_q[-1]), True))
            rc = _fast_fn("biops_varlen_sdpa_fused_planned")(
                nat.dtype_code(query.dtype), heads, kv_heads, head_dim, value_dim,
                q.data_ptr(), q.stride(1), q.stride(2),
                k.data_ptr(), k.stride(1), k.stride(2),
                v.data_ptr(), v.stride(1), v.stride(2),
                output.data_ptr(), output.stride(1), output.stride(2), query.shape[1], key.shape[1],
                nseq, cu_q.ctypes.data, cu_kv.ctypes.data, st.host.data_ptr(), st.view.size,
                st.dev.data_ptr(), causal, scale_value, stream,
            )
            st.event.record()
        if rc == nat.ERR_ARG:
            raise ValueError(nat.last_error())
        nat.check(rc, "biops_varlen_sdpa_fused_planned")
        return output
    # materialised path: plan (validates the offsets, drops empty sequences), zero the output
    # (rows outside the sequences and of sequences without keys stay zero), upload, launch
    with _VarlenStaging._lock:
        st = _VarlenStaging.get(output.device, stream, _varlen_words(nseq, int(cu_q[-1]), False))
        words, ws_bytes = _varlen_plan(cu_q, cu_kv, heads, value_dim, query.dtype, st.view)
        plan = st.view
        if plan[0] == 0:
            return output.zero_()
        output.zero_()
        st.upload(words, stream)
        workspace = torch.empty(max(int(ws_bytes), 16), dtype=torch.uint8, device=query.device)
        nat.call(
            "biops_varlen_sdpa",
            nat.dtype_code(query.dtype), heads, kv_heads, head_dim, value_dim,
            q.data_ptr(), q.stride(1), q.stride(2),
            k.data_ptr(), k.stride(1), k.stride(2),
            v.data_ptr(), v.stride(1), v.stride(2),
            output.data_ptr(), output.stride(1), output.stride(2),
            st.dev.data_ptr(), plan.ctypes.data, causal, scale_value,
            workspace.data_ptr(), workspace.numel(),
            stream,
        )
        return output


# ---------------------------------------------------------------- convolutions ----
def _conv_sizes(values, n, name):
    values = tuple(int(v) for v in values)
    if len(values) == 1 and n > 1:
        return values * n
    assert len(values) == n, f"{name} must have one or {n} values, got {values!r}"
    return values


def _conv_native(input, weight, bias, nd, transposed, stride, padding, dilation, groups, out_channels,
                 out_spatial):
    """One biops_conv call: output [B, out_channels, *out_spatial], fresh and contiguous."""
    out = torch.empty((input.shape[0], out_channels, *out_spatial), dtype=input.dtype, device=input.device)
    if out.numel() == 0:
        return out
    nat.require_gpu_tensors(input, weight, *(() if bias is None else (bias,)))
    x = input
    if transposed and not x[0, 0].is_contiguous():
        x = x.contiguous()  # the GEMM reads the spatial dims as one contiguous run
    w = weight.contiguous()
    b = None if bias is None else bias.contiguous()

    def arr(values):
        return (ctypes.c_int64 * len(values))(*[int(v) for v in values])

    in_size, ksize = arr(input.shape[2:]), arr(weight.shape[2:])
    st, pd, dl, xs = arr(stride), arr(padding), arr(dilation), arr(x.stride())
    code = nat.dtype_code(input.dtype)
    sizes = (code, nd, int(transposed), input.shape[0], input.shape[1], ctypes.addressof(in_size), out_channels,
             ctypes.addressof(ksize), ctypes.addressof(st), ctypes.addressof(pd), ctypes.addressof(dl), groups)
    ws_bytes = int(nat.load().biops_conv_workspace_size(*sizes))
    if ws_bytes < 0:
        raise RuntimeError("biops_conv_workspace_size rejected the convolution sizes")
    workspace = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=input.device)
    nat.call(
        "biops_conv", *sizes,
        x.data_ptr(), ctypes.addressof(xs), w.data_ptr(), 0 if b is None else b.data_ptr(),
        out.data_ptr(), workspace.data_ptr(), workspace.numel(), nat.stream_of(out),
    )
    return out


def _regular_conv(nd, input, weight, bias, stride, padding, dilation, transposed, output_padding, groups):
    """Shared argument rules of the regular 1-D / 2-D / 3-D convolutions (batch_invariant_ops.py
    :505-514, 609-618, 695-704)."""
    names = {1: "1-D", 2: "2-D", 3: "3-D"}
    assert input.ndim == nd + 2 and weight.ndim == nd + 2, f"only {names[nd]} convolution is supported"
    assert not transposed, "transposed convolution is not supported"
    assert all(value == 0 for value in output_padding), (
        f"output_padding requires transposed convolution, got {output_padding!r}"
    )
    assert input.dtype == weight.dtype and (bias is None or bias.dtype == input.dtype), "Incompatible dtypes"
    assert input.shape[1] == weight.shape[1] * groups, "Incompatible channel dimensions"
    assert weight.shape[0] % groups == 0, "output channels must be divisible by groups"
    if nd == 1:
        stride, padding, dilation = (tuple(stride), tuple(padding), tuple(dilation))
        for values, name in ((stride, "stride"), (padding, "padding"), (dilation, "dilation")):
            assert len(values) == 1, f"{name} must have one value, got {values!r}"
    stride = _conv_sizes(stride, nd, "stride")
    padding = _conv_sizes(padding, nd, "padding")
    dilation = _conv_sizes(dilation, nd, "dilation")
    kernel = weight.shape[2:]
    out_spatial = tuple(
        (input.shape[2 + i] + 2 * padding[i] - dilation[i] * (kernel[i] - 1) - 1) // stride[i] + 1
        for i in range(nd)
    )
    return _conv_native(input, weight, bias, nd, False, stride, padding, dilation, groups, weight.shape[0],
                        out_spatial)


def conv1d_batch_invariant(input, weight, bias, stride, padding, dilation, transposed, output_padding, groups):
    """Batch-invariant 1-D convolution (reference conv1d_batch_invariant, batch_invariant_ops.py
    :497-595).  Depthwise (groups == C_in == C_out, one channel per group, 531): fp32 sum over the
    taps in order plus the bias, one rounding, like the reference's dedicated kernel (434-494).
    Every other group layout: one fixed-schedule GEMM dot product over (channel, tap) per output,
    rounded, then the bias added and rounded (the reference's bmm + add, 565-595)."""
    return _regular_conv(1, input, weight, bias, stride, padding, dilation, transposed, output_padding, groups)


def conv2d_batch_invariant(input, weight, bias, stride, padding, dilation, transposed, output_padding, groups):
    """Batch-invariant 2-D convolution (reference conv2d_batch_invariant, batch_invariant_ops.py
    :598-682): per-output GEMM dot products over (channel, kh, kw) of the group (im2col), grouped
    and dilated convolution included, bias added after the GEMM rounding."""
    return _regular_conv(2, input, weight, bias, stride, padding, dilation, transposed, output_padding, groups)


def conv3d_batch_invariant(input, weight, bias, stride, padding, dilation, transposed, output_padding, groups):
    """Batch-invariant 3-D convolution (reference conv3d_batch_invariant, batch_invariant_ops.py
    :685-780), as conv2d with (kd, kh, kw) taps."""
    return _regular_conv(3, input, weight, bias, stride, padding, dilation, transposed, output_padding, groups)


def _transposed_conv(nd, input, weight, bias, stride, padding, dilation, output_padding, groups):
    """Non-overlapping transposed convolution (reference 783-941): stride == kernel, no padding,
    output padding or dilation, so every output position receives one contribution."""
    names = {2: "2-D", 3: "3-D"}
    assert input.ndim == nd + 2 and weight.ndim == nd + 2, f"only {names[nd]} convolution is supported"
    assert input.dtype == weight.dtype and (bias is None or bias.dtype == input.dtype), "Incompatible dtypes"
    assert input.shape[1] == weight.shape[0], "Incompatible input channels"
    assert input.shape[1] % groups == 0, "input channels must be divisible by groups"
    stride = _conv_sizes(stride, nd, "stride")
    padding = _conv_sizes(padding, nd, "padding")
    dilation = _conv_sizes(dilation, nd, "dilation")
    output_padding = _conv_sizes(output_padding, nd, "output_padding")
    kernel = tuple(weight.shape[2:])
    label = "ConvTranspose2d" if nd == 2 else "ConvTranspose3d"
    assert stride == kernel, (
        f"batch-invariant {label} currently requires non-overlapping "
        f"stride == kernel_size, got stride={stride}, kernel_size={kernel}"
    )
    zeros = (0,) * nd
    assert padding == zeros, f"padding is not supported, got {padding}"
    assert output_padding == zeros, f"output_padding is not supported, got {output_padding}"
    assert dilation == (1,) * nd, f"dilation is not supported, got {dilation}"
    out_channels = weight.shape[1] * groups
    if bias is not None:
        assert bias.shape == (out_channels,), "Incompatible bias shape"
    out_spatial = tuple(input.shape[2 + i] * kernel[i] for i in range(nd))
    return _conv_native(input, weight, bias, nd, True, stride, padding, dilation, groups, out_channels,
                        out_spatial)


def conv_transpose2d_batch_invariant(input, weight, bias, stride, padding, dilation, output_padding, groups):
    """Batch-invariant non-overlapping 2-D transposed convolution (reference
    conv_transpose2d_batch_invariant, batch_invariant_ops.py:783-861): one GEMM dot product over
    the group's input channels per output element, rounded, then the bias added and rounded."""
    return _transposed_conv(2, input, weight, bias, stride, padding, dilation, output_padding, groups)


def conv_transpose3d_batch_invariant(input, weight, bias, stride, padding, dilation, output_padding, groups):
    """Batch-invariant non-overlapping 3-D transposed convolution (reference
    conv_transpose3d_batch_invariant, batch_invariant_ops.py:864-941)."""
    return _transposed_conv(3, input, weight, bias, stride, padding, dilation, output_padding, groups)


def convolution_batch_invariant(input, weight, bias, stride, padding, dilation, transposed, output_padding,
                                groups):
    """aten::convolution dispatch to the supported forms (batch_invariant_ops.py:944-971)."""
    if input.ndim == 3 and weight.ndim == 3:
        return conv1d_batch_invariant(input, weight, bias, stride, padding, dilation, transposed,
                                      output_padding, groups)
    if input.ndim == 4 and weight.ndim == 4 and transposed:
        return conv_transpose2d_batch_invariant(input, weight, bias, stride, padding, dilation,
                                                output_padding, groups)
    if input.ndim == 4 and weight.ndim == 4:
        return conv2d_batch_invariant(input, weight, bias, stride, padding, dilation, transposed,
                                      output_padding, groups)
    if input.ndim == 5 and weight.ndim == 5 and transposed:
        return conv_transpose3d_batch_invariant(input, weight, bias, stride, padding, dilation,
                                                output_padding, groups)
    if input.ndim == 5 and weight.ndim == 5:
        return conv3d_batch_invariant(input, weight, bias, stride, padding, dilation, transposed,
                                      output_padding, groups)
    raise AssertionError(
        f"only 1-D, 2-D and 3-D convolution are supported, got input rank {input.ndim} "
        f"and weight rank {weight.ndim}"
    )


# ------------------------------------------------------------ mode / registration ----
_batch_invariant_MODE = False
_batch_invariant_LIB = None

# ROCm PyTorch exposes its GPUs as device type "cuda": the overrides go on dispatch key CUDA.
_DISPATCH_KEY = "CUDA"

_OVERRIDES = (
    ("aten::mm", mm_batch_invariant),
    ("aten::addmm", addmm_batch_invariant),
    ("aten::linear", linear_batch_invariant),
    ("aten::bmm", bmm_batch_invariant),
    ("aten::convolution", convolution_batch_invariant),
    ("aten::scaled_dot_product_attention", scaled_dot_product_attention_batch_invariant),
    ("aten::_softmax", _softmax_batch_invariant),
    ("aten::_log_softmax", _log_softmax_batch_invariant),
    ("aten::mean.dim", mean_batch_invariant),
    ("aten::linalg_vector_norm", linalg_vector_norm_batch_invariant),
)


def is_batch_invariant_mode_enabled():
    return _batch_invariant_MODE


def enable_batch_invariant_mode():
    """Register the overrides (batch_invariant_ops.py:1662-1684) on dispatch key CUDA."""
    global _batch_invariant_MODE, _batch_invariant_LIB
    if _batch_invariant_MODE:
        return
    lib = torch.library.Library("aten", "IMPL")
    for op, fn in _OVERRIDES:
        lib.impl(op, fn, _DISPATCH_KEY)
    _batch_invariant_LIB = lib
    _batch_invariant_MODE = True


def disable_batch_invariant_mode():
    """Remove the overrides (batch_invariant_ops.py:1687-1692), restoring the stock kernels."""
    global _batch_invariant_MODE, _batch_invariant_LIB
    if _batch_invariant_LIB is not None:
        _batch_invariant_LIB._destroy()
    _batch_invariant_MODE = False
    _batch_invariant_LIB = None


@contextlib.contextmanager
def set_batch_invariant_mode(enabled: bool = True):
    """Context manager that enables (or disables) the overrides and restores the previous
    state on exit, also on exceptions; re-entrant (batch_invariant_ops.py:1695-1712)."""
    previously_enabled = is_batch_invariant_mode_enabled()
    if enabled == previously_enabled:
        yield
        return
    if enabled:
        enable_batch_invariant_mode()
    else:
        disable_batch_invariant_mode()
    try:
        yield
    finally:
        if previously_enabled:
            enable_batch_invariant_mode()
        else:
            disable_batch_invariant_mode()


AttentionBlockSize = namedtuple("AttentionBlockSize", ["block_m", "block_n"])


def get_batch_invariant_attention_block_size() -> AttentionBlockSize:
    """Attention block size advertised to serving engines (batch_invariant_ops.py:1715-1719)."""
    return AttentionBlockSize(block_m=16, block_n=16)
