"""ctypes binding of libbiops.so, the gfx950 HIP kernel library behind every operator.

The library is loaded on first use.  There is no fallback: if the shared object is missing or
no ROCm GPU is visible, the first kernel call raises ``RuntimeError`` naming the problem.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import threading

import torch  # loads torch's HIP runtime first, so libbiops.so binds to the same instance

_LIB_PATH = pathlib.Path(__file__).resolve().parent / "libbiops.so"

F32, F16, BF16, BOOL = 0, 1, 2, 3
REDUCE_MEAN, REDUCE_L2 = 0, 1
CAUSAL_NONE, CAUSAL_TOP_LEFT, CAUSAL_BOTTOM_RIGHT = 0, 1, 2

ERR_ARG = 1  # BIOPS_ERR_ARG
_STATUS = {
    1: "invalid argument",
    2: "unsupported layout",
    3: "unsupported dtype",
    4: "HIP runtime error",
    5: "workspace too small",
}

_DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16, torch.bool: BOOL}
# floating dtypes the GEMM / row kernels compute in
DIRECT_DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_i = ctypes.c_int
_l = ctypes.c_int64
_p = ctypes.c_void_p
_f = ctypes.c_float

_SIGNATURES = {
    "biops_version": (ctypes.c_char_p, []),
    "biops_last_error": (ctypes.c_char_p, []),
    "biops_compute_units": (_i, []),
    "biops_gemm": (_i, [_i, _l, _l, _l, _p, _l, _l, _p, _l, _l, _p, _p, _l, _l, _p]),
    "biops_bmm": (
        _i,
        [_i, _l, _l, _l, _l, _l, _p, _l, _l, _l, _l, _p, _l, _l, _l, _l, _l, _p, _l, _l, _l, _l, _p],
    ),
    "biops_pad_rows": (_i, [_i, _l, _l, _p, _l, _l, _l, _p, _p]),
    "biops_gemm_padded_workspace_size": (_l, [_i, _l, _l, _l, _l, _l]),
    "biops_gemm_padded": (_i, [_i, _l, _l, _l, _p, _l, _l, _p, _l, _l, _p, _p, _l, _l, _p, _l, _p]),
    "biops_bmm_padded_workspace_size": (_l, [_i, _l, _l, _l, _l, _l, _l, _l, _l]),
    "biops_bmm_padded": (_i, [_i, _l, _l, _l, _l, _p, _l, _l, _l, _p, _l, _l, _l, _p, _l, _l, _l, _p, _l, _p]),
    "biops_gemm_tile_count": (_i, []),
    "biops_set_gemm_tile": (_i, [_i]),
    "biops_softmax": (_i, [_i, _i, _l, _l, _p, _l, _p, _l, _i, _p]),
    "biops_reduce": (_i, [_i, _i, _i, _l, _l, _l, _p, _l, _l, _l, _p, _p]),
    "biops_sdpa_workspace_size": (_l, [_i, _l, _l, _l, _l]),
    "biops_sdpa": (
        _i,
        [_i, _l, _l, _l, _l, _l, _l, _l]
        + [_p, _l, _l, _l] * 3
        + [_p, _i, _l, _l, _l, _l, _i, _f, _p, _p, _l, _p],
    ),
    "biops_attention_fused_supported": (_i, [_i, _l, _l]),
    "biops_varlen_fused_supported": (_i, [_i, _l, _l]),
    "biops_attention_fused_mask_ok": (_i, [_p, _i, _l, _l, _l, _l, _l]),
    "biops_sdpa_fused": (
        _i,
        [_i, _l, _l, _l, _l, _l, _l, _l]
        + [_p, _l, _l, _l] * 3
        + [_p, _i, _l, _l, _l, _l, _i, _f, _p, _p],
    ),
    "biops_varlen_sdpa_fused": (
        _i,
        [_i, _l, _l, _l, _l] + [_p, _l, _l] * 4 + [_p, _p, _p, _i, _f, _p],
    ),
    "biops_varlen_fused_order": (_l, [_p, _i, _p]),
    "biops_varlen_sdpa_fused_planned": (
        _i,
        [_i, _l, _l, _l, _l] + [_p, _l, _l] * 4 + [_l, _l, _l, _p, _p, _p, _l, _p, _i, _f, _p],
    ),
    "biops_varlen_plan_len": (_l, [_l]),
    "biops_varlen_plan": (_l, [_l, _p, _p, _l, _l, _i, _p]),
    "biops_varlen_sdpa": (
        _i,
        [_i, _l, _l, _l, _l] + [_p, _l, _l] * 4 + [_p, _p, _i, _f, _p, _l, _p],
    ),
    "biops_moe_workspace_size": (_l, [_i, _l, _l, _l, _l]),
    "biops_moe": (
        _i,
        [_i, _l, _l, _l, _l, _l, _p, _l]
        + [_p, _l, _l, _l] * 3
        + [_p, _i, _p, _p, _p, _p, _l, _p],
    ),
    "biops_conv_workspace_size": (_l, [_i, _i, _i, _l, _l, _p, _l, _p, _p, _p, _p, _l]),
    "biops_conv": (_i, [_i, _i, _i, _l, _l, _p, _l, _p, _p, _p, _p, _l, _p, _p, _p, _p, _p, _p, _l, _p]),
    "biops_moe_sparse_workspace_size": (_l, [_i, _l, _l, _l, _l, _l]),
    "biops_moe_sparse": (
        _i,
        [_i, _l, _l, _l, _l, _l, _p, _l]
        + [_p, _l, _l, _l] * 3
        + [_p, _i, _p, _p, _p, _p, _l, _p],
    ),
    "biops_moe_sparse_noalloc": (
        _i,
        [_i, _l, _l, _l, _l, _l, _p, _l]
        + [_p, _l, _l, _l] * 3
        + [_p, _i, _p, _p, _p, _p],
    ),
}

# Bytes of the static device array behind biops_moe_sparse_noalloc (BIOPS_MOE_NOALLOC_SCRATCH_BYTES).
MOE_NOALLOC_SCRATCH_BYTES = 64 << 20

EXPORTED = tuple(_SIGNATURES)

_lib = None
_lock = threading.Lock()


def library_path() -> pathlib.Path:
    return _LIB_PATH


def load(require_gpu: bool = True) -> ctypes.CDLL:
    """Load libbiops.so (once).  With ``require_gpu`` also insist on a visible ROCm GPU."""
    global _lib
    if _lib is not None and (_gpu_seen or not require_gpu):
        return _lib
    if require_gpu and not torch.cuda.is_available():
        raise RuntimeError(
            "batch_invariant_ops needs a ROCm GPU: torch.cuda.is_available() is False"
        )
    if _lib is None:
        with _lock:
            if _lib is None:
                if not _LIB_PATH.exists():
                    raise RuntimeError(
                        f"{_LIB_PATH} is missing; build it with "
                        "`python robotics-batch-invariant-ops_amd/build_lib.py`"
                    )
                lib = ctypes.CDLL(str(_LIB_PATH))
                for name, (res, args) in _SIGNATURES.items():
                    fn = getattr(lib, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = lib
    if require_gpu:
        _set_gpu_seen()
    return _lib


_gpu_seen = False


def _set_gpu_seen() -> None:
    """The GPU check passed once; later loads skip it (devices do not disappear)."""
    global _gpu_seen
    _gpu_seen = True


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"batch_invariant_ops kernels do not support {dtype}") from None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(tensor: torch.Tensor) -> int:
    """Handle of torch's current stream on ``tensor``'s device (the launch stream)."""
    if _raw_stream is not None:
        return _raw_stream(tensor.get_device())
    return torch.cuda.current_stream(tensor.device).cuda_stream


def function(name: str):
    """The bound library entry point ``name`` (the library is loaded on first use)."""
    return getattr(load(), name)


# Entry points with a CPython fast-call binding (_biops_fast, built beside libbiops.so): the
# same C functions and arguments, without ctypes' per-argument conversions.
_FAST = {"biops_gemm": "gemm", "biops_gemm_padded": "gemm_padded", "biops_reduce": "reduce", "biops_softmax": "softmax",
         "biops_sdpa_fused": "sdpa_fused", "biops_varlen_plan": "varlen_plan", "biops_varlen_fused_order": "varlen_fused_order",
         "biops_varlen_sdpa_fused": "varlen_sdpa_fused",
         "biops_varlen_sdpa_fused_planned": "varlen_sdpa_fused_planned"}


def fast_function(name: str):
    """``name`` through the fast-call module when it is built, else the ctypes binding.  The
    library is loaded (and the GPU checked) first either way."""
    lib = load()
    alias = _FAST.get(name)
    if alias is not None:
        try:
            from . import _biops_fast
        except ImportError:
            return getattr(lib, name)
        return getattr(_biops_fast, alias)
    return getattr(lib, name)


def fast_copy_h2d():
    """``copy_h2d(dst, src, bytes, stream)`` (hipMemcpyAsync host to device, returns the HIP
    status) from the fast-call module, or None when the module is not built.  The library is
    loaded (and the GPU checked) first."""
    load()
    try:
        from . import _biops_fast
    except ImportError:
        return None
    return _biops_fast.copy_h2d


def fast_copy_d2h():
    """``copy_d2h(dst, src, bytes, stream)`` (hipMemcpyAsync device to host) from the fast-call
    module, or None when the module is not built."""
    load()
    try:
        from . import _biops_fast
    except ImportError:
        return None
    return _biops_fast.copy_d2h


def last_error() -> str:
    """The library's message for the calling thread's last failed call."""
    return load(require_gpu=False).biops_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = last_error()
        raise RuntimeError(f"{what} failed ({_STATUS.get(rc, rc)}): {msg}")


def call(name: str, *args) -> None:
    lib = load()
    check(getattr(lib, name)(*args), name)


def require_gpu_tensors(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError(
                f"batch_invariant_ops kernels run on ROCm GPU tensors, got device {t.device}"
            )


def lib_version() -> str:
    return load(require_gpu=False).biops_version().decode()


def env_flag(name: str, default: bool) -> bool:
    value = os.environ.get(name)
    if value is None:
        return default
    return value not in {"0", "false", "False", ""}
