"""Composite-op parity checks against the float64 oracle (attention and MoE).

Each check computes the oracle's output and its per-element magnitude (``oracle.sdpa_abs``,
``oracle.varlen_sdpa_abs``, ``oracle.moe_abs``) on the CPU copies of the GPU's inputs and
applies ``assert_composite_close``: a per-element error bound plus the share of elements that
must carry the oracle's exact bits.
"""

from __future__ import annotations

import torch

import oracle

from _tol import assert_composite_close


def _cpu(x):
    return x.cpu() if isinstance(x, torch.Tensor) else x


def check_sdpa(out, q, k, v, *, n=2, min_exact=None, what="", **kw):
    """``out`` = SDPA(q, k, v, **kw) on the GPU; ``kw`` as for ``oracle.sdpa``."""
    q, k, v = _cpu(q), _cpu(k), _cpu(v)
    kw = {key: _cpu(val) for key, val in kw.items()}
    ref = oracle.sdpa(q, k, v, **kw)
    assert_composite_close(out, ref, oracle.sdpa_abs(q, k, v, **kw), n=n, min_exact=min_exact, what=what)


def check_sdpa_against(out, other, q, k, v, *, n=2, min_exact=None, what="", **kw):
    """Two GPU evaluations (fused, materialised) of one SDPA, bounded with the oracle's scale."""
    q, k, v = _cpu(q), _cpu(k), _cpu(v)
    kw = {key: _cpu(val) for key, val in kw.items()}
    assert_composite_close(out, other, oracle.sdpa_abs(q, k, v, **kw), n=n, min_exact=min_exact, what=what)


def check_varlen(out, q, k, v, cu_q, cu_kv, *, n=2, min_exact=None, what="", **kw):
    q, k, v, cu_q, cu_kv = (_cpu(t) for t in (q, k, v, cu_q, cu_kv))
    ref = oracle.varlen_sdpa(q, k, v, cu_q, cu_kv, **kw)
    scale = oracle.varlen_sdpa_abs(q, k, v, cu_q, cu_kv, **kw)
    assert_composite_close(out, ref, scale, n=n, min_exact=min_exact, what=what)


def check_moe(out, hidden, weights, selected, gate, up, down, *, n=None, min_exact=None, what=""):
    """MoE output against the oracle.  n defaults to 2 + top_k: each weighted route and each
    partial slot sum can land one ulp away."""
    args = [_cpu(t) for t in (hidden, weights, selected, gate, up, down)]
    ref = oracle.moe(*args)
    if n is None:
        n = 2 + args[2].shape[1]
    assert_composite_close(out, ref, oracle.moe_abs(*args), n=n, min_exact=min_exact, what=what)
