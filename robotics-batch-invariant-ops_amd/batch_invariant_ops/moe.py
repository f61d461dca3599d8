"""Deterministic token-choice mixture of experts on the library's fixed-schedule kernels."""

from __future__ import annotations

import torch

from . import _native as nat


def _unit_stride_weight(w: torch.Tensor) -> torch.Tensor:
    """[E, rows, K] expert weight with a unit stride in its rows or in K."""
    return w if w.stride(1) == 1 or w.stride(2) == 1 else w.contiguous()


def deterministic_token_choice_moe(
    hidden_states: torch.Tensor,
    routing_weights: torch.Tensor,
    selected_experts: torch.Tensor,
    gate_weight: torch.Tensor,
    up_weight: torch.Tensor,
    down_weight: torch.Tensor,
    workspace: dict[str, torch.Tensor] | None = None,
) -> torch.Tensor:
    """Top-k SwiGLU MoE without atomic routing or accumulation.

    Reference: deterministic_token_choice_moe (moe.py:11-92).  ``gate_weight`` and
    ``up_weight`` have shape ``(E, I, D)`` and ``down_weight`` ``(E, D, I)``.  Each selected
    route (token t, slot s) is computed with fixed-schedule GEMMs (gate and up in one launch
    with the SwiGLU epilogue ``round(round(silu(round(g))) * round(u))``, then the down
    projection), weighted by ``round(routing_weight)`` and summed over the top-k slots left to
    right with a rounding after every add.  ``workspace`` is accepted for drop-in
    compatibility and ignored, as in the reference.

    By default only the selected routes are evaluated: they are packed by expert (ranks from
    wavefront ballots, no atomics) and each expert multiplies its own rows.  Every GEMM row is
    computed by the same fixed instruction sequence whatever the other rows are, so the result
    has the bits of the reference's every-expert evaluation, which ``BIOPS_MOE_DENSE=1``
    selects (also used above 2048 experts).

    Expert indices outside ``[0, E)`` never make a kernel read out of range: the token's output
    row is written as zeros.  The call does not wait for the GPU to report them (a host read
    would synchronise every call, and would fail under stream capture).  With
    ``BIOPS_MOE_CHECK_INDICES=1`` the call waits for the kernels and raises ``RuntimeError``
    when an index was out of range.  The reference asserts on the device instead
    (moe.py:66-73), which ends the process's GPU context.
    """
    del workspace
    return _moe(hidden_states, routing_weights, selected_experts, gate_weight, up_weight, down_weight,
                sparse=not nat.env_flag("BIOPS_MOE_DENSE", False))


def _moe(
    hidden_states: torch.Tensor,
    routing_weights: torch.Tensor,
    selected_experts: torch.Tensor,
    gate_weight: torch.Tensor,
    up_weight: torch.Tensor,
    down_weight: torch.Tensor,
    sparse: bool,
) -> torch.Tensor:
    """deterministic_token_choice_moe with the evaluation chosen explicitly."""
    if hidden_states.ndim != 2:
        raise ValueError(f"hidden_states must have shape (tokens, hidden), got {hidden_states.shape}")
    if routing_weights.ndim != 2 or selected_experts.shape != routing_weights.shape:
        raise ValueError("routing_weights and selected_experts must have the same (tokens, top_k) shape")
    if routing_weights.shape[0] != hidden_states.shape[0]:
        raise ValueError("routing tensors and hidden_states have different token counts")
    if gate_weight.ndim != 3 or up_weight.shape != gate_weight.shape:
        raise ValueError("gate_weight and up_weight must have the same (experts, intermediate, hidden) shape")
    num_experts, intermediate_size, hidden_size = gate_weight.shape
    if hidden_states.shape[1] != hidden_size:
        raise ValueError("hidden_states and expert weights have incompatible hidden dimensions")
    if down_weight.shape != (num_experts, hidden_size, intermediate_size):
        raise ValueError("down_weight must have shape (experts, hidden, intermediate)")
    token_count, top_k = selected_experts.shape
    if token_count == 0:
        return hidden_states.new_empty((0, hidden_size))
    if top_k == 0:
        return hidden_states.new_zeros((token_count, hidden_size))
    dtype = hidden_states.dtype
    if gate_weight.dtype != dtype or up_weight.dtype != dtype or down_weight.dtype != dtype:
        raise ValueError("hidden_states and expert weights must share one dtype")
    nat.require_gpu_tensors(hidden_states, routing_weights, selected_experts, gate_weight, up_weight, down_weight)
    code = nat.dtype_code(dtype)

    x = hidden_states if hidden_states.stride(1) == 1 else hidden_states.contiguous()
    gate = _unit_stride_weight(gate_weight)
    up = _unit_stride_weight(up_weight)
    if gate.stride() != up.stride():
        gate, up = gate.contiguous(), up.contiguous()
    down = _unit_stride_weight(down_weight)
    # The kernels round each routing weight to the activation dtype before the multiply (the
    # reference's routing_weights.to(dtype), moe.py:87), so float weights go in as they are.
    w_code = nat.DIRECT_DTYPES.get(routing_weights.dtype)
    if w_code is None:
        weights, w_code = routing_weights.to(dtype).contiguous(), code
    else:
        weights = routing_weights.contiguous()
    selected = selected_experts.to(torch.int64).contiguous()

    out = torch.empty((token_count, hidden_size), dtype=dtype, device=x.device)
    lib = nat.load()
    ws_bytes = -1
    if sparse:
        ws_bytes = lib.biops_moe_sparse_workspace_size(
            code, token_count, top_k, num_experts, hidden_size, intermediate_size)
    entry = "biops_moe_sparse" if ws_bytes >= 0 else "biops_moe"
    if ws_bytes < 0:
        ws_bytes = lib.biops_moe_workspace_size(code, token_count, num_experts, hidden_size, intermediate_size)
    # torch's caching allocator returns 512-byte aligned blocks (the sparse path needs 256).
    scratch = torch.empty(max(int(ws_bytes), 16), dtype=torch.uint8, device=x.device)
    check = nat.env_flag("BIOPS_MOE_CHECK_INDICES", False)
    bad = torch.zeros(1, dtype=torch.int32, device=x.device) if check else None
    nat.call(
        entry,
        code, token_count, num_experts, hidden_size, intermediate_size, top_k,
        x.data_ptr(), x.stride(0),
        gate.data_ptr(), *gate.stride(),
        up.data_ptr(), *up.stride(),
        down.data_ptr(), *down.stride(),
        weights.data_ptr(), w_code, selected.data_ptr(),
        out.data_ptr(), bad.data_ptr() if check else None,
        scratch.data_ptr(), scratch.numel(),
        nat.stream_of(out),
    )
    if check and int(bad.item()) != 0:
        raise RuntimeError("selected_experts contains an expert index outside [0, num_experts)")
    return out
