"""Deterministic token-choice mixture of experts on the library's fixed-schedule kernels."""

from __future__ import annotations

import threading
import time

import torch

from . import _native as nat

_INDEX_ERROR = "selected_experts contains an expert index outside [0, num_experts)"


class _IndexWatch:
    """Deferred report of out-of-range expert indices on one device, without a host wait.

    Every MoE call passes the device's flag word to the kernels, which set it to 1 when a
    token selects an expert outside [0, E) (and write that token's row as zeros); they never
    clear it.  At most one asynchronous copy of the flag into a pinned host word is in flight,
    started after a call when the last one has landed and ``PERIOD`` seconds have passed (none
    during stream capture).  The next call, or ``check_moe_indices``, reads a landed copy and
    raises ``RuntimeError`` if the flag was set, after clearing it."""

    PERIOD = 1e-3
    _by_device: dict = {}
    _lock = threading.Lock()

    def __init__(self, device: torch.device):
        self.flag = torch.zeros(1, dtype=torch.int32, device=device)
        self.host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self.event = torch.cuda.Event()
        self.pending = False
        self.last = 0.0
        self.copy = nat.fast_copy_d2h()

    @classmethod
    def of(cls, device: torch.device) -> "_IndexWatch":
        watch = cls._by_device.get(device.index)
        if watch is None:
            with cls._lock:
                watch = cls._by_device.setdefault(device.index, cls(device))
        return watch

    def _raise_if_set(self, value: int) -> None:
        if value != 0:
            self.host[0] = 0
            self.flag.zero_()
            raise RuntimeError(f"{_INDEX_ERROR} in a call since the last report")

    def poll(self) -> None:
        """Raise for a flag copy that has landed with the flag set."""
        if self.pending and self.event.query():
            self.pending = False
            self._raise_if_set(int(self.host[0]))

    def after_call(self, stream: int) -> None:
        """Start a flag copy on ``stream`` unless one is in flight, one started less than
        PERIOD seconds ago, or the stream is being captured."""
        if self.pending:
            return
        now = time.monotonic()
        if now - self.last < self.PERIOD or torch.cuda.is_current_stream_capturing():
            return
        self.last = now
        if self.copy is not None:
            rc = self.copy(self.host.data_ptr(), self.flag.data_ptr(), 4, stream)
            if rc != 0:
                raise RuntimeError(f"hipMemcpyAsync of the MoE index flag failed ({rc})")
        else:
            self.host.copy_(self.flag, non_blocking=True)
        self.event.record()
        self.pending = True

    def check(self) -> None:
        """Wait for the work queued so far on the current stream and raise if any of it (or an
        earlier call) saw an out-of-range index."""
        self.pending = False
        self._raise_if_set(int(self.flag.item()))


def check_moe_indices(device: torch.device | int | None = None) -> None:
    """Raise ``RuntimeError`` if a ``deterministic_token_choice_moe`` call on ``device``
    (default: the current device) met an expert index outside [0, num_experts) since the last
    report.  Waits for the work queued on that device's current stream."""
    if device is None:
        device = torch.device("cuda", torch.cuda.current_device())
    elif isinstance(device, int):
        device = torch.device("cuda", device)
    with torch.cuda.device(device):
        _IndexWatch.of(device).check()


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
    row is written as zeros, and the error is reported without a host wait in the call.  The
    kernels set a device flag, an asynchronous copy brings it to the host, and a later call
    (or ``check_moe_indices()``, which waits) raises ``RuntimeError`` once the copy has landed.
    With ``BIOPS_MOE_CHECK_INDICES=1`` each call waits for its kernels and raises at once.  The
    reference asserts on the device instead (moe.py:66-73), which ends the process's GPU
    context.
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
    watch = _IndexWatch.of(x.device)
    watch.poll()
    check = nat.env_flag("BIOPS_MOE_CHECK_INDICES", False)
    stream = nat.stream_of(out)
    nat.call(
        entry,
        code, token_count, num_experts, hidden_size, intermediate_size, top_k,
        x.data_ptr(), x.stride(0),
        gate.data_ptr(), *gate.stride(),
        up.data_ptr(), *up.stride(),
        down.data_ptr(), *down.stride(),
        weights.data_ptr(), w_code, selected.data_ptr(),
        out.data_ptr(), watch.flag.data_ptr(),
        scratch.data_ptr(), scratch.numel(),
        stream,
    )
    if check:
        watch.check()
    else:
        watch.after_call(stream)
    return out
