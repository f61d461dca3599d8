"""biops_moe_sparse_noalloc through the C ABI: the allocation-free variant of biops_moe_sparse
(its route tables and packed matrices live in a static device array of the library) must give
the existing entry point's bits on consecutive calls, the second one smaller, and must reject
sizes beyond its array with BIOPS_ERR_SIZE before any GPU work."""

from __future__ import annotations

import pytest
import torch

from batch_invariant_ops import _native as nat
from batch_invariant_ops.moe import _moe

from _tol import assert_bitwise

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def _experts(E, D, I, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    gate_up = (torch.randn(E, D, 2 * I, generator=g, device="cuda") * 0.02).to(BF16)
    down = (torch.randn(E, I, D, generator=g, device="cuda") * 0.02).to(BF16)
    # the reference's [E, I, D] gate / up and [E, D, I] down views of fused weights (gate first)
    return gate_up[..., :I].transpose(1, 2), gate_up[..., I:].transpose(1, 2), down.transpose(1, 2)


def _tokens(T, D, E, k, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    hidden = torch.randn(T, D, generator=g, device="cuda").to(BF16)
    logits = torch.randn(T, E, generator=g, device="cuda")
    weights, selected = torch.topk(torch.softmax(logits, -1), k, dim=-1)
    return hidden, weights, selected


def _noalloc(hidden, weights, selected, gate, up, down, bad=None):
    """One biops_moe_sparse_noalloc call; the output tensor is the caller's, as for any entry."""
    T, D = hidden.shape
    E, I, _ = gate.shape
    k = selected.shape[1]
    code = nat.dtype_code(hidden.dtype)
    w = weights.to(hidden.dtype).contiguous()
    sel = selected.to(torch.int64).contiguous()
    out = torch.empty(T, D, dtype=hidden.dtype, device=hidden.device)
    rc = nat.load().biops_moe_sparse_noalloc(
        code, T, E, D, I, k,
        hidden.data_ptr(), hidden.stride(0),
        gate.data_ptr(), *gate.stride(),
        up.data_ptr(), *up.stride(),
        down.data_ptr(), *down.stride(),
        w.data_ptr(), code, sel.data_ptr(),
        out.data_ptr(), None if bad is None else bad.data_ptr(),
        nat.stream_of(out),
    )
    nat.check(rc, "biops_moe_sparse_noalloc")
    return out


@pytest.mark.parametrize("shape", ((64, 2048, 768, 8), (9, 96, 40, 3)), ids=("c5", "small"))
def test_noalloc_equals_workspace_entry_on_consecutive_calls(shape):
    """Two calls in a row on the shared array, the second with fewer tokens (and a third, larger
    again): each output has the bits of biops_moe_sparse with a torch-allocated workspace."""
    E, D, I, k = shape
    gate, up, down = _experts(E, D, I, seed=9100 + D)
    for step, T in enumerate((1024, 37, 300)):
        hidden, weights, selected = _tokens(T, D, E, k, seed=9200 + 10 * step + D)
        print(f"[no-alloc] E={E} D={D} I={I} k={k} call {step}: T={T}", flush=True)
        got = _noalloc(hidden, weights, selected, gate, up, down)
        want = _moe(hidden, weights, selected, gate, up, down, sparse=True)
        assert_bitwise(got, want, f"call {step} T={T}")


def test_noalloc_flags_invalid_indices_and_zeroes_their_rows():
    E, D, I, k = 5, 64, 32, 2
    gate, up, down = _experts(E, D, I, seed=9300)
    hidden, weights, selected = _tokens(12, D, E, k, seed=9301)
    selected = selected.clone()
    selected[4, 1] = E
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = _noalloc(hidden, weights, selected, gate, up, down, bad=bad)
    assert int(bad.item()) == 1
    assert torch.count_nonzero(got[4]) == 0 and torch.count_nonzero(got[3]) > 0


def test_noalloc_rejects_sizes_beyond_its_array():
    """4096 C5 tokens need about 184 MB of scratch: BIOPS_ERR_SIZE, nothing launched, and the
    next call still works."""
    lib = nat.load()
    rc = lib.biops_moe_sparse_noalloc(
        nat.BF16, 4096, 64, 2048, 768, 8, None, 2048, None, 1, 2048, 1, None, 1, 2048, 1,
        None, 1, 1, 2048, None, nat.BF16, None, None, None, None)
    assert rc == 5
    assert "scratch" in lib.biops_last_error().decode()
    gate, up, down = _experts(4, 32, 16, seed=9400)
    hidden, weights, selected = _tokens(3, 32, 4, 2, seed=9401)
    assert_bitwise(_noalloc(hidden, weights, selected, gate, up, down),
                   _moe(hidden, weights, selected, gate, up, down, sparse=True), "after a rejected call")


def test_noalloc_captured_in_a_graph_replays_new_routing():
    """The entry's callers include code under stream capture: one call captured in a HIP graph
    (through torch.cuda.graph) with preallocated inputs and output, replayed three times with
    new hidden states and routing written into the captured inputs, eager work and a
    synchronisation between the replays; every replay gives biops_moe_sparse's bits (the array's
    tables are all rewritten by each replay)."""
    E, D, I, k, T = 16, 256, 128, 4, 200
    gate, up, down = _experts(E, D, I, seed=9500)
    hidden, weights, selected = _tokens(T, D, E, k, seed=9501)
    x = hidden.clone()
    w = weights.to(BF16).contiguous()
    sel = selected.to(torch.int64).contiguous()
    out = torch.empty(T, D, dtype=BF16, device="cuda")
    lib = nat.load()

    def call():
        return lib.biops_moe_sparse_noalloc(
            nat.BF16, T, E, D, I, k, x.data_ptr(), x.stride(0),
            gate.data_ptr(), *gate.stride(), up.data_ptr(), *up.stride(), down.data_ptr(), *down.stride(),
            w.data_ptr(), nat.BF16, sel.data_ptr(), out.data_ptr(), None, nat.stream_of(out))

    nat.check(call(), "eager warm-up")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = call()
    nat.check(rc, "captured call")
    for rep in range(3):
        h2, w2, s2 = _tokens(T, D, E, k, seed=9510 + rep)
        x.copy_(h2)
        w.copy_(w2.to(BF16))
        sel.copy_(s2)
        print(f"[no-alloc] graph replay {rep}", flush=True)
        graph.replay()
        want = _moe(h2, w2.to(BF16), s2, gate, up, down, sparse=True)  # eager work between replays
        torch.cuda.synchronize()
        assert_bitwise(out, want, f"replay {rep}")
