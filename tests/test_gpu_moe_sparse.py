"""Sparse MoE evaluation (route packing + grouped GEMMs) against the dense every-expert path.

Every GEMM output row is computed by the same fixed instruction sequence whatever the other
rows of its launch are, so evaluating only the selected routes must reproduce the dense path's
bits exactly; the dense path itself is pinned to the oracle in test_gpu_moe.py.  The cases cover
the packing's corners: several route chunks (over 1024 routes), every route on one expert,
duplicate experts inside a token, empty experts, E = 1 and E not a power of two, out-of-range
indices, hidden sizes that are not a multiple of 8 (no 16-byte rows), N-major weights, every
tile entry of the grouped GEMM (the weight-streaming entries of few-token calls among them),
and both sides of the limits of the one-workgroup packing.
"""

import pytest
import torch

from batch_invariant_ops import _native as nat
from batch_invariant_ops.moe import _IndexWatch, _moe, check_moe_indices

from _parity import check_moe
from _tol import assert_bitwise

pytestmark = pytest.mark.gpu


def randn(*shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def weights_for(E, I, D, seed, dtype, scale=0.1):
    gate = randn(E, I, D, seed=seed, dtype=dtype, scale=scale)
    up = randn(E, I, D, seed=seed + 1, dtype=dtype, scale=scale)
    down = randn(E, D, I, seed=seed + 2, dtype=dtype, scale=scale)
    return gate.cuda(), up.cuda(), down.cuda()


@pytest.fixture
def quiet_index_watch(monkeypatch):
    """Out-of-range indices on purpose: no deferred report between the calls of one test (the
    test reads the flag itself at the end, with check_moe_indices)."""
    monkeypatch.setenv("BIOPS_MOE_CHECK_INDICES", "0")
    monkeypatch.setattr(_IndexWatch, "PERIOD", float("inf"))


def both(hidden, w, sel, gate, up, down):
    dense = _moe(hidden, w, sel, gate, up, down, sparse=False)
    sparse = _moe(hidden, w, sel, gate, up, down, sparse=True)
    return dense, sparse


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("T,E,D,I,k", [(37, 6, 64, 80, 3), (300, 64, 128, 96, 8), (5, 1, 32, 64, 2)])
def test_sparse_equals_dense(dtype, T, E, D, I, k):
    hidden = randn(T, D, seed=7600 + T, dtype=dtype).cuda()
    gate, up, down = weights_for(E, I, D, 7610 + E, dtype)
    g = torch.Generator().manual_seed(7620 + k)
    sel = torch.randint(0, E, (T, k), generator=g).cuda()  # duplicates inside a token allowed
    w = torch.rand(T, k, generator=g).cuda()
    dense, sparse = both(hidden, w, sel, gate, up, down)
    assert_bitwise(sparse, dense, f"sparse vs dense {dtype} T={T} E={E}")


def test_sparse_matches_oracle_bf16():
    T, E, D, I, k = 41, 9, 64, 48, 4
    hidden = randn(T, D, seed=7630, dtype=torch.bfloat16)
    gate = randn(E, I, D, seed=7631, dtype=torch.bfloat16, scale=0.2)
    up = randn(E, I, D, seed=7632, dtype=torch.bfloat16, scale=0.2)
    down = randn(E, D, I, seed=7633, dtype=torch.bfloat16, scale=0.2)
    g = torch.Generator().manual_seed(7634)
    sel = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    w = torch.rand(T, k, generator=g)
    out = _moe(*(t.cuda() for t in (hidden, w, sel, gate, up, down)), sparse=True)
    check_moe(out, hidden, w, sel, gate, up, down, what="sparse moe")


def test_sparse_skewed_routing():
    """All routes on one expert (3000 routes: three packing chunks), the others empty."""
    T, E, D, I, k = 1500, 16, 64, 64, 2
    hidden = randn(T, D, seed=7640, dtype=torch.bfloat16).cuda()
    gate, up, down = weights_for(E, I, D, 7641, torch.bfloat16)
    sel = torch.full((T, k), 11, dtype=torch.int64).cuda()
    w = torch.rand(T, k, generator=torch.Generator().manual_seed(7644)).cuda()
    dense, sparse = both(hidden, w, sel, gate, up, down)
    assert_bitwise(sparse, dense, "one expert")
    # half the routes on expert 0, the rest spread; chunk boundaries fall inside runs
    g = torch.Generator().manual_seed(7645)
    sel = torch.where(torch.rand(T, k, generator=g) < 0.5, torch.zeros(T, k, dtype=torch.int64),
                      torch.randint(0, E, (T, k), generator=g)).cuda()
    dense, sparse = both(hidden, w, sel, gate, up, down)
    assert_bitwise(sparse, dense, "half on expert 0")


def test_sparse_invalid_indices(quiet_index_watch, monkeypatch):
    """Out-of-range indices: those tokens give zeros on both paths, the others are computed."""
    T, E, D, I, k = 20, 5, 32, 32, 3
    hidden = randn(T, D, seed=7650, dtype=torch.bfloat16).cuda()
    gate, up, down = weights_for(E, I, D, 7651, torch.bfloat16)
    g = torch.Generator().manual_seed(7654)
    sel = torch.randint(0, E, (T, k), generator=g)
    sel[3, 1] = E
    sel[7, 0] = -1
    sel[19, 2] = 1 << 40
    sel = sel.cuda()
    w = torch.rand(T, k, generator=g).cuda()
    dense, sparse = both(hidden, w, sel, gate, up, down)
    assert_bitwise(sparse, dense, "invalid indices")
    assert torch.count_nonzero(sparse[[3, 7, 19]]) == 0
    with pytest.raises(RuntimeError, match="outside"):
        check_moe_indices()
    assert torch.count_nonzero(sparse[0]) > 0
    monkeypatch.setenv("BIOPS_MOE_CHECK_INDICES", "1")
    with pytest.raises(RuntimeError, match="outside"):
        _moe(hidden, w, sel, gate, up, down, sparse=True)


@pytest.mark.parametrize("D,I", [(36, 20), (30, 64), (64, 14)])
def test_sparse_unaligned_sizes(D, I):
    """Rows that are not whole 16-byte chunks: element-wise gather and the register-staged GEMM."""
    T, E, k = 23, 5, 2
    hidden = randn(T, D, seed=7660 + D, dtype=torch.bfloat16).cuda()
    gate, up, down = weights_for(E, I, D, 7661 + I, torch.bfloat16)
    g = torch.Generator().manual_seed(7662)
    sel = torch.randint(0, E, (T, k), generator=g).cuda()
    w = torch.rand(T, k, generator=g).cuda()
    dense, sparse = both(hidden, w, sel, gate, up, down)
    assert_bitwise(sparse, dense, f"D={D} I={I}")


def test_sparse_strided_weights_and_hidden():
    """Fused [E, D, 2I] gate/up halves and [E, I, D] down (N-major), hidden with a row pitch."""
    T, E, D, I, k = 33, 6, 64, 48, 3
    base = randn(T, D + 16, seed=7670, dtype=torch.bfloat16).cuda()
    hidden = base[:, 8:8 + D]
    gu = randn(E, D, 2 * I, seed=7671, dtype=torch.bfloat16, scale=0.1).cuda()
    dn = randn(E, I, D, seed=7672, dtype=torch.bfloat16, scale=0.1).cuda()
    gate, up, down = gu[..., :I].transpose(1, 2), gu[..., I:].transpose(1, 2), dn.transpose(1, 2)
    g = torch.Generator().manual_seed(7673)
    sel = torch.randint(0, E, (T, k), generator=g).cuda()
    w = torch.rand(T, k, generator=g).cuda()
    dense, sparse = both(hidden, w, sel, gate, up, down)
    assert_bitwise(sparse, dense, "strided operands")


def test_sparse_every_tile_entry():
    """Forcing each GEMM tile entry changes only the grouped launch's schedule."""
    T, E, D, I, k = 70, 8, 128, 128, 4
    hidden = randn(T, D, seed=7680, dtype=torch.bfloat16).cuda()
    gate, up, down = weights_for(E, I, D, 7681, torch.bfloat16)
    g = torch.Generator().manual_seed(7684)
    sel = torch.randint(0, E, (T, k), generator=g).cuda()
    w = torch.rand(T, k, generator=g).cuda()
    lib = nat.load()
    dense = _moe(hidden, w, sel, gate, up, down, sparse=False)
    try:
        for cfg in range(lib.biops_gemm_tile_count()):
            lib.biops_set_gemm_tile(cfg)
            sparse = _moe(hidden, w, sel, gate, up, down, sparse=True)
            assert_bitwise(sparse, dense, f"tile entry {cfg}")
    finally:
        lib.biops_set_gemm_tile(-1)


def test_sparse_c5_shape_batch_invariant():
    """C5 shapes (D 2048, E 64, top-8, I 768, fused weights): sparse == dense and B=1 == B=N."""
    E, D, I, k, T = 64, 2048, 768, 8, 512
    dt = torch.bfloat16
    gu = randn(E, D, 2 * I, seed=7690, dtype=dt, scale=0.02).cuda()
    dn = randn(E, I, D, seed=7691, dtype=dt, scale=0.02).cuda()
    gate, up, down = gu[..., :I].transpose(1, 2), gu[..., I:].transpose(1, 2), dn.transpose(1, 2)
    hidden = randn(T, D, seed=7692, dtype=dt).cuda()
    logits = randn(T, E, seed=7693).cuda()
    w, sel = torch.softmax(logits, dim=-1).topk(k, dim=-1)
    dense, sparse = both(hidden, w, sel, gate, up, down)
    assert_bitwise(sparse, dense, "C5 T=512")
    one = _moe(hidden[:1], w[:1], sel[:1], gate, up, down, sparse=True)
    assert_bitwise(one, sparse[:1], "token 0 alone")
    mid = _moe(hidden[100:356], w[100:356], sel[100:356], gate, up, down, sparse=True)
    assert_bitwise(mid, sparse[100:356], "tokens 100..355")


def nmajor_weights(E, I, D, seed, dtype, scale=0.1):
    """Fused [E, D, 2I] gate/up and [E, I, D] down storage (the reference MoE's layout): the
    gate / up / down views are N-major, the layout of the weight-streaming entries."""
    gu = randn(E, D, 2 * I, seed=seed, dtype=dtype, scale=scale).cuda()
    dn = randn(E, I, D, seed=seed + 1, dtype=dtype, scale=scale).cuda()
    return gu[..., :I].transpose(1, 2), gu[..., I:].transpose(1, 2), dn.transpose(1, 2)


# GEMM tile entries 20-22: the weight-streaming tile with 16- / 32- / 64-row m-tiles (biops.h).
STREAM_ENTRIES = (20, 21, 22)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("T,E,D,I,k", [
    (5, 4, 192, 72, 2),    # gate/up K = 192 (last stage of one 64-element step), N = 72 (partial block)
    (6, 5, 64, 192, 3),    # gate/up K = 64; down K = 192, N = 64
    (40, 3, 128, 64, 2),   # about 27 rows per expert: two 16-row m-tiles per group
    (1, 64, 256, 136, 8),  # one token on eight experts
])
def test_stream_entries_equal_dense(dtype, T, E, D, I, k):
    """The weight-streaming entries (automatic for few rows per expert, and forced) give the
    dense path's bits on N-major weights, across partial column blocks, K tails and groups
    taller than one m-tile."""
    hidden = randn(T, D, seed=7700 + T, dtype=dtype).cuda()
    gate, up, down = nmajor_weights(E, I, D, 7710 + E, dtype)
    g = torch.Generator().manual_seed(7720 + T)
    sel = torch.randint(0, E, (T, k), generator=g).cuda()
    w = torch.rand(T, k, generator=g).cuda()
    lib = nat.load()
    dense = _moe(hidden, w, sel, gate, up, down, sparse=False)
    try:
        for cfg in (-1,) + STREAM_ENTRIES:
            assert lib.biops_set_gemm_tile(cfg) == 0
            sparse = _moe(hidden, w, sel, gate, up, down, sparse=True)
            assert_bitwise(sparse, dense, f"tile entry {cfg}")
    finally:
        lib.biops_set_gemm_tile(-1)


@pytest.mark.parametrize("T,E,k", [(1, 64, 8), (128, 64, 8), (129, 64, 8), (200, 64, 8), (256, 64, 8), (512, 64, 8),
                                   (513, 64, 8), (300, 127, 8), (300, 128, 8), (4096, 64, 8), (3, 511, 4), (3, 512, 4)])
def test_one_workgroup_packing_limits(quiet_index_watch, T, E, k):
    """Up to 1024 routes and 511 experts the routes are packed by one workgroup in one pass, up
    to 4096 routes and 127 experts in two or four passes, beyond by the rank / plan / route-row
    kernels: both sides of each limit give the dense path's bits, with an out-of-range index
    among the routes."""
    D, I = 64, 64
    hidden = randn(T, D, seed=7740 + T, dtype=torch.bfloat16).cuda()
    gate, up, down = nmajor_weights(E, I, D, 7741, torch.bfloat16)
    g = torch.Generator().manual_seed(7742 + E)
    sel = torch.randint(0, E, (T, k), generator=g)
    if T > 1:
        sel[T - 1, k - 1] = E
    sel = sel.cuda()
    w = torch.rand(T, k, generator=g).cuda()
    dense, sparse = both(hidden, w, sel, gate, up, down)
    assert_bitwise(sparse, dense, f"T={T} E={E}")
    if T > 1:
        assert torch.count_nonzero(sparse[T - 1]) == 0
        with pytest.raises(RuntimeError, match="outside"):
            check_moe_indices()
    else:
        check_moe_indices()
    assert torch.count_nonzero(sparse[0]) > 0


@pytest.mark.parametrize("cfg", (-1, 0, 2))
def test_tail_m_tiles_equal_dense(cfg):
    """Groups of two m-tiles or more (here 530 / 600 / 520 / 700 rows on N-major weights): an
    expert's last m-tile of fewer than 64 rows runs as a separate launch on the
    weight-streaming tile, with the dense path's bits (256- and 128-row main tiles)."""
    sizes = (530, 600, 520, 700)
    E, D, I = len(sizes), 128, 128
    T = sum(sizes)
    sel = torch.cat([torch.full((n,), e, dtype=torch.int64) for e, n in enumerate(sizes)])
    sel = sel[torch.randperm(T, generator=torch.Generator().manual_seed(7760))].reshape(T, 1).cuda()
    w = torch.rand(T, 1, generator=torch.Generator().manual_seed(7761)).cuda()
    hidden = randn(T, D, seed=7762, dtype=torch.bfloat16).cuda()
    gate, up, down = nmajor_weights(E, I, D, 7763, torch.bfloat16)
    lib = nat.load()
    dense = _moe(hidden, w, sel, gate, up, down, sparse=False)
    try:
        assert lib.biops_set_gemm_tile(cfg) == 0
        sparse = _moe(hidden, w, sel, gate, up, down, sparse=True)
    finally:
        lib.biops_set_gemm_tile(-1)
    assert_bitwise(sparse, dense, f"tile entry {cfg}")


def test_plan_over_512_chunks(quiet_index_watch):
    """Over 131072 routes (more than 512 chunks of 256) the plan kernel scans each expert's
    chunk counts in several passes; the sparse path still gives the dense path's bits, with
    out-of-range indices among the routes."""
    T, E, D, I, k = 70000, 5, 64, 64, 2
    hidden = randn(T, D, seed=7770, dtype=torch.bfloat16).cuda()
    gate, up, down = nmajor_weights(E, I, D, 7771, torch.bfloat16)
    g = torch.Generator().manual_seed(7772)
    sel = torch.randint(0, E, (T, k), generator=g)
    sel[12345, 1] = E
    sel[T - 1, 0] = -3
    sel = sel.cuda()
    w = torch.rand(T, k, generator=g).cuda()
    dense, sparse = both(hidden, w, sel, gate, up, down)
    assert_bitwise(sparse, dense, "140000 routes")
    assert torch.count_nonzero(sparse[12345]) == 0 and torch.count_nonzero(sparse[T - 1]) == 0
    with pytest.raises(RuntimeError, match="outside"):
        check_moe_indices()
