"""The drop-in boundary on the CPU: the C ABI library loads and exports every declared symbol,
its host-side planning and validation paths behave, and the Python API mirrors the reference's
surface, argument checks and mode bookkeeping (test_batch_invariance.py:783-792)."""

import ctypes
import os
import re

import numpy as np
import pytest
import torch

import batch_invariant_ops as bio
from batch_invariant_ops import _native as nat
from batch_invariant_ops import batch_invariant_ops as bio_ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "biops.h")

REFERENCE_API = {
    "set_batch_invariant_mode", "is_batch_invariant_mode_enabled", "disable_batch_invariant_mode",
    "enable_batch_invariant_mode", "matmul_persistent", "linear_batch_invariant", "bmm_persistent",
    "conv1d_batch_invariant", "conv2d_batch_invariant", "conv3d_batch_invariant",
    "conv_transpose2d_batch_invariant", "conv_transpose3d_batch_invariant",
    "scaled_dot_product_attention_batch_invariant", "varlen_scaled_dot_product_attention_batch_invariant",
    "linalg_vector_norm_batch_invariant", "softmax", "log_softmax", "mean_dim",
    "get_batch_invariant_attention_block_size", "AttentionBlockSize", "deterministic_token_choice_moe",
}


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(biops_\w+)\s*\(", text))


def lib():
    return nat.load(require_gpu=False)


def test_library_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) >= 14
    handle = ctypes.CDLL(str(nat.library_path()))
    missing = [n for n in sorted(names) if not hasattr(handle, n)]
    assert not missing, f"libbiops.so lacks {missing}"
    assert names == set(nat.EXPORTED), "ctypes signatures and header disagree"


def test_library_version():
    assert lib().biops_version().decode() == "0.2.0-mi355x"


def test_public_api_matches_reference_surface():
    assert set(bio.__all__) == REFERENCE_API
    assert bio.__version__ == "0.2.0"
    assert bio.get_batch_invariant_attention_block_size() == bio.AttentionBlockSize(16, 16)


def test_conv_argument_rules_need_no_gpu():
    """The reference's conv assertions (batch_invariant_ops.py:505-514, 609-618, 795-832) fire on
    the host; valid CPU tensors are refused (no CPU path)."""
    x, w = torch.randn(2, 4, 9, 9), torch.randn(6, 2, 3, 3)
    with pytest.raises(AssertionError, match="only 2-D convolution"):
        bio.conv2d_batch_invariant(x[0], w, None, (1,), (0,), (1,), False, (0,), 2)
    with pytest.raises(AssertionError, match="transposed convolution is not supported"):
        bio.conv2d_batch_invariant(x, w, None, (1,), (0,), (1,), True, (0,), 2)
    with pytest.raises(AssertionError, match="output_padding requires transposed"):
        bio.conv2d_batch_invariant(x, w, None, (1,), (0,), (1,), False, (1, 0), 2)
    with pytest.raises(AssertionError, match="Incompatible dtypes"):
        bio.conv2d_batch_invariant(x, w.double(), None, (1,), (0,), (1,), False, (0,), 2)
    with pytest.raises(AssertionError, match="Incompatible channel dimensions"):
        bio.conv2d_batch_invariant(x, w, None, (1,), (0,), (1,), False, (0,), 1)
    with pytest.raises(AssertionError, match="must have one value"):
        bio.conv1d_batch_invariant(x[:, :, 0], w[:, :, 0], None, (1, 1), (0,), (1,), False, (0,), 2)
    with pytest.raises(AssertionError, match="non-overlapping"):
        bio.conv_transpose2d_batch_invariant(x, torch.randn(4, 3, 3, 3), None, (2, 2), (0, 0), (1, 1), (0, 0), 1)
    from batch_invariant_ops.batch_invariant_ops import convolution_batch_invariant

    with pytest.raises(AssertionError, match="only 1-D, 2-D and 3-D"):
        convolution_batch_invariant(x[0, 0], w[0, 0], None, (1,), (0,), (1,), False, (0,), 1)
    with pytest.raises(ValueError):
        bio.conv2d_batch_invariant(x, w, None, (1,), (0,), (1,), False, (0,), 2)  # CPU tensors
    L = lib()
    import ctypes
    arr = lambda *v: (ctypes.c_int64 * len(v))(*v)  # noqa: E731
    sizes = [arr(9, 9), arr(3, 3), arr(1, 1), arr(0, 0), arr(1, 1)]
    ptrs = [ctypes.addressof(a) for a in sizes]
    # regular 2-D, bf16: padded weights [6, 64] then patches [2 * 2 * 49, 64]
    ws = L.biops_conv_workspace_size(2, 2, 0, 2, 4, ptrs[0], 6, ptrs[1], ptrs[2], ptrs[3], ptrs[4], 2)
    assert ws == 6 * 64 * 2 + 2 * 2 * 49 * 64 * 2
    # transposed requires stride == kernel
    assert L.biops_conv_workspace_size(2, 2, 1, 2, 4, ptrs[0], 6, ptrs[1], ptrs[2], ptrs[3], ptrs[4], 2) == -1
    # groups must divide the channels
    assert L.biops_conv_workspace_size(2, 2, 0, 2, 4, ptrs[0], 6, ptrs[1], ptrs[2], ptrs[3], ptrs[4], 3) == -1


def test_fast_call_module_matches_the_ctypes_binding():
    """The CPython fast-call module (built beside libbiops.so) reaches the same entry points
    with the same arguments: the host checks give the same status codes; wrong argument counts
    and non-integers raise."""
    import importlib

    fast = importlib.import_module("batch_invariant_ops._biops_fast")
    L = lib()
    null = None
    for args in ((9, 4, 4, 4, 16, 4, 1, 16, 4, 1, null, 16, 4, 1, null),
                 (2, -1, 4, 4, 16, 4, 1, 16, 4, 1, null, 16, 4, 1, null),
                 (2, 4, 4, 4, 16, 4, 1, 16, 8, 8, null, 16, 4, 1, null),
                 (2, 0, 4, 4, null, 4, 1, null, 4, 1, null, null, 4, 1, null)):
        assert fast.gemm(*args) == L.biops_gemm(*args)
    assert fast.softmax(2, 7, 4, 4, 16, 4, 16, 4, 0, null) == L.biops_softmax(2, 7, 4, 4, 16, 4, 16, 4, 0, null) == 3
    assert fast.reduce(5, 2, 2, 1, 1, 1, 16, 1, 1, 1, 16, null) == 1
    with pytest.raises(TypeError):
        fast.gemm(2, 4, 4, 4)
    with pytest.raises(TypeError):
        fast.reduce(0, 2, 2, 4, 8, 1, "x", 8, 2, 1, 16, null)
    # the varlen planner and tile order give the ctypes binding's words
    cu_q = np.array([0, 5, 5, 305, 435], dtype=np.int64)
    cu_k = np.array([0, 7, 11, 11, 140], dtype=np.int64)
    a, b = np.zeros(64, dtype=np.int64), np.ones(64, dtype=np.int64)
    assert (fast.varlen_plan(4, cu_q.ctypes.data, cu_k.ctypes.data, 4, 24, 2, a.ctypes.data)
            == L.biops_varlen_plan(4, cu_q.ctypes.data, cu_k.ctypes.data, 4, 24, 2, b.ctypes.data) > 0)
    words = 8 + 8 * int(a[0])  # header and the kept sequences' entries
    assert a[0] == 2 and (a[:words] == b[:words]).all()
    oa, ob = np.zeros(3, dtype=np.int64), np.ones(3, dtype=np.int64)
    assert fast.varlen_fused_order(a.ctypes.data, 2, oa.ctypes.data) == L.biops_varlen_fused_order(
        a.ctypes.data, 2, ob.ctypes.data) == 3
    assert (oa == ob).all()
    args = (2, 8, 2, 64, 64) + (16, 8, 64) * 4 + (null, null, null, 2, 0.125, null)
    assert fast.varlen_sdpa_fused(*args) == L.biops_varlen_sdpa_fused(*args) != 0  # null plan
    # dense fused attention: fp32 outside the envelope, an odd row stride, mask with causal
    qkv = (256, 0, 0, 128) * 3
    for args in ((nat.F32, 1, 1, 1, 4, 4, 128, 128) + qkv + (null, 0, 0, 0, 0, 0, 0, 1.0, 256, null),
                 (nat.BF16, 1, 1, 1, 4, 4, 128, 128, 256, 0, 0, 130) + qkv[4:]
                 + (null, 0, 0, 0, 0, 0, 0, 1.0, 256, null),
                 (nat.BF16, 1, 1, 1, 4, 4, 128, 128) + qkv + (256, nat.BOOL, 0, 0, 4, 1, 1, 1.0, 256, null),
                 (nat.BF16, 0, 1, 1, 4, 4, 128, 128) + qkv + (null, 0, 0, 0, 0, 0, 0, 1.0, 256, null)):
        assert fast.sdpa_fused(*args) == L.biops_sdpa_fused(*args)
    assert [fast.sdpa_fused(*a) for a in (
        (nat.F32, 1, 1, 1, 4, 4, 128, 128) + qkv + (null, 0, 0, 0, 0, 0, 0, 1.0, 256, null),
        (nat.BF16, 0, 1, 1, 4, 4, 128, 128) + qkv + (null, 0, 0, 0, 0, 0, 0, 1.0, 256, null))] == [3, 0]
    with pytest.raises(TypeError):
        fast.sdpa_fused(*((nat.BF16, 1, 1, 1, 4, 4, 128, 128) + qkv + (null, 0, 0, 0, 0, 0, 0, "x", 256, null)))
    # planned fused varlen: host checks before any HIP call (decreasing offsets, a work-list
    # buffer too small, an unsupported dtype, offsets past the packed rows)
    cu_dec = np.array([0, 5, 3], dtype=np.int64)
    cu_ok = np.array([0, 5, 9], dtype=np.int64)
    hb = np.zeros(64, dtype=np.int64)
    cu_one = np.array([1, 5, 9], dtype=np.int64)

    def planned(dtype, cuq, cuk, words, total=9, total_kv=9):
        return (dtype, 8, 2, 64, 64) + (256, 8 * 64, 64) * 4 + (total, total_kv, 2, cuq.ctypes.data,
                                                                  cuk.ctypes.data, hb.ctypes.data, words, 256, 2,
                                                                  0.125, null)
    for args, rc in ((planned(nat.BF16, cu_dec, cu_ok, 64), 1), (planned(nat.BF16, cu_ok, cu_ok, 8), 5),
                     (planned(nat.F32, cu_ok, cu_ok, 64), 3), (planned(nat.BF16, cu_ok, cu_ok, 64, total=8), 1),
                     (planned(nat.BF16, cu_ok, cu_ok, 64, total_kv=8), 1), (planned(nat.BF16, cu_one, cu_ok, 64), 1)):
        assert fast.varlen_sdpa_fused_planned(*args) == L.biops_varlen_sdpa_fused_planned(*args) == rc
    assert fast.varlen_sdpa_fused_planned(*planned(nat.BF16, cu_dec, cu_ok, 64)) == 1
    assert "nondecreasing" in nat.last_error()
    # the work-list upload: argument errors raise before any HIP call
    with pytest.raises(TypeError):
        fast.copy_h2d(256, 256, 16)
    with pytest.raises(ValueError):
        fast.copy_h2d(256, 256, -1, null)
    if torch.cuda.is_available():
        assert nat.fast_function("biops_gemm") is fast.gemm
    else:  # the product path still insists on a GPU
        with pytest.raises(RuntimeError, match="ROCm GPU"):
            nat.fast_function("biops_gemm")


def test_host_validation_needs_no_gpu():
    L = lib()
    null = None
    # unsupported dtype, negative sizes, bad layouts are rejected before any launch
    assert L.biops_gemm(9, 4, 4, 4, 16, 4, 1, 16, 4, 1, null, 16, 4, 1, null) == 3
    assert L.biops_gemm(2, -1, 4, 4, 16, 4, 1, 16, 4, 1, null, 16, 4, 1, null) == 1
    assert L.biops_gemm(2, 4, 4, 4, 16, 1, 4, 16, 4, 1, null, 16, 4, 1, null) == 2  # A not K-contiguous
    assert L.biops_gemm(2, 4, 4, 4, 16, 4, 1, 16, 8, 8, null, 16, 4, 1, null) == 2  # B without unit stride
    assert b"unit stride" in L.biops_last_error()
    assert L.biops_gemm(2, 0, 4, 4, null, 4, 1, null, 4, 1, null, null, 4, 1, null) == 0  # empty
    assert L.biops_bmm(2, 1, 6, 4, 4, 4, 16, 0, 0, 4, 1, 16, 0, 0, 4, 1, 4, 16, 0, 0, 4, 1, null) == 1  # group !| heads
    assert L.biops_softmax(2, 7, 4, 4, 16, 4, 16, 4, 0, null) == 3
    assert L.biops_reduce(5, 2, 2, 1, 1, 1, 16, 1, 1, 1, 16, null) == 1
    assert L.biops_reduce(0, 2, 2, 4, 8, 1, 16, 8, 2, 1, 16, null) == 2  # strided rows with K == 1


def test_fused_attention_envelope_and_host_checks():
    """The fused-attention entry points validate dtype, head sizes, layouts and masks on the
    host and return their status before any launch."""
    L = lib()
    assert L.biops_attention_fused_supported(nat.BF16, 128, 128) == 1
    assert L.biops_attention_fused_supported(nat.F16, 8, 8) == 1
    assert L.biops_attention_fused_supported(nat.F32, 64, 64) == 0
    assert L.biops_attention_fused_supported(nat.BF16, 72, 130) == 0
    assert L.biops_attention_fused_supported(nat.BF16, 256, 200) == 1
    assert L.biops_varlen_fused_supported(nat.BF16, 256, 200) == 0
    assert L.biops_attention_fused_supported(nat.BF16, 12, 64) == 0
    # masks: unit key stride, strides and lk multiples of 4, base aligned to four elements
    assert L.biops_attention_fused_mask_ok(64, nat.BF16, 1024, 1024 * 1024, 0, 1024, 1) == 1
    assert L.biops_attention_fused_mask_ok(4, nat.BOOL, 1024, 1024 * 1024, 0, 1024, 1) == 1
    assert L.biops_attention_fused_mask_ok(4, nat.BF16, 1024, 0, 0, 1024, 1) == 0  # base not 8-byte aligned
    assert L.biops_attention_fused_mask_ok(64, nat.BF16, 1022, 0, 0, 1022, 1) == 0  # keys % 4
    assert L.biops_attention_fused_mask_ok(64, nat.BF16, 1024, 0, 0, 1, 1024) == 0  # keys not contiguous
    assert L.biops_attention_fused_mask_ok(None, nat.BF16, 1024, 0, 0, 1024, 1) == 0
    p = 256  # a 16-byte aligned stand-in address: every call below fails before touching memory
    args = [p, 0, 0, 128] * 3
    # fp32 is outside the envelope; an odd row stride is a layout error; mask with causal
    assert L.biops_sdpa_fused(nat.F32, 1, 1, 1, 4, 4, 128, 128, *args, None, 0, 0, 0, 0, 0, 0, 1.0, p, None) == 3
    bad = [p, 0, 0, 130] + [p, 0, 0, 128] * 2
    assert L.biops_sdpa_fused(nat.BF16, 1, 1, 1, 4, 4, 128, 128, *bad, None, 0, 0, 0, 0, 0, 0, 1.0, p, None) == 2
    assert L.biops_sdpa_fused(nat.BF16, 1, 1, 1, 4, 4, 128, 128, *args, p, nat.BOOL, 0, 0, 4, 1, 1, 1.0, p, None) == 1
    assert L.biops_sdpa_fused(nat.BF16, 1, 4, 3, 4, 4, 128, 128, *args, None, 0, 0, 0, 0, 0, 0, 1.0, p, None) == 1
    # a mask the fused kernel cannot read four keys at a time from
    assert L.biops_sdpa_fused(nat.BF16, 1, 1, 1, 4, 6, 128, 128, *args, p, nat.BOOL, 0, 0, 6, 1, 0, 1.0, p, None) == 2
    assert L.biops_sdpa_fused(nat.BF16, 0, 1, 1, 4, 4, 128, 128, *args, None, 0, 0, 0, 0, 0, 0, 1.0, p, None) == 0


def test_workspace_queries():
    L = lib()
    assert L.biops_sdpa_workspace_size(2, 16, 16, 1024, 1024) == 16 * 16 * 1024 * 1024 * 2
    assert L.biops_sdpa_workspace_size(0, 1, 1, 3, 5) == 3 * 8 * 4  # rows padded to 8 elements
    assert L.biops_moe_workspace_size(2, 4096, 64, 2048, 768) == (64 * 4096 * 768 + 64 * 4096 * 2048) * 2
    assert L.biops_moe_workspace_size(9, 1, 1, 1, 1) == -1


def test_padded_workspace_rule_matches_the_library():
    """The Python wrappers size the workspace of biops_gemm_padded / biops_bmm_padded themselves
    (no extra call per product); their sizes must equal the library's for every layout, and the
    rule must leave direct-load operands alone and pad long or misaligned K of large products."""
    L = lib()
    codes = {torch.bfloat16: nat.BF16, torch.float16: nat.F16, torch.float32: nat.F32}
    for dt, M, N, K in ((torch.bfloat16, 300, 700, 5000), (torch.float16, 257, 515, 2050),
                        (torch.float32, 64, 8192, 2040), (torch.bfloat16, 96, 130, 1027)):
        a = torch.zeros(M, K, dtype=dt)
        for b in (torch.zeros(N, K, dtype=dt).t(), torch.zeros(K, N, dtype=dt)):
            ws = bio_ops._padded_workspace(a, b, M, N, K)
            assert ws > 0, (dt, M, N, K, b.stride())
            assert ws == L.biops_gemm_padded_workspace_size(codes[dt], M, N, K, b.stride(0), b.stride(1))
        a3 = torch.zeros(3, M, K, dtype=dt)
        for b3 in (torch.zeros(3, N, K, dtype=dt).transpose(1, 2), torch.zeros(3, K, N, dtype=dt),
                   torch.zeros(1, K, N, dtype=dt).expand(3, K, N)):
            ws = bio_ops._padded_workspace(a3, b3, M, N, K, 3)
            assert ws == L.biops_bmm_padded_workspace_size(codes[dt], 3, M, N, K, a3.stride(0), b3.stride(0),
                                                           b3.stride(1), b3.stride(2))
    # whole 128-byte steps on aligned rows, and small products, keep biops_gemm
    assert bio_ops._padded_workspace(torch.zeros(64, 2048, dtype=torch.bfloat16),
                                 torch.zeros(2048, 512, dtype=torch.bfloat16), 64, 512, 2048) == 0
    assert bio_ops._padded_workspace(torch.zeros(32, 80, dtype=torch.bfloat16),
                                 torch.zeros(80, 512, dtype=torch.bfloat16), 32, 512, 80) == 0
    assert L.biops_gemm_padded_workspace_size(9, 1, 1, 1, 1, 1) == -1


def plan(cu_q, cu_kv, hq=4, dv=24, dtype=nat.BF16):
    L = lib()
    n = len(cu_q) - 1
    out = np.zeros(L.biops_varlen_plan_len(n), dtype=np.int64)
    q = np.asarray(cu_q, dtype=np.int64)
    k = np.asarray(cu_kv, dtype=np.int64)
    ws = L.biops_varlen_plan(n, q.ctypes.data, k.ctypes.data, hq, dv, dtype, out.ctypes.data)
    return ws, out


def test_varlen_plan_work_list():
    # sequences: (q 5, kv 7), (q 0, kv 4) dropped, (q 300, kv 0) dropped, (q 130, kv 129)
    ws, p = plan([0, 5, 5, 305, 435], [0, 7, 11, 11, 140], hq=4, dv=24)
    items, qk_tiles, pv_tiles, rows, selems = p[:5]
    assert items == 2
    first = p[8:16].tolist()
    second = p[16:24].tolist()
    assert first == [0, 5, 0, 7, 0, 0, 0, 0]
    # second item starts after 4 heads x 5 rows x pitch 8 of the first
    assert second[:5] == [305, 130, 11, 129, 4 * 5 * 8]
    assert second[5:] == [4 * 1 * 1, 4 * 1 * 1, 4 * 5]
    assert qk_tiles == 4 + 4 * 2 * 2 and pv_tiles == 4 + 4 * 2 * 1
    assert rows == 4 * 5 + 4 * 130
    assert selems == 4 * 5 * 8 + 4 * 130 * 136
    assert ws == selems * 2
    assert p[5] == 1 + 2  # 128-row query tiles: 5 rows, then 130 rows


def fused_order(p, causal):
    L = lib()
    order = np.full(int(p[5]), -1, dtype=np.int64)
    n = L.biops_varlen_fused_order(p.ctypes.data, causal, order.ctypes.data)
    return n, [(int(e) >> 32, int(e) & 0xFFFFFFFF) for e in order]


def test_varlen_fused_order_longest_key_range_first():
    # items: (q 5, kv 7) and (q 130, kv 129); entries are (item, query tile)
    _, p = plan([0, 5, 5, 305, 435], [0, 7, 11, 11, 140], hq=4, dv=24)
    # bottom-right: item 1's tiles see keys up to row + (129 - 130) + 1: 127 and 129 keys,
    # item 0's one tile 4 + 2 + 1 = 7 keys
    assert fused_order(p, nat.CAUSAL_BOTTOM_RIGHT) == (3, [(1, 1), (1, 0), (0, 0)])
    # top-left: 128 and min(130, 129) keys against 5
    assert fused_order(p, nat.CAUSAL_TOP_LEFT) == (3, [(1, 1), (1, 0), (0, 0)])
    # no mask: every tile of a sequence sees all its keys; ties keep plan order
    assert fused_order(p, nat.CAUSAL_NONE) == (3, [(1, 0), (1, 1), (0, 0)])
    # a short sequence after a long one still goes after its longer tiles
    _, p = plan([0, 300, 340], [0, 300, 340], hq=2, dv=8)
    assert fused_order(p, nat.CAUSAL_BOTTOM_RIGHT) == (4, [(0, 2), (0, 1), (0, 0), (1, 0)])


def test_varlen_fused_order_rejects_an_inconsistent_plan():
    _, p = plan([0, 5, 135], [0, 7, 140])
    p[5] += 1
    n, _ = fused_order(p, nat.CAUSAL_NONE)
    assert n < 0 and b"word 5" in lib().biops_last_error()


def test_varlen_plan_rejects_decreasing_offsets():
    ws, _ = plan([0, 5, 3], [0, 2, 4])
    assert ws < 0 and b"nondecreasing" in lib().biops_last_error()


def test_ops_reject_cpu_tensors_and_bad_arguments():
    x = torch.randn(3, 4)
    with pytest.raises(AssertionError):
        bio.matmul_persistent(x, torch.randn(5, 2))
    with pytest.raises(AssertionError):
        bio.bmm_persistent(x, x)
    with pytest.raises(ValueError):
        bio.matmul_persistent(x, torch.randn(4, 2))  # CPU tensors: no CPU path
    with pytest.raises(ValueError):
        bio.softmax(torch.ones(2, dtype=torch.int64))
    with pytest.raises(ValueError):
        bio.softmax(x, dtype=torch.int32)
    with pytest.raises(ValueError):
        bio.scaled_dot_product_attention_batch_invariant(x[None], x[None], x[None], dropout_p=0.5)
    with pytest.raises(ValueError):
        bio.scaled_dot_product_attention_batch_invariant(x[None], x[None].double(), x[None])
    with pytest.raises(ValueError):
        bio.scaled_dot_product_attention_batch_invariant(x[None, None], x[None, None], x[None, None], enable_gqa=True,
                                                         attn_mask=torch.ones(3, 3, dtype=torch.bool), is_causal=True)
    with pytest.raises(ValueError):
        bio.varlen_scaled_dot_product_attention_batch_invariant(x, x, x, torch.tensor([0, 3]), torch.tensor([0, 3]))
    q = torch.zeros(1, 4, 2, 8)
    with pytest.raises(ValueError):
        bio.varlen_scaled_dot_product_attention_batch_invariant(q, q, q, torch.tensor([0.0, 4.0]), torch.tensor([0, 4]))
    with pytest.raises(ValueError):
        bio.varlen_scaled_dot_product_attention_batch_invariant(q, q, q, torch.tensor([1, 4]), torch.tensor([0, 4]))
    with pytest.raises(ValueError):
        bio.deterministic_token_choice_moe(x, torch.ones(3, 2), torch.zeros(3, 1, dtype=torch.long),
                                           torch.ones(2, 5, 4), torch.ones(2, 5, 4), torch.ones(2, 4, 5))
    with pytest.raises(ValueError):
        bio.deterministic_token_choice_moe(x, torch.ones(3, 1), torch.zeros(3, 1, dtype=torch.long),
                                           torch.ones(2, 5, 4), torch.ones(2, 5, 4), torch.ones(2, 5, 4))
    with pytest.raises(AssertionError):
        bio.linalg_vector_norm_batch_invariant(x)  # reference asserts a CUDA tensor


def test_mode_context_is_exception_safe_and_reentrant():
    assert not bio.is_batch_invariant_mode_enabled()
    with pytest.raises(RuntimeError, match="sentinel"):
        with bio.set_batch_invariant_mode():
            assert bio.is_batch_invariant_mode_enabled()
            with bio.set_batch_invariant_mode():
                assert bio.is_batch_invariant_mode_enabled()
            with bio.set_batch_invariant_mode(False):
                assert not bio.is_batch_invariant_mode_enabled()
            assert bio.is_batch_invariant_mode_enabled()
            raise RuntimeError("sentinel")
    assert not bio.is_batch_invariant_mode_enabled()
    bio.enable_batch_invariant_mode()
    bio.enable_batch_invariant_mode()  # idempotent
    assert bio.is_batch_invariant_mode_enabled()
    bio.disable_batch_invariant_mode()
    assert not bio.is_batch_invariant_mode_enabled()


def test_mode_registers_gpu_key_only():
    """The ten overrides of the reference (batch_invariant_ops.py:1668-1684) live on dispatch key
    CUDA (ROCm GPUs); CPU tensors keep the stock kernels."""
    a = torch.randn(4, 5)
    b = torch.randn(5, 3)
    with bio.set_batch_invariant_mode():
        assert torch.equal(torch.mm(a, b), a @ b)
        assert torch.softmax(a, -1).shape == (4, 5)
        assert a.mean(-1).shape == (4,)
        assert torch.nn.functional.conv1d(torch.ones(1, 2, 5), torch.ones(3, 2, 2)).shape == (1, 3, 4)
    names = [op for op, _ in bio.batch_invariant_ops._OVERRIDES]
    assert names == [
        "aten::mm", "aten::addmm", "aten::linear", "aten::bmm", "aten::convolution",
        "aten::scaled_dot_product_attention", "aten::_softmax", "aten::_log_softmax", "aten::mean.dim",
        "aten::linalg_vector_norm",
    ]
    assert bio.batch_invariant_ops._DISPATCH_KEY == "CUDA"


def test_missing_gpu_is_a_loud_error():
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        nat.load(require_gpu=True)


def test_get_compute_units_cpu_answer(monkeypatch, capsys):
    """Without a GPU the reference prints a notice and answers with the torch thread count
    (batch_invariant_ops.py:249-251)."""
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert bio_ops.get_compute_units() == torch.get_num_threads()
    assert "Using CPU" in capsys.readouterr().out


@pytest.mark.gpu
def test_get_compute_units_matches_the_device():
    """On the GPU the answer is the device's compute-unit count (256 on an MI355X)."""
    props = torch.cuda.get_device_properties(0)
    assert bio_ops.get_compute_units() == props.multi_processor_count
    assert lib().biops_compute_units() == props.multi_processor_count
    if "gfx950" in getattr(props, "gcnArchName", ""):
        assert bio_ops.get_compute_units() == 256


def test_noalloc_moe_rejects_oversize_before_any_gpu_work():
    """biops_moe_sparse_noalloc checks its sizes on the host first: 4096 C5 tokens need more
    than its static array, so it returns BIOPS_ERR_SIZE without touching a device (this runs
    without a GPU)."""
    handle = lib()
    rc = handle.biops_moe_sparse_noalloc(
        nat.BF16, 4096, 64, 2048, 768, 8, None, 2048, None, 1, 2048, 1, None, 1, 2048, 1,
        None, 1, 1, 2048, None, nat.BF16, None, None, None, None)
    assert rc == 5
    msg = handle.biops_last_error().decode()
    assert "scratch" in msg and str(nat.MOE_NOALLOC_SCRATCH_BYTES) in msg
