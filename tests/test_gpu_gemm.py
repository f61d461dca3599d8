"""GEMM / linear / BMM on the GPU: bitwise batch invariance and parity with the oracle.

Mirrors the reference's operator tests (test_batch_invariance.py:42-172) with inputs made on
the CPU from seeded generators, so that the oracle sees the same values."""

import pytest
import torch

import oracle
from batch_invariant_ops import bmm_persistent, linear_batch_invariant, matmul_persistent

from _tol import assert_bitwise, assert_first_sample_equal, assert_gemm_close

pytestmark = pytest.mark.gpu
DTYPES = (torch.float32, torch.float16, torch.bfloat16)
# Tile entry 12 of the GEMM menu: the skinny entry (include/biops.h, biops_set_gemm_tile).
SKINNY_ENTRY = 12


def randn(*shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * scale).to(dtype)


def gpu(*ts):
    out = tuple(t.cuda() for t in ts)
    return out if len(out) > 1 else out[0]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch_size", (2, 3, 5, 17))
def test_mm_is_batch_invariant(dtype, batch_size):
    x = gpu(randn(batch_size, 257, seed=1000 + batch_size, dtype=dtype))
    w = gpu(randn(257, 129, seed=1100 + batch_size, dtype=dtype))
    assert_first_sample_equal(matmul_persistent(x[:1], w), matmul_persistent(x, w))


@pytest.mark.parametrize("dtype", DTYPES)
def test_mm_rows_do_not_depend_on_position(dtype):
    """Row i computed alone equals row i inside the batch for every i (MFMA lane position)."""
    x = gpu(randn(70, 300, seed=1200, dtype=dtype))
    w = gpu(randn(300, 200, seed=1201, dtype=dtype))
    full = matmul_persistent(x, w)
    for i in (0, 1, 5, 31, 32, 33, 63, 64, 69):
        assert_bitwise(matmul_persistent(x[i : i + 1], w), full[i : i + 1], f"row {i}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_mm_matches_oracle(dtype):
    a = randn(37, 257, seed=2000, dtype=dtype)
    b = randn(257, 91, seed=2001, dtype=dtype)
    out = matmul_persistent(*gpu(a, b))
    assert_gemm_close(out, oracle.matmul(a, b), oracle.gemm_abs(a, b), 257)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ("b_rowmajor", "b_transposed"))
@pytest.mark.parametrize("shape", ((300, 2048, 520), (129, 65, 96), (5, 1, 33), (64, 4096, 256)))
def test_mm_layouts_match_oracle(dtype, layout, shape):
    m, k, n = shape
    a = randn(m, k, seed=2100 + m, dtype=dtype)
    if layout == "b_rowmajor":
        b = randn(k, n, seed=2200 + n, dtype=dtype)
    else:
        b = randn(n, k, seed=2200 + n, dtype=dtype).t()
    out = matmul_persistent(*gpu(a, b))
    assert_gemm_close(out, oracle.matmul(a, b), oracle.gemm_abs(a, b), k)


@pytest.mark.parametrize("dtype", DTYPES)
def test_mm_empty_and_zero_k(dtype):
    a = gpu(randn(4, 0, seed=1, dtype=dtype))
    b = gpu(randn(0, 7, seed=2, dtype=dtype))
    assert torch.equal(matmul_persistent(a, b), torch.zeros(4, 7, dtype=dtype, device="cuda"))
    assert matmul_persistent(gpu(randn(0, 5, seed=3, dtype=dtype)), gpu(randn(5, 3, seed=4, dtype=dtype))).shape == (0, 3)
    bias = gpu(randn(7, seed=5, dtype=dtype))
    assert torch.equal(matmul_persistent(a, b, bias), bias.expand(4, 7))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch_size", (2, 5, 17))
def test_rank3_linear_is_batch_invariant(dtype, batch_size):
    x = gpu(randn(batch_size, 37, 257, seed=2500 + batch_size, dtype=dtype))
    w = gpu(randn(91, 257, seed=2600 + batch_size, dtype=dtype))
    bias = gpu(randn(91, seed=2650 + batch_size, dtype=dtype))
    assert_first_sample_equal(linear_batch_invariant(x[:1], w, bias), linear_batch_invariant(x, w, bias))


@pytest.mark.parametrize("dtype", DTYPES)
def test_linear_matches_oracle(dtype):
    x = randn(3, 37, 257, seed=2700, dtype=dtype)
    w = randn(91, 257, seed=2701, dtype=dtype)
    bias = randn(91, seed=2702, dtype=dtype)
    out = linear_batch_invariant(*gpu(x, w, bias))
    absprod = oracle.gemm_abs(x.reshape(-1, 257), w.t()) + bias.double().abs()
    assert_gemm_close(out.reshape(-1, 91), oracle.linear(x, w, bias).reshape(-1, 91), absprod, 257)


def test_projector_linear_shape_is_batch_invariant():
    x = gpu(randn(2, 256, 1024, seed=2750, dtype=torch.bfloat16))
    w = gpu(randn(4096, 1024, seed=2751, dtype=torch.bfloat16))
    bias = gpu(randn(4096, seed=2752, dtype=torch.bfloat16))
    assert_first_sample_equal(linear_batch_invariant(x[:1], w, bias), linear_batch_invariant(x, w, bias))


def test_small_batch_fp32_projection_is_batch_invariant():
    x = gpu(randn(2, 2304, seed=2775))
    w = gpu(randn(2304, 2304, seed=2776))
    bias = gpu(randn(2304, seed=2777))
    assert_first_sample_equal(linear_batch_invariant(x[:1], w, bias), linear_batch_invariant(x, w, bias))


@pytest.mark.parametrize(("n", "k", "with_bias"), ((8192, 2048, True), (2048, 8192, False)))
def test_metric_gemm_rows_identical_for_every_m(n, k, with_bias):
    """The metric's M sweep: every row of an M-row GEMM equals the same row of the 4096-row GEMM."""
    x = gpu(randn(4096, k, seed=2800 + n, dtype=torch.bfloat16))
    w = gpu(randn(n, k, seed=2801 + n, dtype=torch.bfloat16, scale=0.02))
    bias = gpu(randn(n, seed=2802 + n, dtype=torch.bfloat16, scale=0.02)) if with_bias else None
    full = linear_batch_invariant(x, w, bias)
    for m in (1, 2, 3, 4, 64, 100, 129, 256, 1024, 2048, 4095):
        assert_bitwise(linear_batch_invariant(x[:m], w, bias), full[:m], f"M={m}")
    # rows computed at an offset (the sample sits at a different tile position)
    assert_bitwise(linear_batch_invariant(x[77:200], w, bias), full[77:200], "rows 77..199")


def test_metric_gemm_matches_oracle():
    x = randn(300, 2048, seed=2900, dtype=torch.bfloat16)
    w = randn(8192, 2048, seed=2901, dtype=torch.bfloat16, scale=0.02)
    bias = randn(8192, seed=2902, dtype=torch.bfloat16, scale=0.02)
    out = linear_batch_invariant(*gpu(x, w, bias))
    absprod = oracle.gemm_abs(x, w.t()) + bias.double().abs()
    assert_gemm_close(out, oracle.linear(x, w, bias), absprod, 2048)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch_size", (2, 3, 5, 17))
def test_bmm_is_batch_invariant(dtype, batch_size):
    a = gpu(randn(batch_size, 33, 65, seed=3000 + batch_size, dtype=dtype))
    b = gpu(randn(batch_size, 65, 47, seed=3100 + batch_size, dtype=dtype))
    assert_first_sample_equal(bmm_persistent(a[:1], b[:1]), bmm_persistent(a, b))


@pytest.mark.parametrize("dtype", DTYPES)
def test_bmm_matches_oracle_for_noncontiguous_attention_inputs(dtype):
    q = randn(4, 8, 33, 65, seed=4000, dtype=dtype).reshape(-1, 33, 65)
    k = randn(4, 8, 47, 65, seed=4001, dtype=dtype).reshape(-1, 47, 65).transpose(1, 2)
    out = bmm_persistent(*gpu(q, k))
    assert_gemm_close(out, oracle.bmm(q, k), q.double().abs() @ k.double().abs(), 65)


@pytest.mark.parametrize("dtype", DTYPES)
def test_bmm_row_major_b_on_the_direct_path(dtype):
    """Row-major (N-major) right operands whose K is a whole number of 128-byte steps and whose
    rows are whole 16-byte chunks take the global->LDS path for every dtype (fp32 with 4-byte
    fragment reads): oracle parity, and the bits of the same values stored K-major."""
    a = randn(3, 70, 256, seed=4200, dtype=dtype)
    b = randn(3, 256, 104, seed=4201, dtype=dtype)
    out = bmm_persistent(*gpu(a, b))
    assert_gemm_close(out, oracle.bmm(a, b), a.double().abs() @ b.double().abs(), 256)
    b_kmajor = gpu(b).transpose(1, 2).contiguous().transpose(1, 2)
    assert b_kmajor.stride(1) == 1
    assert_bitwise(bmm_persistent(gpu(a), b_kmajor), out, "K-major B")
    assert_first_sample_equal(bmm_persistent(gpu(a)[:1], gpu(b)[:1]), out)


@pytest.mark.parametrize("dtype", DTYPES)
def test_bmm_broadcast_operand_matches_oracle(dtype):
    """Stride-0 batch operand (the MoE token matrix) and a row-major right operand."""
    x = randn(19, 40, seed=4100, dtype=dtype)
    w = randn(6, 40, 70, seed=4101, dtype=dtype)
    a = x.unsqueeze(0).expand(6, -1, -1)
    out = bmm_persistent(gpu(x).unsqueeze(0).expand(6, -1, -1), gpu(w))
    assert_gemm_close(out, oracle.bmm(a, w), a.double().abs() @ w.double().abs(), 40)


def test_bmm_supports_more_than_grid_limit():
    a = gpu(randn(70_000, 1, 4, seed=4500, dtype=torch.bfloat16))
    b = gpu(randn(70_000, 4, 1, seed=4501, dtype=torch.bfloat16))
    full = bmm_persistent(a, b)
    assert_first_sample_equal(bmm_persistent(a[:1], b[:1]), full)
    ref = oracle.bmm(a.cpu(), b.cpu())
    assert_gemm_close(full, ref, a.cpu().double().abs() @ b.cpu().double().abs(), 4)


def test_bmm_empty():
    a = gpu(randn(0, 3, 4, seed=1))
    b = gpu(randn(0, 4, 5, seed=2))
    assert bmm_persistent(a, b).shape == (0, 3, 5)


@pytest.fixture
def tile_menu():
    from batch_invariant_ops import _native as nat

    lib = nat.load()
    yield lib
    lib.biops_set_gemm_tile(-1)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("m", "k", "n", "layout"), (
    (300, 2048, 520, "w"),      # K-major B (nn.Linear), direct-to-LDS loads
    (512, 256, 768, "w"),       # whole 256x256 blocks (large-tile entry) and 32x32 blocks
    (129, 200, 136, "w"),       # K not a multiple of the step: register path
    (77, 1024, 256, "rowmajor"),  # N-major B
    (33, 65, 47, "w"),          # unaligned rows
))
def test_every_tile_entry_gives_identical_bits(tile_menu, dtype, m, k, n, layout):
    """All entries of the tile menu compute each element with the same MFMA sequence."""
    x = gpu(randn(m, k, seed=5000 + m, dtype=dtype))
    if layout == "w":
        b = gpu(randn(n, k, seed=5001 + n, dtype=dtype)).t()
    else:
        b = gpu(randn(k, n, seed=5001 + n, dtype=dtype))
    bias = gpu(randn(n, seed=5002, dtype=dtype))
    tile_menu.biops_set_gemm_tile(-1)
    ref = matmul_persistent(x, b, bias)
    for cfg in range(tile_menu.biops_gemm_tile_count()):
        assert tile_menu.biops_set_gemm_tile(cfg) == 0
        assert_bitwise(matmul_persistent(x, b, bias), ref, f"tile entry {cfg}")
        assert_bitwise(matmul_persistent(x[5:6], b, bias), ref[5:6], f"tile entry {cfg}, one row")


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("layout", ("kmajor", "broadcast", "nmajor"))
def test_every_tile_entry_gives_identical_bits_bmm(tile_menu, dtype, layout):
    """Batched products (a stride-0 expanded weight and a row-major, N-major B included) keep
    their bits on every entry, the four-wave and skinny entries among them."""
    a = gpu(randn(3, 300, 2048, seed=5500, dtype=dtype))
    if layout == "broadcast":
        b = gpu(randn(520, 2048, seed=5501, dtype=dtype)).t().unsqueeze(0).expand(3, -1, -1)
    elif layout == "nmajor":
        b = gpu(randn(3, 2048, 520, seed=5501, dtype=dtype))
    else:
        b = gpu(randn(3, 520, 2048, seed=5501, dtype=dtype)).transpose(1, 2)
    tile_menu.biops_set_gemm_tile(-1)
    ref = bmm_persistent(a, b)
    for cfg in range(tile_menu.biops_gemm_tile_count()):
        assert tile_menu.biops_set_gemm_tile(cfg) == 0
        assert_bitwise(bmm_persistent(a, b), ref, f"tile entry {cfg}")
        assert_bitwise(bmm_persistent(a[1:2, 7:8], b[1:2]), ref[1:2, 7:8], f"tile entry {cfg}, one row")


def _adversarial(kind, shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    if kind == "wide":  # exponents over +-20 octaves (fp16: +-6)
        span = 6 if dtype == torch.float16 else 20
        x = x * torch.pow(2.0, torch.randint(-span, span + 1, shape, generator=g).float())
    elif kind == "cancel":  # alternating large terms that cancel, small remainders
        x = torch.where(torch.arange(x.numel()).reshape(shape) % 2 == 0, 64.0 + x, -64.0 + x * 1e-2)
    elif kind == "tiny":  # products in the subnormal range of fp32
        x = x * (2.0 ** (-14 if dtype == torch.float16 else -66))
    elif kind == "inf":
        x = x.flatten()
        x[::997] = float("inf")
        x = x.reshape(shape)
    return x.to(dtype)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("kind", ("wide", "cancel", "tiny", "inf"))
@pytest.mark.parametrize("m", (1, 20, 32))
@pytest.mark.parametrize("layout", ("kmajor", "nmajor"))
@pytest.mark.parametrize("entry", ("skinny", 20, 21, 22))
def test_16x16x32_entries_bits_on_adversarial_operands(tile_menu, dtype, kind, m, layout, entry):
    """The entries that issue 16x16x32 MFMAs for 16-bit types -- the skinny entry and the
    weight-streaming entries 20-22 (16-, 32- and 64-row m-tiles) -- against entry 2 (32x32x16
    MFMAs), bit for bit, with K-major and N-major B, on operands that stress the accumulation:
    wide exponents, cancellation, subnormal products and infinities (NaN results compare as
    equal only when both are NaN)."""
    if entry == "skinny" and layout == "nmajor":
        pytest.skip("the skinny entry takes K-major B only (N-major calls go to another entry)")
    k, n = 4096, 1000
    x = gpu(_adversarial(kind, (m, k), 5400 + m, dtype))
    w = gpu(_adversarial(kind, (n, k), 5401, dtype))
    b = w.t() if layout == "kmajor" else w.t().contiguous()
    assert tile_menu.biops_set_gemm_tile(2) == 0
    ref = matmul_persistent(x, w.t())
    assert tile_menu.biops_set_gemm_tile(SKINNY_ENTRY if entry == "skinny" else entry) == 0
    out = matmul_persistent(x, b)
    both_nan = torch.isnan(out) & torch.isnan(ref)
    assert_bitwise(torch.where(both_nan, torch.zeros_like(out), out),
                   torch.where(both_nan, torch.zeros_like(ref), ref), f"entry {entry}, {layout}, {kind}, m={m}")


@pytest.mark.parametrize(("m", "n", "bias"), (
    (2048, 8192, True),    # 8 x 32 = 256 tiles of 256 x 256: the four-wave large-tile entry
    (4096, 2048, False),   # 256 tiles of 256 x 128: a smaller four-wave block
    (2048, 2048, True),    # 256 tiles of 128 x 128
    (1024, 2048, False),   # 256 tiles of 128 x 64
    (512, 2048, True),     # 32x32 blocks on entry 6 (four per compute unit)
    (384, 2048, False),    # partial rounds for every block
    (3072, 4096, True),    # 192 tiles of 256 x 256 (fewer than the compute units)
))
def test_long_k_large_tile_choice_keeps_bits(tile_menu, m, n, bias):
    """At long K the automatic choice may take a four-wave entry (13-19, weighed by the tile
    cost model); rows keep the bits of a table entry and of a one-row call."""
    k = 4096
    x = gpu(randn(m, k, seed=5300 + m, dtype=torch.bfloat16))
    w = gpu(randn(n, k, seed=5301 + n, dtype=torch.bfloat16) * 0.05)
    b = gpu(randn(n, seed=5302, dtype=torch.bfloat16)) if bias else None
    tile_menu.biops_set_gemm_tile(-1)
    auto = matmul_persistent(x, w.t(), b)
    row = min(777, m - 1)
    one = matmul_persistent(x[row:row + 1], w.t(), b)
    assert tile_menu.biops_set_gemm_tile(2) == 0
    ref = matmul_persistent(x, w.t(), b)
    assert_bitwise(auto, ref, "automatic entry vs entry 2")
    assert_bitwise(one, ref[row:row + 1], "one row vs full")


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize(("m", "n"), (
    (1, 2048),     # 8-column skinny blocks (256 of them)
    (20, 1003),    # 8-column blocks, 3-column last block
    (32, 4000),    # 16-column blocks (250 of them)
    (7, 4090),     # 16-column blocks, 10-column last block
    (128, 2048),   # 32-column blocks
))
def test_skinny_block_widths_give_identical_bits(tile_menu, dtype, m, n):
    """The skinny entry narrows its blocks to 16 or 8 columns when a problem has few column
    blocks; the stored columns keep the bits of the table entries."""
    k = 1024
    x = gpu(randn(m, k, seed=5200 + m, dtype=dtype))
    w = gpu(randn(n, k, seed=5201 + n, dtype=dtype))
    bias = gpu(randn(n, seed=5202, dtype=dtype))
    skinny = SKINNY_ENTRY
    assert tile_menu.biops_set_gemm_tile(2) == 0
    ref = matmul_persistent(x, w.t(), bias)
    ref_plain = matmul_persistent(x, w.t())
    assert tile_menu.biops_set_gemm_tile(skinny) == 0
    assert_bitwise(matmul_persistent(x, w.t(), bias), ref, "skinny entry")
    assert_bitwise(matmul_persistent(x[m - 1:], w.t(), bias), ref[m - 1:], "skinny entry, last row")
    assert_bitwise(matmul_persistent(x, w.t()), ref_plain, "skinny entry, no bias")


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize(("m", "n", "k"), (
    (1, 2048, 8192),     # 8 x 8 blocks, 16 stages of 8 K steps, one loader-split block per unit
    (5, 8192, 2048),     # 8 x 32 blocks (four stages: the whole ring)
    (8, 4090, 1024),     # 8 x 16 blocks, 10-column last block, two stages
    (16, 2048, 4096),    # 16 x 8 blocks
    (13, 2048, 512),     # 16 x 8 blocks, one stage (K = 512)
    (16, 4000, 1536),    # 16 x 16 blocks, three stages
    (32, 2048, 8192),    # 32 x 8 blocks, two computing wavefronts of 16 rows
    (20, 1003, 1536),    # 32 x 8 blocks, 3-column last block, three stages
    (16, 8192, 2048),    # 16 x 32 blocks: three-slot rings keep the one-pass kernel
    (64, 2048, 2048),    # 32 x 16 blocks, two row blocks: likewise
    (3, 2048, 8320),     # K not a whole number of 8-step stages: the one-pass kernel
))
def test_skinny_loader_split_gives_identical_bits(tile_menu, dtype, m, n, k):
    """Blocks of up to 16 rows and 16 columns per computing wavefront run on loader wavefronts
    with fragments read three K-step pairs ahead when K is a whole number of 8-step stages; the
    stored rows keep the bits of entry 2, with and without a bias, of a call on the last row
    alone and of the automatic choice."""
    xc = randn(m, k, seed=5600 + m, dtype=dtype)
    wc = randn(n, k, seed=5601 + n, dtype=dtype, scale=0.05)
    bc = randn(n, seed=5602, dtype=dtype)
    x, w, bias = gpu(xc, wc, bc)
    assert tile_menu.biops_set_gemm_tile(2) == 0
    ref = matmul_persistent(x, w.t(), bias)
    ref_plain = matmul_persistent(x, w.t())
    assert tile_menu.biops_set_gemm_tile(SKINNY_ENTRY) == 0
    assert_bitwise(matmul_persistent(x, w.t(), bias), ref, "skinny entry")
    assert_bitwise(matmul_persistent(x, w.t()), ref_plain, "skinny entry, no bias")
    assert_bitwise(matmul_persistent(x[m - 1:], w.t(), bias), ref[m - 1:], "skinny entry, last row")
    assert tile_menu.biops_set_gemm_tile(-1) == 0
    assert_bitwise(matmul_persistent(x, w.t(), bias), ref, "automatic choice")
    absprod = oracle.gemm_abs(xc, wc.t()) + bc.double().abs()
    assert_gemm_close(ref, oracle.linear(xc, wc, bc), absprod, k)


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_skinny_loader_split_batched(tile_menu, dtype):
    """Batched skinny blocks (three products of 4 x 2048 x 2048, and a shared weight matrix)
    on the loader-split schedule keep the bits of entry 2."""
    a = gpu(randn(3, 4, 2048, seed=5610, dtype=dtype))
    b = gpu(randn(3, 2048, 2048, seed=5611, dtype=dtype) * 0.05)
    assert tile_menu.biops_set_gemm_tile(2) == 0
    ref = bmm_persistent(a, b)
    ref_shared = bmm_persistent(a, b[:1].expand(3, -1, -1))
    assert tile_menu.biops_set_gemm_tile(SKINNY_ENTRY) == 0
    assert_bitwise(bmm_persistent(a, b), ref, "skinny entry, batched")
    assert_bitwise(bmm_persistent(a, b[:1].expand(3, -1, -1)), ref_shared, "skinny entry, shared B")
    assert tile_menu.biops_set_gemm_tile(-1) == 0


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
@pytest.mark.parametrize(("m", "n", "k"), (
    (256, 2048, 2048),   # 8 row blocks x 32 blocks of 64 columns: one round
    (64, 8100, 1024),    # 2 x 127 blocks, 36-column last block (its third 16-column part stores 4)
    (256, 2000, 1024),   # 16-column last block: three of its four column parts store nothing
    (33, 16384, 1024),   # 2 x 256 blocks: more than one round, forced
    (512, 2048, 1024),   # 16-bit types: 8 x 32 blocks of 64 rows x 64 columns
    (128, 4096, 1024),   # 16-bit types: 2 x 128 blocks of 64 x 32
    (300, 3000, 1024),   # 16-bit types: 5 x 47 blocks of 64 x 64, partial last rows and columns
))
def test_skinny_64_column_blocks_give_identical_bits(tile_menu, dtype, m, n, k):
    """With at least two row blocks the skinny entry also takes 64-column blocks (and, for 16-bit
    types, 64-row blocks), their MFMA chains split over several computing wavefronts; rows keep
    the bits of entry 2, with and without a bias, and of a call on the last row alone.  The
    automatic choice takes them where they fit one round."""
    x = gpu(randn(m, k, seed=5500 + m, dtype=dtype))
    w = gpu(randn(n, k, seed=5501 + n, dtype=dtype) * 0.05)
    bias = gpu(randn(n, seed=5502, dtype=dtype))
    assert tile_menu.biops_set_gemm_tile(2) == 0
    ref = matmul_persistent(x, w.t(), bias)
    ref_plain = matmul_persistent(x, w.t())
    assert tile_menu.biops_set_gemm_tile(SKINNY_ENTRY) == 0
    assert_bitwise(matmul_persistent(x, w.t(), bias), ref, "skinny entry")
    assert_bitwise(matmul_persistent(x, w.t()), ref_plain, "skinny entry, no bias")
    assert_bitwise(matmul_persistent(x[m - 1:], w.t(), bias), ref[m - 1:], "skinny entry, last row")
    assert tile_menu.biops_set_gemm_tile(-1) == 0
    assert_bitwise(matmul_persistent(x, w.t(), bias), ref, "automatic choice")


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16, torch.float32))
@pytest.mark.parametrize(("m", "k", "n"), (
    (300, 2048, 520),   # N-major direct loads, partial last column tile
    (77, 1024, 256),
    (1, 64, 8),         # one chunk of columns
    (130, 128, 1000),   # N % 256 != 0: clamped chunks in the last tile
    (64, 4096, 24),
    (513, 192, 264),
    (40, 256, 100),     # N % 8 != 0: register path for 16-bit types, fp32 direct
    (33, 256, 98),      # N % 4 != 0: register path for every type
))
def test_nmajor_b_matches_kmajor_bits(tile_menu, dtype, m, k, n):
    """Row-major B (N-major: global->LDS loads and transposing LDS reads when whole 8-column
    chunks allow) gives the bits of the same values stored K-major, on every tile entry."""
    x = gpu(randn(m, k, seed=5100 + m, dtype=dtype))
    b_rows = gpu(randn(k, n, seed=5101 + n, dtype=dtype))
    b_cols = b_rows.t().contiguous().t()
    assert b_rows.stride(1) == 1 and b_cols.stride(0) == 1
    tile_menu.biops_set_gemm_tile(-1)
    ref = matmul_persistent(x, b_cols)
    for cfg in range(tile_menu.biops_gemm_tile_count()):
        assert tile_menu.biops_set_gemm_tile(cfg) == 0
        assert_bitwise(matmul_persistent(x, b_rows), ref, f"tile entry {cfg}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("rows", "cols", "ld", "offset", "rows_out", "cols_out"), (
    (5, 100, 100, 0, 5, 128),     # K tail only
    (7, 1001, 1003, 1, 9, 1024),  # odd pitch, misaligned base, extra zero rows
    (64, 64, 64, 0, 64, 64),      # nothing to pad: a plain copy
    (3, 1, 5, 2, 4, 32),          # one column
))
def test_pad_rows_is_a_zero_extended_copy(dtype, rows, cols, ld, offset, rows_out, cols_out):
    """biops_pad_rows copies [rows, cols] (row pitch ld) into [rows_out, cols_out] and writes
    zeros everywhere else, whatever the alignment of the source."""
    from batch_invariant_ops import _native as nat

    flat = randn(offset + rows * ld + 8, seed=5600 + cols, dtype=dtype)
    src = flat[offset:offset + rows * ld].view(rows, ld)[:, :cols]
    expect = torch.zeros(rows_out, cols_out, dtype=dtype)
    expect[:rows, :cols] = src
    dflat = gpu(flat)
    dst = torch.full((rows_out, cols_out), float("nan"), dtype=dtype, device="cuda")
    nat.call("biops_pad_rows", nat.dtype_code(dtype), rows, cols, dflat.data_ptr() + offset * flat.element_size(),
             ld, rows_out, cols_out, dst.data_ptr(), nat.stream_of(dst))
    assert_bitwise(dst.cpu(), expect, "padded copy")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("m", "k", "n", "layout"), (
    (300, 1000, 700, "w"),    # K % 64 != 0, rows 16-byte aligned
    (257, 2050, 515, "w"),    # K % 8 != 0: unaligned rows
    (64, 3000, 384, "rows"),  # row-major B: zero rows appended to B
    (96, 1027, 130, "rows"),  # row-major B with N % 8 != 0: padded row pitch
))
def test_padded_k_gives_the_register_path_bits(monkeypatch, dtype, m, k, n, layout):
    """Products whose K is not a whole number of 128-byte steps (or whose rows are not 16-byte
    aligned) run on zero-padded copies (biops_gemm_padded) when large enough and on the
    register load path otherwise; both give the same bits, so a row keeps its bits when the
    batch crosses the size at which the copies start (batch invariance), and the result stays
    within the GEMM bound of the oracle."""
    import batch_invariant_ops.batch_invariant_ops as bio

    x = gpu(randn(m, k, seed=5700 + k, dtype=dtype))
    w = gpu(randn(n, k, seed=5701 + n, dtype=dtype) * 0.05)
    b = w.t() if layout == "w" else w.t().contiguous()
    bias = gpu(randn(n, seed=5702, dtype=dtype))
    monkeypatch.setattr(bio, "_PAD_MIN_WORK", 1 << 62)
    reg = matmul_persistent(x, b, bias)
    one = matmul_persistent(x[m // 2:m // 2 + 1], b, bias)
    monkeypatch.setattr(bio, "_PAD_MIN_WORK", 0)
    monkeypatch.setattr(bio, "_PAD_MIN_K_BYTES", 0)
    monkeypatch.setattr(bio, "_PAD_MIN_MISALIGNED_K_BYTES", 0)
    assert bio._padded_workspace(x, b, m, n, k) > 0
    padded = matmul_persistent(x, b, bias)
    assert_bitwise(padded, reg, "padded vs register path")
    assert_bitwise(one, padded[m // 2:m // 2 + 1], "one row (register path) vs batch (padded)")
    if layout == "w":
        assert_bitwise(linear_batch_invariant(x, w, bias), reg, "linear shim")
    ref = oracle.linear(x.cpu(), w.cpu(), bias.cpu()).double()
    absprod = x.cpu().double().abs() @ w.cpu().double().abs().t() + bias.cpu().double().abs()
    assert_gemm_close(padded.cpu(), ref, absprod, k)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("batch", "m", "k", "n", "layout"), (
    (4, 100, 2050, 130, "cols"),   # unaligned rows, K-major B
    (3, 64, 1000, 256, "rows"),    # K % 64 != 0, row-major B
    (5, 40, 333, 72, "shared"),    # A shared by every batch element (stride 0): copied once
))
def test_bmm_padded_k_gives_the_register_path_bits(monkeypatch, dtype, batch, m, k, n, layout):
    """bmm_persistent through biops_bmm_padded (zero-padded copies of the batch's operands)
    gives the bits of the register load path, for one batch element alone as well, and stays
    within the GEMM bound of the oracle."""
    import batch_invariant_ops.batch_invariant_ops as bio

    if layout == "shared":
        a_cpu = randn(1, m, k, seed=5800 + k, dtype=dtype).expand(batch, m, k)
    else:
        a_cpu = randn(batch, m, k, seed=5800 + k, dtype=dtype)
    b_cpu = randn(batch, k, n, seed=5801 + n, dtype=dtype) * 0.05
    a = gpu(a_cpu.contiguous())[:1].expand(batch, m, k) if layout == "shared" else gpu(a_cpu)
    b = gpu(b_cpu).transpose(1, 2).contiguous().transpose(1, 2) if layout == "cols" else gpu(b_cpu)
    monkeypatch.setattr(bio, "_PAD_MIN_WORK", 1 << 62)
    reg = bmm_persistent(a, b)
    monkeypatch.setattr(bio, "_PAD_MIN_WORK", 0)
    monkeypatch.setattr(bio, "_PAD_MIN_K_BYTES", 0)
    monkeypatch.setattr(bio, "_PAD_MIN_MISALIGNED_K_BYTES", 0)
    assert bio._padded_workspace(a, b, m, n, k, batch) > 0
    padded = bmm_persistent(a, b)
    assert_bitwise(padded, reg, "padded vs register path")
    assert_bitwise(bmm_persistent(a[1:2], b[1:2]), reg[1:2], "one batch element")
    ref = oracle.bmm(a_cpu.contiguous(), b_cpu)
    assert_gemm_close(padded, ref, a_cpu.double().abs() @ b_cpu.double().abs(), k)
