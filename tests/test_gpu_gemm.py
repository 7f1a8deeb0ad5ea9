"""GPU parity: mm / bmm / addmm / matmul against the oracle.

Mirrors tests/test_{mm,bmm,addmm,matmul}.py of the reference (m, n, k in
[1, 1024], fp32 and fp16, bmm batch in [4, 16], addmm with gauss alpha/beta,
matmul batch in {None, 1, 2, 3}) with bf16, all four operand layouts, row
bias broadcast, every instantiation of the large-tile kernel, and the three
GEMM configs at full size (oracle on rows in every tile band, exact
small-integer checksums over every output element).

16-bit results are held to tests.helpers.assert_gemm_ulp: every element
within one ulp plus the fp32 summation bound of the exact value, and at most
1 % of elements off the correctly rounded value -- tight enough that a
dropped or repeated K slice fails.  fp32 results use the fp32 reduction
tolerance with an atol scaled by sqrt(k), the typical magnitude of a sum of
k unit-variance products."""

import random

import numpy as np
import pytest
import torch

import ntops_amd
from ntops_amd import _lib
from oracle import ops as O
from tests.helpers import DT_NAME, TOL_GEMM, assert_close, assert_gemm_ulp, from_np, tile_rows, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def rand_sizes():
    return [(random.randint(1, 1024), random.randint(1, 1024), random.randint(1, 1024), dt) for dt in DTYPES]


def expected16(m, n, k, layout, batch=1):
    """Family of the kernel that serves a 16-bit GEMM of fresh (16-byte
    aligned) operands in `layout` ("N" = row-major, "T" = transposed view):
    the matrix-core kernels need one unit-stride axis per operand with 8-element
    multiples, and an output with N % 4 == 0 (an N that would break either is
    rounded up to 8 columns by the wrapper, B copied N-major); products whose
    tiles would not fill the GPU split K."""
    if m == 1:  # a transposed (1, k) view keeps the row-major strides
        layout = "N" + layout[1]
    if layout[0] == "T" and m % 8 and m > 8 and n > 8 and k > 0:
        # an M-major A with M % 8 != 0 is copied row-major by the wrapper
        layout = "N" + layout[1]
    if k > 8 and k % 8 and (layout[0] == "N" or layout[1] == "T") and n > 0:
        # the wrapper zero-extends K to a multiple of 8, both operands copied
        # into fresh row-major tensors
        k, layout = (k + 7) // 8 * 8, "NN"
    if n > 8 and n % 8 and layout[1] == "N" and k > 0:
        # the wrapper runs the product at the width rounded up to 8 columns,
        # B copied into rows of that width (a K-major B runs as it is: the
        # kernels store rows of any width element by element)
        n, layout = (n + 7) // 8 * 8, layout[0] + "N"
    a_k = layout[0] == "N" and k % 8 == 0
    a_m = layout[0] == "T" and m % 8 == 0
    b_n = layout[1] == "N" and n % 8 == 0
    b_k = layout[1] == "T" and k % 8 == 0
    if k == 0 or not (a_k or a_m) or not (b_k or b_n):
        return "gemm_generic"
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tiles = -(-m // 128) * -(-n // 128) * batch
    few_tiles = tiles * 4 <= cus * 3
    if (batch == 1 and n % 4 == 0 and (m > 16 or not a_k) and k >= 1024 and few_tiles
            and min(2 * cus // tiles, k // 512) >= 2):
        return "gemm_mfma 128x128 "  # split K through the wrapper's workspace
    if a_k and (m <= 32 or (m <= 64 and few_tiles)):
        return "gemm_skinny "
    if k <= 128 and m % 128 == 0 and n % 128 == 0:
        return "gemm_panel "
    if -(-m // 256) * -(-n // 256) * batch >= 240 and k > 256:
        return "gemm_mfma 256x256 "
    return "gemm_mfma 128x128 "


def check(got, a, b, dtype, c=None, alpha=1.0, beta=0.0, what=""):
    """The oracle's result for (a, b[, c]): the ulp guard for 16-bit dtypes,
    rtol 1e-5 and atol 1e-5 * sqrt(k) for fp32 (unit-variance operands)."""
    dt = DT_NAME[dtype]
    if dt in ("bf16", "f16"):
        assert_gemm_ulp(got, a, b, dt, c, alpha, beta, what)
        return
    k = a.shape[-1]
    exp = from_np(O.gemm(to_np(a), to_np(b), dt, None if c is None else to_np(c), alpha, beta), dt)
    rtol, atol = TOL_GEMM[dt]
    assert_close(got, exp, rtol, atol * max(1.0, k**0.5), what)


@pytest.mark.parametrize("m, n, k, dtype", rand_sizes())
def test_mm(m, n, k, dtype):
    a = torch.randn(m, k).to(dtype)
    b = torch.randn(k, n).to(dtype)
    got = ntops_amd.torch.mm(a.cuda(), b.cuda())
    check(got, a, b, dtype, what="mm")


@pytest.mark.parametrize("layout", ("NN", "NT", "TN", "TT"))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("m, n, k", [(256, 512, 128), (300, 200, 72), (1000, 1024, 640), (8, 16, 24)])
def test_mm_layouts(m, n, k, dtype, layout):
    a = (0.1 * torch.randn(m, k)).to(dtype)
    b = (0.1 * torch.randn(k, n)).to(dtype)
    ag = a.cuda() if layout[0] == "N" else a.t().contiguous().cuda().t()
    bg = b.cuda() if layout[1] == "N" else b.t().contiguous().cuda().t()
    got = ntops_amd.torch.mm(ag, bg)
    assert _lib.last_kernel().startswith(expected16(m, n, k, layout))
    check(got, a, b, dtype, what=f"mm {layout}")


# The 256 x 256 tile kernel (>= 240 tiles, K > 256): every instantiation --
# bf16 and fp16, K-major or M-major A, N-major or K-major B, even edges
# (M, N multiples of 256, K of 32) and ragged ones (all three off that grid;
# multiples of 8 so that every layout qualifies) -- each as mm and as addmm
# with a row-broadcast bias and alpha, beta != 1.
TILE256 = {"even": (4096, 4352, 512), "ragged": (4104, 4112, 520)}


@pytest.mark.parametrize("edges", sorted(TILE256))
@pytest.mark.parametrize("layout", ("NN", "NT", "TN", "TT"))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_mm_256_tiles(dtype, layout, edges):
    m, n, k = TILE256[edges]
    g = torch.Generator().manual_seed(2 * ("NN", "NT", "TN", "TT").index(layout) + (edges == "ragged"))
    a = (0.1 * torch.randn(m, k, generator=g)).to(dtype)
    b = (0.1 * torch.randn(k, n, generator=g)).to(dtype)
    bias = torch.randn(n, generator=g).to(dtype)
    ag = a.cuda() if layout[0] == "N" else a.t().contiguous().cuda().t()
    bg = b.cuda() if layout[1] == "N" else b.t().contiguous().cuda().t()
    kernel = (f"gemm_mfma 256x256 s4 {'A:K' if layout[0] == 'N' else 'A:M'} "
              f"{'B:N' if layout[1] == 'N' else 'B:K'} {edges}")
    got = ntops_amd.torch.mm(ag, bg)
    assert _lib.last_kernel() == kernel
    check(got, a, b, dtype, what=f"mm 256 {layout} {edges}")
    got = ntops_amd.torch.addmm(bias.cuda(), ag, bg, beta=0.5, alpha=2.0)
    assert _lib.last_kernel() == kernel
    assert_gemm_ulp(got, a, b, DT_NAME[dtype], bias, 2.0, 0.5, f"addmm 256 {layout} {edges}", rows=tile_rows(m))


# Small M (decode shapes): the skinny kernel for a K-major A with either B
# layout -- M across 16-row blocks (1..4), 16-, 32- and 64-column slices
# (wide N), ragged N (multiples of 8 for an N-major B; any N for a K-major
# one) and K (not a multiple of the 32-wide step, shorter than one step per
# wave, longer than one load group), a bias, and small-M bmm.
SKINNY = [
    (1, 4096, 4096),
    (5, 1000, 40),
    (5, 1001, 40),
    (16, 24, 8),
    (17, 520, 1000),
    (33, 2048, 3000),
    (64, 136, 4104),
    (8, 8200, 100),
    (3, 16448, 40),
    (24, 16448, 520),
    (40, 8208, 72),
]


@pytest.mark.parametrize("layout", ("NN", "NT", "TN"))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("m, n, k", SKINNY)
def test_mm_small_m(m, n, k, dtype, layout):
    a = (0.1 * torch.randn(m, k)).to(dtype)
    b = (0.1 * torch.randn(k, n)).to(dtype)
    ag = a.cuda() if layout[0] == "N" else a.t().contiguous().cuda().t()
    bg = b.cuda() if layout[1] == "N" else b.t().contiguous().cuda().t()
    got = ntops_amd.torch.mm(ag, bg)
    assert _lib.last_kernel().startswith(expected16(m, n, k, layout))
    check(got, a, b, dtype, what=f"mm small m {layout}")


# N not a multiple of 8 (or of 4): the product runs at the padded width on
# the matrix cores (a vocabulary-sized projection among them), as mm, as
# addmm with a row bias and as bmm, every element against the oracle.
ODD_N = [(300, 1001, 256), (2048, 50257, 768), (40, 1003, 520), (512, 100, 1024), (256, 13, 512)]


@pytest.mark.parametrize("layout", ("NN", "NT"))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("m, n, k", ODD_N)
def test_mm_odd_n(m, n, k, dtype, layout):
    g = torch.Generator().manual_seed(m + n + k)
    a = (0.1 * torch.randn(m, k, generator=g)).to(dtype)
    b = (0.1 * torch.randn(k, n, generator=g)).to(dtype)
    bg = b.cuda() if layout[1] == "N" else b.t().contiguous().cuda().t()
    rows = tile_rows(m) if m > 1024 else list(range(m))
    got = ntops_amd.torch.mm(a.cuda(), bg)
    if dtype != torch.float32:
        assert _lib.last_kernel().startswith(expected16(m, n, k, "N" + layout[1])), _lib.last_kernel()
        assert not _lib.last_kernel().startswith("gemm_generic")
    check(got[rows], a[rows], b, dtype, what=f"mm odd n {layout}")
    bias = (0.1 * torch.randn(n, generator=g)).to(dtype)
    got = ntops_amd.torch.addmm(bias.cuda(), a.cuda(), bg, beta=0.5, alpha=2.0)
    check(got[rows], a[rows], b, dtype, c=bias.expand(len(rows), n), alpha=2.0, beta=0.5,
          what=f"addmm odd n {layout}")


@pytest.mark.parametrize("form", ("odd_row_stride", "column_major"))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("m, n, k", [(300, 264, 256), (1024, 1000, 512), (40, 129, 520), (600, 50257, 64)])
def test_gemm_ragged_output_through_the_c_abi(m, n, k, dtype, form):
    """Outputs the 4-column vector stores cannot take (a row stride of an odd
    element count at a 2-byte offset, a column-major view) and widths of any
    N, with a K-major B (F.linear's weight) and a bias row: the matrix-core
    kernels store them element by element; the bytes around the view stay
    untouched."""
    lib = _lib.load()
    g = torch.Generator().manual_seed(m + n + k)
    a = (0.1 * torch.randn(m, k, generator=g)).to(dtype)
    w = (0.1 * torch.randn(n, k, generator=g)).to(dtype)  # B = w.t(), K-major
    bias = (0.1 * torch.randn(n, generator=g)).to(dtype)
    ag, wg, biasg = a.cuda(), w.cuda(), bias.cuda()
    if form == "odd_row_stride":
        big = torch.zeros(m, n + 3, dtype=dtype, device="cuda")
        out, ostr = big[:, 1:1 + n], (0, n + 3, 1)
    else:
        big = torch.zeros(n, m + 2, dtype=dtype, device="cuda")
        out, ostr = big[:, :m].t(), (0, 1, m + 2)
    rc = lib.ntops_gemm(_lib.dtype_code(dtype), 1, m, n, k, ag.data_ptr(), _lib.i64_array((0, k, 1)),
                        wg.data_ptr(), _lib.i64_array((0, 1, k)), biasg.data_ptr(), _lib.i64_array((0, 0, 1)),
                        2.0, 0.5, out.data_ptr(), _lib.i64_array(ostr), _lib.stream_of(out))
    _lib.check(rc, "ntops_gemm ragged output")
    assert not _lib.last_kernel().startswith("gemm_generic"), _lib.last_kernel()
    torch.cuda.synchronize()
    if form == "odd_row_stride":
        assert big[:, 0].abs().sum() == 0 and big[:, 1 + n:].abs().sum() == 0
    else:
        assert big[:, m:].abs().sum() == 0
    rows = tile_rows(m) if m > 512 else list(range(m))
    check(out[rows], a[rows], w.t(), dtype, c=bias.expand(len(rows), n), alpha=2.0, beta=0.5,
          what=f"ragged output {form}")


@pytest.mark.parametrize("m, n, k, b_kmajor", [(4100, 4200, 512, False), (4100, 4200, 512, True),
                                              (4136, 4099, 320, True), (4096, 4360, 1024, False)])
def test_mm_even_interior_and_edge_strips(m, n, k, b_kmajor):
    """Large products whose M or N is not a multiple of 256: the even 256 x
    256 kernel on the interior, ragged 128 x 128 tiles on the right and bottom
    strips.  Small-integer operands make every fp32 sum exact, so each output
    equals the double-precision product rounded once to bf16; an addmm with a
    bias row is checked on sampled rows against the oracle."""
    g = torch.Generator().manual_seed(m + n + k)
    a = torch.randint(-8, 9, (m, k), generator=g).to(torch.bfloat16)
    b = torch.randint(-8, 9, (k, n), generator=g).to(torch.bfloat16)
    bg = b.cuda() if not b_kmajor else b.t().contiguous().cuda().t()
    got = ntops_amd.torch.mm(a.cuda(), bg)
    assert _lib.last_kernel().endswith("even+edges"), _lib.last_kernel()
    exp = (a.double() @ b.double()).float().bfloat16()
    assert torch.equal(got.cpu(), exp)
    bias = (0.1 * torch.randn(n, generator=g)).bfloat16()
    af, bf_ = (0.1 * torch.randn(m, k, generator=g)).bfloat16(), (0.1 * torch.randn(k, n, generator=g)).bfloat16()
    bfg = bf_.cuda() if not b_kmajor else bf_.t().contiguous().cuda().t()
    got = ntops_amd.torch.addmm(bias.cuda(), af.cuda(), bfg, beta=0.5, alpha=2.0)
    rows = tile_rows(m)
    check(got[rows], af[rows], bf_, torch.bfloat16, c=bias.expand(len(rows), n), alpha=2.0, beta=0.5,
          what="addmm interior + edges")


def test_bmm_even_interior_and_edge_strips():
    """A batch of products whose M and N are not multiples of 256: the
    interior and both strips of every batch member (the strips offset inside
    each member, the batch strides unchanged).  Exact small-integer sums."""
    g = torch.Generator().manual_seed(23)
    a = torch.randint(-8, 9, (4, 2100, 320), generator=g).to(torch.bfloat16)
    b = torch.randint(-8, 9, (4, 320, 2060), generator=g).to(torch.bfloat16)
    got = ntops_amd.torch.bmm(a.cuda(), b.cuda())
    assert _lib.last_kernel().endswith("even+edges"), _lib.last_kernel()
    assert torch.equal(got.cpu(), torch.bmm(a.double(), b.double()).float().bfloat16())


@pytest.mark.parametrize("m, n, k", [(2048, 16387, 320), (4100, 8195, 512)])
def test_mm_shifted_rows_exact(m, n, k):
    """Odd N with a K-major B (F.linear's weight): output rows start at every
    2-byte offset, so the full interior tiles store 16-byte chunks shifted to
    aligned addresses (plus element stores at each row segment's two ends)
    and the edge strips store element by element.  Small-integer operands:
    every output equals the double-precision product rounded once to bf16."""
    g = torch.Generator().manual_seed(m + n + k)
    a = torch.randint(-8, 9, (m, k), generator=g).to(torch.bfloat16)
    w = torch.randint(-8, 9, (n, k), generator=g).to(torch.bfloat16)
    got = ntops_amd.torch.mm(a.cuda(), w.cuda().t())
    assert _lib.last_kernel().endswith("even+edges"), _lib.last_kernel()
    assert torch.equal(got.cpu(), (a.double() @ w.double().t()).float().bfloat16())


def test_gemm_shifted_rows_full_tiles_through_the_c_abi():
    """A row stride of an odd element count over full 256 x 256 tiles (the
    even kernel alone) with a bias: shifted 16-byte stores everywhere; the
    bytes between the rows stay untouched."""
    lib = _lib.load()
    m, n, k = 4096, 4096, 384
    g = torch.Generator().manual_seed(17)
    a = torch.randint(-8, 9, (m, k), generator=g).to(torch.bfloat16)
    b = torch.randint(-8, 9, (k, n), generator=g).to(torch.bfloat16)
    bias = torch.randint(-8, 9, (n,), generator=g).to(torch.bfloat16)
    big = torch.zeros(m, n + 5, dtype=torch.bfloat16, device="cuda")
    out = big[:, 1:1 + n]
    ag, bg, biasg = a.cuda(), b.cuda(), bias.cuda()
    rc = lib.ntops_gemm(_lib.dtype_code(torch.bfloat16), 1, m, n, k, ag.data_ptr(), _lib.i64_array((0, k, 1)),
                        bg.data_ptr(), _lib.i64_array((0, n, 1)), biasg.data_ptr(), _lib.i64_array((0, 0, 1)),
                        1.0, 1.0, out.data_ptr(), _lib.i64_array((0, n + 5, 1)), _lib.stream_of(out))
    _lib.check(rc, "ntops_gemm shifted rows")
    assert _lib.last_kernel().startswith("gemm_mfma 256x256 s4 A:K B:N even"), _lib.last_kernel()
    torch.cuda.synchronize()
    assert big[:, 0].abs().sum() == 0 and big[:, 1 + n:].abs().sum() == 0
    exp = (a.double() @ b.double() + bias.double()).float().bfloat16()
    assert torch.equal(out.cpu(), exp)


# K not a multiple of 8 (or of 4): A's rows and B's columns zero-extended so
# the matrix cores take the product.
ODD_K = [(300, 256, 100), (1000, 1024, 1001), (40, 512, 77), (2048, 2048, 4095)]


@pytest.mark.parametrize("layout", ("NN", "NT", "TN"))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("m, n, k", ODD_K)
def test_mm_odd_k(m, n, k, dtype, layout):
    g = torch.Generator().manual_seed(m + 3 * n + k)
    a = (0.1 * torch.randn(m, k, generator=g)).to(dtype)
    b = (0.1 * torch.randn(k, n, generator=g)).to(dtype)
    ag = a.cuda() if layout[0] == "N" else a.t().contiguous().cuda().t()
    bg = b.cuda() if layout[1] == "N" else b.t().contiguous().cuda().t()
    rows = tile_rows(m) if m > 1024 else list(range(m))
    got = ntops_amd.torch.mm(ag, bg)
    if dtype != torch.float32:
        assert _lib.last_kernel().startswith(expected16(m, n, k, layout)), _lib.last_kernel()
    check(got[rows], a[rows], b, dtype, what=f"mm odd k {layout}")


# Operands in neither layout the matrix-core kernels read (an M-major A
# whose M is not a multiple of 8, fp32 A that is not K-major, views with no
# unit-stride axis or a start that is not 16-byte aligned) are copied
# row-major by the wrapper; the product leaves the generic kernel.
ODD_M = [(300, 256, 512), (1001, 1024, 768), (40, 512, 520), (2050, 4096, 1024)]


@pytest.mark.parametrize("layout", ("TN", "TT"))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("m, n, k", ODD_M)
def test_mm_m_major_odd_m(m, n, k, dtype, layout):
    g = torch.Generator().manual_seed(7 * m + n + k)
    a = (0.1 * torch.randn(m, k, generator=g)).to(dtype)
    b = (0.1 * torch.randn(k, n, generator=g)).to(dtype)
    ag = a.t().contiguous().cuda().t()
    bg = b.cuda() if layout[1] == "N" else b.t().contiguous().cuda().t()
    rows = tile_rows(m) if m > 1024 else list(range(m))
    got = ntops_amd.torch.mm(ag, bg)
    assert not _lib.last_kernel().startswith("gemm_generic"), _lib.last_kernel()
    if dtype != torch.float32:
        assert _lib.last_kernel().startswith(expected16(m, n, k, layout)), _lib.last_kernel()
    check(got[rows], a[rows], b, dtype, what=f"mm m-major odd m {layout}")
    bias = (0.1 * torch.randn(n, generator=g)).to(dtype)
    got = ntops_amd.torch.addmm(bias.cuda(), ag, bg, beta=0.5, alpha=2.0)
    assert not _lib.last_kernel().startswith("gemm_generic"), _lib.last_kernel()
    check(got[rows], a[rows], b, dtype, c=bias.expand(len(rows), n), alpha=2.0, beta=0.5,
          what=f"addmm m-major odd m {layout}")


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float32))
def test_mm_operands_without_a_kernel_layout(dtype):
    g = torch.Generator().manual_seed(11)
    big_a = (0.1 * torch.randn(600, 1100, generator=g)).to(dtype)
    big_b = (0.1 * torch.randn(520, 1040, generator=g)).to(dtype)
    odd_rows = big_a[:, :513].contiguous()
    views = {  # (A, B) as views of the tensors on each side
        "no unit stride": lambda x, y, z: (x[:300, :1024:2], y[:512, ::2]),
        "misaligned start": lambda x, y, z: (x[:300, 1:513], y[1:513, 3:515]),
        "row stride not a multiple of 8": lambda x, y, z: (z[:300, :512], y[:512, :513]),
    }
    dev = (big_a.cuda(), big_b.cuda(), odd_rows.cuda())
    for what, view in views.items():
        a, b = view(big_a, big_b, odd_rows)
        got = ntops_amd.torch.mm(*view(*dev))
        assert not _lib.last_kernel().startswith("gemm_generic"), (what, _lib.last_kernel())
        check(got, a, b, dtype, what=f"mm {what}")


def test_bmm_m_major_odd_m():
    g = torch.Generator().manual_seed(13)
    a = (0.1 * torch.randn(3, 264, 203, generator=g)).bfloat16()  # (batch, k, m): A = a^T is M-major
    b = (0.1 * torch.randn(3, 264, 256, generator=g)).bfloat16()
    got = ntops_amd.torch.bmm(a.cuda().transpose(1, 2), b.cuda())
    assert not _lib.last_kernel().startswith("gemm_generic"), _lib.last_kernel()
    for i in range(3):
        check(got[i], a[i].t(), b[i], torch.bfloat16, what="bmm m-major odd m")


# Products whose 128 x 128 tiles do not fill the GPU (few rows, long K:
# decode- and prefill-sized linear layers) split K through the wrappers'
# workspace: fp32 partial products summed in a fixed order.  Up to 16 rows
# a K-major A keeps the skinny kernel.
SPLIT_K = [(64, 4096, 4096), (128, 14336, 4096), (100, 1000, 8200), (48, 4096, 14336), (256, 1024, 2048),
           (17, 2048, 4096), (1, 4096, 14336), (16, 4096, 14336), (8, 14336, 4096), (3, 1000, 8200)]


@pytest.mark.parametrize("layout", ("NN", "NT", "TN"))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("m, n, k", SPLIT_K)
def test_mm_split_k(m, n, k, dtype, layout):
    g = torch.Generator().manual_seed(m + 5 * n + k)
    a = (0.1 * torch.randn(m, k, generator=g)).to(dtype)
    b = (0.1 * torch.randn(k, n, generator=g)).to(dtype)
    ag = a.cuda() if layout[0] == "N" else a.t().contiguous().cuda().t()
    bg = b.cuda() if layout[1] == "N" else b.t().contiguous().cuda().t()
    # (a K-major A of at most 16 rows takes the skinny kernel, an M-major A of
    # 2-7 rows the generic one; a transposed (1, k) view is K-major; fp32
    # splits only past the fp32 skinny kernel's 64 rows, where the workspace
    # query returns 0)
    a_kmajor = layout[0] == "N" or m == 1
    splits = (_lib.load().ntops_gemm_workspace(_lib.dtype_code(dtype), 1, m, n, k) > 0
              and (m > 16 or not a_kmajor) and not (layout[0] == "T" and 1 < m < 8))
    got = ntops_amd.torch.mm(ag, bg)
    kern = _lib.last_kernel()
    assert ("splitk" in kern) == splits, kern
    check(got, a, b, dtype, what=f"mm split-k {layout} [{kern}]")
    again = ntops_amd.torch.mm(ag, bg)
    assert torch.equal(got, again), "split-K result depends on the run"
    bias = (0.1 * torch.randn(n, generator=g)).to(dtype)
    got = ntops_amd.torch.addmm(bias.cuda(), ag, bg, beta=0.5, alpha=2.0)
    check(got, a, b, dtype, c=bias.expand(m, n), alpha=2.0, beta=0.5, what=f"addmm split-k {layout}")
    cfull = (0.1 * torch.randn(m, n, generator=g)).to(dtype)
    got = ntops_amd.torch.addmm(cfull.cuda(), ag, bg, beta=-1.5, alpha=0.5)
    check(got, a, b, dtype, c=cfull, alpha=0.5, beta=-1.5, what=f"addmm split-k full C {layout}")


def test_gemm_split_k_through_the_c_abi():
    """ntops_gemm_ws with the workspace ntops_gemm_workspace asks for, with a
    workspace one byte short (then it runs unsplit), and with none; strided
    output rows."""
    lib = _lib.load()
    m, n, k = 96, 2048, 6144
    g = torch.Generator().manual_seed(3)
    a = (0.1 * torch.randn(m, k, generator=g)).bfloat16()
    b = (0.1 * torch.randn(k, n, generator=g)).bfloat16()
    ag, bg = a.cuda(), b.cuda()
    need = lib.ntops_gemm_workspace(_lib.dtype_code(torch.bfloat16), 1, m, n, k)
    assert need > 0
    outs = []
    for size, expect in ((need, True), (need - 1, False), (0, False)):
        big = torch.zeros(m, n + 64, dtype=torch.bfloat16, device="cuda")
        out = big[:, 32:32 + n]
        ws = torch.empty(max(size, 1), dtype=torch.uint8, device="cuda")
        rc = lib.ntops_gemm_ws(_lib.dtype_code(torch.bfloat16), 1, m, n, k,
                               ag.data_ptr(), _lib.i64_array((0, k, 1)), bg.data_ptr(), _lib.i64_array((0, n, 1)),
                               None, None, 1.0, 0.0, out.data_ptr(), _lib.i64_array((0, n + 64, 1)),
                               ws.data_ptr() if size else None, size, _lib.stream_of(out))
        _lib.check(rc, "ntops_gemm_ws")
        assert ("splitk" in _lib.last_kernel()) == expect, _lib.last_kernel()
        torch.cuda.synchronize()
        assert big[:, :32].abs().sum() == 0 and big[:, 32 + n:].abs().sum() == 0
        check(out, a, b, torch.bfloat16, what=f"ntops_gemm_ws {size}")
        outs.append(out.clone())


def test_bmm_odd_n():
    g = torch.Generator().manual_seed(5)
    a = (0.1 * torch.randn(3, 200, 264, generator=g)).bfloat16()
    b = (0.1 * torch.randn(3, 264, 203, generator=g)).bfloat16()
    got = ntops_amd.torch.bmm(a.cuda(), b.cuda())
    assert not _lib.last_kernel().startswith("gemm_generic"), _lib.last_kernel()
    for i in range(3):
        check(got[i], a[i], b[i], torch.bfloat16, what="bmm odd n")


@pytest.mark.parametrize("layout", ("NN", "NT", "TN"))
@pytest.mark.parametrize("m, n, k", SKINNY)
def test_mm_small_m_f32(m, n, k, layout):
    """fp32 with few rows: the fp32 skinny kernel (IEEE fp32 MFMA products,
    fp32 accumulation) against the oracle at the fp32 GEMM tolerance."""
    a = torch.randn(m, k)
    b = torch.randn(k, n)
    ag = a.cuda() if layout[0] == "N" else a.t().contiguous().cuda().t()
    bg = b.cuda() if layout[1] == "N" else b.t().contiguous().cuda().t()
    got = ntops_amd.torch.mm(ag, bg)
    check(got, a, b, torch.float32, what=f"mm f32 small m {layout}")


@pytest.mark.parametrize("layout", ("NN", "NT", "TN"))
@pytest.mark.parametrize("m, n, k", [(256, 512, 128), (300, 200, 72), (1000, 1024, 640), (130, 1000, 4), (65, 129, 1028),
                                     (1100, 260, 132), (1024, 384, 36), (2048, 132, 2052)])
def test_mm_f32_tiles(m, n, k, layout):
    """fp32 beyond the skinny rows: the LDS-tiled fp32 MFMA kernel (K-major
    A; B either way), partial tiles at every edge, K tails of 4-28."""
    a = torch.randn(m, k)
    b = torch.randn(k, n)
    ag = a.cuda() if layout[0] == "N" else a.t().contiguous().cuda().t()
    bg = b.cuda() if layout[1] == "N" else b.t().contiguous().cuda().t()
    got = ntops_amd.torch.mm(ag, bg)
    assert _lib.last_kernel().startswith(f32_expected_kernel(m, n, k, layout[1] == "T"))
    check(got, a, b, torch.float32, what=f"mm f32 tiles {layout}")


def f32_expected_kernel(m, n, k, b_kmajor):
    """The fp32 tile kernel a 2-D product takes.  An N-major B whose N is not
    a multiple of 4 is copied by the wrapper into rows padded to a multiple of
    4 (a K-major B runs as it is); products whose tiles leave CUs idle split K
    when the workspace query says so."""
    bl = "B:K" if b_kmajor else "B:N"
    np_ = n if b_kmajor else -(-n // 4) * 4
    if _lib.load().ntops_gemm_workspace(_lib.dtype_code(torch.float32), 1, m, np_, k) > 0:
        return f"gemm_f32_lds m128 {bl} splitk"
    return f32_tile_kernel(m, np_, 1, bl)


def f32_tile_kernel(m, n, batch, bl):
    """Unsplit fp32 tile kernel: when 128 x 128 tiles fill every CU (and
    there are more than 64 rows) the LDS kernel's 128-row blocks, or the
    LDS-free kernel for an N-major B with three or more tiles per CU; else
    the LDS kernel's 64-row blocks."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tiles = -(-m // 128) * -(-n // 128) * batch
    if m > 64 and tiles >= cus:
        return "gemm_f32_reg B:N" if bl == "B:N" and tiles >= 3 * cus else f"gemm_f32_lds m128 {bl}"
    return f"gemm_f32_lds m64 {bl}"


@pytest.mark.parametrize("m, n, k, bt", [(4096, 4096, 36, False), (4096, 4096, 36, True), (2048, 2048, 100, False),
                                         (2048, 2048, 100, True), (200, 300, 68, False), (200, 300, 68, True),
                                         (512, 1024, 1000, False), (512, 1024, 1000, True)])
def test_mm_f32_tiles_exact_sums(m, n, k, bt):
    """Small-integer operands: every product and partial sum is exact in
    fp32, so every output of each fp32 tile kernel (LDS blocks of 64 and 128
    rows, the LDS-free kernel, K split in slices of 160) must equal the
    integer product (catches a lost, doubled or misplaced k chunk, slice, row
    or column)."""
    g = torch.Generator().manual_seed(5)
    a = torch.randint(-8, 9, (m, k), generator=g).float()
    b = torch.randint(-8, 9, (k, n), generator=g).float()
    bg = b.cuda() if not bt else b.t().contiguous().cuda().t()
    got = ntops_amd.torch.mm(a.cuda(), bg)
    assert _lib.last_kernel().startswith(f32_expected_kernel(m, n, k, bt))
    exp = (a.double() @ b.double()).float()
    assert torch.equal(got.cpu(), exp)


def test_addmm_and_bmm_f32_tiles():
    bias = torch.randn(300)
    x = torch.randn(200, 96)
    y = torch.randn(96, 300)
    got = ntops_amd.torch.addmm(bias.cuda(), x.cuda(), y.cuda(), beta=0.5, alpha=2.0)
    exp = from_np(O.gemm(to_np(x), to_np(y), "f32", to_np(bias), 2.0, 0.5), "f32")
    assert_close(got, exp, 1e-5, 1e-5 * 96**0.5, "addmm f32 tiles")
    a = torch.randn(3, 130, 64)
    b = torch.randn(3, 64, 260)
    got = ntops_amd.torch.bmm(a.cuda(), b.cuda())
    assert_close(got, from_np(O.gemm(to_np(a), to_np(b), "f32"), "f32"), 1e-5, 1e-5 * 8, "bmm f32 tiles")
    a = torch.randn(3, 1030, 64)
    b = torch.randn(3, 64, 260)
    got = ntops_amd.torch.bmm(a.cuda(), b.cuda())
    assert _lib.last_kernel() == f32_tile_kernel(1030, 260, 3, "B:N")
    assert_close(got, from_np(O.gemm(to_np(a), to_np(b), "f32"), "f32"), 1e-5, 1e-5 * 8, "bmm f32 batched tiles")
    g = torch.Generator().manual_seed(11)  # a batch filling the GPU three times over: the LDS-free kernel
    a = torch.randint(-8, 9, (8, 1024, 68), generator=g).float()
    b = torch.randint(-8, 9, (8, 68, 1536), generator=g).float()
    got = ntops_amd.torch.bmm(a.cuda(), b.cuda())
    assert _lib.last_kernel() == f32_tile_kernel(1024, 1536, 8, "B:N")
    assert torch.equal(got.cpu(), torch.bmm(a.double(), b.double()).float()), "bmm f32 exact sums"
    a = torch.randn(5, 40, 72)  # a batch of few-row products: the skinny kernel
    b = torch.randn(5, 72, 200)
    got = ntops_amd.torch.bmm(a.cuda(), b.cuda())
    assert _lib.last_kernel().startswith("gemm_skinny_f32 "), _lib.last_kernel()
    assert_close(got, from_np(O.gemm(to_np(a), to_np(b), "f32"), "f32"), 1e-5, 1e-5 * 9, "bmm f32 few rows")


def test_addmm_and_bmm_small_m():
    bias = torch.randn(1000).bfloat16()
    x = (0.1 * torch.randn(7, 512)).bfloat16()
    w = (0.1 * torch.randn(1000, 512)).bfloat16()  # F.linear-style weight: B = w.t() is K-major
    got = ntops_amd.torch.addmm(bias.cuda(), x.cuda(), w.cuda().t(), beta=0.5, alpha=2.0)
    assert _lib.last_kernel().startswith("gemm_skinny ")
    check(got, x, w.t().contiguous(), torch.bfloat16, bias, 2.0, 0.5, "addmm small m")
    q = (0.1 * torch.randn(12, 1, 128)).bfloat16()
    kt = (0.1 * torch.randn(12, 128, 777 + 7)).bfloat16()
    got = ntops_amd.torch.bmm(q.cuda(), kt.cuda())
    check(got, q, kt, torch.bfloat16, what="bmm small m")


def test_mm_small_integers_exact():
    """Small-integer bf16 operands: fp32 accumulation is exact and the result
    is representable, so the kernel must match integer matmul exactly."""
    for m, n, k in ((512, 512, 64), (256, 768, 128)):
        a = torch.randint(-2, 3, (m, k)).to(torch.bfloat16)
        b = torch.randint(-2, 3, (k, n)).to(torch.bfloat16)
        got = ntops_amd.torch.mm(a.cuda(), b.cuda()).cpu()
        exact = (a.to(torch.int64) @ b.to(torch.int64)).to(torch.bfloat16)
        assert torch.equal(got, exact)


@pytest.mark.parametrize("m, n, k, dtype", rand_sizes())
def test_bmm(m, n, k, dtype):
    bsz = random.randint(4, 16)
    a = torch.randn(bsz, m, k).to(dtype)
    b = torch.randn(bsz, k, n).to(dtype)
    got = ntops_amd.torch.bmm(a.cuda(), b.cuda())
    check(got, a, b, dtype, what="bmm")


@pytest.mark.parametrize("m, n, k, dtype", rand_sizes())
def test_addmm(m, n, k, dtype):
    inp = torch.randn(m, n).to(dtype)
    x = torch.randn(m, k).to(dtype)
    y = torch.randn(k, n).to(dtype)
    beta, alpha = random.gauss(0, 1), random.gauss(0, 1)
    got = ntops_amd.torch.addmm(inp.cuda(), x.cuda(), y.cuda(), beta=beta, alpha=alpha)
    check(got, x, y, dtype, inp, alpha, beta, "addmm")


@pytest.mark.parametrize("dtype", DTYPES)
def test_addmm_bias_and_beta_zero(dtype):
    m, n, k = 200, 136, 96
    bias = torch.randn(n).to(dtype)
    x = (0.1 * torch.randn(m, k)).to(dtype)
    y = (0.1 * torch.randn(k, n)).to(dtype)
    dt = DT_NAME[dtype]
    got = ntops_amd.torch.addmm(bias.cuda(), x.cuda(), y.cuda())
    check(got, x, y, dtype, bias, 1.0, 1.0, "bias")
    nan_c = torch.full((m, n), float("nan"), dtype=dtype)
    got = ntops_amd.torch.addmm(nan_c.cuda(), x.cuda(), y.cuda(), beta=0, alpha=2)
    assert not torch.isnan(got).any()
    check(got, x, y, dtype, None, 2.0, 0.0, "beta=0")


# Every form of addmm's C operand reaches its own epilogue access: a row bias
# and a full contiguous C are read 4 columns per 8-byte load, a transposed or
# misaligned C element by element, a column (or scalar) C once per row --
# on the 128 x 128 kernel with staged and direct stores and on the 256 x 256
# kernel with ragged edges.
C_FORMS = ("row_bias", "full", "transposed", "column", "scalar", "misaligned")
# "direct": the output is a view 8 bytes past a 16-byte boundary, which the
# staged (16-byte) stores cannot serve
C_SHAPES = {"128 staged": (200, 136, 96), "128 direct": (200, 136, 96), "256 ragged": (4104, 4112, 520)}


def c_operand(form, m, n, dtype, g):
    """(CPU C in the oracle's broadcastable form, GPU C as addmm receives it)."""
    if form == "row_bias":
        c = torch.randn(n, generator=g).to(dtype)
        return c, c.cuda()
    if form == "column":
        c = torch.randn(m, 1, generator=g).to(dtype)
        return c, c.cuda()
    if form == "scalar":
        c = torch.randn(1, 1, generator=g).to(dtype)
        return c, c.cuda()
    c = torch.randn(m, n, generator=g).to(dtype)
    if form == "full":
        return c, c.cuda()
    if form == "transposed":
        return c, c.t().contiguous().cuda().t()
    buf = torch.empty(m * n + 1, dtype=dtype, device="cuda")
    cg = buf[1:].view(m, n)
    cg.copy_(c.cuda())
    assert cg.data_ptr() % 8 != 0
    return c, cg


@pytest.mark.parametrize("shape", sorted(C_SHAPES))
@pytest.mark.parametrize("form", C_FORMS)
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_addmm_c_forms(dtype, form, shape):
    m, n, k = C_SHAPES[shape]
    g = torch.Generator().manual_seed(C_FORMS.index(form) * 7 + sorted(C_SHAPES).index(shape))
    a = (0.1 * torch.randn(m, k, generator=g)).to(dtype)
    b = (0.1 * torch.randn(k, n, generator=g)).to(dtype)
    c, cg = c_operand(form, m, n, dtype, g)
    out = None
    if shape.endswith("direct"):
        out = torch.empty(m * n + 4, dtype=dtype, device="cuda")[4:].view(m, n)
        assert out.data_ptr() % 16 == 8
    got = ntops_amd.torch.addmm(cg, a.cuda(), b.cuda(), beta=0.75, alpha=1.5, out=out)
    assert _lib.last_kernel().startswith("gemm_mfma " + shape.split()[0])
    rows = tile_rows(m) if m > 1024 else None
    assert_gemm_ulp(got, a, b, DT_NAME[dtype], c, 1.5, 0.75, f"addmm C {form} {shape}", rows=rows)


# Short-K shapes (K <= 128, M and N multiples of 128): the persistent panel
# kernel.  Tile counts below, at and above one block per CU, divisible by 8
# or not (XCD remap on / off), K below the 128-wide panel (zero-filled tail),
# all four operand layouts, units of several tiles (one operand panel reused
# across them), and an addmm bias read in its epilogue.
SHORT_K = [
    (1, 128, 128, 8),
    (3, 384, 256, 64),
    (7, 384, 640, 120),
    (11, 640, 640, 128),
    (5, 1024, 896, 96),
    (2, 2048, 2048, 128),
    (4, 2048, 2048, 64),
]


@pytest.mark.parametrize("layout", ("NN", "NT", "TN", "TT"))
@pytest.mark.parametrize("bsz, m, n, k", SHORT_K)
def test_bmm_short_k(bsz, m, n, k, layout):
    dtype = torch.bfloat16 if (bsz + k) % 2 else torch.float16
    a = (0.1 * torch.randn(bsz, m, k)).to(dtype)
    b = (0.1 * torch.randn(bsz, k, n)).to(dtype)
    ag = a.cuda() if layout[0] == "N" else a.transpose(1, 2).contiguous().cuda().transpose(1, 2)
    bg = b.cuda() if layout[1] == "N" else b.transpose(1, 2).contiguous().cuda().transpose(1, 2)
    got = ntops_amd.torch.bmm(ag, bg)
    assert _lib.last_kernel().startswith("gemm_panel ")
    check(got, a, b, dtype, what=f"bmm short-k {layout}")


def test_addmm_short_k_bias():
    m, n, k = 512, 768, 64
    bias = torch.randn(n).bfloat16()
    x = (0.1 * torch.randn(m, k)).bfloat16()
    y = (0.1 * torch.randn(k, n)).bfloat16()
    got = ntops_amd.torch.addmm(bias.cuda(), x.cuda(), y.cuda(), beta=0.5, alpha=2.0)
    assert _lib.last_kernel().startswith("gemm_panel ")
    check(got, x, y, torch.bfloat16, bias, 2.0, 0.5, "addmm short-k bias")


def test_gemm_k_zero_strided_views():
    """K == 0 through operand views whose strides would select the MFMA
    layouts: the result is beta * C (zeros for mm)."""
    big_a = torch.randn(256, 64).bfloat16().cuda()
    big_b = torch.randn(64, 512).bfloat16().cuda()
    a, b = big_a[:, :0], big_b[:0, :]
    got = ntops_amd.torch.mm(a, b)
    assert got.shape == (256, 512) and (got == 0).all()
    bias = torch.randn(512).bfloat16()
    got = ntops_amd.torch.addmm(bias.cuda(), a, b, beta=2.0)
    assert torch.equal(got.cpu(), (2.0 * bias.float()).bfloat16().expand(256, 512))


@pytest.mark.parametrize("b", (None, 1, 2, 3))
@pytest.mark.parametrize("m, n, k, dtype", rand_sizes())
def test_matmul(b, m, n, k, dtype):
    a_shape = (b, m, k) if b is not None else (m, k)
    o_shape = (b, k, n) if b is not None else (k, n)
    a = torch.randn(a_shape).to(dtype)
    o = torch.randn(o_shape).to(dtype)
    got = ntops_amd.torch.matmul(a.cuda(), o.cuda())
    check(got, a, o, dtype, what="matmul")
    if b is not None:
        got = ntops_amd.torch.matmul(a[0].cuda(), o.cuda())  # broadcast batch
        check(got, a[0].expand(b, m, k), o, dtype, what="bcast")


def _config_mm():
    g = torch.Generator().manual_seed(0)
    a = (0.02 * torch.randn(8192, 4096, generator=g)).bfloat16()
    b = (0.02 * torch.randn(4096, 14336, generator=g)).bfloat16()
    bias = (0.02 * torch.randn(14336, generator=g)).bfloat16()
    return a, b, bias


CONFIG_KERNEL = "gemm_mfma 256x256 s4 A:K B:N even"


def test_mm_and_addmm_config_full_size():
    """bf16 (8192 x 4096) . (4096 x 14336), fp32 accumulation; addmm with a
    (14336,) bias, beta = alpha = 1: the ulp guard on two rows of every
    256-row tile band (all columns, so every output tile is checked)."""
    a, b, bias = _config_mm()
    ag, bg = a.cuda(), b.cuda()
    rows = tile_rows(8192)
    got = ntops_amd.torch.mm(ag, bg)
    assert _lib.last_kernel() == CONFIG_KERNEL
    assert_gemm_ulp(got, a, b, "bf16", what="mm config", rows=rows)
    del got
    got = ntops_amd.torch.addmm(bias.cuda(), ag, bg)
    assert _lib.last_kernel() == CONFIG_KERNEL
    assert_gemm_ulp(got, a, b, "bf16", bias, 1.0, 1.0, "addmm config", rows=rows)


def _bf16_rounding_bound(r):
    """Per-element bound on |bf16(v) - v| for integer v, given r = bf16(v) in
    float64: 0 where |r| <= 256 (integers are exact there), else half an
    ulp at |r|."""
    e = torch.floor(torch.log2(r.abs().clamp_min(1.0)))
    return torch.where(r.abs() > 256, 0.5 * torch.exp2(e - 7), torch.zeros_like(r))


def test_mm_config_exact_small_integers():
    """The mm / addmm config shapes with operands in {-1, 0, 1} and an integer
    bias: fp32 accumulation is exact, so every output is bf16(exact integer).
    Rows in every tile band must match the oracle bit for bit, and the row
    and column sums of ALL outputs must equal those of the exact product to
    within the rounding of the few outputs above 256 -- a dropped, repeated or
    misplaced K slice or tile anywhere changes them."""
    g = torch.Generator().manual_seed(1)
    a = torch.randint(-1, 2, (8192, 4096), generator=g).bfloat16()
    b = torch.randint(-1, 2, (4096, 14336), generator=g).bfloat16()
    bias = torch.randint(-2, 3, (14336,), generator=g).bfloat16()
    ad, bd = a.double(), b.double()
    rows = tile_rows(8192)
    exact_rows = ad @ bd.sum(1)
    exact_cols = ad.sum(0) @ bd
    for name, c in (("mm", None), ("addmm", bias)):
        if c is None:
            got = ntops_amd.torch.mm(a.cuda(), b.cuda())
        else:
            got = ntops_amd.torch.addmm(c.cuda(), a.cuda(), b.cuda())
        assert _lib.last_kernel() == CONFIG_KERNEL
        exp = from_np(O.gemm(to_np(a[rows]), to_np(b), "bf16", None if c is None else to_np(c), 1.0, 1.0), "bf16")
        assert torch.equal(got[torch.tensor(rows).cuda()].cpu(), exp), f"{name}: tile-band rows differ"
        r = got.double()
        slack = _bf16_rounding_bound(r)
        er = exact_rows + (0.0 if c is None else c.double().sum())
        ec = exact_cols + (0.0 if c is None else 8192 * c.double())
        dr = (r.sum(1).cpu() - er).abs()
        dc = (r.sum(0).cpu() - ec).abs()
        assert (dr <= slack.sum(1).cpu()).all(), f"{name}: row sums off in {(dr > slack.sum(1).cpu()).sum()} rows"
        assert (dc <= slack.sum(0).cpu()).all(), f"{name}: column sums off in {(dc > slack.sum(0).cpu()).sum()} cols"
        del got, r, slack


def test_bmm_config_full_size():
    """bf16 (32, 2048 x 128) . (32, 128 x 2048): every element vs the oracle."""
    g = torch.Generator().manual_seed(0)
    a = (0.02 * torch.randn(32, 2048, 128, generator=g)).bfloat16()
    b = (0.02 * torch.randn(32, 128, 2048, generator=g)).bfloat16()
    got = ntops_amd.torch.bmm(a.cuda(), b.cuda())
    assert _lib.last_kernel().startswith("gemm_panel A:K B:N")
    for i in range(0, 32, 4):
        assert_gemm_ulp(got[i : i + 4], a[i : i + 4], b[i : i + 4], "bf16", what=f"bmm batch {i}")
