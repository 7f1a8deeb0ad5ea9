"""GPU parity: mm / bmm / addmm / matmul against the oracle.

Mirrors tests/test_{mm,bmm,addmm,matmul}.py of the reference (m, n, k in
[1, 1024], fp32 and fp16, bmm batch in [4, 16], addmm with gauss alpha/beta,
matmul batch in {None, 1, 2, 3}) with bf16, all four operand layouts, row
bias broadcast, and the three GEMM configs at full size (oracle on sampled
rows plus a checksum over every output element)."""

import random

import numpy as np
import pytest
import torch

import ntops_amd
from oracle import ops as O
from tests.helpers import DT_NAME, TOL_GEMM, assert_close, from_np, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def rand_sizes():
    return [(random.randint(1, 1024), random.randint(1, 1024), random.randint(1, 1024), dt) for dt in DTYPES]


def tol(dtype, k):
    rtol, atol = TOL_GEMM[DT_NAME[dtype]]
    return rtol, atol


@pytest.mark.parametrize("m, n, k, dtype", rand_sizes())
def test_mm(m, n, k, dtype):
    a = torch.randn(m, k).to(dtype)
    b = torch.randn(k, n).to(dtype)
    got = ntops_amd.torch.mm(a.cuda(), b.cuda())
    dt = DT_NAME[dtype]
    exp = from_np(O.gemm(to_np(a), to_np(b), dt), dt)
    # randn operands: |c| ~ sqrt(k); scale atol with it
    rtol, atol = tol(dtype, k)
    assert_close(got, exp, rtol, atol * max(1.0, k**0.5), "mm")


@pytest.mark.parametrize("layout", ("NN", "NT", "TN", "TT"))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("m, n, k", [(256, 512, 128), (300, 200, 72), (1000, 1024, 640), (8, 16, 24)])
def test_mm_layouts(m, n, k, dtype, layout):
    a = (0.1 * torch.randn(m, k)).to(dtype)
    b = (0.1 * torch.randn(k, n)).to(dtype)
    ag = a.cuda() if layout[0] == "N" else a.t().contiguous().cuda().t()
    bg = b.cuda() if layout[1] == "N" else b.t().contiguous().cuda().t()
    got = ntops_amd.torch.mm(ag, bg)
    dt = DT_NAME[dtype]
    assert_close(got, from_np(O.gemm(to_np(a), to_np(b), dt), dt), 1.6e-2, 1.6e-2, f"mm {layout}")


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
    dt = DT_NAME[dtype]
    assert_close(got, from_np(O.gemm(to_np(a), to_np(b), dt), dt), 1.6e-2, 1.6e-2 * max(1.0, (k / 100) ** 0.5),
                 f"mm small m {layout}")


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
    rtol, atol = tol(torch.float32, k)
    assert_close(got, from_np(O.gemm(to_np(a), to_np(b), "f32"), "f32"), rtol, atol * max(1.0, k**0.5),
                 f"mm f32 small m {layout}")


@pytest.mark.parametrize("layout", ("NN", "NT", "TN"))
@pytest.mark.parametrize("m, n, k", [(256, 512, 128), (300, 200, 72), (1000, 1024, 640), (130, 1000, 4), (65, 129, 1028)])
def test_mm_f32_tiles(m, n, k, layout):
    """fp32 beyond the skinny rows: the LDS-free fp32 MFMA tile kernel
    (K-major A; B either way), partial 64 x 64 wave tiles at every edge."""
    a = torch.randn(m, k)
    b = torch.randn(k, n)
    ag = a.cuda() if layout[0] == "N" else a.t().contiguous().cuda().t()
    bg = b.cuda() if layout[1] == "N" else b.t().contiguous().cuda().t()
    got = ntops_amd.torch.mm(ag, bg)
    rtol, atol = tol(torch.float32, k)
    assert_close(got, from_np(O.gemm(to_np(a), to_np(b), "f32"), "f32"), rtol, atol * max(1.0, k**0.5),
                 f"mm f32 tiles {layout}")


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


def test_addmm_and_bmm_small_m():
    bias = torch.randn(1000).bfloat16()
    x = (0.1 * torch.randn(7, 512)).bfloat16()
    w = (0.1 * torch.randn(1000, 512)).bfloat16()  # F.linear-style weight: B = w.t() is K-major
    got = ntops_amd.torch.addmm(bias.cuda(), x.cuda(), w.cuda().t(), beta=0.5, alpha=2.0)
    exp = from_np(O.gemm(to_np(x), to_np(w.t().contiguous()), "bf16", to_np(bias), 2.0, 0.5), "bf16")
    assert_close(got, exp, 1.6e-2, 1.6e-2, "addmm small m")
    q = (0.1 * torch.randn(12, 1, 128)).bfloat16()
    kt = (0.1 * torch.randn(12, 128, 777 + 7)).bfloat16()
    got = ntops_amd.torch.bmm(q.cuda(), kt.cuda())
    assert_close(got, from_np(O.gemm(to_np(q), to_np(kt), "bf16"), "bf16"), 1.6e-2, 1.6e-2, "bmm small m")


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
    dt = DT_NAME[dtype]
    rtol, atol = tol(dtype, k)
    assert_close(got, from_np(O.gemm(to_np(a), to_np(b), dt), dt), rtol, atol * max(1.0, k**0.5), "bmm")


@pytest.mark.parametrize("m, n, k, dtype", rand_sizes())
def test_addmm(m, n, k, dtype):
    inp = torch.randn(m, n).to(dtype)
    x = torch.randn(m, k).to(dtype)
    y = torch.randn(k, n).to(dtype)
    beta, alpha = random.gauss(0, 1), random.gauss(0, 1)
    got = ntops_amd.torch.addmm(inp.cuda(), x.cuda(), y.cuda(), beta=beta, alpha=alpha)
    dt = DT_NAME[dtype]
    exp = from_np(O.gemm(to_np(x), to_np(y), dt, to_np(inp), alpha, beta), dt)
    rtol, atol = tol(dtype, k)
    assert_close(got, exp, rtol, atol * max(1.0, k**0.5), "addmm")


@pytest.mark.parametrize("dtype", DTYPES)
def test_addmm_bias_and_beta_zero(dtype):
    m, n, k = 200, 136, 96
    bias = torch.randn(n).to(dtype)
    x = (0.1 * torch.randn(m, k)).to(dtype)
    y = (0.1 * torch.randn(k, n)).to(dtype)
    dt = DT_NAME[dtype]
    got = ntops_amd.torch.addmm(bias.cuda(), x.cuda(), y.cuda())
    assert_close(got, from_np(O.gemm(to_np(x), to_np(y), dt, to_np(bias), 1.0, 1.0), dt), *TOL_GEMM[dt], "bias")
    nan_c = torch.full((m, n), float("nan"), dtype=dtype)
    got = ntops_amd.torch.addmm(nan_c.cuda(), x.cuda(), y.cuda(), beta=0, alpha=2)
    assert not torch.isnan(got).any()
    assert_close(got, from_np(O.gemm(to_np(x), to_np(y), dt, None, 2.0, 0.0), dt), *TOL_GEMM[dt], "beta=0")


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
    dt = DT_NAME[dtype]
    assert_close(got, from_np(O.gemm(to_np(a), to_np(b), dt), dt), 1.6e-2, 1.6e-2, f"bmm short-k {layout}")


def test_addmm_short_k_bias():
    m, n, k = 512, 768, 64
    bias = torch.randn(n).bfloat16()
    x = (0.1 * torch.randn(m, k)).bfloat16()
    y = (0.1 * torch.randn(k, n)).bfloat16()
    got = ntops_amd.torch.addmm(bias.cuda(), x.cuda(), y.cuda(), beta=0.5, alpha=2.0)
    exp = from_np(O.gemm(to_np(x), to_np(y), "bf16", to_np(bias), 2.0, 0.5), "bf16")
    assert_close(got, exp, 1.6e-2, 1.6e-2, "addmm short-k bias")


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
    dt = DT_NAME[dtype]
    rtol, atol = tol(dtype, k)
    assert_close(got, from_np(O.gemm(to_np(a), to_np(o), dt), dt), rtol, atol * max(1.0, k**0.5), "matmul")
    if b is not None:
        got = ntops_amd.torch.matmul(a[0].cuda(), o.cuda())  # broadcast batch
        assert_close(got, from_np(O.gemm(to_np(a[0])[None], to_np(o), dt), dt), rtol, atol * max(1.0, k**0.5), "bcast")


def _checksum(got, a, b, bias=None):
    """Row sums of the GPU result against A @ (B @ 1) (+ N * bias mean) in
    fp64: covers every output element with a size-independent bound."""
    ones = torch.ones(b.shape[-1], 1, dtype=torch.float64)
    ref = a.double() @ (b.double() @ ones)
    if bias is not None:
        ref = ref + bias.double().sum()
    got_sum = got.double().sum(-1, keepdim=True).cpu()
    # each of N outputs carries <= 1/2 bf16 ulp of rounding: bound the sum
    bound = 2.0**-8 * got.double().abs().sum(-1, keepdim=True).cpu() + 1e-3
    assert ((got_sum - ref).abs() <= bound).all(), "checksum"


def _config_mm():
    g = torch.Generator().manual_seed(0)
    a = (0.02 * torch.randn(8192, 4096, generator=g)).bfloat16()
    b = (0.02 * torch.randn(4096, 14336, generator=g)).bfloat16()
    bias = (0.02 * torch.randn(14336, generator=g)).bfloat16()
    return a, b, bias


def test_mm_and_addmm_config_full_size():
    """bf16 (8192 x 4096) . (4096 x 14336), fp32 accumulation; addmm with a
    (14336,) bias, beta = alpha = 1."""
    a, b, bias = _config_mm()
    ag, bg = a.cuda(), b.cuda()
    rows = torch.randint(0, 8192, (48,))
    bn = to_np(b)
    for name, fn, bias_ in (
        ("mm", lambda: ntops_amd.torch.mm(ag, bg), None),
        ("addmm", lambda: ntops_amd.torch.addmm(bias.cuda(), ag, bg), bias),
    ):
        got = fn()
        sub = got[rows.cuda()]
        exp = from_np(
            O.gemm(to_np(a[rows]), bn, "bf16", None if bias_ is None else to_np(bias_), 1.0, 0.0 if bias_ is None else 1.0),
            "bf16",
        )
        assert_close(sub, exp, 1.6e-2, 1.6e-2, f"{name} sampled rows")
        _checksum(got, a, b, bias_)
        del got


def test_bmm_config_full_size():
    """bf16 (32, 2048 x 128) . (32, 128 x 2048): every element vs the oracle."""
    g = torch.Generator().manual_seed(0)
    a = (0.02 * torch.randn(32, 2048, 128, generator=g)).bfloat16()
    b = (0.02 * torch.randn(32, 128, 2048, generator=g)).bfloat16()
    got = ntops_amd.torch.bmm(a.cuda(), b.cuda())
    for i in range(0, 32, 4):
        exp = from_np(O.gemm(to_np(a[i : i + 4]), to_np(b[i : i + 4]), "bf16"), "bf16")
        assert_close(got[i : i + 4], exp, 1.6e-2, 1.6e-2, f"bmm batch {i}")
