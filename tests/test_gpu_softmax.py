"""GPU parity: softmax against the oracle (and torch CPU).

Mirrors tests/test_softmax.py:11-21 of the reference (random dim, output
dtype in {fp16, fp32, fp64}) with bf16, every row-width configuration, and
the bf16 (4, 32, 2048, 2048) causal config at full size (oracle on one whole
(batch, head) slice plus size-independent properties on all rows)."""

import math
import random

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import ntops_amd
from oracle import ops as O
from tests.helpers import DT_NAME, TOL_REDUCTION, assert_close, from_np, random_shape, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

FLOATS = (torch.float32, torch.float16, torch.bfloat16)


def cases():
    out = []
    for ndim in range(1, 5):
        for dtype in FLOATS:
            out.append((random_shape(ndim), dtype))
    return out


@pytest.mark.parametrize("shape, dtype", cases())
def test_softmax(shape, dtype):
    x = torch.randn(shape).to(dtype)
    dim = random.randint(0, x.ndim - 1)
    out_dtype = random.choice([torch.float16, torch.float32, torch.float64, None])
    got = ntops_amd.torch.softmax(x.cuda(), dim, out_dtype)
    odt = DT_NAME[out_dtype or dtype]
    exp = from_np(O.softmax(to_np(x), dim, DT_NAME[dtype], odt), odt)
    rtol, atol = TOL_REDUCTION[odt]
    assert_close(got, exp, rtol, atol, "softmax vs oracle")
    assert_close(got, F.softmax(x, dim=dim, dtype=out_dtype), max(rtol, 1e-5), max(atol, 1e-5), "softmax vs torch")


@pytest.mark.parametrize("cols", [1, 7, 64, 512, 1000, 2048, 4096, 8192, 16384, 32768, 65536, 70000])
@pytest.mark.parametrize("dtype", FLOATS)
def test_softmax_widths(cols, dtype):
    x = (torch.randn(3, cols) * 3).to(dtype)
    dt = DT_NAME[dtype]
    got = ntops_amd.torch.softmax(x.cuda(), -1)
    exp = from_np(O.softmax(to_np(x), -1, dt), dt)
    assert_close(got, exp, *TOL_REDUCTION[dt], f"softmax width {cols}")


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("cols", (50257, 1001, 13, 7))
def test_softmax_odd_width_row_views(cols, dtype):
    """Rows whose width is no multiple of a 16-byte pack, read through views
    that start at different offsets (so each row has its own head / pack /
    tail split, and the output rows -- contiguous -- are aligned unlike the
    input rows, the element-store branch)."""
    g = torch.Generator().manual_seed(cols)
    x = (torch.randn(37, cols + 3, generator=g) * 3).to(dtype)
    xg = x.cuda()
    dt = DT_NAME[dtype]
    for lo in (0, 1, 3):
        got = ntops_amd.torch.softmax(xg[:, lo:lo + cols], -1)
        exp = from_np(O.softmax(to_np(x[:, lo:lo + cols].contiguous()), -1, dt), dt)
        assert_close(got, exp, *TOL_REDUCTION[dt], f"softmax row views offset {lo}")


def test_softmax_special_rows():
    x = torch.randn(4, 64)
    x[1] = float("-inf")  # all -inf -> NaN, like torch
    x[2, :10] = float("-inf")
    x[3, 5] = float("inf")
    got = ntops_amd.torch.softmax(x.cuda(), -1).cpu()
    ref = F.softmax(x, -1)
    assert torch.isnan(got[1]).all()
    assert_close(got, ref, 1e-5, 1e-5, "special rows")
    s = torch.tensor(2.0)
    assert ntops_amd.torch.softmax(s.cuda(), 0).item() == 1.0


def test_softmax_noncontiguous():
    x = torch.randn(16, 24, 40).bfloat16()
    xg = x.cuda().permute(2, 0, 1)
    for dim in range(3):
        got = ntops_amd.torch.softmax(xg, dim)
        exp = from_np(O.softmax(to_np(x.permute(2, 0, 1)), dim, "bf16"), "bf16")
        assert_close(got, exp, 1.6e-2, 1.6e-2, f"permuted dim {dim}")


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float32))
def test_softmax_views_read_in_place(dtype):
    """Views whose leading and trailing dims each merge into one stride run
    in place, without a row-major copy: row views of a wider tensor (the
    register-resident, looped and wide-row kernels), a middle dim of a
    transposed tensor, an expanded (stride-0) row, a sliced batch."""
    g = torch.Generator().manual_seed(11)
    dt = DT_NAME[dtype]
    tol = TOL_REDUCTION[dt]
    big = (torch.randn(64, 1024 + 160, generator=g) * 2).to(dtype)
    bg = big.cuda()
    for lo, w in ((0, 128), (8, 1024), (160, 1024), (3, 77)):
        got = ntops_amd.torch.softmax(bg[:, lo:lo + w], -1)
        exp = from_np(O.softmax(to_np(big[:, lo:lo + w].contiguous()), -1, dt), dt)
        assert_close(got, exp, *tol, f"row view [{lo}, {lo + w})")
    wide = (torch.randn(3, 70000 + 64, generator=g)).to(dtype)
    got = ntops_amd.torch.softmax(wide.cuda()[:, 64:], -1)
    exp = from_np(O.softmax(to_np(wide[:, 64:].contiguous()), -1, dt), dt)
    assert_close(got, exp, *tol, "wide row view")
    z = torch.randn(8, 16, 40, generator=g).to(dtype)
    zt = z.transpose(0, 1)  # (16, 8, 40): dim 1 has stride 640, outer stride 40
    got = ntops_amd.torch.softmax(zt.cuda(), 1)
    exp = from_np(O.softmax(to_np(zt.contiguous()), 1, dt), dt)
    assert_close(got, exp, *tol, "transposed middle dim")
    row = torch.randn(1, 256, generator=g).to(dtype)
    got = ntops_amd.torch.softmax(row.cuda().expand(5, 256), -1)
    exp = from_np(O.softmax(to_np(row.expand(5, 256).contiguous()), -1, dt), dt)
    assert_close(got, exp, *tol, "expanded row")
    b = torch.randn(6, 4, 96, generator=g).to(dtype)
    got = ntops_amd.torch.softmax(b.cuda()[1::2], -1)
    exp = from_np(O.softmax(to_np(b[1::2].contiguous()), -1, dt), dt)
    assert_close(got, exp, *tol, "sliced batch")


def test_softmax_config_full_size():
    """bf16 (4, 32, 2048, 2048) scores ~N(0,1)/sqrt(128), -inf above the
    diagonal, softmax over the last dim."""
    B, H, S = 4, 32, 2048
    g = torch.Generator().manual_seed(0)
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool), 1)
    x = torch.empty(B, H, S, S, dtype=torch.bfloat16)
    for b in range(B):
        x[b] = (torch.randn(H, S, S, generator=g) / math.sqrt(128)).masked_fill(mask, float("-inf")).bfloat16()
    got = ntops_amd.torch.softmax(x.cuda(), -1)
    # one whole (batch, head) slice and scattered rows against the oracle
    exp = from_np(O.softmax(to_np(x[1, 7]), -1, "bf16"), "bf16")
    assert_close(got[1, 7], exp, 1.6e-2, 1.6e-2, "softmax slice (1, 7)")
    assert (got[1, 7].cpu() != exp).float().mean().item() < 1e-3
    rows = torch.randint(0, S, (64,))
    for r in rows.tolist():
        b, h = r % B, (r * 7) % H
        exp = from_np(O.softmax(to_np(x[b, h, r]), -1, "bf16"), "bf16")
        assert_close(got[b, h, r], exp, 1.6e-2, 1.6e-2, f"row {b},{h},{r}")
    # size-independent properties on every row
    gf = got.float()
    sums = gf.sum(-1)
    assert torch.allclose(sums, torch.ones_like(sums), atol=2e-2), "row sums"
    assert (got.masked_select(mask.cuda().expand(B, H, S, S)) == 0).all(), "causal zeros"
    assert (got[:, :, 0, 0] == 1).all(), "row 0 is one-hot"


@pytest.mark.parametrize("cols", (8, 7))
def test_softmax_many_rows(cols):
    """200003 rows: the register-resident (8 bf16 columns) and looped (7)
    kernels on a 2-D grid of blocks whose last row has ids past the end."""
    x = (torch.randn(200003, cols, generator=torch.Generator().manual_seed(cols)) * 3).bfloat16()
    got = ntops_amd.torch.softmax(x.cuda(), -1)
    assert_close(got, from_np(O.softmax(to_np(x), -1, "bf16"), "bf16"), *TOL_REDUCTION["bf16"], "softmax")


@pytest.mark.parametrize("shape, dim, dtype", [
    ((32, 2048, 128), 1, torch.bfloat16),
    ((4096, 1024), 0, torch.bfloat16),
    ((3, 517, 1000), 1, torch.float32),
    ((2, 3, 300, 7), 2, torch.float16),
    ((64, 40, 640), 1, torch.bfloat16),
])
def test_softmax_middle_dims(shape, dim, dtype):
    """Softmax over a dim with inner elements after it: column tiles of 8-64
    columns with the dim split over row slices (every tile width the grid
    size selects), against the oracle."""
    g = torch.Generator().manual_seed(sum(shape) + dim)
    x = (torch.randn(shape, generator=g) * 2).to(dtype)
    dt = DT_NAME[dtype]
    got = ntops_amd.torch.softmax(x.cuda(), dim)
    exp = from_np(O.softmax(to_np(x), dim, dt), dt)
    assert_close(got, exp, *TOL_REDUCTION[dt], f"softmax {shape} dim {dim}")
    got = ntops_amd.torch.softmax(x.cuda(), dim, dtype=torch.float32)
    exp = from_np(O.softmax(to_np(x), dim, dt, out_dt="f32"), "f32")
    assert_close(got, exp, *TOL_REDUCTION["f32"], f"softmax {shape} dim {dim} -> f32")
