"""GPU parity over seeded random layouts: elementwise operands that are
transposed, sliced, broadcast (rows, columns, 0-dim) or of mixed dtypes, and
row / middle-dim views of softmax and norm inputs -- each through every
launch shape that can serve it (dense, rows, broadcast element, strided,
fused conversion) -- against torch on the CPU bit for bit (single-rounding
elementwise ops) or the oracle at the reduction tolerance."""

import random

import pytest
import torch

import ntops_amd
from oracle import ops as O
from tests.helpers import DT_NAME, TOL_REDUCTION, assert_close, assert_equal, from_np, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

T = ntops_amd.torch


def _view(rng, t):
    """A random view of t with the same values layout-wise: transposed,
    sliced from a wider buffer, or as is."""
    kind = rng.choice(("plain", "transpose", "slice", "permute"))
    if kind == "transpose" and t.dim() >= 2:
        return t.transpose(-1, -2).contiguous().transpose(-1, -2)
    if kind == "slice" and t.dim() >= 1:
        pad = rng.choice((1, 8, 16))
        big = torch.zeros(*t.shape[:-1], t.shape[-1] + pad, dtype=t.dtype)
        lo = rng.randrange(0, pad + 1)
        big[..., lo:lo + t.shape[-1]] = t
        return big[..., lo:lo + t.shape[-1]]
    if kind == "permute" and t.dim() >= 3:
        perm = list(range(t.dim()))
        rng.shuffle(perm)
        inv = [perm.index(i) for i in range(t.dim())]
        return t.permute(perm).contiguous().permute(inv)
    return t


def _bcast_shape(rng, shape):
    """shape with some dims set to 1 or dropped from the front (broadcast)."""
    s = [1 if rng.random() < 0.3 else n for n in shape]
    drop = rng.randrange(0, len(s) + 1) if rng.random() < 0.3 else 0
    return tuple(s[drop:])


@pytest.mark.parametrize("seed", range(24))
def test_elementwise_random_layouts(seed):
    rng = random.Random(seed)
    g = torch.Generator().manual_seed(seed)
    ndim = rng.randint(1, 4)
    shape = tuple(rng.choice((1, 3, 8, 16, 64, 100, 256)) for _ in range(ndim))
    dts = (torch.float32, torch.bfloat16, torch.float16, torch.int32)
    ad, bd = rng.choice(dts), rng.choice(dts)
    bshape = _bcast_shape(rng, shape)

    def make(sh, dt):
        if dt == torch.int32:
            return torch.randint(-50, 50, sh, generator=g, dtype=dt)
        return torch.randn(sh, generator=g).to(dt)

    a = _view(rng, make(shape, ad))
    b = _view(rng, make(bshape, bd)) if bshape else make((), bd)
    if rng.random() < 0.2:
        a, b = b, a  # the broadcast operand first
    ag, bg = a.cuda(), b.cuda()
    what = f"seed {seed}: {tuple(a.shape)} {ad} stride {a.stride()} / {tuple(b.shape)} {bd} stride {b.stride()}"
    assert_equal(T.add(ag, bg), a + b, "add " + what)
    assert_equal(T.mul(ag, bg), a * b, "mul " + what)
    if torch.result_type(a, b).is_floating_point:
        assert_equal(T.sub(ag, bg, alpha=0.5), torch.sub(a, b, alpha=0.5), "sub " + what)
    assert_equal(T.eq(ag, bg), a == b, "eq " + what)
    if a.dtype.is_floating_point:
        dt = DT_NAME[a.dtype]
        exp = from_np(O.silu(to_np(a.contiguous()), dt), dt).reshape(a.shape)
        assert_close(T.silu(ag), exp, *TOL_REDUCTION[dt], "silu " + what)


@pytest.mark.parametrize("seed", range(12))
def test_rows_random_views(seed):
    rng = random.Random(1000 + seed)
    g = torch.Generator().manual_seed(1000 + seed)
    dtype = rng.choice((torch.float32, torch.bfloat16, torch.float16))
    dt = DT_NAME[dtype]
    cols = rng.choice((64, 96, 1000, 4096, 4100, 33))
    rows = rng.choice((1, 7, 64, 300))
    pad = rng.choice((0, 8, 16, 24, 5))
    lo = rng.randrange(0, pad + 1)
    big = torch.randn(rows, cols + pad, generator=g).to(dtype)
    x = big[:, lo:lo + cols]
    w = (1 + 0.02 * torch.randn(cols, generator=g)).to(dtype)
    xg = big.cuda()[:, lo:lo + cols]
    what = f"seed {seed}: ({rows}, {cols}) view at {lo} of width {cols + pad}, {dtype}"
    exp = from_np(O.softmax(to_np(x.contiguous()), -1, dt), dt)
    assert_close(T.softmax(xg, -1), exp, *TOL_REDUCTION[dt], "softmax " + what)
    exp = from_np(O.rms_norm(to_np(x.contiguous()), dt, cols, to_np(w), 1e-6), dt)
    assert_close(T.rms_norm(xg, (cols,), w.cuda(), 1e-6), exp, *TOL_REDUCTION[dt], "rms_norm " + what)
    exp = from_np(O.layer_norm(to_np(x.contiguous()), dt, cols, to_np(w), None, 1e-5), dt)
    assert_close(T.layer_norm(xg, (cols,), w.cuda(), None, 1e-5), exp, *TOL_REDUCTION[dt], "layer_norm " + what)
    # a middle dim of a 3-D view
    z = torch.randn(rng.choice((2, 5)), rng.choice((3, 17)), rng.choice((8, 40)), generator=g).to(dtype)
    zt = z.transpose(0, 1)
    for d in range(3):
        exp = from_np(O.softmax(to_np(zt.contiguous()), d, dt), dt)
        assert_close(T.softmax(zt.cuda(), d), exp, *TOL_REDUCTION[dt], f"softmax dim {d} of transposed " + what)
