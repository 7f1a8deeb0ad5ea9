"""GPU parity: rms_norm and layer_norm against the oracle (and torch CPU).

Mirrors tests/test_rms_norm.py:11-30 and tests/test_layer_norm.py:11-37 of
the reference (eps sweeps, weight/bias None, random normalized_shape suffix)
with bf16 added, every register-resident row configuration and the looped
fallback, and the bf16 (16384, 4096) config at full size."""

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


@pytest.mark.parametrize("eps", (None, 0, 1e-5, 1e-3))
@pytest.mark.parametrize("weight_is_none", (False, True))
@pytest.mark.parametrize("shape, dtype", cases())
def test_rms_norm(shape, dtype, weight_is_none, eps):
    x = torch.randn(shape).to(dtype)
    normalized_shape = shape[-random.randint(1, len(shape)) :]
    w = None if weight_is_none else torch.randn(normalized_shape).to(dtype)
    got = ntops_amd.torch.rms_norm(x.cuda(), normalized_shape, weight=None if w is None else w.cuda(), eps=eps)
    dt = DT_NAME[dtype]
    cols = int(np.prod(normalized_shape))
    exp = from_np(O.rms_norm(to_np(x), dt, cols, None if w is None else to_np(w), eps), dt)
    rtol, atol = TOL_REDUCTION[dt]
    assert_close(got, exp, rtol, atol, "rms_norm vs oracle")
    ref = F.rms_norm(x, normalized_shape, weight=w, eps=eps)
    assert_close(got, ref, rtol, atol, "rms_norm vs torch cpu")


@pytest.mark.parametrize("cols", (4096, 1000, 12288, 40))
@pytest.mark.parametrize("weight_is_none", (False, True))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_rms_norm_eps_none_bits(dtype, weight_is_none, cols):
    """eps=None resolves to finfo(float32).eps for 16-bit inputs too (ntops'
    finfo(dtype).eps would change most output bits): the output bits against
    the oracle's, fewer than 1 in 1000 allowed to differ (fp32 sums in
    another order may move a rounding boundary), and an input whose mean
    square is below eps where the default dominates the result."""
    g = torch.Generator().manual_seed(cols + (7 if weight_is_none else 0))
    x = torch.randn(256, cols, generator=g).to(dtype)
    w = None if weight_is_none else (1 + 0.02 * torch.randn(cols, generator=g)).to(dtype)
    dt = DT_NAME[dtype]
    got = ntops_amd.torch.rms_norm(x.cuda(), (cols,), None if w is None else w.cuda()).cpu()
    exp = from_np(O.rms_norm(to_np(x), dt, cols, None if w is None else to_np(w), None), dt)
    assert_close(got, exp, *TOL_REDUCTION[dt], "rms_norm eps=None")
    mism = (got.view(torch.int16) != exp.view(torch.int16)).float().mean().item()
    assert mism < 1e-3, f"bit mismatch fraction {mism}"
    # mean square 2^-24 < eps = 2^-23: y = 1 / sqrt(3) (finfo(dtype).eps: < 0.01)
    tiny = torch.full((3, cols), 2.0 ** -12, dtype=dtype, device="cuda")
    y = ntops_amd.torch.rms_norm(tiny, (cols,)).float()
    torch.testing.assert_close(y, torch.full_like(y, 3 ** -0.5), rtol=2 ** -8, atol=0)


@pytest.mark.parametrize("eps", (1e-8, 1e-5, 1e-3))
@pytest.mark.parametrize("bias_is_none", (False, True))
@pytest.mark.parametrize("weight_is_none", (False, True))
@pytest.mark.parametrize("shape, dtype", cases())
def test_layer_norm(shape, dtype, weight_is_none, bias_is_none, eps):
    x = torch.randn(shape).to(dtype)
    normalized_shape = shape[-random.randint(1, len(shape)) :]
    w = None if weight_is_none else torch.randn(normalized_shape).to(dtype)
    b = None if bias_is_none else torch.randn(normalized_shape).to(dtype)
    got = ntops_amd.torch.layer_norm(
        x.cuda(), normalized_shape, weight=None if w is None else w.cuda(), bias=None if b is None else b.cuda(), eps=eps
    )
    dt = DT_NAME[dtype]
    cols = int(np.prod(normalized_shape))
    exp = from_np(O.layer_norm(to_np(x), dt, cols, None if w is None else to_np(w), None if b is None else to_np(b), eps), dt)
    rtol, atol = TOL_REDUCTION[dt]
    assert_close(got, exp, rtol, atol, "layer_norm vs oracle")
    ref = F.layer_norm(x, normalized_shape, weight=w, bias=b, eps=eps)
    assert_close(got, ref, rtol, atol, "layer_norm vs torch cpu")


# Widths that hit every (chunks, waves-per-row) configuration of the vector
# path for 16-bit and fp32 rows, plus widths that force the looped kernel
# (not a multiple of the 16-byte pack, and wider than the register budget).
WIDTHS = [8, 40, 512, 1000, 1024, 2048, 4096, 8192, 12288, 16384, 32768, 65536, 4100, 4099, 70000]


@pytest.mark.parametrize("cols", WIDTHS)
@pytest.mark.parametrize("dtype", FLOATS)
def test_norm_widths(cols, dtype):
    rows = 5
    x = torch.randn(rows, cols).to(dtype)
    w = (1 + 0.02 * torch.randn(cols)).to(dtype)
    b = (0.02 * torch.randn(cols)).to(dtype)
    dt = DT_NAME[dtype]
    rtol, atol = TOL_REDUCTION[dt]
    got = ntops_amd.torch.rms_norm(x.cuda(), (cols,), w.cuda(), 1e-6)
    assert_close(got, from_np(O.rms_norm(to_np(x), dt, cols, to_np(w), 1e-6), dt), rtol, atol, f"rms {cols}")
    got = ntops_amd.torch.layer_norm(x.cuda(), (cols,), w.cuda(), b.cuda(), 1e-5)
    assert_close(got, from_np(O.layer_norm(to_np(x), dt, cols, to_np(w), to_np(b), 1e-5), dt), rtol, atol, f"ln {cols}")


@pytest.mark.parametrize("cols", [64, 1000, 4096, 8192, 16384])
@pytest.mark.parametrize("dtype", FLOATS)
def test_layer_norm_offset_rows(cols, dtype):
    """Rows offset by 30 standard deviations, a row whose first element is
    an outlier (3000 standard deviations for fp32, 300 for 16-bit types) and
    a constant row: the variance must not lose precision to cancellation
    (the fp32 tolerance is 1e-5; larger offsets amplify the rounding of the
    mean through torch's output formula x * rstd - rstd * mean beyond it,
    for torch's CPU kernel as much as for any other summation order)."""
    g = torch.Generator().manual_seed(cols)
    x = torch.randn(5, cols, generator=g)
    x[1] += 30.0
    x[2] -= 30.0
    x[3, 0] = 3000.0 if dtype == torch.float32 else 300.0
    x[4] = 7.0
    x = x.to(dtype)
    w = (1 + 0.02 * torch.randn(cols, generator=g)).to(dtype)
    b = (0.02 * torch.randn(cols, generator=g)).to(dtype)
    dt = DT_NAME[dtype]
    rtol, atol = TOL_REDUCTION[dt]
    got = ntops_amd.torch.layer_norm(x.cuda(), (cols,), w.cuda(), b.cuda(), 1e-5)
    exp = from_np(O.layer_norm(to_np(x), dt, cols, to_np(w), to_np(b), 1e-5), dt)
    assert_close(got, exp, rtol, atol, f"ln offset rows {cols}")


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("cols", (4100, 1001, 13))
def test_rms_norm_odd_width_row_views(cols, dtype):
    """rms_norm on rows that are no multiple of a 16-byte pack, through views
    starting at different offsets (the looped kernel, rows at every 16-byte
    alignment)."""
    g = torch.Generator().manual_seed(cols)
    x = torch.randn(29, cols + 3, generator=g).to(dtype)
    w = (1 + 0.02 * torch.randn(cols, generator=g)).to(dtype)
    xg = x.cuda()
    dt = DT_NAME[dtype]
    rtol, atol = TOL_REDUCTION[dt]
    for lo in (0, 1, 3):
        got = ntops_amd.torch.rms_norm(xg[:, lo:lo + cols], (cols,), w.cuda(), 1e-6)
        exp = from_np(O.rms_norm(to_np(x[:, lo:lo + cols].contiguous()), dt, cols, to_np(w), 1e-6), dt)
        assert_close(got, exp, rtol, atol, f"rms_norm row views offset {lo}")


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float32))
@pytest.mark.parametrize("cols, lo, width", ((4096, 256, 8192), (1024, 8, 1152), (100000, 64, 100064), (1000, 24, 1032)))
def test_norms_on_row_views_in_place(cols, lo, width, dtype):
    """Row views of a wider tensor whose rows start 16-byte aligned like a
    row-major output's run in place (row stride passed to the kernels):
    rms_norm, layer_norm and add_rms_norm equal, bit for bit, the same call
    on a row-major copy of the view, and match the oracle."""
    g = torch.Generator().manual_seed(cols + lo)
    big = torch.randn(19, width, generator=g).to(dtype)
    res_big = torch.randn(19, width, generator=g).to(dtype)
    w = (1 + 0.02 * torch.randn(cols, generator=g)).to(dtype)
    b = (0.02 * torch.randn(cols, generator=g)).to(dtype)
    v, r = big.cuda()[:, lo:lo + cols], res_big.cuda()[:, lo:lo + cols]
    vc, rc = v.contiguous(), r.contiguous()
    T = ntops_amd.torch
    assert torch.equal(T.rms_norm(v, (cols,), w.cuda(), 1e-6), T.rms_norm(vc, (cols,), w.cuda(), 1e-6))
    assert torch.equal(T.layer_norm(v, (cols,), w.cuda(), b.cuda()), T.layer_norm(vc, (cols,), w.cuda(), b.cuda()))
    o1, n1 = T.add_rms_norm(v, r, (cols,), w.cuda(), 1e-6)
    o2, n2 = T.add_rms_norm(vc, rc, (cols,), w.cuda(), 1e-6)
    assert torch.equal(o1, o2) and torch.equal(n1, n2)
    dt = DT_NAME[dtype]
    exp = from_np(O.rms_norm(to_np(big[:, lo:lo + cols].contiguous()), dt, cols, to_np(w), 1e-6), dt)
    assert_close(T.rms_norm(v, (cols,), w.cuda(), 1e-6), exp, *TOL_REDUCTION[dt], "rms_norm row view")


def test_norm_noncontiguous_input_and_fp32_weight():
    x = torch.randn(64, 96).bfloat16()
    xg = x.cuda().t()  # (96, 64) non-contiguous
    w32 = 1 + 0.02 * torch.randn(64)
    got = ntops_amd.torch.rms_norm(xg, (64,), w32.cuda(), 1e-6)
    exp = from_np(O.rms_norm(to_np(x.t()), "bf16", 64, w32.numpy(), 1e-6, w_dt="f32"), "bf16")
    assert_close(got, exp, 1.6e-2, 1.6e-2, "rms fp32 weight")
    got = ntops_amd.torch.layer_norm(xg, (64,), w32.cuda(), w32.cuda() - 1, 1e-5)
    exp = from_np(O.layer_norm(to_np(x.t()), "bf16", 64, w32.numpy(), (w32 - 1).numpy(), 1e-5, wb_dt="f32"), "bf16")
    assert_close(got, exp, 1.6e-2, 1.6e-2, "ln fp32 weight")


# (weight shape, normalized_shape) over a (4, 6, 64) input: the reference
# expands the weight with `weight.expand_as(input)`, so any broadcastable
# shape is legal -- shared rows (incl. broadcast inside a 2-D normalized
# shape) take the vector kernels, weights that differ per row the looped ones.
WEIGHT_FORMS = (
    ((64,), (64,)),
    ((1, 1, 64), (64,)),
    ((64,), (6, 64)),
    ((6, 1), (64,)),
    ((1, 6, 64), (64,)),
    ((4, 6, 64), (64,)),
)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float32))
@pytest.mark.parametrize("w_shape, nshape", WEIGHT_FORMS)
def test_norm_weight_broadcast_forms(w_shape, nshape, dtype):
    dt = DT_NAME[dtype]
    g = torch.Generator().manual_seed(len(w_shape) * 10 + len(nshape))
    x = torch.randn(4, 6, 64, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(w_shape, generator=g)).to(dtype)
    b = (0.1 * torch.randn(w_shape, generator=g)).to(dtype)
    cols = int(np.prod(nshape))
    rtol, atol = TOL_REDUCTION[dt]
    got = ntops_amd.torch.rms_norm(x.cuda(), nshape, w.cuda(), 1e-6)
    assert_close(got, from_np(O.rms_norm(to_np(x), dt, cols, to_np(w), 1e-6), dt), rtol, atol, f"rms {w_shape}")
    got = ntops_amd.torch.layer_norm(x.cuda(), nshape, w.cuda(), b.cuda(), 1e-5)
    assert_close(got, from_np(O.layer_norm(to_np(x), dt, cols, to_np(w), to_np(b), 1e-5), dt), rtol, atol,
                 f"ln {w_shape}")
    # mixed: a shared weight with a bias that differs per row (both laid out per row)
    b_rows = (0.1 * torch.randn(4, 6, 1, generator=g)).to(dtype)
    got = ntops_amd.torch.layer_norm(x.cuda(), nshape, w.cuda(), b_rows.cuda(), 1e-5)
    assert_close(got, from_np(O.layer_norm(to_np(x), dt, cols, to_np(w), to_np(b_rows), 1e-5), dt), rtol, atol,
                 f"ln {w_shape} + per-row bias")
    r = torch.randn(4, 6, 64, generator=g).to(dtype)
    y, h = ntops_amd.torch.add_rms_norm(x.cuda(), r.cuda(), nshape, w.cuda(), 1e-6)
    ey, eh = O.add_rms_norm(to_np(x), to_np(r), dt, cols, to_np(w), 1e-6)
    assert torch.equal(h.cpu(), from_np(eh, dt))
    assert_close(y, from_np(ey, dt), rtol, atol, f"add_rms {w_shape}")
    with pytest.raises(RuntimeError):
        ntops_amd.torch.rms_norm(x.cuda(), nshape, torch.ones(5, device="cuda", dtype=dtype))


def _config_inputs():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(16384, 4096, generator=g).bfloat16()
    w = (1 + 0.02 * torch.randn(4096, generator=g)).bfloat16()
    b = (0.02 * torch.randn(4096, generator=g)).bfloat16()
    return x, w, b


def test_rms_norm_config_full_size():
    """bf16 (16384, 4096), w ~N(1, 0.02), eps = 1e-6: every element against
    the oracle; the output RMS of every row is 1 up to the weight."""
    x, w, _ = _config_inputs()
    got = ntops_amd.torch.rms_norm(x.cuda(), (4096,), w.cuda(), 1e-6)
    exp = from_np(O.rms_norm(to_np(x), "bf16", 4096, to_np(w), 1e-6), "bf16")
    assert_close(got, exp, 1.6e-2, 1.6e-2, "rms_norm config")
    mism = (got.cpu() != exp).float().mean().item()
    assert mism < 1e-3, f"bit mismatch fraction {mism}"
    unweighted = (got.float() / w.cuda().float()).pow(2).mean(-1).sqrt()
    assert torch.allclose(unweighted, torch.ones_like(unweighted), atol=2e-2)


def test_layer_norm_config_full_size():
    x, w, b = _config_inputs()
    got = ntops_amd.torch.layer_norm(x.cuda(), (4096,), w.cuda(), b.cuda(), 1e-5)
    exp = from_np(O.layer_norm(to_np(x), "bf16", 4096, to_np(w), to_np(b), 1e-5), "bf16")
    assert_close(got, exp, 1.6e-2, 1.6e-2, "layer_norm config")
    mism = (got.cpu() != exp).float().mean().item()
    assert mism < 1e-3, f"bit mismatch fraction {mism}"


@pytest.mark.parametrize("cols", (8, 7))
def test_norms_many_rows(cols):
    """200003 rows: more row groups than one grid dimension holds (the
    blocks form a 2-D grid whose last row has ids past the end), on the
    register-resident kernels (8 bf16 columns) and the looped ones (7)."""
    g = torch.Generator().manual_seed(cols)
    rows = 200003
    x = (torch.randn(rows, cols, generator=g) + 0.5).bfloat16()
    w = (1 + 0.1 * torch.randn(cols, generator=g)).bfloat16()
    b = (0.1 * torch.randn(cols, generator=g)).bfloat16()
    rtol, atol = TOL_REDUCTION["bf16"]
    got = ntops_amd.torch.rms_norm(x.cuda(), (cols,), w.cuda(), 1e-6)
    assert_close(got, from_np(O.rms_norm(to_np(x), "bf16", cols, to_np(w), 1e-6), "bf16"), rtol, atol, "rms_norm")
    got = ntops_amd.torch.layer_norm(x.cuda(), (cols,), w.cuda(), b.cuda(), 1e-5)
    assert_close(got, from_np(O.layer_norm(to_np(x), "bf16", cols, to_np(w), to_np(b), 1e-5), "bf16"), rtol, atol,
                 "layer_norm")
    r = torch.randn(rows, cols, generator=g).bfloat16()
    y, h = ntops_amd.torch.add_rms_norm(x.cuda(), r.cuda(), (cols,), w.cuda(), 1e-6)
    ey, eh = O.add_rms_norm(to_np(x), to_np(r), "bf16", cols, to_np(w), 1e-6, "bf16")
    assert torch.equal(h.cpu(), from_np(eh, "bf16")), "add_rms_norm residual"
    assert_close(y, from_np(ey, "bf16"), rtol, atol, "add_rms_norm")
