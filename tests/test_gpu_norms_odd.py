"""GPU parity: the norms on rows that are not whole 16-byte runs, through the
C ABI with input and output views at every offset within 16 bytes.

Rows of an odd width, or views into wider rows, split into a head up to the
first 16-byte boundary, whole 16-byte packs and a tail.  Each case runs
rms_norm, layer_norm and add_rms_norm on views x = X[:, lo:lo + cols] and
y = Y[:, lo:lo + cols] of padded buffers (the same layout, so the head /
pack / tail kernels serve them), against the oracle, and checks that no
element of the padding around the views was written.  add_rms_norm must
equal add followed by rms_norm bit for bit, also when its operands sit at
different offsets (then it runs as those two kernels)."""

import numpy as np
import pytest
import torch

import ntops_amd
from ntops_amd import _lib
from oracle import ops as O
from tests.helpers import DT_NAME, TOL_REDUCTION, assert_close, from_np, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

ROWS = 37
PAD = 11  # row stride = cols + PAD: consecutive rows start at different offsets


def _views(g, dtype, cols, lo, fill):
    big = torch.full((ROWS, cols + PAD), fill, dtype=dtype)
    big[:, lo:lo + cols] = torch.randn(ROWS, cols, generator=g).to(dtype)
    return big


def _call_rms(lib, dt, x, y, cols, w, eps):
    st = torch.cuda.current_stream().cuda_stream
    return lib.ntops_rms_norm(dt, ROWS, cols, x.data_ptr(), x.stride(0), None if w is None else w.data_ptr(), 0,
                              dt if w is None or w.dtype != torch.float32 else _lib.F32, eps, y.data_ptr(),
                              y.stride(0), st)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("cols", (4100, 1001, 13, 3, 4097, 520))
def test_norms_odd_layout_views(dtype, cols):
    g = torch.Generator().manual_seed(cols * 7 + 1)
    lib = _lib.load()
    dt = _lib.dtype_code(dtype)
    name = DT_NAME[dtype]
    rtol, atol = TOL_REDUCTION[name]
    v = 16 // torch.empty(0, dtype=dtype).element_size()
    w = (1 + 0.05 * torch.randn(cols, generator=g)).to(dtype)
    b = (0.05 * torch.randn(cols, generator=g)).to(dtype)
    st = torch.cuda.current_stream().cuda_stream
    for lo in range(v):
        X = _views(g, dtype, cols, lo, 0.0)
        x = X[:, lo:lo + cols]
        xn = to_np(x.contiguous())
        Xg = X.cuda()
        xg = Xg[:, lo:lo + cols]
        for wt in (w, None):
            Y = torch.full((ROWS, cols + PAD), float("nan"), dtype=dtype, device="cuda")
            yg = Y[:, lo:lo + cols]
            wg = None if wt is None else wt.cuda()
            assert _call_rms(lib, dt, xg, yg, cols, wg, 1e-6) == 0, lib.ntops_last_error()
            exp = from_np(O.rms_norm(xn, name, cols, None if wt is None else to_np(wt), 1e-6), name)
            assert_close(yg, exp, rtol, atol, f"rms_norm lo={lo}")
            keep = torch.ones_like(Y, dtype=torch.bool)
            keep[:, lo:lo + cols] = False
            assert torch.isnan(Y[keep].float()).all(), f"rms_norm wrote outside its rows (lo={lo})"
        # layer_norm with weight and bias
        Y = torch.full((ROWS, cols + PAD), float("nan"), dtype=dtype, device="cuda")
        yg = Y[:, lo:lo + cols]
        wg, bg = w.cuda(), b.cuda()
        rc = lib.ntops_layer_norm(dt, ROWS, cols, xg.data_ptr(), xg.stride(0), wg.data_ptr(), bg.data_ptr(), 0, dt,
                                  1e-5, yg.data_ptr(), yg.stride(0), st)
        assert rc == 0, lib.ntops_last_error()
        exp = from_np(O.layer_norm(xn, name, cols, to_np(w), to_np(b), 1e-5), name)
        assert_close(yg, exp, rtol, atol, f"layer_norm lo={lo}")
        assert torch.isnan(Y[keep].float()).all(), f"layer_norm wrote outside its rows (lo={lo})"
        # add_rms_norm: x, residual, new residual and output in one layout
        Rg = _views(g, dtype, cols, lo, 0.0).cuda()
        rg = Rg[:, lo:lo + cols]
        Y = torch.full((ROWS, cols + PAD), float("nan"), dtype=dtype, device="cuda")
        H = torch.full((ROWS, cols + PAD), float("nan"), dtype=dtype, device="cuda")
        yg, hg = Y[:, lo:lo + cols], H[:, lo:lo + cols]
        rc = lib.ntops_add_rms_norm(dt, ROWS, cols, xg.data_ptr(), xg.stride(0), rg.data_ptr(), rg.stride(0),
                                    wg.data_ptr(), 0, dt, 1e-6, yg.data_ptr(), yg.stride(0), hg.data_ptr(),
                                    hg.stride(0), st)
        assert rc == 0, lib.ntops_last_error()
        assert torch.isnan(Y[keep].float()).all() and torch.isnan(H[keep].float()).all()
        # unfused: add into a buffer of the same layout, rms_norm over it
        H2 = torch.full((ROWS, cols + PAD), float("nan"), dtype=dtype, device="cuda")
        h2 = H2[:, lo:lo + cols]
        h2.copy_(ntops_amd.torch.add(xg, rg))
        assert torch.equal(hg, h2), f"new residual lo={lo}"
        Y2 = torch.full((ROWS, cols + PAD), float("nan"), dtype=dtype, device="cuda")
        y2 = Y2[:, lo:lo + cols]
        assert _call_rms(lib, dt, h2, y2, cols, wg, 1e-6) == 0
        assert torch.equal(yg, y2), f"add_rms_norm vs add + rms_norm, lo={lo}"


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float32))
def test_add_rms_norm_mixed_offsets_compose(dtype):
    """x at another offset than the residual and outputs: add_rms_norm runs
    as add then rms_norm over the new residual, so it equals them bit for
    bit (and the odd-width bf16 config runs through the one-pass kernel)."""
    cols = 4100
    g = torch.Generator().manual_seed(5)
    lib = _lib.load()
    dt = _lib.dtype_code(dtype)
    st = torch.cuda.current_stream().cuda_stream
    X = torch.randn(ROWS, cols + 1, generator=g).to(dtype).cuda()
    x = X[:, 1:]  # starts one element in: a different offset from the others
    r = torch.randn(ROWS, cols, generator=g).to(dtype).cuda()
    w = (1 + 0.05 * torch.randn(cols, generator=g)).to(dtype).cuda()
    y, h = torch.empty_like(r), torch.empty_like(r)
    rc = lib.ntops_add_rms_norm(dt, ROWS, cols, x.data_ptr(), x.stride(0), r.data_ptr(), cols, w.data_ptr(), 0, dt,
                                1e-6, y.data_ptr(), cols, h.data_ptr(), cols, st)
    assert rc == 0, lib.ntops_last_error()
    assert torch.equal(h, ntops_amd.torch.add(x, r))
    y2 = torch.empty_like(r)
    assert _call_rms(lib, dt, h, y2, cols, w, 1e-6) == 0
    assert torch.equal(y, y2)


def test_rms_norm_odd_config_width():
    """bf16 (16384, 4100): every element against the oracle within the
    north-star tolerance and at most 1 in 1000 output bits different."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(16384, 4100, generator=g).bfloat16()
    w = (1 + 0.02 * torch.randn(4100, generator=g)).bfloat16()
    got = ntops_amd.torch.rms_norm(x.cuda(), (4100,), w.cuda(), 1e-6).cpu()
    exp = from_np(O.rms_norm(to_np(x), "bf16", 4100, to_np(w), 1e-6), "bf16")
    assert_close(got, exp, 1.6e-2, 1.6e-2, "rms_norm (16384, 4100)")
    mism = (got.view(torch.int16) != exp.view(torch.int16)).float().mean().item()
    assert mism < 1e-3, f"bit mismatch fraction {mism}"


@pytest.mark.parametrize("cols", (7676, 7684))
def test_layer_norm_odd_width_at_the_staging_limit(cols):
    """bf16 rows with fp32 weight and bias staged in LDS: 7676 columns take
    the head / pack / tail kernel at its 60 KiB staging limit (2 x 30704
    bytes), 7684 the looped kernel just past it; both against the oracle."""
    g = torch.Generator().manual_seed(cols)
    x = torch.randn(33, cols, generator=g).bfloat16()
    w = 1 + 0.05 * torch.randn(cols, generator=g)
    b = 0.05 * torch.randn(cols, generator=g)
    got = ntops_amd.torch.layer_norm(x.cuda(), (cols,), w.cuda(), b.cuda(), 1e-5)
    exp = from_np(O.layer_norm(to_np(x), "bf16", cols, w.numpy(), b.numpy(), 1e-5, wb_dt="f32"), "bf16")
    assert_close(got, exp, 1.6e-2, 1.6e-2, f"layer_norm {cols}")
    got = ntops_amd.torch.rms_norm(x.cuda(), (cols,), w.cuda(), 1e-6)
    exp = from_np(O.rms_norm(to_np(x), "bf16", cols, w.numpy(), 1e-6, w_dt="f32"), "bf16")
    assert_close(got, exp, 1.6e-2, 1.6e-2, f"rms_norm {cols}")
