"""GPU parity: rows wider than the register-resident shapes (more than 8192
16-byte packs), which 1024-thread blocks (one per CU, each walking rows and
loading its next row while it writes the current one) read once into VGPRs
and LDS (rms_norm, layer_norm, softmax), against the oracle.

Widths: just past the register budget (one staged pack), the 131072-element
bf16 row, the widest staged row, and one element-pack past it (the looped
kernels), in bf16, fp16 and fp32, with and without parameters; softmax
also with -inf runs and a fully masked row; and the bf16 (512, 131072)
shape on sampled rows plus its row-sum property on every row; every row of
a batch that makes each block walk two or three rows, with a partly filled
last staged run."""

import numpy as np
import pytest
import torch

import ntops_amd
from oracle import ops as O
from tests.helpers import DT_NAME, TOL_REDUCTION, assert_close, from_np, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

T = ntops_amd.torch
REG_PACKS, LDS_PACKS = 8192, 10176


def widths(dtype):
    v = 16 // torch.empty(0, dtype=dtype).element_size()
    return [(REG_PACKS + 1) * v, 131072, (REG_PACKS + LDS_PACKS) * v, (REG_PACKS + LDS_PACKS + 1) * v]


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("k", range(4))
def test_norms_wide_rows(dtype, k):
    cols = widths(dtype)[k]
    g = torch.Generator().manual_seed(cols + k)
    x = torch.randn(3, cols, generator=g).to(dtype)
    x[1] += 5.0  # a row far from zero mean
    w = (1 + 0.05 * torch.randn(cols, generator=g)).to(dtype)
    b = (0.05 * torch.randn(cols, generator=g)).to(dtype)
    dt = DT_NAME[dtype]
    rtol, atol = TOL_REDUCTION[dt]
    xg = x.cuda()
    for wt in (w, None):
        got = T.rms_norm(xg, (cols,), None if wt is None else wt.cuda(), 1e-6)
        exp = from_np(O.rms_norm(to_np(x), dt, cols, None if wt is None else to_np(wt), 1e-6), dt)
        assert_close(got, exp, rtol, atol, f"rms_norm {cols}")
    got = T.layer_norm(xg, (cols,), w.cuda(), b.cuda(), 1e-5)
    exp = from_np(O.layer_norm(to_np(x), dt, cols, to_np(w), to_np(b), 1e-5), dt)
    assert_close(got, exp, rtol, atol, f"layer_norm {cols}")
    got = T.layer_norm(xg, (cols,), None, None, 1e-5)
    exp = from_np(O.layer_norm(to_np(x), dt, cols, None, None, 1e-5), dt)
    assert_close(got, exp, rtol, atol, f"layer_norm plain {cols}")
    if dtype != torch.float32:
        w32 = 1 + 0.05 * torch.randn(cols, generator=g)
        got = T.rms_norm(xg, (cols,), w32.cuda(), 1e-6)
        exp = from_np(O.rms_norm(to_np(x), dt, cols, w32.numpy(), 1e-6, w_dt="f32"), dt)
        assert_close(got, exp, rtol, atol, f"rms_norm fp32 weight {cols}")


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("k", range(4))
def test_softmax_wide_rows(dtype, k):
    cols = widths(dtype)[k]
    g = torch.Generator().manual_seed(cols * 3 + k)
    x = (torch.randn(4, cols, generator=g) * 3).to(dtype)
    x[1, : cols // 3] = float("-inf")  # a masked run, in the VGPR part and the staged part
    x[1, cols - 5:] = float("-inf")
    x[2] = float("-inf")  # fully masked: NaN, as torch
    x[3, 7] = 40.0  # one dominant element
    dt = DT_NAME[dtype]
    got = T.softmax(x.cuda(), -1)
    exp = from_np(O.softmax(to_np(x), -1, dt), dt)
    assert_close(got, exp, *TOL_REDUCTION[dt], f"softmax {cols}")
    assert torch.isnan(got[2].float()).all()


def test_wide_rows_config_512_131072():
    """bf16 (512, 131072): rms_norm and softmax on 8 sampled rows against the
    oracle; every softmax row sums to 1 and every rms_norm row has RMS 1 (no
    weight)."""
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(512, 131072, device="cuda", generator=g).bfloat16()
    rows = [0, 1, 200, 255, 256, 301, 510, 511]
    y = T.rms_norm(x, (131072,), None, 1e-6)
    exp = from_np(O.rms_norm(to_np(x[rows].cpu()), "bf16", 131072, None, 1e-6), "bf16")
    assert_close(y[rows], exp, 1.6e-2, 1.6e-2, "rms_norm (512, 131072)")
    rms = y.float().pow(2).mean(-1).sqrt()
    assert torch.allclose(rms, torch.ones_like(rms), atol=1e-2)
    s = T.softmax(x, -1)
    exp = from_np(O.softmax(to_np(x[rows].cpu()), -1, "bf16"), "bf16")
    assert_close(s[rows], exp, 1.6e-2, 1.6e-2, "softmax (512, 131072)")
    tot = s.float().sum(-1)
    assert torch.allclose(tot, torch.ones_like(tot), atol=2e-2)


def test_wide_rows_walked_by_each_block():
    """549 rows (2-3 per block on a 256-CU part) of 8292 packs (100 staged:
    one whole and one partial LDS run): every row against the oracle, so a
    row loaded into the wrong place or a run left over from the previous row
    fails."""
    rows, cols = 549, (REG_PACKS + 100) * 8
    g = torch.Generator().manual_seed(549)
    x = (torch.randn(rows, cols, generator=g) * (1 + torch.arange(rows) % 7).unsqueeze(1)).bfloat16()
    w = (1 + 0.05 * torch.randn(cols, generator=g)).bfloat16()
    b = (0.05 * torch.randn(cols, generator=g)).bfloat16()
    xg = x.cuda()
    xn = to_np(x)
    rtol, atol = TOL_REDUCTION["bf16"]
    got = T.rms_norm(xg, (cols,), w.cuda(), 1e-6)
    assert_close(got, from_np(O.rms_norm(xn, "bf16", cols, to_np(w), 1e-6), "bf16"), rtol, atol, "rms_norm walk")
    got = T.layer_norm(xg, (cols,), w.cuda(), b.cuda(), 1e-5)
    exp = from_np(O.layer_norm(xn, "bf16", cols, to_np(w), to_np(b), 1e-5), "bf16")
    assert_close(got, exp, rtol, atol, "layer_norm walk")
    got = T.softmax(xg, -1)
    assert_close(got, from_np(O.softmax(xn, -1, "bf16"), "bf16"), rtol, atol, "softmax walk")
