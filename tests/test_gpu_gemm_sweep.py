"""GPU parity over seeded random GEMM problems: sizes from one row to a few
thousand, K tails, both operand layouts, bf16 / fp16 / fp32, C as nothing, a
bias row or a full matrix, and outputs that are fresh tensors or views whose
rows start at odd offsets -- through every kernel the dispatcher picks
(skinny, split over K, 128 / 256 tiles with edge strips, the fp32 kernels,
shifted and element stores) -- against the oracle on sampled rows: the ulp
guard for 16-bit data, the fp32 GEMM tolerance for fp32."""

import random

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


def _case(seed):
    rng = random.Random(seed)
    dtype = rng.choice((torch.bfloat16, torch.float16, torch.float32))
    m = rng.choice((1, 7, 16, 33, 64, 100, 255, 600, 1100, 2050, 4100))
    n = rng.choice((5, 64, 129, 1000, 1001, 2304, 4099, 5003))
    k = rng.choice((8, 40, 255, 320, 768, 1028, 2048))
    b_kmajor = rng.random() < 0.5
    c_form = rng.choice(("none", "row", "full"))
    out_form = rng.choice(("fresh", "fresh", "view"))
    alpha = rng.choice((1.0, 0.5, -2.0))
    beta = rng.choice((1.0, 0.25))
    return dtype, m, n, k, b_kmajor, c_form, out_form, alpha, beta


@pytest.mark.parametrize("seed", range(128))
def test_gemm_random_problems(seed):
    dtype, m, n, k, b_kmajor, c_form, out_form, alpha, beta = _case(seed)
    g = torch.Generator().manual_seed(1000 + seed)
    a = (0.1 * torch.randn(m, k, generator=g)).to(dtype)
    b = (0.1 * torch.randn(k, n, generator=g)).to(dtype)
    bg = b.t().contiguous().cuda().t() if b_kmajor else b.cuda()
    what = f"seed {seed}: {DT_NAME[dtype]} {m}x{n}x{k} B:{'K' if b_kmajor else 'N'} C:{c_form} out:{out_form}"
    rows = tile_rows(m) if m > 600 else list(range(m))
    if c_form == "none":
        c = None
    elif c_form == "row":
        c = (0.1 * torch.randn(n, generator=g)).to(dtype)
    else:
        c = (0.1 * torch.randn(m, n, generator=g)).to(dtype)
    if out_form == "fresh":
        if c is None:
            got = ntops_amd.torch.mm(a.cuda(), bg)
            alpha_e, beta_e = 1.0, 0.0
        else:
            got = ntops_amd.torch.addmm(c.cuda(), a.cuda(), bg, beta=beta, alpha=alpha)
            alpha_e, beta_e = alpha, beta
    else:
        # through the C ABI into a view whose rows start at a 2-byte offset
        # inside rows of n + 3 elements; the bytes around it stay untouched
        lib = _lib.load()
        big = torch.zeros(m, n + 3, dtype=dtype, device="cuda")
        got = big[:, 1:1 + n]
        cg = None if c is None else c.cuda()
        c_str = None if c is None else ((0, 0, 1) if c.dim() == 1 else (0, n, 1))
        rc = lib.ntops_gemm(_lib.dtype_code(dtype), 1, m, n, k, a.cuda().data_ptr(), _lib.i64_array((0, k, 1)),
                            bg.data_ptr(), _lib.i64_array((0,) + tuple(bg.stride())),
                            None if cg is None else cg.data_ptr(), None if c_str is None else _lib.i64_array(c_str),
                            alpha, beta, got.data_ptr(), _lib.i64_array((0, n + 3, 1)), _lib.stream_of(got))
        _lib.check(rc, what)
        alpha_e, beta_e = (alpha, beta) if c is not None else (alpha, 0.0)
        torch.cuda.synchronize()
        assert big[:, 0].abs().sum() == 0 and big[:, 1 + n:].abs().sum() == 0, what
    cc = None if c is None else (c.expand(m, n) if c.dim() == 1 else c)
    if dtype == torch.float32:
        an = to_np(a[rows])
        cn = None if cc is None else to_np(cc[rows])
        exp = from_np(O.gemm(an, to_np(b), "f32", cn, alpha_e, beta_e), "f32")
        rtol, atol = TOL_GEMM["f32"]
        assert_close(got[rows], exp, rtol, atol * max(1.0, k**0.5), what)
    else:
        assert_gemm_ulp(got, a, b, DT_NAME[dtype], cc, alpha_e, beta_e, what, rows=rows)
