"""GPU parity: conv2d through the C ABI against the oracle.

Mirrors the reference's tests/test_conv2d.py grid -- (n, c, h, w, k) =
(2, 3, 112, 112, 4), 1x1 and 3x3 kernels, stride / padding / dilation in
{1, 2 or 0, 1, (2, 3)}, fp32 (1e-5) and fp16 (1e-3) -- plus bf16
(1.6e-2), shapes that take the unfold + matrix-core GEMM path (fp32, fp16,
bf16), several image chunks through a small workspace, strided and
channels-last inputs, unbatched input, 'same' / 'valid' padding, no bias,
the argument checks, and the (32, 256, 56, 56) x (256, 256, 3, 3) workload
on sampled images and channels."""

import itertools

import numpy as np
import pytest
import torch

import ntops_amd
from ntops_amd import _lib
from oracle import ops as O
from tests.helpers import DT_NAME, assert_close, from_np, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

conv2d = ntops_amd.torch.conv2d
TOL = {torch.float32: (1e-5, 1e-5), torch.float16: (1e-3, 1e-3), torch.bfloat16: (1.6e-2, 1.6e-2)}


def pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


def oracle(x, w, b, stride, padding, dilation, out_hw=None):
    dt = DT_NAME[x.dtype]
    return from_np(O.conv2d(to_np(x), to_np(w), dt, None if b is None else to_np(b), pair(stride), pair(padding),
                            pair(dilation), out_hw), dt)


REF_GRID = list(itertools.product(((1, 1), (3, 3)), (1, 2, (2, 3)), (0, 1, (2, 3)), (1, 2, (2, 3))))


@pytest.mark.parametrize("dtype", (torch.float32, torch.float16, torch.bfloat16))
@pytest.mark.parametrize("rs, stride, padding, dilation", REF_GRID)
def test_conv2d_reference_grid(rs, stride, padding, dilation, dtype):
    g = torch.Generator().manual_seed(hash((rs, stride, padding, dilation)) & 0xffff)
    n, c, h, w, k = 2, 3, 112, 112, 4
    x = torch.randn(n, c, h, w, generator=g).to(dtype)
    wt = torch.randn(k, c, *rs, generator=g).to(dtype)
    b = torch.randn(k, generator=g).to(dtype)
    got = conv2d(x.cuda(), wt.cuda(), bias=b.cuda(), stride=stride, padding=padding, dilation=dilation)
    assert_close(got, oracle(x, wt, b, stride, padding, dilation), *TOL[dtype], "conv2d")


GEMM_CASES = [
    # (n, c, h, w, k, r, s, stride, padding, dilation, bias)
    (2, 64, 28, 28, 64, 3, 3, 1, 1, 1, True),
    (3, 32, 17, 19, 48, 3, 3, 2, 1, 1, True),
    (2, 64, 20, 21, 40, 3, 3, (2, 3), (2, 3), (2, 3), False),
    (1, 128, 14, 14, 256, 1, 1, 1, 0, 1, True),
    (2, 16, 31, 29, 64, 5, 5, 1, 2, 1, True),
    (2, 48, 16, 16, 64, 3, 3, 1, 1, 1, True),
    (1, 128, 16, 16, 256, 1, 1, 1, 0, 1, True),
    (2, 32, 33, 22, 64, 3, 3, (2, 1), (1, 2), (2, 3), True),
    # output planes of P Q % 8 != 0 pixels (7 x 7, 9 x 9): unfold + GEMM at the
    # padded width, then the planes copied out
    (4, 64, 7, 7, 64, 3, 3, 1, 1, 1, True),
    (3, 32, 9, 9, 40, 3, 3, 1, 1, 1, False),
    # 16-63 output pixels, which the GEMM paths take from 16 on: 4 x 4 and
    # 6 x 6 planes (channels-last), 5 x 5 with C % 32 != 0 (padded unfold)
    (8, 64, 4, 4, 64, 3, 3, 1, 1, 1, True),
    (4, 64, 6, 6, 96, 3, 3, 1, 1, 1, False),
    (4, 48, 5, 5, 64, 3, 3, 1, 1, 1, True),
    # C R S not a multiple of 8: unfold into KP = C R S rounded up to 8 rows
    # (zero pad rows) against a zero-padded K x KP copy of W -- a 3-channel
    # 7 x 7 stride-2 stem (147 -> 152), 5 x 5 over 5 channels (125 -> 128),
    # and 3 x 3 over 9 channels (81 -> 88) on an 11 x 13 plane (also padded
    # output rows)
    (2, 3, 64, 64, 64, 7, 7, 2, 3, 1, True),
    (2, 5, 20, 20, 32, 5, 5, 1, 2, 1, False),
    (3, 9, 11, 13, 40, 3, 3, 1, 1, 1, True),
]


def expected_path(dtype, c, p, q, stride, crs):
    """Kernel family of the GEMM paths: the channels-last implicit GEMM for
    16-bit data with C % 32 == 0 and P * Q % 4 == 0, the implicit GEMM over
    shifted planes for the rest of the 16-bit stride-1 problems with
    Q % 8 == 0 and C R S % 8 == 0, otherwise unfold + GEMM."""
    if dtype != torch.float32 and c % 32 == 0 and (p * q) % 4 == 0:
        return " conv_cl"
    if dtype != torch.float32 and pair(stride) == (1, 1) and q % 8 == 0 and crs % 8 == 0:
        return " conv"
    return ""


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("case", GEMM_CASES)
def test_conv2d_gemm_path(case, dtype):
    n, c, h, w, k, r, s, stride, padding, dilation, has_bias = case
    g = torch.Generator().manual_seed(n * 1000 + c + k)
    x = torch.randn(n, c, h, w, generator=g).to(dtype)
    wt = (torch.randn(k, c, r, s, generator=g) / (c * r * s) ** 0.5).to(dtype)
    b = torch.randn(k, generator=g).to(dtype) if has_bias else None
    (sh, sw), (ph, pw), (dh, dw) = pair(stride), pair(padding), pair(dilation)
    P = (h + 2 * ph - dh * (r - 1) - 1) // sh + 1
    Q = (w + 2 * pw - dw * (s - 1) - 1) // sw + 1
    ws = _lib.load().ntops_conv2d_workspace(_lib.dtype_code(dtype), n, c, h, w, k, r, s, P, Q, sh, sw, ph, pw, dh, dw,
                                            _lib.i64_array(wt.stride()), _lib.i64_array((k * P * Q, P * Q, Q, 1)))
    assert ws > 0, "expected the GEMM path"
    got = conv2d(x.cuda(), wt.cuda(), bias=None if b is None else b.cuda(), stride=stride, padding=padding,
                 dilation=dilation)
    kern = _lib.last_kernel()
    want = expected_path(dtype, c, P, Q, stride, c * r * s)
    assert kern.startswith("gemm_") and (kern.endswith(want) if want else not kern.endswith("conv") and
                                         not kern.endswith("conv_cl")), kern
    exp = oracle(x, wt, b, stride, padding, dilation)
    tol = (2e-5, 2e-5) if dtype == torch.float32 else TOL[dtype]
    assert_close(got, exp, *tol, "conv2d gemm path")


def test_conv2d_padded_unfold_past_2_24_outputs():
    """bf16 (256, 512, 7, 7) * (2048, 512, 1, 1): 49-pixel output planes take
    the unfold + GEMM at the padded width, whose planes are then copied out of
    the workspace; 256 x 2048 x 49 = 25.7M outputs, more than the copy's
    capped grid covers in one pass (2^24 threads), so the copy must loop.
    Images at both ends and in the middle against the oracle, and the output
    must hold no element the copy skipped (the output is pre-filled with NaN)."""
    g = torch.Generator().manual_seed(29)
    n, c, h, k = 256, 512, 7, 2048
    x = torch.randn(n, c, h, h, generator=g).bfloat16()
    wt = (torch.randn(k, c, 1, 1, generator=g) / c ** 0.5).bfloat16()
    b = torch.randn(k, generator=g).bfloat16()
    out = torch.full((n, k, h, h), float("nan"), dtype=torch.bfloat16, device="cuda")
    lib = _lib.load()
    geo = (n, c, h, h, k, 1, 1, h, h, 1, 1, 0, 0, 1, 1)
    st = lambda t: _lib.i64_array(t.stride())  # noqa: E731
    need = lib.ntops_conv2d_workspace(_lib.BF16, *geo, st(wt), st(out))
    assert 0 < need <= 1 << 28  # every image in one chunk
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    xg, wg, bg = x.cuda(), wt.cuda(), b.cuda()
    rc = lib.ntops_conv2d(_lib.BF16, *geo, xg.data_ptr(), st(xg), wg.data_ptr(), st(wg), bg.data_ptr(), 1,
                          out.data_ptr(), st(out), ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.ntops_last_error()
    assert not _lib.last_kernel().endswith("conv_cl"), _lib.last_kernel()
    torch.cuda.synchronize()
    assert n * k * h * h > 1 << 24
    assert not torch.isnan(out).any().item(), "output elements left unwritten"
    got = out.cpu()
    for img in (0, 128, 255):
        exp = oracle(x[img:img + 1], wt, b, 1, 0, 1)
        assert_close(got[img:img + 1], exp, *TOL[torch.bfloat16], f"image {img}")


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_conv2d_channels_last_256_tiles(dtype):
    """240 images of 16 x 16 pixels into 256 channels: 240 full 256 x 256
    tiles, the channels-last implicit GEMM's even large-tile kernel (K = 288);
    images at both ends and in the middle against the oracle."""
    g = torch.Generator().manual_seed(17)
    n, c, h, k = 240, 32, 16, 256
    x = torch.randn(n, c, h, h, generator=g).to(dtype)
    wt = (torch.randn(k, c, 3, 3, generator=g) / 17).to(dtype)
    b = torch.randn(k, generator=g).to(dtype)
    got = conv2d(x.cuda(), wt.cuda(), b.cuda(), padding=1)
    assert _lib.last_kernel() == "gemm_mfma 256x256 s4 A:K B:K even conv_cl"
    for img in (0, 119, 239):
        exp = oracle(x[img:img + 1], wt, b, 1, 1, 1)
        assert_close(got[img:img + 1], exp, *TOL[dtype], f"image {img}")


def test_conv2d_workspace_chunks():
    """One image per chunk (workspace of exactly what one image needs), and a
    workspace too small for one image (direct kernel): both equal the
    one-chunk run."""
    dtype = torch.bfloat16
    n, c, h, w, k = 5, 64, 18, 18, 64
    g = torch.Generator().manual_seed(9)
    x = torch.randn(n, c, h, w, generator=g).to(dtype).cuda()
    wt = (torch.randn(k, c, 3, 3, generator=g) / 24).to(dtype).cuda()
    b = torch.randn(k, generator=g).to(dtype).cuda()
    full = conv2d(x, wt, bias=b, padding=1)
    lib = _lib.load()
    geo = (n, c, h, w, k, 3, 3, h, w, 1, 1, 1, 1, 1, 1)
    st = lambda t: _lib.i64_array(t.stride())  # noqa: E731
    total = lib.ntops_conv2d_workspace(_lib.dtype_code(dtype), *geo, st(wt), st(full))
    one = lib.ntops_conv2d_workspace(_lib.dtype_code(dtype), 1, *geo[1:], st(wt), st(full))
    # the bytes of every image plus a per-call part (the reordered weights)
    assert 0 < one < total and (total - one) % (n - 1) == 0
    for ws_bytes in (one, one - 16):
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")
        out = torch.empty_like(full)
        rc = lib.ntops_conv2d(_lib.dtype_code(dtype), *geo, x.data_ptr(), st(x), wt.data_ptr(), st(wt), b.data_ptr(), 1,
                              out.data_ptr(), st(out), ws.data_ptr(), ws_bytes, _lib.stream_of(out))
        _lib.check(rc, "conv2d")
        assert_close(out, full, 1.6e-2, 1.6e-2, f"workspace {ws_bytes}")
    assert_close(full, oracle(x.cpu(), wt.cpu(), b.cpu(), 1, 1, 1), 1.6e-2, 1.6e-2, "one chunk")


@pytest.mark.parametrize("n, c, h, k, stride", [(8, 256, 14, 256, 1), (6, 128, 28, 128, 2), (3, 96, 20, 96, 1)])
def test_conv2d_f32_split_k(n, c, h, k, stride):
    """fp32 unfold + GEMM with few output tiles: the batched GEMM splits K
    through the rest of the workspace (padded output planes included), and
    equals the oracle; with a workspace that holds the images but not the
    partial products it runs unsplit and agrees to fp32 summation order."""
    g = torch.Generator().manual_seed(n + c + k)
    x = torch.randn(n, c, h, h, generator=g)
    wt = torch.randn(k, c, 3, 3, generator=g) / (9 * c) ** 0.5
    b = torch.randn(k, generator=g)
    got = conv2d(x.cuda(), wt.cuda(), bias=b.cuda(), stride=stride, padding=1)
    assert _lib.last_kernel().startswith("gemm_f32_lds m128 B:N splitk"), _lib.last_kernel()
    assert_close(got, oracle(x, wt, b, stride, 1, 1), 2e-5, 2e-5, "conv2d f32 split-K")
    lib = _lib.load()
    p = (h + 2 - 3) // stride + 1
    geo = (n, c, h, h, k, 3, 3, p, p, stride, stride, 1, 1, 1, 1)
    st = lambda t: _lib.i64_array(t.stride())  # noqa: E731
    total = lib.ntops_conv2d_workspace(_lib.dtype_code(torch.float32), *geo, st(wt), st(got))
    one = lib.ntops_conv2d_workspace(_lib.dtype_code(torch.float32), 1, *geo[1:], st(wt), st(got))
    assert total > 0 and one > 0
    # the images' bytes without the split's: total less the partial products (and their alignment room)
    split = lib.ntops_gemm_workspace(_lib.dtype_code(torch.float32), n, k, -(-p * p // 8) * 8, c * 9)
    assert split > 0
    images = total - (split + 511) // 256 * 256
    ws = torch.empty(images, dtype=torch.uint8, device="cuda")
    out = torch.empty_like(got)
    xg, wg, bg = x.cuda(), wt.cuda(), b.cuda()
    rc = lib.ntops_conv2d(_lib.dtype_code(torch.float32), *geo, xg.data_ptr(), st(xg), wg.data_ptr(), st(wg),
                          bg.data_ptr(), 1, out.data_ptr(), st(out), ws.data_ptr(), images, _lib.stream_of(out))
    _lib.check(rc, "conv2d")
    assert "splitk" not in _lib.last_kernel(), _lib.last_kernel()
    assert_close(out, got, 2e-5, 2e-5, "unsplit against split")


@pytest.mark.parametrize("dtype", (torch.float32, torch.bfloat16))
def test_conv2d_layouts_and_forms(dtype):
    g = torch.Generator().manual_seed(3)
    tol = TOL[dtype] if dtype != torch.float32 else (2e-5, 2e-5)
    # channels-last input (strided NCHW view) on both paths
    for c, k in ((3, 4), (64, 64)):
        x = torch.randn(2, c, 15, 16, generator=g).to(dtype)
        wt = (torch.randn(k, c, 3, 3, generator=g) / (9 * c) ** 0.5).to(dtype)
        xc = x.cuda().to(memory_format=torch.channels_last)
        assert not xc.is_contiguous()
        assert_close(conv2d(xc, wt.cuda(), padding=1), oracle(x, wt, None, 1, 1, 1), *tol, "channels-last")
        # a sliced (non-contiguous) weight: the direct kernel for 3
        # channels, a K x C R S copy in the workspace for the unfold path
        # for 64
        wbig = torch.randn(k, c, 3, 5, generator=g).to(dtype)
        ws = wbig[:, :, :, 1:4]
        assert_close(conv2d(x.cuda(), wbig.cuda()[:, :, :, 1:4], stride=2), oracle(x, ws.contiguous(), None, 2, 0, 1),
                     *tol, "strided weight")
    # unbatched input, 'valid' and 'same' (asymmetric: even kernel)
    x = torch.randn(3, 12, 13, generator=g).to(dtype)
    wt = torch.randn(5, 3, 2, 4, generator=g).to(dtype)
    b = torch.randn(5, generator=g).to(dtype)
    got = conv2d(x.cuda(), wt.cuda(), b.cuda(), padding="valid")
    assert got.shape == (5, 11, 10)
    assert_close(got, oracle(x[None], wt, b, 1, 0, 1)[0], *tol, "valid")
    got = conv2d(x.cuda(), wt.cuda(), b.cuda(), padding="same")
    assert got.shape == (5, 12, 13)
    assert_close(got, oracle(x[None], wt, b, 1, (0, 1), 1, (12, 13))[0], *tol, "same")


def test_conv2d_argument_checks():
    x = torch.randn(1, 4, 8, 8, device="cuda")
    w = torch.randn(4, 4, 3, 3, device="cuda")
    with pytest.raises(AssertionError):
        conv2d(x, w, groups=2)
    with pytest.raises(RuntimeError):
        conv2d(x, w.half())
    with pytest.raises(RuntimeError):
        conv2d(x, w, padding="same", stride=2)
    with pytest.raises(RuntimeError):
        conv2d(x, torch.randn(4, 4, 9, 9, device="cuda"))
    with pytest.raises(RuntimeError):
        conv2d(x, torch.randn(4, 3, 3, 3, device="cuda"))


def test_conv2d_workload_full_size():
    """bf16 (32, 256, 56, 56) * (256, 256, 3, 3), padding 1: images 0 and 31
    on 16 output channels against the oracle, and every output finite."""
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(0)
    x = torch.randn(32, 256, 56, 56, generator=g).to(dtype)
    wt = (torch.randn(256, 256, 3, 3, generator=g) / 48).to(dtype)
    b = torch.randn(256, generator=g).to(dtype)
    got = conv2d(x.cuda(), wt.cuda(), b.cuda(), padding=1)
    ch = torch.arange(0, 256, 16)
    for img in (0, 31):
        exp = oracle(x[img:img + 1], wt[ch], b[ch], 1, 1, 1)
        assert_close(got[img:img + 1, ch], exp, 1.6e-2, 1.6e-2, f"image {img}")
    assert torch.isfinite(got).all()


@pytest.mark.parametrize("form", ("misaligned", "padded channel stride"))
def test_conv2d_output_views_the_implicit_gemm_cannot_store(form):
    """Outputs the implicit GEMM's 8-byte stores cannot serve -- an address
    2 bytes past alignment, or a channel stride that is not a multiple of 4
    elements -- take the unfold + GEMM path instead of failing."""
    dtype = torch.bfloat16
    n, c, h, k = 2, 64, 16, 64
    g = torch.Generator().manual_seed(11)
    x = torch.randn(n, c, h, h, generator=g).to(dtype)
    wt = (torch.randn(k, c, 3, 3, generator=g) / 24).to(dtype)
    b = torch.randn(k, generator=g).to(dtype)
    if form == "misaligned":
        buf = torch.empty(n * k * h * h + 1, dtype=dtype, device="cuda")
        out = buf[1:].view(n, k, h, h)
    else:
        buf = torch.empty(n, k, h * h + 2, dtype=dtype, device="cuda")
        out = buf[:, :, : h * h].view(n, k, h, h)
    lib = _lib.load()
    st = lambda t: _lib.i64_array(t.stride())  # noqa: E731
    geo = (n, c, h, h, k, 3, 3, h, h, 1, 1, 1, 1, 1, 1)
    ws_bytes = lib.ntops_conv2d_workspace(_lib.BF16, *geo, st(wt), st(out)) * 16  # room for the unfold path
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    xg, wg, bg = x.cuda(), wt.cuda(), b.cuda()
    rc = lib.ntops_conv2d(_lib.BF16, *geo, xg.data_ptr(), st(xg), wg.data_ptr(), st(wg), bg.data_ptr(), 1,
                          out.data_ptr(), st(out), ws.data_ptr(), ws_bytes, _lib.stream_of(out))
    _lib.check(rc, f"conv2d into a {form} output")
    assert _lib.last_kernel().startswith("gemm_") and not _lib.last_kernel().endswith(" conv")
    assert_close(out, oracle(x, wt, b, 1, 1, 1), 1.6e-2, 1.6e-2, form)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float32))
def test_conv2d_padded_depth_weight_copies(dtype):
    """The unfold path with W copied into the workspace (zero columns past
    C R S): weights whose rows are not C R S contiguous elements (a slice,
    an odd row stride from a wider allocation) and C R S % 8 != 0, with and
    without bias, against the oracle; the second call reuses a workspace
    whose pad rows held other data."""
    g = torch.Generator().manual_seed(21)
    tol = TOL[dtype] if dtype != torch.float32 else (2e-5, 2e-5)
    x = torch.randn(2, 3, 40, 36, generator=g).to(dtype)
    wfull = (torch.randn(64, 3, 7, 9, generator=g) / 12).to(dtype)
    wsl = wfull[:, :, :, 1:8]  # (64, 3, 7, 7), rows of 147 elements at stride 189
    b = torch.randn(64, generator=g).to(dtype)
    got = conv2d(x.cuda(), wfull.cuda()[:, :, :, 1:8], bias=b.cuda(), stride=2, padding=3)
    assert _lib.last_kernel().startswith("gemm_"), _lib.last_kernel()
    assert_close(got, oracle(x, wsl.contiguous(), b, 2, 3, 1), *tol, "sliced 7 x 7 weight")
    # through the C ABI, one workspace for both calls: call 1 (C R S = 588,
    # 592 rows) fills the workspace with its W copy and unfold rows, call 2
    # (C R S = 147, 152 rows) must see zeros in its pad rows, which lie over
    # call 1's data
    lib = _lib.load()
    st = lambda t: _lib.i64_array(t.stride())  # noqa: E731
    dt = _lib.dtype_code(dtype)
    x1 = torch.randn(2, 12, 40, 36, generator=g).to(dtype).cuda()
    w1 = (torch.randn(64, 12, 7, 7, generator=g) / 24).to(dtype).cuda()
    w2 = wsl.contiguous().cuda()
    outs = []
    geo1 = (2, 12, 40, 36, 64, 7, 7, 20, 18, 2, 2, 3, 3, 1, 1)
    geo2 = (2, 3, 40, 36, 64, 7, 7, 20, 18, 2, 2, 3, 3, 1, 1)
    o1 = torch.empty(2, 64, 20, 18, dtype=dtype, device="cuda")
    o2 = torch.empty_like(o1)
    need = max(lib.ntops_conv2d_workspace(dt, *geo1, st(w1), st(o1)), lib.ntops_conv2d_workspace(dt, *geo2, st(w2), st(o2)))
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    for geo, xx, ww, oo in ((geo1, x1, w1, o1), (geo2, x.cuda(), w2, o2)):
        rc = lib.ntops_conv2d(dt, *geo, xx.data_ptr(), st(xx), ww.data_ptr(), st(ww), None, 0, oo.data_ptr(), st(oo),
                              ws.data_ptr(), need, _lib.stream_of(oo))
        _lib.check(rc, "conv2d")
        assert _lib.last_kernel().startswith("gemm_"), _lib.last_kernel()
        outs.append(oo)
    torch.cuda.synchronize()
    assert_close(outs[0], oracle(x1.cpu(), w1.cpu(), None, 2, 3, 1), *tol, "C R S = 588")
    assert_close(outs[1], oracle(x, wsl.contiguous(), None, 2, 3, 1), *tol, "C R S = 147 after 588")


@pytest.mark.parametrize(
    "dtype, n, c, h, w, k, r, stride, pad, dil",
    [
        # input planes past the 64 KiB that k_im2col_plane stages whole: the
        # unfold stages a band of input rows per (image, channel, 512 pixels)
        (torch.bfloat16, 2, 3, 192, 192, 64, 7, 2, 3, 1),  # stem: C R S = 147 -> 152 rows
        (torch.float32, 1, 4, 130, 130, 32, 5, 1, 2, 2),  # dilated, 126 x 126 plane (padded out rows)
        (torch.bfloat16, 1, 8, 200, 180, 32, 3, 1, 1, 1),  # Q % 8 != 0 keeps it off the shifted planes
    ],
)
def test_conv2d_band_unfold(dtype, n, c, h, w, k, r, stride, pad, dil):
    g = torch.Generator().manual_seed(c * 100 + h)
    x = torch.randn(n, c, h, w, generator=g).to(dtype)
    wt = (torch.randn(k, c, r, r, generator=g) / (c * r * r) ** 0.5).to(dtype)
    b = torch.randn(k, generator=g).to(dtype)
    got = conv2d(x.cuda(), wt.cuda(), bias=b.cuda(), stride=stride, padding=pad, dilation=dil)
    assert _lib.last_kernel().startswith("gemm_"), _lib.last_kernel()
    tol = TOL[dtype] if dtype != torch.float32 else (2e-5, 2e-5)
    assert_close(got, oracle(x, wt, b, stride, pad, dil), *tol, "band unfold")
