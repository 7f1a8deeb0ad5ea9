"""ntops_conv2d_noalloc -- the library's fixed per-GPU scratch in place of a
workspace argument -- against ntops_conv2d with a caller-owned workspace,
through the C ABI: two calls in a row, the second smaller and on the other
workspace path (so it runs over scratch that still holds the first call's
data), each checked against the workspace entry point at the bf16 / fp16
tolerance and the small one also against the oracle."""


import pytest
import torch

from ntops_amd import _lib
from oracle import ops as O
from tests.helpers import assert_close, from_np, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

MAX_SCRATCH = 64 << 20  # NTOPS_CONV2D_NOALLOC_MAX_SCRATCH


def _st(t):
    return _lib.i64_array(t.stride())


def _out_size(h, r, stride, pad, dil):
    return (h + 2 * pad - dil * (r - 1) - 1) // stride + 1


def _conv(entry, x, wt, b, stride, pad):
    lib = _lib.load()
    n, c, h, w = x.shape
    k, _, r, s = wt.shape
    p, q = _out_size(h, r, stride, pad, 1), _out_size(w, s, stride, pad, 1)
    out = torch.empty(n, k, p, q, dtype=x.dtype, device=x.device)
    geo = (n, c, h, w, k, r, s, p, q, stride, stride, pad, pad, 1, 1)
    dt = _lib.dtype_code(x.dtype)
    args = (x.data_ptr(), _st(x), wt.data_ptr(), _st(wt), b.data_ptr(), b.stride(0), out.data_ptr(), _st(out))
    stream = _lib.stream_of(out)
    if entry == "noalloc":
        rc = lib.ntops_conv2d_noalloc(dt, *geo, *args, stream)
    else:
        ws_bytes = lib.ntops_conv2d_workspace(dt, *geo, _st(wt), _st(out))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        rc = lib.ntops_conv2d(dt, *geo, *args, ws.data_ptr(), ws_bytes, stream)
        per_image = lib.ntops_conv2d_workspace(dt, 1, *geo[1:], _st(wt), _st(out))
        assert per_image > 0, "expected a workspace path"
        torch.cuda.synchronize()
        del ws
    _lib.check(rc, f"conv2d {entry}")
    return out, geo


def _inputs(n, c, h, k, r, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, c, h, h, generator=g).to(dtype)
    wt = (torch.randn(k, c, r, r, generator=g) / (c * r * r) ** 0.5).to(dtype)
    b = torch.randn(k, generator=g).to(dtype)
    return x, wt, b


def test_conv2d_noalloc_matches_workspace_entry():
    # 1) bf16 (32, 256, 56, 56) * (256, 256, 3, 3), padding 1: the
    #    channels-last implicit GEMM, 1.7 MB per padded image plus 1.2 MB of
    #    reordered weights, all in the scratch at once.
    # 2) fp16 (3, 64, 21, 21) * (96, 64, 3, 3), stride 2, padding 1: the
    #    unfold + GEMM path (11 x 11 output pixels), smaller, over scratch
    #    holding call 1's padded images.
    cases = [
        ((32, 256, 56, 256, 3, torch.bfloat16, 0), 1, 1),
        ((3, 64, 21, 96, 3, torch.float16, 1), 2, 1),
    ]
    for (n, c, h, k, r, dtype, seed), stride, pad in cases:
        x, wt, b = _inputs(n, c, h, k, r, dtype, seed)
        xg, wg, bg = x.cuda(), wt.cuda(), b.cuda()
        ref, geo = _conv("workspace", xg, wg, bg, stride, pad)
        got, _ = _conv("noalloc", xg, wg, bg, stride, pad)
        torch.cuda.synchronize()
        what = f"conv2d_noalloc {tuple(x.shape)} stride {stride}"
        assert_close(got, ref, 1.6e-2, 1.6e-2, what)
        same = (got == ref).float().mean().item()
        assert same >= 0.99, f"{what}: only {same:.2%} of elements equal the workspace entry's"
        if n * c * h * h < 100000:
            dt = "bf16" if dtype == torch.bfloat16 else "f16"
            exp = from_np(O.conv2d(to_np(x), to_np(wt), dt, to_np(b), (stride, stride), (pad, pad), (1, 1)), dt)
            assert_close(got, exp, 1.6e-2, 1.6e-2, what + " vs oracle")
        del ref, got


def test_conv2d_noalloc_rejects_images_beyond_the_scratch():
    """One image needing more than the scratch holds: an error naming the
    limit, before any launch.  The tensors are null pointers, so a
    regression in the size check stops at ntops_conv2d's null-pointer check
    (a different message, the test fails) instead of launching kernels."""
    lib = _lib.load()
    n, c, h, k = 1, 256, 400, 64
    geo = (n, c, h, h, k, 3, 3, h, h, 1, 1, 1, 1, 1, 1)
    wst = _lib.i64_array((c * 9, 9, 3, 1))
    ost = _lib.i64_array((k * h * h, h * h, h, 1))
    need = lib.ntops_conv2d_workspace(_lib.BF16, *geo, wst, ost)
    assert need > MAX_SCRATCH
    xst = _lib.i64_array((c * h * h, h * h, h, 1))
    rc = lib.ntops_conv2d_noalloc(_lib.BF16, *geo, None, xst, None, wst, None, 0, None, ost, None)
    assert rc == 2 and "maximum" in lib.ntops_last_error().decode()
