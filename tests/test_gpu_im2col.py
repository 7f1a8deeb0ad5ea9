"""GPU parity: im2col through the C ABI against the oracle, bit for bit.

Mirrors the reference's tests/test_im2col.py -- its six (shape, kernel,
dilation, padding, stride) cases x fp32 / fp16 / bf16 / fp64 / bool / int32 /
int64 x contiguous and transposed (non-contiguous) input, and the empty
output shape rejection -- plus int8 / uint8 / int16, the torch CPU golden
vectors, every kernel variant (LDS-staged and direct planes, vector and
element stores, 1- to 8-byte elements), 1-element argument iterables, the
argument checks, and a conv-sized (32, 256, 56, 56) bf16 unfold on sampled
images."""

import os

import numpy as np
import pytest
import torch

import ntops_amd
from ntops_amd import _lib
from oracle import ops as O
from tests.helpers import DT_NAME, TORCH_DT, from_np, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

im2col = ntops_amd.torch.im2col
HERE = os.path.dirname(os.path.abspath(__file__))

REF_CASES = (
    ((2, 3, 8, 8), (3, 3), 1, 0, 1),
    ((1, 4, 10, 12), (5, 3), 1, 1, (2, 1)),
    ((2, 2, 16, 16), (4, 4), 1, 0, (4, 4)),
    ((3, 6, 7, 9), (3, 2), 1, 0, (1, 1)),
    ((1, 8, 9, 11), (2, 3), 1, 1, (1, 2)),
    ((2, 5, 12, 6), (3, 3), 2, (2, 1), (2, 1)),
)
DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.float64, torch.bool, torch.int32, torch.int64,
          torch.int8, torch.uint8, torch.int16)


def pair(v):
    if isinstance(v, int):
        return (v, v)
    v = tuple(v)
    return (v[0], v[0]) if len(v) == 1 else v


def make_input(shape, dtype, g):
    if dtype == torch.bool:
        return torch.randint(0, 2, shape, generator=g).bool()
    if dtype.is_floating_point:
        return torch.randn(shape, generator=g).to(dtype)
    return torch.randint(-100, 100, shape, generator=g).to(dtype)


def expect(x, ks, dil, pad, st):
    return from_np(O.im2col(to_np(x), pair(ks), pair(dil), pair(pad), pair(st)), DT_NAME[x.dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("noncontiguous", (False, True))
@pytest.mark.parametrize("shape, ks, dil, pad, st", REF_CASES)
def test_im2col_reference_grid(shape, ks, dil, pad, st, noncontiguous, dtype):
    g = torch.Generator().manual_seed(sum(shape))
    x = make_input(shape, dtype, g)
    xg = x.cuda()
    if noncontiguous:  # the reference's transposed input
        x = x.transpose(2, 3)
        xg = xg.transpose(2, 3)
    got = im2col(xg, kernel_size=ks, dilation=dil, padding=pad, stride=st)
    assert got.dtype == dtype
    assert torch.equal(got.cpu(), expect(x, ks, dil, pad, st))


def test_im2col_golden_vectors():
    gold = np.load(os.path.join(HERE, "golden", "golden_im2col.npz"))
    cases = {
        "k33": ((3, 3), 1, 0, 1), "k53_p1_s21": ((5, 3), 1, 1, (2, 1)), "k44_s44": ((4, 4), 1, 0, (4, 4)),
        "k32": ((3, 2), 1, 0, (1, 1)), "k23_p1_s12": ((2, 3), 1, 1, (1, 2)),
        "k33_d2_p21_s21": ((3, 3), 2, (2, 1), (2, 1)), "k11_d3": ((1, 1), 3, 0, 1),
        "k33_d23_p32": ((3, 3), (2, 3), (3, 2), 1),
    }
    for name, (ks, dil, pad, st) in cases.items():
        for dt in ("f32", "f16", "bf16", "f64", "bool", "i32", "i64"):
            x = from_np(gold[f"{name}_x_{dt}"], dt).cuda()
            got = im2col(x, ks, dil, pad, st)
            assert torch.equal(got.cpu(), from_np(gold[f"{name}_y_{dt}"], dt)), f"{name} {dt}"


# (shape, kernel, padding, stride, dtype, expected kernel): planes up to 64
# KiB are staged in LDS, larger ones gathered from global memory; rows whose
# length keeps every row start on the run's byte size take vector stores;
# 16-bit stride-1 problems with output rows of a multiple of 8 pixels take
# the zero-padded LDS plane with register-selected taps (kernel widths 1-9;
# plane loaded by 16-byte rows, or element by element when W % 8 != 0).
VARIANTS = (
    ((2, 3, 18, 24), 3, 1, 1, torch.bfloat16, "im2col_s1 kw3"),
    ((1, 2, 12, 16), 5, 2, 1, torch.float16, "im2col_s1 kw5"),
    ((1, 3, 9, 9), 2, 0, 1, torch.bfloat16, "im2col_s1 kw2"),
    ((1, 2, 8, 16), 1, 0, 1, torch.bfloat16, "im2col_s1 kw1"),
    ((1, 2, 10, 16), 7, 3, 1, torch.bfloat16, "im2col_s1 kw7"),
    ((2, 1, 9, 8), 9, 4, 1, torch.float16, "im2col_s1 kw9"),
    ((1, 2, 6, 17), 4, 1, 1, torch.bfloat16, "im2col_s1 kw4"),          # ow = 16, W % 8 != 0
    ((2, 3, 20, 20), 3, 1, 1, torch.bfloat16, "im2col_lds es2 vec"),        # L = 400
    ((2, 3, 20, 21), 3, 1, 1, torch.bfloat16, "im2col_lds es2 scalar"),     # L = 420
    ((2, 3, 20, 20), 3, 1, 1, torch.uint8, "im2col_lds es1 vec"),
    ((1, 2, 10, 14), 2, 0, 1, torch.int8, "im2col_lds es1 scalar"),       # L = 117
    ((2, 4, 16, 16), 3, 1, 1, torch.float32, "im2col_lds es4 vec"),
    ((2, 4, 16, 16), 3, 1, 1, torch.float64, "im2col_lds es8 vec"),
    ((1, 2, 7, 7), 3, 0, 1, torch.float64, "im2col_lds es8 scalar"),
    ((1, 2, 130, 130), 3, 1, 1, torch.float32, "im2col_direct es4 vec"),    # 66 KiB plane
    ((1, 2, 181, 183), 5, 2, 2, torch.bfloat16, "im2col_direct es2 scalar"),
    ((1, 1, 91, 91), 2, 0, 2, torch.int64, "im2col_direct es8 scalar"),   # L = 2025
    ((2, 1, 260, 264), 3, 1, 1, torch.uint8, "im2col_direct es1 vec"),
)


@pytest.mark.parametrize("shape, ks, pad, st, dtype, kernel", VARIANTS)
def test_im2col_kernel_variants(shape, ks, pad, st, dtype, kernel):
    g = torch.Generator().manual_seed(7)
    x = make_input(shape, dtype, g)
    got = im2col(x.cuda(), ks, 1, pad, st)
    assert _lib.last_kernel() == kernel
    assert torch.equal(got.cpu(), expect(x, ks, 1, pad, st))


def test_im2col_stride1_strided_input():
    """The stride-1 16-bit kernel on a channels-last view (column stride C):
    the plane is loaded element by element, the taps as for a contiguous one."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 16, 16, 5, generator=g).bfloat16()  # N, H, W, C
    xv = x.cuda().permute(0, 3, 1, 2)                         # (2, 5, 16, 16), strides (1280, 1, 80, 5)
    got = im2col(xv, 3, 1, 1, 1)
    assert _lib.last_kernel() == "im2col_s1 kw3"
    assert torch.equal(got.cpu(), expect(x.permute(0, 3, 1, 2).contiguous(), 3, 1, 1, 1))


def test_im2col_argument_forms_and_checks():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 2, 9, 10, generator=g)
    xg = x.cuda()
    got = im2col(xg, (3,), dilation=[2], padding=(1,), stride=[2])
    assert torch.equal(got.cpu(), expect(x, 3, 2, 1, 2))
    with pytest.raises(RuntimeError):
        im2col(torch.randn((1, 1, 2, 2), device="cuda"), kernel_size=(3, 3), padding=0, stride=1)
    with pytest.raises(RuntimeError):
        im2col(xg[0], 3)
    for bad in ({"kernel_size": 0}, {"kernel_size": 3, "dilation": 0}, {"kernel_size": 3, "stride": (1, 0)},
                {"kernel_size": 3, "padding": -1}):
        with pytest.raises(RuntimeError):
            im2col(xg, **bad)
    with pytest.raises(TypeError):
        im2col(xg, (3, 3, 3))
    with pytest.raises(RuntimeError):
        im2col(x, 3)  # CPU tensor: no fallback
    empty = im2col(torch.empty(0, 3, 8, 8, device="cuda"), 3)
    assert empty.shape == (0, 27, 36)


def test_im2col_conv_sized():
    """bf16 (32, 256, 56, 56), 3x3, padding 1 (the conv2d workload's
    unfold): images 0, 17 and 31 against the oracle bit for bit, and the
    padding zeros counted over the whole output."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(32, 256, 56, 56, generator=g).bfloat16()
    got = im2col(x.cuda(), 3, padding=1)
    assert got.shape == (32, 256 * 9, 3136)
    for n in (0, 17, 31):
        assert torch.equal(got[n:n + 1].cpu(), expect(x[n:n + 1], 3, 1, 1, 1)), f"image {n}"
    # the border taps read padding: per channel, 8 of 9 taps lose one row or
    # column of 56 pixels (corners two), 4 * 56 + 4 * (2 * 56 - 1) = 668 zeros
    # (randn inputs are never exactly zero)
    zeros = (got == 0).sum().item()
    assert zeros == 32 * 256 * 668


@pytest.mark.parametrize("dtype, hw, ks, kernel", [
    (torch.float32, (2, 2), (2, 2), "im2col_lds"),  # 256-thread blocks: 2^24 planes fill one grid dimension
    (torch.bfloat16, (1, 8), (1, 1), "im2col_s1"),
])
def test_im2col_more_than_2_24_planes(dtype, hw, ks, kernel):
    """2^24 + 37 (image, channel) planes, one workgroup each: the grid is two
    dimensional (one dimension's work-item count is 32-bit).  A kernel that
    covers a whole plane unfolds it into one output column run, so the
    expected output is a reshape of the input."""
    c = (1 << 24) + 37
    x = torch.randn(1, c, *hw, device="cuda").to(dtype)
    got = im2col(x, ks)
    assert _lib.last_kernel().startswith(kernel), _lib.last_kernel()
    oh, ow = hw[0] - ks[0] + 1, hw[1] - ks[1] + 1
    assert got.shape == (1, c * ks[0] * ks[1], oh * ow)
    exp = x.reshape(1, c, hw[0] * hw[1]) if ks == (1, 1) else x.reshape(1, c * 4, 1)
    assert torch.equal(got, exp.reshape(got.shape))
    del got, x, exp
    torch.cuda.empty_cache()
