"""Pins oracle.ops.im2col: torch CPU F.unfold golden vectors (bit-exact, every
dtype of the reference's test grid), a brute-force loop over every output
element, closed forms (a 1x1 window is a reshape, a strided 1x1 window is
subsampling, padding contributes exact zeros), and planted mistakes -- tap
order, ignored dilation, one-sided padding, swapped strides -- that those
checks must catch."""

import os

import numpy as np
import pytest

from oracle import ops as O

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = np.load(os.path.join(HERE, "golden", "golden_im2col.npz"))
CASES = {
    "k33": ((3, 3), 1, 0, 1),
    "k53_p1_s21": ((5, 3), 1, 1, (2, 1)),
    "k44_s44": ((4, 4), 1, 0, (4, 4)),
    "k32": ((3, 2), 1, 0, (1, 1)),
    "k23_p1_s12": ((2, 3), 1, 1, (1, 2)),
    "k33_d2_p21_s21": ((3, 3), 2, (2, 1), (2, 1)),
    "k11_d3": ((1, 1), 3, 0, 1),
    "k33_d23_p32": ((3, 3), (2, 3), (3, 2), 1),
}
DTS = ("f32", "f16", "bf16", "f64", "bool", "i32", "i64")


def pair(v):
    return (v, v) if isinstance(v, int) else tuple(v)


def args(name):
    ks, dil, pad, st = CASES[name]
    return pair(ks), pair(dil), pair(pad), pair(st)


def brute(x, ks, dil, pad, st, mistake=None):
    """Every output element from its definition, one (r, s, p, q) at a time;
    `mistake` plants one error."""
    N, C, H, W = x.shape
    (kh, kw), (dh, dw), (ph, pw), (sh, sw) = ks, dil, pad, st
    oh = (H + 2 * ph - dh * (kh - 1) - 1) // sh + 1
    ow = (W + 2 * pw - dw * (kw - 1) - 1) // sw + 1
    out = np.zeros((N, C * kh * kw, oh * ow), dtype=x.dtype)
    for r in range(kh):
        for s in range(kw):
            for p in range(oh):
                for q in range(ow):
                    ih, iw = p * sh - ph + r * dh, q * sw - pw + s * dw
                    if mistake == "no_dilation_w":
                        iw = q * sw - pw + s
                    elif mistake == "one_sided_pad":
                        ih = p * sh + r * dh
                    elif mistake == "swapped_strides":
                        ih, iw = p * sw - ph + r * dh, q * sh - pw + s * dw
                    rows = np.arange(C) * kh * kw + (s * kh + r if mistake == "tap_order" else r * kw + s)
                    if 0 <= ih < H and 0 <= iw < W:
                        out[:, rows, p * ow + q] = x[:, :, ih, iw]
    return out


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("name", sorted(CASES))
def test_golden(name, dt):
    x, y = GOLD[f"{name}_x_{dt}"], GOLD[f"{name}_y_{dt}"]
    got = O.im2col(x, *args(name))
    assert got.dtype == y.dtype and got.shape == y.shape
    assert np.array_equal(got, y)


@pytest.mark.parametrize("name", sorted(CASES))
def test_brute_force(name):
    x = GOLD[f"{name}_x_f32"]
    assert np.array_equal(O.im2col(x, *args(name)), brute(x, *args(name)))


def test_closed_forms():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 3, 7, 9)).astype(np.float32)
    # a 1x1 window, stride 1, no padding: a reshape
    assert np.array_equal(O.im2col(x, (1, 1)), x.reshape(2, 3, 63))
    # a strided 1x1 window: subsampling
    assert np.array_equal(O.im2col(x, (1, 1), stride=(2, 3)), x[:, :, ::2, ::3].reshape(2, 3, -1))
    # padding only ever contributes zeros, and every in-image element appears
    ones = np.ones((1, 1, 4, 5), np.float32)
    y = O.im2col(ones, (3, 3), padding=(1, 1))
    assert set(np.unique(y)) == {0.0, 1.0}
    # output column (p, q) of tap (r, s) counts taps inside the image
    assert y.sum() == sum(1 for r in range(3) for s in range(3) for p in range(4) for q in range(5)
                          if 0 <= p - 1 + r < 4 and 0 <= q - 1 + s < 5)
    # window at the centre tap of a 3x3, padding 1, stride 1 is the input itself
    assert np.array_equal(O.im2col(x, (3, 3), padding=(1, 1))[:, 4::9].reshape(x.shape), x)


@pytest.mark.parametrize("mistake", ("tap_order", "no_dilation_w", "one_sided_pad", "swapped_strides"))
def test_planted_mistakes_are_caught(mistake):
    caught = False
    for name in CASES:
        x, y = GOLD[f"{name}_x_f32"], GOLD[f"{name}_y_f32"]
        m = brute(x, *args(name), mistake=mistake)
        if m.shape != y.shape or not np.array_equal(m, y):
            caught = True
    assert caught, f"planted mistake {mistake} passed every golden vector"
