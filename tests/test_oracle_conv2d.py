"""Pins the conv2d oracle -- CPU only.  Golden vectors written by torch CPU
(tests/golden/golden_conv2d.npz), closed forms that a plausible mistake
breaks (a 1x1 identity kernel returns the input; an off-centre delta tap
shifts it one way -- a flipped, convolution-style kernel shifts it the
other; a dilated tap lands dilation * index away; a strided output is the
unit-stride output subsampled; linearity in the weight and the bias), a
brute-force loop on a tiny case, and planted mistakes that the checks must
catch."""

import os

import numpy as np
import pytest
import torch

from oracle import ops as O
from tests.helpers import from_np

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_conv2d.npz"))
# name: (stride, padding as top/left pair, dilation, output size or None)
CASES = {
    "k1": ((1, 1), (0, 0), (1, 1), None),
    "k3": ((1, 1), (1, 1), (1, 1), None),
    "k3_s2_p23_d2": ((2, 2), (2, 3), (2, 2), None),
    "k3_s23_p0_d23": ((2, 3), (0, 0), (2, 3), None),
    "k24_same": ((1, 1), (0, 1), (1, 1), (9, 10)),
    "k3_c16": ((1, 1), (1, 1), (1, 1), None),
}
# torch's CPU convolution accumulates 16-bit inputs in fp32 and rounds once;
# the oracle accumulates in float64 and rounds once
TOL = {"f32": (1e-5, 1e-5), "f16": (2e-3, 2e-3), "bf16": (1.6e-2, 1.6e-2)}


@pytest.mark.parametrize("dt", ("f32", "f16", "bf16"))
@pytest.mark.parametrize("name", list(CASES))
def test_golden(name, dt):
    stride, pad, dil, out_hw = CASES[name]
    b = G.get(f"{name}_b_{dt}")
    got = O.conv2d(G[f"{name}_x_{dt}"], G[f"{name}_w_{dt}"], dt, b, stride, pad, dil, out_hw)
    exp = G[f"{name}_y_{dt}"]
    assert got.shape == exp.shape
    rtol, atol = TOL[dt]
    torch.testing.assert_close(from_np(got, dt).double(), from_np(exp, dt).double(), rtol=rtol, atol=atol)


def brute(x, w, b, stride, pad, dil):
    N, C, H, W = x.shape
    K, _, R, S = w.shape
    P = (H + 2 * pad[0] - dil[0] * (R - 1) - 1) // stride[0] + 1
    Q = (W + 2 * pad[1] - dil[1] * (S - 1) - 1) // stride[1] + 1
    out = np.zeros((N, K, P, Q))
    for n in range(N):
        for k in range(K):
            for p in range(P):
                for q in range(Q):
                    acc = b[k] if b is not None else 0.0
                    for c in range(C):
                        for r in range(R):
                            for s in range(S):
                                ih = p * stride[0] - pad[0] + r * dil[0]
                                iw = q * stride[1] - pad[1] + s * dil[1]
                                if 0 <= ih < H and 0 <= iw < W:
                                    acc += x[n, c, ih, iw] * w[k, c, r, s]
                    out[n, k, p, q] = acc
    return out


def pin_conv(f):
    """True when f (the oracle's signature) passes every closed form."""
    rng = np.random.default_rng(5)
    try:
        ok = True
        x = rng.standard_normal((2, 3, 9, 11))
        # 1x1 identity kernel
        eye = np.eye(3).reshape(3, 3, 1, 1)
        ok &= np.allclose(f(x, eye, "f64"), x, atol=1e-12)
        # off-centre delta tap (r = 0, s = 2) with padding 1: out[p, q] = x[p - 1, q + 1]
        d = np.zeros((3, 3, 3, 3))
        for c in range(3):
            d[c, c, 0, 2] = 1.0
        shifted = np.zeros_like(x)
        shifted[:, :, 1:, :-1] = x[:, :, :-1, 1:]
        ok &= np.allclose(f(x, d, "f64", None, (1, 1), (1, 1), (1, 1)), shifted, atol=1e-12)
        # dilated tap (r = 2, s = 1), dilation (2, 3), no padding: out[p, q] = x[p + 4, q + 3]
        t = np.zeros((3, 3, 3, 3))
        for c in range(3):
            t[c, c, 2, 1] = 1.0
        got = f(x, t, "f64", None, (1, 1), (0, 0), (2, 3))
        ok &= got.shape == (2, 3, 5, 5) and np.allclose(got, x[:, :, 4:9, 3:8], atol=1e-12)
        # stride: the unit-stride output subsampled (taps and padding unchanged)
        w = rng.standard_normal((4, 3, 3, 2))
        full = f(x, w, "f64", None, (1, 1), (1, 2), (1, 1))
        ok &= np.allclose(f(x, w, "f64", None, (2, 3), (1, 2), (1, 1)), full[:, :, ::2, ::3], atol=1e-12)
        # linearity in the weight, bias added once per output channel
        w2 = rng.standard_normal((4, 3, 3, 2))
        b = rng.standard_normal(4)
        lin = f(x, 2 * w - w2, "f64", b, (1, 1), (1, 2), (1, 1))
        ok &= np.allclose(lin, 2 * full - f(x, w2, "f64", None, (1, 1), (1, 2), (1, 1)) + b[None, :, None, None],
                          atol=1e-10)
        # brute force on a tiny case with everything non-trivial
        xs = rng.standard_normal((1, 2, 7, 8))
        ws = rng.standard_normal((3, 2, 2, 3))
        bs = rng.standard_normal(3)
        ok &= np.allclose(f(xs, ws, "f64", bs, (2, 1), (1, 2), (2, 1)), brute(xs, ws, bs, (2, 1), (1, 2), (2, 1)),
                          atol=1e-12)
        return bool(ok)
    except (ValueError, IndexError):
        return False


def test_closed_forms():
    assert pin_conv(O.conv2d)


MUTANTS = {
    "flipped kernel (convolution, not correlation)":
        lambda x, w, dt, b=None, st=(1, 1), p=(0, 0), d=(1, 1), hw=None: O.conv2d(x, w[:, :, ::-1, ::-1], dt, b, st, p, d, hw),
    "dilation ignored": lambda x, w, dt, b=None, st=(1, 1), p=(0, 0), d=(1, 1), hw=None: O.conv2d(x, w, dt, b, st, p, (1, 1), hw),
    "bias dropped": lambda x, w, dt, b=None, st=(1, 1), p=(0, 0), d=(1, 1), hw=None: O.conv2d(x, w, dt, None, st, p, d, hw),
    "strides swapped": lambda x, w, dt, b=None, st=(1, 1), p=(0, 0), d=(1, 1), hw=None: O.conv2d(x, w, dt, b, st[::-1], p, d, hw),
    "padding off by one": lambda x, w, dt, b=None, st=(1, 1), p=(0, 0), d=(1, 1), hw=None: O.conv2d(
        x, w, dt, b, st, (p[0] + 1, p[1]), d,
        hw or ((x.shape[2] + 2 * p[0] - d[0] * (w.shape[2] - 1) - 1) // st[0] + 1,
               (x.shape[3] + 2 * p[1] - d[1] * (w.shape[3] - 1) - 1) // st[1] + 1)),
}


@pytest.mark.parametrize("name", list(MUTANTS))
def test_planted_mistakes_are_caught(name):
    assert not pin_conv(MUTANTS[name]), f"the checks missed: {name}"
