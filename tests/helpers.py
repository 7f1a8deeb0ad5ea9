"""Shared test helpers: torch <-> oracle array conversion, tolerances."""

import math
import random

import numpy as np
import pytest
import torch

from oracle import ops as O

DT_NAME = {
    torch.float32: "f32",
    torch.float16: "f16",
    torch.bfloat16: "bf16",
    torch.float64: "f64",
    torch.bool: "bool",
    torch.uint8: "u8",
    torch.int8: "i8",
    torch.int16: "i16",
    torch.int32: "i32",
    torch.int64: "i64",
}
TORCH_DT = {v: k for k, v in DT_NAME.items()}

# Tolerances bound by the build's target (rtol, atol).
TOL_ELEMENTWISE = {"f32": (1e-6, 1e-6), "f64": (1e-12, 1e-12), "f16": (1.6e-2, 1.6e-2), "bf16": (1.6e-2, 1.6e-2)}
TOL_REDUCTION = {"f32": (1e-5, 1e-5), "f64": (1e-12, 1e-12), "f16": (1.6e-2, 1.6e-2), "bf16": (1.6e-2, 1.6e-2)}
TOL_GEMM = {"f32": (1e-5, 1e-5), "f16": (1.6e-2, 1.6e-2), "bf16": (1.6e-2, 1.6e-2)}

requires_gpu = pytest.mark.gpu


def to_np(t):
    """torch tensor (any device) -> oracle array (bf16 as uint16 bits)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def from_np(a, dt):
    """oracle array -> CPU torch tensor of dtype name dt."""
    a = np.ascontiguousarray(a)
    if dt == "bf16":
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(a.copy())


def assert_close(actual, expected, rtol, atol, what=""):
    a = actual.detach().cpu().double()
    e = expected.detach().cpu().double()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    torch.testing.assert_close(a, e, rtol=rtol, atol=atol, equal_nan=True, msg=lambda m: f"{what}: {m}")


def assert_equal(actual, expected, what=""):
    a = actual.detach().cpu()
    e = expected.detach().cpu()
    assert a.dtype == e.dtype, f"{what}: dtype {a.dtype} != {e.dtype}"
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    assert torch.equal(a, e), f"{what}: {(a != e).sum().item()} elements differ"


def random_shape(ndim, min_num_elements=2**8, max_num_elements=2**10):
    """tests/utils.py:34-48 of the reference: random shape with 256..1024
    elements spread over ndim dims."""
    num_elements = random.randint(min_num_elements, max_num_elements)
    shape = []
    remaining = num_elements
    for _ in range(ndim - 1):
        size = random.randint(1, max(1, math.isqrt(remaining)))
        shape.append(size)
        remaining //= size
    shape.append(remaining)
    random.shuffle(shape)
    return shape


def randn(shape, dtype, device="cpu", scale=1.0, gen=None):
    """fp32 randn on the CPU (optionally from a generator), scaled, cast to dtype."""
    x = torch.randn(shape, generator=gen) * scale
    return x.to(dtype).to(device)


# mantissa bits and smallest normal of the 16-bit float formats
_FMT16 = {"bf16": (7, 2.0**-126), "f16": (10, 2.0**-14)}


def ulp16(x, dt):
    """Spacing of the dt grid (bf16 / f16) at magnitude |x| (float64 array);
    subnormal spacing below the smallest normal."""
    bits, tiny = _FMT16[dt]
    e = np.floor(np.log2(np.maximum(np.abs(x), tiny)))
    return np.exp2(e - bits)


def assert_gemm_ulp(got, a, b, dt, c=None, alpha=1.0, beta=0.0, what="", rows=None, max_inexact=0.01):
    """16-bit GEMM parity against the oracle, tight enough to see a dropped or
    repeated K slice.  For every checked element e of the exact (float64)
    result x and the kernel's value y:

        |y - x| <= ulp(max(|x|, |y|)) + (K + 2) * 2^-24 * m

    where m = |alpha| sum_k |a b| + |beta| |c| bounds the error of fp32
    summation in any order (the products of 16-bit operands are exact in
    fp32), and at most `max_inexact` of the elements may differ from the
    oracle's correctly rounded value.  a, b (and c) are CPU tensors in the
    operand layout of the oracle ((batch,) M x K, K x N); rows selects output
    rows (of every batch) to check, None checks all."""
    y = got.detach()
    an, bn = to_np(a), to_np(b)
    cn = None if c is None else to_np(c)
    if rows is not None:
        y = y[..., torch.as_tensor(rows, device=y.device), :]
        an = an[..., np.asarray(rows), :]
        if cn is not None and cn.ndim >= 2 and cn.shape[-2] > 1:
            cn = cn[..., np.asarray(rows), :]
    x, m = O.gemm_f64(an, bn, dt, cn, alpha, beta, magnitude=True)
    ref = from_np(O.round_to(x.astype(np.float32), dt), dt).double().numpy()
    yv = y.cpu().double().numpy()
    assert yv.shape == x.shape, f"{what}: shape {yv.shape} != {x.shape}"
    k = a.shape[-1]
    bound = ulp16(np.maximum(np.abs(x), np.abs(yv)), dt) + (k + 2) * 2.0**-24 * m
    err = np.abs(yv - x)
    bad = ~(err <= bound)
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err / np.maximum(bound, 1e-300), 0)), bad.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} elements beyond one ulp + the fp32 "
                             f"summation bound; worst at {i}: got {yv[i]!r}, exact {x[i]!r}, bound {bound[i]!r}")
    inexact = float(np.mean(yv != ref))
    assert inexact <= max_inexact, f"{what}: {inexact:.4%} of elements differ from the correctly rounded value"


def tile_rows(m, tile=256):
    """Two output rows in every `tile`-row band (at offsets that vary from band
    to band) plus the first and the last row."""
    rows = {0, m - 1}
    for t in range((m + tile - 1) // tile):
        rows.add(min(m - 1, t * tile + (37 * t + 5) % tile))
        rows.add(min(m - 1, t * tile + tile - 1 - (53 * t) % tile))
    return sorted(rows)
