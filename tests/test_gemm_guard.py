"""CPU checks of the GEMM parity guard used by the GPU tests
(tests/helpers.assert_gemm_ulp): it accepts any fp32 summation order of the
exact products and rejects the mistakes a pipelined K loop can make (a
dropped or repeated 32-wide K slice, a wrong column)."""

import numpy as np
import pytest
import torch

from oracle import ops as O
from tests.helpers import assert_gemm_ulp, from_np, tile_rows, to_np, ulp16


def _operands(m, n, k, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    a = (0.02 * torch.randn(m, k, generator=g)).to(dtype)
    b = (0.02 * torch.randn(k, n, generator=g)).to(dtype)
    return a, b


def _fp32_chunked(a, b, chunk=16):
    """fp32 accumulation over 16-k chunks in sequence: a summation order
    other than the oracle's."""
    af, bf = a.float().numpy(), b.float().numpy()
    acc = np.zeros((a.shape[0], b.shape[1]), np.float32)
    for k0 in range(0, a.shape[1], chunk):
        part = (af[:, k0:k0 + chunk].astype(np.float64) @ bf[k0:k0 + chunk].astype(np.float64)).astype(np.float32)
        acc = (acc + part).astype(np.float32)
    return acc


@pytest.mark.parametrize("dtype, dt", ((torch.bfloat16, "bf16"), (torch.float16, "f16")))
def test_guard_accepts_other_summation_orders(dtype, dt):
    a, b = _operands(64, 384, 4096, dtype)
    got = torch.from_numpy(_fp32_chunked(a, b)).to(dtype)
    assert_gemm_ulp(got, a, b, dt, what="chunked fp32")
    exact = from_np(O.gemm(to_np(a), to_np(b), dt), dt)
    assert_gemm_ulp(exact, a, b, dt, what="oracle itself", max_inexact=0.0)


@pytest.mark.parametrize("dtype, dt", ((torch.bfloat16, "bf16"), (torch.float16, "f16")))
def test_guard_rejects_dropped_and_repeated_k_slices(dtype, dt):
    a, b = _operands(64, 384, 4096, dtype)
    for lo in (0, 2048, 4064):
        keep = torch.cat([torch.arange(0, lo), torch.arange(lo + 32, 4096)])
        dropped = from_np(O.gemm(to_np(a[:, keep]), to_np(b[keep]), dt), dt)
        with pytest.raises(AssertionError):
            assert_gemm_ulp(dropped, a, b, dt, what="dropped slice")
        rep = torch.cat([torch.arange(0, 4096), torch.arange(lo, lo + 32)])
        repeated = from_np(O.gemm(to_np(a[:, rep]), to_np(b[rep]), dt), dt)
        with pytest.raises(AssertionError):
            assert_gemm_ulp(repeated, a, b, dt, what="repeated slice")


def test_guard_rejects_a_wrong_column_and_a_wrong_bias():
    a, b = _operands(32, 256, 512, torch.bfloat16)
    good = from_np(O.gemm(to_np(a), to_np(b), "bf16"), "bf16")
    swapped = good.clone()
    swapped[:, [7, 8]] = swapped[:, [8, 7]]
    with pytest.raises(AssertionError):
        assert_gemm_ulp(swapped, a, b, "bf16", what="swapped columns")
    bias = torch.randn(256).bfloat16()
    with_bias = from_np(O.gemm(to_np(a), to_np(b), "bf16", to_np(bias), 1.0, 1.0), "bf16")
    assert_gemm_ulp(with_bias, a, b, "bf16", c=bias, beta=1.0, what="bias")
    with pytest.raises(AssertionError):
        assert_gemm_ulp(with_bias, a, b, "bf16", c=bias, beta=0.5, what="wrong beta")


def test_guard_rows_and_ulp_grid():
    a, b = _operands(300, 64, 96, torch.float16)
    good = from_np(O.gemm(to_np(a), to_np(b), "f16"), "f16")
    rows = tile_rows(300)
    assert rows[0] == 0 and rows[-1] == 299 and all(0 <= r < 300 for r in rows)
    assert_gemm_ulp(good, a, b, "f16", rows=rows, what="rows")
    # ulp16 against numpy's float16 spacing and bf16's 8-bit significand
    xs = np.array([1.0, 3.0, 1e-3, 6e-6, 60000.0])
    assert np.array_equal(ulp16(xs, "f16"), np.spacing(xs.astype(np.float16)).astype(np.float64))
    assert ulp16(np.array([1.0]), "bf16")[0] == 2.0**-7 and ulp16(np.array([3.0]), "bf16")[0] == 2.0**-6


def test_gemm_f64_magnitude():
    """magnitude = |alpha| sum |a b| + |beta c|: equal to the value for
    non-negative operands, unchanged when an operand's sign flips."""
    g = torch.Generator().manual_seed(3)
    a = torch.rand(8, 40, generator=g).bfloat16()
    b = torch.rand(40, 16, generator=g).bfloat16()
    c = torch.rand(16, generator=g).bfloat16()
    x, m = O.gemm_f64(to_np(a), to_np(b), "bf16", to_np(c), 2.0, 0.5, magnitude=True)
    assert np.allclose(x, m, rtol=1e-15)
    x2, m2 = O.gemm_f64(to_np(-a), to_np(b), "bf16", to_np(-c), 2.0, 0.5, magnitude=True)
    assert np.allclose(x2, -x, rtol=1e-15) and np.array_equal(m2, m)
