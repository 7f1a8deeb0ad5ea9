"""Shared test helpers: torch <-> oracle array conversion, tolerances."""

import math
import random

import numpy as np
import pytest
import torch

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
