"""Writes tests/golden/golden_elementwise.npz: torch CPU outputs of the rest
of the elementwise family (relu, sigmoid, tanh, neg, abs, rsqrt, sin, cos,
sub, div in its three modes, pow, the six comparisons, isinf, isnan, clamp)
on small seeded inputs with the special values (+-0, +-inf, NaN, tiny,
large).  bf16 tensors are stored as uint16 bit patterns.  Regenerate with:

    python tests/golden/make_golden_elementwise.py
"""

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
FLOATS = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
INTS = {"i8": torch.int8, "i16": torch.int16, "i32": torch.int32, "i64": torch.int64}
POW_SCALARS = (2, 3, 0.5, -0.5, -1, -2, 1.7)
CMPS = ("eq", "ne", "gt", "ge", "lt", "le")


def to_np(t):
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    return t.contiguous().numpy().copy()


def main():
    g = torch.Generator().manual_seed(4321)
    out = {}
    specials = [0.0, -0.0, float("inf"), float("-inf"), float("nan"), 1e-30, -88.0, 88.0, 1.0, -1.0]
    for name, dt in FLOATS.items():
        x = torch.randn(1000, generator=g) * 3
        x[: len(specials)] = torch.tensor(specials)
        x = x.to(dt)
        y = (torch.randn(1000, generator=g) * 3).to(dt)
        y[:4] = torch.tensor([0.0, -0.0, float("inf"), float("-inf")]).to(dt)
        y[20:30] = x[20:30]  # equal pairs for the comparisons
        out[f"x_{name}"], out[f"y_{name}"] = to_np(x), to_np(y)
        for op in ("relu", "sigmoid", "tanh", "neg", "abs", "rsqrt", "sin", "cos", "isinf", "isnan"):
            out[f"{op}_{name}"] = to_np(getattr(torch, op)(x))
        out[f"sub_{name}"] = to_np(torch.sub(x, y, alpha=0.7))
        out[f"sub_scalar_{name}"] = to_np(torch.sub(x, 1.1, alpha=1.3))
        for mode in (None, "trunc", "floor"):
            tag = mode or "true"
            out[f"div_{tag}_{name}"] = to_np(torch.div(x, y, rounding_mode=mode))
            out[f"div_{tag}_scalar_{name}"] = to_np(torch.div(x, 1.1, rounding_mode=mode))
        out[f"pow_{name}"] = to_np(torch.pow(x, y))
        for i, e in enumerate(POW_SCALARS):
            out[f"pow_scalar{i}_{name}"] = to_np(torch.pow(x, e))
        for op in CMPS:
            out[f"{op}_{name}"] = to_np(getattr(torch, op)(x, y))
            out[f"{op}_scalar_{name}"] = to_np(getattr(torch, op)(x, 1.001))
        lo = (torch.randn(1000, generator=g) - 1).to(dt)
        hi = (torch.randn(1000, generator=g) + 1).to(dt)
        lo[5], hi[6] = float("nan"), float("nan")
        out[f"lo_{name}"], out[f"hi_{name}"] = to_np(lo), to_np(hi)
        out[f"clamp_{name}"] = to_np(torch.clamp(x, lo, hi))
        out[f"clamp_min_{name}"] = to_np(torch.clamp(x, min=lo))
        out[f"clamp_scalar_{name}"] = to_np(torch.clamp(x, -0.11, 0.5003))
        out[f"clamp_max_scalar_{name}"] = to_np(torch.clamp(x, max=0.3))

    for name, dt in INTS.items():
        a = torch.randint(-100, 100, (500,), generator=g, dtype=dt)
        b = torch.randint(-9, 10, (500,), generator=g, dtype=dt)
        b[b == 0] = 3  # torch's CPU kernel raises on an integer division by zero
        e = torch.randint(-3, 6, (500,), generator=g, dtype=dt)
        out[f"ia_{name}"], out[f"ib_{name}"], out[f"ie_{name}"] = a.numpy().copy(), b.numpy().copy(), e.numpy().copy()
        for op in ("relu", "neg", "abs"):
            out[f"i{op}_{name}"] = getattr(torch, op)(a).numpy().copy()
        out[f"isub_{name}"] = torch.sub(a, b, alpha=3).numpy().copy()
        out[f"idiv_trunc_{name}"] = torch.div(a, b, rounding_mode="trunc").numpy().copy()
        out[f"idiv_floor_{name}"] = torch.div(a, b, rounding_mode="floor").numpy().copy()
        out[f"ipow_{name}"] = torch.pow(b, e).numpy().copy()
        for op in CMPS:
            out[f"i{op}_{name}"] = getattr(torch, op)(a, b).numpy().copy()
        out[f"iclamp_{name}"] = torch.clamp(a, b * 5, b * 5 + 40).numpy().copy()
        out[f"iclamp_scalar_{name}"] = torch.clamp(a, -7, 50).numpy().copy()

    np.savez_compressed(os.path.join(HERE, "golden_elementwise.npz"), **out)
    print(f"wrote {len(out)} arrays")


if __name__ == "__main__":
    main()
