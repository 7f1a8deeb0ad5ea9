"""Writes tests/golden/golden_im2col.npz: torch CPU F.unfold outputs on small
seeded inputs over the reference's im2col test grid (kernel sizes, strides,
paddings, dilations incl. asymmetric pairs) plus a dilated 1x1 case, for
fp32, fp16, bf16 (uint16 bit patterns), fp64 and bool; int32 / int64
vectors are F.unfold of the same small integers held exactly in float64.
Regenerate with:

    python tests/golden/make_golden_im2col.py
"""

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
# name: (shape, kernel_size, dilation, padding, stride)
CASES = {
    "k33": ((2, 3, 8, 8), (3, 3), 1, 0, 1),
    "k53_p1_s21": ((1, 4, 10, 12), (5, 3), 1, 1, (2, 1)),
    "k44_s44": ((2, 2, 16, 16), (4, 4), 1, 0, (4, 4)),
    "k32": ((3, 6, 7, 9), (3, 2), 1, 0, (1, 1)),
    "k23_p1_s12": ((1, 8, 9, 11), (2, 3), 1, 1, (1, 2)),
    "k33_d2_p21_s21": ((2, 5, 12, 6), (3, 3), 2, (2, 1), (2, 1)),
    "k11_d3": ((1, 3, 5, 7), (1, 1), 3, 0, 1),
    "k33_d23_p32": ((1, 2, 9, 10), (3, 3), (2, 3), (3, 2), 1),
}
FLOATS = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "f64": torch.float64}
INTS = {"i32": torch.int32, "i64": torch.int64}


def to_np(t):
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    return t.contiguous().numpy().copy()


def main():
    g = torch.Generator().manual_seed(77)
    out = {}
    for name, (shape, ks, dil, pad, st) in CASES.items():
        x = torch.randn(shape, generator=g)
        for dn, dt in FLOATS.items():
            xd = x.to(dt)
            out[f"{name}_x_{dn}"] = to_np(xd)
            out[f"{name}_y_{dn}"] = to_np(F.unfold(xd, ks, dilation=dil, padding=pad, stride=st))
        xb = torch.randint(0, 2, shape, generator=g).bool()
        out[f"{name}_x_bool"] = to_np(xb)
        out[f"{name}_y_bool"] = to_np(F.unfold(xb, ks, dilation=dil, padding=pad, stride=st))
        xi = torch.randint(-10, 10, shape, generator=g)
        y = F.unfold(xi.double(), ks, dilation=dil, padding=pad, stride=st)
        for dn, dt in INTS.items():
            out[f"{name}_x_{dn}"] = to_np(xi.to(dt))
            out[f"{name}_y_{dn}"] = to_np(y.to(dt))
    np.savez_compressed(os.path.join(HERE, "golden_im2col.npz"), **out)
    print(f"wrote {len(out)} arrays")


if __name__ == "__main__":
    main()
