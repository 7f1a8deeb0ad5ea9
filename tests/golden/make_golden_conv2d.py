"""Writes tests/golden/golden_conv2d.npz: torch CPU F.conv2d outputs on small
seeded inputs -- 1x1 and 3x3 (and a 2x4) kernels, strides 1 / 2 / (2, 3),
paddings 0 / 1 / (2, 3) / 'same', dilations 1 / 2 / (2, 3), with and without
bias, fp32, fp16 and bf16.  bf16 tensors are stored as uint16 bit patterns.
Regenerate with:

    python tests/golden/make_golden_conv2d.py
"""

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
DTS = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
# name: (n, c, h, w, k, r, s, stride, padding, dilation, bias)
CASES = {
    "k1": (2, 3, 11, 13, 4, 1, 1, 1, 0, 1, True),
    "k3": (2, 3, 11, 13, 4, 3, 3, 1, 1, 1, True),
    "k3_s2_p23_d2": (2, 3, 14, 15, 4, 3, 3, 2, (2, 3), 2, True),
    "k3_s23_p0_d23": (1, 5, 16, 17, 3, 3, 3, (2, 3), 0, (2, 3), False),
    "k24_same": (1, 4, 9, 10, 5, 2, 4, 1, "same", 1, True),
    "k3_c16": (2, 16, 10, 9, 8, 3, 3, 1, 1, 1, True),
}


def to_np(t):
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    return t.contiguous().numpy().copy()


def main():
    g = torch.Generator().manual_seed(2024)
    out = {}
    for name, (n, c, h, w, k, r, s, stride, padding, dilation, has_bias) in CASES.items():
        x = torch.randn(n, c, h, w, generator=g)
        wt = torch.randn(k, c, r, s, generator=g)
        b = torch.randn(k, generator=g) if has_bias else None
        for dn, dt in DTS.items():
            xd, wd = x.to(dt), wt.to(dt)
            bd = b.to(dt) if b is not None else None
            out[f"{name}_x_{dn}"], out[f"{name}_w_{dn}"] = to_np(xd), to_np(wd)
            if bd is not None:
                out[f"{name}_b_{dn}"] = to_np(bd)
            out[f"{name}_y_{dn}"] = to_np(F.conv2d(xd, wd, bd, stride=stride, padding=padding, dilation=dilation))
    np.savez_compressed(os.path.join(HERE, "golden_conv2d.npz"), **out)
    print(f"wrote {len(out)} arrays")


if __name__ == "__main__":
    main()
