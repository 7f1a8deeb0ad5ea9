"""Writes tests/golden/golden_fused.npz: torch CPU results of the two fused
variants' compositions on small seeded inputs --

  * residual + rms_norm: h = x + residual, y = torch.rms_norm(h, (cols,), w,
    eps) for fp32, fp16 and bf16, with and without a weight;
  * q / k rotary embedding: torch's eager rotation formula (half and
    interleaved pairs, (S, D/2) tables) on q (2, 5, 4, 16) and k (2, 5, 2, 16).

bf16 tensors are stored as uint16 bit patterns.  Regenerate with:

    python tests/golden/make_golden_fused.py
"""

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
DTS = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def to_np(t):
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    return t.contiguous().numpy().copy()


def rope(x, sin, cos, interleaved):
    # torch eager, every product and sum in the tensor dtype
    if interleaved:
        x0, x1 = x[..., 0::2], x[..., 1::2]
    else:
        half = x.shape[-1] // 2
        x0, x1 = x[..., :half], x[..., half:]
    s = sin[None, :, None, :]
    c = cos[None, :, None, :]
    o0 = x0 * c - x1 * s
    o1 = x1 * c + x0 * s
    if interleaved:
        return torch.stack((o0, o1), dim=-1).flatten(-2)
    return torch.cat((o0, o1), dim=-1)


def main():
    g = torch.Generator().manual_seed(31)
    out = {}
    rows, cols = 7, 96
    for name, dt in DTS.items():
        x = torch.randn(rows, cols, generator=g).to(dt)
        r = torch.randn(rows, cols, generator=g).to(dt)
        w = (1 + 0.1 * torch.randn(cols, generator=g)).to(dt)
        h = x + r
        out[f"arn_x_{name}"], out[f"arn_r_{name}"], out[f"arn_w_{name}"] = to_np(x), to_np(r), to_np(w)
        out[f"arn_h_{name}"] = to_np(h)
        out[f"arn_y_{name}"] = to_np(torch.rms_norm(h, (cols,), w, 1e-6))
        out[f"arn_ynw_{name}"] = to_np(torch.rms_norm(h, (cols,), None, None))
        q = torch.randn(2, 5, 4, 16, generator=g).to(dt)
        k = torch.randn(2, 5, 2, 16, generator=g).to(dt)
        ang = torch.arange(5).float()[:, None] * (10000.0 ** (-torch.arange(8).float() / 8))[None, :]
        sin, cos = torch.sin(ang).to(dt), torch.cos(ang).to(dt)
        out[f"qk_q_{name}"], out[f"qk_k_{name}"] = to_np(q), to_np(k)
        out[f"qk_sin_{name}"], out[f"qk_cos_{name}"] = to_np(sin), to_np(cos)
        for il in (0, 1):
            out[f"qk_qo{il}_{name}"] = to_np(rope(q, sin, cos, il))
            out[f"qk_ko{il}_{name}"] = to_np(rope(k, sin, cos, il))
    np.savez_compressed(os.path.join(HERE, "golden_fused.npz"), **out)
    print(f"wrote {len(out)} arrays")


if __name__ == "__main__":
    main()
