"""Writes tests/golden/golden_attention.npz: torch CPU
F.scaled_dot_product_attention outputs on small seeded inputs -- GQA
(4 query heads over 2 key / value heads), Sq != Skv, no mask / bool mask /
additive float mask / causal upper-left / causal lower-right, fp32, fp16 and
bf16.  bf16 tensors are stored as uint16 bit patterns.  Regenerate with:

    python tests/golden/make_golden_attention.py
"""

import os

import numpy as np
import torch
import torch.nn.functional as F
from torch.nn.attention.bias import causal_lower_right

HERE = os.path.dirname(os.path.abspath(__file__))
DTS = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def to_np(t):
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    return t.contiguous().numpy().copy()


def main():
    g = torch.Generator().manual_seed(777)
    out = {}
    B, Hq, Hkv, Sq, Skv, D = 2, 4, 2, 33, 47, 64
    bool_mask = torch.rand(Sq, Skv, generator=g) > 0.4
    bool_mask[5] = False  # one fully masked row
    float_mask = torch.randn(Sq, Skv, generator=g)
    out["bool_mask"] = bool_mask.numpy().copy()
    for name, dt in DTS.items():
        q = torch.randn(B, Hq, Sq, D, generator=g).to(dt)
        k = torch.randn(B, Hkv, Skv, D, generator=g).to(dt)
        v = torch.randn(B, Hkv, Skv, D, generator=g).to(dt)
        fm = float_mask.to(dt)
        out[f"q_{name}"], out[f"k_{name}"], out[f"v_{name}"] = to_np(q), to_np(k), to_np(v)
        out[f"float_mask_{name}"] = to_np(fm)
        sd = F.scaled_dot_product_attention
        out[f"plain_{name}"] = to_np(sd(q, k, v, enable_gqa=True))
        out[f"scaled_{name}"] = to_np(sd(q, k, v, enable_gqa=True, scale=0.3))
        out[f"bool_{name}"] = to_np(sd(q, k, v, attn_mask=bool_mask, enable_gqa=True))
        out[f"float_{name}"] = to_np(sd(q, k, v, attn_mask=fm, enable_gqa=True))
        out[f"causal_ul_{name}"] = to_np(sd(q, k, v, is_causal=True, enable_gqa=True))
        out[f"causal_lr_{name}"] = to_np(sd(q, k, v, attn_mask=causal_lower_right(Sq, Skv), enable_gqa=True))
    np.savez_compressed(os.path.join(HERE, "golden_attention.npz"), **out)
    print(f"wrote {len(out)} arrays")


if __name__ == "__main__":
    main()
