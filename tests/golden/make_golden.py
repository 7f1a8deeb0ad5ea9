"""Writes the golden vectors in tests/golden/*.npz.

The configs name PyTorch's CPU implementation as the reference of every op
(and the ntops tests compare against the same torch ops), so the expected
outputs are produced by torch CPU on small seeded inputs.  bf16 tensors are
stored as uint16 bit patterns.  Regenerate with:

    python tests/golden/make_golden.py
"""

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))

DTS = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def to_np(t):
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()
    return t.contiguous().numpy().copy()


def rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def rotate_every_two(x):
    x0, x1 = x[..., 0::2], x[..., 1::2]
    return torch.stack((-x1, x0), dim=-1).reshape(x.shape)


def main():
    g = torch.Generator().manual_seed(1234)
    out = {}

    # elementwise, unary
    for name, dt in DTS.items():
        x = torch.randn(1000, generator=g) * 3
        x[:8] = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), float("nan"), 1e-30, -88.0, 88.0])
        x = x.to(dt)
        out[f"unary_{name}_x"] = to_np(x)
        out[f"silu_{name}"] = to_np(F.silu(x))
        out[f"gelu_{name}"] = to_np(F.gelu(x))
        out[f"gelu_tanh_{name}"] = to_np(F.gelu(x, approximate="tanh"))
        out[f"exp_{name}"] = to_np(torch.exp(x))
        y = (torch.randn(1000, generator=g) * 3).to(dt)
        out[f"binary_{name}_y"] = to_np(y)
        out[f"add_{name}"] = to_np(torch.add(x, y, alpha=-0.3))
        out[f"add_scalar_{name}"] = to_np(torch.add(x, 0.1, alpha=0.7))
        out[f"mul_{name}"] = to_np(x * y)
        out[f"mul_scalar_{name}"] = to_np(x * 0.1)

    # integer / bitwise
    for name, dt in (("i8", torch.int8), ("i16", torch.int16), ("i32", torch.int32), ("i64", torch.int64)):
        a = torch.randint(-100, 100, (500,), generator=g, dtype=dt)
        b = torch.randint(-100, 100, (500,), generator=g, dtype=dt)
        out[f"int_{name}_a"] = a.numpy().copy()
        out[f"int_{name}_b"] = b.numpy().copy()
        out[f"and_{name}"] = torch.bitwise_and(a, b).numpy().copy()
        out[f"or_{name}"] = torch.bitwise_or(a, b).numpy().copy()
        out[f"not_{name}"] = torch.bitwise_not(a).numpy().copy()
        out[f"iadd_{name}"] = torch.add(a, b, alpha=3).numpy().copy()
        out[f"imul_{name}"] = torch.mul(a, b).numpy().copy()
    ab = torch.rand(64, generator=g) > 0.5
    bb = torch.rand(64, generator=g) > 0.5
    out["bool_a"], out["bool_b"] = ab.numpy().copy(), bb.numpy().copy()
    out["and_bool"] = torch.bitwise_and(ab, bb).numpy().copy()
    out["or_bool"] = torch.bitwise_or(ab, bb).numpy().copy()
    out["not_bool"] = torch.bitwise_not(ab).numpy().copy()

    # row reductions
    for name, dt in DTS.items():
        x = torch.randn(16, 256, generator=g).to(dt)
        w = (1 + 0.02 * torch.randn(256, generator=g)).to(dt)
        b = (0.02 * torch.randn(256, generator=g)).to(dt)
        out[f"norm_{name}_x"], out[f"norm_{name}_w"], out[f"norm_{name}_b"] = to_np(x), to_np(w), to_np(b)
        out[f"rms_{name}"] = to_np(F.rms_norm(x, (256,), w, 1e-6))
        out[f"rms_noweight_epsnone_{name}"] = to_np(F.rms_norm(x, (256,), None, None))
        out[f"ln_{name}"] = to_np(F.layer_norm(x, (256,), w, b, 1e-5))
        out[f"ln_noaffine_{name}"] = to_np(F.layer_norm(x, (256,), None, None, 1e-5))
        s = (torch.randn(2, 3, 64, 64, generator=g) / np.sqrt(128)).masked_fill(
            torch.triu(torch.ones(64, 64, dtype=torch.bool), 1), float("-inf")
        )
        s = s.to(dt)
        out[f"softmax_{name}_x"] = to_np(s)
        out[f"softmax_{name}"] = to_np(F.softmax(s, -1))
        out[f"softmax_dim1_{name}"] = to_np(F.softmax(s, 1))
        out[f"softmax_f32out_{name}"] = to_np(F.softmax(s, -1, dtype=torch.float32))

    # RoPE: half-rotation with (S, D) tables (rotate_half form), interleaved
    # with (S, D) tables (rotate_every_two form), and ntops' (S, D/2) form.
    for name, dt in DTS.items():
        B, S, H, D = 2, 16, 3, 64
        q = torch.randn(B, S, H, D, generator=g).to(dt)
        i = torch.arange(D // 2, dtype=torch.float32)
        theta = 10000.0 ** (-2 * (i / D))
        ang = torch.arange(S, dtype=torch.float32)[:, None] * theta[None, :]
        sh, ch = torch.sin(ang), torch.cos(ang)
        sf, cf = torch.cat([sh, sh], -1).to(dt), torch.cat([ch, ch], -1).to(dt)
        si, ci = sh.repeat_interleave(2, -1).to(dt), ch.repeat_interleave(2, -1).to(dt)
        out[f"rope_{name}_x"] = to_np(q)
        out[f"rope_{name}_sin_full"], out[f"rope_{name}_cos_full"] = to_np(sf), to_np(cf)
        out[f"rope_{name}_sin_inter"], out[f"rope_{name}_cos_inter"] = to_np(si), to_np(ci)
        out[f"rope_{name}_sin_half"], out[f"rope_{name}_cos_half"] = to_np(sh.to(dt)), to_np(ch.to(dt))
        out[f"rope_half_{name}"] = to_np(q * cf[None, :, None, :] + rotate_half(q) * sf[None, :, None, :])
        out[f"rope_inter_{name}"] = to_np(q * ci[None, :, None, :] + rotate_every_two(q) * si[None, :, None, :])
        # ntops' own test formula with (S, D/2) tables, non-interleaved
        c2, s2 = ch.to(dt)[None, :, None, :], sh.to(dt)[None, :, None, :]
        x0, x1 = q[..., : D // 2], q[..., D // 2 :]
        out[f"rope_ntops_half_{name}"] = to_np(torch.cat((x0 * c2 - x1 * s2, x0 * s2 + x1 * c2), -1))
        p = q.view(B, S, H, D // 2, 2)
        y0, y1 = p[..., 0], p[..., 1]
        out[f"rope_ntops_inter_{name}"] = to_np(torch.stack((y0 * c2 - y1 * s2, y0 * s2 + y1 * c2), -1).view(q.shape))

    # GEMM family
    for name, dt in DTS.items():
        a = (0.02 * torch.randn(48, 96, generator=g)).to(dt)
        b = (0.02 * torch.randn(96, 40, generator=g)).to(dt)
        bias = (0.02 * torch.randn(40, generator=g)).to(dt)
        c = (0.02 * torch.randn(48, 40, generator=g)).to(dt)
        ba = (0.02 * torch.randn(3, 32, 64, generator=g)).to(dt)
        bb = (0.02 * torch.randn(3, 64, 24, generator=g)).to(dt)
        out[f"mm_{name}_a"], out[f"mm_{name}_b"] = to_np(a), to_np(b)
        out[f"mm_{name}_bias"], out[f"mm_{name}_c"] = to_np(bias), to_np(c)
        out[f"bmm_{name}_a"], out[f"bmm_{name}_b"] = to_np(ba), to_np(bb)
        out[f"mm_{name}"] = to_np(torch.mm(a, b))
        out[f"addmm_bias_{name}"] = to_np(torch.addmm(bias, a, b))
        out[f"addmm_full_{name}"] = to_np(torch.addmm(c, a, b, beta=0.5, alpha=-1.5))
        out[f"bmm_{name}"] = to_np(torch.bmm(ba, bb))

    np.savez_compressed(os.path.join(HERE, "golden.npz"), **out)
    print(f"wrote {len(out)} arrays")


if __name__ == "__main__":
    main()
