"""bmm -- mirror of src/ntops/torch/bmm.py:7-18 (math: kernels/bmm.py:8-43)."""

import torch

from ntops_amd.torch._gemm import gemm


def bmm(input, mat2, *, out=None):
    if input.dim() != 3 or mat2.dim() != 3:
        raise RuntimeError("bmm: expected 3-D tensors")
    b, m, k = input.shape
    b2, k2, n = mat2.shape
    if b != b2 or k != k2:
        raise RuntimeError(f"bmm: shapes {tuple(input.shape)} and {tuple(mat2.shape)} cannot be multiplied")

    if out is None:
        out = torch.empty((b, m, n), dtype=input.dtype, device=input.device)
    elif tuple(out.shape) != (b, m, n):
        out.resize_((b, m, n))

    return gemm(input, mat2, out, what="ntops_amd.bmm")
