"""mm -- mirror of src/ntops/torch/mm.py:7-18 (math: kernels/mm.py:54-65)."""

import torch

from ntops_amd.torch._gemm import gemm


def mm(input, mat2, *, out=None):
    if input.dim() != 2 or mat2.dim() != 2:
        raise RuntimeError("mm: expected 2-D tensors")
    m, k = input.shape
    k2, n = mat2.shape
    if k != k2:
        raise RuntimeError(f"mm: shapes {tuple(input.shape)} and {tuple(mat2.shape)} cannot be multiplied")

    if out is None:
        out = torch.empty((m, n), dtype=input.dtype, device=input.device)
    elif tuple(out.shape) != (m, n):
        out.resize_((m, n))

    return gemm(input, mat2, out, what="ntops_amd.mm")
