"""addmm -- mirror of src/ntops/torch/addmm.py:7-18 (math: kernels/addmm.py:64-67).

`input` broadcasts to (m, n) as in torch (a 1-D bias is a stride-0 row);
beta == 0 ignores `input` entirely, as torch does."""

import torch

from ntops_amd.torch._gemm import gemm


def addmm(input, mat1, mat2, *, beta=1, alpha=1, out=None):
    if mat1.dim() != 2 or mat2.dim() != 2:
        raise RuntimeError("addmm: expected 2-D matrices")
    m, k = mat1.shape
    k2, n = mat2.shape
    if k != k2:
        raise RuntimeError(f"addmm: shapes {tuple(mat1.shape)} and {tuple(mat2.shape)} cannot be multiplied")

    if out is None:
        out = torch.empty((m, n), dtype=input.dtype, device=input.device)
    elif tuple(out.shape) != (m, n):
        out.resize_((m, n))

    c = input.expand(m, n) if beta != 0 else None
    return gemm(mat1, mat2, out, c=c, alpha=alpha, beta=beta, what="ntops_amd.addmm")
