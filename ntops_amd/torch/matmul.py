"""matmul -- mirror of src/ntops/torch/matmul.py:4-18.

2-D x 2-D goes to mm; otherwise operands are lifted to 3-D and sent to the
batched GEMM, a batch of 1 broadcasting against the other operand (stride 0)
as torch.matmul does."""

import torch

import ntops_amd
from ntops_amd.torch._gemm import gemm


def matmul(input, other, *, out=None):
    assert input.ndim in (2, 3) and other.ndim in (2, 3), (
        "Currently, only 2D and 3D tensors are supported."
    )

    if input.ndim == 2 and other.ndim == 2:
        return ntops_amd.torch.mm(input, other, out=out)

    if input.ndim < 3:
        input = input.unsqueeze(0)

    if other.ndim < 3:
        other = other.unsqueeze(0)

    b = max(input.shape[0], other.shape[0])
    if input.shape[0] not in (1, b) or other.shape[0] not in (1, b):
        raise RuntimeError("matmul: batch dimensions cannot be broadcast")
    if input.shape[2] != other.shape[1]:
        raise RuntimeError("matmul: inner dimensions do not match")
    input = input.expand(b, -1, -1)
    other = other.expand(b, -1, -1)
    m, n = input.shape[1], other.shape[2]
    if out is None:
        out = torch.empty((b, m, n), dtype=input.dtype, device=input.device)
    elif tuple(out.shape) != (b, m, n):
        out.resize_((b, m, n))
    return gemm(input, other, out, what="ntops_amd.matmul")
