"""sub -- mirror of src/ntops/torch/sub.py:7-15 (math: kernels/sub.py:10).

torch semantics: broadcasting, type promotion, Python-number operands, and
a - alpha * b evaluated as torch's add with -alpha (same roundings)."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _binary, _split_other


def sub(input, other, *, alpha=1, out=None):
    _, _, dtype = _split_other(input, other, "ntops_amd.sub")
    if dtype == torch.bool:
        raise RuntimeError(
            "Subtraction, the `-` operator, with two bool tensors is not supported. "
            "Use the `^` or `logical_xor()` operator instead."
        )
    return _binary(_lib.BINARY_SUB, input, other, alpha, out, "ntops_amd.sub")
