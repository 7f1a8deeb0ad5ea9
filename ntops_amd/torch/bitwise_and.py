"""bitwise_and -- mirror of src/ntops/torch/bitwise_and.py:7-15
(math: kernels/bitwise_and.py:9)."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _binary


def bitwise_and(input, other, *, out=None):
    dt = torch.result_type(input, other)
    if dt.is_floating_point or dt.is_complex:
        raise RuntimeError(f'"bitwise_and" not implemented for {dt}')
    return _binary(_lib.BINARY_BITWISE_AND, input, other, None, out, "ntops_amd.bitwise_and")
