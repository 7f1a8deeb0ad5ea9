"""bitwise_or -- mirror of src/ntops/torch/bitwise_or.py:7-15
(math: kernels/bitwise_or.py:9)."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _binary


def bitwise_or(input, other, *, out=None):
    dt = torch.result_type(input, other)
    if dt.is_floating_point or dt.is_complex:
        raise RuntimeError(f'"bitwise_or" not implemented for {dt}')
    return _binary(_lib.BINARY_BITWISE_OR, input, other, None, out, "ntops_amd.bitwise_or")
