"""silu -- mirror of src/ntops/torch/silu.py:7-17 (math: kernels/silu.py:10)."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _unary


def silu(input, inplace=False):
    if not input.dtype.is_floating_point:
        raise RuntimeError(f'"silu" not implemented for {input.dtype}')

    if inplace:
        output = input
    else:
        output = torch.empty_like(input)

    return _unary(_lib.UNARY_SILU, input, output, "ntops_amd.silu")
