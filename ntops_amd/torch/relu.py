"""relu -- mirror of src/ntops/torch/relu.py:7-19 (math: kernels/relu.py:9).

max(0, x) with torch's NaN rule (NaN stays NaN); integer inputs allowed,
bool rejected as torch does."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _unary


def relu(input, inplace=False):
    if input.dtype == torch.bool:
        raise RuntimeError("Boolean inputs not supported for relu")
    _lib.require_cuda(input)
    output = input if inplace else torch.empty_like(input)
    return _unary(_lib.UNARY_RELU, input, output, "ntops_amd.relu")
