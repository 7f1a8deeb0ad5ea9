"""gelu -- mirror of src/ntops/torch/gelu.py:7-14 (math: kernels/gelu.py:10-39)."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _unary


def gelu(input, approximate="none"):
    if approximate not in ("none", "tanh"):
        raise RuntimeError(f"approximate argument must be either none or tanh, got {approximate}")
    if not input.dtype.is_floating_point:
        raise RuntimeError(f'"gelu" not implemented for {input.dtype}')

    output = torch.empty_like(input)

    op = _lib.UNARY_GELU_TANH if approximate == "tanh" else _lib.UNARY_GELU
    return _unary(op, input, output, "ntops_amd.gelu")
