"""abs -- mirror of src/ntops/torch/abs.py:7-15 (math: kernels/abs.py).

Integers wrap like torch (the minimum value maps to itself); bool inputs are
rejected as torch does."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _cast_into, _prepare_out, _unary


def abs(input, *, out=None):
    if input.dtype == torch.bool:
        raise NotImplementedError('"abs" not implemented for Bool')
    dev = _lib.require_cuda(input)
    target, res = _prepare_out(out, input.shape, input.dtype, dev, like=input)
    _unary(_lib.UNARY_ABS, input, res, "ntops_amd.abs")
    if res is not target:
        _cast_into(res, target)
    return target
