"""neg -- mirror of src/ntops/torch/neg.py:7-15 (math: kernels/neg.py).

Integers wrap like torch (the minimum value maps to itself); bool inputs are
rejected as torch does."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _cast_into, _prepare_out, _unary


def neg(input, *, out=None):
    if input.dtype == torch.bool:
        raise RuntimeError(
            "Negation, the `-` operator, on a bool tensor is not supported. "
            "If you are trying to invert a mask, use the `~` or `logical_not()` operator instead."
        )
    dev = _lib.require_cuda(input)
    target, res = _prepare_out(out, input.shape, input.dtype, dev, like=input)
    _unary(_lib.UNARY_NEG, input, res, "ntops_amd.neg")
    if res is not target:
        _cast_into(res, target)
    return target
