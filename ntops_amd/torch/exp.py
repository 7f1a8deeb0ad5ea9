"""exp -- mirror of src/ntops/torch/exp.py:7-15 (math: kernels/exp.py:10).

Integer and bool inputs are promoted to the default floating dtype first, as
torch.exp does."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _cast_into, _prepare_out, _to_dtype, _unary


def exp(input, *, out=None):
    dev = _lib.require_cuda(input)
    dtype = input.dtype if input.dtype.is_floating_point else torch.get_default_dtype()
    x = _to_dtype(input, dtype)
    target, res = _prepare_out(out, input.shape, dtype, dev, like=x)
    _unary(_lib.UNARY_EXP, x, res, "ntops_amd.exp")
    if res is not target:
        _cast_into(res, target)
    return target
