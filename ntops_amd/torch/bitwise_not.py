"""bitwise_not -- mirror of src/ntops/torch/bitwise_not.py:7-17
(math: kernels/bitwise_not.py:9-14; bool inputs use logical not)."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _cast_into, _prepare_out, _unary


def bitwise_not(input, *, out=None):
    if input.dtype.is_floating_point or input.dtype.is_complex:
        raise RuntimeError(f'"bitwise_not" not implemented for {input.dtype}')
    dev = _lib.require_cuda(input)
    target, res = _prepare_out(out, input.shape, input.dtype, dev, like=input)
    _unary(_lib.UNARY_BITWISE_NOT, input, res, "ntops_amd.bitwise_not")
    if res is not target:
        _cast_into(res, target)
    return target
