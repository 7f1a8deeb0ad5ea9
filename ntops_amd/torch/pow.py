"""pow -- mirror of src/ntops/torch/pow.py:7-15 (math: kernels/pow.py:10).

Accepts tensor ** tensor, tensor ** number and number ** tensor with torch's
promotion and broadcasting.  A number exponent is rounded to the tensor's
dtype and the exponents torch special-cases (2, 3, 0.5, -0.5, -1, -2) are
computed as torch computes them; integer tensors follow torch's rule for
negative exponents."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _binary, _is_number, _split_other


def pow(input, exponent, *, out=None):
    if _is_number(input):
        if not isinstance(exponent, torch.Tensor):
            raise TypeError("ntops_amd.pow: at least one operand must be a tensor")
        dtype = torch.result_type(input, exponent)
        input = torch.tensor(input, dtype=dtype, device=exponent.device)
    _, _, dtype = _split_other(input, exponent, "ntops_amd.pow")
    if dtype == torch.bool:
        raise NotImplementedError('"pow" not implemented for Bool')
    if not dtype.is_floating_point and _is_number(exponent) and exponent < 0:
        raise RuntimeError("Integers to negative integer powers are not allowed.")
    return _binary(_lib.BINARY_POW, input, exponent, None, out, "ntops_amd.pow")
