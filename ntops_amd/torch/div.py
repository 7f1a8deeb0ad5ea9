"""div -- mirror of src/ntops/torch/div.py:7-15 (math: kernels/div.py:9-18).

rounding_mode None: true division (integers promote to the default float
dtype); "trunc": the quotient rounded toward zero; "floor": Python's floor
division (kernels/div.py:18 writes floor(a / b); the kernel uses the
fmod-based form that torch and Python use, which differs from floor(a / b)
when the rounded quotient lands on an integer).  Integer "trunc" / "floor"
by zero gives 0 (torch's CPU kernel raises ZeroDivisionError)."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _binary, _split_other


def _true_div_dtype(dtype):
    return dtype if dtype.is_floating_point else torch.get_default_dtype()


def div(input, other, *, rounding_mode=None, out=None):
    if rounding_mode is None:
        return _binary(_lib.BINARY_DIV, input, other, None, out, "ntops_amd.div", _true_div_dtype)
    if rounding_mode not in ("trunc", "floor"):
        raise RuntimeError(
            f"div expected rounding_mode to be one of None, 'trunc', or 'floor' but found '{rounding_mode}'"
        )
    _, _, dtype = _split_other(input, other, "ntops_amd.div")
    if dtype == torch.bool:
        raise NotImplementedError(f'"div_{rounding_mode}" not implemented for Bool')
    op = _lib.BINARY_DIV_TRUNC if rounding_mode == "trunc" else _lib.BINARY_DIV_FLOOR
    return _binary(op, input, other, None, out, "ntops_amd.div")
