"""lt -- mirror of src/ntops/torch/lt.py:7-15 (math: kernels/lt.py:9).

Returns a bool tensor and promotes / broadcasts like torch.lt (the reference
writes the result into a tensor of input's dtype)."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _compare


def lt(input, other, *, out=None):
    return _compare(_lib.CMP_LT, input, other, out, "ntops_amd.lt")
