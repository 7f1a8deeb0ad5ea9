"""eq -- mirror of src/ntops/torch/eq.py:7-15 (math: kernels/eq.py:9).

Returns a bool tensor and promotes / broadcasts like torch.eq (the reference
writes the result into a tensor of input's dtype)."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _compare


def eq(input, other, *, out=None):
    return _compare(_lib.CMP_EQ, input, other, out, "ntops_amd.eq")
