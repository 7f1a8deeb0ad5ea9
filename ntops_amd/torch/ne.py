"""ne -- mirror of src/ntops/torch/ne.py:7-15 (math: kernels/ne.py:9).

Returns a bool tensor and promotes / broadcasts like torch.ne (the reference
writes the result into a tensor of input's dtype)."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _compare


def ne(input, other, *, out=None):
    return _compare(_lib.CMP_NE, input, other, out, "ntops_amd.ne")
