"""gt -- mirror of src/ntops/torch/gt.py:7-15 (math: kernels/gt.py:9).

Returns a bool tensor and promotes / broadcasts like torch.gt (the reference
writes the result into a tensor of input's dtype)."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _compare


def gt(input, other, *, out=None):
    return _compare(_lib.CMP_GT, input, other, out, "ntops_amd.gt")
