"""le -- mirror of src/ntops/torch/le.py:7-15 (math: kernels/le.py:9).

Returns a bool tensor and promotes / broadcasts like torch.le (the reference
writes the result into a tensor of input's dtype)."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _compare


def le(input, other, *, out=None):
    return _compare(_lib.CMP_LE, input, other, out, "ntops_amd.le")
