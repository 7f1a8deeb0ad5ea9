"""ge -- mirror of src/ntops/torch/ge.py:7-15 (math: kernels/ge.py:9).

Returns a bool tensor and promotes / broadcasts like torch.ge (the reference
writes the result into a tensor of input's dtype)."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _compare


def ge(input, other, *, out=None):
    return _compare(_lib.CMP_GE, input, other, out, "ntops_amd.ge")
