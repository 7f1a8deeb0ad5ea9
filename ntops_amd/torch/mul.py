"""mul -- mirror of src/ntops/torch/mul.py:7-15 (math: kernels/mul.py:9)."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _binary


def mul(input, other, *, out=None):
    return _binary(_lib.BINARY_MUL, input, other, None, out, "ntops_amd.mul")
