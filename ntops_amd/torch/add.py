"""add -- mirror of src/ntops/torch/add.py:7-15 (math: kernels/add.py:10).

Follows torch's semantics for broadcasting, type promotion and Python-number
operands (ntops requires equal shapes and dtypes)."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _binary


def add(input, other, *, alpha=1, out=None):
    return _binary(_lib.BINARY_ADD, input, other, alpha, out, "ntops_amd.add")
