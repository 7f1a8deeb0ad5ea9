"""tanh -- mirror of src/ntops/torch/tanh.py:7-15 (math: kernels/tanh.py).

Integer and bool inputs are promoted to the default floating dtype first, as
torch.tanh does; 16-bit floats compute in fp32 and round once."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _float_unary


def tanh(input, *, out=None):
    return _float_unary(_lib.UNARY_TANH, input, out, "ntops_amd.tanh")
