"""sigmoid -- mirror of src/ntops/torch/sigmoid.py:7-15 (math: kernels/sigmoid.py).

Integer and bool inputs are promoted to the default floating dtype first, as
torch.sigmoid does; 16-bit floats compute in fp32 and round once."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _float_unary


def sigmoid(input, *, out=None):
    return _float_unary(_lib.UNARY_SIGMOID, input, out, "ntops_amd.sigmoid")
