"""sin -- mirror of src/ntops/torch/sin.py:7-15 (math: kernels/sin.py).

Integer and bool inputs are promoted to the default floating dtype first, as
torch.sin does; 16-bit floats compute in fp32 and round once."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _float_unary


def sin(input, *, out=None):
    return _float_unary(_lib.UNARY_SIN, input, out, "ntops_amd.sin")
