"""rsqrt -- mirror of src/ntops/torch/rsqrt.py:7-15 (math: kernels/rsqrt.py).

Integer and bool inputs are promoted to the default floating dtype first, as
torch.rsqrt does; 16-bit floats compute in fp32 and round once."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _float_unary


def rsqrt(input, *, out=None):
    return _float_unary(_lib.UNARY_RSQRT, input, out, "ntops_amd.rsqrt")
