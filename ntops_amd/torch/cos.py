"""cos -- mirror of src/ntops/torch/cos.py:7-15 (math: kernels/cos.py).

Integer and bool inputs are promoted to the default floating dtype first, as
torch.cos does; 16-bit floats compute in fp32 and round once."""

from ntops_amd import _lib
from ntops_amd.torch.utils import _float_unary


def cos(input, *, out=None):
    return _float_unary(_lib.UNARY_COS, input, out, "ntops_amd.cos")
