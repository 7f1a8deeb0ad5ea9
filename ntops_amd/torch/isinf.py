"""isinf -- mirror of src/ntops/torch/isinf.py:7-14 (math: kernels/isinf.py:9).

Returns a bool tensor like torch.isinf (the reference writes into a tensor of
input's dtype); integer and bool inputs give false everywhere."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard, _strides


def isinf(input):
    dev = _lib.require_cuda(input)
    output = torch.empty(input.shape, dtype=torch.bool, device=dev)
    lib = _lib.load()
    with _DeviceGuard(dev):
        rc = lib.ntops_classify(
            _lib.CLASSIFY_ISINF, _lib.dtype_code(input.dtype), input.dim(), _lib.i64_array(input.shape),
            input.data_ptr(), _strides(input), output.data_ptr(), _strides(output), _lib.stream_of(output),
        )
    _lib.check(rc, "ntops_amd.isinf")
    return output
