"""isnan -- mirror of src/ntops/torch/isnan.py:7-14 (math: kernels/isnan.py:9).

Returns a bool tensor like torch.isnan (the reference writes into a tensor of
input's dtype); integer and bool inputs give false everywhere."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard, _strides


def isnan(input):
    dev = _lib.require_cuda(input)
    output = torch.empty(input.shape, dtype=torch.bool, device=dev)
    lib = _lib.load()
    with _DeviceGuard(dev):
        rc = lib.ntops_classify(
            _lib.CLASSIFY_ISNAN, _lib.dtype_code(input.dtype), input.dim(), _lib.i64_array(input.shape),
            input.data_ptr(), _strides(input), output.data_ptr(), _strides(output), _lib.stream_of(output),
        )
    _lib.check(rc, "ntops_amd.isnan")
    return output
