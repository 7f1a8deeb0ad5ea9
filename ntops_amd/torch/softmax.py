"""softmax -- mirror of src/ntops/torch/softmax.py:7-16
(math: kernels/softmax.py:9-29 with fp32 max/sum accumulation)."""

import math

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard, _contiguous


def softmax(input, dim, dtype=None):
    tensor_dtype = dtype if dtype is not None else input.dtype
    if tensor_dtype not in (torch.float32, torch.float16, torch.bfloat16, torch.float64):
        raise RuntimeError(f"softmax: unsupported output dtype {tensor_dtype}")
    if input.dtype not in (torch.float32, torch.float16, torch.bfloat16, torch.float64):
        raise RuntimeError(f"softmax: unsupported input dtype {input.dtype}")

    ndim = input.dim()
    if ndim == 0:
        if dim not in (0, -1):
            raise IndexError("Dimension out of range (expected to be in range of [-1, 0])")
        outer, size, inner = 1, 1, 1
    else:
        if not -ndim <= dim < ndim:
            raise IndexError(f"Dimension out of range (expected to be in range of [{-ndim}, {ndim - 1}])")
        dim = dim % ndim
        outer = math.prod(input.shape[:dim])
        size = input.shape[dim]
        inner = math.prod(input.shape[dim + 1 :])

    dev = _lib.require_cuda(input)
    x = _contiguous(input)
    output = torch.empty(input.shape, dtype=tensor_dtype, device=input.device)
    strides = (size * inner, inner, 1)

    lib = _lib.load()
    with _DeviceGuard(dev):
        rc = lib.ntops_softmax(
            _lib.dtype_code(input.dtype),
            _lib.dtype_code(tensor_dtype),
            outer,
            size,
            inner,
            x.data_ptr(),
            _lib.i64_array(strides),
            output.data_ptr(),
            _lib.i64_array(strides),
            _lib.stream_of(output),
        )
    _lib.check(rc, "ntops_amd.softmax")
    return output
