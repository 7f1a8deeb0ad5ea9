"""softmax -- mirror of src/ntops/torch/softmax.py:7-16
(math: kernels/softmax.py:9-29 with fp32 max/sum accumulation)."""

import math

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard, _contiguous


def _merged_stride(shape, stride, lo, hi):
    """The one stride that walks dims lo .. hi - 1 of a view as a single
    dim (size-1 dims ignored; 1 when all are size 1), or None when they do
    not merge."""
    dims = [d for d in range(lo, hi) if shape[d] != 1]
    if not dims:
        return 1
    for a, b in zip(dims, dims[1:]):
        if stride[a] != stride[b] * shape[b]:
            return None
    return stride[dims[-1]]


def _view_strides(input, dim):
    """(outer, dim, inner) element strides of `input` seen as
    (outer, size, inner) around `dim`, when the leading and the trailing dims
    each merge into one; else None (the input is then copied row-major).
    Row views of a wider tensor run in place this way."""
    shape, stride = input.shape, input.stride()
    s_outer = _merged_stride(shape, stride, 0, dim)
    s_inner = _merged_stride(shape, stride, dim + 1, input.dim())
    if s_outer is None or s_inner is None:
        return None
    return (s_outer, stride[dim], s_inner)


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
    strides = (size * inner, inner, 1)
    x_strides = _view_strides(input, dim) if ndim > 0 else strides
    x = input
    if x_strides is None:
        x = _contiguous(input)
        x_strides = strides
    output = torch.empty(input.shape, dtype=tensor_dtype, device=input.device)

    lib = _lib.load()
    with _DeviceGuard(dev):
        rc = lib.ntops_softmax(
            _lib.dtype_code(input.dtype),
            _lib.dtype_code(tensor_dtype),
            outer,
            size,
            inner,
            x.data_ptr(),
            _lib.i64_array(x_strides),
            output.data_ptr(),
            _lib.i64_array(strides),
            _lib.stream_of(output),
        )
    _lib.check(rc, "ntops_amd.softmax")
    return output
