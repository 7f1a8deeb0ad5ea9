"""im2col -- mirror of src/ntops/torch/im2col.py:44-135 (arrangement:
kernels/im2col.py:10-80).

Same arguments, checks and messages as the reference: kernel_size /
dilation / padding / stride each an int or a 1- or 2-element iterable, a
4-D input of any dtype, output (N, C * kh * kw, oh * ow) of the input's
dtype with the floor-mode output size of torch/im2col.py:28-31.  The input is
read through its strides (no contiguous copy); the native kernel moves every
dtype as its bits, so the result is exact."""

import math
from collections.abc import Iterable

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard, _strides


def _pair(value, name):
    if isinstance(value, int):
        return value, value
    if isinstance(value, Iterable):
        value = tuple(value)
        if len(value) == 1:
            return value[0], value[0]
        if len(value) == 2:
            return value
    raise TypeError(f"{name} must be an int or a pair of ints")


def _calculate_output_size(input_size, kernel_size, dilation, padding, stride):
    return math.floor((input_size + 2 * padding - dilation * (kernel_size - 1) - 1) / stride + 1)


def im2col(input, kernel_size, dilation=1, padding=0, stride=1):
    if input.ndim != 4:
        raise RuntimeError(f"Expected 4D input tensor, but got tensor with {input.ndim} dimensions")

    kernel_size = _pair(kernel_size, "kernel_size")
    dilation = _pair(dilation, "dilation")
    padding = _pair(padding, "padding")
    stride = _pair(stride, "stride")

    if any(size <= 0 for size in kernel_size):
        raise RuntimeError("kernel_size should be greater than zero")
    if any(size <= 0 for size in dilation):
        raise RuntimeError("dilation should be greater than zero")
    if any(size <= 0 for size in stride):
        raise RuntimeError("stride should be greater than zero")
    if any(size < 0 for size in padding):
        raise RuntimeError("padding should be non-negative")

    n, c, h, w = input.shape
    out_h = _calculate_output_size(h, kernel_size[0], dilation[0], padding[0], stride[0])
    out_w = _calculate_output_size(w, kernel_size[1], dilation[1], padding[1], stride[1])
    if out_h < 1 or out_w < 1:
        raise RuntimeError(
            f"Given input with spatial size ({h}, {w}), kernel_size={kernel_size}, dilation={dilation}, "
            f"padding={padding}, calculated output shape ({out_h}, {out_w}), "
            "but its components must be at least one."
        )

    dev = _lib.require_cuda(input)
    output = torch.empty((n, c * kernel_size[0] * kernel_size[1], out_h * out_w), dtype=input.dtype, device=dev)
    lib = _lib.load()
    with _DeviceGuard(dev):
        rc = lib.ntops_im2col(
            _lib.dtype_code(input.dtype), n, c, h, w, kernel_size[0], kernel_size[1], dilation[0], dilation[1],
            padding[0], padding[1], stride[0], stride[1],
            input.data_ptr(), _strides(input), output.data_ptr(), _strides(output), _lib.stream_of(output),
        )
    _lib.check(rc, "ntops_amd.im2col")
    return output
