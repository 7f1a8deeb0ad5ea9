"""conv2d -- mirror of src/ntops/torch/conv2d.py:8-53 (math: kernels/conv2d.py:12-104).

Same arguments as the reference: stride / padding / dilation as ints or
pairs, padding "valid" (= 0), groups must be 1 (asserted), bias optional;
the output dtype is the input's and its size follows
torch/pooling.py:4-19 (floor mode).  Also accepted, as torch does: padding
"same" (stride 1; an odd total padding puts the extra row / column at the
bottom / right) and unbatched (C, H, W) input.  Problems with enough
channels run as an unfold into a workspace (allocated here, at most
_WORKSPACE_CAP bytes, so large batches run in chunks) plus a matrix-core
GEMM; small ones run a direct kernel."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard, _strides

_WORKSPACE_CAP = 512 << 20


def _pair(v, what):
    if isinstance(v, int):
        return (v, v)
    v = tuple(int(e) for e in v)
    if len(v) != 2:
        raise RuntimeError(f"ntops_amd.conv2d: expected {what} to be a single int or a pair")
    return v


def _output_size(size, kernel, stride, padding, dilation):
    return (size + 2 * padding - dilation * (kernel - 1) - 1) // stride + 1


def conv2d(input, weight, bias=None, stride=1, padding=0, dilation=1, groups=1):
    assert groups == 1, "`groups` is not supported yet."
    stride = _pair(stride, "stride")
    dilation = _pair(dilation, "dilation")
    unbatched = input.dim() == 3
    if unbatched:
        input = input.unsqueeze(0)
    if input.dim() != 4 or weight.dim() != 4:
        raise RuntimeError("ntops_amd.conv2d: expected 4-D input (or 3-D unbatched) and 4-D weight")
    n, c, h, w = input.shape
    k, cw, r, s = weight.shape
    if cw != c:
        raise RuntimeError(f"ntops_amd.conv2d: weight expects {cw} input channels, input has {c}")
    if input.dtype != weight.dtype or (bias is not None and bias.dtype != input.dtype):
        raise RuntimeError("ntops_amd.conv2d: input, weight and bias must have the same dtype")
    if bias is not None and (bias.dim() != 1 or bias.shape[0] != k):
        raise RuntimeError(f"ntops_amd.conv2d: bias must have shape ({k},)")

    if isinstance(padding, str):
        if padding == "valid":
            top, left, p, q = 0, 0, _output_size(h, r, stride[0], 0, dilation[0]), _output_size(
                w, s, stride[1], 0, dilation[1])
        elif padding == "same":
            if stride != (1, 1):
                raise RuntimeError("ntops_amd.conv2d: padding='same' is not supported for strided convolutions")
            top, left = dilation[0] * (r - 1) // 2, dilation[1] * (s - 1) // 2
            p, q = h, w
        else:
            raise RuntimeError(f"ntops_amd.conv2d: invalid padding string {padding!r}")
    else:
        top, left = _pair(padding, "padding")
        p = _output_size(h, r, stride[0], top, dilation[0])
        q = _output_size(w, s, stride[1], left, dilation[1])
    if p <= 0 or q <= 0:
        raise RuntimeError("ntops_amd.conv2d: kernel size can't be greater than the padded input size")

    dev = _lib.require_cuda(input, weight, bias)
    output = torch.empty((n, k, p, q), dtype=input.dtype, device=dev)
    dt = _lib.dtype_code(input.dtype)
    geometry = (n, c, h, w, k, r, s, p, q, stride[0], stride[1], top, left, dilation[0], dilation[1])
    lib = _lib.load()
    ws_bytes = lib.ntops_conv2d_workspace(dt, *geometry, _strides(weight), _strides(output))
    workspace = None
    if ws_bytes > 0:
        # the whole batch in one pass if it fits the cap, else chunks: at
        # least what one image needs (its bytes plus any per-call part)
        one = lib.ntops_conv2d_workspace(dt, 1, *geometry[1:], _strides(weight), _strides(output))
        size = min(ws_bytes, max(one, _WORKSPACE_CAP))
        workspace = torch.empty(size, dtype=torch.uint8, device=dev)
    with _DeviceGuard(dev):
        rc = lib.ntops_conv2d(
            dt, *geometry,
            input.data_ptr(), _strides(input), weight.data_ptr(), _strides(weight),
            None if bias is None else bias.data_ptr(), 0 if bias is None else bias.stride(0),
            output.data_ptr(), _strides(output),
            None if workspace is None else workspace.data_ptr(), 0 if workspace is None else workspace.numel(),
            _lib.stream_of(output),
        )
    _lib.check(rc, "ntops_amd.conv2d")
    return output.squeeze(0) if unbatched else output
