"""add_rms_norm -- the residual step of an LLM block in one pass:

    new_residual = input + residual          (rounded to the dtype, as torch's `+`)
    output = rms_norm(new_residual, normalized_shape, weight, eps)

No ntops counterpart: it fuses torch/add.py:7-15 and torch/rms_norm.py:9-31
(math: kernels/rms_norm.py:10-20), with rms_norm's conventions here (eps=None
is torch.finfo(torch.float32).eps; the weight is applied in fp32 before the
single rounding).  Returns (output, new_residual), each element equal to the
two separate ops.  With inplace=True the new residual is written into
`residual` and the output into `input`, and those two tensors are returned."""

import math

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard, _norm_param, _rows_of


def add_rms_norm(input, residual, normalized_shape, weight=None, eps=None, *, inplace=False):
    if isinstance(normalized_shape, int):
        normalized_shape = (normalized_shape,)
    normalized_shape = tuple(normalized_shape)
    nd = len(normalized_shape)
    if nd > input.dim() or tuple(input.shape[input.dim() - nd:]) != normalized_shape:
        raise RuntimeError(
            f"add_rms_norm: normalized_shape {normalized_shape} does not match input shape {tuple(input.shape)}")
    if residual.shape != input.shape or residual.dtype != input.dtype:
        raise RuntimeError("add_rms_norm: residual must match input in shape and dtype")
    if input.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"add_rms_norm: unsupported dtype {input.dtype}")
    if eps is None:
        eps = torch.finfo(torch.float32).eps

    dev = _lib.require_cuda(input, residual, weight)
    cols = math.prod(normalized_shape)
    rows = input.numel() // cols if cols else 0
    if inplace:
        if not (input.is_contiguous() and residual.is_contiguous()):
            raise RuntimeError("add_rms_norm: inplace needs contiguous input and residual")
        if input.data_ptr() == residual.data_ptr():
            raise RuntimeError("add_rms_norm: inplace needs distinct input and residual")
        x, res, output, new_residual = input, residual, input, residual
        x_rs = r_rs = cols
    else:
        (x, x_rs), (res, r_rs) = _rows_of(input, nd), _rows_of(residual, nd)
        output = torch.empty(input.shape, dtype=input.dtype, device=input.device)
        new_residual = torch.empty(input.shape, dtype=input.dtype, device=input.device)

    w_ptr, w_rs, w_code = None, 0, _lib.dtype_code(input.dtype)
    if weight is not None:
        w_dtype = weight.dtype if weight.dtype in (input.dtype, torch.float32) else input.dtype
        weight, w_rs = _norm_param(weight, input, len(normalized_shape), w_dtype)
        if weight is not None:
            w_ptr, w_code = weight.data_ptr(), _lib.dtype_code(w_dtype)

    lib = _lib.load()
    with _DeviceGuard(dev):
        rc = lib.ntops_add_rms_norm(
            _lib.dtype_code(input.dtype), rows, cols, x.data_ptr(), x_rs, res.data_ptr(), r_rs, w_ptr, w_rs, w_code,
            float(eps), output.data_ptr(), cols, new_residual.data_ptr(), cols, _lib.stream_of(output))
    _lib.check(rc, "ntops_amd.add_rms_norm")
    return output, new_residual
