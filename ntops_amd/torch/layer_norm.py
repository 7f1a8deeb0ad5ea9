"""layer_norm -- mirror of src/ntops/torch/layer_norm.py:9-33
(math: kernels/layer_norm.py:11-31; fp32 moments, biased variance)."""

import math

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard, _norm_param, _rows_of


def layer_norm(input, normalized_shape, weight=None, bias=None, eps=1e-5):
    if isinstance(normalized_shape, int):
        normalized_shape = (normalized_shape,)

    normalized_shape = tuple(normalized_shape)
    nd = len(normalized_shape)
    if tuple(input.shape[input.dim() - nd :]) != normalized_shape or nd > input.dim():
        raise RuntimeError(
            f"layer_norm: normalized_shape {normalized_shape} does not match input shape {tuple(input.shape)}"
        )
    if input.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"layer_norm: unsupported dtype {input.dtype}")

    dev = _lib.require_cuda(input, weight, bias)
    cols = math.prod(normalized_shape)
    rows = input.numel() // cols if cols else 0
    x, x_rs = _rows_of(input, nd)
    output = torch.empty(input.shape, dtype=input.dtype, device=input.device)

    # weight and bias share one dtype (the input's, or fp32 for both) and
    # one row stride: each is expanded like the reference's
    # `expand_as(input)`; if either differs per row, both are laid out per row.
    params = [p for p in (weight, bias) if p is not None]
    wb_dtype = input.dtype
    if params and all(p.dtype == torch.float32 for p in params):
        wb_dtype = torch.float32
    laid = [_norm_param(p, input, nd, wb_dtype) if p is not None else (None, 0) for p in (weight, bias)]
    wb_rs = max(rs for _, rs in laid)
    if wb_rs:
        laid = [_norm_param(p, input, nd, wb_dtype, per_row=True) if p is not None else (None, 0)
                for p in (weight, bias)]
    (weight, _), (bias, _) = laid

    lib = _lib.load()
    with _DeviceGuard(dev):
        rc = lib.ntops_layer_norm(
            _lib.dtype_code(input.dtype),
            rows,
            cols,
            x.data_ptr(),
            x_rs,
            weight.data_ptr() if weight is not None else None,
            bias.data_ptr() if bias is not None else None,
            wb_rs,
            _lib.dtype_code(wb_dtype),
            float(eps),
            output.data_ptr(),
            cols,
            _lib.stream_of(output),
        )
    _lib.check(rc, "ntops_amd.layer_norm")
    return output
