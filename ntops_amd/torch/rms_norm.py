"""rms_norm -- mirror of src/ntops/torch/rms_norm.py:9-31
(math: kernels/rms_norm.py:10-20).

The weight is expanded like the reference's `weight.expand_as(input)`: any
shape that broadcasts to the input is accepted.  Semantic deltas from ntops,
following torch (the parity reference the reference's own test compares
against): `eps=None` uses torch.finfo(torch.float32).eps (what torch 2.10's
fused CPU kernel uses for fp32/fp16/bf16 inputs; ntops takes the input
dtype's eps, 7.8e-3 for bf16), and the weight is applied in fp32 before the
single rounding of each output element."""

import math

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard, _norm_param, _rows_of


def rms_norm(input, normalized_shape, weight=None, eps=None):
    if isinstance(normalized_shape, int):
        normalized_shape = (normalized_shape,)

    normalized_shape = tuple(normalized_shape)
    nd = len(normalized_shape)
    if tuple(input.shape[input.dim() - nd :]) != normalized_shape or nd > input.dim():
        raise RuntimeError(
            f"rms_norm: normalized_shape {normalized_shape} does not match input shape {tuple(input.shape)}"
        )
    if input.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"rms_norm: unsupported dtype {input.dtype}")

    if eps is None:
        eps = torch.finfo(torch.float32).eps

    dev = _lib.require_cuda(input, weight)
    cols = math.prod(normalized_shape)
    rows = input.numel() // cols if cols else 0
    x, x_rs = _rows_of(input, nd)
    output = torch.empty(input.shape, dtype=input.dtype, device=input.device)

    w_ptr, w_rs, w_code = None, 0, _lib.dtype_code(input.dtype)
    if weight is not None:
        w_dtype = weight.dtype if weight.dtype in (input.dtype, torch.float32) else input.dtype
        weight, w_rs = _norm_param(weight, input, nd, w_dtype)
        if weight is not None:
            w_ptr, w_code = weight.data_ptr(), _lib.dtype_code(w_dtype)

    lib = _lib.load()
    with _DeviceGuard(dev):
        rc = lib.ntops_rms_norm(
            _lib.dtype_code(input.dtype),
            rows,
            cols,
            x.data_ptr(),
            x_rs,
            w_ptr,
            w_rs,
            w_code,
            float(eps),
            output.data_ptr(),
            cols,
            _lib.stream_of(output),
        )
    _lib.check(rc, "ntops_amd.rms_norm")
    return output
