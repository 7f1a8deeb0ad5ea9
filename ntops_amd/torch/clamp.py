"""clamp -- mirror of src/ntops/torch/clamp.py:7-15 (math: kernels/clamp.py:9).

min / max may each be None, a Python number or a tensor (broadcast), like
torch.clamp; the result dtype, shape and argument checks are torch's.  Number bounds are rounded
to the result dtype; a NaN in the input or a bound propagates."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import (
    _broadcast_shape,
    _DeviceGuard,
    _cast_into,
    _expand_to,
    _is_number,
    _prepare_out,
    _strides,
    _to_dtype,
)


def _as_bound(v):
    if isinstance(v, torch.Tensor) and v.dim() == 0 and not v.is_cuda:
        return v.item()
    return v


def _proxy(v):
    """A one-element CPU tensor standing in for tensor v in torch's type
    promotion (same dtype, zero-dim or not like v), or v itself."""
    if isinstance(v, torch.Tensor):
        return torch.zeros((1,) * v.dim(), dtype=v.dtype)
    return v


def _result(input, lo, hi):
    """torch.clamp's result dtype and shape, with its argument errors, at a
    few microseconds of host time: number bounds on a floating tensor keep
    its dtype and shape; otherwise torch.clamp decides on one-element CPU
    stand-ins (the dtype) and the shapes broadcast (the shape)."""
    if input.dtype.is_floating_point and not any(isinstance(v, torch.Tensor) for v in (lo, hi)):
        return input.dtype, input.shape
    dtype = torch.clamp(_proxy(input), _proxy(lo), _proxy(hi)).dtype
    shape = input.shape
    for v in (lo, hi):
        if isinstance(v, torch.Tensor):
            shape = _broadcast_shape(shape, v.shape)
    return dtype, shape


def clamp(input, min=None, max=None, *, out=None):
    lo, hi = _as_bound(min), _as_bound(max)
    if lo is None and hi is None:
        raise RuntimeError("torch.clamp: At least one of 'min' or 'max' must not be None")
    for v in (lo, hi):
        if v is not None and not isinstance(v, torch.Tensor) and not _is_number(v):
            raise TypeError(f"ntops_amd.clamp: unsupported bound {type(v)}")
    dtype, shape = _result(input, lo, hi)
    dev = _lib.require_cuda(input, *(v for v in (lo, hi) if isinstance(v, torch.Tensor)))
    target, res = _prepare_out(out, shape, dtype, dev, like=input)
    x = _expand_to(_to_dtype(input, dtype), shape)

    def bound(v):
        if v is None:
            return None, None, 0.0, 0, 0
        if isinstance(v, torch.Tensor):
            t = _expand_to(_to_dtype(v, dtype), shape)
            return t, t.data_ptr(), 0.0, 0, 1
        return None, None, float(v), int(v) if not isinstance(v, float) else 0, 1

    lib = _lib.load()
    with _DeviceGuard(dev):
        lt, lp, lf, li, lh = bound(lo)
        ht, hp, hf, hi_i, hh = bound(hi)
        rc = lib.ntops_clamp(
            _lib.dtype_code(dtype), len(shape), _lib.i64_array(shape), x.data_ptr(), _strides(x),
            lp, _strides(lt) if lt is not None else None, lf, li, lh,
            hp, _strides(ht) if ht is not None else None, hf, hi_i, hh,
            res.data_ptr(), _strides(res), _lib.stream_of(res),
        )
        _lib.check(rc, "ntops_amd.clamp")
        if res is not target:
            _cast_into(res, target)
    return target
