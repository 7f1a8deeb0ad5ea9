"""Shared launch of the native GEMM (ntops_gemm) for mm / bmm / addmm."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard

_GEMM_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _strides3(t):
    """(batch, row, col) strides of a 2-D or 3-D operand (batch 0 for 2-D)."""
    if t.dim() == 2:
        return (0, t.stride(0), t.stride(1))
    return (t.stride(0) if t.shape[0] > 1 else 0, t.stride(1), t.stride(2))


def gemm(a, b, out, c=None, alpha=1.0, beta=0.0, what="ntops_amd.mm"):
    """out = alpha * (a @ b) + beta * c for 2-D (mm) or 3-D (bmm) operands;
    c is already expanded to out's shape (stride 0 where broadcast)."""
    if a.dtype not in _GEMM_DTYPES:
        raise RuntimeError(f"{what}: unsupported dtype {a.dtype}")
    for t in (b, out) + ((c,) if c is not None else ()):
        if t.dtype != a.dtype:
            raise RuntimeError(
                f"{what}: expected all operands to have dtype {a.dtype}, got {t.dtype}"
            )
    dev = _lib.require_cuda(a, b, out, c)
    batch = a.shape[0] if a.dim() == 3 else 1
    m, k = a.shape[-2], a.shape[-1]
    n = b.shape[-1]
    lib = _lib.load()
    with _DeviceGuard(dev):
        rc = lib.ntops_gemm(
            _lib.dtype_code(a.dtype),
            batch,
            m,
            n,
            k,
            a.data_ptr(),
            _lib.i64_array(_strides3(a)),
            b.data_ptr(),
            _lib.i64_array(_strides3(b)),
            c.data_ptr() if c is not None else None,
            _lib.i64_array(_strides3(c)) if c is not None else None,
            float(alpha),
            float(beta),
            out.data_ptr(),
            _lib.i64_array(_strides3(out)),
            _lib.stream_of(out),
        )
    _lib.check(rc, what)
    return out
