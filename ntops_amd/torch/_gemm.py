"""Shared launch of the native GEMM (ntops_gemm) for mm / bmm / addmm."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard, _cast_into

_GEMM_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _strides3(t):
    """(batch, row, col) strides of a 2-D or 3-D operand (batch 0 for 2-D)."""
    if t.dim() == 2:
        return (0, t.stride(0), t.stride(1))
    return (t.stride(0) if t.shape[0] > 1 else 0, t.stride(1), t.stride(2))


def _padded_width(a, b, n):
    """Column count to run the GEMM at when n columns would send it to the
    generic kernel (None otherwise): the matrix-core kernels load an N-major
    B in 16-byte row pieces (16-bit: N % 8 == 0; fp32: N % 4 == 0).  A K-major
    B has no such limit, and output rows of any width are stored element by
    element."""
    unit = 4 if a.dtype == torch.float32 else 8
    if n <= unit or n % unit == 0 or a.shape[-1] == 0 or a.shape[-2] == 0:
        return None
    if b.stride(-2) == 1 and b.stride(-1) != 1:  # K-major B: N is free
        return None
    return (n + unit - 1) // unit * unit


def _padded_depth(a, b, k):
    """Depth to run the GEMM at when a K-major operand's rows of k elements
    would send it to the generic kernel (None otherwise)."""
    unit = 4 if a.dtype == torch.float32 else 8
    if k <= unit or k % unit == 0 or a.shape[-2] == 0 or b.shape[-1] == 0:
        return None
    a_kmajor = a.stride(-1) == 1
    b_kmajor = b.stride(-2) == 1 and b.stride(-1) != 1
    if not (a_kmajor or b_kmajor):
        return None
    return (k + unit - 1) // unit * unit


def _kernel_layout(t, unit, other_major=True):
    """True when operand t (A as (m, k), B as (k, n)) is in a layout the
    matrix-core kernels read: its last axis with unit stride and rows of a
    multiple of `unit` elements (A K-major, B N-major), or, when other_major,
    its first axis with unit stride and columns of a multiple of `unit`
    elements (A M-major, which also needs M % unit == 0; B K-major); a
    contiguous axis whose length is not a multiple of `unit` is fine too (the
    padded paths below copy it); and a 16-byte aligned start and batch
    stride."""
    r, c = t.shape[-2], t.shape[-1]
    if t.data_ptr() % 16 or not (t.dim() == 2 or t.shape[0] == 1 or t.stride(0) % unit == 0):
        return False
    if t.stride(-1) == 1:
        return t.stride(-2) % unit == 0 or c % unit != 0 or r == 1
    if other_major and t.stride(-2) == 1:
        return t.stride(-1) % unit == 0 or r % unit != 0 or c == 1
    return False


def _layout_copies(a, b):
    """A and B as the matrix-core kernels can read them: an operand in
    neither of their layouts (an M-major A whose M is not a multiple of 8,
    an fp32 A that is not K-major, an operand with no unit-stride axis, a
    start that is not 16-byte aligned) is copied into a fresh row-major
    tensor by the native cast kernel, so the product leaves the generic
    kernel.  Products too small to matter keep the operands as they are."""
    unit = 4 if a.dtype == torch.float32 else 8
    m, k, n = a.shape[-2], a.shape[-1], b.shape[-1]
    if m <= unit or n <= unit or k == 0:
        return a, b
    m_major_ok = a.dtype != torch.float32 and m % unit == 0
    if not _kernel_layout(a, unit, other_major=m_major_ok):
        ac = torch.empty(a.shape, dtype=a.dtype, device=a.device)
        _cast_into(a, ac)
        a = ac
    if not _kernel_layout(b, unit):
        bc = torch.empty(b.shape, dtype=b.dtype, device=b.device)
        _cast_into(b, bc)
        b = bc
    return a, b


def _pad_last_two(t, rows, cols):
    """A new tensor of t's batch shape x (rows, cols) holding t in its leading
    corner and zeros elsewhere (copies and fills by the native cast kernel)."""
    p = torch.empty(t.shape[:-2] + (rows, cols), dtype=t.dtype, device=t.device)
    zero = torch.zeros((), dtype=t.dtype, device=t.device)
    r, c = t.shape[-2], t.shape[-1]
    _cast_into(t, p[..., :r, :c])
    if cols > c:
        _cast_into(zero.expand(p[..., :, c:].shape), p[..., :, c:])
    if rows > r:
        _cast_into(zero.expand(p[..., r:, :c].shape), p[..., r:, :c])
    return p


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
    with _DeviceGuard(dev):
        a, b = _layout_copies(a, b)
    k = a.shape[-1]
    kp = _padded_depth(a, b, k)
    if kp is not None:
        # A's rows and B's columns extended with zeros to depth kp (the
        # products they add are exact zeros)
        with _DeviceGuard(dev):
            ap = _pad_last_two(a, a.shape[-2], kp)
            bp = _pad_last_two(b, kp, b.shape[-1])
        return gemm(ap, bp, out, c, alpha, beta, what)
    n = b.shape[-1]
    np_ = _padded_width(a, b, n)
    if np_ is not None:
        # B (and C) copied into rows of np_ columns, the product computed at
        # that width, its first n columns copied out (the extra columns only
        # ever meet the extra columns of B and C)
        with _DeviceGuard(dev):
            bp = torch.empty(b.shape[:-1] + (np_,), dtype=b.dtype, device=b.device)
            _cast_into(b, bp[..., :n])
            cp = None
            if c is not None:
                if all(s == 0 for s in c.stride()[:-1]):  # one row broadcast (a bias)
                    row = torch.empty(np_, dtype=c.dtype, device=c.device)
                    _cast_into(c[(0,) * (c.dim() - 1)], row[:n])
                    cp = row.expand(out.shape[:-1] + (np_,))
                else:
                    cp = torch.empty(out.shape[:-1] + (np_,), dtype=c.dtype, device=c.device)
                    _cast_into(c, cp[..., :n])
            # the first n0 columns go straight into out (the kernels store rows
            # that start anywhere; 16-bit tiles take 256 columns at a time,
            # fp32 ones 4), only the last np_ - n0 through the temporary; the
            # interior is launched last
            n0 = n // 256 * 256 if out.dtype != torch.float32 else n // 4 * 4
            op = torch.empty(out.shape[:-1] + (np_ - n0,), dtype=out.dtype, device=out.device)
        gemm(a, bp[..., n0:], op, None if cp is None else cp[..., n0:], alpha, beta, what)
        if n0:
            gemm(a, bp[..., :n0], out[..., :n0], None if c is None else c[..., :n0], alpha, beta, what)
        with _DeviceGuard(dev):
            _cast_into(op[..., :n - n0], out[..., n0:])
        return out
    batch = a.shape[0] if a.dim() == 3 else 1
    m, k = a.shape[-2], a.shape[-1]
    n = b.shape[-1]
    lib = _lib.load()
    dt = _lib.dtype_code(a.dtype)
    with _DeviceGuard(dev):
        # products that would not fill the GPU split K through a workspace
        # (fp32 partial products, summed in a fixed order)
        ws_bytes = lib.ntops_gemm_workspace(dt, batch, m, n, k)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
        rc = lib.ntops_gemm_ws(
            dt,
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
            ws.data_ptr() if ws is not None else None,
            ws_bytes,
            _lib.stream_of(out),
        )
    _lib.check(rc, what)
    return out
