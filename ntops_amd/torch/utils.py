"""Configuration knobs and shared launch helpers of ntops_amd.torch.

The default-knob setters/getters keep the reference's public surface
(src/ntops/torch/utils.py:10-43; tests/conftest.py:14 calls
`set_default_max_num_configs`).  They tune NineToothed's Triton code
generation in the reference; here every kernel is prebuilt for gfx950 with
its launch shape chosen per call from the problem size, so the values are
stored and returned but do not change any launch.
"""

import torch

from ntops_amd import _lib
from ntops_amd.kernels.mm import InputPrecisionVariant


class _CachedMakeDefaultConfig:
    def __init__(self, num_warps=None, num_stages=None, max_num_configs=None):
        self.num_warps = num_warps
        self.num_stages = num_stages
        self.max_num_configs = max_num_configs


_cached_make_default_config = _CachedMakeDefaultConfig()


def get_default_num_warps():
    return _cached_make_default_config.num_warps


def set_default_num_warps(num_warps):
    _cached_make_default_config.num_warps = num_warps


def get_default_num_stages():
    return _cached_make_default_config.num_stages


def set_default_num_stages(num_stages):
    _cached_make_default_config.num_stages = num_stages


def get_default_max_num_configs():
    return _cached_make_default_config.max_num_configs


def set_default_max_num_configs(max_num_configs):
    _cached_make_default_config.max_num_configs = max_num_configs


def _get_matmul_input_precision():
    """Mirror of src/ntops/torch/utils.py:218-222.

    gfx950 has no reduced-precision (TF32/XF32) fp32 matrix path, so fp32
    GEMMs always run IEEE fp32 whatever this returns."""
    if torch.get_float32_matmul_precision() == "highest":
        return InputPrecisionVariant.IEEE
    return InputPrecisionVariant.TF32


# --------------------------------------------------------------- helpers --


_get_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def _broadcast_shape(a, b):
    """torch.broadcast_shapes(a, b) for two concrete shapes, without its
    symbolic-shape machinery (tens of microseconds of host time per call)."""
    if a == b:
        return a
    n = max(len(a), len(b))
    pa = (1,) * (n - len(a)) + tuple(a)
    pb = (1,) * (n - len(b)) + tuple(b)
    out = []
    for x, y in zip(pa, pb):
        if x != y and x != 1 and y != 1:
            raise RuntimeError(
                f"shape mismatch: objects cannot be broadcast to a single shape.  Mismatch is between "
                f"{tuple(a)} and {tuple(b)}"
            )
        out.append(y if x == 1 else x)
    return torch.Size(out)


class _DeviceGuard:
    """Makes `device` current for the duration of a library call."""

    def __init__(self, device):
        self.device = device
        self.prev = None

    def __enter__(self):
        idx = self.device.index if self.device.index is not None else 0
        cur = _get_device()
        if cur != idx:
            self.prev = cur
            torch.cuda.set_device(idx)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def _strides(t):
    return _lib.i64_array(t.stride())


def _cast_into(src, dst):
    """dst[...] = src converted to dst.dtype (same shape; any strides)."""
    lib = _lib.load()
    rc = lib.ntops_cast(
        _lib.dtype_code(src.dtype),
        _lib.dtype_code(dst.dtype),
        src.dim(),
        _lib.i64_array(src.shape),
        src.data_ptr(),
        _strides(src),
        dst.data_ptr(),
        _strides(dst),
        _lib.stream_of(dst),
    )
    _lib.check(rc, "ntops_amd cast")
    return dst


def _to_dtype(t, dtype):
    """t converted to `dtype` by the native cast kernel (t itself if equal)."""
    if t.dtype == dtype:
        return t
    out = torch.empty(t.shape, dtype=dtype, device=t.device)
    return _cast_into(t, out)


def _expand_to(t, shape):
    """t broadcast to `shape` (t itself when it already has that shape)."""
    return t if t.shape == shape else t.expand(shape)


def _contiguous(t):
    """A row-major copy of t made by the native copy kernel (t if already)."""
    if t.is_contiguous():
        return t
    out = torch.empty(t.shape, dtype=t.dtype, device=t.device)
    return _cast_into(t, out)


def _rows_of(t, nd):
    """(rows tensor, row stride) for a norm over t's last nd dims: t itself
    when those dims are one contiguous run per row, the leading dims walk
    the rows with a single stride, and every row starts at the same offset
    within 16 bytes as the matching row of a row-major output (row views of
    a wider tensor read in place, on the kernels a row-major copy would
    take), else a row-major copy made by the native copy kernel (row
    stride = the row length)."""
    shape, stride = t.shape, t.stride()
    lead = t.dim() - nd
    cols = 1
    for n in shape[lead:]:
        cols *= n
    expect = 1
    for d in range(t.dim() - 1, lead - 1, -1):
        if shape[d] != 1 and stride[d] != expect:
            return _contiguous(t), cols
        expect *= shape[d]
    dims = [d for d in range(lead) if shape[d] != 1]
    if t.data_ptr() % 16:
        return _contiguous(t), cols
    if not dims:
        return t, cols
    for a, b in zip(dims, dims[1:]):
        if stride[a] != stride[b] * shape[b]:
            return _contiguous(t), cols
    rs = stride[dims[-1]]
    if ((rs - cols) * t.element_size()) % 16:
        return _contiguous(t), cols
    return t, rs


def _norm_param(param, input, nd, dtype, per_row=False):
    """A norm's weight or bias as the reference passes it to its kernel,
    `param.expand_as(input)` (src/ntops/torch/rms_norm.py:17-18,
    layer_norm.py:17-25; a shape that does not broadcast raises there too),
    cast to `dtype` by the native kernel and laid out for the C ABI: one
    contiguous row of the normalized elements and row stride 0 when every
    row of the expanded parameter is the same (the usual case, incl.
    broadcasting inside the normalized dims), else a contiguous copy of all
    rows and row stride cols (always so with per_row).  Returns (tensor,
    row_stride); (None, 0) for an empty input."""
    if input.numel() == 0:
        param.expand_as(input)  # raises for a shape that does not broadcast
        return None, 0
    lead = input.dim() - nd
    if (
        not per_row
        and param.dtype == dtype
        and param.shape == input.shape[lead:]
        and param.is_contiguous()
    ):
        return param, 0  # the usual case: one contiguous row of the normalized dims
    pe = param.expand_as(input)
    if not per_row and all(pe.shape[i] == 1 or pe.stride(i) == 0 for i in range(lead)):
        row = pe[(0,) * lead] if lead else pe
        return _contiguous(_to_dtype(row, dtype)), 0
    cols = 1
    for n in input.shape[lead:]:
        cols *= n
    return _contiguous(_to_dtype(pe, dtype)), cols


def _prepare_out(out, shape, dtype, device, like=None):
    """Output tensor for an elementwise result.

    Returns (target, compute): `compute` has the compute dtype and is written
    by the kernel; if it differs from `target` (an `out=` of another dtype),
    the caller casts it into `target` afterwards."""
    shape = torch.Size(shape)
    if out is None:
        if like is not None and like.shape == shape and like.dtype == dtype:
            target = torch.empty_like(like)
        else:
            target = torch.empty(shape, dtype=dtype, device=device)
        return target, target
    _lib.require_cuda(out)
    if out.shape != shape:
        out.resize_(shape)
    if out.dtype == dtype:
        return out, out
    if not torch.can_cast(dtype, out.dtype):
        raise RuntimeError(f"result type {dtype} can't be cast to the desired output type {out.dtype}")
    return out, torch.empty(shape, dtype=dtype, device=device)


def _unary(op, input, output, what):
    lib = _lib.load()
    dev = _lib.require_cuda(input, output)
    with _DeviceGuard(dev):
        rc = lib.ntops_unary(
            op,
            _lib.dtype_code(input.dtype),
            input.dim(),
            _lib.i64_array(input.shape),
            input.data_ptr(),
            _strides(input),
            output.data_ptr(),
            _strides(output),
            _lib.stream_of(output),
        )
    _lib.check(rc, what)
    return output


def _is_number(x):
    return isinstance(x, (bool, int, float))


def _split_other(input, other, what):
    """(other, other_is_tensor, result_dtype) with torch's promotion rules; a
    0-d CPU tensor `other` is treated as a Python number, as torch does."""
    if not isinstance(input, torch.Tensor):
        raise TypeError(f"{what}: input must be a tensor")
    if isinstance(other, torch.Tensor) and other.dim() == 0 and not other.is_cuda:
        return other.item(), False, torch.result_type(input, other)
    if isinstance(other, torch.Tensor):
        return other, True, torch.result_type(input, other)
    if _is_number(other):
        return other, False, torch.result_type(input, other)
    raise TypeError(f"{what}: unsupported operand {type(other)}")


def _scalar_parts(value):
    """A Python number as the (double, int64) pair the C ABI takes."""
    return float(value), (int(value) if not isinstance(value, float) else 0)


def _launch2(entry, op, dtype, shape, a, other, other_is_tensor, res, what, alpha=(1.0, 1)):
    """Calls ntops_binary (entry "binary") or ntops_compare ("compare") on
    `a` (already of `dtype`, broadcast to `shape`) and `other` (a tensor of
    `dtype` broadcast to `shape`, or a Python number)."""
    lib = _lib.load()
    if other_is_tensor:
        b = other if other.shape == shape else other.expand(shape)
        b_ptr, b_strides, b_f, b_i = b.data_ptr(), _strides(b), 0.0, 0
    else:
        b_ptr, b_strides = None, None
        b_f, b_i = _scalar_parts(other)
    head = (op, _lib.dtype_code(dtype), len(shape), _lib.i64_array(shape), a.data_ptr(), _strides(a),
            b_ptr, b_strides, b_f, b_i)
    tail = (res.data_ptr(), _strides(res), _lib.stream_of(res))
    if entry == "binary":
        rc = lib.ntops_binary(*head, alpha[0], alpha[1], *tail)
    else:
        rc = lib.ntops_compare(*head, *tail)
    _lib.check(rc, what)


# ops and operand dtypes of ntops_binary_cvt (mixed dtypes, fp32 result)
_CVT_OPS = (_lib.BINARY_ADD, _lib.BINARY_SUB, _lib.BINARY_MUL, _lib.BINARY_DIV)
_CVT_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.int32)


def _binary(op, input, other, alpha, out, what, compute_dtype=None):
    """Shared body of the binary arithmetic ops (add, sub, mul, div, pow,
    bitwise_and / or) with torch's promotion (torch.result_type) and
    broadcasting rules.  `compute_dtype` maps the promoted dtype to the one
    the kernel runs in (true division promotes integers to float)."""
    other, other_is_tensor, result_dtype = _split_other(input, other, what)
    if compute_dtype is not None:
        result_dtype = compute_dtype(result_dtype)
    dev = _lib.require_cuda(input, other if other_is_tensor else None)
    shape = _broadcast_shape(input.shape, other.shape) if other_is_tensor else input.shape
    target, res = _prepare_out(out, shape, result_dtype, dev, like=input)

    is_float = result_dtype.is_floating_point
    if alpha is None:
        alpha_f, alpha_i = 1.0, 1
    else:
        if not is_float and isinstance(alpha, float):
            raise RuntimeError(
                "For integral input tensors, argument alpha must not be a floating point number."
            )
        if result_dtype == torch.bool and not isinstance(alpha, bool):
            raise RuntimeError("Boolean alpha only supported for Boolean results.")
        alpha_f, alpha_i = _scalar_parts(alpha)

    with _DeviceGuard(dev):
        if (
            other_is_tensor
            and result_dtype == torch.float32
            and op in _CVT_OPS
            and (input.dtype != result_dtype or other.dtype != result_dtype)
            and input.dtype in _CVT_DTYPES
            and other.dtype in _CVT_DTYPES
            and input.shape == shape
            and other.shape == shape
            and input.is_contiguous()
            and other.is_contiguous()
            and res.is_contiguous()
            and input.data_ptr() % 16 == 0
            and other.data_ptr() % 16 == 0
            and res.data_ptr() % 16 == 0
        ):
            # mixed operand dtypes promoted to fp32: the conversion fused into
            # the elementwise pass instead of a cast kernel per operand
            rc = _lib.load().ntops_binary_cvt(
                op, _lib.dtype_code(input.dtype), _lib.dtype_code(other.dtype), _lib.F32, res.numel(),
                input.data_ptr(), other.data_ptr(), alpha_f, res.data_ptr(), _lib.stream_of(res))
            _lib.check(rc, what)
        else:
            a = _expand_to(_to_dtype(input, result_dtype), shape)
            b = _to_dtype(other, result_dtype) if other_is_tensor else other
            _launch2("binary", op, result_dtype, shape, a, b, other_is_tensor, res, what, (alpha_f, alpha_i))
        if res is not target:
            _cast_into(res, target)
    return target


def _compare(op, input, other, out, what):
    """eq / ne / gt / ge / lt / le: compares in the promoted dtype and returns
    bool, like torch (the reference writes into a tensor of input's dtype)."""
    other, other_is_tensor, common = _split_other(input, other, what)
    dev = _lib.require_cuda(input, other if other_is_tensor else None)
    shape = _broadcast_shape(input.shape, other.shape) if other_is_tensor else input.shape
    target, res = _prepare_out(out, shape, torch.bool, dev)
    a = _expand_to(_to_dtype(input, common), shape)
    with _DeviceGuard(dev):
        b = _to_dtype(other, common) if other_is_tensor else other
        _launch2("compare", op, common, shape, a, b, other_is_tensor, res, what)
        if res is not target:
            _cast_into(res, target)
    return target


def _float_unary(op, input, out, what):
    """Unary floating op (sigmoid, tanh, rsqrt, sin, cos, exp): integer and
    bool inputs are promoted to the default floating dtype first, as torch
    does."""
    dev = _lib.require_cuda(input)
    dtype = input.dtype if input.dtype.is_floating_point else torch.get_default_dtype()
    x = _to_dtype(input, dtype)
    target, res = _prepare_out(out, input.shape, dtype, dev, like=x)
    _unary(op, x, res, what)
    if res is not target:
        _cast_into(res, target)
    return target
