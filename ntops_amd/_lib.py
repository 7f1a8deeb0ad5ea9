"""ctypes binding of libntops_amd.so (the C ABI declared in include/ntops_amd.h).

This module replaces the reference's kernel factory (`_cached_make`,
src/ntops/torch/utils.py:46-64) and the NineToothed/Triton launch below it:
every op is a direct call into the prebuilt gfx950 library, launched
asynchronously on torch's current HIP stream.  There is no fallback: if the
library is missing or a call fails, a RuntimeError is raised.
"""

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libntops_amd.so")

# enum ntops_dtype
F32, F16, BF16, F64, BOOL, U8, I8, I16, I32, I64 = range(10)

DTYPE_CODE = {
    torch.float32: F32,
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.float64: F64,
    torch.bool: BOOL,
    torch.uint8: U8,
    torch.int8: I8,
    torch.int16: I16,
    torch.int32: I32,
    torch.int64: I64,
}

# enum ntops_unary_op / ntops_binary_op / ntops_compare_op / ntops_classify_op
UNARY_SILU, UNARY_GELU, UNARY_GELU_TANH, UNARY_EXP, UNARY_BITWISE_NOT = 1, 2, 3, 4, 5
UNARY_RELU, UNARY_SIGMOID, UNARY_TANH, UNARY_NEG, UNARY_ABS, UNARY_RSQRT, UNARY_SIN, UNARY_COS = range(6, 14)
BINARY_ADD, BINARY_MUL, BINARY_BITWISE_AND, BINARY_BITWISE_OR = 1, 2, 3, 4
BINARY_SUB, BINARY_DIV, BINARY_DIV_TRUNC, BINARY_DIV_FLOOR, BINARY_POW = 5, 6, 7, 8, 9
CMP_EQ, CMP_NE, CMP_GT, CMP_GE, CMP_LT, CMP_LE = 1, 2, 3, 4, 5, 6
CLASSIFY_ISINF, CLASSIFY_ISNAN = 1, 2

_c_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_d = ctypes.c_double

_SIGNATURES = {
    "ntops_abi_version": (_i, []),
    "ntops_last_error": (ctypes.c_char_p, []),
    "ntops_last_kernel": (ctypes.c_char_p, []),
    "ntops_unary": (_i, [_i, _i, _i, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp]),
    "ntops_binary": (
        _i,
        [_i, _i, _i, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _d, _i64, _d, _i64, _vp, _c_i64p, _vp],
    ),
    "ntops_binary_cvt": (_i, [_i, _i, _i, _i, _i64, _vp, _vp, _d, _vp, _vp]),
    "ntops_compare": (
        _i,
        [_i, _i, _i, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _d, _i64, _vp, _c_i64p, _vp],
    ),
    "ntops_classify": (_i, [_i, _i, _i, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp]),
    "ntops_clamp": (
        _i,
        [_i, _i, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _d, _i64, _i, _vp, _c_i64p, _d, _i64, _i,
         _vp, _c_i64p, _vp],
    ),
    "ntops_cast": (_i, [_i, _i, _i, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp]),
    "ntops_rms_norm": (_i, [_i, _i64, _i64, _vp, _i64, _vp, _i64, _i, _d, _vp, _i64, _vp]),
    "ntops_layer_norm": (_i, [_i, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _i, _d, _vp, _i64, _vp]),
    "ntops_softmax": (_i, [_i, _i, _i64, _i64, _i64, _vp, _c_i64p, _vp, _c_i64p, _vp]),
    "ntops_rope": (
        _i,
        [_i, _i64, _i64, _i64, _i64, _vp, _c_i64p, _vp, _vp, _i64, _i64, _i, _vp, _c_i64p, _vp],
    ),
    "ntops_sdpa": (
        _i,
        [_i, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _i, _c_i64p,
         _i, _d, _vp, _c_i64p, _vp],
    ),
    "ntops_add_rms_norm": (
        _i,
        [_i, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i, _d, _vp, _i64, _vp, _i64, _vp],
    ),
    "ntops_rope_qk": (
        _i,
        [_i, _i64, _i64, _i64, _i64, _i64, _vp, _c_i64p, _vp, _c_i64p, _vp, _vp, _i64, _i64, _i, _vp, _c_i64p,
         _vp, _c_i64p, _vp],
    ),
    "ntops_conv2d_workspace": (
        _i64,
        [_i] + [_i64] * 15 + [_c_i64p, _c_i64p],
    ),
    "ntops_conv2d": (
        _i,
        [_i] + [_i64] * 15 + [_vp, _c_i64p, _vp, _c_i64p, _vp, _i64, _vp, _c_i64p, _vp, _i64, _vp],
    ),
    "ntops_conv2d_noalloc": (
        _i,
        [_i] + [_i64] * 15 + [_vp, _c_i64p, _vp, _c_i64p, _vp, _i64, _vp, _c_i64p, _vp],
    ),
    "ntops_im2col": (
        _i,
        [_i] + [_i64] * 12 + [_vp, _c_i64p, _vp, _c_i64p, _vp],
    ),
    "ntops_mfma_rate_probe": (_i, [_i64, _i64, _vp, _vp]),
    "ntops_gemm": (
        _i,
        [_i, _i64, _i64, _i64, _i64, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _d, _d, _vp, _c_i64p, _vp],
    ),
    "ntops_gemm_ws": (
        _i,
        [_i, _i64, _i64, _i64, _i64, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _d, _d, _vp, _c_i64p, _vp, _i64,
         _vp],
    ),
    "ntops_gemm_workspace": (_i64, [_i, _i64, _i64, _i64, _i64]),
}

EXPORTED = tuple(_SIGNATURES)

_lib = None


def load():
    """Loads (once) and returns the CDLL; raises if the library is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"ntops_amd: native library {LIB_PATH} is missing; build it with "
                "`make -C ntops_amd/csrc` (or __graft_entry__.build())"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def i64_array(values):
    """The sizes or strides `values` (Python ints) as an int64_t[] argument."""
    return (ctypes.c_int64 * (len(values) or 1))(*values)


def dtype_code(dtype):
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"ntops_amd: unsupported dtype {dtype}") from None


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(tensor):
    """torch's current HIP stream on tensor's device (the raw handle; torch's
    Stream object costs microseconds of host time per call to build)."""
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(tensor.device.index))
    return ctypes.c_void_p(torch.cuda.current_stream(tensor.device).cuda_stream)


def last_kernel():
    """Name of the kernel this thread's most recent GEMM-family call launched."""
    return load().ntops_last_kernel().decode()


def check(rc, what):
    if rc != 0:
        msg = load().ntops_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg} (status {rc})")


def require_cuda(*tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                f"ntops_amd: expected a GPU tensor, got a tensor on {t.device}"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"ntops_amd: tensors on different devices ({dev} and {t.device})")
    return dev
