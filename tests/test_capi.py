"""C ABI checks that need no GPU: the library loads, exports every symbol
include/ntops_amd.h declares, and rejects invalid calls with a status code and
a message before any HIP call is made.  The torch wrappers refuse CPU tensors
(there is no CPU fallback anywhere on the product path)."""

import ctypes
import os
import re

import pytest
import torch

import ntops_amd
from ntops_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ntops_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"NTOPS_API\s+[\w\s\*]+?\b(ntops_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "ntops_gemm" in names and "ntops_rope" in names and len(names) >= 10


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), f"{name} is declared in ntops_amd.h but not exported"
    # the ctypes binding covers the same set
    assert sorted(_lib.EXPORTED) == declared_symbols()


def test_abi_version():
    assert _lib.load().ntops_abi_version() == 2


def _err(lib):
    return lib.ntops_last_error().decode()


def _arr(*v):
    return _lib.i64_array(v)


def test_unary_rejects_bad_arguments():
    lib = _lib.load()
    shape = _arr(4)
    st = _arr(1)
    rc = lib.ntops_unary(_lib.UNARY_SILU, _lib.F32, 1, shape, None, st, ctypes.c_void_p(16), st, None)
    assert rc == 1 and "null input" in _err(lib)
    rc = lib.ntops_unary(99, _lib.F32, 1, shape, ctypes.c_void_p(16), st, ctypes.c_void_p(16), st, None)
    assert rc == 2 and "unknown op" in _err(lib)
    rc = lib.ntops_unary(_lib.UNARY_SILU, _lib.I32, 1, shape, ctypes.c_void_p(16), st, ctypes.c_void_p(16), st, None)
    assert rc == 2 and "unsupported" in _err(lib)
    rc = lib.ntops_unary(_lib.UNARY_BITWISE_NOT, _lib.F32, 1, shape, ctypes.c_void_p(16), st, ctypes.c_void_p(16), st, None)
    assert rc == 2
    rc = lib.ntops_unary(_lib.UNARY_SILU, _lib.F32, -1, shape, ctypes.c_void_p(16), st, ctypes.c_void_p(16), st, None)
    assert rc == 1 and "ndim" in _err(lib)


def test_empty_tensors_launch_nothing():
    lib = _lib.load()
    shape = _arr(0, 5)
    st = _arr(5, 1)
    # numel == 0 returns before any HIP call, so this is safe without a GPU
    assert lib.ntops_unary(_lib.UNARY_EXP, _lib.F32, 2, shape, ctypes.c_void_p(16), st, ctypes.c_void_p(16), st, None) == 0
    assert lib.ntops_rms_norm(_lib.BF16, 0, 4096, None, 4096, None, 0, _lib.BF16, 1e-6, None, 4096, None) == 0
    assert lib.ntops_softmax(_lib.F32, _lib.F32, 0, 3, 1, None, st, None, st, None) == 0
    assert lib.ntops_gemm(_lib.BF16, 1, 0, 4, 4, None, _arr(0, 4, 1), None, _arr(0, 4, 1), None, None, 1.0, 0.0, None, _arr(0, 4, 1), None) == 0


def test_more_than_max_dims_rejected():
    lib = _lib.load()
    nd = 10
    shape = _arr(*([2] * nd))
    # strides that cannot merge: every dim strided by a non-multiple
    xs = _arr(*[3 ** (nd - i) for i in range(nd)])
    ys = _arr(*[2 ** (nd - 1 - i) for i in range(nd)])
    rc = lib.ntops_unary(_lib.UNARY_EXP, _lib.F32, nd, shape, ctypes.c_void_p(16), xs, ctypes.c_void_p(16), ys, None)
    assert rc == 1 and "non-mergeable" in _err(lib)


def test_rows_and_rope_and_gemm_validation():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    assert lib.ntops_rms_norm(_lib.BF16, -1, 8, p, 8, None, 0, _lib.BF16, 1e-6, p, 8, None) == 1
    assert lib.ntops_rms_norm(_lib.BF16, 2, 8, p, 8, p, 0, _lib.F16, 1e-6, p, 8, None) == 2
    assert "weight dtype" in _err(lib)
    assert lib.ntops_layer_norm(_lib.F64, 2, 8, p, 8, None, None, 0, _lib.F64, 1e-5, p, 8, None) == 2
    st4 = _arr(8, 8, 8, 1)
    assert lib.ntops_rope(_lib.BF16, 1, 1, 1, 7, p, st4, p, p, 7, 7, 0, p, st4, None) == 1
    assert "even" in _err(lib)
    assert lib.ntops_rope(_lib.BF16, 1, 1, 1, 8, p, st4, p, p, 8, 3, 0, p, st4, None) == 1
    assert lib.ntops_rope(_lib.BF16, 1, 1, 1, 2048, p, st4, p, p, 1024, 1024, 0, p, st4, None) == 2
    s3 = _arr(0, 8, 1)
    assert lib.ntops_gemm(_lib.BF16, 1, -1, 8, 8, p, s3, p, s3, None, None, 1.0, 0.0, p, s3, None) == 1
    assert lib.ntops_gemm(_lib.I32, 1, 8, 8, 8, p, s3, p, s3, None, None, 1.0, 0.0, p, s3, None) == 2
    assert lib.ntops_gemm(_lib.BF16, 1, 8, 8, 8, None, s3, p, s3, None, None, 1.0, 0.0, p, s3, None) == 1
    assert lib.ntops_softmax(_lib.I32, _lib.F32, 1, 3, 1, p, _arr(3, 1, 1), p, _arr(3, 1, 1), None) == 2


def test_wrappers_refuse_cpu_tensors():
    x = torch.randn(8, 8)
    for fn, args in [
        (ntops_amd.torch.silu, (x,)),
        (ntops_amd.torch.exp, (x,)),
        (ntops_amd.torch.add, (x, x)),
        (ntops_amd.torch.rms_norm, (x, (8,))),
        (ntops_amd.torch.layer_norm, (x, (8,))),
        (ntops_amd.torch.softmax, (x, -1)),
        (ntops_amd.torch.mm, (x, x)),
    ]:
        with pytest.raises(RuntimeError, match="GPU tensor"):
            fn(*args)


def test_wrapper_type_errors_match_torch():
    x = torch.randn(4)
    with pytest.raises(RuntimeError):
        ntops_amd.torch.bitwise_and(x, x)
    with pytest.raises(RuntimeError):
        ntops_amd.torch.bitwise_not(x)
    with pytest.raises(RuntimeError):
        ntops_amd.torch.gelu(x, approximate="cubic")


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libntops_amd.so")
    with pytest.raises(RuntimeError, match="missing"):
        _lib.load()


def test_knobs_are_kept():
    from ntops_amd.torch import utils

    utils.set_default_num_warps(4)
    utils.set_default_num_stages(2)
    assert utils.get_default_num_warps() == 4 and utils.get_default_num_stages() == 2
    from ntops_amd.kernels.mm import InputPrecisionVariant

    torch.set_float32_matmul_precision("highest")
    assert utils._get_matmul_input_precision() == InputPrecisionVariant.IEEE
    torch.set_float32_matmul_precision("high")
    assert utils._get_matmul_input_precision() == InputPrecisionVariant.TF32
    torch.set_float32_matmul_precision("highest")
