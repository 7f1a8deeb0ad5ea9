"""CPU checks of the torch wrappers' host-side helpers that replace torch
utilities on the launch path (they run on every call, so they avoid
torch's slower general forms): two-shape broadcasting and the int64 array
argument of the C ABI."""

import ctypes

import pytest
import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _broadcast_shape, _expand_to


@pytest.mark.parametrize(
    "a, b",
    [
        ((16, 64), (16, 64)),
        ((16, 64), (64,)),
        ((64,), (16, 64)),
        ((4, 1, 8), (3, 1)),
        ((1,), (2, 3, 4)),
        ((), (5, 6)),
        ((5, 6), ()),
        ((0, 3), (1, 3)),
        ((2, 1, 0), (7, 1)),
        ((1, 1), (1,)),
    ],
)
def test_broadcast_shape_matches_torch(a, b):
    got = _broadcast_shape(torch.Size(a), torch.Size(b))
    assert isinstance(got, torch.Size)
    assert got == torch.broadcast_shapes(a, b)


@pytest.mark.parametrize("a, b", [((16, 64), (16, 63)), ((3,), (4,)), ((2, 3), (3, 2)), ((0,), (2,))])
def test_broadcast_shape_rejects_like_torch(a, b):
    with pytest.raises(RuntimeError):
        torch.broadcast_shapes(a, b)
    with pytest.raises(RuntimeError, match="cannot be broadcast"):
        _broadcast_shape(torch.Size(a), torch.Size(b))


def test_expand_to_keeps_equal_shapes_and_broadcasts_others():
    t = torch.arange(6.0).reshape(2, 3)
    assert _expand_to(t, torch.Size((2, 3))) is t
    e = _expand_to(torch.arange(3.0), torch.Size((2, 3)))
    assert e.shape == (2, 3) and e.stride() == (0, 1)
    assert torch.equal(e, torch.arange(3.0).expand(2, 3))


def test_i64_array_holds_the_values():
    for values in ((), (7,), torch.Size([4, 4096]), (-3, 2**40, 0)):
        arr = _lib.i64_array(values)
        assert isinstance(arr, ctypes.Array)
        assert list(arr)[: len(values)] == list(values)
        assert len(arr) == max(len(values), 1)


_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.float64, torch.int32, torch.int64, torch.uint8,
           torch.bool)


def _bounds():
    yield None
    yield 2
    yield -1.5
    yield True
    for dt in (torch.float32, torch.bfloat16, torch.int64, torch.int16):
        yield torch.ones((), dtype=dt)  # zero-dim tensor
        yield torch.ones(3, dtype=dt)  # broadcasts along the last dim
        yield torch.ones(2, 1, dtype=dt)  # broadcasts along the first dim


@pytest.mark.parametrize("dtype", _DTYPES)
def test_clamp_result_matches_torch(dtype):
    """The wrappers' clamp result dtype / shape (and the combinations torch
    refuses) against torch.clamp evaluated on CPU tensors of the same
    shapes."""
    from ntops_amd.torch.clamp import _result

    x = torch.zeros(2, 3, dtype=dtype)
    for lo in _bounds():
        for hi in _bounds():
            if lo is None and hi is None:
                continue
            try:
                ref = torch.clamp(x, lo, hi)
            except (RuntimeError, TypeError):
                with pytest.raises((RuntimeError, TypeError)):
                    _result(x, lo, hi)
                continue
            assert _result(x, lo, hi) == (ref.dtype, ref.shape), (dtype, lo, hi)


def test_rows_of_reads_row_views_in_place():
    """Norm inputs: row views whose rows start 16-byte aligned like a
    row-major output's are passed with their row stride; other layouts are
    copied row-major (here on the CPU the copy is torch's, the rule is the
    same)."""
    import ntops_amd.torch.utils as U

    copied = []
    real = U._contiguous
    U._contiguous = lambda t: copied.append(t.shape) or t.contiguous()
    try:
        base = torch.zeros(64, 1024, dtype=torch.bfloat16)
        t, rs = U._rows_of(base[:, :512], 1)
        assert rs == 1024 and t.data_ptr() == base.data_ptr() and not copied
        t, rs = U._rows_of(base.view(8, 8, 1024)[:, :, 128:640], 1)  # leading dims merge
        assert rs == 1024 and not copied
        t, rs = U._rows_of(base.view(8, 8, 1024)[:, :4, :], 1)  # leading dims do not merge
        assert rs == 1024 and copied and t.is_contiguous()
        copied.clear()
        t, rs = U._rows_of(base[:, 1:513], 1)  # rows at a 2-byte offset
        assert rs == 512 and copied
        copied.clear()
        t, rs = U._rows_of(base[:, :100], 1)  # (1024 - 100) * 2 bytes is not a multiple of 16
        assert rs == 100 and copied
        copied.clear()
        t, rs = U._rows_of(base.view(64, 16, 64)[:, :, :], 2)  # two normalized dims, contiguous
        assert rs == 1024 and not copied
        t, rs = U._rows_of(base.view(64, 16, 64).transpose(1, 2), 2)  # normalized dims not one run
        assert rs == 1024 and copied
    finally:
        U._contiguous = real
