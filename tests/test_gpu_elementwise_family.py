"""GPU parity: the rest of the elementwise family (relu, sigmoid, tanh, neg,
abs, rsqrt, sin, cos, sub, div, pow, eq/ne/gt/ge/lt/le, isinf, isnan, clamp)
through the C ABI, against the oracle.

Mirrors the reference's tests (tests/test_<op>.py: random shapes of 256-1024
elements over 1-4 dims, fp32 and fp16, gauss alpha for sub, None / floor
rounding for div, tensor min / max for clamp, inf / NaN injection for isinf /
isnan) with bf16 and the integer dtypes added, special values, Python-number
operands, type promotion, broadcasting, non-contiguous inputs and `out=`.
Exact operations (relu, neg, abs, rsqrt, sub, div, the special pow exponents,
comparisons, classification, clamp) are compared bit for bit (NaN = NaN, and
the sign of zero must match); the library transcendentals (sigmoid, tanh,
sin, cos, general pow) within the elementwise tolerance (fp32 1e-6; 16-bit
types 1.6e-2)."""

import random

import numpy as np
import pytest
import torch

import ntops_amd
from oracle import ops as O
from tests.helpers import DT_NAME, TOL_ELEMENTWISE, assert_close, from_np, random_shape, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

FLOATS = (torch.float32, torch.float16, torch.bfloat16)
INTS = (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8)
T = ntops_amd.torch


def cases(dtypes=FLOATS):
    return [(random_shape(ndim), dt) for ndim in range(1, 5) for dt in dtypes]


def same(got, exp, what=""):
    """Bit-level equality of two CPU/GPU tensors: NaN == NaN, signed zeros must
    match."""
    g, e = got.detach().cpu(), exp.detach().cpu()
    assert g.dtype == e.dtype, f"{what}: dtype {g.dtype} != {e.dtype}"
    assert g.shape == e.shape, f"{what}: shape {tuple(g.shape)} != {tuple(e.shape)}"
    if g.dtype.is_floating_point:
        gd, ed = g.double(), e.double()
        nan = torch.isnan(gd) & torch.isnan(ed)
        bad = ((gd != ed) | (torch.signbit(gd) != torch.signbit(ed))) & ~nan
    else:
        bad = g != e
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.numel()} elements differ"


def with_specials(x):
    flat = x.reshape(-1)
    sp = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), float("nan"), 1e-30, 1.0, -1.0])
    k = min(len(sp), flat.numel())
    flat[:k] = sp[:k].to(x.dtype)
    return x


def ora(fn, *arrs, dt):
    return from_np(fn(*arrs, dt), dt)


# ---------------------------------------------------------------- unary ---


EXACT_UNARY = {"relu": O.relu, "neg": O.neg, "abs": O.abs, "rsqrt": O.rsqrt}
APPROX_UNARY = {"sigmoid": O.sigmoid, "tanh": O.tanh, "sin": O.sin, "cos": O.cos}


@pytest.mark.parametrize("op", sorted(EXACT_UNARY) + sorted(APPROX_UNARY))
@pytest.mark.parametrize("shape, dtype", cases())
def test_unary_float(op, shape, dtype):
    x = with_specials(torch.randn(shape).mul(3).to(dtype))
    dt = DT_NAME[dtype]
    got = getattr(T, op)(x.cuda())
    if op in EXACT_UNARY:
        same(got, ora(EXACT_UNARY[op], to_np(x), dt=dt), op)
    else:
        assert_close(got, ora(APPROX_UNARY[op], to_np(x), dt=dt), *TOL_ELEMENTWISE[dt], op)


@pytest.mark.parametrize("op", ("relu", "neg", "abs"))
@pytest.mark.parametrize("dtype", INTS)
def test_unary_integer(op, dtype):
    info = torch.iinfo(dtype)
    x = torch.randint(max(info.min, -1000), min(info.max, 1000) + 1, (777,), dtype=dtype)
    x[0], x[1] = info.min, info.max
    got = getattr(T, op)(x.cuda())
    same(got, ora(getattr(O, op), x.numpy(), dt=DT_NAME[dtype]), f"{op} {dtype}")
    same(got, getattr(torch, op)(x), f"{op} {dtype} vs torch")


@pytest.mark.parametrize("op", ("sigmoid", "tanh", "rsqrt", "sin", "cos"))
def test_unary_promotes_integers(op):
    x = torch.randint(1, 50, (300,), dtype=torch.int32)
    got = getattr(T, op)(x.cuda())
    assert got.dtype == torch.float32
    exp = getattr(O, op)(x.numpy().astype(np.float32), "f32")
    assert_close(got, torch.from_numpy(exp), *TOL_ELEMENTWISE["f32"], op)


def test_relu_inplace_noncontiguous_and_out():
    x = torch.randn(64, 48)
    xg = x.cuda().t()  # non-contiguous
    same(T.relu(xg), ora(O.relu, to_np(x.t()), dt="f32"), "relu non-contiguous")
    y = x.clone().cuda()
    r = T.relu(y, inplace=True)
    assert r.data_ptr() == y.data_ptr()
    same(y, ora(O.relu, to_np(x), dt="f32"), "relu inplace")
    out = torch.empty(64, 48, dtype=torch.float64, device="cuda")
    T.sin(x.cuda(), out=out)
    assert_close(out, torch.sin(x.double()), 1e-6, 1e-6, "sin out=f64")


def test_bool_inputs_raise():
    b = torch.tensor([True, False]).cuda()
    for op in ("relu", "neg", "abs"):
        with pytest.raises((RuntimeError, NotImplementedError)):
            getattr(T, op)(b)
    with pytest.raises(RuntimeError):
        T.sub(b, b)
    with pytest.raises((RuntimeError, NotImplementedError)):
        T.div(b, b, rounding_mode="floor")
    with pytest.raises((RuntimeError, NotImplementedError)):
        T.pow(b, b)


# --------------------------------------------------------------- binary ---


@pytest.mark.parametrize("shape, dtype", cases())
def test_sub(shape, dtype):
    x, y = torch.randn(shape).to(dtype), torch.randn(shape).to(dtype)
    alpha = random.gauss(0, 1)
    dt = DT_NAME[dtype]
    same(T.sub(x.cuda(), y.cuda(), alpha=alpha), ora(lambda a, b, d: O.sub(a, b, d, alpha), to_np(x), to_np(y), dt=dt), "sub")
    same(T.sub(x.cuda(), 0.37, alpha=1.5), ora(lambda a, d: O.sub(a, 0.37, d, 1.5), to_np(x), dt=dt), "sub scalar")
    rtol, atol = TOL_ELEMENTWISE[dt]
    assert_close(T.sub(x.cuda(), y.cuda(), alpha=alpha), torch.sub(x, y, alpha=alpha), rtol, atol, "sub vs torch")


@pytest.mark.parametrize("rounding_mode", (None, "trunc", "floor"))
@pytest.mark.parametrize("shape, dtype", cases())
def test_div(shape, dtype, rounding_mode):
    x = with_specials(torch.randn(shape).mul(4).to(dtype))
    y = torch.randn(shape).to(dtype)
    y.reshape(-1)[8:12] = torch.tensor([0.0, -0.0, float("inf"), float("-inf")]).to(dtype)
    dt = DT_NAME[dtype]
    got = T.div(x.cuda(), y.cuda(), rounding_mode=rounding_mode)
    same(got, ora(lambda a, b, d: O.div(a, b, d, rounding_mode), to_np(x), to_np(y), dt=dt), f"div {rounding_mode}")
    got = T.div(x.cuda(), 1.1, rounding_mode=rounding_mode)
    same(got, ora(lambda a, d: O.div(a, 1.1, d, rounding_mode), to_np(x), dt=dt), f"div {rounding_mode} scalar")


@pytest.mark.parametrize("rounding_mode", ("trunc", "floor"))
@pytest.mark.parametrize("dtype", INTS)
def test_div_integer(dtype, rounding_mode):
    info = torch.iinfo(dtype)
    lo = max(info.min, -1000)
    a = torch.randint(lo, min(info.max, 1000) + 1, (999,), dtype=dtype)
    b = torch.randint(max(info.min, -13), 14, (999,), dtype=dtype)
    b[b == 0] = 5
    got = T.div(a.cuda(), b.cuda(), rounding_mode=rounding_mode)
    same(got, torch.div(a, b, rounding_mode=rounding_mode), f"div {rounding_mode} {dtype} vs torch")
    same(got, ora(lambda x, y, d: O.div(x, y, d, rounding_mode), a.numpy(), b.numpy(), dt=DT_NAME[dtype]), "oracle")
    # division by zero: 0 (torch's CPU kernel raises)
    z = T.div(a[:8].cuda(), torch.zeros(8, dtype=dtype).cuda(), rounding_mode=rounding_mode)
    assert (z.cpu() == 0).all()


def test_div_true_promotes_integers():
    a = torch.randint(-50, 50, (500,), dtype=torch.int32)
    b = torch.randint(1, 9, (500,), dtype=torch.int32)
    got = T.div(a.cuda(), b.cuda())
    assert got.dtype == torch.float32
    same(got, torch.div(a, b), "int true division")


POW_SCALARS = (2, 3, 0.5, -0.5, -1, -2, 1.7, 0)


@pytest.mark.parametrize("shape, dtype", cases())
def test_pow(shape, dtype):
    x = with_specials(torch.randn(shape).mul(2).to(dtype))
    e = torch.randn(shape).to(dtype)
    dt = DT_NAME[dtype]
    rtol, atol = TOL_ELEMENTWISE[dt]
    assert_close(T.pow(x.cuda(), e.cuda()), ora(O.pow, to_np(x), to_np(e), dt=dt), rtol, atol, "pow tensor")
    for s in POW_SCALARS:
        got = T.pow(x.cuda(), s)
        exp = ora(lambda a, d: O.pow(a, s, d), to_np(x), dt=dt)
        if s in (2, 3, -1, -2, -0.5, 0.5) and dtype != torch.float16:
            same(got, exp, f"pow {s}")
        else:
            assert_close(got, exp, rtol, atol, f"pow {s}")


@pytest.mark.parametrize("dtype", (torch.int8, torch.int16, torch.int32, torch.int64))
def test_pow_integer(dtype):
    b = torch.randint(-6, 7, (600,), dtype=dtype)
    e = torch.randint(-3, 9, (600,), dtype=dtype)
    got = T.pow(b.cuda(), e.cuda())
    same(got, torch.pow(b, e), "int pow vs torch")
    same(T.pow(b.cuda(), 3), torch.pow(b, 3), "int pow scalar")
    with pytest.raises(RuntimeError):
        T.pow(b.cuda(), -1)


def test_pow_number_base():
    e = torch.randn(300)
    assert_close(T.pow(2.0, e.cuda()), torch.pow(2.0, e), 1e-6, 1e-6, "2 ** tensor")


# ----------------------------------------------------------- comparisons --


CMPS = ("eq", "ne", "gt", "ge", "lt", "le")


@pytest.mark.parametrize("op", CMPS)
@pytest.mark.parametrize("shape, dtype", cases(FLOATS + (torch.int32, torch.int8)))
def test_compare(op, shape, dtype):
    if dtype.is_floating_point:
        x, y = with_specials(torch.randn(shape).to(dtype)), torch.randn(shape).to(dtype)
    else:
        x, y = torch.randint(-5, 6, shape, dtype=dtype), torch.randint(-5, 6, shape, dtype=dtype)
    n = x.numel()
    y.reshape(-1)[n // 2:] = x.reshape(-1)[n // 2:]  # equal pairs
    got = getattr(T, op)(x.cuda(), y.cuda())
    assert got.dtype == torch.bool
    same(got, getattr(torch, op)(x, y), f"{op} vs torch")
    same(got, torch.from_numpy(O.compare(op, to_np(x), to_np(y), DT_NAME[dtype])), f"{op} oracle")
    same(getattr(T, op)(x.cuda(), 1.001), getattr(torch, op)(x, 1.001), f"{op} scalar vs torch")


def test_compare_promotion_and_broadcast():
    a = torch.randint(-3, 4, (7, 1, 5), dtype=torch.int32)
    b = torch.randn(6, 5)
    for op in CMPS:
        same(getattr(T, op)(a.cuda(), b.cuda()), getattr(torch, op)(a, b), f"{op} int32 vs f32 broadcast")
        same(getattr(T, op)(a.cuda(), 0.5), getattr(torch, op)(a, 0.5), f"{op} int vs float scalar")
    x = torch.tensor([1.0, 1.001, 1.01]).bfloat16()
    same(T.eq(x.cuda(), 1.001), torch.eq(x, 1.001), "bf16 eq rounds the scalar")
    out = torch.empty(3, dtype=torch.float32, device="cuda")
    T.gt(x.cuda(), 1.0, out=out)
    same(out, torch.gt(x, 1.0).float(), "gt out=f32")


# ------------------------------------------------------- isinf / isnan ----


@pytest.mark.parametrize("shape, dtype", cases())
def test_isinf_isnan(shape, dtype):
    x = torch.randn(shape)
    p = torch.rand(shape)
    x[(0.2 < p) & (p < 0.4)] = float("inf")
    x[(0.4 < p) & (p < 0.6)] = float("-inf")
    x[p > 0.8] = float("nan")
    x = x.to(dtype)
    same(T.isinf(x.cuda()), torch.isinf(x), "isinf")
    same(T.isnan(x.cuda()), torch.isnan(x), "isnan")
    i = torch.arange(10, dtype=torch.int32).cuda()
    assert not T.isinf(i).any() and not T.isnan(i).any()


# ---------------------------------------------------------------- clamp ---


@pytest.mark.parametrize("shape, dtype", cases())
def test_clamp(shape, dtype):
    x = with_specials(torch.randn(shape).to(dtype))
    lo, hi = torch.randn(shape).to(dtype), torch.randn(shape).to(dtype)
    lo.reshape(-1)[-1], hi.reshape(-1)[-2] = float("nan"), float("nan")
    dt = DT_NAME[dtype]
    same(T.clamp(x.cuda(), lo.cuda(), hi.cuda()), ora(O.clamp, to_np(x), to_np(lo), to_np(hi), dt=dt), "clamp")
    same(T.clamp(x.cuda(), lo.cuda(), hi.cuda()), torch.clamp(x, lo, hi), "clamp vs torch")
    same(T.clamp(x.cuda(), min=lo.cuda()), torch.clamp(x, min=lo), "clamp min tensor")
    same(T.clamp(x.cuda(), max=hi.cuda()), torch.clamp(x, max=hi), "clamp max tensor")
    same(T.clamp(x.cuda(), -0.11, 0.5003), torch.clamp(x, -0.11, 0.5003), "clamp scalars")
    same(T.clamp(x.cuda(), max=0.3), torch.clamp(x, max=0.3), "clamp max scalar")
    same(T.clamp(x.cuda(), 0.7, 0.2), torch.clamp(x, 0.7, 0.2), "clamp lo > hi")


def test_clamp_integer_broadcast_promotion():
    x = torch.randint(-50, 50, (4, 33), dtype=torch.int16)
    lo = torch.randint(-20, 0, (33,), dtype=torch.int16)
    hi = torch.randint(0, 20, (4, 1), dtype=torch.int16)
    same(T.clamp(x.cuda(), lo.cuda(), hi.cuda()), torch.clamp(x, lo, hi), "int16 broadcast bounds")
    same(T.clamp(x.cuda(), -7, 9), torch.clamp(x, -7, 9), "int16 scalar bounds")
    same(T.clamp(x.cuda(), 0.5, 2.5), torch.clamp(x, 0.5, 2.5), "int16 with float bounds promotes")
    xt = torch.randn(40, 30)
    same(T.clamp(xt.cuda().t(), -0.5, 0.5), torch.clamp(xt.t(), -0.5, 0.5), "non-contiguous")
    with pytest.raises(RuntimeError):
        T.clamp(xt.cuda())


# ------------------------------------------------- full-size bandwidth case


def test_div_floor_full_size_fp32():
    """fp32 (8192, 4096) floor division (the elementwise config shape): every
    element against the oracle, plus the size-independent identity
    q * b + r == a for r = a - q * b with |r| < |b| and sign(r) = sign(b)."""
    g = torch.Generator().manual_seed(0)
    a = torch.randn(8192, 4096, generator=g) * 10
    b = torch.randn(8192, 4096, generator=g) + 0.5
    got = T.div(a.cuda(), b.cuda(), rounding_mode="floor")
    same(got, ora(lambda x, y, d: O.div(x, y, d, "floor"), a.numpy(), b.numpy(), dt="f32"), "floor full size")
    del got


def _floor_div_hard_cases(seed=3):
    """fp32 (a, b) pairs aimed at the exact-remainder fast path of floor
    division: quotients within a few ulps of an integer (the rounded quotient
    can round up across it), |a| just below |b|, subnormal operands, huge
    quotients (|a / b| >= 2^23, the fallback), signed zeros, infinities and
    NaN."""
    rng = np.random.default_rng(seed)
    a_parts, b_parts = [], []
    b = (rng.standard_normal(20000) * 10.0 ** rng.uniform(-2, 2, 20000)).astype(np.float32)
    k = rng.integers(-5_000_000, 5_000_000, 20000).astype(np.float32)
    a = (k * b).astype(np.float32)
    for steps in (-2, -1, 0, 1, 2):
        s = a.copy()
        for _ in range(abs(steps)):
            s = np.nextafter(s, np.float32(np.inf if steps > 0 else -np.inf)).astype(np.float32)
        a_parts.append(s)
        b_parts.append(b)
    bb = rng.standard_normal(20000).astype(np.float32)
    near = np.nextafter(bb, np.float32(0)).astype(np.float32)
    a_parts.append(np.where(rng.random(20000) < 0.5, near, -near).astype(np.float32))
    b_parts.append(bb)
    tiny = np.float32(1e-45)
    a_parts.append((rng.integers(-10**6, 10**6, 20000).astype(np.float32) * tiny).astype(np.float32))
    b_parts.append((rng.integers(1, 1000, 20000) * rng.choice([-1, 1], 20000)).astype(np.float32) * tiny)
    a_parts.append((rng.standard_normal(20000) * 1e30).astype(np.float32))
    b_parts.append((rng.standard_normal(20000) * 1e-3).astype(np.float32))
    sp_a = np.array([0.0, -0.0, -0.0, 5.0, -5.0, np.inf, np.nan, 2.0, 3e38, -7.5, 7.5, 1.0], np.float32)
    sp_b = np.array([3.0, 3.0, -3.0, np.inf, -np.inf, 2.0, 2.0, np.nan, 1e-3, 2.5, -2.5, 0.0], np.float32)
    a_parts.append(sp_a)
    b_parts.append(sp_b)
    return np.concatenate(a_parts), np.concatenate(b_parts)


def test_div_floor_exact_remainder_cases():
    """Floor division's remainder is computed exactly (fast fma path for
    |a / b| < 2^23, library fmod beyond): bit-exact against the oracle's
    numpy fmod on the hard cases, fp32 and bf16 (bf16 computes in fp32)."""
    a, b = _floor_div_hard_cases()
    got = T.div(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), rounding_mode="floor")
    same(got, ora(lambda x, y, d: O.div(x, y, d, "floor"), a, b, dt="f32"), "floor hard cases f32")
    ab, bb = torch.from_numpy(a).bfloat16(), torch.from_numpy(b).bfloat16()
    got = T.div(ab.cuda(), bb.cuda(), rounding_mode="floor")
    same(got, ora(lambda x, y, d: O.div(x, y, d, "floor"), to_np(ab), to_np(bb), dt="bf16"), "floor hard cases bf16")


@pytest.mark.parametrize("dtype", (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8))
@pytest.mark.parametrize("rounding_mode", ("trunc", "floor"))
def test_div_integer_extremes(dtype, rounding_mode):
    """Integer division at the type's extremes (the 32-bit arithmetic used
    for types up to 32 bits, 64-bit for int64): min / -1 wraps, every sign
    combination, |b| > |a|, tensor and number divisors (a number past the
    32-bit range takes the 64-bit form), against torch on the CPU."""
    info = torch.iinfo(dtype)
    vals = sorted(v for v in {info.min, info.min + 1, -7, -3, -1, 0, 1, 2, 3, 7, info.max - 1, info.max}
                  if info.min <= v <= info.max)
    a = torch.tensor(vals, dtype=dtype).repeat_interleave(len(vals))
    b = torch.tensor(vals, dtype=dtype).repeat(len(vals))
    # min / -1 wraps to min; torch's CPU kernel traps on it for int32 / int64
    wrap = (a == info.min) & (b == -1)
    got_wrap = T.div(a[wrap].cuda(), b[wrap].cuda(), rounding_mode=rounding_mode)
    assert (got_wrap.cpu() == info.min).all()
    keep = (b != 0) & ~wrap
    a, b = a[keep], b[keep]
    got = T.div(a.cuda(), b.cuda(), rounding_mode=rounding_mode)
    same(got, torch.div(a, b, rounding_mode=rounding_mode), f"div {rounding_mode} {dtype} extremes")
    for num in (3, -7, info.max) + ((2**40,) if dtype == torch.int64 else ()):
        got = T.div(a.cuda(), num, rounding_mode=rounding_mode)
        same(got, torch.div(a, num, rounding_mode=rounding_mode), f"div {rounding_mode} {dtype} by {num}")


def test_binary_zero_dim_gpu_operand():
    """A 0-dim GPU tensor operand (broadcast from one element in memory) on
    either side of a non-commutative op, bit for bit against torch."""
    x = torch.randn(1000, 77).bfloat16()
    s = torch.tensor(0.37).bfloat16()
    xg, sg = x.cuda(), s.cuda()
    same(T.sub(xg, sg), x - s, "x - s")
    same(T.sub(sg, xg), s - x, "s - x")
    same(T.div(sg, xg), s / x, "s / x")
    same(T.mul(xg.t(), sg), x.t() * s, "transposed x * s")
    i = torch.randint(-100, 100, (4096,), dtype=torch.int32)
    d = torch.tensor(7, dtype=torch.int32)
    same(T.div(i.cuda(), d.cuda(), rounding_mode="floor"), torch.div(i, d, rounding_mode="floor"), "int floor by 0-dim")
