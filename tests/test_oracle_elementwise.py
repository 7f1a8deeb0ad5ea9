"""Pins the CPU oracle of the rest of the elementwise family (relu, sigmoid,
tanh, neg, abs, rsqrt, sin, cos, sub, div, pow, comparisons, isinf, isnan,
clamp) -- CPU only.  Three independent checks, as for the hot-path ops:
golden vectors written by torch CPU (tests/golden/golden_elementwise.npz),
closed forms / brute force over Python numbers, and planted mistakes that
those checks must catch."""

import math
import os

import numpy as np
import pytest
import torch

from oracle import ops as O
from tests.helpers import TOL_ELEMENTWISE, from_np

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_elementwise.npz"))
FDTS = ("f32", "f16", "bf16")
IDTS = ("i8", "i16", "i32", "i64")
POW_SCALARS = (2, 3, 0.5, -0.5, -1, -2, 1.7)
CMPS = ("eq", "ne", "gt", "ge", "lt", "le")


def equal(a, b, dt, what):
    ta, tb = from_np(np.asarray(a), dt), from_np(np.asarray(b), dt)
    if dt in FDTS:
        nan = torch.isnan(ta.double()) & torch.isnan(tb.double())
        diff = (ta.double() != tb.double()) & ~nan
        # -0 and +0 must match too
        diff |= (torch.signbit(ta.double()) != torch.signbit(tb.double())) & ~nan & (ta.double() == 0)
    else:
        diff = ta != tb
    assert not diff.any(), f"{what}: {int(diff.sum())} elements differ"


def close(a, b, dt, what, ulps=None):
    """Within the elementwise tolerance; for 16-bit types also within `ulps`
    units of the output type (the opmath results agree to ~1e-7, so a 16-bit
    rounding can differ by at most one ulp)."""
    rtol, atol = TOL_ELEMENTWISE[dt]
    ta, tb = from_np(np.asarray(a), dt).double(), from_np(np.asarray(b), dt).double()
    if dt != "f32":
        eps = torch.finfo(from_np(np.asarray(a), dt).dtype).eps
        rtol, atol = max(rtol, eps), max(atol, eps)
    torch.testing.assert_close(ta, tb, rtol=rtol, atol=atol, equal_nan=True, msg=lambda m: f"{what}: {m}")


def equal_bulk(a, b, dt, what):
    """torch's CPU loops run a vectorised bulk (one fp32 evaluation, one
    rounding, or a single fused multiply-add -- what the oracle does) and a
    scalar tail (up to two vector widths, 64 16-bit elements) that rounds
    after every operation; compare the bulk bit for bit and the tail within
    tolerance."""
    a, b = np.asarray(a), np.asarray(b)
    bulk = (a.size // 64) * 64
    equal(a[:bulk], b[:bulk], dt, what)
    if bulk < a.size:
        close(a[bulk:], b[bulk:], dt, what + " tail")


# ----------------------------------------------------------- golden vectors


@pytest.mark.parametrize("dt", FDTS)
def test_golden_unary(dt):
    x = G[f"x_{dt}"]
    for op in ("relu", "neg", "abs"):
        equal(getattr(O, op)(x, dt), G[f"{op}_{dt}"], dt, op)
    equal_bulk(O.rsqrt(x, dt), G[f"rsqrt_{dt}"], dt, "rsqrt")
    for op in ("sigmoid", "tanh", "sin", "cos"):
        close(getattr(O, op)(x, dt), G[f"{op}_{dt}"], dt, op)
    np.testing.assert_array_equal(O.isinf(x, dt), G[f"isinf_{dt}"])
    np.testing.assert_array_equal(O.isnan(x, dt), G[f"isnan_{dt}"])


@pytest.mark.parametrize("dt", FDTS)
def test_golden_binary(dt):
    x, y = G[f"x_{dt}"], G[f"y_{dt}"]
    # sub runs torch's add kernel: vectorised bulk bit-exact, scalar tail
    # within tolerance
    equal_bulk(O.sub(x, y, dt, 0.7), G[f"sub_{dt}"], dt, "sub")
    equal_bulk(O.sub(x, 1.1, dt, 1.3), G[f"sub_scalar_{dt}"], dt, "sub scalar")
    for mode in (None, "trunc", "floor"):
        tag = mode or "true"
        equal(O.div(x, y, dt, mode), G[f"div_{tag}_{dt}"], dt, f"div {tag}")
        equal(O.div(x, 1.1, dt, mode), G[f"div_{tag}_scalar_{dt}"], dt, f"div {tag} scalar")
    close(O.pow(x, y, dt), G[f"pow_{dt}"], dt, "pow")
    for i, e in enumerate(POW_SCALARS):
        got = O.pow(x, e, dt)
        if e in (2, 3, -2, -1) and dt != "f16":
            equal(got, G[f"pow_scalar{i}_{dt}"], dt, f"pow {e}")
        elif e == -0.5 and dt != "f16":
            equal_bulk(got, G[f"pow_scalar{i}_{dt}"], dt, f"pow {e}")
        else:
            # torch's CPU sqrt / powf are not correctly rounded (1 ulp away on
            # ~0.6 % of inputs); the oracle's are
            close(got, G[f"pow_scalar{i}_{dt}"], dt, f"pow {e}")
    for op in CMPS:
        np.testing.assert_array_equal(O.compare(op, x, y, dt), G[f"{op}_{dt}"], err_msg=op)
        np.testing.assert_array_equal(O.compare(op, x, 1.001, dt), G[f"{op}_scalar_{dt}"], err_msg=op)
    lo, hi = G[f"lo_{dt}"], G[f"hi_{dt}"]
    equal(O.clamp(x, lo, hi, dt), G[f"clamp_{dt}"], dt, "clamp")
    equal(O.clamp(x, lo, None, dt), G[f"clamp_min_{dt}"], dt, "clamp min")
    equal(O.clamp(x, -0.11, 0.5003, dt), G[f"clamp_scalar_{dt}"], dt, "clamp scalar")
    equal(O.clamp(x, None, 0.3, dt), G[f"clamp_max_scalar_{dt}"], dt, "clamp max scalar")


@pytest.mark.parametrize("dt", IDTS)
def test_golden_integer(dt):
    a, b, e = G[f"ia_{dt}"], G[f"ib_{dt}"], G[f"ie_{dt}"]
    for op in ("relu", "neg", "abs"):
        np.testing.assert_array_equal(getattr(O, op)(a, dt), G[f"i{op}_{dt}"], err_msg=op)
    np.testing.assert_array_equal(O.sub(a, b, dt, 3), G[f"isub_{dt}"])
    np.testing.assert_array_equal(O.div(a, b, dt, "trunc"), G[f"idiv_trunc_{dt}"])
    np.testing.assert_array_equal(O.div(a, b, dt, "floor"), G[f"idiv_floor_{dt}"])
    np.testing.assert_array_equal(O.pow(b, e, dt), G[f"ipow_{dt}"])
    for op in CMPS:
        np.testing.assert_array_equal(O.compare(op, a, b, dt), G[f"i{op}_{dt}"], err_msg=op)
    np.testing.assert_array_equal(O.clamp(a, b * 5, b * 5 + 40, dt), G[f"iclamp_{dt}"])
    np.testing.assert_array_equal(O.clamp(a, -7, 50, dt), G[f"iclamp_scalar_{dt}"])


# ------------------------------------------------ closed forms, brute force


def _f32(v):
    return np.asarray(v, dtype=np.float32)


def pin_relu(relu):
    x = _f32([-2.0, -0.0, 0.0, 3.5, np.nan, -np.inf, np.inf])
    r = relu(x, "f32")
    ok = np.array_equal(r[[0, 2, 3, 5, 6]], _f32([0, 0, 3.5, 0, np.inf])) and np.isnan(r[4])
    ok &= bool(np.signbit(r[1]))  # -0 passes through (clamp_min keeps x when not below 0)
    xi = np.arange(-50, 50, dtype=np.int16)
    ok &= np.array_equal(relu(xi, "i16"), np.array([max(0, int(v)) for v in xi], np.int16))
    fin = np.random.default_rng(0).standard_normal(1000).astype(np.float32)
    ok &= np.array_equal(relu(fin, "f32"), (fin + np.abs(fin)) / 2)
    return bool(ok)


def pin_sigmoid(sigmoid):
    x = np.random.default_rng(1).standard_normal(10000).astype(np.float64) * 5
    s = sigmoid(x, "f64")
    ok = np.allclose(s + sigmoid(-x, "f64"), 1.0, rtol=0, atol=1e-15)
    ok &= np.allclose(s, (1 + np.tanh(x / 2)) / 2, rtol=1e-14, atol=1e-15)
    ok &= sigmoid(np.float64([0.0]), "f64")[0] == 0.5
    return bool(ok)


def pin_tanh(tanh):
    x = np.random.default_rng(2).standard_normal(10000).astype(np.float64) * 3
    t = tanh(x, "f64")
    ok = np.array_equal(tanh(-x, "f64"), -t)
    ok &= np.allclose(t, 2 / (1 + np.exp(-2 * x)) - 1, rtol=1e-13, atol=1e-15)
    ok &= tanh(np.float64([1000.0]), "f64")[0] == 1.0  # no overflow to NaN
    return bool(ok)


def pin_neg(neg):
    x = _f32([1.5, -0.0, 0.0, np.inf, np.nan])
    n = neg(x, "f32")
    ok = n[0] == -1.5 and not np.signbit(n[1]) and np.signbit(n[2]) and n[3] == -np.inf and np.isnan(n[4])
    i = np.array([-128, -1, 0, 1, 127], np.int8)
    ok &= np.array_equal(neg(i, "i8"), np.array([-128, 1, 0, -1, -127], np.int8))
    bf = O.f32_to_bf16(_f32([2.0, -3.0]))
    ok &= np.array_equal(O.bf16_to_f32(neg(bf, "bf16")), _f32([-2.0, 3.0]))
    return bool(ok)


def pin_abs(abs_):
    x = _f32([-1.5, -0.0, 2.0, -np.inf, np.nan])
    a = abs_(x, "f32")
    ok = a[0] == 1.5 and a[1] == 0 and not np.signbit(a[1]) and a[2] == 2 and a[3] == np.inf and np.isnan(a[4])
    i = np.array([-128, -5, 0, 7], np.int8)
    ok &= np.array_equal(abs_(i, "i8"), np.array([-128, 5, 0, 7], np.int8))
    v = np.random.default_rng(3).standard_normal(1000).astype(np.float32)
    ok &= np.array_equal(abs_(v, "f32"), np.maximum(v, -v))
    return bool(ok)


def pin_rsqrt(rsqrt):
    x = _f32([4.0, 0.25, 0.0, -0.0, -1.0, np.inf])
    r = rsqrt(x, "f32")
    ok = r[0] == 0.5 and r[1] == 2.0 and r[2] == np.inf and r[3] == -np.inf and np.isnan(r[4]) and r[5] == 0
    v = np.random.default_rng(4).random(10000) * 100 + 1e-3
    ok &= np.allclose(rsqrt(v, "f64") ** 2 * v, 1.0, rtol=1e-14)
    return bool(ok)


def pin_sin(sin):
    x = np.random.default_rng(5).standard_normal(10000) * 4
    ok = np.allclose(sin(x, "f64") ** 2 + O.cos(x, "f64") ** 2, 1.0, rtol=0, atol=1e-14)
    ok &= np.array_equal(sin(-x, "f64"), -sin(x, "f64"))
    ok &= abs(sin(np.float64([math.pi / 6]), "f64")[0] - 0.5) < 1e-15
    return bool(ok)


def pin_cos(cos):
    x = np.random.default_rng(6).standard_normal(10000) * 4
    ok = np.allclose(O.sin(x, "f64") ** 2 + cos(x, "f64") ** 2, 1.0, rtol=0, atol=1e-14)
    ok &= np.array_equal(cos(-x, "f64"), cos(x, "f64"))
    ok &= cos(np.float64([0.0]), "f64")[0] == 1.0 and abs(cos(np.float64([math.pi / 3]), "f64")[0] - 0.5) < 1e-15
    return bool(ok)


def pin_sub(sub):
    rng = np.random.default_rng(7)
    a = rng.integers(-1000, 1000, 2000).astype(np.int32)
    b = rng.integers(-1000, 1000, 2000).astype(np.int32)
    ok = np.array_equal(sub(a, b, "i32", 3), np.array([int(x) - 3 * int(y) for x, y in zip(a, b)], np.int32))
    f = rng.standard_normal(1000).astype(np.float64)
    ok &= np.array_equal(sub(f, f, "f64", 1), np.zeros_like(f))
    ok &= np.array_equal(sub(f, 2.0, "f64", 1), f - 2.0)
    return bool(ok)


def pin_div(div):
    rng = np.random.default_rng(8)
    a = rng.standard_normal(20000) * 10
    b = rng.standard_normal(20000)
    a[:6] = [7.5, 0.0, -0.0, 5.0, -5.0, 1.0]
    b[:6] = [-np.inf, -3.0, 3.0, -2.0, 2.0, np.inf]
    fl = div(a, b, "f64", "floor")
    py = np.array([x // y for x, y in zip(a.tolist(), b.tolist())])  # Python's float floor division
    ok = np.array_equal(fl, py) and np.array_equal(np.signbit(fl), np.signbit(py))
    ok &= np.array_equal(div(a, b, "f64", "trunc"), np.trunc(a / b))
    ok &= np.array_equal(div(a, b, "f64"), a / b)
    ia = rng.integers(-300, 300, 5000).astype(np.int16)
    ib = rng.integers(-20, 20, 5000).astype(np.int16)
    ib[ib == 0] = 7
    fi = [int(x) // int(y) for x, y in zip(ia, ib)]
    ti = [int(x / y) if (x % y == 0) else (abs(int(x)) // abs(int(y))) * (1 if (x < 0) == (y < 0) else -1)
          for x, y in zip(ia.tolist(), ib.tolist())]
    ok &= np.array_equal(div(ia, ib, "i16", "floor"), np.array(fi, np.int16))
    ok &= np.array_equal(div(ia, ib, "i16", "trunc"), np.array(ti, np.int16))
    return bool(ok)


def pin_pow(pow_):
    rng = np.random.default_rng(9)
    x = np.abs(rng.standard_normal(5000)).astype(np.float32) + np.float32(1e-3)
    ok = np.array_equal(pow_(x, 2, "f32"), x * x)
    ok &= np.array_equal(pow_(x, 0.5, "f32"), np.sqrt(x))
    ok &= np.array_equal(pow_(x, 3, "f32"), x * x * x)
    xb = O.f32_to_bf16(x)
    xbf = O.bf16_to_f32(xb)
    ok &= np.array_equal(pow_(xb, 3, "bf16"), O.f32_to_bf16(O.bf16_to_f32(O.f32_to_bf16(xbf * xbf)) * xbf))
    ok &= np.isinf(O.to_compute(pow_(np.float16([-np.inf]), 0.5, "f16"), "f16")[0])  # f16: powf, no sqrt
    ok &= np.array_equal(pow_(x, -1, "f32"), np.float32(1) / x)
    ok &= np.allclose(pow_(x, 1.7, "f32"), (x.astype(np.float64) ** 1.7), rtol=1e-6)
    ok &= np.allclose(pow_(x.astype(np.float64), np.full(5000, 2.5), "f64"), x.astype(np.float64) ** 2.5, rtol=1e-14)
    ok &= pow_(_f32([np.nan]), _f32([0.0]), "f32")[0] == 1.0
    base = rng.integers(-6, 7, 3000)
    ex = rng.integers(-3, 9, 3000)
    def ref(b, e):
        if e >= 0:
            return int(b) ** int(e)
        return 1 if b == 1 else ((-1) ** (-e) if b == -1 else 0)
    exp_ = np.array([ref(b, e) for b, e in zip(base.tolist(), ex.tolist())], np.int64)
    ok &= np.array_equal(pow_(base.astype(np.int64), ex.astype(np.int64), "i64"), exp_)
    ok &= np.array_equal(pow_(np.array([3], np.int8), np.array([5], np.int8), "i8"), np.array([243 - 256], np.int8))
    return bool(ok)


def pin_compare(compare):
    a = np.repeat(np.arange(-128, 128, dtype=np.int8), 256)
    b = np.tile(np.arange(-128, 128, dtype=np.int8), 256)
    pa, pb = a.astype(np.int64).tolist(), b.astype(np.int64).tolist()
    import operator as op
    pyops = {"eq": op.eq, "ne": op.ne, "gt": op.gt, "ge": op.ge, "lt": op.lt, "le": op.le}
    ok = True
    for name, f in pyops.items():
        ok &= np.array_equal(compare(name, a, b, "i8"), np.array([f(x, y) for x, y in zip(pa, pb)]))
    n = _f32([np.nan, 1.0])
    ok &= not compare("eq", n, n, "f32")[0] and compare("ne", n, n, "f32")[0] and not compare("ge", n, n, "f32")[0]
    ok &= compare("eq", _f32([0.0]), _f32([-0.0]), "f32")[0]
    one = O.f32_to_bf16(_f32([1.0]))
    ok &= compare("eq", one, 1.001, "bf16")[0] and not compare("lt", one, 1.001, "bf16")[0]  # scalar rounds to bf16
    return bool(ok)


def pin_isinf(isinf):
    x = _f32([np.inf, -np.inf, np.nan, 0.0, 3.4e38, -1.0])
    return bool(np.array_equal(isinf(x, "f32"), [True, True, False, False, False, False])
                and not isinf(np.array([1, 2], np.int32), "i32").any())


def pin_isnan(isnan):
    x = _f32([np.inf, -np.inf, np.nan, 0.0, -np.nan])
    return bool(np.array_equal(isnan(x, "f32"), [False, False, True, False, True])
                and not isnan(np.array([1, 2], np.int32), "i32").any())


def pin_clamp(clamp):
    rng = np.random.default_rng(10)
    x = rng.standard_normal(5000).astype(np.float32)
    lo = rng.standard_normal(5000).astype(np.float32) - 1
    hi = rng.standard_normal(5000).astype(np.float32) + 1
    ok = np.array_equal(clamp(x, lo, hi, "f32"), np.minimum(np.maximum(x, lo), hi))
    ok &= np.array_equal(clamp(x, None, hi, "f32"), np.minimum(x, hi))
    ok &= np.array_equal(clamp(x, 0.5, 0.1, "f32"), np.full_like(x, np.float32(0.1)))  # lo > hi -> hi
    n = _f32([np.nan, -1.5, 2.0, 0.5])
    r = clamp(n, _f32([0, np.nan, 0, 0]), _f32([1, 1, np.nan, 1]), "f32")
    ok &= bool(np.isnan(r[:3]).all()) and r[3] == 0.5
    i = np.arange(-20, 20, dtype=np.int32)
    ok &= np.array_equal(clamp(i, -3, 5, "i32"), np.clip(i, -3, 5))
    return bool(ok)


PINS = {
    "relu": pin_relu, "sigmoid": pin_sigmoid, "tanh": pin_tanh, "neg": pin_neg, "abs": pin_abs,
    "rsqrt": pin_rsqrt, "sin": pin_sin, "cos": pin_cos, "sub": pin_sub, "div": pin_div, "pow": pin_pow,
    "compare": pin_compare, "isinf": pin_isinf, "isnan": pin_isnan, "clamp": pin_clamp,
}


@pytest.mark.parametrize("name", sorted(PINS))
def test_closed_forms(name):
    assert PINS[name](getattr(O, name)), f"oracle {name} fails its closed-form pins"


# ------------------------------------------------------------ planted mistakes


def _m_relu_nan_to_zero(x, dt):
    if dt not in O.FLOAT_DTYPES:
        return O.relu(x, dt)
    c = O.to_compute(x, dt)
    return np.where(c > 0, np.asarray(x), O.round_to(np.zeros_like(c), dt))


def _m_floor_naive(a, b, dt, rounding_mode=None):
    if rounding_mode == "floor" and dt in O.FLOAT_DTYPES:
        return O.round_to(np.floor(O.to_compute(a, dt) / O.to_compute(b, dt)), dt)
    return O.div(a, b, dt, rounding_mode)


def _m_trunc_as_floor(a, b, dt, rounding_mode=None):
    return O.div(a, b, dt, "floor" if rounding_mode == "trunc" else rounding_mode)


def _m_pow_neg_int_one(a, b, dt):
    r = O.pow(a, b, dt)
    if dt not in O.FLOAT_DTYPES:
        r = np.where(np.asarray(b) < 0, 1, r).astype(r.dtype)
    return r


def _m_pow_sqrt_as_pow(a, b, dt):
    if np.isscalar(b) and b == 0.5 and dt == "f32":
        return np.power(O.to_compute(a, dt), np.float32(0.5) + np.float32(1e-7))
    return O.pow(a, b, dt)


def _m_compare_swapped(op, a, b, dt):
    return O.compare(op, b, a, dt) if not np.isscalar(b) else O.compare(op, a, b, dt)


def _m_clamp_order(x, lo, hi, dt):
    # max(min(x, hi), lo): differs when lo > hi
    if lo is None or hi is None:
        return O.clamp(x, lo, hi, dt)
    return O.clamp(O.clamp(x, None, hi, dt), lo, None, dt)


def _m_sub_sign(a, b, dt, alpha=1):
    return O.add(a, b, dt, alpha)


def _m_sigmoid_sign(x, dt):
    return O.sigmoid(-np.asarray(x), dt)


def _m_rsqrt_no_recip(x, dt):
    return O.round_to(np.sqrt(O.to_compute(x, dt)), dt)


def _m_isinf_pos_only(x, dt):
    c = O.to_compute(x, dt)
    return c == np.inf


@pytest.mark.parametrize("name,mutant", [
    ("relu", _m_relu_nan_to_zero), ("div", _m_floor_naive), ("div", _m_trunc_as_floor),
    ("pow", _m_pow_neg_int_one), ("pow", _m_pow_sqrt_as_pow), ("compare", _m_compare_swapped),
    ("clamp", _m_clamp_order), ("sub", _m_sub_sign), ("sigmoid", _m_sigmoid_sign),
    ("rsqrt", _m_rsqrt_no_recip), ("isinf", _m_isinf_pos_only),
])
def test_planted_mistakes_are_caught(name, mutant):
    assert not PINS[name](mutant), f"a planted mistake in {name} went unnoticed"


def test_oracle_int_div_number_wraps_to_dtype():
    """An integer tensor divided by a Python number: the number is converted
    to the tensor's dtype with wrap-around first, as torch's CPU kernel does
    (uint8 // -7 divides by 249, int8 // 300 by 44)."""
    for dt, vals, num in (("u8", [0, 5, 200, 255], -7), ("u8", [0, 5, 200, 255], 300), ("i8", [-100, 5, 100], 300),
                          ("i8", [-100, 5, 100], -300), ("i32", [-7, 7, 2**31 - 1], 3)):
        tdt = {"u8": torch.uint8, "i8": torch.int8, "i32": torch.int32}[dt]
        a = torch.tensor(vals, dtype=tdt)
        for mode in ("trunc", "floor"):
            exp = torch.div(a, num, rounding_mode=mode).numpy()
            got = O.div(a.numpy(), num, dt, mode)
            np.testing.assert_array_equal(got, exp, err_msg=f"{dt} {vals} // {num} {mode}")
