"""CPU oracle for the ntops LLM hot path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of each operator's algorithm, used by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker of
the HIP kernels.  Nothing in the product (ntops_amd/) imports it.

Representation: arrays are numpy arrays in their storage dtype, with bf16
carried as uint16 bit patterns and tagged by the dtype string "bf16"
(numpy has no bfloat16).  dtype strings: "f32", "f16", "bf16", "f64",
"bool", "u8", "i8", "i16", "i32", "i64".

Each function cites the reference file it restates (paths relative to the
mygitljf/ntops tree).  Where ntops and torch differ, the oracle follows torch's
CPU kernels, which is the parity reference this build is held to; the
deviation is stated in the docstring.

Pinning (tests/test_oracle.py): every function is checked against golden
vectors written by torch CPU (tests/golden/), against live torch CPU, and
against closed forms / invariants / brute force chosen so that a dropped
term, a wrong sign or a transposed operand fails.  No function is unpinned.
"""

import numpy as np

FLOAT_DTYPES = ("f32", "f16", "bf16", "f64")
INT_DTYPES = ("bool", "u8", "i8", "i16", "i32", "i64")

_NP = {
    "f32": np.float32,
    "f16": np.float16,
    "bf16": np.uint16,
    "f64": np.float64,
    "bool": np.bool_,
    "u8": np.uint8,
    "i8": np.int8,
    "i16": np.int16,
    "i32": np.int32,
    "i64": np.int64,
}


def np_dtype(dt):
    return _NP[dt]


# ---------------------------------------------------------------- bf16 ----


def bf16_to_f32(u):
    """bf16 bit patterns -> float32 (exact)."""
    u = np.asarray(u, dtype=np.uint16)
    return (u.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16(f):
    """float32 -> bf16 bit patterns, round to nearest even; NaN -> 0x7FC0
    (c10::BFloat16's round_to_nearest_even)."""
    f = np.ascontiguousarray(np.asarray(f, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(np.isnan(f), np.uint16(0x7FC0), r)
    return r.astype(np.uint16)


def compute_type(dt):
    """Opmath type: fp32 for 16-bit floats and fp32, fp64 for fp64."""
    return np.float64 if dt == "f64" else np.float32


def to_compute(a, dt):
    """Storage -> opmath value (exact)."""
    if dt == "bf16":
        return bf16_to_f32(a)
    if dt == "f64":
        return np.asarray(a, dtype=np.float64)
    return np.asarray(a).astype(np.float32)


def round_to(v, dt):
    """Opmath value -> storage dtype with one rounding (RNE)."""
    if dt == "bf16":
        return f32_to_bf16(np.asarray(v, dtype=np.float32))
    if dt == "f16":
        return np.asarray(v, dtype=np.float32).astype(np.float16)
    if dt == "f32":
        return np.asarray(v, dtype=np.float32)
    if dt == "f64":
        return np.asarray(v, dtype=np.float64)
    raise ValueError(dt)


def rnd(v, dt):
    """Round an opmath value to dt and return it as opmath again."""
    return to_compute(round_to(v, dt), dt)


def _fma32(a, b, c):
    """fp32 fused multiply-add a*b + c with a single rounding, computed in
    fp64 (a*b is exact in fp64 for fp32 operands) then rounded to fp32."""
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def _with_errstate(fn):
    def wrapped(*args, **kwargs):
        with np.errstate(all="ignore"):
            return fn(*args, **kwargs)

    wrapped.__name__ = fn.__name__
    wrapped.__doc__ = fn.__doc__
    return wrapped


# ------------------------------------------------------------ unary ops ---


@_with_errstate
def silu(x, dt):
    """kernels/silu.py:10 -- output = input / (1 + exp(-fp32(input)))."""
    c = to_compute(x, dt)
    one = compute_type(dt)(1)
    return round_to(c / (one + np.exp(-c)), dt)


@_with_errstate
def gelu(x, dt, approximate="none"):
    """kernels/gelu.py:10-26.  "none": x * 0.5 * (1 + erf(x / sqrt 2)), the
    division by sqrt 2 applied as a multiply by 1/sqrt 2 (torch's CPU form);
    "tanh": 0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 x^3)))."""
    from scipy.special import erf

    c = to_compute(x, dt)
    T = compute_type(dt)
    if approximate == "tanh":
        beta = T(np.sqrt(2.0) * (2.0 / np.sqrt(np.pi)) * 0.5)
        kappa = T(0.044715)
        inner = beta * (c + kappa * (c * c * c))
        return round_to(T(0.5) * c * (T(1) + np.tanh(inner)), dt)
    y = c * T(0.5) * (T(1) + erf(c * T(1.0 / np.sqrt(2.0))).astype(T))
    return round_to(y, dt)


@_with_errstate
def exp(x, dt):
    """kernels/exp.py:10 -- exp(input) in opmath, rounded to dt."""
    return round_to(np.exp(to_compute(x, dt)), dt)


def bitwise_not(x, dt):
    """kernels/bitwise_not.py:9-14 -- ~x; logical not for bool."""
    x = np.asarray(x)
    if dt == "bool":
        return np.logical_not(x)
    return np.invert(x)


# ----------------------------------------------------------- binary ops ---


def _int_wrap(v, dt):
    """int64 arithmetic result -> dt with two's-complement wrap-around."""
    if dt == "bool":
        return v != 0
    return v.astype(np.int64).astype(np_dtype(dt))


@_with_errstate
def add(a, b, dt, alpha=1):
    """kernels/add.py:10 -- input + alpha * other.

    Floating: alpha is first rounded to dt, then a single-rounding fma in
    opmath (torch's CPU kernel: vec::fmadd(other, alpha, self)); `b` may be a
    Python number, which torch's CPU add rounds to dt as well.  Integral:
    modular arithmetic; bool: (a + alpha*b) != 0."""
    if dt in FLOAT_DTYPES:
        al = to_compute(round_to(np.asarray(alpha, dtype=np.float64), dt), dt)
        ac = to_compute(a, dt)
        if np.isscalar(b) or np.ndim(b) == 0 and not isinstance(b, np.ndarray):
            bc = to_compute(round_to(np.asarray(float(b)), dt), dt)
        else:
            bc = to_compute(b, dt)
        bc, ac = np.broadcast_arrays(bc, ac)
        if dt == "f64":
            return ac + bc * al  # exactness of the fp64 fma is not needed at fp64 tolerance
        return round_to(_fma32(bc, np.broadcast_to(al, bc.shape), ac), dt)
    av = np.asarray(a).astype(np.int64)
    bv = np.asarray(b).astype(np.int64)
    with np.errstate(over="ignore"):
        return _int_wrap(av + np.int64(int(alpha)) * bv, dt)


@_with_errstate
def mul(a, b, dt):
    """kernels/mul.py:9 -- input * other in opmath, one rounding.  A Python
    number `b` stays in opmath (torch's CPU mul does not round it to dt)."""
    if dt in FLOAT_DTYPES:
        ac = to_compute(a, dt)
        if np.isscalar(b):
            bc = compute_type(dt)(b)
        else:
            bc = to_compute(b, dt)
        return round_to(ac * bc, dt)
    if dt == "bool":
        return np.logical_and(a, b)
    with np.errstate(over="ignore"):
        return _int_wrap(np.asarray(a).astype(np.int64) * np.asarray(b).astype(np.int64), dt)


def bitwise_and(a, b, dt):
    """kernels/bitwise_and.py:9 -- input & other (logical for bool)."""
    if dt == "bool":
        return np.logical_and(a, b)
    return np.bitwise_and(np.asarray(a), np.asarray(b)).astype(np_dtype(dt))


def bitwise_or(a, b, dt):
    """kernels/bitwise_or.py:9 -- input | other (logical for bool)."""
    if dt == "bool":
        return np.logical_or(a, b)
    return np.bitwise_or(np.asarray(a), np.asarray(b)).astype(np_dtype(dt))


# ------------------------------------------- rest of the elementwise family


def _is_number(b):
    return isinstance(b, (bool, int, float, np.integer, np.floating))


def _sign_bits(x, dt):
    """Unsigned view of a float array's storage and its sign-bit mask."""
    if dt == "bf16":
        return np.asarray(x, dtype=np.uint16), np.uint16(0x8000)
    if dt == "f16":
        return np.asarray(x, dtype=np.float16).view(np.uint16), np.uint16(0x8000)
    if dt == "f32":
        return np.asarray(x, dtype=np.float32).view(np.uint32), np.uint32(0x80000000)
    return np.asarray(x, dtype=np.float64).view(np.uint64), np.uint64(0x8000000000000000)


def _from_bits(u, dt):
    if dt == "bf16":
        return u.astype(np.uint16)
    return u.view({"f16": np.float16, "f32": np.float32, "f64": np.float64}[dt])


@_with_errstate
def relu(x, dt):
    """kernels/relu.py:9 -- max(0, x) as torch's clamp_min: x where x is not
    below 0 (so NaN and -0 pass through), else +0."""
    if dt in FLOAT_DTYPES:
        c = to_compute(x, dt)
        zero = round_to(np.zeros_like(c), dt)
        return np.where(c < 0, zero, np.asarray(x))
    if dt == "bool":
        raise ValueError("relu: bool")
    x = np.asarray(x)
    return np.where(x < 0, np.zeros_like(x), x)


@_with_errstate
def sigmoid(x, dt):
    """kernels/sigmoid.py:10 -- 1 / (1 + exp(-x)) in opmath, one rounding."""
    c = to_compute(x, dt)
    one = compute_type(dt)(1)
    return round_to(one / (one + np.exp(-c)), dt)


@_with_errstate
def tanh(x, dt):
    """kernels/tanh.py:10-13 -- tanh(x) in opmath, one rounding.  The reference
    writes (e^x - e^-x) / (e^x + e^-x), which is NaN once e^x overflows
    (|x| > 88 in fp32); the library tanh is the function torch evaluates."""
    return round_to(np.tanh(to_compute(x, dt)), dt)


def neg(x, dt):
    """kernels/neg.py:9 -- -x (sign bit flipped for floats, NaN included;
    two's-complement wrap for integers)."""
    if dt in FLOAT_DTYPES:
        u, m = _sign_bits(x, dt)
        return _from_bits(u ^ m, dt)
    if dt == "bool":
        raise ValueError("neg: bool")
    with np.errstate(over="ignore"):
        return _int_wrap(-np.asarray(x).astype(np.int64), dt)


def abs(x, dt):  # noqa: A001 (mirrors the operator's name)
    """kernels/abs.py:10 -- |x| (sign bit cleared for floats; the integer
    minimum wraps to itself)."""
    if dt in FLOAT_DTYPES:
        u, m = _sign_bits(x, dt)
        return _from_bits(u & ~m, dt)
    if dt == "bool":
        raise ValueError("abs: bool")
    with np.errstate(over="ignore"):
        return _int_wrap(np.abs(np.asarray(x).astype(np.int64)), dt)


@_with_errstate
def rsqrt(x, dt):
    """kernels/rsqrt.py:10 -- 1 / sqrt(x): an IEEE square root, then an IEEE
    division, in opmath (the form torch's CPU kernel evaluates)."""
    c = to_compute(x, dt)
    return round_to(compute_type(dt)(1) / np.sqrt(c), dt)


@_with_errstate
def sin(x, dt):
    """kernels/sin.py:10 -- sin(x) in opmath, one rounding."""
    return round_to(np.sin(to_compute(x, dt)), dt)


@_with_errstate
def cos(x, dt):
    """kernels/cos.py:10 -- cos(x) in opmath, one rounding."""
    return round_to(np.cos(to_compute(x, dt)), dt)


def sub(a, b, dt, alpha=1):
    """kernels/sub.py:10 -- input - alpha * other, evaluated as torch does:
    add(input, other, -alpha) (same roundings as add)."""
    if dt == "bool":
        raise ValueError("sub: bool")
    return add(a, b, dt, -alpha)


def _opmath_operand(b, dt):
    """A tensor operand in opmath, or a Python number kept in opmath."""
    if _is_number(b):
        return compute_type(dt)(b)
    return to_compute(b, dt)


@_with_errstate
def floor_divide_float(a, b):
    """Python's float floor division (CPython's float divmod), elementwise on
    arrays of one float type: q = (a - fmod(a, b)) / b, minus one when the
    remainder's sign differs from b's, then rounded to the nearest integer;
    a zero quotient takes the sign of a / b; b == 0 gives a / b."""
    a, b = np.broadcast_arrays(a, b)
    T = a.dtype.type
    mod = np.fmod(a, b)
    div = (a - mod) / b
    adj = (mod != 0) & ((b < 0) != (mod < 0))
    div = np.where(adj, div - T(1), div)
    fl = np.floor(div)
    fl = np.where(div - fl > T(0.5), fl + T(1), fl)
    res = np.where(div == 0, np.copysign(T(0), a / b), fl)
    return np.where(b == 0, a / b, res).astype(a.dtype)


def _int_divide(a, b, floor):
    """Integer trunc / floor division in int64: 0 where b == 0 (torch's CPU
    kernel raises instead), wrap-around negation where b == -1."""
    a = np.asarray(a).astype(np.int64)
    b = np.asarray(b).astype(np.int64)
    a, b = np.broadcast_arrays(a, b)
    safe = np.where(b == 0, 1, b)
    q = np.abs(a) // np.abs(safe)  # magnitude of the truncated quotient
    with np.errstate(over="ignore"):
        q = np.where((a < 0) != (safe < 0), -q, q)
        if floor:
            q = np.where((q * safe != a) & ((a < 0) != (safe < 0)), q - 1, q)
        q = np.where(b == -1, -a, q)
    return np.where(b == 0, 0, q)


@_with_errstate
def div(a, b, dt, rounding_mode=None):
    """kernels/div.py:9-18.  Floating, in opmath with one rounding: a / b,
    trunc(a / b) (for two 16-bit tensors, of the quotient already rounded to
    dt, as torch's CPU kernel evaluates it), or Python's floor division (the reference's floor(a / b)
    differs when the rounded quotient lands on an integer; torch uses the
    floor-division form).  A Python-number divisor stays in opmath.  Integer
    dtypes: trunc / floor only (true division promotes to float first)."""
    if dt in FLOAT_DTYPES:
        ac, bc = to_compute(a, dt), _opmath_operand(b, dt)
        if rounding_mode is None:
            q = ac / bc
        elif rounding_mode == "trunc":
            # torch rounds a 16-bit tensor / tensor quotient to dt first; a
            # Python-number divisor truncates the opmath quotient
            q = np.trunc(ac / bc if _is_number(b) else rnd(ac / bc, dt))
        else:
            q = floor_divide_float(ac, np.asarray(bc, dtype=ac.dtype))
        return round_to(q, dt)
    if dt == "bool" or rounding_mode is None:
        raise ValueError("div: integer true division promotes to float first")
    if _is_number(b):
        # a Python-number divisor is converted to dt with wrap-around first
        # (torch: uint8 // -7 divides by 249)
        b = _int_wrap(np.asarray(int(b), dtype=np.int64), dt)
    return _int_wrap(_int_divide(a, b, rounding_mode == "floor"), dt)


def _int_pow(a, e):
    """Integer power with wrap-around; negative exponents follow torch: base 1
    -> 1, base -1 -> +-1 by parity, anything else -> 0."""
    a = np.asarray(a).astype(np.int64)
    e = np.asarray(e).astype(np.int64)
    a, e = np.broadcast_arrays(a, e)
    r = np.ones(a.shape, dtype=np.uint64)
    base = a.astype(np.uint64)
    ee = np.where(e < 0, 0, e)
    with np.errstate(over="ignore"):
        while np.any(ee):
            r = np.where(ee & 1, r * base, r)
            base = base * base
            ee = ee >> 1
    r = r.astype(np.int64)
    neg = np.where(a == 1, 1, np.where(a == -1, np.where(e & 1, -1, 1), 0))
    return np.where(e < 0, neg, r)


@_with_errstate
def pow(a, b, dt):  # noqa: A001
    """kernels/pow.py:10 -- a ** b.  Floating tensor ** tensor: the library
    pow in opmath, one rounding.  A Python-number exponent follows torch's CPU
    dispatch per dtype: f32 / f64 keep the exponent in double and evaluate
    0.5 -> sqrt, -0.5 -> 1/sqrt, -1 -> 1/x, 2 -> x*x, 3 -> x*x*x,
    -2 -> 1/(x*x), anything else -> pow in double, rounded once; bf16 rounds
    the exponent to bf16, has the same special cases with every product
    rounded to bf16, else powf; f16 rounds the exponent to f16 and always uses
    powf.  Integers: see _int_pow."""
    if dt not in FLOAT_DTYPES:
        if dt == "bool":
            raise ValueError("pow: bool")
        return _int_wrap(_int_pow(a, b), dt)
    ac = to_compute(a, dt)
    T = compute_type(dt)
    if not _is_number(b):
        return round_to(np.power(ac, to_compute(b, dt)), dt)
    if dt in ("f32", "f64"):
        e = float(b)
    else:
        e = float(to_compute(round_to(np.asarray([float(b)], dtype=np.float32), dt), dt)[0])
    one = T(1)
    if dt != "f16":
        r = lambda v: rnd(v, dt) if dt == "bf16" else v  # noqa: E731 (bf16: round each product)
        special = {0.5: np.sqrt, -0.5: lambda x: one / np.sqrt(x), -1.0: lambda x: one / x,
                   2.0: lambda x: x * x, 3.0: lambda x: r(x * x) * x, -2.0: lambda x: one / r(x * x)}
        if e in special:
            return round_to(special[e](ac), dt)
    if dt == "f32":
        return round_to(np.power(ac.astype(np.float64), e), dt)
    return round_to(np.power(ac, T(e)), dt)


_CMP = {"eq": np.equal, "ne": np.not_equal, "gt": np.greater, "ge": np.greater_equal,
        "lt": np.less, "le": np.less_equal}


@_with_errstate
def compare(op, a, b, dt):
    """kernels/{eq,ne,gt,ge,lt,le}.py:9 -> bool, compared in dt's opmath (exact
    for the 16-bit floats); a Python-number b is first rounded to dt (the
    common dtype, as in torch); integers compare as int64."""
    f = _CMP[op]
    if dt in FLOAT_DTYPES:
        ac = to_compute(a, dt)
        if _is_number(b):
            bc = to_compute(round_to(np.asarray(float(b), dtype=compute_type(dt)), dt), dt)
        else:
            bc = to_compute(b, dt)
        return f(ac, bc)
    return f(np.asarray(a).astype(np.int64), np.asarray(b).astype(np.int64))


def isinf(x, dt):
    """kernels/isinf.py:9-11 -> bool (false for integer inputs)."""
    if dt in FLOAT_DTYPES:
        return np.isinf(to_compute(x, dt))
    return np.zeros(np.shape(x), dtype=bool)


def isnan(x, dt):
    """kernels/isnan.py:9 -- x != x -> bool (false for integer inputs)."""
    if dt in FLOAT_DTYPES:
        c = to_compute(x, dt)
        return c != c
    return np.zeros(np.shape(x), dtype=bool)


@_with_errstate
def clamp(x, lo, hi, dt):
    """kernels/clamp.py:9 -- min(max(x, lo), hi) with torch's NaN rule: a NaN
    in x, then in lo, then in hi, is the result (so lo > hi gives hi).  lo /
    hi are arrays of dt, Python numbers (rounded to dt) or None (absent)."""
    x = np.asarray(x)

    def bound(v):
        if v is None:
            return None
        if _is_number(v):
            if dt in FLOAT_DTYPES:
                return np.broadcast_to(round_to(np.asarray(float(v), dtype=compute_type(dt)), dt), x.shape)
            return np.broadcast_to(np.asarray(v).astype(np_dtype(dt)), x.shape)
        return np.broadcast_to(np.asarray(v), x.shape)

    lo, hi = bound(lo), bound(hi)
    if dt in FLOAT_DTYPES:
        val = lambda v: to_compute(v, dt)  # noqa: E731
        xv = val(x)
        r = x.copy()
        rv = xv
        if lo is not None:
            lv = val(lo)
            r = np.where(rv < lv, lo, r)
            rv = val(r)
        if hi is not None:
            hv = val(hi)
            r = np.where(hv < rv, hi, r)
        if hi is not None:
            r = np.where(hv != hv, hi, r)
        if lo is not None:
            r = np.where(lv != lv, lo, r)
        return np.where(xv != xv, x, r).astype(x.dtype)
    r = x.copy()
    if lo is not None:
        r = np.where(r < lo, lo, r)
    if hi is not None:
        r = np.where(hi < r, hi, r)
    return r.astype(x.dtype)


# --------------------------------------------------------- row reductions -


def _rows(x, cols):
    return np.asarray(x).reshape(-1, cols)


@_with_errstate
def rms_norm(x, dt, cols, weight=None, eps=None, w_dt=None):
    """kernels/rms_norm.py:10-20 -- per row: rms = sqrt(sum(x^2)/N + eps) with
    fp32 accumulation; y = x / rms * w.

    Follows torch's fused CPU kernel: eps=None means finfo(float32).eps and
    the output is bf16/f16(x * (1/rms) * w) with x, 1/rms and w in fp32 and a
    single rounding (ntops instead rounds x / rms to dt before the weight and
    uses finfo(dt).eps)."""
    shape = np.shape(x)
    xf = _rows(to_compute(x, dt), cols).astype(np.float32)
    if eps is None:
        eps = float(np.finfo(np.float32).eps)
    ss = np.sum(xf * xf, axis=1, dtype=np.float32)
    rstd = np.float32(1) / np.sqrt(ss / np.float32(cols) + np.float32(eps))
    y = xf * rstd[:, None]
    if weight is not None:
        y = y * _expanded_rows(weight, w_dt or dt, shape, cols)
    return round_to(y, dt).reshape(shape)


def _expanded_rows(param, dt, shape, cols):
    """A norm parameter as the reference's `param.expand_as(input)`
    (torch/rms_norm.py:17-18, torch/layer_norm.py:17-25): broadcast to the
    input's shape, as fp32 rows of the normalized elements."""
    return np.broadcast_to(to_compute(param, dt).astype(np.float32), shape).reshape(-1, cols)


@_with_errstate
def layer_norm(x, dt, cols, weight=None, bias=None, eps=1e-5, wb_dt=None):
    """kernels/layer_norm.py:11-31 -- mean and biased variance of each row in
    fp32 (two passes), rstd = 1 / sqrt(var + eps), y = (x - mean) * rstd * w + b,
    evaluated in torch's CPU order (x * rstd + (-rstd * mean)) * w + b."""
    shape = np.shape(x)
    xf = _rows(to_compute(x, dt), cols).astype(np.float32)
    mean = np.sum(xf, axis=1, dtype=np.float32) / np.float32(cols)
    d = xf - mean[:, None]
    var = np.sum(d * d, axis=1, dtype=np.float32) / np.float32(cols)
    rstd = np.float32(1) / np.sqrt(np.maximum(var, np.float32(0)) + np.float32(eps))
    y = xf * rstd[:, None] + (-rstd * mean)[:, None]
    if weight is not None:
        y = y * _expanded_rows(weight, wb_dt or dt, shape, cols)
    if bias is not None:
        y = y + _expanded_rows(bias, wb_dt or dt, shape, cols)
    return round_to(y, dt).reshape(shape)


@_with_errstate
def softmax(x, dim, in_dt, out_dt=None):
    """kernels/softmax.py:9-29 -- max, sum of exp(x - max), exp(x - max)/sum.

    The input is rounded to the output dtype first; max/sum accumulate in
    fp32 (fp64 for fp64 output) and the result is exp(x - max) * (1/sum)
    rounded once -- torch's CPU kernel.  (ntops accumulates in the output
    dtype.)  An all -inf row gives NaN."""
    out_dt = out_dt or in_dt
    xin = to_compute(x, in_dt)
    xo = to_compute(round_to(xin, out_dt), out_dt)
    T = compute_type(out_dt)
    xo = xo.astype(T)
    if xo.ndim == 0:
        return round_to(np.ones((), dtype=T), out_dt)
    m = np.max(xo, axis=dim, keepdims=True)
    e = np.exp(xo - m)
    s = np.sum(e, axis=dim, keepdims=True, dtype=T)
    return round_to(e * (T(1) / s), out_dt)


# ------------------------------------------------------------------ RoPE --


@_with_errstate
def rotary_position_embedding(x, sin_table, cos_table, dt, interleaved=True):
    """kernels/rotary_position_embedding.py:6-47 on (B, S, H, D) input.

    Pairs are (2i, 2i+1) when interleaved, else (i, i + D/2).  Tables are
    (S, D/2) -- one angle per pair, ntops' form -- or (S, D), one value per
    element (x*cos + rotate_half(x)*sin).  out0 = x0*c0 - x1*s0,
    out1 = x1*c1 + x0*s1, with every product and sum rounded to dt (torch's
    eager evaluation order)."""
    xc = to_compute(x, dt)
    B, S, H, D = xc.shape
    sn = to_compute(sin_table, dt)[:S]
    cs = to_compute(cos_table, dt)[:S]
    half = D // 2
    if interleaved:
        i0 = np.arange(0, D, 2)
        i1 = i0 + 1
    else:
        i0 = np.arange(half)
        i1 = i0 + half
    x0 = xc[..., i0]
    x1 = xc[..., i1]
    if sn.shape[1] == D:
        c0, s0, c1, s1 = cs[:, i0], sn[:, i0], cs[:, i1], sn[:, i1]
    else:
        c0 = c1 = cs
        s0 = s1 = sn
    c0, s0, c1, s1 = (t[None, :, None, :] for t in (c0, s0, c1, s1))
    o0 = rnd(rnd(x0 * c0, dt) - rnd(x1 * s0, dt), dt)
    o1 = rnd(rnd(x1 * c1, dt) + rnd(x0 * s1, dt), dt)
    out = np.empty_like(xc)
    out[..., i0] = o0
    out[..., i1] = o1
    return round_to(out, dt)


def rope_tables(seq_len, emb_dim, base=10000.0, full=False):
    """fp32 sin/cos tables built like tests/test_rotary_position_embedding.py:
    37-45: theta_i = base^(-2i/D), angles = positions * theta.  With
    full=True the (S, D/2) tables are duplicated to (S, D) (rotate_half form)."""
    i = np.arange(emb_dim // 2, dtype=np.float32)
    theta = np.float32(base) ** (-np.float32(2) * (i / np.float32(emb_dim)))
    pos = np.arange(seq_len, dtype=np.float32)[:, None]
    ang = (pos * theta[None, :]).astype(np.float32)
    s, c = np.sin(ang).astype(np.float32), np.cos(ang).astype(np.float32)
    if full:
        s = np.concatenate([s, s], axis=1)
        c = np.concatenate([c, c], axis=1)
    return s, c


# ------------------------------------------------------------------ GEMM --


def gemm_f64(a, b, dt, c=None, alpha=1.0, beta=0.0, magnitude=False):
    """The unrounded value of gemm() in float64: alpha * sum_k a[..., m, k] *
    b[..., k, n] + beta * c (beta == 0 ignores c).  With magnitude=True also
    returns |alpha| * sum_k |a b| + |beta| |c|, the quantity that bounds any
    fp32 summation order's error (Higham, Accuracy and Stability of Numerical
    Algorithms, 2nd ed., eq. 4.4: |error| <= (n - 1) u sum |x_i|)."""
    af = to_compute(a, dt).astype(np.float64)
    bf = to_compute(b, dt).astype(np.float64)
    out = np.float64(alpha) * np.matmul(af, bf)
    mag = np.abs(np.float64(alpha)) * np.matmul(np.abs(af), np.abs(bf)) if magnitude else None
    if c is not None and beta != 0:
        cf = np.float64(beta) * to_compute(c, dt).astype(np.float64)
        out = out + cf
        if magnitude:
            mag = mag + np.abs(cf)
    return (out, mag) if magnitude else out


def gemm(a, b, dt, c=None, alpha=1.0, beta=0.0):
    """kernels/mm.py:54-65, kernels/bmm.py:26-39, kernels/addmm.py:64-67 --
    acc = sum_k a[..., m, k] * b[..., k, n] accumulated at (at least) fp32
    precision (here fp64, exact enough to bound the kernel's fp32 summation
    error), out = alpha * acc + beta * c rounded once to dt.  beta == 0
    ignores c."""
    out = gemm_f64(a, b, dt, c, alpha, beta)
    return round_to(out.astype(np.float32) if dt != "f64" else out, dt)


# ---------------------------------------------------------------- attention


@_with_errstate
def scaled_dot_product_attention(q, k, v, dt, mask=None, mask_dt=None, causal=0, scale=None, round_p=False):
    """kernels/scaled_dot_product_attention.py:154-201 (an online, base-2
    softmax over key blocks) restated as its closed form, in float64:
    out = softmax(q k^T * scale + mask) v per (batch, query head), with query
    head h reading key / value head h // (Hq // Hkv) (GQA,
    torch/scaled_dot_product_attention.py:33-45).  mask: None, bool (True =
    attend) or additive float of mask_dt, broadcast to (B, Hq, Sq, Skv).
    causal: 0 none, 1 upper-left (j <= i), 2 lower-right (j <= i + Skv - Sq).
    scale defaults to 1 / sqrt(D).  A row with every key masked gives 0, as
    torch's CPU kernel does (the reference's loop would give NaN).  Inputs are
    (B, H, S, D) arrays of dt; the result is rounded to dt once.

    round_p: the probabilities enter P @ V rounded to dt, as the reference's
    `ntl.dot(stable_qk.to(value[i].dtype), value[j])` (line 196) and the
    matrix-core kernels do, while the denominator sums them unrounded (its
    `lse`, line 198).  They are rounded relative to the row's exact max; a
    blockwise kernel rounds exp2(s - m) for its running or reference max m,
    which rounds the same up to a power-of-two rescaling."""
    qf = to_compute(q, dt).astype(np.float64)
    kf = to_compute(k, dt).astype(np.float64)
    vf = to_compute(v, dt).astype(np.float64)
    B, Hq, Sq, D = qf.shape
    Hkv, Skv = kf.shape[1], kf.shape[2]
    rep = Hq // Hkv
    kf = np.repeat(kf, rep, axis=1)
    vf = np.repeat(vf, rep, axis=1)
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    sc = np.matmul(qf, kf.swapaxes(-1, -2)) * scale
    allowed = np.ones(sc.shape, dtype=bool)
    if mask is not None:
        m = np.broadcast_to(np.asarray(mask), sc.shape)
        if m.dtype == np.bool_:
            allowed &= m
        else:
            sc = sc + to_compute(m, mask_dt).astype(np.float64)
    if causal:
        off = Skv - Sq if causal == 2 else 0
        i = np.arange(Sq)[:, None]
        j = np.arange(Skv)[None, :]
        allowed &= (j <= i + off)[None, None]
    sc = np.where(allowed, sc, -np.inf)
    mx = np.max(sc, axis=-1, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    p = np.exp(sc - mx)
    den = np.sum(p, axis=-1, keepdims=True)
    if round_p and dt != "f32" and dt != "f64":
        p = to_compute(round_to(p.astype(np.float32), dt), dt).astype(np.float64)
    out = np.matmul(p, vf) / np.where(den > 0, den, 1.0)
    out = np.where(den > 0, out, 0.0)
    return round_to(out.astype(np.float32) if dt != "f64" else out, dt)


def conv2d(x, w, dt, bias=None, stride=(1, 1), pad=(0, 0), dilation=(1, 1), out_hw=None):
    """kernels/conv2d.py:12-104 (the padded input unfolded with the given
    stride and dilation, times the flattened weight, fp32 product plus bias,
    lines 102-104) with the output size of torch/pooling.py:4-19, restated
    directly in float64: out[n, k, p, q] = bias[k] + sum_{c, r, s}
    x[n, c, p*sh - ph + r*dh, q*sw - pw + s*dw] * w[k, c, r, s], zero outside
    the image, rounded to dt once.  x (N, C, H, W), w (K, C, R, S), bias (K,)
    or None, all of dt.  pad is the top / left padding; out_hw overrides the
    symmetric-padding output size (asymmetric 'same' padding)."""
    xf = to_compute(x, dt).astype(np.float64)
    wf = to_compute(w, dt).astype(np.float64)
    N, C, H, W = xf.shape
    K, _, R, S = wf.shape
    sh, sw = stride
    ph, pw = pad
    dh, dw = dilation
    if out_hw is None:
        P = (H + 2 * ph - dh * (R - 1) - 1) // sh + 1
        Q = (W + 2 * pw - dw * (S - 1) - 1) // sw + 1
    else:
        P, Q = out_hw
    # zero-pad far enough on every side for every tap of every output
    hb = max(0, (P - 1) * sh - ph + (R - 1) * dh + 1 - H)
    wb = max(0, (Q - 1) * sw - pw + (S - 1) * dw + 1 - W)
    xp = np.zeros((N, C, ph + H + hb, pw + W + wb))
    xp[:, :, ph:ph + H, pw:pw + W] = xf
    out = np.zeros((N, K, P, Q))
    for r in range(R):
        for s in range(S):
            tap = xp[:, :, r * dh: r * dh + sh * (P - 1) + 1: sh, s * dw: s * dw + sw * (Q - 1) + 1: sw]
            out += np.einsum("ncpq,kc->nkpq", tap, wf[:, :, r, s], optimize=True)
    if bias is not None:
        out += to_compute(bias, dt).astype(np.float64)[None, :, None, None]
    return round_to(out.astype(np.float32) if dt != "f64" else out, dt)


def im2col(x, kernel_size, dilation=(1, 1), padding=(0, 0), stride=(1, 1)):
    """kernels/im2col.py:10-80 (the input padded by `padding` on both sides
    of each spatial axis, tiled into kernel_size windows with the given
    strides and dilation in floor mode, each window's (c, r, s) elements
    laid out along the output's middle axis) with the output size of
    torch/im2col.py:28-31:

        out[n, (c * kh + r) * kw + s, p * ow + q]
            = xpad[n, c, p * sh + r * dh, q * sw + s * dw]

    where xpad is x with ph zero rows above and below and pw zero columns left
    and right.  Pure data movement: any dtype, bf16 as its uint16 bits."""
    x = np.asarray(x)
    N, C, H, W = x.shape
    kh, kw = kernel_size
    dh, dw = dilation
    ph, pw = padding
    sh, sw = stride
    oh = (H + 2 * ph - dh * (kh - 1) - 1) // sh + 1
    ow = (W + 2 * pw - dw * (kw - 1) - 1) // sw + 1
    xp = np.zeros((N, C, H + 2 * ph, W + 2 * pw), dtype=x.dtype)
    xp[:, :, ph:ph + H, pw:pw + W] = x
    out = np.empty((N, C, kh, kw, oh, ow), dtype=x.dtype)
    for r in range(kh):
        for s in range(kw):
            out[:, :, r, s] = xp[:, :, r * dh: r * dh + sh * (oh - 1) + 1: sh, s * dw: s * dw + sw * (ow - 1) + 1: sw]
    return out.reshape(N, C * kh * kw, oh * ow)


def add_rms_norm(x, residual, dt, cols, weight=None, eps=None, w_dt=None):
    """No ntops counterpart: the composition add (kernels/add.py:10, alpha 1)
    then rms_norm (kernels/rms_norm.py:10-20) that the fused kernel computes in
    one pass.  Returns (rms_norm(h), h) with h = x + residual rounded to dt."""
    h = add(x, residual, dt)
    return rms_norm(h, dt, cols, weight, eps, w_dt), h


def rotary_position_embedding_qk(q, k, sin_table, cos_table, dt, interleaved=True):
    """No ntops counterpart: kernels/rotary_position_embedding.py:6-47 applied
    to q and to k with the same tables (two calls of
    rotary_position_embedding).  Returns (q_out, k_out)."""
    return (rotary_position_embedding(q, sin_table, cos_table, dt, interleaved),
            rotary_position_embedding(k, sin_table, cos_table, dt, interleaved))
