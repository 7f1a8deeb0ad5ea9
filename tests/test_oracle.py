"""Pins the CPU oracle (oracle/ops.py) -- runs on the CPU, no GPU needed.

Each oracle function is checked three independent ways:
  1. golden vectors written by torch CPU (tests/golden/golden.npz), the
     reference the configs name;
  2. closed forms, invariants and brute force that a plausible mistake (a
     dropped term, a wrong sign or index, a transposed operand) breaks;
  3. planted mistakes: mutated copies of the oracle must fail the checks of 2.
"""

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops as O
from tests.helpers import TOL_ELEMENTWISE, TOL_GEMM, TOL_REDUCTION, from_np

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
FDTS = ("f32", "f16", "bf16")


def close(a, b, dt, tol, what):
    rtol, atol = tol[dt]
    ta, tb = from_np(a, dt).double(), from_np(b, dt).double()
    torch.testing.assert_close(ta, tb, rtol=rtol, atol=atol, equal_nan=True, msg=lambda m: f"{what}: {m}")


def equal(a, b, dt, what):
    ta, tb = from_np(a, dt), from_np(b, dt)
    both_nan = torch.isnan(ta.double()) & torch.isnan(tb.double()) if dt in FDTS else torch.zeros_like(ta, dtype=torch.bool)
    diff = (ta != tb) & ~both_nan
    assert not diff.any(), f"{what}: {diff.sum().item()} elements differ"


# ---------------------------------------------------------- golden vectors


@pytest.mark.parametrize("dt", FDTS)
def test_golden_unary(dt):
    x = GOLD[f"unary_{dt}_x"]
    close(O.silu(x, dt), GOLD[f"silu_{dt}"], dt, TOL_ELEMENTWISE, "silu")
    # Element 2 is +inf: torch's vectorised CPU erf yields NaN there, while
    # x * 0.5 * (1 + erf(x / sqrt 2)) is +inf (torch's scalar and GPU paths,
    # and the oracle, give +inf).
    g = O.gelu(x, dt)
    assert np.isinf(from_np(g, dt)[2].item()) and from_np(g, dt)[2].item() > 0
    keep = np.ones(x.shape, bool)
    keep[2] = False
    close(g[keep], GOLD[f"gelu_{dt}"][keep], dt, TOL_ELEMENTWISE, "gelu")
    close(O.gelu(x, dt, "tanh"), GOLD[f"gelu_tanh_{dt}"], dt, TOL_ELEMENTWISE, "gelu tanh")
    close(O.exp(x, dt), GOLD[f"exp_{dt}"], dt, TOL_ELEMENTWISE, "exp")
    if dt != "f32":
        # 16-bit outputs: the single fp32 evaluation rounds to the same bits
        equal(O.exp(x, dt), GOLD[f"exp_{dt}"], dt, "exp bits")


@pytest.mark.parametrize("dt", FDTS)
def test_golden_binary_float(dt):
    x, y = GOLD[f"unary_{dt}_x"], GOLD[f"binary_{dt}_y"]
    # torch's CPU add runs a vectorised bulk (alpha*b + a with one rounding,
    # what the oracle and the kernel do) and a scalar tail over the last
    # n % 32 elements that rounds alpha*b to the 16-bit type first; compare
    # the bulk bit for bit and the tail within tolerance.
    bulk = (x.size // 32) * 32
    got = O.add(x, y, dt, -0.3)
    equal(got[:bulk], GOLD[f"add_{dt}"][:bulk], dt, "add")
    close(got[bulk:], GOLD[f"add_{dt}"][bulk:], dt, TOL_ELEMENTWISE, "add tail")
    equal(O.add(x, 0.1, dt, 0.7), GOLD[f"add_scalar_{dt}"], dt, "add scalar")
    equal(O.mul(x, y, dt), GOLD[f"mul_{dt}"], dt, "mul")
    equal(O.mul(x, 0.1, dt), GOLD[f"mul_scalar_{dt}"], dt, "mul scalar")


@pytest.mark.parametrize("dt", ("i8", "i16", "i32", "i64"))
def test_golden_integer(dt):
    a, b = GOLD[f"int_{dt}_a"], GOLD[f"int_{dt}_b"]
    np.testing.assert_array_equal(O.bitwise_and(a, b, dt), GOLD[f"and_{dt}"])
    np.testing.assert_array_equal(O.bitwise_or(a, b, dt), GOLD[f"or_{dt}"])
    np.testing.assert_array_equal(O.bitwise_not(a, dt), GOLD[f"not_{dt}"])
    np.testing.assert_array_equal(O.add(a, b, dt, 3), GOLD[f"iadd_{dt}"])
    np.testing.assert_array_equal(O.mul(a, b, dt), GOLD[f"imul_{dt}"])


def test_golden_bool():
    a, b = GOLD["bool_a"], GOLD["bool_b"]
    np.testing.assert_array_equal(O.bitwise_and(a, b, "bool"), GOLD["and_bool"])
    np.testing.assert_array_equal(O.bitwise_or(a, b, "bool"), GOLD["or_bool"])
    np.testing.assert_array_equal(O.bitwise_not(a, "bool"), GOLD["not_bool"])


@pytest.mark.parametrize("dt", FDTS)
def test_golden_norms(dt):
    x, w, b = GOLD[f"norm_{dt}_x"], GOLD[f"norm_{dt}_w"], GOLD[f"norm_{dt}_b"]
    close(O.rms_norm(x, dt, 256, w, 1e-6), GOLD[f"rms_{dt}"], dt, TOL_REDUCTION, "rms_norm")
    close(O.rms_norm(x, dt, 256, None, None), GOLD[f"rms_noweight_epsnone_{dt}"], dt, TOL_REDUCTION, "rms_norm eps=None")
    if dt != "f32":
        # the eps=None default (finfo(float32).eps) is visible in the 16-bit
        # bits: ntops' finfo(dtype).eps changes about three quarters of them
        equal(O.rms_norm(x, dt, 256, None, None), GOLD[f"rms_noweight_epsnone_{dt}"], dt, "rms_norm eps=None bits")
        equal(O.rms_norm(x, dt, 256, w, 1e-6), GOLD[f"rms_{dt}"], dt, "rms_norm bits")
    close(O.layer_norm(x, dt, 256, w, b, 1e-5), GOLD[f"ln_{dt}"], dt, TOL_REDUCTION, "layer_norm")
    close(O.layer_norm(x, dt, 256, None, None, 1e-5), GOLD[f"ln_noaffine_{dt}"], dt, TOL_REDUCTION, "layer_norm plain")


@pytest.mark.parametrize("dt", FDTS)
def test_golden_softmax(dt):
    x = GOLD[f"softmax_{dt}_x"]
    close(O.softmax(x, -1, dt), GOLD[f"softmax_{dt}"], dt, TOL_REDUCTION, "softmax")
    close(O.softmax(x, 1, dt), GOLD[f"softmax_dim1_{dt}"], dt, TOL_REDUCTION, "softmax dim=1")
    close(O.softmax(x, -1, dt, "f32"), GOLD[f"softmax_f32out_{dt}"], "f32", TOL_REDUCTION, "softmax f32 out")
    if dt != "f32":
        equal(O.softmax(x, -1, dt), GOLD[f"softmax_{dt}"], dt, "softmax bits")


@pytest.mark.parametrize("dt", FDTS)
def test_golden_rope(dt):
    x = GOLD[f"rope_{dt}_x"]
    sf, cf = GOLD[f"rope_{dt}_sin_full"], GOLD[f"rope_{dt}_cos_full"]
    si, ci = GOLD[f"rope_{dt}_sin_inter"], GOLD[f"rope_{dt}_cos_inter"]
    sh, ch = GOLD[f"rope_{dt}_sin_half"], GOLD[f"rope_{dt}_cos_half"]
    # per-op rounding reproduces torch eager bit for bit
    equal(O.rotary_position_embedding(x, sf, cf, dt, interleaved=False), GOLD[f"rope_half_{dt}"], dt, "rope half (S,D)")
    equal(O.rotary_position_embedding(x, si, ci, dt, interleaved=True), GOLD[f"rope_inter_{dt}"], dt, "rope interleaved (S,D)")
    equal(O.rotary_position_embedding(x, sh, ch, dt, interleaved=False), GOLD[f"rope_ntops_half_{dt}"], dt, "rope half (S,D/2)")
    equal(O.rotary_position_embedding(x, sh, ch, dt, interleaved=True), GOLD[f"rope_ntops_inter_{dt}"], dt, "rope interleaved (S,D/2)")


@pytest.mark.parametrize("dt", FDTS)
def test_golden_gemm(dt):
    a, b = GOLD[f"mm_{dt}_a"], GOLD[f"mm_{dt}_b"]
    close(O.gemm(a, b, dt), GOLD[f"mm_{dt}"], dt, TOL_GEMM, "mm")
    close(O.gemm(a, b, dt, GOLD[f"mm_{dt}_bias"], 1.0, 1.0), GOLD[f"addmm_bias_{dt}"], dt, TOL_GEMM, "addmm bias")
    close(O.gemm(a, b, dt, GOLD[f"mm_{dt}_c"], -1.5, 0.5), GOLD[f"addmm_full_{dt}"], dt, TOL_GEMM, "addmm full")
    close(O.gemm(GOLD[f"bmm_{dt}_a"], GOLD[f"bmm_{dt}_b"], dt), GOLD[f"bmm_{dt}"], dt, TOL_GEMM, "bmm")


# ------------------------------------------------------ live torch CPU ---


@pytest.mark.parametrize("dt", ("bf16", "f16"))
def test_live_torch_config_shapes_small(dt):
    """Same draw as the bench configs, cut to a few rows: bit-level agreement
    with torch CPU on the 16-bit paths."""
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16}[dt]
    g = torch.Generator().manual_seed(0)
    x = torch.randn(32, 4096, generator=g).to(tdt)
    w = (1 + 0.02 * torch.randn(4096, generator=g)).to(tdt)
    ref = F.rms_norm(x, (4096,), w, 1e-6)
    got = from_np(O.rms_norm(x.view(torch.int16).numpy().view(np.uint16) if dt == "bf16" else x.numpy(), dt, 4096,
                             w.view(torch.int16).numpy().view(np.uint16) if dt == "bf16" else w.numpy(), 1e-6), dt)
    mism = (got != ref).float().mean().item()
    assert mism < 1e-3, f"rms_norm bit mismatch fraction {mism}"


# --------------------------------------- closed forms, invariants, brute force


def pin_silu(fn):
    x = np.array([0.0, 20.0, -20.0, 1.0, -1.0, 3.5], dtype=np.float64)
    y = fn(x, "f64")
    ok = y[0] == 0.0 and abs(y[1] - 20.0) < 1e-6 and abs(y[2]) < 1e-7
    # silu(x) - silu(-x) = x
    ok = ok and abs((y[3] - y[4]) - 1.0) < 1e-12
    ok = ok and abs(y[5] - 3.5 / (1 + np.exp(-3.5))) < 1e-12
    return bool(ok)


def pin_gelu(fn):
    x = np.linspace(-4, 4, 81, dtype=np.float64)
    y = fn(x, "f64")
    odd = np.abs((y - y[::-1]) - x).max() < 1e-12  # gelu(x) - gelu(-x) = x
    ref_at_1 = 0.5 * (1 + 0.8427007929497149)  # erf(1/sqrt2)... gelu(sqrt2) / sqrt2
    val = fn(np.array([np.sqrt(2.0)]), "f64")[0]
    return bool(odd and abs(val - np.sqrt(2.0) * ref_at_1) < 1e-12 and fn(np.array([0.0]), "f64")[0] == 0)


def pin_exp(fn):
    a = np.linspace(-5, 5, 41)
    ok = np.allclose(fn(a, "f64") * fn(-a, "f64"), 1.0, rtol=1e-14)
    return bool(ok and fn(np.array([0.0]), "f64")[0] == 1.0 and abs(fn(np.array([1.0]), "f64")[0] - np.e) < 1e-15)


def pin_add(fn):
    a = np.arange(-50, 50, dtype=np.float32)
    b = np.arange(100, 0, -1, dtype=np.float32)
    exact = a.astype(np.float64) + 3.0 * b.astype(np.float64)
    ok = np.array_equal(fn(a, b, "f32", 3).astype(np.float64), exact)
    ai = np.array([127, -128, 5], dtype=np.int8)
    bi = np.array([1, -1, 3], dtype=np.int8)
    ok = ok and np.array_equal(fn(ai, bi, "i8", 2), np.array([-127, 126, 11], dtype=np.int8))  # wraps
    return bool(ok)


def pin_rms(fn):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((8, 64)).astype(np.float32)
    y1 = fn(x, "f32", 64, None, 0.0)
    y2 = fn(x * np.float32(4), "f32", 64, None, 0.0)  # scale invariant, exactly
    rms = np.sqrt(np.mean(y1.astype(np.float64) ** 2, axis=1))
    const = fn(np.full((1, 64), 0.5, np.float32), "f32", 64, None, 0.25)  # 0.5/sqrt(0.25+0.25)
    w = np.arange(64, dtype=np.float32) / 64
    yw = fn(x, "f32", 64, w, 0.0)
    ok = bool(np.array_equal(y1, y2) and np.allclose(rms, 1.0, atol=1e-6)
              and np.allclose(const, 0.5 / np.sqrt(0.5), rtol=1e-7)
              and np.allclose(yw, y1 * w, rtol=1e-6, atol=1e-7))
    # eps=None is finfo(float32).eps = 2^-23 for every input dtype: a constant
    # 16-bit row of 2^-12 has mean square 2^-24, so y = 2^-12 / sqrt(3 * 2^-24)
    # = 1 / sqrt(3); finfo(bf16).eps (2^-7) or finfo(f16).eps (2^-10) would
    # give 0.003 or 0.008
    for dt in ("bf16", "f16"):
        tiny = O.round_to(np.full((2, 64), 2.0 ** -12, np.float32), dt)
        yt = O.to_compute(fn(tiny, dt, 64, None, None), dt)
        ok = ok and bool(np.allclose(yt, 1 / np.sqrt(3), rtol=2.0 ** -8, atol=0))
    return ok


def pin_layer_norm(fn):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((8, 128)).astype(np.float32)
    y = fn(x, "f32", 128, None, None, 0.0).astype(np.float64)
    ok = np.allclose(y.mean(1), 0, atol=1e-6) and np.allclose(y.var(1), 1, atol=1e-5)
    b = np.linspace(-1, 1, 128).astype(np.float32)
    ok = ok and np.allclose(fn(np.full((2, 128), 3.0, np.float32), "f32", 128, None, b, 1e-5), b[None, :], atol=1e-7)
    ys = fn(x + np.float32(8), "f32", 128, None, None, 0.0)
    return bool(ok and np.allclose(ys, y, atol=2e-5))


def pin_softmax(fn):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((6, 33)).astype(np.float32)
    y = fn(x, -1, "f32").astype(np.float64)
    ok = np.allclose(y.sum(-1), 1, atol=1e-6)
    ok = ok and np.allclose(fn(x + np.float32(64), -1, "f32"), y, atol=1e-6)  # shift invariance
    two = fn(np.array([[0.0, np.log(3.0)]], np.float64), -1, "f64")
    ok = ok and np.allclose(two, [[0.25, 0.75]], rtol=1e-14)
    causal = np.where(np.triu(np.ones((4, 4), bool), 1), -np.inf, rng.standard_normal((4, 4))).astype(np.float32)
    yc = fn(causal, -1, "f32")
    ok = ok and yc[0, 0] == 1.0 and np.all(yc[0, 1:] == 0)
    ok = ok and np.all(np.isnan(fn(np.full((1, 5), -np.inf, np.float32), -1, "f32")))
    y0 = fn(x, 0, "f32").astype(np.float64)
    return bool(ok and np.allclose(y0.sum(0), 1, atol=1e-6))


def pin_rope(fn):
    rng = np.random.default_rng(3)
    B, S, H, D = 1, 4, 2, 8
    x = rng.standard_normal((B, S, H, D)).astype(np.float32)
    ang = rng.uniform(-3, 3, (S, D // 2)).astype(np.float32)
    s, c = np.sin(ang).astype(np.float32), np.cos(ang).astype(np.float32)
    ok = True
    for inter in (False, True):
        y = fn(x, s, c, "f32", interleaved=inter).astype(np.float64)
        i0 = np.arange(0, D, 2) if inter else np.arange(D // 2)
        i1 = i0 + 1 if inter else i0 + D // 2
        n_in = x[..., i0].astype(np.float64) ** 2 + x[..., i1].astype(np.float64) ** 2
        n_out = y[..., i0] ** 2 + y[..., i1] ** 2
        ok = ok and np.allclose(n_in, n_out, rtol=1e-5)  # rotation keeps pair norms
        # a rotation by +90 degrees: (x0, x1) -> (-x1, x0) exactly
        y90 = fn(x, np.ones_like(s), np.zeros_like(c), "f32", interleaved=inter)
        ok = ok and np.array_equal(y90[..., i0], -x[..., i1]) and np.array_equal(y90[..., i1], x[..., i0])
        # angle 0 is the identity
        ok = ok and np.array_equal(fn(x, np.zeros_like(s), np.ones_like(c), "f32", interleaved=inter), x)
    # interleaved == half-rotation after permuting pairs
    perm = np.concatenate([np.arange(0, D, 2), np.arange(1, D, 2)])
    yi = fn(x, s, c, "f32", interleaved=True)
    yh = fn(x[..., perm], s, c, "f32", interleaved=False)
    return bool(ok and np.array_equal(yi[..., perm], yh))


def pin_gemm(fn):
    rng = np.random.default_rng(4)
    a = rng.integers(-2, 3, (3, 17, 64)).astype(np.float32)
    b = rng.integers(-2, 3, (3, 64, 9)).astype(np.float32)
    exact = np.einsum("bmk,bkn->bmn", a.astype(np.int64), b.astype(np.int64))
    ok = np.array_equal(fn(a, b, "f32").astype(np.int64), exact)
    ok = ok and np.array_equal(fn(np.swapaxes(b, 1, 2), np.swapaxes(a, 1, 2), "f32"), np.swapaxes(fn(a, b, "f32"), 1, 2))
    c = np.full((17, 9), np.nan, np.float32)
    ok = ok and np.array_equal(fn(a[0], b[0], "f32", c, 1.0, 0.0), fn(a[0], b[0], "f32"))  # beta=0 ignores c
    bias = np.arange(9, dtype=np.float32)
    ok = ok and np.array_equal(fn(a[0], b[0], "f32", bias, 2.0, 1.0), 2 * exact[0] + bias)
    return bool(ok)


PINS = {
    "silu": pin_silu,
    "gelu": pin_gelu,
    "exp": pin_exp,
    "add": pin_add,
    "rms_norm": pin_rms,
    "layer_norm": pin_layer_norm,
    "softmax": pin_softmax,
    "rotary_position_embedding": pin_rope,
    "gemm": pin_gemm,
}


@pytest.mark.parametrize("name", sorted(PINS))
def test_closed_forms(name):
    assert PINS[name](getattr(O, name)), f"oracle {name} fails its closed-form pins"


def test_bitwise_exhaustive_int8():
    a = np.repeat(np.arange(-128, 128, dtype=np.int8), 256)
    b = np.tile(np.arange(-128, 128, dtype=np.int8), 256)
    pa = [int(v) for v in a]
    pb = [int(v) for v in b]
    exp_and = np.array([x & y for x, y in zip(pa, pb)], dtype=np.int8)
    exp_or = np.array([x | y for x, y in zip(pa, pb)], dtype=np.int8)
    np.testing.assert_array_equal(O.bitwise_and(a, b, "i8"), exp_and)
    np.testing.assert_array_equal(O.bitwise_or(a, b, "i8"), exp_or)
    np.testing.assert_array_equal(O.bitwise_not(a[:256], "i8"), np.array([~x for x in pa[:256]], np.int8))
    t, f = True, False
    tt = np.array([t, t, f, f]), np.array([t, f, t, f])
    np.testing.assert_array_equal(O.bitwise_and(*tt, "bool"), [t, f, f, f])
    np.testing.assert_array_equal(O.bitwise_or(*tt, "bool"), [t, t, t, f])
    np.testing.assert_array_equal(O.bitwise_not(tt[0], "bool"), [f, f, t, t])


def test_bf16_rounding_special_cases():
    f = np.array([1.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, np.inf, -np.inf, np.nan, -0.0, 3.0e38], np.float32)
    u = O.f32_to_bf16(f)
    assert u[0] == 0x3F80
    assert u[1] == 0x3F80  # tie -> even
    assert u[2] == 0x3F82  # tie -> even (up)
    assert u[3] == 0x7F80 and u[4] == 0xFF80 and u[5] == 0x7FC0 and u[6] == 0x8000
    assert u[7] == 0x7F62  # 3.0e38 rounds to the nearest bf16 below the max
    assert np.array_equal(O.bf16_to_f32(u[:3]), np.array([1.0, 1.0, 1.0 + 2**-6], np.float32))


# ---------------------------------------------------------- planted mistakes


def _mutant_rope_sign(x, s, c, dt, interleaved=True):
    return O.rotary_position_embedding(x, -np.asarray(s), c, dt, interleaved)


def _mutant_rope_index(x, s, c, dt, interleaved=True):
    return O.rotary_position_embedding(x, s, c, dt, not interleaved)


def _mutant_rms_no_mean(x, dt, cols, weight=None, eps=None, w_dt=None):
    return O.rms_norm(x, dt, cols, weight, eps, w_dt) / np.sqrt(np.float32(cols))


def _mutant_rms_eps_outside(x, dt, cols, weight=None, eps=None, w_dt=None):
    y = O.rms_norm(x, dt, cols, weight, 0.0, w_dt)
    return y + np.float32(eps or 0)


def _mutant_rms_eps_of_dtype(x, dt, cols, weight=None, eps=None, w_dt=None):
    # ntops' own default, finfo(input dtype).eps, in place of finfo(float32).eps
    if eps is None:
        eps = {"f32": 2.0 ** -23, "bf16": 2.0 ** -7, "f16": 2.0 ** -10}[dt]
    return O.rms_norm(x, dt, cols, weight, eps, w_dt)


def _mutant_gemm_transposed(a, b, dt, c=None, alpha=1.0, beta=0.0):
    if np.ndim(a) == 2 and a.shape[0] == a.shape[1]:
        a = a.T
    out = O.gemm(a, b, dt, c, alpha, beta)
    return out if c is None or beta == 0 else out + np.float32(beta) * 0  # drop nothing else


def _mutant_gemm_drop_bias(a, b, dt, c=None, alpha=1.0, beta=0.0):
    return O.gemm(a, b, dt, None, alpha, 0.0)


def _mutant_softmax_no_max(x, dim, in_dt, out_dt=None):
    y = O.softmax(x, dim, in_dt, out_dt)
    return y * 1.0001


def _mutant_ln_no_mean(x, dt, cols, weight=None, bias=None, eps=1e-5, wb_dt=None):
    xf = np.asarray(x, np.float32)
    return O.rms_norm(xf, dt, cols, None, eps) if weight is None else O.rms_norm(xf, dt, cols, weight, eps)


def _mutant_silu_sign(x, dt):
    return O.silu(-np.asarray(x), dt) * -1


def _mutant_add_alpha_on_a(a, b, dt, alpha=1):
    return O.add(b, a, dt, alpha)


@pytest.mark.parametrize(
    "name,mutant",
    [
        ("rotary_position_embedding", _mutant_rope_sign),
        ("rotary_position_embedding", _mutant_rope_index),
        ("rms_norm", _mutant_rms_no_mean),
        ("rms_norm", _mutant_rms_eps_outside),
        ("rms_norm", _mutant_rms_eps_of_dtype),
        ("gemm", _mutant_gemm_drop_bias),
        ("softmax", _mutant_softmax_no_max),
        ("layer_norm", _mutant_ln_no_mean),
        ("silu", _mutant_silu_sign),
        ("add", _mutant_add_alpha_on_a),
    ],
)
def test_planted_mistakes_are_caught(name, mutant):
    assert not PINS[name](mutant), f"a planted mistake in {name} went unnoticed"


@pytest.mark.parametrize("dt", ("f32", "bf16"))
def test_norm_params_expand_like_the_reference(dt):
    """Weights / biases broadcast against the input (the reference's
    `expand_as(input)`): each row must equal the one-row computation (pinned
    by the golden vectors above) with that row of the expanded parameter --
    a per-row weight, a (6, 1) weight constant along the row, and a (32,)
    weight broadcast inside a 2-D normalized shape."""
    rng = np.random.default_rng(11)

    def arr(*shape, scale=1.0, shift=0.0):
        return O.round_to(rng.standard_normal(shape).astype(np.float32) * scale + shift, dt)

    x = arr(4, 6, 32)
    cases = (arr(4, 6, 32, scale=0.1, shift=1.0), arr(6, 1, scale=0.1, shift=1.0), arr(1, 6, 32, scale=0.1))
    for w in cases:
        wf = np.broadcast_to(O.to_compute(w, dt), x.shape)
        got = O.rms_norm(x, dt, 32, w, 1e-6).reshape(24, 32)
        b = arr(6, 1, scale=0.1)
        got_ln = O.layer_norm(x, dt, 32, w, b, 1e-5).reshape(24, 32)
        bf = np.broadcast_to(O.to_compute(b, dt), x.shape)
        for i in range(4):
            for j in range(6):
                wr = O.round_to(wf[i, j], dt)
                np.testing.assert_array_equal(got[6 * i + j], O.rms_norm(x[i, j][None], dt, 32, wr, 1e-6)[0])
                br = O.round_to(bf[i, j], dt)
                np.testing.assert_array_equal(got_ln[6 * i + j], O.layer_norm(x[i, j][None], dt, 32, wr, br, 1e-5)[0])
    # a (32,) weight over normalized_shape (6, 32): the same 32 values in every
    # 32-element run of each 192-element row
    w = arr(32, scale=0.1, shift=1.0)
    got = O.rms_norm(x, dt, 192, w, 1e-6)
    tiled = O.round_to(np.tile(O.to_compute(w, dt), 6), dt)
    np.testing.assert_array_equal(got.reshape(4, 192), O.rms_norm(x.reshape(4, 192), dt, 192, tiled, 1e-6))
