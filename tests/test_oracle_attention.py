"""Pins the scaled_dot_product_attention oracle -- CPU only.  Golden vectors
written by torch CPU (tests/golden/golden_attention.npz), closed forms that a
plausible mistake breaks (uniform keys -> mean of V, causal row 0 -> V[0], a
dominant score -> its V row, GQA = repeated key / value heads, a fully masked
row -> 0, lower-right = upper-left when Sq == Skv), and planted mistakes."""

import os

import numpy as np
import pytest
import torch

from oracle import ops as O
from tests.helpers import from_np

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_attention.npz"))
# torch's CPU kernel computes 16-bit attention with reduced-precision
# intermediates; the oracle is exact (float64) and rounds once
TOL = {"f32": (2e-6, 2e-6), "f16": (1e-2, 1e-2), "bf16": (2e-2, 2e-2)}


def close(got, exp, dt, what):
    rtol, atol = TOL[dt]
    torch.testing.assert_close(from_np(got, dt).double(), from_np(exp, dt).double(), rtol=rtol, atol=atol,
                               msg=lambda m: f"{what}: {m}")


@pytest.mark.parametrize("dt", ("f32", "f16", "bf16"))
def test_golden(dt):
    q, k, v = G[f"q_{dt}"], G[f"k_{dt}"], G[f"v_{dt}"]
    f = O.scaled_dot_product_attention
    close(f(q, k, v, dt), G[f"plain_{dt}"], dt, "plain")
    close(f(q, k, v, dt, scale=0.3), G[f"scaled_{dt}"], dt, "scale")
    close(f(q, k, v, dt, mask=G["bool_mask"]), G[f"bool_{dt}"], dt, "bool mask")
    close(f(q, k, v, dt, mask=G[f"float_mask_{dt}"], mask_dt=dt), G[f"float_{dt}"], dt, "float mask")
    close(f(q, k, v, dt, causal=1), G[f"causal_ul_{dt}"], dt, "causal upper-left")
    close(f(q, k, v, dt, causal=2), G[f"causal_lr_{dt}"], dt, "causal lower-right")
    assert (from_np(f(q, k, v, dt, mask=G["bool_mask"]), dt)[:, :, 5] == 0).all()


def pin_sdpa(f):
    rng = np.random.default_rng(0)
    B, H, S, D = 2, 3, 9, 8
    q = rng.standard_normal((B, H, S, D))
    v = rng.standard_normal((B, H, S, D))
    ok = True
    # identical keys: every query attends uniformly -> mean of V
    k_same = np.broadcast_to(rng.standard_normal((1, 1, 1, D)), (B, H, S, D)).copy()
    ok &= np.allclose(f(q, k_same, v, "f64"), np.broadcast_to(v.mean(axis=2, keepdims=True), v.shape), atol=1e-12)
    k = rng.standard_normal((B, H, S, D))
    # causal: query 0 sees only key 0
    ok &= np.allclose(f(q, k, v, "f64", causal=1)[:, :, 0], v[:, :, 0], atol=1e-12)
    # causal row i = plain attention over keys 0..i (inclusive)
    full = f(q[:, :, 5:6], k[:, :, :6], v[:, :, :6], "f64")
    ok &= np.allclose(f(q, k, v, "f64", causal=1)[:, :, 5:6], full, atol=1e-12)
    # lower-right with 4 queries over 9 keys: query i sees keys 0..i + 5
    ok &= np.allclose(f(q[:, :, :4], k, v, "f64", causal=2)[:, :, 1:2],
                      f(q[:, :, 1:2], k[:, :, :7], v[:, :, :7], "f64"), atol=1e-12)
    # causal with Sq == Skv: the two corners coincide
    ok &= np.allclose(f(q, k, v, "f64", causal=1), f(q, k, v, "f64", causal=2), atol=1e-12)
    # a dominant score picks its V row
    kd = k.copy()
    kd[:, :, 4] = q[:, :, 2] * 1e3
    ok &= np.allclose(f(q, kd, v, "f64")[:, :, 2], v[:, :, 4], atol=1e-9)
    # GQA: 6 query heads over 3 key / value heads = explicit repetition
    q6 = rng.standard_normal((B, 6, S, D))
    ok &= np.allclose(f(q6, k, v, "f64"), f(q6, np.repeat(k, 2, 1), np.repeat(v, 2, 1), "f64"), atol=1e-12)
    # against a direct two-head loop (catches a wrong head mapping)
    ref = np.empty((B, 6, S, D))
    for b in range(B):
        for h in range(6):
            s = q6[b, h] @ k[b, h // 2].T / np.sqrt(D)
            p = np.exp(s - s.max(-1, keepdims=True))
            ref[b, h] = (p / p.sum(-1, keepdims=True)) @ v[b, h // 2]
    ok &= np.allclose(f(q6, k, v, "f64"), ref, atol=1e-12)
    # fully masked row -> 0; bool False == additive -inf
    m = np.ones((S, S), bool)
    m[3] = False
    mb = f(q, k, v, "f64", mask=m)
    ok &= np.all(mb[:, :, 3] == 0)
    mf = np.where(m, 0.0, -np.inf)
    ok &= np.allclose(mb, f(q, k, v, "f64", mask=mf, mask_dt="f64"), atol=1e-12)
    return bool(ok)


def test_closed_forms():
    assert pin_sdpa(O.scaled_dot_product_attention)


def _m_gqa_modulo(q, k, v, dt, mask=None, mask_dt=None, causal=0, scale=None):
    rep = q.shape[1] // k.shape[1]
    if rep > 1:  # head h -> h % Hkv instead of h // rep
        k = np.concatenate([k] * rep, axis=1)
        v = np.concatenate([v] * rep, axis=1)
    return O.scaled_dot_product_attention(q, k, v, dt, mask, mask_dt, causal, scale)


def _m_causal_strict(q, k, v, dt, mask=None, mask_dt=None, causal=0, scale=None):
    if causal:
        S, T = q.shape[2], k.shape[2]
        m = np.arange(T)[None, :] < np.arange(S)[:, None] + (T - S if causal == 2 else 0)
        m[0, 0] = True
        return O.scaled_dot_product_attention(q, k, v, dt, m if mask is None else mask, mask_dt, 0, scale)
    return O.scaled_dot_product_attention(q, k, v, dt, mask, mask_dt, causal, scale)


def _m_no_scale(q, k, v, dt, mask=None, mask_dt=None, causal=0, scale=None):
    return O.scaled_dot_product_attention(q, k, v, dt, mask, mask_dt, causal, 1.0 if scale is None else scale)


def _m_masked_row_nan(q, k, v, dt, mask=None, mask_dt=None, causal=0, scale=None):
    out = O.scaled_dot_product_attention(q, k, v, dt, mask, mask_dt, causal, scale)
    return np.where(out == 0, np.nan, out)


@pytest.mark.parametrize("mutant", (_m_gqa_modulo, _m_causal_strict, _m_no_scale, _m_masked_row_nan))
def test_planted_mistakes_are_caught(mutant):
    assert not pin_sdpa(mutant)


def pin_round_p(f):
    """round_p: the probabilities of P @ V rounded to the dtype, the
    denominator summing them unrounded.  One key scores 0 and n keys score
    s < 0, every value row is 1: the exact output is (1 + n round(e^s)) /
    (1 + n e^s).  With e^s just below the bf16 midpoint above 0.25 (rounded
    down by almost half a step, 0.39 % relative) that is 1 - 0.39 % ->
    0.99609375 after the output's rounding, where ignoring round_p, or
    summing the rounded probabilities in the denominator too, gives exactly
    1."""
    D, n = 8, 255
    # e^s = p1 just below 0.25 + 2^-10, the midpoint above 0.25 in bf16: it
    # rounds down to 0.25 (0.39 % relative); s = -1 * scale with scale = -ln p1
    p1 = 0.25 + 2.0 ** -10 * 0.999
    scale = -np.log(p1)
    q = np.zeros((1, 1, 1, D), np.float32)
    q[..., 0] = 1.0
    k = np.zeros((1, 1, n + 1, D), np.float32)
    k[0, 0, 1:, 0] = -1.0
    v = np.ones((1, 1, n + 1, D), np.float32)
    qb, kb, vb = (O.round_to(a, "bf16") for a in (q, k, v))
    p1r = float(O.to_compute(O.round_to(np.float32(p1), "bf16"), "bf16"))
    exp = (1.0 + n * p1r) / (1.0 + n * p1)
    want = O.to_compute(O.round_to(np.full((1, 1, 1, D), exp, np.float32), "bf16"), "bf16")
    got = O.to_compute(f(qb, kb, vb, "bf16", scale=scale, round_p=True), "bf16")
    ok = bool(np.array_equal(got, want)) and bool(np.all(want < 1.0))
    # fp32 data: round_p changes nothing
    rng = np.random.default_rng(3)
    a, b, c = (rng.standard_normal((1, 2, 5, D)).astype(np.float32) for _ in range(3))
    ok &= np.array_equal(f(a, b, c, "f32", round_p=True), f(a, b, c, "f32"))
    return ok


def test_round_p_closed_form():
    assert pin_round_p(O.scaled_dot_product_attention)


def _m_round_p_ignored(q, k, v, dt, mask=None, mask_dt=None, causal=0, scale=None, round_p=False):
    return O.scaled_dot_product_attention(q, k, v, dt, mask, mask_dt, causal, scale)


def _m_round_p_denominator_too(q, k, v, dt, mask=None, mask_dt=None, causal=0, scale=None, round_p=False):
    # the denominator summing the rounded probabilities: sum(round(p)) v / sum(round(p))
    qf, kf, vf = (O.to_compute(a, dt).astype(np.float64) for a in (q, k, v))
    s = qf @ kf.swapaxes(-1, -2) * (1.0 / np.sqrt(qf.shape[-1]) if scale is None else scale)
    p = np.exp(s - s.max(-1, keepdims=True))
    if round_p:
        p = O.to_compute(O.round_to(p.astype(np.float32), dt), dt).astype(np.float64)
    return O.round_to(((p @ vf) / p.sum(-1, keepdims=True)).astype(np.float32), dt)


@pytest.mark.parametrize("mutant", (_m_round_p_ignored, _m_round_p_denominator_too))
def test_round_p_planted_mistakes_are_caught(mutant):
    assert not pin_round_p(mutant)
