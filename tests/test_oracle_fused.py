"""Pins the oracle of the two fused variants -- CPU only.  Golden vectors
written by torch CPU compositions (tests/golden/golden_fused.npz): h = x +
residual bit-exact, torch.rms_norm(h) bit-exact for fp16 and bf16 and within
the fp32 reduction tolerance (1e-5; torch sums in another order) for fp32,
with and without a weight; the eager q / k rotation bit-exact for both pair
layouts.
Planted mistakes -- normalising x instead of h, returning the unrounded sum,
rotating k with q's pair layout, swapping sin and cos -- must be caught."""

import os

import numpy as np
import pytest

from oracle import ops as O

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_fused.npz"))


def arn_matches(f, dt):
    x, r, w = G[f"arn_x_{dt}"], G[f"arn_r_{dt}"], G[f"arn_w_{dt}"]
    cols = x.shape[1]
    y, h = f(x, r, dt, cols, w, 1e-6)
    ynw, _ = f(x, r, dt, cols)
    same = np.array_equal if dt != "f32" else (lambda a, b: np.allclose(a, b, rtol=1e-5, atol=1e-5))
    return (np.array_equal(h, G[f"arn_h_{dt}"]) and same(y, G[f"arn_y_{dt}"])
            and same(ynw, G[f"arn_ynw_{dt}"]))


def qk_matches(f, dt):
    q, k, sn, cs = G[f"qk_q_{dt}"], G[f"qk_k_{dt}"], G[f"qk_sin_{dt}"], G[f"qk_cos_{dt}"]
    ok = True
    for il in (0, 1):
        qo, ko = f(q, k, sn, cs, dt, bool(il))
        ok = ok and np.array_equal(qo, G[f"qk_qo{il}_{dt}"]) and np.array_equal(ko, G[f"qk_ko{il}_{dt}"])
    return ok


@pytest.mark.parametrize("dt", ("f32", "f16", "bf16"))
def test_golden(dt):
    assert arn_matches(O.add_rms_norm, dt)
    assert qk_matches(O.rotary_position_embedding_qk, dt)


def _norm_x(x, r, dt, cols, w=None, eps=None, w_dt=None):
    return O.rms_norm(x, dt, cols, w, eps, w_dt), O.add(x, r, dt)


def _unrounded(x, r, dt, cols, w=None, eps=None, w_dt=None):
    h = (O.to_compute(x, dt).astype(np.float64) + O.to_compute(r, dt)).astype(np.float32)
    return O.rms_norm(O.round_to(h, "f32") if dt == "f32" else h.astype(np.float32), "f32", cols,
                      None if w is None else O.to_compute(w, dt), eps), O.add(x, r, dt)


def _k_layout(q, k, sn, cs, dt, interleaved=True):
    return (O.rotary_position_embedding(q, sn, cs, dt, interleaved),
            O.rotary_position_embedding(k, sn, cs, dt, not interleaved))


def _swap(q, k, sn, cs, dt, interleaved=True):
    return (O.rotary_position_embedding(q, sn, cs, dt, interleaved),
            O.rotary_position_embedding(k, cs, sn, dt, interleaved))


@pytest.mark.parametrize("dt", ("f16", "bf16"))
def test_planted_mistakes_are_caught(dt):
    assert not arn_matches(_norm_x, dt)
    assert not arn_matches(_unrounded, dt)
    assert not qk_matches(_k_layout, dt)
    assert not qk_matches(_swap, dt)
