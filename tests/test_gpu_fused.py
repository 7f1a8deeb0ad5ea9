"""GPU parity: the fused variants against the unfused ntops kernels (element
for element) and against the oracle composition.

add_rms_norm: every register-resident row width, the looped fallback (odd and
very wide rows), weight None / of the dtype / fp32, eps None / values,
in-place, multi-dim normalized_shape, and the (16384, 4096) bf16 config.
rotary_position_embedding_qk: grouped-query head counts, both pair layouts,
(S, D/2) and (S, D) tables, strided q / k, in-place, a key with no heads,
and q / k of the (4, 4096, 32, 128) bf16 config."""

import pytest
import torch

import ntops_amd
from oracle import ops as O
from tests.helpers import DT_NAME, TOL_REDUCTION, assert_close, assert_equal, from_np, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

T = ntops_amd.torch
FLOATS = (torch.float32, torch.float16, torch.bfloat16)
# rows x cols: each vector row configuration, then looped (odd / > 64K) widths
ARN_SHAPES = [(3, 8), (5, 64), (7, 512), (9, 1024), (6, 2048), (4, 4096), (3, 8192), (2, 16384), (2, 32768),
              (33, 4096), (5, 100), (3, 70001)]


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("shape", ARN_SHAPES)
@pytest.mark.parametrize("wmode", ("none", "same", "f32"))
def test_add_rms_norm(shape, dtype, wmode):
    g = torch.Generator().manual_seed(shape[0] * 100003 + shape[1])
    x = torch.randn(shape, generator=g).to(dtype)
    r = torch.randn(shape, generator=g).to(dtype)
    w = None if wmode == "none" else (1 + 0.1 * torch.randn(shape[1], generator=g)).to(
        torch.float32 if wmode == "f32" else dtype)
    eps = None if wmode == "none" else 1e-6
    xg, rg = x.cuda(), r.cuda()
    wg = None if w is None else w.cuda()
    y, h = T.add_rms_norm(xg, rg, (shape[1],), wg, eps)
    # the unfused kernels
    h2 = T.add(xg, rg)
    y2 = T.rms_norm(h2, (shape[1],), wg, eps)
    assert_equal(h, h2, "new residual vs add")
    assert_equal(y, y2, "output vs add + rms_norm")
    # the oracle composition
    dt = DT_NAME[dtype]
    ey, eh = O.add_rms_norm(to_np(x), to_np(r), dt, shape[1], None if w is None else to_np(w), eps,
                            None if w is None else DT_NAME[w.dtype])
    assert_equal(h, from_np(eh, dt), "new residual vs oracle")
    assert_close(y, from_np(ey, dt), *TOL_REDUCTION[dt], "output vs oracle")


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float32))
def test_add_rms_norm_forms(dtype):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 3, 8, 256, generator=g).to(dtype)
    r = torch.randn(2, 3, 8, 256, generator=g).to(dtype)
    w = torch.randn(8, 256, generator=g).to(dtype)
    y, h = T.add_rms_norm(x.cuda(), r.cuda(), (8, 256), w.cuda(), 1e-5)
    h2 = T.add(x.cuda(), r.cuda())
    assert_equal(y, T.rms_norm(h2, (8, 256), w.cuda(), 1e-5), "2-d normalized_shape")
    # in place: the new residual lands in `residual`, the output in `input`
    xi, ri = x.cuda(), r.cuda()
    yi, hi = T.add_rms_norm(xi, ri, (8, 256), w.cuda(), 1e-5, inplace=True)
    assert yi.data_ptr() == xi.data_ptr() and hi.data_ptr() == ri.data_ptr()
    assert_equal(yi, y, "in-place output")
    assert_equal(hi, h, "in-place residual")
    # strided input is made contiguous for the out-of-place form
    xt = x.cuda().transpose(0, 1)
    rt = r.cuda().transpose(0, 1)
    y3, h3 = T.add_rms_norm(xt, rt, (8, 256), w.cuda(), 1e-5)
    assert_equal(y3, y.transpose(0, 1).contiguous(), "strided input")
    with pytest.raises(RuntimeError):
        T.add_rms_norm(x.cuda(), r.cuda()[:1], (8, 256))


def test_add_rms_norm_config_full_size():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(16384, 4096, generator=g).bfloat16().cuda()
    r = torch.randn(16384, 4096, generator=g).bfloat16().cuda()
    w = (1 + 0.02 * torch.randn(4096, generator=g)).bfloat16().cuda()
    y, h = T.add_rms_norm(x, r, (4096,), w, 1e-6)
    h2 = T.add(x, r)
    assert_equal(h, h2, "config residual")
    assert_equal(y, T.rms_norm(h2, (4096,), w, 1e-6), "config output")


def tables(S, D, dtype, full):
    s, c = O.rope_tables(S, D, full=full)
    return torch.from_numpy(s).to(dtype), torch.from_numpy(c).to(dtype)


@pytest.mark.parametrize("dtype", FLOATS)
@pytest.mark.parametrize("interleaved", (False, True))
@pytest.mark.parametrize("full", (False, True))
@pytest.mark.parametrize("heads", ((8, 2), (4, 4), (6, 1), (3, 0)))
def test_rope_qk(heads, full, interleaved, dtype):
    hq, hk = heads
    B, S, D = 2, 48, 64
    g = torch.Generator().manual_seed(hq * 10 + hk)
    q = torch.randn(B, S, hq, D, generator=g).to(dtype)
    k = torch.randn(B, S, hk, D, generator=g).to(dtype)
    sn, cs = tables(S, D, dtype, full)
    qo, ko = T.rotary_position_embedding_qk(q.cuda(), k.cuda(), sn.cuda(), cs.cuda(), interleaved)
    assert_equal(qo, T.rotary_position_embedding(q.cuda(), sn.cuda(), cs.cuda(), interleaved), "q vs single call")
    if hk:
        assert_equal(ko, T.rotary_position_embedding(k.cuda(), sn.cuda(), cs.cuda(), interleaved), "k vs single call")
    dt = DT_NAME[dtype]
    eq, ek = O.rotary_position_embedding_qk(to_np(q), to_np(k), to_np(sn), to_np(cs), dt, interleaved)
    assert_equal(qo, from_np(eq, dt), "q vs oracle")
    assert_equal(ko, from_np(ek, dt), "k vs oracle")


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float32))
def test_rope_qk_layouts(dtype):
    B, S, Hq, Hk, D = 2, 40, 8, 2, 128
    g = torch.Generator().manual_seed(1)
    sn, cs = (t.cuda() for t in tables(S, D, dtype, False))
    # (B, H, S, D) storage viewed as (B, S, H, D): strided q and k
    qs = torch.randn(B, Hq, S, D, generator=g).to(dtype).cuda().transpose(1, 2)
    ks = torch.randn(B, Hk, S, D, generator=g).to(dtype).cuda().transpose(1, 2)
    qo, ko = T.rotary_position_embedding_qk(qs, ks, sn, cs, False)
    assert_equal(qo, T.rotary_position_embedding(qs, sn, cs, False), "strided q")
    assert_equal(ko, T.rotary_position_embedding(ks, sn, cs, False), "strided k")
    # in place
    q = torch.randn(B, S, Hq, D, generator=g).to(dtype).cuda()
    k = torch.randn(B, S, Hk, D, generator=g).to(dtype).cuda()
    eq = T.rotary_position_embedding(q, sn, cs, True)
    ek = T.rotary_position_embedding(k, sn, cs, True)
    qi, ki = T.rotary_position_embedding_qk(q, k, sn, cs, True, inplace=True)
    assert qi.data_ptr() == q.data_ptr() and ki.data_ptr() == k.data_ptr()
    assert_equal(q, eq, "in-place q")
    assert_equal(k, ek, "in-place k")
    with pytest.raises(RuntimeError):
        T.rotary_position_embedding_qk(q, k[:, :10], sn, cs)


def test_rope_qk_config_full_size():
    B, S, H, D = 4, 4096, 32, 128
    g = torch.Generator().manual_seed(0)
    q = torch.randn(B, S, H, D, generator=g).bfloat16().cuda()
    k = torch.randn(B, S, H, D, generator=g).bfloat16().cuda()
    sn, cs = (t.cuda() for t in tables(S, D, torch.bfloat16, True))
    qo, ko = T.rotary_position_embedding_qk(q, k, sn, cs, False)
    assert_equal(qo, T.rotary_position_embedding(q, sn, cs, False), "config q")
    assert_equal(ko, T.rotary_position_embedding(k, sn, cs, False), "config k")
