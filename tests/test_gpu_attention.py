"""GPU parity: scaled_dot_product_attention through the C ABI against the
oracle.

Mirrors the reference's tests/test_scaled_dot_product_attention.py: batch
1-4, 2-32 query heads over a power-of-two divisor of key / value heads (GQA),
sequence lengths 1-512, head dim 32 / 64 (plus 128), no mask / bool / float
masks, both causal variants, random scales, the KV-cache slot write, fp32
and fp16 -- with bf16 added, edge shapes (one query, one key, fully masked
rows, Sq > Skv), strided inputs, and the config shape at full size.
Tolerances: 16-bit (the MFMA path rounds P to the input dtype before P @ V,
as the reference does) 2.5e-2 -- the reference test's fp16 bound; fp32
(fp32 throughout) 1e-4."""

import itertools
import math
import random

import numpy as np
import pytest
import torch

import ntops_amd
from ntops_amd import _lib
from ntops_amd.kernels.scaled_dot_product_attention import CausalVariant
from oracle import ops as O
from tests.helpers import DT_NAME, assert_close, from_np, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

# 16-bit data: the north-star bound, against the oracle with P rounded to
# the dtype before P @ V (as the reference's kernel and this one do)
TOL = {torch.float32: (1e-4, 1e-4), torch.float16: (1.6e-2, 1.6e-2), torch.bfloat16: (1.6e-2, 1.6e-2)}
sdpa = ntops_amd.torch.scaled_dot_product_attention


def oracle(q, k, v, mask=None, causal=0, scale=None):
    dt = DT_NAME[q.dtype]
    m, mdt = None, None
    if mask is not None:
        m = to_np(mask)
        mdt = DT_NAME[mask.dtype]
    return from_np(O.scaled_dot_product_attention(to_np(q), to_np(k), to_np(v), dt, m, mdt, causal, scale,
                                                  round_p=True), dt)


def cases():
    random.seed(0)
    out = []
    for mask_type, is_causal, scale, dtype, kv_cache, variant in itertools.product(
        (None, torch.bool, torch.float32), (False, True), (None, random.uniform(0.05, 0.5)),
        (torch.float32, torch.float16, torch.bfloat16), (False, True),
        (None, CausalVariant.LOWER_RIGHT, CausalVariant.UPPER_LEFT),
    ):
        if mask_type is not None and is_causal:
            continue
        hq = 2 ** random.randint(1, 5)
        hkv = 2 ** random.randint(1, int(math.log2(hq)))
        sq, skv = random.randint(1, 512), random.randint(1, 512)
        if variant == CausalVariant.LOWER_RIGHT and sq > skv:
            continue
        d = random.choice([32, 64, 128])
        out.append((random.randint(1, 4), hq, sq, d, hkv, skv, mask_type, is_causal, scale, variant, kv_cache, dtype))
    return out


@pytest.mark.parametrize("b, hq, sq, d, hkv, skv, mask_type, is_causal, scale, variant, kv_cache, dtype", cases())
def test_sdpa(b, hq, sq, d, hkv, skv, mask_type, is_causal, scale, variant, kv_cache, dtype):
    torch.manual_seed(b * 1000 + sq * 7 + skv)
    q = torch.randn(b, hq, sq, d).to(dtype)
    k = torch.randn(b, hkv, skv, d).to(dtype)
    v = torch.randn(b, hkv, skv, d).to(dtype)
    mask = None
    if mask_type is not None:
        r = torch.rand(sq, skv)
        mask = r > 0.5 if mask_type is torch.bool else torch.where(r > 0.5, 0.0, float("-inf")).to(dtype)
    kg, vg = k.clone().cuda(), v.clone().cuda()
    pk = pv = sk = sv = None
    if kv_cache:
        pk, pv = kg[:, :, -1:, :].clone(), vg[:, :, -1:, :].clone()
        sk, sv = kg[:, :, -1:, :], vg[:, :, -1:, :]
        sk[...] = 0
        sv[...] = 0
    got = sdpa(q.cuda(), kg, vg, attn_mask=None if mask is None else mask.cuda(), is_causal=is_causal, scale=scale,
               enable_gqa=True, causal_variant=variant, present_key=pk, present_value=pv,
               present_key_slot=sk, present_value_slot=sv)
    causal = 0
    if is_causal:
        causal = 2 if variant == CausalVariant.LOWER_RIGHT else 1
    exp = oracle(q, k, v, mask, causal, scale)
    assert got.dtype == dtype and got.shape == q.shape
    assert_close(got, exp, *TOL[dtype], "sdpa")


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
# head dims below 64 / 128 (16-bit data): the D = 64 / 128 kernels with the
# columns past the head dim read as zero and never stored
@pytest.mark.parametrize("d", (64, 128, 80, 96, 32, 48, 120))
def test_sdpa_edges(dtype, d):
    g = torch.Generator().manual_seed(d)
    rt = lambda *s: torch.randn(*s, generator=g).to(dtype)  # noqa: E731
    for (sq, skv, causal) in ((1, 300, 0), (1, 300, 2), (300, 1, 1), (200, 70, 1), (70, 200, 2), (129, 129, 1), (128, 64, 0)):
        q, k, v = rt(2, 4, sq, d), rt(2, 2, skv, d), rt(2, 2, skv, d)
        variant = CausalVariant.LOWER_RIGHT if causal == 2 else None
        got = sdpa(q.cuda(), k.cuda(), v.cuda(), is_causal=causal > 0, enable_gqa=True, causal_variant=variant)
        assert_close(got, oracle(q, k, v, None, causal), *TOL[dtype], f"sq {sq} skv {skv} causal {causal}")
    # fully masked rows give zeros
    q, k, v = rt(1, 2, 40, d), rt(1, 2, 50, d), rt(1, 2, 50, d)
    m = torch.rand(40, 50, generator=g) > 0.3
    m[7] = False
    got = sdpa(q.cuda(), k.cuda(), v.cuda(), attn_mask=m.cuda())
    assert (got[:, :, 7].cpu() == 0).all()
    assert_close(got, oracle(q, k, v, m), *TOL[dtype], "bool mask with a masked row")
    # (B, S, H, D) storage viewed as (B, H, S, D): strided inputs and a 3-D call
    qs, ks, vs = rt(2, 96, 4, d), rt(2, 80, 4, d), rt(2, 80, 4, d)
    qt, kt, vt = (t.cuda().transpose(1, 2) for t in (qs, ks, vs))
    got = sdpa(qt, kt, vt, is_causal=True)
    assert_close(got, oracle(qs.transpose(1, 2), ks.transpose(1, 2), vs.transpose(1, 2), None, 1), *TOL[dtype], "strided")
    got3 = sdpa(qs[0].cuda().transpose(0, 1), ks[0].cuda().transpose(0, 1), vs[0].cuda().transpose(0, 1))
    exp3 = oracle(qs[:1].transpose(1, 2), ks[:1].transpose(1, 2), vs[:1].transpose(1, 2))[0]
    assert_close(got3, exp3, *TOL[dtype], "3-D")


@pytest.mark.parametrize("d, causal", ((96, 1), (80, 2), (96, 0), (40, 1)))
def test_sdpa_head_dim_tail_on_matrix_cores(d, causal):
    """bf16 head dims that are not 64 / 128 run on the matrix-core kernels
    (asserted by name) with the tail columns zero: against the oracle on
    every element, for the flash kernel (Sq > 128) and the masked one."""
    g = torch.Generator().manual_seed(d * 10 + causal)
    b, h, s = 2, 4, 384
    q, k, v = (torch.randn(b, h, s, d, generator=g).bfloat16() for _ in range(3))
    variant = CausalVariant.LOWER_RIGHT if causal == 2 else None
    got = sdpa(q.cuda(), k.cuda(), v.cuda(), is_causal=causal > 0, causal_variant=variant)
    dk = 128 if d > 64 else 64
    assert _lib.last_kernel().startswith(f"sdpa_flash d{dk}"), _lib.last_kernel()
    assert got.shape == (b, h, s, d)
    assert_close(got, oracle(q, k, v, None, causal), *TOL[torch.bfloat16], f"d {d}")
    m = torch.rand(s, s, generator=g) > 0.4
    got = sdpa(q.cuda(), k.cuda(), v.cuda(), attn_mask=m.cuda())
    assert _lib.last_kernel().startswith(f"sdpa_fwd d{dk}"), _lib.last_kernel()
    assert_close(got, oracle(q, k, v, m), *TOL[torch.bfloat16], f"d {d} masked")


@pytest.mark.parametrize("sq", (1, 256))
def test_sdpa_rounds_p_before_pv(sq):
    """P enters P @ V rounded to bf16 while the denominator sums it
    unrounded: one key scores 0, 255 score ln(p1) with p1 just below the bf16
    midpoint above 0.25, all values 1 -> (1 + 255 * 0.25) / (1 + 255 * p1)
    = 0.99615 -> 0.99609375 (summing unrounded P everywhere, or rounded P
    everywhere, gives 1).  sq = 1: the masked-path kernel; 256: the flash
    kernel."""
    D, n = 64, 255
    p1 = 0.25 + 2.0 ** -10 * 0.999
    scale = float(-math.log(p1))
    q = torch.zeros(1, 2, sq, D)
    q[..., 0] = 1.0
    k = torch.zeros(1, 2, n + 1, D)
    k[0, :, 1:, 0] = -1.0
    v = torch.ones(1, 2, n + 1, D)
    got = sdpa(q.bfloat16().cuda(), k.bfloat16().cuda(), v.bfloat16().cuda(), scale=scale)
    assert _lib.last_kernel().startswith("sdpa_flash" if sq > 128 else "sdpa_fwd"), _lib.last_kernel()
    assert (got.float() == 0.99609375).all(), got.float().unique()
    exp = oracle(q.bfloat16(), k.bfloat16(), v.bfloat16(), None, 0, scale)
    assert torch.equal(got.cpu(), exp)


def test_sdpa_argument_checks():
    q = torch.randn(1, 4, 8, 64, device="cuda")
    k = torch.randn(1, 2, 8, 64, device="cuda")
    with pytest.raises(AssertionError):
        sdpa(q, k, k)  # GQA not enabled
    with pytest.raises(AssertionError):
        sdpa(q, q, q, attn_mask=torch.ones(8, 8, dtype=torch.bool, device="cuda"), is_causal=True)
    with pytest.raises(AssertionError):
        sdpa(q, q, q, dropout_p=0.1)
    with pytest.raises(RuntimeError):
        sdpa(q, q.half(), q)


def test_sdpa_config_full_size():
    """bf16 (4, 32, 2048, 128) causal, the softmax / bmm config shape: three
    (batch, head) pairs against the oracle on every row, and on every head
    the size-independent facts that causal query 0 returns exactly V[0] and
    every output is finite."""
    B, H, S, D = 4, 32, 2048, 128
    g = torch.Generator().manual_seed(0)
    q = torch.randn(B, H, S, D, generator=g).bfloat16()
    k = torch.randn(B, H, S, D, generator=g).bfloat16()
    v = torch.randn(B, H, S, D, generator=g).bfloat16()
    got = sdpa(q.cuda(), k.cuda(), v.cuda(), is_causal=True)
    for b, h in ((0, 0), (1, 17), (3, 31)):
        exp = oracle(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1], None, 1)
        assert_close(got[b:b + 1, h:h + 1], exp, 2.5e-2, 2.5e-2, f"config head ({b}, {h})")
    assert torch.equal(got[:, :, 0].cpu(), v[:, :, 0])
    assert torch.isfinite(got).all()


@pytest.mark.parametrize("b, hq, hkv, sq, skv, d, variant, dtype", [
    (4, 64, 16, 384, 384, 128, CausalVariant.UPPER_LEFT, torch.bfloat16),
    (2, 128, 32, 320, 700, 64, CausalVariant.LOWER_RIGHT, torch.float16),
    (3, 96, 96, 520, 520, 128, CausalVariant.UPPER_LEFT, torch.float16),
])
def test_sdpa_causal_many_items_per_workgroup(b, hq, hkv, sq, skv, d, variant, dtype):
    """Causal attention runs one workgroup per CU over several (batch, head,
    query block) items, each item starting on K / V tiles and Q rows its
    predecessor loaded: more items than CUs (ragged last query blocks,
    unequal key counts, GQA, both causal corners), every head against the
    oracle."""
    torch.manual_seed(sq * 31 + skv)
    q = torch.randn(b, hq, sq, d).to(dtype)
    k = torch.randn(b, hkv, skv, d).to(dtype)
    v = torch.randn(b, hkv, skv, d).to(dtype)
    assert b * hq * ((sq + 255) // 256) > 256
    got = sdpa(q.cuda(), k.cuda(), v.cuda(), is_causal=True, enable_gqa=True, causal_variant=variant)
    causal = 2 if variant == CausalVariant.LOWER_RIGHT else 1
    exp = oracle(q, k, v, None, causal)
    assert_close(got, exp, *TOL[dtype], "sdpa causal, many items per workgroup")


@pytest.mark.parametrize("b, hq, hkv, sq, skv, d, dtype", [
    (4, 64, 64, 300, 448, 128, torch.bfloat16),
    (3, 96, 24, 260, 260, 64, torch.float16),
])
def test_sdpa_many_items_per_workgroup(b, hq, hkv, sq, skv, d, dtype):
    """Non-causal attention over more items than CUs (one persistent
    workgroup per CU, chained items, ragged last query blocks, GQA): every
    head against the oracle."""
    torch.manual_seed(sq * 13 + skv)
    q = torch.randn(b, hq, sq, d).to(dtype)
    k = torch.randn(b, hkv, skv, d).to(dtype)
    v = torch.randn(b, hkv, skv, d).to(dtype)
    assert b * hq * ((sq + 255) // 256) > 256
    got = sdpa(q.cuda(), k.cuda(), v.cuda(), enable_gqa=True)
    assert_close(got, oracle(q, k, v), *TOL[dtype], "sdpa, many items per workgroup")


@pytest.mark.parametrize("skv", (384, 383))
@pytest.mark.parametrize("mask_dtype", (torch.bool, torch.float32, torch.float16, torch.bfloat16))
@pytest.mark.parametrize("d", (64, 128))
def test_sdpa_mask_load_paths(skv, mask_dtype, d):
    """Explicit masks enter S through the MFMA accumulator, loaded four keys
    per access when mask rows are 4-element aligned (skv 384) and key by key
    otherwise (skv 383), for every mask element type; broadcast over batch
    and heads, and per (batch, head)."""
    dtype = torch.bfloat16 if mask_dtype is torch.bfloat16 else torch.float16
    torch.manual_seed(skv + d)
    b, h, sq = 2, 4, 200
    q, k, v = torch.randn(b, h, sq, d).to(dtype), torch.randn(b, h, skv, d).to(dtype), torch.randn(b, h, skv, d).to(dtype)
    for shape in ((sq, skv), (b, h, sq, skv)):
        r = torch.rand(shape)
        if mask_dtype is torch.bool:
            mask = r > 0.3
        else:
            mask = torch.where(r > 0.3, torch.randn(shape) * 0.5, torch.tensor(float("-inf"))).to(mask_dtype)
        got = sdpa(q.cuda(), k.cuda(), v.cuda(), attn_mask=mask.cuda())
        assert_close(got, oracle(q, k, v, mask), *TOL[dtype], f"mask {mask_dtype} {tuple(shape)}")


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_sdpa_lower_right_more_queries_than_keys(dtype):
    """Lower-right causal with Sq - Skv = 400: query row i sees keys
    j <= i + Skv - Sq, so rows 0..399 see none and give 0 (torch's CPU
    kernel and the oracle); the flash kernel's first 256-row query block has
    zero key tiles and the second starts inside the fully masked rows.  The
    same pattern as an explicit bool mask runs the masked kernel."""
    from ntops_amd import _lib

    g = torch.Generator().manual_seed(700)
    b, h, sq, skv, d = 2, 4, 700, 300, 128
    q, k, v = (torch.randn(b, h, s, d, generator=g).to(dtype) for s in (sq, skv, skv))
    qg, kg, vg = q.cuda(), k.cuda(), v.cuda()
    got = sdpa(qg, kg, vg, is_causal=True, causal_variant=CausalVariant.LOWER_RIGHT)
    assert _lib.last_kernel().startswith("sdpa_flash d128 causal_lr")
    assert (got[:, :, : sq - skv] == 0).all()
    assert_close(got, oracle(q, k, v, None, 2), *TOL[dtype], "lower-right, Sq > Skv")
    m = torch.ones(sq, skv, dtype=torch.bool).tril(skv - sq)
    got_m = sdpa(qg, kg, vg, attn_mask=m.cuda())
    assert _lib.last_kernel().startswith("sdpa_fwd d128")
    assert (got_m[:, :, : sq - skv] == 0).all()
    assert_close(got_m, oracle(q, k, v, m), *TOL[dtype], "bool mask, fully masked leading rows")


def test_sdpa_lower_right_chained_zero_tile_items():
    """More work items than CUs (3 x 32 heads x 4 query blocks), lower-right
    causal with Sq - Skv = 512: every head's first two query blocks have no
    key tile and are chained with blocks that do.  All masked rows are 0;
    sampled heads (GQA, 4 query heads per key head) match the oracle."""
    from ntops_amd import _lib

    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(1024)
    b, hq, hkv, sq, skv, d = 3, 32, 8, 1024, 512, 128
    q = torch.randn(b, hq, sq, d, generator=g).to(dtype)
    k = torch.randn(b, hkv, skv, d, generator=g).to(dtype)
    v = torch.randn(b, hkv, skv, d, generator=g).to(dtype)
    got = sdpa(q.cuda(), k.cuda(), v.cuda(), is_causal=True, enable_gqa=True,
               causal_variant=CausalVariant.LOWER_RIGHT)
    name = _lib.last_kernel()
    assert name.startswith("sdpa_flash d128 causal_lr items384 grid")
    assert int(name.split("grid")[1]) < 384, name
    assert (got[:, :, : sq - skv] == 0).all()
    for bi, h0 in ((0, 0), (1, 12), (2, 28)):
        exp = oracle(q[bi:bi + 1, h0:h0 + 4], k[bi:bi + 1, h0 // 4:h0 // 4 + 1], v[bi:bi + 1, h0 // 4:h0 // 4 + 1],
                     None, 2)
        assert_close(got[bi:bi + 1, h0:h0 + 4], exp, *TOL[dtype], f"batch {bi} heads {h0}..{h0 + 3}")


@pytest.mark.parametrize("d", (4, 36, 64, 100, 128))
def test_sdpa_f32_matrix_core_kernel(d):
    """fp32 attention on the matrix-core kernel (IEEE fp32 products, fp32
    accumulation): head dims in multiples of 4 up to 128, causal in both
    corners over many query blocks (dealt longest first), GQA, an additive
    float mask with a scale, against the oracle at the fp32 tolerance."""
    g = torch.Generator().manual_seed(100 + d)
    rt = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    for (sq, skv, causal) in ((700, 700, 1), (300, 650, 2), (650, 300, 2), (257, 33, 0)):
        q, k, v = rt(2, 8, sq, d), rt(2, 4, skv, d), rt(2, 4, skv, d)
        variant = CausalVariant.LOWER_RIGHT if causal == 2 else None
        got = sdpa(q.cuda(), k.cuda(), v.cuda(), is_causal=causal > 0, enable_gqa=True, causal_variant=variant)
        assert _lib.last_kernel() == f"sdpa_f32 d{32 if d <= 32 else 64 if d <= 64 else 128}", _lib.last_kernel()
        assert_close(got, oracle(q, k, v, None, causal), *TOL[torch.float32], f"d {d} sq {sq} skv {skv} causal {causal}")
    q, k, v = rt(1, 4, 100, d), rt(1, 4, 90, d), rt(1, 4, 90, d)
    m = rt(1, 4, 100, 90) * 2
    got = sdpa(q.cuda(), k.cuda(), v.cuda(), attn_mask=m.cuda(), scale=0.3)
    assert_close(got, oracle(q, k, v, m, 0, 0.3), *TOL[torch.float32], f"d {d} float mask")


def test_sdpa_f32_generic_fallbacks():
    """A head dim past 128 takes the generic kernel; a strided head dim is
    laid out by the wrapper and runs on the matrix cores."""
    g = torch.Generator().manual_seed(7)
    rt = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    q, k, v = rt(1, 2, 50, 132), rt(1, 2, 60, 132), rt(1, 2, 60, 132)
    got = sdpa(q.cuda(), k.cuda(), v.cuda(), is_causal=True)
    assert _lib.last_kernel() == "sdpa_generic"
    assert_close(got, oracle(q, k, v, None, 1), *TOL[torch.float32], "d 132")
    qs = rt(1, 2, 50, 64 * 2)[..., ::2]  # head-dim stride 2 (the wrapper lays it out for the kernels)
    got = sdpa(qs.cuda(), k[..., :64].cuda(), v[..., :64].cuda())
    assert_close(got, oracle(qs.contiguous(), k[..., :64].contiguous(), v[..., :64].contiguous()), *TOL[torch.float32],
                 "strided head dim")
