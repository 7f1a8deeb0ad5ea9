"""GPU parity: rotary_position_embedding against the oracle.

Mirrors tests/test_rotary_position_embedding.py:48-89 of the reference (B in
{1,4}, S in {1,128}, H in {1,8}, D in {32,64}, interleaved x inplace, fp32 and
fp16) with bf16 and (S, D) tables added, plus the bf16 (4, 4096, 32, 128)
config with (4096, 128) tables at full size."""

import numpy as np
import pytest
import torch

import ntops_amd
from oracle import ops as O
from tests.helpers import DT_NAME, assert_close, assert_equal, from_np, to_np

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]


def tables(seq_len, emb_dim, dtype, full):
    s, c = O.rope_tables(seq_len, emb_dim, full=full)
    return torch.from_numpy(s).to(dtype), torch.from_numpy(c).to(dtype)


def reference_formula(x, sin_table, cos_table, interleaved):
    """tests/test_rotary_position_embedding.py:8-29 of the reference, in
    torch on the CPU ((S, D/2) tables)."""
    batch_size, seq_len, num_heads, emb_dim = x.shape
    sin_table = sin_table[None, :, None, :]
    cos_table = cos_table[None, :, None, :]
    if interleaved:
        p = x.view(batch_size, seq_len, num_heads, emb_dim // 2, 2)
        x0, x1 = p[..., 0], p[..., 1]
        return torch.stack((x0 * cos_table - x1 * sin_table, x0 * sin_table + x1 * cos_table), dim=-1).view(x.shape)
    x0, x1 = x[..., : emb_dim // 2], x[..., emb_dim // 2 :]
    return torch.cat((x0 * cos_table - x1 * sin_table, x0 * sin_table + x1 * cos_table), dim=-1)


@pytest.mark.parametrize("dtype", (torch.float32, torch.float16, torch.bfloat16))
@pytest.mark.parametrize("full_tables", (False, True))
@pytest.mark.parametrize("inplace", (False, True))
@pytest.mark.parametrize("interleaved", (False, True))
@pytest.mark.parametrize("emb_dim", (32, 64))
@pytest.mark.parametrize("num_heads", (1, 8))
@pytest.mark.parametrize("seq_len", (1, 128))
@pytest.mark.parametrize("batch_size", (1, 4))
def test_rope(batch_size, seq_len, num_heads, emb_dim, interleaved, inplace, full_tables, dtype):
    x = torch.randn(batch_size, seq_len, num_heads, emb_dim).to(dtype)
    if full_tables and interleaved:
        sh, ch = tables(seq_len, emb_dim, torch.float32, False)
        sin_t, cos_t = sh.repeat_interleave(2, -1).to(dtype), ch.repeat_interleave(2, -1).to(dtype)
    else:
        sin_t, cos_t = tables(seq_len, emb_dim, dtype, full_tables)
    xg = x.cuda()
    got = ntops_amd.torch.rotary_position_embedding(
        xg.clone() if inplace else xg, sin_t.cuda(), cos_t.cuda(), interleaved=interleaved, inplace=inplace
    )
    dt = DT_NAME[dtype]
    exp = from_np(O.rotary_position_embedding(to_np(x), to_np(sin_t), to_np(cos_t), dt, interleaved), dt)
    # per-operation rounding is deterministic: the kernel matches bit for bit
    assert_equal(got, exp, "rope vs oracle")
    if not full_tables:
        assert_close(got, reference_formula(x, sin_t, cos_t, interleaved), 1e-3, 1e-3, "rope vs reference formula")


def test_rope_noncontiguous_and_longer_tables():
    x = torch.randn(2, 16, 4, 64).bfloat16()
    xg = x.cuda().transpose(1, 2).contiguous().transpose(1, 2)  # BSHD view of a BHSD buffer
    s, c = tables(32, 64, torch.bfloat16, True)  # longer than seq_len: rows 0..15 used
    got = ntops_amd.torch.rotary_position_embedding(xg, s.cuda(), c.cuda(), interleaved=False)
    exp = from_np(O.rotary_position_embedding(to_np(x), to_np(s), to_np(c), "bf16", False), "bf16")
    assert_equal(got, exp, "rope strided")
    odd = torch.randn(1, 3, 2, 10)  # D/2 = 5: generic path
    s, c = tables(3, 10, torch.float32, False)
    got = ntops_amd.torch.rotary_position_embedding(odd.cuda(), s.cuda(), c.cuda(), interleaved=True)
    assert_equal(got, from_np(O.rotary_position_embedding(odd.numpy(), s.numpy(), c.numpy(), "f32", True), "f32"), "generic")


def test_rope_config_full_size():
    """bf16 q and k (4, 4096, 32, 128) ~N(0,1), non-interleaved, (4096, 128)
    tables from theta = 10000, positions 0..4095; every element of q and k
    against the oracle."""
    g = torch.Generator().manual_seed(0)
    q = torch.randn(4, 4096, 32, 128, generator=g).bfloat16()
    k = torch.randn(4, 4096, 32, 128, generator=g).bfloat16()
    s, c = tables(4096, 128, torch.bfloat16, True)
    sg, cg = s.cuda(), c.cuda()
    for name, t in (("q", q), ("k", k)):
        got = ntops_amd.torch.rotary_position_embedding(t.cuda(), sg, cg, interleaved=False)
        for b in range(4):
            exp = from_np(O.rotary_position_embedding(to_np(t[b : b + 1]), to_np(s), to_np(c), "bf16", False), "bf16")
            assert_equal(got[b : b + 1], exp, f"rope config {name} batch {b}")


def test_rope_past_65536_blocks():
    """bf16 (9, 8192, 32, 128): 18.9M items of one 16-byte pack pair, 73728
    blocks on a 2-D grid; the first batch's first and the last batch's last
    1024 positions against the oracle, bit for bit."""
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(9, 8192, 32, 128, device="cuda", generator=g).bfloat16()
    s, c = tables(8192, 128, torch.bfloat16, True)
    got = ntops_amd.torch.rotary_position_embedding(x, s.cuda(), c.cuda(), interleaved=False)
    for b, p0 in ((0, 0), (8, 7168)):  # first and last 1024 positions
        xs = x[b:b + 1, p0:p0 + 1024].cpu()
        exp = from_np(O.rotary_position_embedding(to_np(xs), to_np(s[p0:p0 + 1024]), to_np(c[p0:p0 + 1024]), "bf16",
                                                  False), "bf16")
        assert_equal(got[b:b + 1, p0:p0 + 1024], exp, f"batch {b}")
