"""rotary_position_embedding_qk -- rotary_position_embedding applied to the
query and key of one attention layer in a single launch.

No ntops counterpart: it is two calls of torch/rotary_position_embedding.py:7-29
(math: kernels/rotary_position_embedding.py:6-47) with the same tables, and
its results equal those two calls element for element.  q is
(batch, seq, q_heads, dim) and k (batch, seq, k_heads, dim) (the head counts
may differ, as in grouped-query attention); tables are (seq, dim / 2) or
(seq, dim).  Returns (q_out, k_out); inplace=True rotates q and k in place."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard, _contiguous, _to_dtype


def rotary_position_embedding_qk(q, k, sin_table, cos_table, interleaved=True, inplace=False):
    if q.dim() != 4 or k.dim() != 4:
        raise RuntimeError("rotary_position_embedding_qk: q and k must be (batch, seq, heads, dim)")
    batch_size, seq_len, q_heads, emb_dim = q.shape
    if k.shape[0] != batch_size or k.shape[1] != seq_len or k.shape[3] != emb_dim:
        raise RuntimeError("rotary_position_embedding_qk: q and k differ in batch, seq or dim")
    if k.dtype != q.dtype:
        raise RuntimeError("rotary_position_embedding_qk: q and k must have the same dtype")
    if emb_dim % 2 != 0:
        raise RuntimeError("The embedding dimension must be even.")
    if q.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"rotary_position_embedding_qk: unsupported dtype {q.dtype}")
    for name, tab in (("sin_table", sin_table), ("cos_table", cos_table)):
        if tab.dim() != 2 or tab.shape[0] < seq_len or tab.shape[1] not in (emb_dim // 2, emb_dim):
            raise RuntimeError(
                f"rotary_position_embedding_qk: {name} must be (seq_len, dim/2) or (seq_len, dim), "
                f"got {tuple(tab.shape)}")
    if sin_table.shape[1] != cos_table.shape[1]:
        raise RuntimeError("rotary_position_embedding_qk: sin and cos tables differ in width")

    dev = _lib.require_cuda(q, k, sin_table, cos_table)
    q_out = q if inplace else torch.empty_like(q)
    k_out = k if inplace else torch.empty_like(k)
    sin_table = _to_dtype(sin_table, q.dtype)
    cos_table = _to_dtype(cos_table, q.dtype)
    if sin_table.stride(1) != 1 or cos_table.stride(1) != 1 or sin_table.stride(0) != cos_table.stride(0):
        sin_table = _contiguous(sin_table)
        cos_table = _contiguous(cos_table)
        if sin_table.stride(0) != cos_table.stride(0):
            raise RuntimeError("rotary_position_embedding_qk: table layouts differ")

    st = lambda t: _lib.i64_array(t.stride())  # noqa: E731
    lib = _lib.load()
    with _DeviceGuard(dev):
        rc = lib.ntops_rope_qk(
            _lib.dtype_code(q.dtype), batch_size, seq_len, q_heads, k.shape[2], emb_dim,
            q.data_ptr(), st(q), k.data_ptr(), st(k), sin_table.data_ptr(), cos_table.data_ptr(),
            sin_table.stride(0), sin_table.shape[1], 1 if interleaved else 0,
            q_out.data_ptr(), st(q_out), k_out.data_ptr(), st(k_out), _lib.stream_of(q_out))
    _lib.check(rc, "ntops_amd.rotary_position_embedding_qk")
    return q_out, k_out
