"""rotary_position_embedding -- mirror of
src/ntops/torch/rotary_position_embedding.py:7-29
(math: kernels/rotary_position_embedding.py:6-47).

Accepts ntops' (S, D/2) tables and also full (S, D) tables (the
x*cos + rotate_half(x)*sin convention); per-operation rounding in the tensor
dtype, as torch evaluates the formula eagerly."""

import torch

from ntops_amd import _lib
from ntops_amd.torch.utils import _DeviceGuard, _contiguous, _to_dtype


def rotary_position_embedding(input, sin_table, cos_table, interleaved=True, inplace=False):
    if input.dim() != 4:
        raise RuntimeError("rotary_position_embedding: input must be (batch, seq, heads, dim)")
    batch_size, seq_len, num_heads, emb_dim = input.shape
    if emb_dim % 2 != 0:
        raise RuntimeError("The embedding dimension must be even.")
    if input.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise RuntimeError(f"rotary_position_embedding: unsupported dtype {input.dtype}")
    for name, tab in (("sin_table", sin_table), ("cos_table", cos_table)):
        if tab.dim() != 2 or tab.shape[0] < seq_len or tab.shape[1] not in (emb_dim // 2, emb_dim):
            raise RuntimeError(
                f"rotary_position_embedding: {name} must be (seq_len, dim/2) or (seq_len, dim), got {tuple(tab.shape)}"
            )
    if sin_table.shape[1] != cos_table.shape[1]:
        raise RuntimeError("rotary_position_embedding: sin and cos tables differ in width")

    dev = _lib.require_cuda(input, sin_table, cos_table)

    if inplace:
        output = input
    else:
        output = torch.empty_like(input)

    sin_table = _to_dtype(sin_table, input.dtype)
    cos_table = _to_dtype(cos_table, input.dtype)
    if sin_table.stride(1) != 1 or cos_table.stride(1) != 1 or sin_table.stride(0) != cos_table.stride(0):
        sin_table = _contiguous(sin_table)
        cos_table = _contiguous(cos_table)
        if sin_table.stride(0) != cos_table.stride(0):
            raise RuntimeError("rotary_position_embedding: table layouts differ")

    lib = _lib.load()
    with _DeviceGuard(dev):
        rc = lib.ntops_rope(
            _lib.dtype_code(input.dtype),
            batch_size,
            seq_len,
            num_heads,
            emb_dim,
            input.data_ptr(),
            _lib.i64_array(input.stride()),
            sin_table.data_ptr(),
            cos_table.data_ptr(),
            sin_table.stride(0),
            sin_table.shape[1],
            1 if interleaved else 0,
            output.data_ptr(),
            _lib.i64_array(output.stride()),
            _lib.stream_of(output),
        )
    _lib.check(rc, "ntops_amd.rotary_position_embedding")
    return output
