"""scaled_dot_product_attention -- mirror of
src/ntops/torch/scaled_dot_product_attention.py:10-108 (math:
kernels/scaled_dot_product_attention.py:154-201).

Same arguments and checks as the reference: dropout_p must be 0, attn_mask
and is_causal are exclusive, key / value heads must match and divide the
query heads when enable_gqa (equal otherwise); a bool mask keeps True
positions; scale defaults to 1 / sqrt(head_dim); causal_variant defaults to
UPPER_LEFT; present_key / present_value (KV cache) are first written into
present_key_slot / present_value_slot (views into key / value).  Inputs are
(batch, heads, seq, head_dim) or (heads, seq, head_dim).  A row with every
key masked yields zeros, as torch's CPU kernel does."""

import math

import torch

from ntops_amd import _lib
from ntops_amd.kernels.scaled_dot_product_attention import CausalVariant
from ntops_amd.torch.utils import _DeviceGuard, _cast_into, _strides, _to_dtype

_MASK_DTYPES = (torch.bool, torch.float32, torch.float16, torch.bfloat16)


def scaled_dot_product_attention(
    query,
    key,
    value,
    attn_mask=None,
    dropout_p=0,
    is_causal=False,
    scale=None,
    enable_gqa=False,
    causal_variant=None,
    present_key=None,
    present_value=None,
    present_key_slot=None,
    present_value_slot=None,
):
    assert dropout_p == 0, "`dropout_p` is not supported yet."
    assert attn_mask is None or not is_causal, "Cannot use `attn_mask` and `is_causal` together."

    num_heads_q, num_heads_kv = query.shape[-3], key.shape[-3]
    assert num_heads_kv == value.shape[-3], "Number of heads in `key` and `value` must be the same."
    if not enable_gqa:
        assert num_heads_q == num_heads_kv, (
            "Number of heads in `query`, `key`, and `value` must be the same when GQA is not enabled."
        )
    else:
        assert num_heads_q % num_heads_kv == 0, (
            "Number of heads in `query` must be divisible by number of heads in `key` and `value` "
            "when GQA is enabled."
        )
    if not (query.dtype == key.dtype == value.dtype):
        raise RuntimeError(
            f"Expected query, key, and value to have the same dtype, but got {query.dtype}, "
            f"{key.dtype} and {value.dtype}"
        )
    dev = _lib.require_cuda(query, key, value, attn_mask, present_key, present_value)

    if present_key is not None:
        # the reference's kernel assigns present_key_slot = present_key
        # (kernels/scaled_dot_product_attention.py:139-140) before attending
        _cast_into(present_key, present_key_slot)
        _cast_into(present_value, present_value_slot)

    squeeze = query.dim() == 3
    if squeeze:
        query, key, value = query.unsqueeze(0), key.unsqueeze(0), value.unsqueeze(0)
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise RuntimeError("ntops_amd.scaled_dot_product_attention: expected 3-D or 4-D query, key and value")
    B, Hq, Sq, D = query.shape
    Skv = key.shape[-2]
    if key.shape[0] != B or value.shape[0] != B or value.shape[-2] != Skv or key.shape[-1] != D or value.shape[-1] != D:
        raise RuntimeError("ntops_amd.scaled_dot_product_attention: incompatible query / key / value shapes")

    mask_ptr, mask_strides, mask_code = None, None, 0
    if attn_mask is not None:
        m = attn_mask
        if m.dtype not in _MASK_DTYPES:
            m = _to_dtype(m, torch.float32)
        m = m.expand(B, Hq, Sq, Skv)
        mask_ptr, mask_strides, mask_code = m.data_ptr(), _strides(m), _lib.dtype_code(m.dtype)

    causal = 0
    if is_causal:
        variant = CausalVariant.UPPER_LEFT if causal_variant is None else CausalVariant(causal_variant)
        causal = int(variant)
    if scale is None:
        scale = 1 / math.sqrt(D)

    output = torch.empty(query.shape[:-1] + (value.shape[-1],), dtype=value.dtype, device=dev)
    lib = _lib.load()
    with _DeviceGuard(dev):
        rc = lib.ntops_sdpa(
            _lib.dtype_code(query.dtype), B, Hq, key.shape[1], Sq, Skv, D,
            query.data_ptr(), _strides(query), key.data_ptr(), _strides(key), value.data_ptr(), _strides(value),
            mask_ptr, mask_code, mask_strides, causal, float(scale),
            output.data_ptr(), _strides(output), _lib.stream_of(output),
        )
    _lib.check(rc, "ntops_amd.scaled_dot_product_attention")
    return output.squeeze(0) if squeeze else output
