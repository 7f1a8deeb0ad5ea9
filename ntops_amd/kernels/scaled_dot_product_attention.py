"""`CausalVariant` of kernels/scaled_dot_product_attention.py:11-17 (callers
import it from here); the values are the causal modes of ntops_sdpa."""

import enum


class CausalVariant(enum.IntEnum):
    """Which corner the causal mask is anchored to, as in
    torch.nn.attention.bias.CausalVariant: UPPER_LEFT lets query i see keys
    0..i; LOWER_RIGHT lets it see keys 0..i + (kv_len - q_len)."""

    UPPER_LEFT = enum.auto()

    LOWER_RIGHT = enum.auto()
