"""Compatibility namespace for `ntops.kernels`.

The reference's kernels/ package holds NineToothed kernel descriptions; here
the kernels are the HIP sources under ntops_amd/csrc, so this package only
keeps the public symbols callers use (`mm.InputPrecisionVariant`,
`scaled_dot_product_attention.CausalVariant`)."""

from ntops_amd.kernels import mm, scaled_dot_product_attention

__all__ = ["mm", "scaled_dot_product_attention"]
