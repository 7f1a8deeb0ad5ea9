"""Compatibility namespace for `ntops.kernels`.

The reference's kernels/ package holds NineToothed kernel descriptions; here
the kernels are the HIP sources under ntops_amd/csrc, so this package only
keeps the one public symbol callers use (`mm.InputPrecisionVariant`)."""

from ntops_amd.kernels import mm

__all__ = ["mm"]
