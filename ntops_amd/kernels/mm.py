"""Matmul input-precision enum, kept for source compatibility with
src/ntops/kernels/mm.py:13-16 (`ntops.kernels.mm.InputPrecisionVariant`)."""

import enum


class InputPrecisionVariant(enum.IntEnum):
    TF32 = enum.auto()

    IEEE = enum.auto()
