"""ntops_amd -- the ntops LLM operator hot path on MI355X (gfx950).

`ntops_amd.torch.<op>` keeps the call signatures of `ntops.torch.<op>`; every
op runs a hand-written HIP kernel from lib/libntops_amd.so through the C ABI
declared in include/ntops_amd.h."""

from ntops_amd import kernels, torch

__all__ = ["kernels", "torch"]
