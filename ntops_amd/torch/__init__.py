"""PyTorch-facing operators, a drop-in for `ntops.torch`
(src/ntops/torch/__init__.py) on the LLM hot path."""

from ntops_amd.torch.add import add
from ntops_amd.torch.addmm import addmm
from ntops_amd.torch.bitwise_and import bitwise_and
from ntops_amd.torch.bitwise_not import bitwise_not
from ntops_amd.torch.bitwise_or import bitwise_or
from ntops_amd.torch.bmm import bmm
from ntops_amd.torch.exp import exp
from ntops_amd.torch.gelu import gelu
from ntops_amd.torch.layer_norm import layer_norm
from ntops_amd.torch.matmul import matmul
from ntops_amd.torch.mm import mm
from ntops_amd.torch.mul import mul
from ntops_amd.torch.rms_norm import rms_norm
from ntops_amd.torch.rotary_position_embedding import rotary_position_embedding
from ntops_amd.torch.silu import silu
from ntops_amd.torch.softmax import softmax

__all__ = [
    "add",
    "addmm",
    "bitwise_and",
    "bitwise_not",
    "bitwise_or",
    "bmm",
    "exp",
    "gelu",
    "layer_norm",
    "matmul",
    "mm",
    "mul",
    "rms_norm",
    "rotary_position_embedding",
    "silu",
    "softmax",
]
