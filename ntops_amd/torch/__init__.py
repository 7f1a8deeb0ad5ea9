"""PyTorch-facing operators, a drop-in for `ntops.torch`
(src/ntops/torch/__init__.py) on the LLM hot path and its elementwise
family."""

from ntops_amd.torch.abs import abs
from ntops_amd.torch.add import add
from ntops_amd.torch.add_rms_norm import add_rms_norm
from ntops_amd.torch.addmm import addmm
from ntops_amd.torch.bitwise_and import bitwise_and
from ntops_amd.torch.bitwise_not import bitwise_not
from ntops_amd.torch.bitwise_or import bitwise_or
from ntops_amd.torch.bmm import bmm
from ntops_amd.torch.clamp import clamp
from ntops_amd.torch.conv2d import conv2d
from ntops_amd.torch.cos import cos
from ntops_amd.torch.div import div
from ntops_amd.torch.eq import eq
from ntops_amd.torch.exp import exp
from ntops_amd.torch.ge import ge
from ntops_amd.torch.gelu import gelu
from ntops_amd.torch.gt import gt
from ntops_amd.torch.im2col import im2col
from ntops_amd.torch.isinf import isinf
from ntops_amd.torch.isnan import isnan
from ntops_amd.torch.layer_norm import layer_norm
from ntops_amd.torch.le import le
from ntops_amd.torch.lt import lt
from ntops_amd.torch.matmul import matmul
from ntops_amd.torch.mm import mm
from ntops_amd.torch.mul import mul
from ntops_amd.torch.ne import ne
from ntops_amd.torch.neg import neg
from ntops_amd.torch.pow import pow
from ntops_amd.torch.relu import relu
from ntops_amd.torch.rms_norm import rms_norm
from ntops_amd.torch.rotary_position_embedding import rotary_position_embedding
from ntops_amd.torch.rotary_position_embedding_qk import rotary_position_embedding_qk
from ntops_amd.torch.rsqrt import rsqrt
from ntops_amd.torch.scaled_dot_product_attention import scaled_dot_product_attention
from ntops_amd.torch.sigmoid import sigmoid
from ntops_amd.torch.silu import silu
from ntops_amd.torch.sin import sin
from ntops_amd.torch.softmax import softmax
from ntops_amd.torch.sub import sub
from ntops_amd.torch.tanh import tanh

__all__ = [
    "abs",
    "add",
    "add_rms_norm",
    "addmm",
    "bitwise_and",
    "bitwise_not",
    "bitwise_or",
    "bmm",
    "clamp",
    "conv2d",
    "cos",
    "div",
    "eq",
    "exp",
    "ge",
    "gelu",
    "gt",
    "im2col",
    "isinf",
    "isnan",
    "layer_norm",
    "le",
    "lt",
    "matmul",
    "mm",
    "mul",
    "ne",
    "neg",
    "pow",
    "relu",
    "rms_norm",
    "rotary_position_embedding",
    "rotary_position_embedding_qk",
    "rsqrt",
    "scaled_dot_product_attention",
    "sigmoid",
    "silu",
    "sin",
    "softmax",
    "sub",
    "tanh",
]
