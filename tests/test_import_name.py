"""The package answers to the reference's import name (src/ntops/__init__.py,
tests/conftest.py:7,14 of the reference): `import ntops.torch.utils` and
`ntops.torch.<op>` bind to the same objects as ntops_amd."""

import importlib
import subprocess
import sys

import ntops_amd


def test_ntops_names_are_ntops_amd_objects():
    import ntops
    import ntops.torch.utils
    from ntops.kernels.mm import InputPrecisionVariant
    from ntops.kernels.scaled_dot_product_attention import CausalVariant

    assert ntops.torch is ntops_amd.torch
    assert ntops.torch.utils is ntops_amd.torch.utils
    assert ntops.kernels.mm is ntops_amd.kernels.mm
    assert InputPrecisionVariant is ntops_amd.kernels.mm.InputPrecisionVariant
    assert CausalVariant is ntops_amd.kernels.scaled_dot_product_attention.CausalVariant
    for op in ntops_amd.torch.__all__:
        assert getattr(ntops.torch, op) is getattr(ntops_amd.torch, op)
    for op in ("rms_norm", "layer_norm", "softmax", "rotary_position_embedding", "mm", "bmm", "addmm", "matmul",
               "silu", "gelu", "exp", "add", "mul", "bitwise_and", "bitwise_or", "bitwise_not"):
        assert callable(getattr(ntops.torch, op))


def test_knob_setters_shared():
    """The reference conftest's call: the knob set through ntops is the one
    ntops_amd reads."""
    import ntops.torch.utils

    old = ntops_amd.torch.utils.get_default_max_num_configs()
    try:
        ntops.torch.utils.set_default_max_num_configs(3)
        assert ntops_amd.torch.utils.get_default_max_num_configs() == 3
    finally:
        ntops.torch.utils.set_default_max_num_configs(old)


def test_fresh_process_imports_submodule_first():
    """`import ntops.torch.utils` as the very first import of a process (the
    reference conftest's order) resolves through the alias."""
    code = ("import ntops.torch.utils, ntops_amd; "
            "assert ntops.torch.utils is ntops_amd.torch.utils; "
            "ntops.torch.utils.set_default_max_num_configs(3); "
            "import ntops; assert callable(ntops.torch.rms_norm)")
    subprocess.run([sys.executable, "-c", code], check=True, cwd=importlib.import_module("tests").__path__[0] + "/..")
