"""The reference's import name, `ntops` (src/ntops/__init__.py:1-3), bound to
the MI355X implementation in ntops_amd.

`import ntops`, `ntops.torch.<op>(...)`, `import ntops.torch.utils` and
`from ntops.kernels.mm import InputPrecisionVariant` resolve to the very same
module objects as their ntops_amd counterparts (registered below under the
ntops names), so the default-knob setters, the enums and every operator are
shared rather than copied."""

import importlib
import sys

import ntops_amd
from ntops_amd import kernels, torch

# Every module of the public surface, under its ntops name.  Listing them
# here (instead of walking sys.modules) keeps the alias set fixed and makes
# `import ntops.torch.utils` work before anything else imported it.
_ALIASED = (
    "torch",
    "torch.utils",
    "kernels",
    "kernels.mm",
    "kernels.scaled_dot_product_attention",
)

for _name in _ALIASED:
    sys.modules[f"{__name__}.{_name}"] = importlib.import_module(f"ntops_amd.{_name}")

__all__ = ["kernels", "torch"]
