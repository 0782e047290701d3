"""zeninfer_amd -- MI355X (gfx950) block-quantised projection backend.

The product is the C-ABI library built from ``csrc/`` (``include/zq_hip.h``);
``zq`` is its Python binding.
"""
from . import zq  # noqa: F401
