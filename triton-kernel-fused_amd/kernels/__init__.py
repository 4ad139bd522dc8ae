"""MoE expert pipeline for AMD MI355X (gfx950).

    from kernels import moe, moe_per_expert, moe_eager

The public names follow the reference package `kernels` (kernels/sm75/__init__.py:13,
kernels/sm120/__init__.py:20); `kernels.sm75` and `kernels.sm120` are import-path aliases of the
single gfx950 implementation so existing imports keep working.
"""
from .gfx950 import *  # noqa: F401,F403
from .gfx950 import __all__  # noqa: F401
