"""Import-path alias: `from kernels.sm120 import moe` resolves to the gfx950 implementation."""
from ..gfx950.grouped import moe  # noqa: F401
from ..gfx950 import moe_per_expert, moe_eager  # noqa: F401

__all__ = ["moe", "moe_per_expert", "moe_eager"]
