"""Import-path alias of kernels.gfx950.moe (reference module kernels/sm75/moe.py)."""
from ..gfx950.moe import *  # noqa: F401,F403
from ..gfx950.moe import __all__, _code_max  # noqa: F401
