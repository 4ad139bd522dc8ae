"""Import-path alias of the reference module kernels/sm120/moe_grouped.py."""
from ..gfx950.grouped import *  # noqa: F401,F403
from ..gfx950.grouped import __all__  # noqa: F401
