"""Import-path alias: `from kernels.sm120 import moe` resolves to the gfx950 implementation.
The MoE and router names of the reference package (kernels/sm120/__init__.py:22-23) are bound from
the submodules, so importing `kernels.sm120.moe` later does not rebind `kernels.sm120.moe`."""
from .router import fused_router, router_bias_update, FusedConvRouterCuDNN  # noqa: F401
from .moe import moe, moe_per_expert, moe_eager  # noqa: F401
from . import moe_grouped  # noqa: F401

__all__ = ["fused_router", "router_bias_update", "FusedConvRouterCuDNN",
           "moe", "moe_per_expert", "moe_eager"]
