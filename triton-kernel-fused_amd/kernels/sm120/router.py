"""Import-path alias: `from kernels.sm120.router import fused_router` resolves to the gfx950
router epilogue (reference: kernels/sm120/router.py)."""
from ..gfx950.router import (fused_router, fused_mlp_router, router_bias_update,  # noqa: F401
                             FusedConvRouterFused, FusedConvRouterCuDNN, FusedMLPRouter)

__all__ = ["fused_router", "fused_mlp_router", "router_bias_update", "FusedConvRouterFused",
           "FusedConvRouterCuDNN", "FusedMLPRouter"]
