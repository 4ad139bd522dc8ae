"""Import-path alias: `from kernels.sm75.router import fused_mlp_router` resolves to the gfx950
router epilogue (reference: kernels/sm75/router.py:29-30)."""
from ..gfx950.router import (fused_router, fused_mlp_router, router_bias_update,  # noqa: F401
                             FusedConvRouterCuDNN, FusedMLPRouter)

__all__ = ["fused_router", "fused_mlp_router", "router_bias_update", "FusedConvRouterCuDNN",
           "FusedMLPRouter"]
