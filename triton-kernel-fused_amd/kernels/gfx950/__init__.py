"""gfx950 (MI355X) MoE expert pipeline: HIP kernels behind the reference's `kernels` MoE API."""
from .moe import (moe, moe_per_expert, moe_grouped, moe_grouped_cublas, moe_eager, BatchedGLU,
                  GROUPED_MIN_TOKENS, dispatch)
from .lowp import moe_fp8, moe_mxfp8, rowquant_fp8
from .router import (router_topk, fused_mlp_router, fused_router, router_bias_update,
                     FusedMLPRouter, FusedConvRouterCuDNN)
from .grouped import (moe_grouped_cublas_polyglu, grouped_supported, prefer_grouped,
                          GROUPED_TOKENS_PER_EXPERT_MAX)

__all__ = ["moe", "moe_per_expert", "moe_grouped", "moe_grouped_cublas", "moe_eager", "BatchedGLU",
           "GROUPED_MIN_TOKENS", "dispatch", "moe_grouped_cublas_polyglu", "grouped_supported",
           "prefer_grouped", "GROUPED_TOKENS_PER_EXPERT_MAX", "moe_fp8", "moe_mxfp8", "rowquant_fp8",
           "router_topk", "fused_mlp_router", "fused_router", "router_bias_update", "FusedMLPRouter",
           "FusedConvRouterCuDNN"]
