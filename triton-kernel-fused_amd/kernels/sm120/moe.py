"""Import-path alias of the reference module kernels/sm120/moe.py."""
from ..gfx950.moe import (moe_per_expert, moe_eager, moe_grouped, moe_grouped_cublas,  # noqa: F401
                          GROUPED_MIN_TOKENS, _code_max)
from ..gfx950.grouped import (moe, moe_grouped_cublas_polyglu, grouped_supported,  # noqa: F401
                                  prefer_grouped, GROUPED_TOKENS_PER_EXPERT_MAX)
