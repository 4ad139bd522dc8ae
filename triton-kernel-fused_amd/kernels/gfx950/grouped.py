"""The grouped entry points of the reference's Blackwell package, kept by name for drop-in use
(/root/reference/kernels/sm120/moe_grouped.py, kernels/sm120/moe.py). On gfx950 they run the same
HIP grouped kernels as `moe`; the helpers answer for this library instead of torch._grouped_mm."""
import torch

from .moe import _code_max, moe_per_expert, _MoEFunction

__all__ = ["moe_grouped_cublas_polyglu", "grouped_supported", "prefer_grouped",
           "GROUPED_TOKENS_PER_EXPERT_MAX"]

# Kept for API compatibility (moe_grouped.py:51). The gfx950 grouped kernels serve every
# tokens-per-expert, so nothing dispatches on it.
GROUPED_TOKENS_PER_EXPERT_MAX = 2048


def grouped_supported(hidden, gate_up_proj, down_proj):
    """True iff the HIP grouped path can run these tensors: a device tensor of float32 / float16 /
    bfloat16 and H, 2I, I multiples of 8 (16-byte rows), as in moe_grouped.py:54-66."""
    if hidden.device.type != "cuda":
        return False
    if hidden.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        return False
    h = hidden.shape[1]
    two_i = gate_up_proj.shape[1]
    inner = down_proj.shape[2]
    return h % 8 == 0 and two_i % 8 == 0 and inner % 8 == 0


def prefer_grouped(top_k_indices, gate_up_proj):
    """The reference's tokens-per-expert heuristic (moe_grouped.py:69-74). The answer does not
    change the path here; it is kept so callers that consult it keep working."""
    e_glu = gate_up_proj.shape[0]
    return top_k_indices.numel() / max(e_glu, 1) <= GROUPED_TOKENS_PER_EXPERT_MAX


def moe_grouped_cublas_polyglu(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj,
                               act_codes):
    """Grouped PolyGLU MoE over GLU experts plus Identity (3) / Zero (4) specials on the tail
    (moe_grouped.py:77-122). Like the reference it rejects code 5 (SiTU needs act_params)."""
    if _code_max(act_codes) > 4:
        raise ValueError("code 5 (SiTU) unsupported on the grouped path; use moe_per_expert(act_params=...)")
    return _MoEFunction.apply(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj,
                              act_codes, None)


def moe(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj, act_codes, act_params=None):
    """Drop-in for kernels/sm120/moe.py:32-48; one implementation serves both of its branches."""
    return moe_per_expert(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj, act_codes,
                          act_params)
