"""Router epilogue on gfx950: the step between the router logits and dispatch.

API follows the reference `kernels.sm75.router` / `kernels.sm120.router`
(/root/reference/kernels/sm75/router.py:29-30,170-301):
    fused_mlp_router(x, gate_weight, bias, top_k, num_experts, norm_topk_prob=True,
                     routed_scaling_factor=1.0, return_counts=False)            (router.py:269)
    fused_router(x, conv_weight, bias, top_k, num_experts, ...)                (router.py:254)
    router_bias_update(bias, counts, u)                                        (router.py:293)
    FusedMLPRouter.apply / FusedConvRouterCuDNN.apply (same arguments, (idx, w, counts))
and one addition, `router_topk(logits, ...)`, the epilogue alone for callers that make their own
logits. Every entry point also takes `score_func="sigmoid"` (the reference's gate) or "softmax".

The epilogue (scores, bias-steered top-k, unbiased gathered weights, sum-to-1 norm, routed scaling,
per-expert counts) and its backward are HIP kernels (csrc/moe_router.hip). The logits projection
itself is a plain dense GEMM (MLP router) or a causal conv1d (conv router) and runs
as a PyTorch op (hipBLASLt / MIOpen), as the reference runs it in cuBLAS / cuDNN.
"""
import torch
import torch.nn.functional as F

from .. import _lib

__all__ = ["router_topk", "fused_mlp_router", "fused_router", "router_bias_update",
           "FusedMLPRouter", "FusedConvRouterCuDNN", "FusedConvRouterFused"]

_SCORE = {"sigmoid": 0, "softmax": 1}


def _score_code(score_func):
    try:
        return _SCORE[score_func]
    except KeyError:
        raise ValueError(f"score_func must be 'sigmoid' or 'softmax', got {score_func!r}") from None


class _RouterTopk(torch.autograd.Function):
    """logits (N,E) -> (idx (N,k) int64, w (N,k) fp32, counts (E,) int32 or None); only w is
    differentiable (kernels/sm75/router.py:40-150)."""

    @staticmethod
    def forward(ctx, logits, bias, top_k, num_experts, norm, scale, softmax):
        if not logits.is_cuda:
            raise RuntimeError("router_topk runs on the GPU only (HIP kernels, no CPU fallback)")
        if logits.dim() != 2:
            raise ValueError("logits must be (N, E)")
        if logits.stride(1) != 1:
            logits = logits.contiguous()
        n, e = logits.shape
        if num_experts is not None and num_experts != e:
            raise ValueError(f"num_experts={num_experts} but logits have {e} columns")
        dev = logits.device
        idx = torch.empty(n, top_k, device=dev, dtype=torch.long)
        w = torch.empty(n, top_k, device=dev, dtype=torch.float32)
        counts = torch.zeros(e, device=dev, dtype=torch.int32) if num_experts else None
        b = bias.detach().float().contiguous() if bias is not None else None
        _lib.call("moe_router_topk_fwd", _lib.dtype_code(logits.dtype), _lib.ptr(logits),
                  logits.stride(0), n, e, _lib.ptr(b), top_k, softmax, int(norm), float(scale),
                  _lib.ptr(idx), _lib.ptr(w), _lib.ptr(counts), _lib.stream_of(dev))
        ctx.save_for_backward(logits, idx)
        ctx.cfg = (top_k, int(norm), float(scale), softmax)
        ctx.mark_non_differentiable(idx)
        if counts is not None:
            ctx.mark_non_differentiable(counts)
        return idx, w, counts

    @staticmethod
    def backward(ctx, grad_idx, grad_w, grad_counts):
        logits, idx = ctx.saved_tensors
        top_k, norm, scale, softmax = ctx.cfg
        n, e = logits.shape
        g = torch.empty(n, e, device=logits.device, dtype=logits.dtype)
        if grad_w is None:
            return g.zero_(), None, None, None, None, None, None
        gw = grad_w.float().contiguous()
        _lib.call("moe_router_topk_bwd", _lib.dtype_code(logits.dtype), _lib.ptr(logits),
                  logits.stride(0), n, e, _lib.ptr(idx), _lib.ptr(gw), top_k, softmax, norm,
                  scale, _lib.ptr(g), e, _lib.stream_of(logits.device))
        return g, None, None, None, None, None, None


def router_topk(logits, bias, top_k, num_experts=None, norm_topk=True, scale=1.0,
                score_func="sigmoid"):
    """The fused epilogue alone: (idx (N,k) long, weights (N,k) fp32 FINAL, counts (E,) int32 or
    None). norm_topk applies for top_k > 1, as in the reference (router.py:142)."""
    return _RouterTopk.apply(logits, bias, int(top_k), num_experts, bool(norm_topk and top_k > 1),
                             float(scale), _score_code(score_func))


def _amp(*ts):
    if torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        return tuple(t.to(dt) for t in ts)
    return ts


class FusedMLPRouter:
    """MLP router as one call: logits = x @ gate_weight^T, then the fused epilogue. Returns
    (idx (N,k) long, weights (N,k) fp32, counts (E,) int32); only weights are differentiable
    (kernels/sm75/router.py:208-250)."""

    @staticmethod
    def apply(x, weight, bias, top_k, num_experts, norm_topk=True, scale=1.0, score_func="sigmoid"):
        x, weight = _amp(x, weight)
        logits = x.reshape(-1, x.shape[-1]) @ weight.t()
        return router_topk(logits, bias, top_k, num_experts, norm_topk, scale, score_func)


class FusedConvRouterCuDNN:
    """Conv router as one call: causal conv1d over the sequence (padding K-1, first S outputs),
    then the fused epilogue. x (B,S,H), weight (E,H,K) (kernels/sm75/router.py:170-205)."""

    @staticmethod
    def apply(x, weight, bias, top_k, num_experts, norm_topk=True, scale=1.0, score_func="sigmoid"):
        x, weight = _amp(x, weight)
        b, s, _ = x.shape
        e, _, k = weight.shape
        conv = F.conv1d(x.transpose(1, 2), weight, padding=k - 1)[..., :s]   # (B,E,S), causal
        logits = conv.transpose(1, 2).reshape(b * s, e)
        return router_topk(logits, bias, top_k, num_experts, norm_topk, scale, score_func)


FusedConvRouterFused = FusedConvRouterCuDNN   # sm120 name (kernels/sm120/router.py)


def fused_mlp_router(x, gate_weight, bias, top_k, num_experts, norm_topk_prob=True,
                     routed_scaling_factor=1.0, return_counts=False, score_func="sigmoid"):
    """x (B,S,H) or (N,H), gate_weight (E,H), bias (E,) fp32 or None. Returns (idx, weights) with
    (B,S,k) shapes for 3-D x — or (..., counts) when return_counts (router.py:269-290)."""
    idx, w, counts = FusedMLPRouter.apply(x, gate_weight, bias, top_k, num_experts,
                                          norm_topk_prob, routed_scaling_factor, score_func)
    if x.ndim == 3:
        b, s, _ = x.shape
        idx, w = idx.view(b, s, top_k), w.view(b, s, top_k)
    return (idx, w, counts) if return_counts else (idx, w)


def fused_router(x, conv_weight, bias, top_k, num_experts, norm_topk_prob=True,
                 routed_scaling_factor=1.0, return_counts=False, score_func="sigmoid"):
    """Conv router. x (B,S,H), conv_weight (E,H,K). Returns (idx (B,S,k), weights (B,S,k)) — or
    (..., counts) when return_counts (router.py:254-266)."""
    b, s, _ = x.shape
    idx, w, counts = FusedConvRouterCuDNN.apply(x, conv_weight, bias, top_k, num_experts,
                                                norm_topk_prob, routed_scaling_factor, score_func)
    idx, w = idx.view(b, s, top_k), w.view(b, s, top_k)
    return (idx, w, counts) if return_counts else (idx, w)


@torch.no_grad()
def router_bias_update(bias, counts, u):
    """bias += u * sign(mean(counts) - counts), in place, fp32 bias; counts must already be the
    global load (router.py:293-301). No-op for u <= 0."""
    if u <= 0:
        return
    if bias.dtype != torch.float32 or not bias.is_contiguous():
        raise ValueError("bias must be a contiguous fp32 tensor")
    c = counts.detach().to(device=bias.device, dtype=torch.int32).contiguous()
    _lib.call("moe_router_bias_update", _lib.ptr(bias), _lib.ptr(c), bias.numel(), float(u),
              _lib.stream_of(bias.device))
