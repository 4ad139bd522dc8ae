"""Quantised MoE forwards on gfx950 (inference; no autograd): fp8-e4m3 and MXFP8 weights.

    moe_fp8(x_q, x_scale, top_k_indices, top_k_weights, gate_up_q, gate_up_scale, down_q, down_scale)
    moe_mxfp8(hidden, top_k_indices, top_k_weights, gate_up_q, gate_up_scale, down_q, down_scale)

The reference has no quantised MoE; these follow its weight layout (gate_up (E,2I,H) with gate
rows first, down (E,H,I); kernels/sm75/moe.py:65-68) and its SwiGLU experts, and reuse the same
dispatch and gate-weighted combine. Formats (produce them with kernels.gfx950.quant):
  fp8:   x_q (N,H) float8_e4m3fn + x_scale (N,) fp32 per token; gate_up_q (E,2I,H) e4m3 +
         gate_up_scale (E,2I) fp32 per output channel; down_q (E,H,I) + down_scale (E,H).
  MXFP8: hidden (N,H) bf16; gate_up_q (E,2I,H) e4m3 + gate_up_scale (E,2I,H/32) uint8 E8M0;
         down_q (E,H,I) + down_scale (E,H,I/32).
The fp8 path re-quantises the SwiGLU intermediate before the down projection with one
power-of-two scale per routed row and 128-channel block (the smallest 2^e with 448 * 2^e >= the
block's absmax; oracle.moe_oracle.e8m0_block_requant states it). Output: (N,H) bf16.
"""
import torch

from .. import _lib
from .moe import _CHECK_INDICES, _Routing

__all__ = ["moe_fp8", "moe_mxfp8", "rowquant_fp8"]


def _check_common(idx, wt, n_tokens, gate_up_q, down_q):
    if not gate_up_q.is_cuda:
        raise RuntimeError("the gfx950 MoE path needs device tensors")
    if idx.dim() != 2 or idx.shape[0] != n_tokens or wt.shape != idx.shape:
        raise ValueError("top_k_indices / top_k_weights must be (N, k)")
    if idx.dtype != torch.int64:
        raise TypeError("top_k_indices must be int64")
    if gate_up_q.dtype != torch.float8_e4m3fn or down_q.dtype != torch.float8_e4m3fn:
        raise TypeError("quantised weights must be torch.float8_e4m3fn")
    e, two_i, h = gate_up_q.shape
    if down_q.shape != (e, h, two_i // 2):
        raise ValueError("expected gate_up_q (E,2I,H) and down_q (E,H,I)")
    return e, h, two_i // 2


_ZERO_CODES = {}   # (device index, E) -> all-SwiGLU act codes, read-only


def _combine(eo, wt, idx, routing, n_tok, h, e):
    out = torch.empty(n_tok, h, device=eo.device, dtype=torch.bfloat16)
    key = (eo.device.index, e)
    codes = _ZERO_CODES.get(key)
    if codes is None:
        codes = _ZERO_CODES[key] = torch.zeros(e, device=eo.device, dtype=torch.int32)
    _lib.call("moe_combine_fwd", _lib.dtype_code(torch.bfloat16), _lib.ptr(eo), _lib.ptr(eo),
              _lib.ptr(wt), _lib.ptr(idx), _lib.ptr(codes), e, e, _lib.ptr(routing.flat_to_sorted),
              n_tok, idx.shape[1], h, 0, _lib.ptr(out), _lib.stream_of(eo.device))
    return out


@torch.no_grad()
def moe_fp8(x_q, x_scale, top_k_indices, top_k_weights, gate_up_q, gate_up_scale, down_q,
            down_scale):
    n_tok, h_in = x_q.shape
    e, h, inter_dim = _check_common(top_k_indices, top_k_weights, n_tok, gate_up_q, down_q)
    if h_in != h or x_q.dtype != torch.float8_e4m3fn:
        raise ValueError("x_q must be (N, H) float8_e4m3fn")
    if h % 128 or inter_dim % 128:
        raise ValueError("the fp8 path needs H and I to be multiples of 128")
    dev = x_q.device
    idx = top_k_indices.contiguous()
    wt = top_k_weights.to(torch.bfloat16).contiguous()
    m = idx.numel()
    routing = _Routing(idx, e, want_status=_CHECK_INDICES)
    inter_q = torch.empty(m, inter_dim, device=dev, dtype=torch.float8_e4m3fn)
    inter_bs = torch.empty(max(1, _lib.lib().moe_fp8_inter_bscale_bytes(inter_dim, m, e)),
                           device=dev, dtype=torch.uint8)
    eo = torch.empty(m, h, device=dev, dtype=torch.bfloat16)
    if m:
        _lib.call("moe_fp8_fwd", _lib.ptr(x_q.contiguous()), _lib.ptr(x_scale.float().contiguous()),
                  n_tok, h, _lib.ptr(gate_up_q.contiguous()),
                  _lib.ptr(gate_up_scale.float().contiguous()), _lib.ptr(down_q.contiguous()),
                  _lib.ptr(down_scale.float().contiguous()), e, inter_dim,
                  _lib.ptr(routing.offsets), _lib.ptr(routing.sorted_token), m, _lib.ptr(inter_q),
                  _lib.ptr(inter_bs), _lib.ptr(eo), _lib.stream_of(dev))
    return _combine(eo, wt, idx, routing, n_tok, h, e)


@torch.no_grad()
def moe_mxfp8(hidden, top_k_indices, top_k_weights, gate_up_q, gate_up_scale, down_q, down_scale):
    n_tok, h_in = hidden.shape
    e, h, inter_dim = _check_common(top_k_indices, top_k_weights, n_tok, gate_up_q, down_q)
    if h_in != h:
        raise ValueError("hidden must be (N, H)")
    if h % 512 or inter_dim % 512:
        raise ValueError("the MXFP8 path needs H and I to be multiples of 512")
    if gate_up_scale.shape != (e, 2 * inter_dim, h // 32) or down_scale.shape != (e, h, inter_dim // 32):
        raise ValueError("MXFP8 scales must be (E,2I,H/32) and (E,H,I/32) uint8 E8M0")
    dev = hidden.device
    x = hidden.to(torch.bfloat16).contiguous()
    idx = top_k_indices.contiguous()
    wt = top_k_weights.to(torch.bfloat16).contiguous()
    m = idx.numel()
    routing = _Routing(idx, e, want_status=_CHECK_INDICES)
    inter = torch.empty(m, inter_dim, device=dev, dtype=torch.bfloat16)
    eo = torch.empty(m, h, device=dev, dtype=torch.bfloat16)
    if m:
        _lib.call("moe_mxfp8_fwd", _lib.ptr(x), n_tok, h, _lib.ptr(gate_up_q.contiguous()),
                  _lib.ptr(gate_up_scale.contiguous()), _lib.ptr(down_q.contiguous()),
                  _lib.ptr(down_scale.contiguous()), e, inter_dim, _lib.ptr(routing.offsets),
                  _lib.ptr(routing.sorted_token), m, _lib.ptr(inter), _lib.ptr(eo),
                  _lib.stream_of(dev))
    return _combine(eo, wt, idx, routing, n_tok, h, e)


@torch.no_grad()
def rowquant_fp8(x):
    """Per-row absmax e4m3 quantisation of a bf16 (M, K) matrix on the device."""
    x = x.to(torch.bfloat16).contiguous()
    m, k = x.shape
    q = torch.empty(m, k, device=x.device, dtype=torch.float8_e4m3fn)
    s = torch.empty(max(m, 1), device=x.device, dtype=torch.float32)
    _lib.call("moe_rowquant_fp8", _lib.ptr(x), m, k, _lib.ptr(q), _lib.ptr(s),
              _lib.stream_of(x.device))
    return q, s[:m]
