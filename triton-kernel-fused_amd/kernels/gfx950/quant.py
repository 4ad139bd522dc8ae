"""fp8-e4m3 and MXFP8 quantisers: the weight / activation formats the fp8 kernels read.

fp8 (per-channel / per-token): q = round_e4m3(x / s) with s = absmax(row) / 448, so the largest
element maps to the largest finite e4m3fn value (448) and nothing saturates. Scales are fp32.

MXFP8 (OCP Microscaling v1.0, e4m3 elements): along the last dim every block of 32 elements shares
one E8M0 scale 2^(floor(log2(absmax)) - 8) (8 = exponent of e4m3's largest normal); elements are
round_e4m3(x / 2^e) clamped to +-448. The scale is stored as the biased exponent byte e + 127
(0 means 2^-127; an all-zero block stores 0).
"""
import torch

FP8_MAX = 448.0
MX_BLOCK = 32
_E4M3_EMAX = 8


def quantize_fp8_rows(x):
    """Per-row (last dim) absmax fp8-e4m3 quantisation. Returns (q float8_e4m3fn, scale fp32 (...))."""
    xf = x.float()
    amax = xf.abs().amax(dim=-1)
    scale = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = (xf / scale.unsqueeze(-1)).clamp_(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q, scale


def dequantize_fp8_rows(q, scale):
    return q.float() * scale.unsqueeze(-1)


def quantize_mxfp8(x):
    """MXFP8 along the last dim (a multiple of 32). Returns (q float8_e4m3fn same shape,
    scale_e8m0 uint8 (..., K/32))."""
    *lead, k = x.shape
    if k % MX_BLOCK:
        raise ValueError(f"MXFP8 needs the last dim to be a multiple of {MX_BLOCK}, got {k}")
    xb = x.float().reshape(*lead, k // MX_BLOCK, MX_BLOCK)
    amax = xb.abs().amax(dim=-1)
    e = torch.floor(torch.log2(amax.clamp_min(torch.finfo(torch.float32).tiny))) - _E4M3_EMAX
    e = torch.where(amax > 0, e, torch.full_like(e, -127.0)).clamp_(-127.0, 127.0)
    q = (xb * torch.exp2(-e).unsqueeze(-1)).clamp_(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.reshape(*lead, k), (e + 127).to(torch.uint8)


def dequantize_mxfp8(q, scale_e8m0):
    *lead, k = q.shape
    s = torch.exp2(scale_e8m0.float() - 127.0)
    return (q.float().reshape(*lead, k // MX_BLOCK, MX_BLOCK) * s.unsqueeze(-1)).reshape(*lead, k)
