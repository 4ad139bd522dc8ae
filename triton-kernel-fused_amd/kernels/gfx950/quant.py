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


# ───────────────────────── persisted expert-weight format ─────────────────────────
# One safetensors file per MoE layer (a JSON header + raw little-endian tensors; no code is
# executed on load, and a C reader needs only the 8-byte header length and the JSON offsets).
# Tensor names and layouts are exactly what moe_fp8 / moe_mxfp8 read, so a loaded file goes to the
# kernels without any re-layout (only a host-to-device copy):
#   "gate_up_q"     (E, 2I, H) float8_e4m3fn  rows [0, I) gate, rows [I, 2I) up (the reference's
#                                             gate_up_proj layout, kernels/sm75/moe.py:65-68,170-171)
#   "down_q"        (E, H, I)  float8_e4m3fn  (the reference's down_proj layout)
#   fp8:   "gate_up_scale" (E, 2I) float32, "down_scale" (E, H) float32: one scale per output
#          channel (weight row), dequantised w = q * scale[row]
#   mxfp8: "gate_up_scale" (E, 2I, H/32) uint8, "down_scale" (E, H, I/32) uint8: E8M0 exponent
#          byte per 32 consecutive K values of a row, dequantised w = q * 2^(byte - 127)
# Header metadata: format = "moe-gfx950-fp8" | "moe-gfx950-mxfp8", version = "1", and E, H, I.
EXPERT_FORMAT_VERSION = "1"
_FORMATS = ("fp8", "mxfp8")


def quantize_experts(gate_up_proj, down_proj, fmt):
    """Quantise a layer's expert weights (E,2I,H) / (E,H,I) to `fmt` ("fp8" per-channel or
    "mxfp8" E8M0 blocks along K). Returns dict(gate_up_q, gate_up_scale, down_q, down_scale)."""
    if fmt not in _FORMATS:
        raise ValueError(f"format must be one of {_FORMATS}, got {fmt!r}")
    qf = quantize_fp8_rows if fmt == "fp8" else quantize_mxfp8
    guq, gus = qf(gate_up_proj)
    dq, ds = qf(down_proj)
    return dict(gate_up_q=guq, gate_up_scale=gus, down_q=dq, down_scale=ds)


def _check_expert_tensors(t, fmt):
    guq, gus, dq, ds = t["gate_up_q"], t["gate_up_scale"], t["down_q"], t["down_scale"]
    if guq.dtype != torch.float8_e4m3fn or dq.dtype != torch.float8_e4m3fn:
        raise ValueError("gate_up_q / down_q must be float8_e4m3fn")
    if guq.dim() != 3 or guq.shape[1] % 2:
        raise ValueError("gate_up_q must be (E, 2I, H)")
    e, two_i, h = guq.shape
    i = two_i // 2
    if tuple(dq.shape) != (e, h, i):
        raise ValueError(f"down_q must be (E, H, I) = {(e, h, i)}, got {tuple(dq.shape)}")
    if fmt == "fp8":
        want = ((e, two_i), (e, h), torch.float32)
    else:
        if h % MX_BLOCK or i % MX_BLOCK:
            raise ValueError("MXFP8 needs H and I to be multiples of 32")
        want = ((e, two_i, h // MX_BLOCK), (e, h, i // MX_BLOCK), torch.uint8)
    if tuple(gus.shape) != want[0] or tuple(ds.shape) != want[1] or gus.dtype != want[2] \
            or ds.dtype != want[2]:
        raise ValueError(f"{fmt} scales must be {want[0]} / {want[1]} {want[2]}, got "
                         f"{tuple(gus.shape)} {gus.dtype} / {tuple(ds.shape)} {ds.dtype}")
    return e, h, i


def save_experts(path, tensors, fmt):
    """Write quantised expert weights (the dict quantize_experts returns) to `path`."""
    from safetensors.torch import save_file
    if fmt not in _FORMATS:
        raise ValueError(f"format must be one of {_FORMATS}, got {fmt!r}")
    e, h, i = _check_expert_tensors(tensors, fmt)
    meta = dict(format=f"moe-gfx950-{fmt}", version=EXPERT_FORMAT_VERSION, E=str(e), H=str(h),
                I=str(i))
    save_file({k: tensors[k].detach().contiguous().cpu()
               for k in ("gate_up_q", "gate_up_scale", "down_q", "down_scale")}, path,
              metadata=meta)


def load_experts(path, device="cpu"):
    """Read a file written by save_experts. Returns (fmt, dict of tensors on `device`); raises
    ValueError for another format, an unknown version or inconsistent shapes."""
    from safetensors import safe_open
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        fmt_tag = meta.get("format", "")
        if not fmt_tag.startswith("moe-gfx950-") or fmt_tag[len("moe-gfx950-"):] not in _FORMATS:
            raise ValueError(f"{path}: not a gfx950 MoE expert-weight file (format {fmt_tag!r})")
        if meta.get("version") != EXPERT_FORMAT_VERSION:
            raise ValueError(f"{path}: format version {meta.get('version')!r}, this library reads "
                             f"{EXPERT_FORMAT_VERSION!r}")
        fmt = fmt_tag[len("moe-gfx950-"):]
        names = set(f.keys())
        need = {"gate_up_q", "gate_up_scale", "down_q", "down_scale"}
        if names != need:
            raise ValueError(f"{path}: tensors {sorted(names)}, expected {sorted(need)}")
        t = {k: f.get_tensor(k) for k in need}
    e, h, i = _check_expert_tensors(t, fmt)
    if (str(e), str(h), str(i)) != (meta.get("E"), meta.get("H"), meta.get("I")):
        raise ValueError(f"{path}: header E/H/I {meta.get('E')}/{meta.get('H')}/{meta.get('I')} "
                         f"disagree with the tensors {e}/{h}/{i}")
    return fmt, {k: v.to(device) for k, v in t.items()}
