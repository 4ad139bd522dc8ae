"""Seeded synthetic MoE workloads: the five benchmark configurations of this build.

    1 "cpu_plumbing"   fp32  N=1024  H=256  I=512  E=8   k=2  router x@W_r (W_r~N(0,0.02)), softmax
    2 "dense_bf16"     bf16  N=8192  H=1024 I=2816 E=8   k=2  Gaussian logits, softmax
    3 "many_experts"   bf16  N=16384 H=2048 I=1024 E=64  k=8  Gaussian logits + log-Zipf bias, sigmoid
    4 "fp8_fwd"        fp8   N=16384 H=4096 I=1536 E=128 k=8  Gaussian logits, softmax
    5 "mxfp8_decode"   MXFP8 N=128   H=7168 I=2048 E=256 k=8  uniform-random experts, sigmoid gates

Every config: SwiGLU experts (act code 0); weights ~ N(0, 1/sqrt(fan_in)) laid out as the reference
expects (gate_up_proj (E,2I,H), down_proj (E,H,I)); x ~ N(0,1); top-k gates renormalised to sum 1;
upstream grad dY ~ N(0,1). One torch.Generator seeded with `seed` draws, in order: x, gate_up_proj,
down_proj, router, dY.

Config 3's bias: experts are ranked by a seeded random permutation (rank 1..E) and expert e gets
bias c * ln(rank_e^-1.2) with c = ZIPF_C = 1.75 (a Zipf(1.2) popularity on a log scale). The top
ranks are picked by nearly every token and the tail by almost none, so group sizes span 0..N.

The reference's own MoE benchmark stack (bench_moe, /root/reference/bench.py:617-631), by name:
  "bench_moe_stack"      bf16 N=16384 H=512 I=768, 9 GLU experts with codes i % 3 (SiLU, ReLU^2,
                         NormSiLU) + Identity + Zero, k=2; hidden ~ 0.1 N(0,1), weights ~ 0.02 N(0,1),
                         top-2 of softmax(N(0,1) logits) over all 11 experts, not renormalised
  "bench_moe_stack_e32"  the same with 32 GLU experts (the size of the reference's published
                         grouped-path run, .autoresearch/moe_grouped_results.jsonl:23)
Code 2 is RMS-normalised, so these stacks take the unfused GLU path (row kernels between the GEMMs).

Routing variants of config 3's shapes (same N, H, I, E, k, sigmoid gates), for robustness lines:
  router="zipf_power_sigmoid"  bias c * rank^-1.2 (the power form, c = ZIPF_C): milder skew
  router="uniform_topk_sigmoid" Gaussian logits only: near-uniform groups
"""
import math

import torch

from .gfx950.quant import quantize_fp8_rows, quantize_mxfp8

ZIPF_ALPHA = 1.2
ZIPF_C = 1.75

CONFIGS = {
    1: dict(name="cpu_plumbing", N=1024, H=256, I=512, E=8, k=2, dtype=torch.float32,
            router="linear_softmax", fmt="dense"),
    2: dict(name="dense_bf16", N=8192, H=1024, I=2816, E=8, k=2, dtype=torch.bfloat16,
            router="gauss_softmax", fmt="dense"),
    3: dict(name="many_experts_zipf", N=16384, H=2048, I=1024, E=64, k=8, dtype=torch.bfloat16,
            router="zipf_sigmoid", fmt="dense"),
    4: dict(name="fp8_fwd", N=16384, H=4096, I=1536, E=128, k=8, dtype=torch.bfloat16,
            router="gauss_softmax", fmt="fp8"),
    5: dict(name="mxfp8_decode", N=128, H=7168, I=2048, E=256, k=8, dtype=torch.bfloat16,
            router="uniform_sigmoid", fmt="mxfp8"),
    "bench_moe_stack": dict(name="bench_moe_stack", N=16384, H=512, I=768, E=11, k=2,
                            dtype=torch.bfloat16, router="stack_softmax", fmt="dense",
                            codes=[i % 3 for i in range(9)] + [3, 4]),
    "bench_moe_stack_e32": dict(name="bench_moe_stack_e32", N=16384, H=512, I=768, E=34, k=2,
                                dtype=torch.bfloat16, router="stack_softmax", fmt="dense",
                                codes=[i % 3 for i in range(32)] + [3, 4]),
}


def n_glu(cfg):
    """Weight slots of a config: the experts whose code is a GLU code (all of them by default)."""
    codes = cfg.get("codes")
    return cfg["E"] if codes is None else sum(1 for c in codes if c not in (3, 4))


def glu_rows(cfg, idx):
    """Routed rows that run through the GLU experts' GEMMs (specials run none)."""
    return int(((idx >= 0) & (idx < n_glu(cfg))).sum())


def flops(cfg_or_m, H=None, I=None, backward=True):
    """Algorithmic FLOPs of the three projections over M routed rows: forward 6*M*H*I, backward
    12*M*H*I (dX and dW of each GEMM)."""
    if isinstance(cfg_or_m, dict):
        c = cfg_or_m
        m, H, I = c["N"] * c["k"], c["H"], c["I"]
    else:
        m = cfg_or_m
    f = 6 * m * H * I
    return f * 3 if backward else f


def _route(cfg, hidden, g, dev):
    n, e, k = cfg["N"], cfg["E"], cfg["k"]
    kind = cfg["router"]
    if kind == "linear_softmax":
        w_r = torch.randn(cfg["H"], e, generator=g, device=dev) * 0.02
        logits = hidden.float() @ w_r
        probs = torch.softmax(logits, dim=-1)
        w, idx = torch.topk(probs, k, dim=-1)
    elif kind == "gauss_softmax":
        logits = torch.randn(n, e, generator=g, device=dev)
        w, idx = torch.topk(torch.softmax(logits, dim=-1), k, dim=-1)
    elif kind == "zipf_sigmoid":
        logits = torch.randn(n, e, generator=g, device=dev)
        rank = torch.randperm(e, generator=g, device=dev).float() + 1.0
        bias = ZIPF_C * torch.log(rank ** -ZIPF_ALPHA)
        w, idx = torch.topk(torch.sigmoid(logits + bias), k, dim=-1)
    elif kind == "zipf_power_sigmoid":
        logits = torch.randn(n, e, generator=g, device=dev)
        rank = torch.randperm(e, generator=g, device=dev).float() + 1.0
        bias = ZIPF_C * rank ** -ZIPF_ALPHA
        w, idx = torch.topk(torch.sigmoid(logits + bias), k, dim=-1)
    elif kind == "uniform_topk_sigmoid":
        logits = torch.randn(n, e, generator=g, device=dev)
        w, idx = torch.topk(torch.sigmoid(logits), k, dim=-1)
    elif kind == "stack_softmax":   # bench.py:630-631: softmax top-k, gates not renormalised
        logits = torch.randn(n, e, generator=g, device=dev)
        w, idx = torch.topk(torch.softmax(logits, dim=-1), k, dim=-1)
        return idx.long(), w
    elif kind == "uniform_sigmoid":
        logits = torch.randn(n, e, generator=g, device=dev)
        choice = torch.rand(n, e, generator=g, device=dev)
        idx = torch.topk(choice, k, dim=-1).indices
        w = torch.sigmoid(logits.gather(1, idx))
    else:
        raise ValueError(kind)
    w = w / w.sum(-1, keepdim=True)
    return idx.long(), w


def make_workload(config, device="cpu", seed=0, gen_device=None, scale=None):
    """Build the inputs of a config. `gen_device` is where the random numbers are drawn (default
    `device`); drawing on the CPU makes small configs identical across hosts. `scale` overrides
    sizes, e.g. dict(N=256) for a reduced parity case of the same routing and dtype."""
    cfg = dict(CONFIGS[config]) if isinstance(config, (int, str)) else dict(config)
    if scale:
        cfg.update(scale)
    gd = torch.device(gen_device or device)
    g = torch.Generator(device=gd).manual_seed(seed)
    n, h, i, e, k = cfg["N"], cfg["H"], cfg["I"], cfg["E"], cfg["k"]
    dt = cfg["dtype"]
    e_w = n_glu(cfg)
    if cfg["router"] == "stack_softmax":   # the reference bench's value scales (bench.py:626-628)
        hidden = torch.randn(n, h, generator=g, device=gd) * 0.1
        gate_up = torch.randn(e_w, 2 * i, h, generator=g, device=gd) * 0.02
        down = torch.randn(e_w, h, i, generator=g, device=gd) * 0.02
    else:
        hidden = torch.randn(n, h, generator=g, device=gd)
        gate_up = torch.randn(e_w, 2 * i, h, generator=g, device=gd) * (1.0 / math.sqrt(h))
        down = torch.randn(e_w, h, i, generator=g, device=gd) * (1.0 / math.sqrt(i))
    idx, wt = _route(cfg, hidden, g, gd)
    grad_out = torch.randn(n, h, generator=g, device=gd)
    codes = cfg.get("codes") or [0] * e
    out = dict(cfg=cfg, idx=idx.to(device),
               act_codes=torch.tensor(codes, dtype=torch.int32, device=device))
    if cfg["fmt"] == "dense":
        out.update(hidden=hidden.to(device, dt), wt=wt.to(device, dt),
                   gate_up_proj=gate_up.to(device, dt), down_proj=down.to(device, dt),
                   grad_out=grad_out.to(device, dt))
    elif cfg["fmt"] == "fp8":
        xq, xs = quantize_fp8_rows(hidden)
        guq, gus = quantize_fp8_rows(gate_up)
        dq, ds = quantize_fp8_rows(down)
        out.update(hidden=hidden.to(device, dt),
                   x_q=xq.to(device), x_scale=xs.to(device), wt=wt.to(device, dt),
                   gate_up_q=guq.to(device), gate_up_scale=gus.to(device),
                   down_q=dq.to(device), down_scale=ds.to(device))
    elif cfg["fmt"] == "mxfp8":
        guq, gus = quantize_mxfp8(gate_up)
        dq, ds = quantize_mxfp8(down)
        out.update(hidden=hidden.to(device, dt), wt=wt.to(device, dt),
                   gate_up_q=guq.to(device), gate_up_scale=gus.to(device),
                   down_q=dq.to(device), down_scale=ds.to(device))
    return out
