"""Benchmark of the gfx950 MoE layer (one GPU). Prints ONE JSON line.

    python bench.py [--steps K] [--warmup W] [--config 3] [--no-cpu] [--no-extra]

Workload (value): BASELINE config 3 — bf16 MoE layer fwd+bwd, N=16384 tokens, d_model=2048,
d_ff=1024, E=64 SwiGLU experts, top-8 sigmoid routing with log-Zipf expert bias (imbalanced, some
experts empty). One step = dispatch + grouped gate/up GEMM with SwiGLU + grouped down GEMM +
combine, then the full backward (combine bwd, down dX + SwiGLU bwd, both wgrads, gate/up dX,
un-permute) for every input and weight, with inputs already resident in HBM.
value = algorithmic TFLOP/s = 18*M*H*I / step time (M = N*k routed rows; forward 6*M*H*I,
backward 12*M*H*I; routing, elementwise and scatter work excluded).

Extra fields beside the contract: per-kernel HIP-event timings over the timed region ("kernels"),
the roofline of the dominant kernel ("roofline"), the CPU baseline ("cpu_baseline") and the
other bf16 config ("extra_configs").
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "triton-kernel-fused_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MoE layer TFLOP/s (bf16 fwd+bwd, fp8/MXFP8 fwd) and % of MI355X MFMA/HBM peak"
PEAK_BF16_TFLOPS = 2500.0    # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0     # MI355X dense fp8 MFMA
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E

# algorithmic FLOPs per call of each entry point, in units of M*H*I (M = routed GLU rows)
KERNEL_MHI = {
    "moe_grouped_gateup_swiglu_fwd": 4, "moe_grouped_down_fwd": 2,
    "moe_grouped_down_dx_swiglu_bwd": 2, "moe_grouped_down_dx_gated_bwd": 2, "moe_grouped_gateup_dx": 4,
    "moe_grouped_wgrad:down": 2, "moe_grouped_wgrad:gate_up": 4,
}


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _traffic(kernel, workload):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summary, if any."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f)[workload][kernel]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def run_bf16(config, steps, warmup, timer=True, router=None):
    import torch
    import kernels
    from kernels import _lib
    from kernels.workloads import make_workload, flops, glu_rows

    wl = make_workload(config, device="cuda", seed=0, scale=dict(router=router) if router else None)
    cfg = wl["cfg"]
    leaves = [wl[k].detach().requires_grad_(True) for k in ("hidden", "wt", "gate_up_proj", "down_proj")]
    idx, codes, dy = wl["idx"], wl["act_codes"], wl["grad_out"]

    last = {}

    def step():
        for t in leaves:
            t.grad = None
        out = kernels.moe(leaves[0], idx, leaves[1], leaves[2], leaves[3], codes)
        out.backward(dy)
        last["out"] = out

    ms, records, k_steps = _two_passes(step, steps, warmup, timer)
    parity = _parity_sample(last["out"], leaves[0].grad, wl)
    m = glu_rows(cfg, idx)
    f = flops(m, cfg["H"], cfg["I"])
    mhi = m * cfg["H"] * cfg["I"]
    per = {}
    for name, e0, e1 in records:
        per.setdefault(name, []).append(e0.elapsed_time(e1))
    kern = {}
    for name, ts in per.items():
        avg = statistics.mean(ts)
        d = {"ms": round(avg, 4), "calls_per_step": len(ts) // k_steps}
        if name in KERNEL_MHI:
            tf = KERNEL_MHI[name] * mhi / (avg * 1e-3) / 1e12
            d.update(tflops=round(tf, 1), frac=round(tf / PEAK_BF16_TFLOPS, 4))
        kern[name] = d
    return dict(cfg=cfg, ms=ms, tflops=f / (ms * 1e-3) / 1e12, kernels=kern, mhi=mhi,
                parity=parity, glu_rows=m)


def _parity_sample(out, grad_hidden, wl, n_sample=256, seed=1):
    """Checks the output and grad_hidden of the last timed step on a seeded sample of tokens
    against the layer's fp32 math: the library's pure-PyTorch moe_eager (the reference's eager
    algorithm, kernels/sm75/moe.py:884-909) in fp32 with autograd, on the sampled tokens only
    (a token's output and input gradient depend on its own row alone). Gate: max|d| / max|ref| <
    1.5e-2 per tensor, the reference bench's pass rule (/root/reference/bench.py:151-163)."""
    import torch
    import kernels
    n = wl["hidden"].shape[0]
    g = torch.Generator(device="cpu").manual_seed(seed)
    rows = torch.randperm(n, generator=g)[:min(n_sample, n)].sort().values.to(out.device)
    x = wl["hidden"][rows].float().requires_grad_(True)
    ref = kernels.moe_eager(x, wl["idx"][rows], wl["wt"][rows].float(),
                            wl["gate_up_proj"].float(), wl["down_proj"].float(), wl["act_codes"])
    ref.backward(wl["grad_out"][rows].float())
    res = {}
    for name, mine, truth in (("out", out[rows], ref), ("grad_hidden", grad_hidden[rows], x.grad)):
        d = (mine.float() - truth).abs().max().item()
        res[name] = round(d / (truth.abs().max().item() + 1e-12), 6)
    res["tokens_checked"] = int(rows.numel())
    res["parity_ok"] = all(v < 1.5e-2 for k, v in res.items() if k in ("out", "grad_hidden"))
    return res


# The reference's published fwd+bwd times of its MoE stack (bf16, N=16384, H=512, I=768, k=2) on an
# RTX PRO 6000 (Blackwell): its grouped path and its per-expert path, 32 GLU experts
# (/root/reference/.autoresearch/moe_grouped_results.jsonl:23). Other hardware: context only.
REF_STACK_MS = {"grouped_cublas_polyglu": 3.526, "per_expert": 8.864, "E_glu": 32,
                "gpu": "RTX PRO 6000 Blackwell"}


def run_stack(name, steps, warmup):
    """The reference bench_moe stack (PolyGLU codes i % 3 with NormSiLU, plus Identity and Zero):
    bf16 fwd+bwd of kernels.moe, step time, TFLOP/s over the GLU-routed rows (18*M_glu*H*I), the
    per-kernel times and the sampled parity check."""
    r = run_bf16(name, steps, warmup)
    cfg = r["cfg"]
    out = {"ms_per_step": round(r["ms"], 4), "tflops": round(r["tflops"], 2),
           "frac_of_peak": round(r["tflops"] / PEAK_BF16_TFLOPS, 4), "glu_rows": r["glu_rows"],
           "kernels_ms": {k: v["ms"] for k, v in r["kernels"].items()}, "parity": r["parity"],
           "workload": (f"{name}: bf16 fwd+bwd N={cfg['N']} H={cfg['H']} I={cfg['I']} "
                        f"codes={cfg['codes']} k={cfg['k']} (reference bench.py:617-631 shape)")}
    if cfg["E"] - 2 == REF_STACK_MS["E_glu"]:
        out["reference_published_context"] = dict(REF_STACK_MS, note=(
            "the reference's own published times for this stack size on other hardware; context, "
            "not a target"))
    return out


def _two_passes(fn, steps, warmup, timer=True):
    """W untimed warmup calls, then EXACTLY `steps` timed calls between two synchronisations
    with nothing else on the stream (the step time), then, when `timer`, a second untimed pass of
    up to 10 calls with a HIP event pair around every library call (the per-kernel times: the
    event records add a few microseconds between kernels, which the first pass does not pay).
    Returns (ms per step, [(name, ev0, ev1)], calls in the event pass)."""
    import torch
    from kernels import _lib
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    records, k_steps = [], min(steps, 10)
    if timer:
        _lib.set_timer(records)
        try:
            for _ in range(k_steps):
                fn()
            torch.cuda.synchronize()
        finally:
            _lib.set_timer(None)
    return (t1 - t0) * 1e3 / steps, records, k_steps


def _timed(fn, steps, warmup, timer=True):
    ms, records, _ = _two_passes(fn, steps, warmup, timer)
    per = {}
    for name, e0, e1 in records:
        per.setdefault(name, []).append(e0.elapsed_time(e1))
    return ms, {k: statistics.mean(v) for k, v in per.items()}


def run_fp8(steps, warmup):
    """Config 4: fp8 forward from bf16 activations (per-token e4m3 quantisation of x, then the
    fp8 layer); FLOPs 6*M*H*I over the routed rows."""
    import kernels
    from kernels.gfx950.lowp import rowquant_fp8
    from kernels.workloads import make_workload, flops
    w = make_workload(4, device="cuda", seed=0)
    cfg = w["cfg"]
    args = (w["idx"], w["wt"], w["gate_up_q"], w["gate_up_scale"], w["down_q"], w["down_scale"])

    def step():   # a caller holds bf16 activations: the per-token quantisation is in the step
        x_q, x_scale = rowquant_fp8(w["hidden"])
        return kernels.moe_fp8(x_q, x_scale, *args)
    ms, kern = _timed(step, steps, warmup)
    f = flops(cfg, backward=False)
    call = kern.get("moe_fp8_fwd")
    return {"tflops": round(f / (ms * 1e-3) / 1e12, 2), "ms_per_step": round(ms, 4),
            "frac_of_peak": round(f / (ms * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4),
            "gemm_call_ms": round(call, 4) if call else None,
            "gemm_call_tflops": round(f / (call * 1e-3) / 1e12, 1) if call else None,
            "kernels_ms": {k: round(v, 4) for k, v in kern.items()},
            "workload": (f"{cfg['name']}: bf16 x -> per-token e4m3 quantisation -> fp8-e4m3 fwd "
                         f"N={cfg['N']} H={cfg['H']} I={cfg['I']} E={cfg['E']} k={cfg['k']}, "
                         f"peak {PEAK_FP8_TFLOPS} TFLOP/s")}


def run_mxfp8(steps, warmup):
    """Config 5: MXFP8-weight decode forward; algorithmic bytes = every touched expert's weights
    (e4m3 + one E8M0 byte per 32) + x read + out written + routing metadata."""
    import torch
    import kernels
    from kernels.workloads import make_workload
    w = make_workload(5, device="cuda", seed=0)
    cfg = w["cfg"]
    n, h, i, k = cfg["N"], cfg["H"], cfg["I"], cfg["k"]
    touched = int(torch.unique(w["idx"]).numel())
    weight_bytes = touched * 3 * h * i * (1 + 1 / 32)
    io_bytes = 2 * n * h * 2 + n * k * (8 + 2)
    args = (w["hidden"], w["idx"], w["wt"], w["gate_up_q"], w["gate_up_scale"], w["down_q"],
            w["down_scale"])
    ms, kern = _timed(lambda: kernels.moe_mxfp8(*args), steps, warmup)
    gbs = (weight_bytes + io_bytes) / (ms * 1e-3) / 1e9
    call = kern.get("moe_mxfp8_fwd")
    return {"gbs": round(gbs, 1), "ms_per_step": round(ms, 4),
            "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4), "touched_experts": touched,
            "algorithmic_bytes": int(weight_bytes + io_bytes),
            "gemm_call_ms": round(call, 4) if call else None,
            "gemm_call_gbs": round(weight_bytes / (call * 1e-3) / 1e9, 1) if call else None,
            "kernels_ms": {k2: round(v, 4) for k2, v in kern.items()},
            "workload": (f"{cfg['name']}: MXFP8 weights, bf16 activations, fwd N={n} H={h} I={i} "
                         f"E={cfg['E']} k={k}, peak {PEAK_HBM_GBS} GB/s")}


def run_router(steps, warmup):
    """Router epilogue on config 3's routing shape: fp32 logits (N=16384, E=64),
    sigmoid + selection bias + top-8 + norm + counts, then the backward from a random grad_w.
    HBM-bound; algorithmic bytes: fwd N*E*4 read + N*k*12 written, bwd N*E*4 + N*k*12 read +
    N*E*4 written."""
    import torch
    from kernels.gfx950.router import router_topk
    n, e, k = 16384, 64, 8
    g = torch.Generator(device="cuda").manual_seed(0)
    logits = torch.randn(n, e, device="cuda", generator=g).requires_grad_(True)
    bias = torch.randn(e, device="cuda", generator=g) * 0.01
    gw = torch.randn(n, k, device="cuda", generator=g)

    def step():
        _, w, _ = router_topk(logits, bias, k, e)
        w.backward(gw)
    ms, kern = _timed(step, steps, warmup)
    fwd, bwd = kern.get("moe_router_topk_fwd"), kern.get("moe_router_topk_bwd")
    fb = n * e * 4 + n * k * 12
    bb = n * e * 8 + n * k * 12
    return {"fwd_us": round(fwd * 1e3, 2), "bwd_us": round(bwd * 1e3, 2),
            "fwd_gbs": round(fb / (fwd * 1e-3) / 1e9, 1), "bwd_gbs": round(bb / (bwd * 1e-3) / 1e9, 1),
            "frac_of_peak": round((fb + bb) / ((fwd + bwd) * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "workload": f"router epilogue fwd+bwd, fp32 logits N={n} E={e} top-{k}, sigmoid, bias, norm"}


def run_vendor_dense(config, steps, warmup):
    """Context, not a product path: the six GEMMs of one fwd+bwd step of `config` as DENSE bf16
    torch.matmul calls (hipBLASLt) on the same shapes (M = N*k rows: 2*M*H*2I, 2*M*I*H, 2*M*H*I,
    2*M*I*H, 2*M*2I*H, 2*M*2I*H FLOP), with no grouping, gather, routing or fused epilogue: the
    vendor library's rate for the layer's FLOPs on this chip."""
    import torch
    from kernels.workloads import CONFIGS
    c = CONFIGS[config]
    m, h, i = c["N"] * c["k"], c["H"], c["I"]
    g = torch.Generator(device="cuda").manual_seed(0)
    r = lambda *sh: torch.randn(*sh, device="cuda", generator=g, dtype=torch.bfloat16)
    x, wgu, wd = r(m, h), r(2 * i, h), r(h, i)
    gu, inter, go, ggu = r(m, 2 * i), r(m, i), r(m, h), r(m, 2 * i)
    gemms = [("gateup_fwd", lambda: x @ wgu.t()), ("down_fwd", lambda: inter @ wd.t()),
             ("down_dx", lambda: go @ wd), ("wgrad_down", lambda: go.t() @ inter),
             ("wgrad_gateup", lambda: ggu.t() @ x), ("gateup_dx", lambda: ggu @ wgu)]
    out = {}
    total_ms = 0.0
    for name, fn in gemms:
        for _ in range(warmup):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        total_ms += ms
        out[name] = round(ms, 4)
    f = 18 * m * h * i
    return {"tflops": round(f / (total_ms * 1e-3) / 1e12, 1), "ms_sum": round(total_ms, 4),
            "frac_of_peak": round(f / (total_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "gemm_ms": out,
            "what": (f"dense torch.matmul (hipBLASLt) bf16 on config {config}'s six GEMM shapes "
                     f"(M={m}, H={h}, I={i}); context for the grouped kernels, not a path of "
                     f"this library")}


def run_vendor_dense_fp8(steps, warmup):
    """Context, not a product path: config 4's two forward GEMMs as DENSE fp8-e4m3
    torch._scaled_mm calls (hipBLASLt) with per-row x per-column fp32 scales and bf16 output, on
    the same shapes (M = N*k rows: 2*M*H*2I and 2*M*I*H FLOP), no grouping, gather or SwiGLU."""
    import torch
    from kernels.workloads import CONFIGS
    c = CONFIGS[4]
    m, h, i = c["N"] * c["k"], c["H"], c["I"]
    g = torch.Generator(device="cuda").manual_seed(0)
    f8 = torch.float8_e4m3fn
    r = lambda *sh: torch.randn(*sh, device="cuda", generator=g).to(f8)
    x, wgu, inter, wd = r(m, h), r(2 * i, h), r(m, i), r(h, i)
    sx, si = torch.rand(m, 1, device="cuda") + 0.5, torch.rand(m, 1, device="cuda") + 0.5
    sgu, sd = torch.rand(1, 2 * i, device="cuda") + 0.5, torch.rand(1, h, device="cuda") + 0.5
    gemms = [("gateup", lambda: torch._scaled_mm(x, wgu.t(), sx, sgu, out_dtype=torch.bfloat16)),
             ("down", lambda: torch._scaled_mm(inter, wd.t(), si, sd, out_dtype=torch.bfloat16))]
    out, total_ms = {}, 0.0
    for name, fn in gemms:
        for _ in range(warmup):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        total_ms += ms
        out[name] = round(ms, 4)
    f = 6 * m * h * i
    return {"tflops": round(f / (total_ms * 1e-3) / 1e12, 1), "ms_sum": round(total_ms, 4),
            "frac_of_peak": round(f / (total_ms * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4),
            "gemm_ms": out,
            "what": (f"dense torch._scaled_mm (hipBLASLt) fp8-e4m3 with row/column scales on config "
                     f"4's two forward GEMM shapes (M={m}, H={h}, I={i}); context, not a path of "
                     f"this library")}


def cpu_baseline(config, sample_tokens, reps=3):
    """The oracle's fp32 eager MoE fwd+bwd (a restatement of the reference moe_eager, PyTorch on
    the host cores), on the first `sample_tokens` tokens of the same workload."""
    import torch
    from kernels.workloads import make_workload, flops
    from oracle import moe_oracle as orc

    torch.set_num_threads(os.cpu_count() or 1)
    wl = make_workload(config, device="cpu", seed=0, gen_device="cpu",
                       scale=dict(N=sample_tokens))
    cfg = wl["cfg"]
    args = [wl[k].float() for k in ("hidden", "idx", "wt", "gate_up_proj", "down_proj")]
    args[1] = wl["idx"]
    med = _cpu_median(lambda: orc.moe_fwd_bwd(*args, [0] * cfg["E"], wl["grad_out"].float()),
                      reps, f"config {config}")
    f = flops(cfg)
    return {"value": round(f / med / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": (f"config {config} routing/weights with N={sample_tokens} tokens "
                       f"(M={sample_tokens * cfg['k']} rows), fp32 fwd+bwd, median of {reps} after 1 "
                       f"warmup; os.cpu_count()={os.cpu_count()}")}


def _cpu_median(fn, reps, tag):
    times = []
    for r in range(reps + 1):
        t0 = time.perf_counter()
        fn()
        dt = time.perf_counter() - t0
        if r:
            times.append(dt)
        _log(f"cpu {tag} rep {r}: {dt:.2f}s")
    return statistics.median(times)


def cpu_baseline_lowp(config, sample_tokens, reps=3, scale=None):
    """fp8 (config 4) / MXFP8 (config 5) forwards of the oracle on the host cores: each expert's
    quantised weights are dequantised to fp32 inside the expert loop (config 5's dequantised
    weights would not fit in host memory at once), fp32 math. Config 4 in TFLOP/s (6*M*H*I), config
    5 in GB/s of the sample's algorithmic bytes (touched experts' e4m3 + E8M0 bytes, x, out,
    routing), the units of the GPU lines."""
    import torch
    from kernels.workloads import make_workload, flops
    from oracle import moe_oracle as orc

    torch.set_num_threads(os.cpu_count() or 1)
    # drawn and quantised on the GPU (config 5's fp32 weights are 45 GB), then copied to the host
    gen = "cuda" if torch.cuda.is_available() else "cpu"
    w = make_workload(config, device=gen, seed=0, scale=scale)
    w = {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in w.items()}
    if gen == "cuda":
        torch.cuda.empty_cache()
    cfg = dict(w["cfg"], N=sample_tokens)
    n, h, i, k = sample_tokens, cfg["H"], cfg["I"], cfg["k"]
    idx, wt = w["idx"][:n], w["wt"][:n]
    if config == 4:
        fn = lambda: orc.fp8_forward(w["x_q"][:n], w["x_scale"][:n], idx, wt, w["gate_up_q"],
                                     w["gate_up_scale"], w["down_q"], w["down_scale"])
    else:
        fn = lambda: orc.mxfp8_forward(w["hidden"][:n], idx, wt, w["gate_up_q"],
                                       w["gate_up_scale"], w["down_q"], w["down_scale"])
    med = _cpu_median(fn, reps, f"config {config}")
    out = {"cores": torch.get_num_threads(), "kind": "port",
           "sample": (f"config {config} full weights, first {n} of {w['cfg']['N']} tokens "
                      f"(M={n * k} rows), fp32 fwd with per-expert dequantisation, median of {reps} "
                      f"after 1 warmup; os.cpu_count()={os.cpu_count()}")}
    if config == 4:
        out.update(value=round(flops(cfg, backward=False) / med / 1e12, 4), unit="TFLOP/s")
    else:
        touched = int(torch.unique(idx).numel())
        b = touched * 3 * h * i * (1 + 1 / 32) + 2 * n * h * 2 + n * k * (8 + 2)
        out.update(value=round(b / med / 1e9, 2), unit="GB/s", touched_experts=touched)
    return out


def routing_stats(config, router=None):
    """Group sizes of a config's routing: max, median of the non-empty, empty count, and the share
    of routed rows on the 8 largest experts."""
    import torch
    from kernels.workloads import make_workload
    w = make_workload(config, device="cpu", gen_device="cpu",
                      scale=dict(H=8, I=8, **({"router": router} if router else {})))
    e = w["cfg"]["E"]
    c = torch.bincount(w["idx"].reshape(-1), minlength=e)
    return {"max_rows": int(c.max()), "median_nonempty_rows": int(c[c > 0].median()),
            "empty_experts": int((c == 0).sum()),
            "top8_share": round(float(c.sort(descending=True).values[:8].sum() / c.sum()), 3)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=lambda v: int(v) if v.isdigit() else v, default=3,
                    help="1-5, or bench_moe_stack / bench_moe_stack_e32")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=1024)
    ap.add_argument("--profile-pass", action="store_true",
                    help="for rocprofv3 --pmc runs: 1 warmup + 1 step of the workload, then a plain "
                         "1 GiB device copy whose counters calibrate the traffic counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (all experts resident, "
              "no collectives); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs the GPU", file=sys.stderr)
        sys.exit(1)

    if args.profile_pass:
        if args.config == 4:
            run_fp8(1, 1)
        elif args.config == 5:
            run_mxfp8(1, 1)
        else:
            run_bf16(args.config, 1, 1, timer=False)
        src = torch.empty(1 << 29, device="cuda", dtype=torch.bfloat16).fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)             # the calibration kernel: reads 1 GiB, writes 1 GiB
        torch.cuda.synchronize()
        print(json.dumps({"profile_pass": args.config, "calibration_copy_bytes": 1 << 30}))
        return

    _log(f"config {args.config}: warmup {args.warmup}, steps {args.steps}")
    r = run_bf16(args.config, args.steps, args.warmup)
    cfg = r["cfg"]
    kern = r["kernels"]
    gemms = {k: v for k, v in kern.items() if k in KERNEL_MHI}
    dom = max(gemms, key=lambda k: gemms[k]["ms"])
    wl_name = cfg["name"]
    achieved = gemms[dom]["tflops"]
    roofline = {"kernel": dom, "bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "traffic": _traffic(dom, wl_name),
                "flops_per_launch": KERNEL_MHI[dom] * r["mhi"]}
    line = {
        "metric": METRIC, "value": round(r["tflops"], 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(r["ms"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded; random-init weights of the config's shapes)",
        "config": {"workload": (f"{wl_name}: bf16 MoE layer fwd+bwd N={cfg['N']} H={cfg['H']} "
                                f"I={cfg['I']} E={cfg['E']} k={cfg['k']} SwiGLU"),
                   "global_batch": cfg["N"], "seq_len": None, "parallelism": "single GPU"},
        "frac_of_peak": round(r["tflops"] / PEAK_BF16_TFLOPS, 4),
        "roofline": roofline, "kernels": kern,
        "parity": r["parity"], "parity_ok": r["parity"]["parity_ok"],
    }
    if not args.no_extra:
        other = 2 if args.config != 2 else 3
        _log(f"extra config {other}")
        r2 = run_bf16(other, max(5, args.steps // 2), 2, timer=False)
        line["extra_configs"] = {r2["cfg"]["name"]: {"tflops": round(r2["tflops"], 2),
                                                     "ms_per_step": round(r2["ms"], 4),
                                                     "frac_of_peak": round(r2["tflops"] / PEAK_BF16_TFLOPS, 4),
                                                     "parity": r2["parity"]}}
        for stack in ("bench_moe_stack", "bench_moe_stack_e32"):
            _log(f"extra {stack} (the reference bench's PolyGLU stack; unfused GLU path)")
            line["extra_configs"][stack] = run_stack(stack, max(10, args.steps), 3)
        _log("extra config 4 (fp8 fwd)")
        line["extra_configs"]["fp8_fwd"] = run_fp8(max(5, args.steps // 2), 2)
        _log("extra config 5 (MXFP8 decode)")
        line["extra_configs"]["mxfp8_decode"] = run_mxfp8(max(10, args.steps), 3)
        for router, label in (("zipf_power_sigmoid", "many_experts_zipf_power"),
                              ("uniform_topk_sigmoid", "many_experts_uniform")):
            _log(f"extra config 3 routing {router}")
            r3 = run_bf16(3, max(5, args.steps // 2), 2, timer=False, router=router)
            line["extra_configs"][label] = {
                "tflops": round(r3["tflops"], 2), "ms_per_step": round(r3["ms"], 4),
                "frac_of_peak": round(r3["tflops"] / PEAK_BF16_TFLOPS, 4),
                "routing": dict(router=router, **routing_stats(3, router))}
        line["extra_configs"]["many_experts_zipf_routing"] = routing_stats(3)
        _log("extra: vendor dense GEMM reference")
        line["extra_configs"]["vendor_dense_gemm"] = run_vendor_dense(args.config, 10, 3)
        try:
            line["extra_configs"]["vendor_dense_gemm_fp8"] = run_vendor_dense_fp8(10, 3)
        except (RuntimeError, TypeError) as exc:  # a torch build without row-wise fp8 scaling
            line["extra_configs"]["vendor_dense_gemm_fp8"] = {"error": str(exc)[:200]}
        _log("extra: router epilogue")
        line["extra_configs"]["router_epilogue"] = run_router(max(10, args.steps), 3)
    if not args.no_cpu:
        _log("cpu baseline")
        line["cpu_baseline"] = cpu_baseline(args.config, args.cpu_tokens)
        if not args.no_extra:
            other = 2 if args.config != 2 else 3
            line["cpu_baseline"]["other_configs"] = {
                f"config{other}": cpu_baseline(other, 512 if other == 2 else args.cpu_tokens),
                "config4": cpu_baseline_lowp(4, 1024),
                "config5": cpu_baseline_lowp(5, 16),
            }
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
