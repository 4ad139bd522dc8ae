"""GPU parity of the full MoE pipeline (forward + backward) through the HIP library.

Reference of truth: the CPU oracle (fp32 / fp64 torch restatement of moe_eager + autograd) for
small cases; at full BASELINE sizes the same fp32 torch math evaluated on the GPU.

Tolerances:
  fp32 inputs: max|ours - ref| <= 1e-4 * max|ref|                    (parity_situ.py:30-32)
  bf16/fp16 inputs: tests/parity.py — the absolute form |d| <= 1e-2 + 1e-2*|ref| wherever the
               reference's own eager path in that dtype meets it, never less accurate than that
               path (max and RMS error), and the reference bench gate max|d|/max|ref| < 1.5e-2.
"""
import numpy as np
import pytest
import torch

import kernels
from kernels.workloads import make_workload
from oracle import moe_oracle as orc
from parity import assert_16bit_parity, eager_16bit

pytestmark = pytest.mark.gpu
GRADS = ("out", "grad_hidden", "grad_wt", "grad_gate_up", "grad_down")


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _run(fn, hidden, idx, wt, gu, dw, codes_t, go, ap=None):
    leaves = [t.detach().clone().requires_grad_(True) for t in (hidden, wt, gu, dw)]
    a = ap.detach().clone().requires_grad_(True) if ap is not None else None
    h, w, g, d = leaves
    out = fn(h, idx, w, g, d, codes_t, a) if a is not None else fn(h, idx, w, g, d, codes_t)
    out.backward(go)
    torch.cuda.synchronize()
    return dict(out=out.detach(), grad_hidden=h.grad, grad_wt=w.grad, grad_gate_up=g.grad,
                grad_down=d.grad, grad_act_params=(a.grad if a is not None else None))


def _rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-12)).item()


def _assert_fp32(mine, ref, keys=GRADS, tol=1e-4):
    for k in keys:
        assert mine[k] is not None, k
        r = _rel(mine[k], ref[k])
        assert r < tol, f"{k}: max|d|/max|ref| = {r:.3e} >= {tol}"


def _assert_bf16(mine, ref, inputs, codes, keys=GRADS, dtype=torch.bfloat16):
    """inputs = (hidden, idx, wt, gate_up_proj, down_proj, grad_out) as given to the kernel."""
    eager = eager_16bit(orc, *inputs[:5], codes, inputs[5], dtype)
    assert_16bit_parity(mine, ref, eager, keys)


def _case(codes, e_glu, n=512, h=128, i=96, k=2, dtype=torch.float32, cap=None, seed=0):
    """parity_situ.py-shaped inputs (parity_situ.py:12-27), drawn on the CPU."""
    g = torch.Generator().manual_seed(seed)
    hid = torch.randn(n, h, generator=g) * 0.5
    gu = torch.randn(e_glu, 2 * i, h, generator=g) * 0.1
    dw = torch.randn(e_glu, h, i, generator=g) * 0.1
    lim = cap or len(codes)
    w, idx = torch.rand(n, lim, generator=g).topk(k, dim=-1)
    w = w / w.sum(-1, keepdim=True)
    ap = torch.stack([torch.rand(len(codes), generator=g) + 0.5,
                      torch.rand(len(codes), generator=g) + 0.5], dim=1)
    go = torch.randn(n, h, generator=g) * 0.1
    return (hid.to(dtype), idx, w.to(dtype), gu.to(dtype), dw.to(dtype),
            torch.tensor(codes, dtype=torch.int32), ap, go.to(dtype))


FP32_CASES = [
    ("all-silu", [0] * 6, 6, None, 96, False),
    ("all-relu2", [1] * 6, 6, None, 96, False),
    ("all-normsilu", [2] * 6, 6, None, 96, False),
    ("mixed-all-codes", [0, 1, 2, 5, 6, 7], 6, None, 96, True),
    ("situ+specials", [0, 5, 2, 5, 3, 4], 4, None, 96, True),
    ("silu+specials", [0, 0, 1, 0, 3, 4], 4, None, 96, False),
    ("empty-experts", [5, 5, 5, 5, 0, 2], 6, 4, 96, True),
    ("wide-I", [0, 1, 2, 5, 0, 5], 6, None, 1536, True),
]


@pytest.mark.parametrize("name,codes,e_glu,cap,inter,with_ap", FP32_CASES, ids=[c[0] for c in FP32_CASES])
def test_fp32_parity_vs_oracle(name, codes, e_glu, cap, inter, with_ap):
    hid, idx, w, gu, dw, codes_t, ap, go = _case(codes, e_glu, i=inter, cap=cap)
    _say(f"fp32 {name}")
    ref = orc.moe_fwd_bwd(hid, idx, w, gu, dw, codes, go, act_params=ap if with_ap else None,
                          dtype=torch.float64)
    dev = [t.cuda() for t in (hid, idx, w, gu, dw, codes_t, go)]
    mine = _run(kernels.moe_per_expert, *dev, ap=ap.cuda() if with_ap else None)
    _assert_fp32(mine, ref)
    if with_ap and 5 in codes:
        _assert_fp32(mine, ref, keys=("grad_act_params",))


BF16_CASES = [
    ("silu", [0] * 6, 6, None),
    ("mixed", [0, 1, 2, 5, 0, 5], 6, None),
    ("specials", [0, 1, 0, 1, 3, 4], 4, None),
    ("empty", [0, 0, 0, 0, 0, 0], 6, 3),
]


@pytest.mark.parametrize("name,codes,e_glu,cap", BF16_CASES, ids=[c[0] for c in BF16_CASES])
def test_bf16_parity_vs_oracle(name, codes, e_glu, cap):
    hid, idx, w, gu, dw, codes_t, ap, go = _case(codes, e_glu, dtype=torch.bfloat16, cap=cap, n=700,
                                                 h=256, i=192, k=3)
    _say(f"bf16 {name}")
    ref = orc.moe_fwd_bwd(hid, idx, w, gu, dw, codes, go, dtype=torch.float64)
    dev = [t.cuda() for t in (hid, idx, w, gu, dw, codes_t, go)]
    mine = _run(kernels.moe, *dev)
    _assert_bf16(mine, ref, (hid, idx, w, gu, dw, go), codes)


def test_bf16_max_experts():
    """MAX_GLU_EXPERTS = 1024 experts, ~5 rows each (many empty), top-8: the dispatch's largest
    histogram, the GEMMs' expert walk over 1024 groups and the gated backward."""
    e = 1024
    hid, idx, w, gu, dw, codes_t, ap, go = _case([0] * e, e, dtype=torch.bfloat16, n=600, h=128,
                                                 i=128, k=8, seed=3)
    _say("bf16 1024 experts")
    ref = orc.moe_fwd_bwd(hid, idx, w, gu, dw, [0] * e, go, dtype=torch.float64)
    dev = [t.cuda() for t in (hid, idx, w, gu, dw, codes_t, go)]
    mine = _run(kernels.moe, *dev)
    _assert_bf16(mine, ref, (hid, idx, w, gu, dw, go), [0] * e)


def test_fp16_parity_vs_oracle():
    hid, idx, w, gu, dw, codes_t, ap, go = _case([0, 1, 0, 0], 4, dtype=torch.float16, n=300)
    _say("fp16 silu/relu2")
    ref = orc.moe_fwd_bwd(hid, idx, w, gu, dw, [0, 1, 0, 0], go, dtype=torch.float64)
    mine = _run(kernels.moe, *[t.cuda() for t in (hid, idx, w, gu, dw, codes_t, go)])
    _assert_bf16(mine, ref, (hid, idx, w, gu, dw, go), [0, 1, 0, 0], dtype=torch.float16)


def test_config1_fp32_vs_golden_and_oracle():
    _say("config 1 fp32 full size")
    wl = make_workload(1, device="cpu", seed=0)
    fx = np.load(__file__.replace("test_gpu_moe.py", "golden/config1.npz"))
    ref = orc.moe_fwd_bwd(wl["hidden"], wl["idx"], wl["wt"], wl["gate_up_proj"], wl["down_proj"],
                          [0] * 8, wl["grad_out"])
    dev = {k: (v.cuda() if torch.is_tensor(v) else v) for k, v in wl.items()}
    mine = _run(kernels.moe, dev["hidden"], dev["idx"], dev["wt"], dev["gate_up_proj"],
                dev["down_proj"], dev["act_codes"], dev["grad_out"])
    _assert_fp32(mine, ref)
    np.testing.assert_allclose(mine["out"][::16].cpu().numpy(), fx["out_rows"], rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(mine["grad_wt"].cpu().numpy(), fx["grad_wt"], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("config", [2, 3])
def test_full_size_bf16_vs_fp32_reference(config):
    _say(f"config {config} bf16 full size fwd+bwd")
    wl = make_workload(config, device="cuda", seed=0)
    e = wl["cfg"]["E"]
    mine = _run(kernels.moe, wl["hidden"], wl["idx"], wl["wt"], wl["gate_up_proj"], wl["down_proj"],
                wl["act_codes"], wl["grad_out"])
    ref = orc.moe_fwd_bwd(wl["hidden"], wl["idx"], wl["wt"], wl["gate_up_proj"], wl["down_proj"],
                          [0] * e, wl["grad_out"], device="cuda")
    _assert_bf16(mine, ref, (wl["hidden"], wl["idx"], wl["wt"], wl["gate_up_proj"],
                             wl["down_proj"], wl["grad_out"]), [0] * e)


def test_deterministic_bitwise():
    hid, idx, w, gu, dw, codes_t, ap, go = _case([0] * 6, 6, dtype=torch.bfloat16, n=2000)
    dev = [t.cuda() for t in (hid, idx, w, gu, dw, codes_t, go)]
    _say("determinism")
    a = _run(kernels.moe, *dev)
    b = _run(kernels.moe, *dev)
    for k in GRADS:
        assert torch.equal(a[k], b[k]), k


def test_expanded_grad_and_autocast():
    hid, idx, w, gu, dw, codes_t, ap, go = _case([0, 1, 2, 0], 4, n=256)
    _say("expanded grad_out + autocast")
    dev = [t.cuda() for t in (hid, idx, w, gu, dw, codes_t)]
    h = dev[0].clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = kernels.moe(h, dev[1], dev[2], dev[3], dev[4], dev[5])
    assert out.dtype == torch.bfloat16
    g = torch.ones(1, hid.shape[1], device="cuda", dtype=torch.bfloat16).expand_as(out)
    out.backward(g)
    ref = orc.moe_fwd_bwd(hid.bfloat16(), idx, w.bfloat16(), gu.bfloat16(), dw.bfloat16(),
                          [0, 1, 2, 0], torch.ones_like(hid), dtype=torch.float64)
    assert h.grad.dtype == torch.float32
    _assert_bf16(dict(out=out, grad_hidden=h.grad), ref,
                 (hid.bfloat16(), idx, w.bfloat16(), gu.bfloat16(), dw.bfloat16(),
                  torch.ones_like(hid).bfloat16()), [0, 1, 2, 0], keys=("out", "grad_hidden"))


@pytest.mark.parametrize("dtype,i", [(torch.float32, 200), (torch.bfloat16, 196),
                                     (torch.bfloat16, 768), (torch.bfloat16, 3000)],
                         ids=["fp32-vec", "bf16-scalar", "bf16-vec", "bf16-vec-fwd-scalar-bwd"])
def test_batched_glu_all_codes(dtype, i):
    """Every code with per-row SiTU parameters. fp32 I=200 and bf16 I=768 take the one-wave-per-row
    vector kernels; I=196 (not a multiple of 8) the scalar ones; I=3000 the vector forward and
    the scalar backward (too long to keep three rows in registers)."""
    g = torch.Generator().manual_seed(3)
    m = 333
    gu = torch.randn(m, 2 * i, generator=g, dtype=torch.float64)
    row_act = torch.tensor([0, 1, 2, 5, 6, 7], dtype=torch.int32).repeat(m // 6 + 1)[:m]
    ra = torch.rand(m, generator=g, dtype=torch.float64) + 0.5
    rg = torch.rand(m, generator=g, dtype=torch.float64) + 0.5
    go = torch.randn(m, i, generator=g, dtype=torch.float64)
    _say(f"BatchedGLU all codes {dtype} I={i}")
    x = gu.to(dtype).cuda().requires_grad_(True)
    a_, g_ = ra.float().cuda().requires_grad_(True), rg.float().cuda().requires_grad_(True)
    y = kernels.BatchedGLU.apply(x, row_act.cuda(), a_, g_)
    y.backward(go.to(dtype).cuda())
    # oracle: per-row activation with autograd in fp64, on the same (dtype-rounded) inputs
    gu, go = gu.to(dtype).double(), go.to(dtype).double()
    xr = gu.clone().requires_grad_(True)
    ar, gr = ra.clone().requires_grad_(True), rg.clone().requires_grad_(True)
    rows = []
    for r in range(m):
        c = int(row_act[r])
        rows.append(orc.act(xr[r:r + 1, :i], c, ar[r], gr[r]) * xr[r:r + 1, i:])
    yr = torch.cat(rows)
    yr.backward(go)
    tol, tol_p = (1e-5, 1e-4) if dtype == torch.float32 else (1e-2, 1e-2)
    assert _rel(y, yr) < tol
    assert _rel(x.grad, xr.grad) < tol
    assert _rel(a_.grad, ar.grad) < tol_p and _rel(g_.grad, gr.grad) < tol_p


@pytest.mark.parametrize("needs", ["wt", "down", "gate_up", "hidden"])
def test_bf16_partial_grads_and_strided_grad_out(needs):
    """Each leaf alone requiring grad (the backward skips the other products), with grad_out a
    column slice of a wider tensor so its rows are 384 elements apart."""
    codes = [0, 1, 0, 1, 3, 4]
    hid, idx, w, gu, dw, codes_t, ap, go = _case(codes, 4, dtype=torch.bfloat16, n=333, h=256,
                                                 i=320, k=2, seed=5)
    _say(f"bf16 partial grads: {needs}")
    ref = orc.moe_fwd_bwd(hid, idx, w, gu, dw, codes, go, dtype=torch.float64)
    d = {n: t.cuda() for n, t in zip(("hidden", "wt", "gate_up", "down"), (hid, w, gu, dw))}
    d[needs].requires_grad_(True)
    out = kernels.moe(d["hidden"], idx.cuda(), d["wt"], d["gate_up"], d["down"], codes_t.cuda())
    wide = torch.zeros(hid.shape[0], 384, device="cuda", dtype=torch.bfloat16)
    wide[:, :256] = go.cuda()
    out.backward(wide[:, :256])
    torch.cuda.synchronize()
    key = {"wt": "grad_wt", "down": "grad_down", "gate_up": "grad_gate_up",
           "hidden": "grad_hidden"}[needs]
    _assert_bf16({key: d[needs].grad}, ref, (hid, idx, w, gu, dw, go), codes, keys=(key,))


@pytest.mark.parametrize("h,i", [(64, 64), (128, 64), (64, 192), (192, 320)])
def test_bf16_short_k_loops(h, i):
    """One- to five-step K loops of the ring kernels (every K here is a multiple of 64): the
    prologue and refills past the last step must not disturb the result."""
    codes = [0, 1, 0, 1, 3]
    hid, idx, w, gu, dw, codes_t, ap, go = _case(codes, 4, dtype=torch.bfloat16, n=300, h=h, i=i,
                                                 k=2, seed=h + i)
    _say(f"bf16 short K h={h} i={i}")
    ref = orc.moe_fwd_bwd(hid, idx, w, gu, dw, codes, go, dtype=torch.float64)
    mine = _run(kernels.moe, *[t.cuda() for t in (hid, idx, w, gu, dw, codes_t, go)])
    _assert_bf16(mine, ref, (hid, idx, w, gu, dw, go), codes)


@pytest.mark.parametrize("h,i", [(96, 80), (160, 200)])
def test_bf16_k_not_multiple_of_64(h, i):
    """K not a multiple of the ring kernels' 64-value step (H = 96 / 160, 2I = 160 / 400): the
    forwards and the non-gated down-dX take the first-generation kernels, the gate/up dX the
    five-stage fallback."""
    codes = [0, 1, 0, 1, 3]
    hid, idx, w, gu, dw, codes_t, ap, go = _case(codes, 4, dtype=torch.bfloat16, n=300, h=h, i=i,
                                                 k=2, seed=h * i)
    _say(f"bf16 K % 64 != 0 h={h} i={i}")
    ref = orc.moe_fwd_bwd(hid, idx, w, gu, dw, codes, go, dtype=torch.float64)
    mine = _run(kernels.moe, *[t.cuda() for t in (hid, idx, w, gu, dw, codes_t, go)])
    _assert_bf16(mine, ref, (hid, idx, w, gu, dw, go), codes)


def test_bf16_out_of_range_expert_ids():
    """Out-of-range expert ids (>= E and negative) are dropped, as the oracle's mask drops them:
    their slots add nothing and their gate gradients are zero. Exercises the folded backward with
    routed rows fewer than N*k (the gates gathered into sorted order past the routed count)."""
    codes = [0, 1, 0, 1, 0, 0]
    hid, idx, w, gu, dw, codes_t, ap, go = _case(codes, 6, dtype=torch.bfloat16, n=400, h=128,
                                                 i=96, k=3, seed=7)
    idx[::7, 0] = 6
    idx[::11, 1] = -1
    _say("bf16 out-of-range expert ids")
    ref = orc.moe_fwd_bwd(hid, idx, w, gu, dw, codes, go, dtype=torch.float64)
    mine = _run(kernels.moe, *[t.cuda() for t in (hid, idx, w, gu, dw, codes_t, go)])
    _assert_bf16(mine, ref, (hid, idx, w, gu, dw, go), codes)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_unfused_codes_out_of_range_expert_ids(dtype):
    """Unfused codes (RMS-normalised 2/6/7, SiTU 5 with act_params) plus an Identity slot, with
    ids of -1 and >= E in the routing: the routed rows are fewer than N*k, so the per-row code and
    SiTU-parameter gathers run past the routed count. Dropped ids add nothing, as the reference's
    mask drops them (kernels/sm75/moe.py:895-899)."""
    codes = [2, 5, 6, 7, 0, 3]
    hid, idx, w, gu, dw, codes_t, ap, go = _case(codes, 5, dtype=dtype, n=400, h=128, i=96, k=3,
                                                 seed=11)
    idx[::5, 0] = 6
    idx[::9, 1] = -1
    idx[::13, 2] = 1000
    _say(f"{dtype} unfused codes with out-of-range ids")
    ref = orc.moe_fwd_bwd(hid, idx, w, gu, dw, codes, go, act_params=ap, dtype=torch.float64)
    dev = [t.cuda() for t in (hid, idx, w, gu, dw, codes_t, go)]
    mine = _run(kernels.moe_per_expert, *dev, ap=ap.cuda())
    if dtype == torch.float32:
        _assert_fp32(mine, ref, keys=GRADS + ("grad_act_params",))
    else:
        eager = eager_16bit(orc, hid, idx, w, gu, dw, codes, go, dtype, act_params=ap)
        assert_16bit_parity(mine, ref, eager, GRADS)
        assert _rel(mine["grad_act_params"], ref["grad_act_params"]) < 3e-2
