"""GPU parity of the router epilogue (HIP kernels) against the CPU oracle.

Selection (idx) must match exactly, except where two experts' selection values are within 2e-6
of each other (fp32 rounding of sigmoid/softmax may order such a pair either way; the check
then asserts the swap is one of those near-ties). Weights: |Δ| <= 2e-6·max(1, |ref|) (fp32
kernel vs fp64 oracle). Counts: exact (bincount of the kernel's own picks and equal to the
oracle's where idx matches). grad_logits: |Δ| <= 1e-5·max|ref| + 1e-7 vs autograd of the fp64
oracle; bf16 logits: 1e-2 relative. Bias update: bitwise.
"""
import pytest
import torch

import kernels
from kernels.gfx950.router import router_topk
from oracle import router_oracle as ro

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _check_idx(idx, ref_idx, sel, k, tol=2e-6):
    idx, ref_idx = idx.cpu(), ref_idx.cpu()
    bad = (idx != ref_idx).any(-1).nonzero().flatten()
    for r in bad.tolist():
        a, b = set(idx[r].tolist()), set(ref_idx[r].tolist())
        kth = sel[r].sort(descending=True).values[k - 1].item()
        for e in a ^ b:
            assert abs(sel[r, e].item() - kth) <= tol, f"row {r}: expert {e} is no near-tie"
    return bad


CASES = [  # (N, E, k, bias, norm, scale, softmax, dtype)
    (1000, 8, 2, False, True, 1.0, False, torch.float32),
    (777, 64, 8, True, True, 1.0, False, torch.float32),
    (777, 64, 8, True, True, 2.5, True, torch.float32),
    (300, 256, 8, True, False, 1.0, False, torch.float32),
    (129, 1000, 4, True, True, 1.0, False, torch.float32),
    (513, 128, 1, False, True, 1.0, True, torch.float32),
    (640, 64, 6, True, True, 1.0, False, torch.bfloat16),
    (200, 96, 32, False, True, 1.0, True, torch.float16),
]


@pytest.mark.parametrize("n,e,k,has_bias,norm,scale,softmax,dt", CASES)
def test_router_topk_fwd_bwd(n, e, k, has_bias, norm, scale, softmax, dt):
    _say(f"router N={n} E={e} k={k} bias={has_bias} norm={norm} softmax={softmax} {dt}")
    g = torch.Generator().manual_seed(n + e + k)
    logits = (torch.randn(n, e, generator=g) * 2).to(dt)
    bias = torch.randn(e, generator=g) * 0.05 if has_bias else None
    gw = torch.randn(n, k, generator=g)
    x = logits.cuda().requires_grad_(True)
    idx, w, counts = router_topk(x, bias.cuda() if has_bias else None, k, e, norm, scale,
                                 "softmax" if softmax else "sigmoid")
    w.backward(gw.cuda())
    torch.cuda.synchronize()
    lr = logits.double().requires_grad_(True)
    ridx, rw, rcounts = ro.router_topk(lr, bias.double() if has_bias else None, k, norm, scale,
                                       softmax, dtype=torch.float64)
    s = torch.softmax(lr.detach(), -1) if softmax else torch.sigmoid(lr.detach())
    sel = s + (bias.double() if has_bias else 0.0)
    bad = _check_idx(idx, ridx, sel, k)
    assert torch.equal(counts.cpu().long(), torch.bincount(idx.cpu().reshape(-1), minlength=e))
    ok = torch.ones(n, dtype=torch.bool)
    ok[bad] = False
    if len(bad) == 0:
        assert torch.equal(counts.cpu().long(), rcounts)
    wr = rw.detach()[ok]
    assert ((w.detach().cpu().double()[ok] - wr).abs() <= 2e-6 * wr.abs().clamp_min(1)).all()
    # backward on the rows whose selection matches
    (rw * gw.double()).sum().backward()
    gr = lr.grad[ok]
    tol = (1e-2 if dt != torch.float32 else 1e-5) * gr.abs().max().item() + 1e-7
    assert (x.grad.cpu().double()[ok] - gr).abs().max().item() <= tol
    assert x.grad.dtype == dt


def test_router_empty_and_single_row():
    _say("router empty / one row")
    x = torch.randn(0, 16, device="cuda")
    idx, w, counts = router_topk(x, None, 2, 16)
    assert idx.shape == (0, 2) and int(counts.sum()) == 0
    x = torch.tensor([[0.0, 3.0, -1.0, 2.0]], device="cuda")
    idx, w, _ = router_topk(x, None, 2, None, False)
    assert idx.cpu().tolist() == [[1, 3]]
    torch.testing.assert_close(w.cpu(), torch.sigmoid(torch.tensor([[3.0, 2.0]])))


def test_fused_mlp_router_end_to_end():
    _say("fused_mlp_router (B,S,H) with autograd")
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, 300, 256, generator=g).cuda().requires_grad_(True)
    wg = (torch.randn(64, 256, generator=g) * 0.02).cuda().requires_grad_(True)
    bias = (torch.randn(64, generator=g) * 0.01).cuda()
    idx, w, counts = kernels.fused_mlp_router(x, wg, bias, 8, 64, return_counts=True)
    assert idx.shape == (2, 300, 8) and w.shape == (2, 300, 8) and counts.shape == (64,)
    gw = torch.randn(2, 300, 8, generator=g).cuda()
    w.backward(gw)
    # eager reference on the GPU from the same logits
    x2 = x.detach().clone().requires_grad_(True)
    wg2 = wg.detach().clone().requires_grad_(True)
    logits = x2.reshape(-1, 256) @ wg2.t()
    ridx, rw, rc = ro.router_topk(logits.cpu(), bias.cpu(), 8, True, 1.0, False)
    assert torch.equal(idx.reshape(-1, 8).cpu(), ridx)
    assert torch.equal(counts.cpu().long(), rc)
    s = torch.sigmoid(logits)
    rwg = s.gather(1, ridx.cuda())
    rwg = rwg / (rwg.sum(-1, keepdim=True) + 1e-20)
    (rwg * gw.reshape(-1, 8)).sum().backward()
    torch.testing.assert_close(w.reshape(-1, 8), rwg.detach(), rtol=2e-6, atol=2e-7)
    torch.testing.assert_close(x.grad, x2.grad, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(wg.grad, wg2.grad, rtol=1e-4, atol=1e-6)


def test_fused_conv_router_end_to_end():
    _say("fused_router (causal conv) with autograd")
    g = torch.Generator().manual_seed(12)
    x = torch.randn(2, 128, 64, generator=g).cuda().requires_grad_(True)
    cw = (torch.randn(32, 64, 4, generator=g) * 0.05).cuda().requires_grad_(True)
    idx, w = kernels.fused_router(x, cw, None, 4, 32)
    gw = torch.randn(2, 128, 4, generator=g).cuda()
    w.backward(gw)
    x2 = x.detach().clone().requires_grad_(True)
    cw2 = cw.detach().clone().requires_grad_(True)
    conv = torch.nn.functional.conv1d(torch.nn.functional.pad(x2.transpose(1, 2), (3, 0)), cw2)
    logits = conv.transpose(1, 2).reshape(-1, 32)
    ridx, _, _ = ro.router_topk(logits.detach().cpu(), None, 4)
    assert torch.equal(idx.reshape(-1, 4).cpu(), ridx)
    s = torch.sigmoid(logits)
    rw = s.gather(1, ridx.cuda())
    rw = rw / (rw.sum(-1, keepdim=True) + 1e-20)
    (rw * gw.reshape(-1, 4)).sum().backward()
    torch.testing.assert_close(x.grad, x2.grad, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(cw.grad, cw2.grad, rtol=1e-4, atol=1e-6)


def test_router_bias_update_bitwise():
    _say("router_bias_update")
    g = torch.Generator().manual_seed(5)
    for e in (8, 64, 256, 1000):
        bias = torch.randn(e, generator=g) * 0.01
        counts = torch.randint(0, 5000, (e,), generator=g, dtype=torch.int32)
        counts[: e // 4] = int(counts.float().mean())   # some exact ties with the mean are possible
        ref = ro.bias_update(bias, counts, 1e-3)
        b = bias.cuda()
        kernels.router_bias_update(b, counts.cuda(), 1e-3)
        assert torch.equal(b.cpu(), ref)
        kernels.router_bias_update(b, counts.cuda(), 0.0)
        assert torch.equal(b.cpu(), ref)


def test_router_counts_deterministic():
    _say("router counts run to run")
    x = torch.randn(16384, 64, device="cuda")
    a = router_topk(x, None, 8, 64)[2]
    b = router_topk(x, None, 8, 64)[2]
    assert torch.equal(a, b) and int(a.sum()) == 16384 * 8


@pytest.mark.parametrize("e", [64, 200, 300])
def test_router_exact_ties_pick_lower_expert(e):
    _say(f"router ties E={e}")
    g = torch.Generator().manual_seed(e)
    logits = torch.randint(-3, 4, (500, e), generator=g).float()
    idx, w, counts = router_topk(logits.cuda(), None, 8, e, False)
    ridx, rw, rc = ro.router_topk(logits, None, 8, False)
    assert torch.equal(idx.cpu(), ridx)
    assert torch.equal(counts.cpu().long(), rc)
    torch.testing.assert_close(w.cpu(), rw, rtol=1e-6, atol=1e-7)
