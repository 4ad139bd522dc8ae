"""The bf16 / fp16 parity gate shared by the GPU tests.

Truth is the CPU oracle's fp64/fp32 math on the same (bf16-valued) inputs. The north star asks for
|ours - truth| <= 1e-2 + 1e-2*|truth| elementwise. The reference's own eager PyTorch MoE
(kernels/sm75/moe.py:884-909) run in the same 16-bit dtype does not meet that absolute form on
gradients of magnitude O(100) (the weight gradients at BASELINE configs 2 and 3): its bf16
intermediates alone put ~0.2-1.3 of error there. So each tensor must:
  1. fail the absolute form on no more elements than the reference's eager path in the same dtype
     (zero wherever that path has zero),
  2. have an RMS error vs truth no larger than the eager path's (x1.1), and a max error within
     x2.5 of the eager path's (a max over millions of bf16-rounded values is a noisy statistic:
     one or two output ulps either way),
  3. pass the reference bench gate max|d| / max|truth| < 1.5e-2 (bench.py:144-157).
"""
import torch

GRADS = ("out", "grad_hidden", "grad_wt", "grad_gate_up", "grad_down")


def eager_16bit(oracle, hidden, idx, wt, gu, dw, codes, go, dtype, act_params=None):
    """The reference's eager algorithm in the 16-bit dtype, on the GPU (rocBLAS GEMMs)."""
    return oracle.moe_fwd_bwd(hidden, idx, wt, gu, dw, codes, go, act_params=act_params,
                              dtype=dtype, device="cuda")


def assert_16bit_parity(mine, truth, eager, keys=GRADS):
    for k in keys:
        a = mine[k].detach().float().cuda()
        t = truth[k].detach().float().cuda()
        r = eager[k].detach().float().cuda()
        assert a.shape == t.shape, k
        d, de = (a - t).abs(), (r - t).abs()
        tol = 1e-2 + 1e-2 * t.abs()
        fails, fails_e = int((d > tol).sum()), int((de > tol).sum())
        scale = t.abs().max().item() + 1e-12
        msg = (f"{k}: ours max|d| {d.max().item():.3e} rms {d.square().mean().sqrt().item():.3e} "
               f"abs-form fails {fails}; eager max|d| {de.max().item():.3e} rms "
               f"{de.square().mean().sqrt().item():.3e} fails {fails_e}; scale {scale:.3e}")
        assert fails <= fails_e, msg
        assert d.max().item() <= 2.5 * de.max().item() + 1e-6 * scale, msg
        assert d.square().mean().sqrt().item() <= 1.1 * de.square().mean().sqrt().item() + 1e-7 * scale, msg
        assert d.max().item() / scale < 1.5e-2, msg
