"""GPU parity through every reference entry point of the MoE path.

The reference exposes the same layer under several names (kernels/sm75/moe.py:621-629 moe_grouped,
:829-835 moe_per_expert, :838-855 moe; kernels/sm120/moe.py:32-48 moe; kernels/sm120/
moe_grouped.py:77-122 moe_grouped_cublas_polyglu; moe_grouped_cublas, kernels/sm75/moe.py:638).
Each one is called here through its import path, forward and backward, on a stack with an empty
GLU expert and the Identity (3) / Zero (4) specials on the tail, and compared with the CPU oracle
(fp64 restatement of moe_eager, kernels/sm75/moe.py:884-909, plus autograd).

bf16 tolerance: tests/parity.py (the absolute form |d| <= 1e-2 + 1e-2*|ref| wherever the reference's
own eager bf16 path meets it, never less accurate than that path, and the reference bench gate
max|d| / max|ref| < 1.5e-2, bench.py:144-157).
fp32 tolerance: max|d| / max|ref| < 1e-4 (parity_situ.py:30-32).
"""
import importlib

import pytest
import torch

from oracle import moe_oracle as orc
from parity import GRADS, assert_16bit_parity, eager_16bit

pytestmark = pytest.mark.gpu

ENTRY_POINTS = [
    ("kernels", "moe"),
    ("kernels", "moe_per_expert"),
    ("kernels.sm75", "moe"),
    ("kernels.sm75.moe", "moe_grouped"),
    ("kernels.sm120", "moe"),
    ("kernels.sm120.moe", "moe_grouped_cublas"),
    ("kernels.sm120.moe_grouped", "moe_grouped_cublas_polyglu"),
]


def _fn(mod, name):
    return getattr(importlib.import_module(mod), name)


def _case(dtype, seed=0, n=600, h=256, i=192, k=3):
    """Six GLU experts (SiLU and ReLU^2; expert 2 gets no rows) then Identity and Zero."""
    codes = [0, 1, 0, 0, 1, 0, 3, 4]
    g = torch.Generator().manual_seed(seed)
    hid = torch.randn(n, h, generator=g) * 0.5
    gu = torch.randn(6, 2 * i, h, generator=g) * 0.1
    dw = torch.randn(6, h, i, generator=g) * 0.1
    score = torch.rand(n, len(codes), generator=g)
    score[:, 2] = -1.0                                   # nobody picks expert 2
    w, idx = score.topk(k, dim=-1)
    w = w / w.sum(-1, keepdim=True)
    go = torch.randn(n, h, generator=g) * 0.1
    return codes, [t.to(dtype) for t in (hid, w, gu, dw, go)], idx


def _run(fn, codes, tensors, idx):
    hid, w, gu, dw, go = [t.cuda() for t in tensors]
    leaves = [t.clone().requires_grad_(True) for t in (hid, w, gu, dw)]
    out = fn(leaves[0], idx.cuda(), leaves[1], leaves[2], leaves[3],
             torch.tensor(codes, dtype=torch.int32, device="cuda"))
    out.backward(go)
    torch.cuda.synchronize()
    h, ww, g, d = leaves
    return dict(out=out.detach(), grad_hidden=h.grad, grad_wt=ww.grad, grad_gate_up=g.grad,
                grad_down=d.grad)


@pytest.mark.parametrize("mod,name", ENTRY_POINTS, ids=[f"{m}.{n}" for m, n in ENTRY_POINTS])
def test_entry_point_bf16_fwd_bwd(mod, name):
    print(f"[gpu-case] entry point {mod}.{name} bf16", flush=True)
    codes, tensors, idx = _case(torch.bfloat16)
    ref = orc.moe_fwd_bwd(tensors[0], idx, tensors[1], tensors[2], tensors[3], codes, tensors[4],
                          dtype=torch.float64)
    mine = _run(_fn(mod, name), codes, tensors, idx)
    assert mine["out"].dtype == torch.bfloat16
    assert mine["grad_gate_up"][2].abs().max().item() == 0.0       # the empty expert
    eager = eager_16bit(orc, tensors[0], idx, tensors[1], tensors[2], tensors[3], codes,
                        tensors[4], torch.bfloat16)
    assert_16bit_parity(mine, ref, eager)


@pytest.mark.parametrize("mod,name", ENTRY_POINTS, ids=[f"{m}.{n}" for m, n in ENTRY_POINTS])
def test_entry_point_fp32_fwd_bwd(mod, name):
    print(f"[gpu-case] entry point {mod}.{name} fp32", flush=True)
    codes, tensors, idx = _case(torch.float32, seed=1, n=300)
    ref = orc.moe_fwd_bwd(tensors[0], idx, tensors[1], tensors[2], tensors[3], codes, tensors[4],
                          dtype=torch.float64)
    mine = _run(_fn(mod, name), codes, tensors, idx)
    for k in GRADS:
        a, b = mine[k].double().cpu(), ref[k]
        r = ((a - b).abs().max() / (b.abs().max() + 1e-12)).item()
        assert r < 1e-4, f"{k}: {r:.3e}"


@pytest.mark.parametrize("mod,name", [e for e in ENTRY_POINTS if "grouped" in e[1]],
                         ids=[f"{m}.{n}" for m, n in ENTRY_POINTS if "grouped" in n])
def test_grouped_entry_points_reject_situ(mod, name):
    codes, tensors, idx = _case(torch.bfloat16, n=64)
    codes = [5] + codes[1:]
    hid, w, gu, dw, _ = [t.cuda() for t in tensors]
    with pytest.raises(ValueError):
        _fn(mod, name)(hid, idx.cuda(), w, gu, dw, torch.tensor(codes, dtype=torch.int32,
                                                                   device="cuda"))
