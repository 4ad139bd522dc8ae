"""CPU checks of bench.py's host logic: the sampled parity check each bf16 line carries, the
reference-stack workloads, and the one-GPU contract. No GPU work."""
import os
import subprocess
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [ROOT, os.path.join(ROOT, "triton-kernel-fused_amd")]

import bench  # noqa: E402
from kernels.workloads import make_workload, glu_rows, n_glu  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402


def _stack(n=300):
    return make_workload("bench_moe_stack", device="cpu", scale=dict(N=n, H=64, I=64))


def test_parity_sample_passes_the_reference_math_and_catches_an_error():
    wl = _stack()
    ref = orc.moe_fwd_bwd(wl["hidden"], wl["idx"], wl["wt"], wl["gate_up_proj"], wl["down_proj"],
                          wl["act_codes"].tolist(), wl["grad_out"])
    ok = bench._parity_sample(ref["out"].to(torch.bfloat16), ref["grad_hidden"], wl)
    assert ok["parity_ok"] and ok["tokens_checked"] == 256
    assert ok["out"] < 1e-2 and ok["grad_hidden"] < 1e-6
    bad_out = bench._parity_sample(ref["out"] * 1.05, ref["grad_hidden"], wl)
    assert not bad_out["parity_ok"] and abs(bad_out["out"] - 0.05) < 1e-3
    g = ref["grad_hidden"].clone()
    g[5] += 0.1 * g.abs().max()
    bad_grad = bench._parity_sample(ref["out"], g, wl, n_sample=300)
    assert not bad_grad["parity_ok"]


def test_reference_stack_workloads():
    for name, e_glu in (("bench_moe_stack", 9), ("bench_moe_stack_e32", 32)):
        wl = make_workload(name, device="cpu", scale=dict(N=2048, H=16, I=16))
        cfg = wl["cfg"]
        assert n_glu(cfg) == e_glu and wl["gate_up_proj"].shape[0] == e_glu
        assert wl["act_codes"].tolist() == [i % 3 for i in range(e_glu)] + [3, 4]
        idx = wl["idx"]
        assert int(idx.max()) < e_glu + 2 and idx.shape == (2048, 2)
        # specials take a share of the routing and run no GEMM
        m = glu_rows(cfg, idx)
        assert 0 < m < idx.numel() and m == int((idx < e_glu).sum())


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2 and "one GPU" in r.stderr
