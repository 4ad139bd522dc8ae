"""Write tests/golden/config1.npz: the oracle's results on BASELINE config 1 (fp32, N=1024, H=256,
I=512, E=8, k=2, seed 0, inputs drawn on the CPU by kernels.workloads).

    python tests/golden/make_golden.py

The fixture keeps the full dispatch (small ints), fp64-oracle checksums of the output and every
gradient, and every 16th row of the output / grad_hidden, so a later change to the oracle, the
generator or the GPU path shows up as a mismatch without re-deriving anything. Inputs are not
stored: they are regenerated from the seed.
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "triton-kernel-fused_amd"))

from kernels.workloads import make_workload  # noqa: E402
from oracle import moe_oracle as orc  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config1.npz")


def build():
    w = make_workload(1, device="cpu", seed=0)
    d = orc.dispatch_np(w["idx"].numpy(), w["cfg"]["E"])
    r = orc.moe_fwd_bwd(w["hidden"], w["idx"], w["wt"], w["gate_up_proj"], w["down_proj"],
                        [0] * w["cfg"]["E"], w["grad_out"], dtype=torch.float64)
    fx = dict(
        idx=w["idx"].numpy().astype(np.int16),
        counts=d["counts"].astype(np.int32), offsets=d["offsets"].astype(np.int32),
        sorted_flat=d["sorted_flat"].astype(np.int32),
        out_rows=r["out"][::16].float().numpy(), grad_hidden_rows=r["grad_hidden"][::16].float().numpy(),
        grad_wt=r["grad_wt"].float().numpy(),
    )
    for name in ("out", "grad_hidden", "grad_wt", "grad_gate_up", "grad_down"):
        t = r[name].double()
        fx[f"norm_{name}"] = np.array([t.norm().item(), t.sum().item(), t.abs().max().item()])
    return fx


if __name__ == "__main__":
    fx = build()
    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")
