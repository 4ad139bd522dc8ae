"""GPU parity of moe_dispatch (histogram, scan, stable permutation): bit-exact vs the oracle."""
import numpy as np
import pytest
import torch

from kernels import _lib
from kernels.gfx950.moe import dispatch
from kernels.workloads import make_workload
from oracle import moe_oracle as orc

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def _check(idx_cpu, n_experts):
    _say(f"dispatch N={idx_cpu.shape[0]} k={idx_cpu.shape[1]} E={n_experts}")
    r = dispatch(idx_cpu.cuda(), n_experts)
    torch.cuda.synchronize()
    ref = orc.dispatch_np(idx_cpu.numpy(), n_experts)
    m = idx_cpu.numel()
    np.testing.assert_array_equal(r.counts.cpu().numpy(), ref["counts"])
    np.testing.assert_array_equal(r.offsets.cpu().numpy(), ref["offsets"])
    np.testing.assert_array_equal(r.tile_offsets.cpu().numpy(),
                                  orc.tile_offsets(ref["counts"], _lib.lib().moe_tile_rows()))
    np.testing.assert_array_equal(r.expert_order.cpu().numpy(),
                                  np.argsort(-ref["counts"], kind="stable"))
    n_valid = int(ref["offsets"][-1])
    np.testing.assert_array_equal(r.sorted_flat.cpu().numpy()[:n_valid], ref["sorted_flat"])
    np.testing.assert_array_equal(r.sorted_token.cpu().numpy()[:n_valid], ref["sorted_token"])
    np.testing.assert_array_equal(r.flat_to_sorted.cpu().numpy()[:m], ref["flat_to_sorted"])
    # positions past the routed count (dropped ids) hold -1
    assert (r.sorted_flat.cpu().numpy()[n_valid:m] == -1).all()
    assert (r.sorted_token.cpu().numpy()[n_valid:m] == -1).all()
    assert int(r.status.item()) == int((ref["flat_to_sorted"] < 0).sum())
    return r


@pytest.mark.parametrize("config", [1, 2, 3, 4, 5])
def test_dispatch_baseline_routing(config):
    # the real routing of every config (H/I shrunk: only idx matters here)
    w = make_workload(config, scale=dict(H=32, I=32))
    _check(w["idx"], w["cfg"]["E"])


@pytest.mark.parametrize("n,k,e,seed", [(1, 1, 1, 0), (4096, 1, 3, 1), (4097, 1, 3, 2),
                                        (2048, 2, 2, 3), (1000, 8, 1024, 4), (33333, 4, 257, 5),
                                        (5, 3, 7, 6), (1024, 1, 5, 8), (1025, 1, 5, 9),
                                        (128, 8, 256, 10), (129, 8, 256, 11), (511, 2, 1000, 12)])
def test_dispatch_random(n, k, e, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.rand(n, max(e, k), generator=g).topk(k, dim=-1).indices % e
    _check(idx.long(), e)


def test_dispatch_skewed_and_out_of_range():
    g = torch.Generator().manual_seed(7)
    idx = torch.randint(0, 3, (20000, 4), generator=g)
    idx[::7, 1] = 63           # a hot expert at the end
    idx[5, 0] = -1             # out of range: dropped, counted in status
    idx[9, 3] = 64
    _check(idx, 64)


def test_dispatch_empty():
    r = dispatch(torch.zeros(0, 2, dtype=torch.long, device="cuda"), 8)
    assert r.counts.cpu().tolist() == [0] * 8
    assert r.offsets.cpu().tolist() == [0] * 9


def test_dispatch_deterministic():
    g = torch.Generator().manual_seed(11)
    idx = torch.randint(0, 16, (50000, 2), generator=g).cuda()
    a = dispatch(idx, 16)
    b = dispatch(idx, 16)
    assert torch.equal(a.sorted_flat, b.sorted_flat) and torch.equal(a.flat_to_sorted, b.flat_to_sorted)
