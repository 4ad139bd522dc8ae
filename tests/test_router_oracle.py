"""CPU pins of the router-epilogue oracle (oracle/router_oracle.py) and host-side argument checks
of the router entry points (no GPU compute)."""
import pytest
import torch

from kernels import _lib
from oracle import router_oracle as ro

CASES = [  # (N, E, k, bias, norm, scale, softmax)
    (40, 8, 2, False, True, 1.0, False),
    (40, 8, 2, True, True, 2.5, False),
    (30, 16, 4, True, False, 1.0, False),
    (30, 16, 4, False, True, 1.0, True),
    (25, 12, 1, True, True, 1.0, True),     # top-1: no norm (reference: norm only for k > 1)
    (20, 70, 8, True, True, 0.7, False),    # E > 64
]


@pytest.mark.parametrize("n,e,k,has_bias,norm,scale,softmax", CASES)
def test_topk_matches_python_loops(n, e, k, has_bias, norm, scale, softmax):
    g = torch.Generator().manual_seed(n * e + k)
    logits = torch.randn(n, e, generator=g, dtype=torch.float64)
    bias = torch.randn(e, generator=g, dtype=torch.float64) * 0.1 if has_bias else None
    idx, w, counts = ro.router_topk(logits, bias, k, norm, scale, softmax, dtype=torch.float64)
    li, lw = ro.router_topk_loops(logits, bias, k, norm, scale, softmax)
    assert torch.equal(idx, li)
    torch.testing.assert_close(w, lw, rtol=1e-12, atol=1e-14)
    assert torch.equal(counts, torch.bincount(li.reshape(-1), minlength=e))
    assert int(counts.sum()) == n * k


def test_ties_go_to_the_lower_expert():
    logits = torch.zeros(3, 6, dtype=torch.float64)
    logits[1, 4] = 1.0
    idx, _, _ = ro.router_topk(logits, None, 3, dtype=torch.float64)
    assert idx[0].tolist() == [0, 1, 2]
    assert idx[1].tolist() == [4, 0, 1]
    li, _ = ro.router_topk_loops(logits, None, 3)
    assert torch.equal(idx, li)


def test_bias_steers_selection_not_weights():
    logits = torch.tensor([[0.0, 1.0, 2.0, 3.0]], dtype=torch.float64)
    bias = torch.tensor([10.0, 0.0, 0.0, 0.0], dtype=torch.float64)
    idx, w, _ = ro.router_topk(logits, bias, 2, norm=False, dtype=torch.float64)
    assert idx[0].tolist() == [0, 3]
    torch.testing.assert_close(w[0], torch.sigmoid(logits[0, [0, 3]]))


@pytest.mark.parametrize("softmax", [False, True])
@pytest.mark.parametrize("norm", [False, True])
def test_backward_gradcheck(softmax, norm):
    g = torch.Generator().manual_seed(7)
    logits = torch.randn(6, 10, generator=g, dtype=torch.float64, requires_grad=True)
    bias = torch.randn(10, generator=g, dtype=torch.float64) * 0.05
    f = lambda x: ro.router_topk(x, bias, 3, norm, 1.7, softmax, dtype=torch.float64)[1]
    assert torch.autograd.gradcheck(f, (logits,))


def test_backward_matches_reference_jacobian():
    # kernels/sm75/router.py:105-113: grad_w_j = c/T (G_j - <G, w>/T), T = sum w + 1e-20, then
    # scattered to the picks and multiplied by sigmoid'.
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(9, 12, generator=g, dtype=torch.float64, requires_grad=True)
    idx, w, _ = ro.router_topk(logits, None, 4, True, 2.0, False, dtype=torch.float64)
    gw = torch.randn(9, 4, generator=g, dtype=torch.float64)
    w.backward(gw)
    s = torch.sigmoid(logits.detach())
    raw = s.gather(1, idx)
    t = raw.sum(-1, keepdim=True) + 1e-20
    graw = 2.0 / t * (gw - (gw * raw).sum(-1, keepdim=True) / t)
    dense = torch.zeros_like(s).scatter_add_(1, idx, graw)
    torch.testing.assert_close(logits.grad, dense * s * (1 - s), rtol=1e-10, atol=1e-12)


def test_bias_update_closed_form():
    bias = torch.tensor([0.5, -0.25, 0.0, 1.0])
    counts = torch.tensor([1, 2, 3, 6], dtype=torch.int32)     # mean 3
    out = ro.bias_update(bias, counts, 0.125)
    assert out.tolist() == [0.625, -0.125, 0.0, 0.875]
    assert torch.equal(ro.bias_update(bias, counts, 0.0), bias)


def test_router_entry_points_reject_bad_arguments():
    h = _lib.lib()
    # dtype, logits, ld, N, E, bias, k, softmax, norm, scale, idx, w, counts, stream
    assert h.moe_router_topk_fwd(7, None, 8, 4, 8, None, 2, 0, 1, 1.0, None, None, None, None) == 4
    assert h.moe_router_topk_fwd(0, None, 8, 4, 2000, None, 2, 0, 1, 1.0, None, None, None, None) == 1
    assert h.moe_router_topk_fwd(0, None, 8, 4, 8, None, 9, 0, 1, 1.0, None, None, None, None) == 1
    assert h.moe_router_topk_fwd(0, None, 4, 4, 8, None, 2, 0, 1, 1.0, None, None, None, None) == 1
    assert h.moe_router_topk_fwd(0, None, 8, 4, 8, None, 2, 0, 1, 1.0, None, None, None, None) == 1
    assert h.moe_router_topk_fwd(0, None, 8, 0, 8, None, 2, 0, 1, 1.0, None, None, None, None) == 0
    assert h.moe_router_topk_bwd(0, None, 8, 4, 8, None, None, 2, 0, 1, 1.0, None, 4, None) == 1
    assert h.moe_router_bias_update(None, None, 0, 1.0, None) == 1
    assert h.moe_router_bias_update(None, None, 8, 0.0, None) == 0
