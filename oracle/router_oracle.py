"""CPU oracle of the router epilogue — TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py's CPU leg may import this module, and only as the checker.

It restates in PyTorch-on-CPU (fp32 or fp64):
  router_topk        the fused router epilogue of kernels/sm75/router.py:40-103 (forward):
                     scores = sigmoid(logits) (or softmax over experts), selection on scores + bias,
                     top-k (ties to the lower expert index: a stable descending sort), unbiased
                     scores gathered at the picks, optional sum-to-1 norm (+1e-20), routed scaling,
                     per-expert pick counts. Its backward is autograd through these operations.
  router_topk_loops  the selection and weights by plain Python loops (small cases; pins
                     router_topk's sort / gather / norm).
  bias_update        router_bias_update, kernels/sm75/router.py:293-301.
Parity pins are in tests/test_oracle.py.
"""
import torch


def router_topk(logits, bias, top_k, norm=True, scale=1.0, softmax=False, dtype=torch.float32):
    """logits (N,E) -> (idx (N,k) int64, w (N,k), counts (E,) int64). Differentiable in logits."""
    x = logits.to(dtype)
    s = torch.softmax(x, dim=-1) if softmax else torch.sigmoid(x)
    sel = s.detach() + (bias.to(dtype) if bias is not None else 0.0)
    idx = torch.sort(sel, dim=-1, descending=True, stable=True).indices[:, :top_k]
    w = s.gather(1, idx)
    if norm and top_k > 1:
        w = w / (w.sum(-1, keepdim=True) + 1e-20)
    w = w * scale
    counts = torch.bincount(idx.reshape(-1), minlength=logits.shape[1])
    return idx, w, counts


def router_topk_loops(logits, bias, top_k, norm=True, scale=1.0, softmax=False):
    """Python-loop restatement for small inputs (float64 math)."""
    import math
    rows = logits.double().tolist()
    b = bias.double().tolist() if bias is not None else None
    idx_out, w_out = [], []
    for r in rows:
        if softmax:
            m = max(r)
            ex = [math.exp(v - m) for v in r]
            z = sum(ex)
            s = [v / z for v in ex]
        else:
            s = [1.0 / (1.0 + math.exp(-v)) for v in r]
        sel = [s[e] + (b[e] if b is not None else 0.0) for e in range(len(r))]
        picked = []
        for _ in range(top_k):
            best = None
            for e in range(len(r)):
                if e in picked:
                    continue
                if best is None or sel[e] > sel[best]:
                    best = e
            picked.append(best)
        w = [s[e] for e in picked]
        if norm and top_k > 1:
            t = sum(w) + 1e-20
            w = [v / t for v in w]
        idx_out.append(picked)
        w_out.append([v * scale for v in w])
    return torch.tensor(idx_out, dtype=torch.int64), torch.tensor(w_out, dtype=torch.float64)


def bias_update(bias, counts, u):
    """bias + u * sign(mean(counts) - counts), fp32 (a new tensor)."""
    if u <= 0:
        return bias.clone()
    tpe = counts.float()
    return bias + u * (tpe.mean() - tpe).sign()
