"""CPU oracle of the MoE expert pipeline — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and
only as the checker (or the timed CPU baseline), never as the product path.

It restates, in numpy / PyTorch-on-CPU:
  dispatch_np          the dispatch contract: counts = bincount, rows sorted by (expert, flat
                       index t*k+j), stable. Reference: _sort_by_expert, kernels/sm75/moe.py:564-572
                       (which uses an unstable sort; only the grouping is observable there).
  dispatch_loops       the same by brute-force Python loops (small cases; pins dispatch_np).
  act                  _act_eager, kernels/sm75/moe.py:859-881 (codes 0,1,2,5,6,7).
  moe_forward          moe_eager, kernels/sm75/moe.py:884-909, in fp32 (or fp64): per expert a
                       mask, gather, F.linear, activation, weighting, fp32 accumulation.
  moe_fwd_bwd          moe_forward + autograd: the fp32 "truth" of .autoresearch/grouped_parity.py:28-49.
  moe_dense            an independent formulation: every expert on every token, combined with a
                       dense (N,E) gate matrix (pins moe_forward: indexing, weighting, specials).
  manual_backward      the grouped backward formulas of kernels/sm75/moe.py:602-618 written out
                       per expert (pins moe_fwd_bwd's autograd and our reading of those formulas).
  fp8_forward          the fp8 pipeline (per-token x, per-channel W, SwiGLU, per-token
                       re-quantised intermediate) computed in fp32 from the quantised values.
  mxfp8_forward        MXFP8 weights dequantised per expert, bf16 activations, fp32 math.
Parity pins for each function are in tests/test_oracle.py.
"""
import numpy as np
import torch
import torch.nn.functional as F

NS_EPS = 1e-6
GLU_CODES = (0, 1, 2, 5, 6, 7)


# ───────────────────────── dispatch ─────────────────────────
def dispatch_np(idx, n_experts):
    """idx (N,k) int -> dict(counts, offsets, sorted_token, sorted_flat, flat_to_sorted).
    Out-of-range ids are dropped (flat_to_sorted = -1)."""
    idx = np.asarray(idx, dtype=np.int64)
    n, k = idx.shape
    flat = idx.reshape(-1)
    valid = (flat >= 0) & (flat < n_experts)
    key = np.where(valid, flat, n_experts)
    order = np.argsort(key, kind="stable")
    order = order[valid[order]]
    counts = np.bincount(flat[valid], minlength=n_experts).astype(np.int64)
    offsets = np.zeros(n_experts + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    f2s = np.full(n * k, -1, dtype=np.int64)
    f2s[order] = np.arange(order.size)
    return dict(counts=counts, offsets=offsets, sorted_token=order // k, sorted_flat=order,
                flat_to_sorted=f2s)


def dispatch_loops(idx, n_experts):
    """Brute force: walk experts in order, and flat indices in order within each expert."""
    idx = [list(map(int, r)) for r in np.asarray(idx)]
    n = len(idx)
    k = len(idx[0]) if n else 0
    sorted_flat = []
    counts = []
    for e in range(n_experts):
        c = 0
        for t in range(n):
            for j in range(k):
                if idx[t][j] == e:
                    sorted_flat.append(t * k + j)
                    c += 1
        counts.append(c)
    f2s = [-1] * (n * k)
    for p, f in enumerate(sorted_flat):
        f2s[f] = p
    offsets = [0]
    for c in counts:
        offsets.append(offsets[-1] + c)
    return dict(counts=np.array(counts), offsets=np.array(offsets),
                sorted_token=np.array([f // k for f in sorted_flat], dtype=np.int64),
                sorted_flat=np.array(sorted_flat, dtype=np.int64), flat_to_sorted=np.array(f2s))


def tile_offsets(counts, tile_rows):
    t = np.zeros(len(counts) + 1, dtype=np.int64)
    t[1:] = np.cumsum((np.asarray(counts) + tile_rows - 1) // tile_rows)
    return t


# ───────────────────────── activations ─────────────────────────
def act(gate, code, alpha=1.0, gamma=1.0):
    """GLU activation of the gate half (fp32 math)."""
    g = gate
    if code == 0:
        return F.silu(g)
    if code == 1:
        return F.relu(g) ** 2
    if code == 5:
        return gamma * torch.tanh(alpha * g) * torch.sigmoid(g)
    gn = g * torch.rsqrt(g.square().mean(-1, keepdim=True) + NS_EPS)
    if code == 6:
        return F.relu(gn) ** 2
    if code == 7:
        return torch.tanh(gn) * torch.sigmoid(gn)
    if code == 2:
        return F.silu(gn)
    raise ValueError(f"not a GLU code: {code}")


# ───────────────────────── MoE forward / backward ─────────────────────────
def moe_forward(hidden, idx, wt, gate_up_proj, down_proj, codes, act_params=None):
    """fp32 (input dtype) eager MoE on the CPU. codes: list/tuple of ints."""
    n, h = hidden.shape
    inter = gate_up_proj.shape[1] // 2
    # fp32 (or wider) accumulation, cast to the input dtype at the end (moe.py:893,909)
    acc = torch.promote_types(hidden.dtype, torch.float32)
    out = torch.zeros(n, h, dtype=acc, device=hidden.device)
    for e, code in enumerate(codes):
        hit = idx == e
        rows = hit.any(-1)
        if not bool(rows.any()) or code == 4:
            continue
        w = (wt * hit).sum(-1)[rows].unsqueeze(-1)
        x = hidden[rows]
        if code == 3:
            out[rows] += (x * w).to(acc)
            continue
        gu = F.linear(x, gate_up_proj[e])
        a, g = (act_params[e, 0], act_params[e, 1]) if (code == 5 and act_params is not None) else (1.0, 1.0)
        y = act(gu[:, :inter], code, a, g) * gu[:, inter:]
        out[rows] += (F.linear(y, down_proj[e]) * w).to(acc)
    return out.to(hidden.dtype)


def moe_fwd_bwd(hidden, idx, wt, gate_up_proj, down_proj, codes, grad_out, act_params=None,
                dtype=torch.float32, device="cpu"):
    """Forward + autograd backward in `dtype`. Runs on the CPU by default; `device` lets a GPU test
    evaluate the same fp32 torch math at sizes the CPU cannot finish quickly. Returns dict of out
    and grads."""
    leaves = [t.detach().to(device, dtype).requires_grad_(True)
              for t in (hidden, wt, gate_up_proj, down_proj)]
    ap = act_params.detach().to(device, dtype).requires_grad_(True) if act_params is not None else None
    h, w, gu, dw = leaves
    out = moe_forward(h, idx.to(device), w, gu, dw, codes, ap)
    out.backward(grad_out.detach().to(device, dtype))
    return dict(out=out.detach(), grad_hidden=h.grad, grad_wt=w.grad, grad_gate_up=gu.grad,
                grad_down=dw.grad, grad_act_params=(ap.grad if ap is not None else None))


def moe_dense(hidden, idx, wt, gate_up_proj, down_proj, codes, act_params=None):
    """Independent formulation: run every expert on every token, then out = sum_e G[:, e] * y_e
    with G the dense (N,E) gate matrix (sum of the top-k weights that picked e)."""
    n, h = hidden.shape
    e_all = len(codes)
    inter = gate_up_proj.shape[1] // 2
    gmat = torch.zeros(n, e_all, dtype=hidden.dtype)
    valid = (idx >= 0) & (idx < e_all)
    gmat.scatter_add_(1, idx.clamp(0, e_all - 1), wt * valid)
    ys = []
    for e, code in enumerate(codes):
        if code == 3:
            ys.append(hidden)
        elif code == 4:
            ys.append(torch.zeros_like(hidden))
        else:
            gu = hidden @ gate_up_proj[e].T
            a, g = (act_params[e, 0], act_params[e, 1]) if (code == 5 and act_params is not None) else (1.0, 1.0)
            ys.append((act(gu[:, :inter], code, a, g) * gu[:, inter:]) @ down_proj[e].T)
    return torch.einsum("ne,enh->nh", gmat, torch.stack(ys))


def manual_backward(hidden, idx, wt, gate_up_proj, down_proj, grad_out):
    """The grouped backward of kernels/sm75/moe.py:602-618 for an all-SiLU stack, written out per
    expert with the closed-form SiLU derivative sigma(g)(1+g(1-sigma(g))) (moe.py:206)."""
    n, h = hidden.shape
    k = idx.shape[1]
    inter = gate_up_proj.shape[1] // 2
    d = dispatch_np(idx.numpy(), gate_up_proj.shape[0])
    st = torch.from_numpy(d["sorted_token"])
    sf = torch.from_numpy(d["sorted_flat"])
    sw = wt.reshape(-1)[sf]
    g_x = torch.zeros_like(hidden)
    g_wt = torch.zeros(n * k, dtype=hidden.dtype)
    g_gu = torch.zeros_like(gate_up_proj)
    g_dw = torch.zeros_like(down_proj)
    off = d["offsets"]
    for e in range(gate_up_proj.shape[0]):
        s, t = int(off[e]), int(off[e + 1])
        if s == t:
            continue
        rows, w = st[s:t], sw[s:t].unsqueeze(-1)
        x = hidden[rows]
        gu = x @ gate_up_proj[e].T
        gate, up = gu[:, :inter], gu[:, inter:]
        sg = torch.sigmoid(gate)
        y = gate * sg * up
        eo = y @ down_proj[e].T
        go = grad_out[rows]
        g_wt[sf[s:t]] = (go * eo).sum(-1)
        g_eo = go * w
        g_y = g_eo @ down_proj[e]
        g_dw[e] = g_eo.T @ y
        g_gate = g_y * up * sg * (1 + gate * (1 - sg))
        g_up = g_y * gate * sg
        ggu = torch.cat([g_gate, g_up], dim=1)
        g_gu[e] = ggu.T @ x
        g_x.index_add_(0, rows, ggu @ gate_up_proj[e])
    return dict(grad_hidden=g_x, grad_wt=g_wt.view(n, k), grad_gate_up=g_gu, grad_down=g_dw)


# ───────────────────────── fp8 / MXFP8 forwards ─────────────────────────
FP8_MAX = 448.0


def e4m3_round(x):
    """Round fp32 to the nearest e4m3fn value (saturating at +-448)."""
    return x.clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn).to(x.dtype)


def e8m0_block_requant(y, block):
    """Re-quantise the rows of y to e4m3 with one power-of-two scale per `block` consecutive
    values: 2^e with e the smallest integer for which 448 * 2^e >= the block's absmax (so no value
    saturates; e = -127 for an all-zero block, and e >= -127 always, the E8M0 range). Returns the
    dequantised values and the E8M0 codes e + 127 of shape (rows, cols / block)."""
    n, k = y.shape
    yb = y.reshape(n, k // block, block)
    amax = yb.abs().amax(-1)
    m, ex = torch.frexp(amax)                      # amax = m * 2^ex, m in [0.5, 1); 448 = 0.875 * 2^9
    e = ex - 9 + (m > 0.875).to(ex.dtype)
    e = torch.where(amax > 0, e, torch.full_like(e, -127)).clamp(min=-127)
    sc = torch.exp2(e.to(y.dtype)).unsqueeze(-1)
    return (e4m3_round(yb / sc) * sc).reshape(n, k), e + 127


def fp8_forward(x_q, x_scale, idx, wt, gate_up_q, gate_up_scale, down_q, down_scale,
                requant_inter=True, inter_bf16=False, requant_block=128, dtype=torch.float32):
    """fp8 MoE forward in fp32 from quantised operands.
    gate_up = (x_q . W_q^T) * x_scale[t] * w_scale[n]; inter = SiLU(gate)*up (rounded to bf16 first
    when inter_bf16), re-quantised to e4m3 when requant_inter: with requant_block > 0 one
    power-of-two scale per block of that many channels of a routed row (e8m0_block_requant, what
    the gfx950 kernels do with 128), with requant_block = 0 one scale per row (absmax/448);
    eo = inter_q . Wd^T * wd_scale[h]; out[t] = sum_j w[t,j] * eo, all in `dtype` (fp32 by default).
    Returns (N,H) in `dtype`."""
    n, h = x_q.shape
    inter = gate_up_q.shape[1] // 2
    xf = x_q.to(dtype)
    xs = x_scale.to(dtype)
    out = torch.zeros(n, h, device=x_q.device, dtype=dtype)
    for e in range(gate_up_q.shape[0]):
        hit = idx == e
        rows = hit.any(-1)
        if not bool(rows.any()):
            continue
        w = (wt.to(dtype) * hit).sum(-1)[rows].unsqueeze(-1)
        gu = (xf[rows] @ gate_up_q[e].to(dtype).T) * xs[rows].unsqueeze(-1) * gate_up_scale[e].to(dtype)
        y = F.silu(gu[:, :inter]) * gu[:, inter:]
        if inter_bf16:
            y = y.bfloat16().to(dtype)
        if requant_inter and requant_block > 0:
            y = e8m0_block_requant(y, requant_block)[0]
        elif requant_inter:
            amax = y.abs().amax(-1, keepdim=True)
            s = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
            y = e4m3_round(y / s) * s
        eo = (y @ down_q[e].to(dtype).T) * down_scale[e].to(dtype)
        out[rows] += eo * w
    return out


def mxfp8_forward(hidden, idx, wt, gate_up_q, gate_up_scale, down_q, down_scale,
                  dtype=torch.float32):
    """MXFP8-weight MoE forward: weights dequantised per expert (E8M0 block scales along K),
    activations as given (bf16 values), math in `dtype` (fp32 by default). Returns (N,H)."""
    n, h = hidden.shape
    inter = gate_up_q.shape[1] // 2
    x = hidden.to(dtype)
    out = torch.zeros(n, h, device=hidden.device, dtype=dtype)

    def deq(q, s):
        k = q.shape[-1]
        return (q.to(dtype).reshape(q.shape[0], k // 32, 32) *
                torch.exp2(s.to(dtype) - 127.0).unsqueeze(-1)).reshape(q.shape[0], k)

    for e in range(gate_up_q.shape[0]):
        hit = idx == e
        rows = hit.any(-1)
        if not bool(rows.any()):
            continue
        w = (wt.to(dtype) * hit).sum(-1)[rows].unsqueeze(-1)
        gu = x[rows] @ deq(gate_up_q[e], gate_up_scale[e]).T
        y = F.silu(gu[:, :inter]) * gu[:, inter:]
        out[rows] += (y @ deq(down_q[e], down_scale[e]).T) * w
    return out
