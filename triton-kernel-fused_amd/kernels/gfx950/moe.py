"""PolyGLU MoE expert pipeline on gfx950 (MI355X): dispatch -> grouped gate/up GEMM + GLU ->
grouped down GEMM -> gate-weighted combine, with a hand-written backward. Every step runs in the HIP
library libmoe_gfx950.so (C ABI in include/moe_gfx950.h); this module only allocates buffers,
checks arguments and wires the autograd contract.

API and contract follow the reference `kernels.sm75.moe` (/root/reference/kernels/sm75/moe.py):
    moe(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj, act_codes, act_params=None)
    moe_per_expert(...)  same signature                              (moe.py:829)
    moe_grouped(hidden, idx, wt, gate_up_proj, down_proj, act_codes) (moe.py:621)
    moe_eager(...)       the slow pure-PyTorch reference             (moe.py:884-909)
    BatchedGLU.apply(gate_up, row_act, row_alpha=None, row_gamma=None)  (moe.py:450-474)
Weights: gate_up_proj (E_glu, 2I, H) with gate = rows [0, I) and up = rows [I, 2I); down_proj
(E_glu, H, I); act_codes (E,) int32 with GLU codes (0 SiLU, 1 ReLU^2, 2 NormSiLU, 5 SiTU,
6 NormReLU^2, 7 NormSiTU) first and the weightless specials (3 Identity, 4 Zero) after them.
The backward returns (grad_hidden, None, grad_top_k_weights, grad_gate_up_proj, grad_down_proj,
None, grad_act_params) (moe.py:825-826).

There is one implementation. `moe_per_expert`, `moe_grouped` and `moe` all run the same grouped
kernels: on this device a per-expert loop of library GEMMs has nothing to win over one grouped
launch, and no host sync happens anywhere on the path (the reference syncs at moe.py:568,741).
"""
import os

import torch
import torch.nn.functional as F

from .. import _lib

__all__ = ["moe", "moe_per_expert", "moe_grouped", "moe_grouped_cublas", "moe_eager",
           "BatchedGLU", "GROUPED_MIN_TOKENS"]

GROUPED_MIN_TOKENS = 4096   # kept for API compatibility (moe.py:78); every size takes one path
_NS_EPS = 1e-6              # RMS epsilon of the normalised codes 2/6/7 (moe.py:80)
GLU_CODES = (0, 1, 2, 5, 6, 7)
SPECIAL_CODES = (3, 4)
FUSED_CODES = (0, 1)        # codes the GEMM epilogues apply in registers
_CHECK_INDICES = os.environ.get("MOE_CHECK_INDICES", "0") == "1"


def _code_list(act_codes):
    """Host copy of the activation codes, cached on the tensor: act_codes is static model config,
    so this costs one device->host copy per tensor lifetime (the reference caches its max the
    same way, moe.py:84-94)."""
    c = getattr(act_codes, "_moe_codes_cache", None)
    if c is None:
        c = tuple(int(v) for v in act_codes.tolist())
        try:
            act_codes._moe_codes_cache = c
        except Exception:
            pass
    return c


def _code_max(act_codes):
    return max(_code_list(act_codes), default=0)


def _amp_cast(*ts):
    """Under autocast, cast float tensors to the active autocast dtype (moe.py:97-104)."""
    if torch.is_autocast_enabled("cuda"):
        dt = torch.get_autocast_dtype("cuda")
        return tuple(t.to(dt) if (t is not None and t.is_floating_point()) else t for t in ts)
    return ts


def _check_codes(codes, e_glu):
    for e, c in enumerate(codes):
        if e < e_glu and c not in GLU_CODES:
            raise ValueError(f"act code {c} at expert {e}: GLU experts (codes {GLU_CODES}) must come "
                             f"first, one per weight slot")
        if e >= e_glu and c not in SPECIAL_CODES:
            raise ValueError(f"act code {c} at expert {e}: experts past the {e_glu} weight slots must "
                             f"be Identity (3) or Zero (4)")


def _check_inputs(hidden, idx, wt, gate_up_proj, down_proj, act_codes):
    if not hidden.is_cuda:
        raise RuntimeError("the gfx950 MoE path needs device tensors (ROCm 'cuda' device); "
                           "moe_eager is the pure-PyTorch reference")
    if hidden.dim() != 2 or idx.dim() != 2 or wt.shape != idx.shape or idx.shape[0] != hidden.shape[0]:
        raise ValueError("expected hidden (N,H), top_k_indices and top_k_weights (N,k)")
    if gate_up_proj.dim() != 3 or down_proj.dim() != 3:
        raise ValueError("expected gate_up_proj (E,2I,H) and down_proj (E,H,I)")
    e_glu, two_i, h = gate_up_proj.shape
    if h != hidden.shape[1] or two_i % 2 or down_proj.shape != (e_glu, h, two_i // 2):
        raise ValueError(f"weight shapes {tuple(gate_up_proj.shape)} / {tuple(down_proj.shape)} do not "
                         f"match hidden {tuple(hidden.shape)}")
    if act_codes.dim() != 1 or act_codes.numel() < e_glu:
        raise ValueError("act_codes must be (E,) with E >= number of weight slots")
    if h % 8 or (two_i // 2) % 8:
        raise ValueError("H and I must be multiples of 8 (16-byte rows)")
    if idx.dtype not in (torch.int64,):
        raise TypeError("top_k_indices must be int64")


_STATUS_SINK = {}   # device index -> int32 scratch for dispatch counts nobody reads


def _status_sink(dev):
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    t = _STATUS_SINK.get(key)
    if t is None:
        t = _STATUS_SINK[key] = torch.zeros(1, device=dev, dtype=torch.int32)
    return t


class _Routing:
    """Device-resident dispatch result (see moe_dispatch in include/moe_gfx950.h). With
    want_status False the out-of-range count goes to a per-device scratch word that is never read
    (no zero-fill launch per call); `status` is then None."""

    def __init__(self, idx, n_experts, want_status=True):
        dev = idx.device
        n, k = idx.shape
        m = n * k
        i32 = dict(device=dev, dtype=torch.int32)
        self.counts = torch.empty(n_experts, **i32)
        self.offsets = torch.empty(n_experts + 1, **i32)
        self.tile_offsets = torch.empty(n_experts + 1, **i32)
        self.expert_order = torch.empty(n_experts, **i32)
        self.n_experts = n_experts
        self.sorted_token = torch.empty(max(m, 1), **i32)
        self.sorted_flat = torch.empty(max(m, 1), **i32)
        self.flat_to_sorted = torch.empty(max(m, 1), **i32)
        status = torch.zeros(1, **i32) if want_status else _status_sink(dev)
        self.status = status if want_status else None
        ws = _lib.lib().moe_get_workspace_size(n, k, n_experts)
        self.workspace = torch.empty(max(ws, 256), device=dev, dtype=torch.uint8)
        _lib.call("moe_dispatch", _lib.ptr(idx), n, k, n_experts, _lib.ptr(self.counts),
                  _lib.ptr(self.offsets), _lib.ptr(self.tile_offsets), _lib.ptr(self.expert_order),
                  _lib.ptr(self.sorted_token),
                  _lib.ptr(self.sorted_flat), _lib.ptr(self.flat_to_sorted), _lib.ptr(status),
                  _lib.ptr(self.workspace), self.workspace.numel(), _lib.stream_of(dev))
        if want_status and _CHECK_INDICES and int(self.status.item()) != 0:
            raise ValueError(f"{int(self.status.item())} top_k_indices outside [0, {n_experts})")

    def row_expert(self, n_experts, m):
        """Expert id of every sorted row (device op, no host sync): the e with
        offsets[e] <= r < offsets[e+1]. Rows past the routed count offsets[E] (there are fewer than
        N*k routed rows when some ids lie outside [0, E), which dispatch drops) get the value
        n_experts, which indexes nothing: callers clamp it for gathers and mask it for scatters."""
        rows = torch.arange(m, device=self.offsets.device, dtype=torch.int32)
        return torch.searchsorted(self.offsets[1:n_experts + 1], rows, right=True)


def dispatch(top_k_indices, n_experts):
    """Public dispatch: returns the _Routing of (N,k) int64 expert ids."""
    return _Routing(top_k_indices.contiguous(), n_experts)


def _row_params(routing, codes_t, ap32, n_experts, m):
    """Per sorted row: act code, SiTU alpha/gamma (or None) and expert id (unfused GLU path).
    The returned expert id is n_experts for rows past the routed count; the per-row gathers here
    read a clamped copy (those rows are computed by the row kernels but never read downstream)."""
    rexp = routing.row_expert(n_experts, m)
    rclamp = rexp.clamp(max=max(n_experts - 1, 0))
    row_act = codes_t.to(torch.int32).index_select(0, rclamp).contiguous()
    if ap32 is not None:
        ap_full = torch.ones(n_experts, 2, device=ap32.device, dtype=torch.float32)
        n_ap = min(ap32.shape[0], n_experts)
        ap_full[:n_ap] = ap32[:n_ap]
        row_alpha = ap_full[:, 0].index_select(0, rclamp).contiguous()
        row_gamma = ap_full[:, 1].index_select(0, rclamp).contiguous()
    else:
        row_alpha = row_gamma = None
    return row_act, row_alpha, row_gamma, rexp


def _gated_bwd(fused, e_glu, m, dt, h):
    """Whether the backward folds the combine backward into the down-dX GEMM (fused codes,
    16-bit dtypes, H a multiple of the GEMM's 64-wide K step)."""
    return fused and e_glu > 0 and m > 0 and dt != torch.float32 and h % 64 == 0


class _MoEFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, idx, wt, gate_up_proj, down_proj, act_codes, act_params):
        hidden, wt, gate_up_proj, down_proj = _amp_cast(hidden, wt, gate_up_proj, down_proj)
        _check_inputs(hidden, idx, wt, gate_up_proj, down_proj, act_codes)
        dt = hidden.dtype
        dtc = _lib.dtype_code(dt)
        hidden = hidden.contiguous()
        idx = idx.contiguous()
        wt = wt.to(dt).contiguous()
        gate_up_proj = gate_up_proj.to(dt).contiguous()
        down_proj = down_proj.to(dt).contiguous()
        codes = _code_list(act_codes)
        n_tok, h = hidden.shape
        k = idx.shape[1]
        e_glu, two_i, _ = gate_up_proj.shape
        inter_dim = two_i // 2
        n_exp = len(codes)
        _check_codes(codes, e_glu)
        codes_t = act_codes.to(device=hidden.device, dtype=torch.int32).contiguous()
        ap32 = act_params.float().contiguous() if act_params is not None else None
        fused = all(c in FUSED_CODES for c in codes[:e_glu])
        m = n_tok * k
        dev = hidden.device
        stream = _lib.stream_of(dev)
        routing = _Routing(idx, n_exp, want_status=_CHECK_INDICES)

        gate_up = torch.empty(m, two_i, device=dev, dtype=dt)
        inter = torch.empty(m, inter_dim, device=dev, dtype=dt)
        eo = torch.empty(m, h, device=dev, dtype=dt)
        row = None
        # With the folded backward the saved intermediate is gate-weighted (w * act(g) * u): the
        # down projection then yields w * eo, the combine only sums, and the backward's down
        # weight gradient reads it as is.
        gated = _gated_bwd(fused, e_glu, m, dt, h)
        # Gates in sorted-row order (one load per row in the GEMM epilogues instead of two). Rows
        # past the routed count (out-of-range expert ids) hold no index: clamped, never read.
        w_sorted = (torch.index_select(wt.view(-1), 0, routing.sorted_flat.clamp(0, m - 1))
                    if gated else None)
        if e_glu > 0 and m > 0:
            _lib.call("moe_grouped_gateup_swiglu_fwd", dtc, _lib.ptr(hidden), n_tok, h,
                      _lib.ptr(gate_up_proj), e_glu, inter_dim, _lib.ptr(codes_t),
                      _lib.ptr(routing.offsets), _lib.ptr(routing.tile_offsets),
                      _lib.ptr(routing.sorted_token), m, _lib.ptr(gate_up),
                      _lib.ptr(inter) if fused else None, _lib.ptr(w_sorted), None, stream)
            if not fused:
                row = _row_params(routing, codes_t, ap32, n_exp, m)
                row_act, ra, rg, _ = row
                _lib.call("moe_glu_fwd", dtc, _lib.ptr(gate_up), two_i, _lib.ptr(row_act),
                          _lib.ptr(ra), _lib.ptr(rg), 1, m, inter_dim, _lib.ptr(inter), inter_dim,
                          stream)
            _lib.call("moe_grouped_down_fwd", dtc, _lib.ptr(inter), _lib.ptr(down_proj), e_glu, h,
                      inter_dim, _lib.ptr(routing.offsets), _lib.ptr(routing.tile_offsets), m,
                      _lib.ptr(eo), *_lib.split_workspace(dev), stream)
        out = torch.empty(n_tok, h, device=dev, dtype=dt)
        _lib.call("moe_combine_fwd", dtc, _lib.ptr(eo), _lib.ptr(hidden), _lib.ptr(wt),
                  _lib.ptr(idx), _lib.ptr(codes_t), n_exp, e_glu, _lib.ptr(routing.flat_to_sorted),
                  n_tok, k, h, int(gated), _lib.ptr(out), stream)

        # The folded backward recomputes <grad_out, eo> from gate_up, so eo need not stay alive.
        keep_eo = torch.empty(0) if gated else eo
        ctx.save_for_backward(hidden, idx, wt, gate_up_proj, down_proj, codes_t,
                              ap32 if ap32 is not None else torch.empty(0), gate_up, inter, keep_eo)
        ctx.routing = routing
        ctx.w_sorted = w_sorted
        ctx.row = row
        ctx.meta = (n_tok, h, inter_dim, k, e_glu, n_exp, fused, ap32 is not None)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        (hidden, idx, wt, gate_up_proj, down_proj, codes_t, ap32, gate_up, inter,
         eo) = ctx.saved_tensors
        n_tok, h, inter_dim, k, e_glu, n_exp, fused, has_ap = ctx.meta
        routing = ctx.routing
        dt = hidden.dtype
        dtc = _lib.dtype_code(dt)
        dev = hidden.device
        stream = _lib.stream_of(dev)
        m = n_tok * k
        two_i = 2 * inter_dim
        vec = 4 if dt == torch.float32 else 8
        go = grad_out.to(dt)
        if (go.stride(1) != 1 or go.stride(0) % vec or go.stride(0) < h
                or go.data_ptr() % 16):
            go = go.contiguous()
        go_ld = go.stride(0)
        need_x, need_wt, need_gu, need_dw = (ctx.needs_input_grad[0], ctx.needs_input_grad[2],
                                             ctx.needs_input_grad[3], ctx.needs_input_grad[4])
        need_ap = has_ap and ctx.needs_input_grad[6]

        if _gated_bwd(fused, e_glu, m, dt, h):
            return _backward_gated(ctx, go, need_x, need_wt, need_gu, need_dw, need_ap)

        grad_eo = torch.empty(m, h, device=dev, dtype=dt)
        grad_wt = torch.zeros(n_tok * k, device=dev, dtype=dt)
        if m > 0:
            _lib.call("moe_combine_bwd", dtc, _lib.ptr(go), go_ld, _lib.ptr(eo), _lib.ptr(hidden),
                      _lib.ptr(wt), _lib.ptr(idx), _lib.ptr(codes_t), n_exp, e_glu,
                      _lib.ptr(routing.sorted_token), _lib.ptr(routing.sorted_flat), m, k, h,
                      _lib.ptr(grad_eo), _lib.ptr(grad_wt), stream)

        g_gu = g_dw = g_x = g_ap = None
        ggu = None
        if e_glu > 0 and m > 0 and (need_x or need_gu or need_dw or need_ap):
            if need_x or need_gu or need_ap:
                ggu = torch.empty(m, two_i, device=dev, dtype=dt)
                if fused:
                    _lib.call("moe_grouped_down_dx_swiglu_bwd", dtc, _lib.ptr(grad_eo),
                              _lib.ptr(down_proj), e_glu, h, inter_dim, _lib.ptr(gate_up),
                              _lib.ptr(codes_t), _lib.ptr(routing.offsets),
                              _lib.ptr(routing.tile_offsets), m, _lib.ptr(ggu), None, stream)
                else:
                    grad_inter = torch.empty(m, inter_dim, device=dev, dtype=dt)
                    _lib.call("moe_grouped_down_dx_swiglu_bwd", dtc, _lib.ptr(grad_eo),
                              _lib.ptr(down_proj), e_glu, h, inter_dim, None, None,
                              _lib.ptr(routing.offsets), _lib.ptr(routing.tile_offsets), m, None,
                              _lib.ptr(grad_inter), stream)
                    row_act, ra, rg, rexp = ctx.row
                    da = dg = None
                    if need_ap:
                        da = torch.empty(m, device=dev, dtype=torch.float32)
                        dg = torch.empty(m, device=dev, dtype=torch.float32)
                    _lib.call("moe_glu_bwd", dtc, _lib.ptr(grad_inter), inter_dim, 1,
                              _lib.ptr(gate_up), two_i, _lib.ptr(row_act), _lib.ptr(ra),
                              _lib.ptr(rg), 1, m, inter_dim, _lib.ptr(ggu), two_i, _lib.ptr(da),
                              _lib.ptr(dg), stream)
                    if need_ap:
                        g_ap = torch.zeros(ap32.shape[0], 2, device=dev, dtype=torch.float32)
                        valid = rexp < min(ap32.shape[0], n_exp)   # routed rows only
                        g_ap[:, 0].index_add_(0, rexp[valid], da[valid])
                        g_ap[:, 1].index_add_(0, rexp[valid], dg[valid])
            if need_dw:
                g_dw = torch.empty_like(down_proj)
                _lib.call("moe_grouped_wgrad", dtc, _lib.ptr(inter), inter_dim, None,
                          _lib.ptr(grad_eo), h, None, inter_dim, h, _lib.ptr(routing.offsets),
                          _lib.ptr(routing.expert_order), n_exp, e_glu, _lib.ptr(g_dw),
                          *_lib.split_workspace(dev), stream, tag="down")
            if need_gu:
                g_gu = torch.empty_like(gate_up_proj)
                _lib.call("moe_grouped_wgrad", dtc, _lib.ptr(hidden), h,
                          _lib.ptr(routing.sorted_token), _lib.ptr(ggu), two_i, None, h, two_i,
                          _lib.ptr(routing.offsets), _lib.ptr(routing.expert_order), n_exp, e_glu,
                          _lib.ptr(g_gu), *_lib.split_workspace(dev), stream, tag="gate_up")
        elif e_glu > 0:
            if need_dw:
                g_dw = torch.zeros_like(down_proj)
            if need_gu:
                g_gu = torch.zeros_like(gate_up_proj)
        if need_ap and g_ap is None:
            g_ap = torch.zeros_like(ap32)
        if need_x:
            gxs = None
            if ggu is not None:
                gxs = torch.empty(m, h, device=dev, dtype=dt)
                _lib.call("moe_grouped_gateup_dx", dtc, _lib.ptr(ggu), _lib.ptr(gate_up_proj),
                          e_glu, h, inter_dim, _lib.ptr(routing.offsets),
                          _lib.ptr(routing.tile_offsets), m, _lib.ptr(gxs),
                          *_lib.split_workspace(dev), stream)
            g_x = torch.empty(n_tok, h, device=dev, dtype=dt)
            _lib.call("moe_unpermute_bwd", dtc, _lib.ptr(gxs), _lib.ptr(go), go_ld, _lib.ptr(wt),
                      _lib.ptr(idx), _lib.ptr(codes_t), n_exp, e_glu if gxs is not None else 0,
                      _lib.ptr(routing.flat_to_sorted), n_tok, k, h, _lib.ptr(g_x), stream)
        return (g_x, None, grad_wt.view(n_tok, k) if need_wt else None, g_gu, g_dw, None, g_ap)


def _backward_gated(ctx, go, need_x, need_wt, need_gu, need_dw, need_ap):
    """Backward for fused activation codes with the combine backward folded into the down-dX GEMM:
    grad_eo = w * grad_out is never stored; that GEMM gathers grad_out rows itself, applies w in
    its epilogue and writes per-slice partials of the gate gradient <grad_out, eo> =
    <grad_out @ W_d, inter> with inter recomputed from gate_up (kernels/sm75/moe.py:606-617,712-720).
    The forward saved the gate-weighted intermediate w * inter, which is what the down weight
    gradient sum_m (w inter)^T grad_out needs."""
    (hidden, idx, wt, gate_up_proj, down_proj, codes_t, ap32, gate_up, inter_w,
     _eo) = ctx.saved_tensors
    n_tok, h, inter_dim, k, e_glu, n_exp, _fused, _has_ap = ctx.meta
    routing = ctx.routing
    dt = hidden.dtype
    dtc = _lib.dtype_code(dt)
    dev = hidden.device
    stream = _lib.stream_of(dev)
    m = n_tok * k
    go_ld = go.stride(0)
    if not (need_x or need_wt or need_gu or need_dw):
        return (None, None, None, None, None, None, torch.zeros_like(ap32) if need_ap else None)
    n_parts = _lib.lib().moe_gate_grad_parts(inter_dim)
    part = torch.empty(n_parts, m, device=dev, dtype=torch.float32)
    ggu = torch.empty(m, 2 * inter_dim, device=dev, dtype=dt) if (need_x or need_gu) else None
    _lib.call("moe_grouped_down_dx_gated_bwd", dtc, _lib.ptr(go), go_ld, _lib.ptr(down_proj),
              e_glu, h, inter_dim, _lib.ptr(gate_up), _lib.ptr(codes_t), _lib.ptr(ctx.w_sorted),
              _lib.ptr(routing.offsets), _lib.ptr(routing.sorted_token), None, m, _lib.ptr(ggu),
              None, _lib.ptr(part), stream)
    g_wt = g_dw = g_gu = g_x = None
    if need_wt:
        g_wt = torch.empty(n_tok, k, device=dev, dtype=dt)
        _lib.call("moe_gate_grad", dtc, _lib.ptr(part), n_parts, m, _lib.ptr(go), go_ld,
                  _lib.ptr(hidden), _lib.ptr(idx), _lib.ptr(codes_t), n_exp, e_glu,
                  _lib.ptr(routing.flat_to_sorted), n_tok, k, h, _lib.ptr(g_wt), stream)
    if need_dw:
        g_dw = torch.empty_like(down_proj)
        _lib.call("moe_grouped_wgrad", dtc, _lib.ptr(inter_w), inter_dim, None, _lib.ptr(go),
                  go_ld, _lib.ptr(routing.sorted_token), inter_dim, h, _lib.ptr(routing.offsets),
                  _lib.ptr(routing.expert_order), n_exp, e_glu, _lib.ptr(g_dw),
                  *_lib.split_workspace(dev), stream, tag="down")
    if need_gu:
        g_gu = torch.empty_like(gate_up_proj)
        _lib.call("moe_grouped_wgrad", dtc, _lib.ptr(hidden), h, _lib.ptr(routing.sorted_token),
                  _lib.ptr(ggu), 2 * inter_dim, None, h, 2 * inter_dim, _lib.ptr(routing.offsets),
                  _lib.ptr(routing.expert_order), n_exp, e_glu, _lib.ptr(g_gu),
                  *_lib.split_workspace(dev), stream, tag="gate_up")
    if need_x:
        gxs = torch.empty(m, h, device=dev, dtype=dt)
        _lib.call("moe_grouped_gateup_dx", dtc, _lib.ptr(ggu), _lib.ptr(gate_up_proj), e_glu, h,
                  inter_dim, _lib.ptr(routing.offsets), _lib.ptr(routing.tile_offsets), m,
                  _lib.ptr(gxs), *_lib.split_workspace(dev), stream)
        g_x = torch.empty(n_tok, h, device=dev, dtype=dt)
        _lib.call("moe_unpermute_bwd", dtc, _lib.ptr(gxs), _lib.ptr(go), go_ld, _lib.ptr(wt),
                  _lib.ptr(idx), _lib.ptr(codes_t), n_exp, e_glu, _lib.ptr(routing.flat_to_sorted),
                  n_tok, k, h, _lib.ptr(g_x), stream)
    g_ap = torch.zeros_like(ap32) if need_ap else None
    return (g_x, None, g_wt, g_gu, g_dw, None, g_ap)


def moe_per_expert(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj, act_codes,
                   act_params=None):
    """Full PolyGLU MoE with a hand-written backward (reference moe.py:829-835). act_params: (E,2)
    fp32 [alpha, gamma] for SiTU experts (code 5); None means alpha = gamma = 1."""
    return _MoEFunction.apply(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj,
                              act_codes, act_params)


def moe_grouped(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj, act_codes):
    """Grouped entry point (reference moe.py:621-629); like the reference it rejects code 5,
    which needs act_params that only moe_per_expert carries."""
    if _code_max(act_codes) > 4:
        raise ValueError("code 5 (SiTU) unsupported on the grouped path; use moe_per_expert(act_params=...)")
    return _MoEFunction.apply(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj,
                              act_codes, None)


def moe_grouped_cublas(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj, act_codes):
    """Name kept from the reference's library-grouped candidate (moe.py:637-665); same kernels."""
    return moe_grouped(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj, act_codes)


def moe(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj, act_codes, act_params=None):
    """Auto entry point (reference moe.py:838-855). One path serves every shape and code here."""
    return moe_per_expert(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj, act_codes,
                          act_params)


# ───────────────────────── PolyGLU activation as a standalone op ─────────────────────────
class BatchedGLU(torch.autograd.Function):
    """out = act_{row}(gate) * up with a per-row activation code (reference moe.py:450-474).
    Optional per-row SiTU scalars (code 5); their grads come back per row in fp32."""

    @staticmethod
    def forward(ctx, gate_up, row_act, row_alpha=None, row_gamma=None):
        if (row_alpha is None) != (row_gamma is None):
            raise ValueError("row_alpha and row_gamma must be passed together (both or neither)")
        if not gate_up.is_cuda:
            raise RuntimeError("BatchedGLU runs on the device; gate_up is on the host")
        m, two_i = gate_up.shape
        inter_dim = two_i // 2
        gu = gate_up if gate_up.stride(1) == 1 else gate_up.contiguous()
        ra = row_alpha.float().contiguous() if row_alpha is not None else None
        rg = row_gamma.float().contiguous() if row_gamma is not None else None
        ap_stride = 0 if (ra is not None and ra.numel() == 1) else 1
        ra_ = row_act.to(torch.int32).contiguous()
        out = torch.empty(m, inter_dim, device=gate_up.device, dtype=gate_up.dtype)
        _lib.call("moe_glu_fwd", _lib.dtype_code(gate_up.dtype), _lib.ptr(gu), gu.stride(0),
                  _lib.ptr(ra_), _lib.ptr(ra), _lib.ptr(rg), ap_stride, m, inter_dim,
                  _lib.ptr(out), inter_dim, _lib.stream_of(gate_up.device))
        ctx.save_for_backward(gu, ra_, ra if ra is not None else torch.empty(0),
                              rg if rg is not None else torch.empty(0))
        ctx.has_situ = ra is not None
        ctx.ap_stride = ap_stride
        return out

    @staticmethod
    def backward(ctx, grad_out):
        gu, row_act, ra, rg = ctx.saved_tensors
        m, two_i = gu.shape
        inter_dim = two_i // 2
        go = grad_out.to(gu.dtype)
        ggu = torch.empty(m, two_i, device=gu.device, dtype=gu.dtype)
        want = ctx.has_situ and (ctx.needs_input_grad[2] or ctx.needs_input_grad[3])
        da = torch.empty(m, device=gu.device, dtype=torch.float32) if want else None
        dg = torch.empty(m, device=gu.device, dtype=torch.float32) if want else None
        _lib.call("moe_glu_bwd", _lib.dtype_code(gu.dtype), _lib.ptr(go), go.stride(0),
                  go.stride(1), _lib.ptr(gu), gu.stride(0), _lib.ptr(row_act),
                  _lib.ptr(ra) if ctx.has_situ else None, _lib.ptr(rg) if ctx.has_situ else None,
                  ctx.ap_stride, m, inter_dim, _lib.ptr(ggu), two_i, _lib.ptr(da), _lib.ptr(dg),
                  _lib.stream_of(gu.device))
        if want:
            if ctx.ap_stride == 0:   # one broadcast scalar: its grad is the sum over rows
                da, dg = da.sum().reshape(1), dg.sum().reshape(1)
            return ggu, None, da, dg
        return ggu, None, None, None


# ───────────────────────── eager reference (the slow baseline) ─────────────────────────
def _act_eager(gate, code, alpha=None, gamma=None):
    """Activation of one GLU expert on its gate half (reference moe.py:859-881)."""
    if code == 0:
        return F.silu(gate)
    if code == 1:
        return F.relu(gate) ** 2
    g = gate.float()
    if code == 5:
        return (gamma * torch.tanh(alpha * g) * torch.sigmoid(g)).to(gate.dtype)
    g = g * torch.rsqrt(g.square().mean(-1, keepdim=True) + _NS_EPS)
    if code == 6:
        return (F.relu(g) ** 2).to(gate.dtype)
    if code == 7:
        return (torch.tanh(g) * torch.sigmoid(g)).to(gate.dtype)
    return F.silu(g).to(gate.dtype)   # code 2


def moe_eager(hidden, top_k_indices, top_k_weights, gate_up_proj, down_proj, act_codes,
              act_params=None):
    """Plain PyTorch MoE: per-expert mask, gather, two linears, activation, weighted fp32
    accumulation (reference moe.py:884-909). Autograd gives its backward. Slow by design."""
    n, h = hidden.shape
    inter_dim = gate_up_proj.shape[1] // 2
    codes = _code_list(act_codes)
    out = torch.zeros(n, h, device=hidden.device, dtype=torch.float32)
    for e, code in enumerate(codes):
        hit = top_k_indices == e
        rows = hit.any(-1)
        if not bool(rows.any()):
            continue
        w = (top_k_weights * hit).sum(-1)[rows]
        if code == 4:
            continue
        if code == 3:
            out[rows] += (hidden[rows] * w.unsqueeze(-1)).float()
            continue
        gu = hidden[rows] @ gate_up_proj[e].t()
        a, g = ((act_params[e, 0], act_params[e, 1]) if code == 5 and act_params is not None
                else (1.0, 1.0))
        inter = _act_eager(gu[:, :inter_dim], code, a, g) * gu[:, inter_dim:]
        out[rows] += ((inter @ down_proj[e].t()) * w.unsqueeze(-1)).float()
    return out.to(hidden.dtype)
