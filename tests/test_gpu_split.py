"""The long-K split of the plain-store token GEMMs (moe_grouped_down_fwd, moe_grouped_gateup_dx).

With a split workspace, K of at least 40 ring steps (K >= 2560) and an XCD whose share of tiles
leaves a partial last wave, each such tile is cut along K into pieces whose fp32 partials the last
arriving piece sums in piece order. These shapes (K = 2816 and 5632, a few ragged experts) put
every tile in a partial wave, so every tile splits. Checked: the result against fp32 torch and
against the same call without a workspace (no split), two calls bit-identical (the sum order does
not depend on which piece arrives last), and the workspace's counters back at zero afterwards.
"""
import pytest
import torch

from kernels import _lib

pytestmark = pytest.mark.gpu

COUNTS = [300, 517, 0, 9]      # ragged experts, one empty
H, I = 1024, 2816


def _offsets(counts):
    o = torch.zeros(len(counts) + 1, dtype=torch.int32)
    o[1:] = torch.cumsum(torch.tensor(counts), 0)
    return o.cuda()


def _ref(a, w, counts, transpose_w):
    out, s = [], 0
    for e, c in enumerate(counts):
        we = w[e].float()
        out.append(a[s:s + c].float() @ (we if transpose_w else we.t()))
        s += c
    return torch.cat(out)


def _call(name, a, w, offs, m, out_shape, ws):
    out = torch.full(out_shape, float("nan"), device="cuda", dtype=torch.bfloat16)
    _lib.call(name, _lib.dtype_code(torch.bfloat16), _lib.ptr(a), _lib.ptr(w), w.shape[0], H, I,
              _lib.ptr(offs), None, m, _lib.ptr(out), _lib.ptr(ws),
              ws.numel() if ws is not None else 0, _lib.stream_of(a.device))
    return out


@pytest.mark.parametrize("which", ["down_fwd", "gateup_dx"])
def test_split_matches_unsplit_is_deterministic_and_clears_counters(which):
    print(f"[gpu-case] K split {which}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(3)
    m = sum(COUNTS)
    e = len(COUNTS)
    offs = _offsets(COUNTS)
    if which == "down_fwd":                    # eo = inter @ down^T, K = I
        name, a = "moe_grouped_down_fwd", torch.randn(m, I, generator=g, device="cuda")
        w, tw = torch.randn(e, H, I, generator=g, device="cuda") / I ** 0.5, False
    else:                                      # grad_x_s = ggu @ gate_up, K = 2I
        name, a = "moe_grouped_gateup_dx", torch.randn(m, 2 * I, generator=g, device="cuda")
        w, tw = torch.randn(e, 2 * I, H, generator=g, device="cuda") / (2 * I) ** 0.5, True
    a, w = a.bfloat16(), w.bfloat16()
    n_ws = _lib.lib().moe_token_split_workspace_size()
    ws = torch.zeros(n_ws, device="cuda", dtype=torch.uint8)
    s1 = _call(name, a, w, offs, m, (m, H), ws)
    s2 = _call(name, a, w, offs, m, (m, H), ws)
    plain = _call(name, a, w, offs, m, (m, H), None)
    torch.cuda.synchronize()
    ref = _ref(a, w, COUNTS, tw)
    assert torch.equal(s1, s2)
    for got in (s1, plain):
        d = (got.float() - ref).abs()
        assert bool(torch.isfinite(got).all())
        assert (d <= 1e-2 * ref.abs() + 1e-2).all(), d.max().item()
    # the split and unsplit sums differ only by fp32 summation order before the bf16 store
    assert ((s1.float() - plain.float()).abs() <= 2 ** -7 * plain.float().abs() + 1e-3).all()
    n_cus = torch.cuda.get_device_properties(0).multi_processor_count
    # the split path ran: its fp32 partial sums were written into the (zeroed) workspace
    assert bool(ws[: n_cus * 65536 * 4].view(torch.int32).ne(0).any())
    counters = ws[n_cus * 65536 * 4:].view(torch.int32)
    assert int(counters.abs().sum()) == 0


WG_CASES = [  # (row counts per expert, R, C, gathered rows): expert tiles <= CUs / 4, so the
    # split runs (2 pieces per tile)
    ([3000, 2950, 0, 3100, 2990, 3007, 2800, 3333, 2999], 768, 512, True),    # 54 tiles
    ([700, 0, 65, 1], 256, 256, False),                                       # 4 tiles
]


@pytest.mark.parametrize("counts,R,C,gather", WG_CASES, ids=["stack-down", "tiny"])
def test_wgrad_split_matches_unsplit_is_deterministic_and_clears_counters(counts, R, C, gather):
    """moe_grouped_wgrad with the split workspace, when the experts' tiles fill at most a quarter
    of the CUs: each tile's rows are cut into two pieces (whole 64-row steps, empty pieces for short or empty
    experts) summed in piece order. Checked against fp32 torch, against the call without a
    workspace (no split), run to run bitwise, counters left at zero, partial slots written."""
    print(f"[gpu-case] wgrad split counts={counts} R={R} C={C}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(5)
    m, e = sum(counts), len(counts)
    offs = _offsets(counts)
    n_src = m + 17
    rsrc = torch.randn(n_src, R, generator=g, device="cuda").bfloat16()
    csrc = torch.randn(m, C, generator=g, device="cuda").bfloat16()
    gat = torch.randperm(n_src, generator=g, device="cuda")[:m].int() if gather else None
    n_ws = _lib.lib().moe_token_split_workspace_size()
    ws = torch.zeros(n_ws, device="cuda", dtype=torch.uint8)

    def run(w):
        out = torch.full((e, C, R), float("nan"), device="cuda", dtype=torch.bfloat16)
        _lib.call("moe_grouped_wgrad", _lib.dtype_code(torch.bfloat16), _lib.ptr(rsrc), R,
                  _lib.ptr(gat), _lib.ptr(csrc), C, None, R, C, _lib.ptr(offs), None, e, e,
                  _lib.ptr(out), _lib.ptr(w), w.numel() if w is not None else 0,
                  _lib.stream_of(rsrc.device))
        return out
    s1, s2, plain = run(ws), run(ws), run(None)
    torch.cuda.synchronize()
    rows = rsrc[gat.long()] if gather else rsrc[:m]
    s = 0
    for x, c in enumerate(counts):
        ref = csrc[s:s + c].float().t() @ rows[s:s + c].float()
        d = (s1[x].float() - ref).abs()
        assert bool(torch.isfinite(s1[x]).all())
        assert (d <= 1e-2 * ref.abs() + 2e-2).all(), (x, d.max().item())
        assert ((plain[x].float() - s1[x].float()).abs() <= 2 ** -7 * ref.abs() + 2e-2).all()
        s += c
    assert torch.equal(s1, s2)
    n_cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert bool(ws[: n_cus * 65536 * 4].view(torch.int32).ne(0).any())
    assert int(ws[n_cus * 65536 * 4:].view(torch.int32).abs().sum()) == 0
