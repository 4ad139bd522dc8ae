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
