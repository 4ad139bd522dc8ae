"""Pins of the CPU oracle (oracle/moe_oracle.py) against independent checks.

The reference ships no golden vectors or fixtures for this path (its gates are executable CUDA
scripts: parity_situ.py, bench.py:638-646, .autoresearch/grouped_parity.py), so each oracle
function is pinned by something that does not share its formula:
  dispatch_np     vs brute-force loops, plus permutation / grouping invariants;
  act             vs closed forms at chosen points and vs torch autograd of a second formulation;
  moe_forward     vs moe_dense (every expert on every token, dense gate matrix);
  moe_fwd_bwd     vs manual_backward (the reference's grouped backward formulas, per expert);
  fp8 / MXFP8     quantiser round trips, exact powers of two, and error bounds;
  fixture         vs tests/golden/config1.npz (regression of generator + oracle).
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe_oracle as orc
from kernels.workloads import make_workload, CONFIGS
from kernels.gfx950 import quant

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config1.npz")


def _rand_idx(n, k, e, seed, lo=0, hi=None):
    g = torch.Generator().manual_seed(seed)
    hi = e if hi is None else hi
    # k distinct experts per token from [lo, hi)
    s = torch.rand(n, hi - lo, generator=g)
    return (s.topk(k, dim=-1).indices + lo).numpy()


@pytest.mark.parametrize("n,k,e,seed", [(1, 1, 1, 0), (7, 2, 5, 1), (64, 4, 16, 2), (300, 8, 64, 3),
                                        (129, 3, 9, 4)])
def test_dispatch_np_matches_loops(n, k, e, seed):
    idx = _rand_idx(n, k, e, seed)
    a, b = orc.dispatch_np(idx, e), orc.dispatch_loops(idx, e)
    for key in ("counts", "offsets", "sorted_token", "sorted_flat", "flat_to_sorted"):
        np.testing.assert_array_equal(a[key], b[key], err_msg=key)


def test_dispatch_invariants_and_empty_experts():
    idx = _rand_idx(500, 4, 8, 5, lo=0, hi=5)   # experts 5..7 get no rows
    e = 12
    d = orc.dispatch_np(idx, e)
    m = idx.size
    assert d["counts"].sum() == m and (d["counts"][5:] == 0).all()
    assert sorted(d["sorted_flat"].tolist()) == list(range(m))            # bijection
    flat = idx.reshape(-1)
    ex = flat[d["sorted_flat"]]
    assert (np.diff(ex) >= 0).all()                                       # grouped by expert
    for g in range(e):                                                    # stable within groups
        s, t = d["offsets"][g], d["offsets"][g + 1]
        assert (np.diff(d["sorted_flat"][s:t]) > 0).all()
    assert (d["flat_to_sorted"][d["sorted_flat"]] == np.arange(m)).all()
    assert (d["sorted_token"] == d["sorted_flat"] // 4).all()


def test_dispatch_drops_out_of_range():
    idx = np.array([[0, 3], [-1, 1], [2, 9]])
    d = orc.dispatch_np(idx, 4)
    assert d["counts"].tolist() == [1, 1, 1, 1]
    assert d["flat_to_sorted"][2] == -1 and d["flat_to_sorted"][5] == -1
    assert d["sorted_flat"].tolist() == [0, 3, 4, 1]


def test_tile_offsets():
    assert orc.tile_offsets([0, 1, 128, 129, 0], 128).tolist() == [0, 0, 1, 2, 4, 4]


def test_act_closed_forms():
    g = torch.tensor([[-3.0, -0.5, 0.0, 0.7, 2.5]], dtype=torch.float64)
    sig = 1 / (1 + torch.exp(-g))
    torch.testing.assert_close(orc.act(g, 0), g * sig)
    torch.testing.assert_close(orc.act(g, 1), torch.clamp(g, min=0) ** 2)
    torch.testing.assert_close(orc.act(g, 5, 0.5, 2.0), 2.0 * torch.tanh(0.5 * g) * sig)
    r = torch.sqrt((g ** 2).mean() + orc.NS_EPS)
    gn = g / r
    torch.testing.assert_close(orc.act(g, 2), gn / (1 + torch.exp(-gn)))
    torch.testing.assert_close(orc.act(g, 6), torch.clamp(gn, min=0) ** 2)
    torch.testing.assert_close(orc.act(g, 7), torch.tanh(gn) / (1 + torch.exp(-gn)))


def test_silu_derivative_closed_form():
    # kernels/sm75/moe.py:206 uses d silu = s(1 + g(1 - s)); check against autograd
    g = torch.linspace(-6, 6, 101, dtype=torch.float64, requires_grad=True)
    F.silu(g).sum().backward()
    s = torch.sigmoid(g.detach())
    torch.testing.assert_close(g.grad, s * (1 + g.detach() * (1 - s)))


def _small_case(codes, e_glu, n=64, h=32, i=24, k=2, seed=0, dtype=torch.float64, cap=None):
    g = torch.Generator().manual_seed(seed)
    hid = torch.randn(n, h, generator=g, dtype=dtype)
    gu = torch.randn(e_glu, 2 * i, h, generator=g, dtype=dtype) * 0.2
    dw = torch.randn(e_glu, h, i, generator=g, dtype=dtype) * 0.2
    idx = torch.from_numpy(_rand_idx(n, k, len(codes), seed + 1, hi=cap))
    wt = torch.rand(n, k, generator=g, dtype=dtype)
    wt = wt / wt.sum(-1, keepdim=True)
    ap = torch.rand(len(codes), 2, generator=g, dtype=dtype) + 0.5
    return hid, idx, wt, gu, dw, ap


@pytest.mark.parametrize("codes,e_glu,cap", [
    ([0] * 6, 6, None), ([0, 1, 2, 5, 6, 7], 6, None), ([0, 5, 2, 5, 3, 4], 4, None),
    ([5, 5, 5, 5, 0, 2], 6, 4),
])
def test_moe_forward_vs_dense(codes, e_glu, cap):
    hid, idx, wt, gu, dw, ap = _small_case(codes, e_glu, cap=cap)
    a = orc.moe_forward(hid, idx, wt, gu, dw, codes, ap)
    b = orc.moe_dense(hid, idx, wt, gu, dw, codes, ap)
    torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-10)


def test_autograd_vs_manual_backward():
    hid, idx, wt, gu, dw, _ = _small_case([0] * 5, 5, n=80, k=3, seed=3)
    go = torch.randn(hid.shape, generator=torch.Generator().manual_seed(9), dtype=torch.float64)
    r = orc.moe_fwd_bwd(hid, idx, wt, gu, dw, [0] * 5, go, dtype=torch.float64)
    m = orc.manual_backward(hid, idx, wt, gu, dw, go)
    for key in ("grad_hidden", "grad_wt", "grad_gate_up", "grad_down"):
        torch.testing.assert_close(r[key], m[key], rtol=1e-10, atol=1e-10, msg=key)


def test_gradcheck_small_mixed_codes():
    # finite differences pin the autograd of every code, the specials and the SiTU params
    codes = [0, 1, 2, 5, 6, 7, 3, 4]
    hid, idx, wt, gu, dw, ap = _small_case(codes, 6, n=12, h=8, i=8, k=3, seed=11)

    def f(h_, w_, gu_, dw_, ap_):
        return orc.moe_forward(h_, idx, w_, gu_, dw_, codes, ap_)

    args = tuple(t.clone().requires_grad_(True) for t in (hid, wt, gu, dw, ap))
    assert torch.autograd.gradcheck(f, args, eps=1e-6, atol=1e-6)


def test_fp8_row_quantiser():
    x = torch.randn(37, 96, generator=torch.Generator().manual_seed(0))
    q, s = quant.quantize_fp8_rows(x)
    assert q.dtype == torch.float8_e4m3fn
    assert torch.all(q.float().abs().amax(-1) == 448.0)           # absmax maps to 448 exactly
    rel = (quant.dequantize_fp8_rows(q, s) - x).abs() / x.abs().clamp_min(1e-30)
    big = x.abs() >= s.unsqueeze(-1) * 2 ** -6                     # e4m3 normal range
    assert rel[big].max() <= 2 ** -4 + 1e-7                         # half an ulp of 3 mantissa bits


def test_e4m3_round_matches_table():
    # every finite positive e4m3fn value round-trips; midpoints go to even
    vals = torch.arange(0, 127, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    assert torch.equal(orc.e4m3_round(vals), vals)
    assert orc.e4m3_round(torch.tensor([1.0625])).item() == 1.0    # midpoint of 1.0 / 1.125
    assert orc.e4m3_round(torch.tensor([1.1875])).item() == 1.25   # midpoint of 1.125 / 1.25
    assert orc.e4m3_round(torch.tensor([1e6])).item() == 448.0


def test_mxfp8_quantiser():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 256, generator=g) * torch.logspace(-3, 3, 5).unsqueeze(-1)
    x[2, 32:64] = 0.0
    q, s = quant.quantize_mxfp8(x)
    assert s.shape == (5, 8) and s.dtype == torch.uint8 and s[2, 1] == 0
    xb = x.reshape(5, 8, 32)
    amax = xb.abs().amax(-1)
    exp = torch.floor(torch.log2(amax[amax > 0])) - 8 + 127
    assert torch.equal(s[amax > 0].float(), exp)                    # OCP MX shared exponent
    d = quant.dequantize_mxfp8(q, s)
    scale = torch.exp2(s.float() - 127).repeat_interleave(32, -1)
    err = (d - x).abs()
    sat = x.abs() > 448 * scale          # OCP MX clamps block elements in (448, 512) * scale
    bound = torch.maximum(x.abs() * 2 ** -4, scale * 2 ** -10)   # half ulp (normal / subnormal)
    assert torch.all(err[~sat] <= bound[~sat] + 1e-30)
    assert torch.allclose(d[sat].abs(), 448 * scale[sat])
    assert torch.all(q.float().abs() <= 448)


def test_fp8_forward_requant_only_differs_by_intermediate():
    w = make_workload(4, scale=dict(N=64, H=64, I=128, E=4, k=2))
    args = (w["x_q"], w["x_scale"], w["idx"], w["wt"], w["gate_up_q"], w["gate_up_scale"],
            w["down_q"], w["down_scale"])
    b = orc.fp8_forward(*args, requant_inter=False)
    for blk in (0, 128, 32):
        a = orc.fp8_forward(*args, requant_inter=True, requant_block=blk)
        rel = ((a - b).norm() / b.norm()).item()
        assert 1e-4 < rel < 5e-2, (blk, rel)


# ── independent pins of the fp8 / MXFP8 forwards ──
# The reference has no quantised path, so these pins come from the mathematics: (1) without the
# intermediate re-quantisation, the fp8 forward is the plain MoE forward on dequantised operands
# (the scales factor out of every dot product); (2) the MXFP8 forward is the plain MoE forward on
# block-dequantised weights; (3) the whole fp8 pipeline, re-quantisation included, equals scalar
# Python loops whose e4m3 rounding is a nearest-value search over the 8-bit code table decoded
# from its bit fields (no torch float8 conversion involved).

def _e4m3_table():
    """All finite non-negative e4m3fn values from their bit fields: (value, code) pairs."""
    out = []
    for code in range(0x7F):                       # 0x7F is NaN; the sign bit is handled apart
        e, m = code >> 3, code & 7
        v = (m / 8.0) * 2.0 ** -6 if e == 0 else (1.0 + m / 8.0) * 2.0 ** (e - 7)
        out.append((v, code))
    return out


_E4M3 = _e4m3_table()


def _e4m3_round_loop(x):
    """Nearest e4m3fn value by exhaustive search, ties to the even code, saturating at 448."""
    a = min(abs(x), 448.0)
    best = min(_E4M3, key=lambda vc: (abs(vc[0] - a), vc[1] & 1))
    return best[0] if x >= 0 else -best[0]


def test_e4m3_table_is_the_format():
    vals = [v for v, _ in _E4M3]
    assert vals[1] == 2.0 ** -9 and vals[8] == 2.0 ** -6 and vals[-1] == 448.0
    assert len(set(vals)) == 127 and vals == sorted(vals)
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(400, generator=g, dtype=torch.float64) * torch.logspace(-4, 3, 400,
                                                                            dtype=torch.float64))
    x = torch.cat([x, torch.tensor([1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, 500.0, -1e9],
                                   dtype=torch.float64)])
    ref = torch.tensor([_e4m3_round_loop(float(v)) for v in x], dtype=torch.float64)
    assert torch.equal(orc.e4m3_round(x), ref)


def _tiny_fp8_case(seed=0):
    return make_workload(4, seed=seed, scale=dict(N=6, H=32, I=32, E=3, k=2))


def test_fp8_forward_without_requant_is_moe_forward_on_dequantised_operands():
    w = make_workload(4, scale=dict(N=48, H=64, I=64, E=5, k=3), seed=2)
    f64 = torch.float64
    got = orc.fp8_forward(w["x_q"], w["x_scale"], w["idx"], w["wt"], w["gate_up_q"],
                          w["gate_up_scale"], w["down_q"], w["down_scale"], requant_inter=False,
                          dtype=f64)
    x = w["x_q"].to(f64) * w["x_scale"].to(f64).unsqueeze(-1)
    gu = w["gate_up_q"].to(f64) * w["gate_up_scale"].to(f64).unsqueeze(-1)
    dw = w["down_q"].to(f64) * w["down_scale"].to(f64).unsqueeze(-1)
    ref = orc.moe_dense(x, w["idx"], w["wt"].to(f64), gu, dw, [0] * 5)
    torch.testing.assert_close(got, ref, rtol=1e-10, atol=1e-10)
    ref2 = orc.moe_forward(x, w["idx"], w["wt"].to(f64), gu, dw, [0] * 5)
    torch.testing.assert_close(got, ref2, rtol=1e-10, atol=1e-10)


def test_fp8_forward_with_requant_matches_scalar_loops():
    w = _tiny_fp8_case(seed=3)
    got = orc.fp8_forward(w["x_q"], w["x_scale"], w["idx"], w["wt"], w["gate_up_q"],
                          w["gate_up_scale"], w["down_q"], w["down_scale"], requant_inter=True,
                          requant_block=0, dtype=torch.float64)
    xq, xs = w["x_q"].double().tolist(), w["x_scale"].double().tolist()
    gq, gs = w["gate_up_q"].double().tolist(), w["gate_up_scale"].double().tolist()
    dq, ds = w["down_q"].double().tolist(), w["down_scale"].double().tolist()
    idx, wt = w["idx"].tolist(), w["wt"].double().tolist()
    n, h, i = 6, 32, 32
    ref = [[0.0] * h for _ in range(n)]
    for t in range(n):
        for j, e in enumerate(idx[t]):
            gu = [sum(xq[t][c] * gq[e][r][c] for c in range(h)) * xs[t] * gs[e][r]
                  for r in range(2 * i)]
            y = [gu[c] / (1.0 + math.exp(-gu[c])) * gu[i + c] for c in range(i)]
            amax = max(abs(v) for v in y)
            s = amax / 448.0 if amax > 0 else 1.0
            y = [_e4m3_round_loop(v / s) * s for v in y]
            for r in range(h):
                ref[t][r] += wt[t][j] * sum(y[c] * dq[e][r][c] for c in range(i)) * ds[e][r]
    torch.testing.assert_close(got, torch.tensor(ref, dtype=torch.float64), rtol=1e-9, atol=1e-9)


def _e8m0_exponent_loop(amax):
    """Smallest integer e >= -127 with 448 * 2^e >= amax, by counting (no logarithms)."""
    e = -127
    while 448.0 * 2.0 ** e < amax:
        e += 1
    return e


def test_e8m0_block_requant_matches_loops():
    g = torch.Generator().manual_seed(6)
    y = torch.randn(5, 256, generator=g, dtype=torch.float64) * torch.tensor(
        [[1e-30], [1e-3], [1.0], [300.0], [1.0]], dtype=torch.float64)
    y[4, 128:] = 0                                  # an all-zero block
    y[2, 5] = 448.0                                 # amax exactly 448 * 2^0
    y[2, 200] = 448.0 * 2 ** -3 * (1 + 2 ** -20)    # just above a power-of-two boundary
    got, codes = orc.e8m0_block_requant(y, 128)
    for r in range(5):
        for b in range(2):
            blk = y[r, 128 * b:128 * b + 128].tolist()
            e = _e8m0_exponent_loop(max(abs(v) for v in blk))
            assert int(codes[r, b]) == e + 127
            ref = [_e4m3_round_loop(v / 2.0 ** e) * 2.0 ** e for v in blk]
            assert got[r, 128 * b:128 * b + 128].tolist() == ref
    assert int(codes[4, 1]) == 0 and int(codes[2, 0]) == 127 and int(codes[2, 1]) == 125


def test_fp8_forward_with_block_requant_matches_scalar_loops():
    w = make_workload(4, seed=7, scale=dict(N=5, H=32, I=128, E=3, k=2))
    got = orc.fp8_forward(w["x_q"], w["x_scale"], w["idx"], w["wt"], w["gate_up_q"],
                          w["gate_up_scale"], w["down_q"], w["down_scale"], dtype=torch.float64)
    xq, xs = w["x_q"].double().tolist(), w["x_scale"].double().tolist()
    gq, gs = w["gate_up_q"].double().tolist(), w["gate_up_scale"].double().tolist()
    dq, ds = w["down_q"].double().tolist(), w["down_scale"].double().tolist()
    idx, wt = w["idx"].tolist(), w["wt"].double().tolist()
    n, h, i = 5, 32, 128
    ref = [[0.0] * h for _ in range(n)]
    for t in range(n):
        for j, e in enumerate(idx[t]):
            gu = [sum(xq[t][c] * gq[e][r][c] for c in range(h)) * xs[t] * gs[e][r]
                  for r in range(2 * i)]
            y = [gu[c] / (1.0 + math.exp(-gu[c])) * gu[i + c] for c in range(i)]
            ex = _e8m0_exponent_loop(max(abs(v) for v in y))   # one 128-channel block
            y = [_e4m3_round_loop(v / 2.0 ** ex) * 2.0 ** ex for v in y]
            for r in range(h):
                ref[t][r] += wt[t][j] * sum(y[c] * dq[e][r][c] for c in range(i)) * ds[e][r]
    torch.testing.assert_close(got, torch.tensor(ref, dtype=torch.float64), rtol=1e-9, atol=1e-9)


def test_e8m0_block_dequantisation_loops():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 96, generator=g) * torch.tensor([[1e-3], [1.0], [40.0]])
    q, s = quant.quantize_mxfp8(x)
    qs, ss = q.float().tolist(), s.tolist()
    ref = [[qs[r][c] * 2.0 ** (ss[r][c // 32] - 127) for c in range(96)] for r in range(3)]
    assert torch.equal(quant.dequantize_mxfp8(q, s).double(), torch.tensor(ref, dtype=torch.float64))


def test_mxfp8_forward_is_moe_forward_on_dequantised_weights():
    w = make_workload(5, scale=dict(N=24, H=64, I=64, E=9, k=3), seed=1)
    f64 = torch.float64
    got = orc.mxfp8_forward(w["hidden"], w["idx"], w["wt"], w["gate_up_q"], w["gate_up_scale"],
                            w["down_q"], w["down_scale"], dtype=f64)
    # weights dequantised by explicit loops over the E8M0 blocks
    def deq(q, s):
        qs, ss = q.double(), s.double()
        out = torch.empty_like(qs)
        for b in range(q.shape[-1] // 32):
            out[..., 32 * b:32 * b + 32] = qs[..., 32 * b:32 * b + 32] * (2.0 ** (ss[..., b:b + 1] - 127))
        return out
    ref = orc.moe_dense(w["hidden"].to(f64), w["idx"], w["wt"].to(f64),
                        deq(w["gate_up_q"], w["gate_up_scale"]), deq(w["down_q"], w["down_scale"]),
                        [0] * 9)
    torch.testing.assert_close(got, ref, rtol=1e-10, atol=1e-10)
    # and the fp32 default agrees with the fp64 pin to fp32 accuracy
    got32 = orc.mxfp8_forward(w["hidden"], w["idx"], w["wt"], w["gate_up_q"], w["gate_up_scale"],
                              w["down_q"], w["down_scale"])
    assert ((got32.double() - ref).norm() / ref.norm()).item() < 1e-6


def test_golden_config1():
    fx = np.load(GOLDEN)
    w = make_workload(1, device="cpu", seed=0)
    np.testing.assert_array_equal(w["idx"].numpy(), fx["idx"])
    d = orc.dispatch_np(w["idx"].numpy(), 8)
    np.testing.assert_array_equal(d["counts"], fx["counts"])
    np.testing.assert_array_equal(d["sorted_flat"], fx["sorted_flat"])
    r = orc.moe_fwd_bwd(w["hidden"], w["idx"], w["wt"], w["gate_up_proj"], w["down_proj"], [0] * 8,
                        w["grad_out"], dtype=torch.float32)
    np.testing.assert_allclose(r["out"][::16].numpy(), fx["out_rows"], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(r["grad_hidden"][::16].numpy(), fx["grad_hidden_rows"], rtol=1e-4,
                               atol=1e-5)
    for name in ("out", "grad_hidden", "grad_wt", "grad_gate_up", "grad_down"):
        assert abs(r[name].double().norm().item() - fx[f"norm_{name}"][0]) <= 1e-4 * fx[f"norm_{name}"][0]


def test_workload_routing_properties():
    for c in CONFIGS:
        small = dict(N=512, H=64, I=64)
        w = make_workload(c, scale=small)
        idx, wt = w["idx"], w["wt"]
        k, e = w["cfg"]["k"], w["cfg"]["E"]
        assert idx.shape == (512, k) and idx.dtype == torch.int64
        assert int(idx.min()) >= 0 and int(idx.max()) < e
        assert torch.all(idx.sort(-1).values.diff(dim=-1) > 0)          # distinct experts per token
        if w["cfg"]["router"] == "stack_softmax":   # the reference bench keeps softmax top-k gates
            assert bool((wt.float().sum(-1) < 1).all()) and bool((wt > 0).all())
        else:
            torch.testing.assert_close(wt.float().sum(-1), torch.ones(512), rtol=1e-2, atol=1e-2)


def test_zipf_config_has_empty_and_full_experts():
    g = torch.Generator().manual_seed(0)
    w = make_workload(3, scale=dict(H=8, I=8))   # full N=16384, E=64, k=8 routing, tiny weights
    counts = torch.bincount(w["idx"].reshape(-1), minlength=64)
    assert int((counts == 0).sum()) >= 1
    assert int(counts.max()) > 12 * int(counts[counts > 0].median())
    del g
