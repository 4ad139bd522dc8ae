"""CPU checks of the C-ABI library and the host-side Python layer (no GPU compute)."""
import ctypes
import os
import re

import pytest
import torch

from kernels import _lib
import kernels
import importlib
moe_mod = importlib.import_module("kernels.gfx950.moe")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "moe_gfx950.h")


def _header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    h = _lib.lib()
    declared = _header_symbols()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(h, name), name
    assert set(declared) == set(_lib.declared_symbols())


def test_version_and_tile_rows():
    assert _lib.lib().moe_version().startswith(b"moe_gfx950")
    assert _lib.lib().moe_tile_rows() == 128


def test_workspace_size():
    ws = _lib.lib().moe_get_workspace_size
    assert ws(16384, 8, 64) >= (131072 // 4096) * 64 * 4
    assert ws(0, 2, 8) > 0
    assert ws(-1, 2, 8) == 0


# Argument validation happens on the host before any HIP call, so these run without a GPU.
def test_dispatch_rejects_bad_arguments():
    h = _lib.lib()
    nul = [None] * 8
    assert h.moe_dispatch(None, 4, 2, 0, *nul, None, 0, None) == 1
    assert h.moe_dispatch(None, 4, 2, 2000, *nul, None, 0, None) == 1
    fake = ctypes.c_void_p(16)
    assert h.moe_dispatch(fake, 4, 2, 8, *([fake] * 8), None, 0, None) == 6


def test_gemm_entry_points_reject_bad_arguments():
    h = _lib.lib()
    fake = 256
    # dtype
    assert h.moe_grouped_down_fwd(7, fake, fake, 4, 64, 64, fake, None, 10, fake, None, 0, None) == 4
    # H not a multiple of 8
    assert h.moe_grouped_down_fwd(2, fake, fake, 4, 60, 64, fake, None, 10, fake, None, 0, None) == 2
    # misaligned pointer
    assert h.moe_grouped_down_fwd(2, fake + 2, fake, 4, 64, 64, fake, None, 10, fake, None, 0, None) == 2
    # no experts
    assert h.moe_grouped_down_fwd(2, fake, fake, 0, 64, 64, fake, None, 10, fake, None, 0, None) == 1
    # zero rows is a no-op success
    assert h.moe_grouped_down_fwd(2, fake, fake, 4, 64, 64, fake, None, 0, fake, None, 0, None) == 0
    assert h.moe_grouped_wgrad(2, fake, 64, None, fake, 60, None, 64, 60, fake, None, 4, 4, fake, None, 0, None) == 2
    assert h.moe_grouped_wgrad(2, fake, 64, None, fake, 64, None, 64, 64, fake, fake, 3, 4, fake, None, 0, None) == 1
    assert h.moe_combine_fwd(2, fake, fake, fake, fake, fake, 4, 5, fake, 10, 2, 64, 0, fake, None) == 1
    assert h.moe_glu_fwd(2, fake, 10, fake, fake, None, 1, 4, 8, fake, 8, None) == 1
    # gate-weighted intermediate: 16-bit only, H % 64 == 0, inter_out required
    gu = [2, fake, 10, 64, fake, 4, 64, fake, fake, None, fake, 20, fake]
    assert h.moe_grouped_gateup_swiglu_fwd(0, *gu[1:], fake, fake, None, None) == 1  # fp32
    assert h.moe_grouped_gateup_swiglu_fwd(*gu, None, fake, None, None) == 1  # no inter_out
    gu96 = [2, fake, 10, 96, fake, 4, 64, fake, fake, None, fake, 20, fake]
    assert h.moe_grouped_gateup_swiglu_fwd(*gu96, fake, fake, None, None) == 1  # H % 64 != 0


def test_call_maps_status_to_exceptions():
    with pytest.raises(TypeError):
        _lib.call("moe_grouped_down_fwd", 9, 16, 16, 4, 64, 64, 16, None, 10, 16, None, 0, None)
    with pytest.raises(ValueError):
        _lib.call("moe_grouped_down_fwd", 2, 18, 16, 4, 64, 64, 16, None, 10, 16, None, 0, None)


def test_host_tensors_fail_loudly():
    x = torch.randn(8, 16)
    idx = torch.zeros(8, 2, dtype=torch.long)
    w = torch.ones(8, 2) / 2
    gu = torch.randn(2, 16, 16)
    dw = torch.randn(2, 16, 8)
    codes = torch.zeros(2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="device"):
        kernels.moe(x, idx, w, gu, dw, codes)


def test_code_order_validation():
    with pytest.raises(ValueError):
        moe_mod._check_codes((0, 3, 0), 3)
    with pytest.raises(ValueError):
        moe_mod._check_codes((0, 0, 1), 2)
    moe_mod._check_codes((0, 1, 2, 5, 6, 7, 3, 4), 6)


def test_grouped_rejects_situ_like_reference():
    codes = torch.tensor([0, 5], dtype=torch.int32)
    with pytest.raises(ValueError, match="code 5"):
        kernels.moe_grouped(torch.zeros(1, 8), torch.zeros(1, 1, dtype=torch.long),
                            torch.ones(1, 1), torch.zeros(2, 16, 8), torch.zeros(2, 8, 8), codes)
    with pytest.raises(ValueError, match="code 5"):
        kernels.moe_grouped_cublas_polyglu(torch.zeros(1, 8), torch.zeros(1, 1, dtype=torch.long),
                                           torch.ones(1, 1), torch.zeros(2, 16, 8),
                                           torch.zeros(2, 8, 8), codes)


def test_batched_glu_half_specified_params():
    with pytest.raises(ValueError):
        kernels.BatchedGLU.apply(torch.zeros(2, 8), torch.zeros(2, dtype=torch.int32),
                                 torch.ones(2), None)


def test_import_aliases():
    from kernels.sm75 import moe as m75
    from kernels.sm120 import moe as m120
    from kernels.sm120.moe_grouped import grouped_supported, prefer_grouped
    from kernels.sm75.moe import moe_eager
    assert callable(m75) and callable(m120) and callable(moe_eager)
    assert not grouped_supported(torch.zeros(2, 8), torch.zeros(1, 16, 8), torch.zeros(1, 8, 8))
    assert prefer_grouped(torch.zeros(4, 2), torch.zeros(8, 2, 2))


def test_moe_eager_matches_oracle_on_cpu():
    # the API's eager reference (pure PyTorch) agrees with the oracle restatement
    from oracle import moe_oracle as orc
    g = torch.Generator().manual_seed(0)
    codes = [0, 1, 2, 5, 3, 4]
    x = torch.randn(40, 16, generator=g)
    gu = torch.randn(4, 32, 16, generator=g) * 0.3
    dw = torch.randn(4, 16, 16, generator=g) * 0.3
    idx = torch.rand(40, 6, generator=g).topk(2, -1).indices
    wt = torch.rand(40, 2, generator=g)
    ap = torch.rand(6, 2, generator=g) + 0.5
    a = kernels.moe_eager(x, idx, wt, gu, dw, torch.tensor(codes, dtype=torch.int32), ap)
    b = orc.moe_forward(x, idx, wt, gu, dw, codes, ap)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


def test_row_expert_with_dropped_ids():
    """Per-sorted-row expert ids from the dispatch offsets when out-of-range ids leave fewer routed
    rows than N*k: rows past offsets[E] get E (no expert), the per-row gathers clamp it and the
    SiTU-parameter scatter masks it."""
    from kernels.gfx950.moe import _Routing, _row_params
    # routing [[0, 2], [-1, 2], [2, 5], [1, 0]] over 4 experts: ids -1 and 5 are dropped
    n_exp = 4
    offsets = torch.tensor([0, 2, 3, 6, 6], dtype=torch.int32)   # counts 2, 1, 3, 0
    r = _Routing.__new__(_Routing)
    r.offsets = offsets
    rexp = r.row_expert(n_exp, 8)
    assert rexp.tolist() == [0, 0, 1, 2, 2, 2, 4, 4]
    codes_t = torch.tensor([5, 2, 5, 3], dtype=torch.int32)
    ap = torch.tensor([[2.0, 3.0], [4.0, 5.0], [6.0, 7.0], [8.0, 9.0]])
    row_act, ra, rg, rexp2 = _row_params(r, codes_t, ap, n_exp, 8)
    assert row_act.tolist() == [5, 5, 2, 5, 5, 5, 3, 3]
    assert ra.tolist() == [2, 2, 4, 6, 6, 6, 8, 8] and rg.tolist() == [3, 3, 5, 7, 7, 7, 9, 9]
    valid = rexp2 < min(ap.shape[0], n_exp)
    assert valid.tolist() == [True] * 6 + [False] * 2


def _header_params():
    """name -> list of C parameter types, parsed from the declarations in the header."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|size_t|int64_t|const char\*)\s+(moe_[a-z0-9_]+)\s*\(([^)]*)\)\s*;",
                         text):
        args = [a.strip() for a in m.group(2).replace("\n", " ").split(",") if a.strip()]
        if args == ["void"]:
            args = []
        out[m.group(1)] = [re.sub(r"\s*\b\w+$", "", a).replace(" ", "") for a in args]
    return out


def test_binding_argtypes_match_the_header():
    """Every ctypes argtype list in kernels/_lib.py has the header's parameter count, and each
    pointer / 32-bit / 64-bit / size_t / float parameter maps to the matching ctypes type."""
    import ctypes
    decl = _header_params()
    assert set(decl) == set(_lib.declared_symbols())
    kind = {ctypes.c_void_p: "p", ctypes.c_int: "i32", ctypes.c_int64: "i64", ctypes.c_size_t: "sz",
            ctypes.c_float: "f32"}
    for name, params in decl.items():
        argtypes = _lib._SIGS[name]
        assert len(argtypes) == len(params), (name, params, argtypes)
        for c, a in zip(params, argtypes):
            want = ("p" if "*" in c else "i32" if c in ("int", "unsignedint") else
                    "i64" if c == "int64_t" else "sz" if c == "size_t" else "f32" if c == "float"
                    else c)
            assert kind[a] == want, (name, c, a)
