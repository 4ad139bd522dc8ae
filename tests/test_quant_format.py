"""The persisted expert-weight format (kernels.gfx950.quant save_experts / load_experts).

Round trips are bit-exact for both formats; the header's format tag, version and shapes are
checked on load; the file holds exactly what moe_fp8 / moe_mxfp8 read (names, dtypes, layouts).
"""
import json
import struct

import pytest
import torch

from kernels.gfx950 import quant


def _weights(e=3, h=64, i=96, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(e, 2 * i, h, generator=g) / h ** 0.5,
            torch.randn(e, h, i, generator=g) / i ** 0.5)


@pytest.mark.parametrize("fmt", ["fp8", "mxfp8"])
def test_round_trip_is_bit_exact(tmp_path, fmt):
    gu, dw = _weights()
    t = quant.quantize_experts(gu, dw, fmt)
    p = str(tmp_path / f"layer0.{fmt}.safetensors")
    quant.save_experts(p, t, fmt)
    fmt2, t2 = quant.load_experts(p)
    assert fmt2 == fmt
    for k in t:
        assert t2[k].dtype == t[k].dtype and t2[k].shape == t[k].shape, k
        assert torch.equal(t2[k].view(torch.uint8), t[k].contiguous().view(torch.uint8)), k


def test_header_is_plain_json_with_layout_contract(tmp_path):
    gu, dw = _weights(e=2, h=32, i=64)
    p = str(tmp_path / "l.safetensors")
    quant.save_experts(p, quant.quantize_experts(gu, dw, "mxfp8"), "mxfp8")
    raw = open(p, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    hdr = json.loads(raw[8:8 + n])
    assert hdr["__metadata__"] == dict(format="moe-gfx950-mxfp8", version="1", E="2", H="32", I="64")
    assert hdr["gate_up_q"]["dtype"] == "F8_E4M3" and hdr["gate_up_q"]["shape"] == [2, 128, 32]
    assert hdr["gate_up_scale"]["dtype"] == "U8" and hdr["gate_up_scale"]["shape"] == [2, 128, 1]
    assert hdr["down_scale"]["shape"] == [2, 32, 2]


def test_dequantised_weights_reconstruct_the_originals():
    gu, dw = _weights(seed=1)
    f = quant.quantize_experts(gu, dw, "fp8")
    m = quant.quantize_experts(gu, dw, "mxfp8")
    for ref, q, s in ((gu, f["gate_up_q"], f["gate_up_scale"]), (dw, f["down_q"], f["down_scale"])):
        assert ((quant.dequantize_fp8_rows(q, s) - ref).norm() / ref.norm()).item() < 4e-2
    for ref, q, s in ((gu, m["gate_up_q"], m["gate_up_scale"]), (dw, m["down_q"], m["down_scale"])):
        assert ((quant.dequantize_mxfp8(q, s) - ref).norm() / ref.norm()).item() < 4e-2


def test_load_rejects_bad_files(tmp_path):
    from safetensors.torch import save_file
    gu, dw = _weights(e=2, h=32, i=32)
    t = quant.quantize_experts(gu, dw, "fp8")
    p = str(tmp_path / "bad.safetensors")
    save_file({k: v.contiguous() for k, v in t.items()}, p,
              metadata=dict(format="moe-gfx950-fp8", version="2", E="2", H="32", I="32"))
    with pytest.raises(ValueError, match="version"):
        quant.load_experts(p)
    save_file({k: v.contiguous() for k, v in t.items()}, p, metadata=dict(format="other"))
    with pytest.raises(ValueError, match="not a gfx950"):
        quant.load_experts(p)
    save_file({k: v.contiguous() for k, v in t.items()}, p,
              metadata=dict(format="moe-gfx950-fp8", version="1", E="3", H="32", I="32"))
    with pytest.raises(ValueError, match="disagree"):
        quant.load_experts(p)
    bad = dict(t, down_scale=t["down_scale"][:, :5].contiguous())
    with pytest.raises(ValueError, match="scales"):
        quant.save_experts(p, bad, "fp8")
    with pytest.raises(ValueError, match="format"):
        quant.quantize_experts(gu, dw, "int4")
