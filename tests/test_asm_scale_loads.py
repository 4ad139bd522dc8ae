"""Build check of the fp8 down GEMM's block-scale loads (v4::KcLoadS).

Those loads are inline asm, so the compiler inserts no wait for them: their destination registers
must not be read or rewritten on any path before one of the ring's own waits covers them
(s_waitcnt vmcnt(n) with n <= 3 slots of DMAs). This compiles csrc/moe_fp8.hip to gfx950
assembly with the library's flags and follows every control-flow path from each such load.
CPU only (hipcc cross-compiles); skipped when hipcc is absent.
"""
import os
import re
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "triton-kernel-fused_amd"))
import build_lib  # noqa: E402

KERNEL = "_ZN3moe15fp8_gemm_kernelILb0EEEvNS_7Fp8ArgsE"
MAX_COVERING = 12   # the prologue wait leaves three slots of four DMAs in flight


def _regs(text):
    out = {int(m) for m in re.findall(r"\bv(\d+)\b", text)}
    for a, b in re.findall(r"\bv\[(\d+):(\d+)\]", text):
        out.update(range(int(a), int(b) + 1))
    return out


def _check(lines):
    labels = {l.split(":")[0]: i for i, l in enumerate(lines) if re.match(r"^\.LBB\w+:", l)}
    loads = [(i, int(m.group(1))) for i, l in enumerate(lines)
             if (m := re.search(r"global_load_ushort v(\d+),", l))]
    bad = []
    for i0, reg in loads:
        seen, todo = set(), [i0 + 1]
        while todo:
            i = todo.pop()
            while i < len(lines) and i not in seen:
                seen.add(i)
                t = lines[i].split(";")[0].strip()
                w = re.search(r"s_waitcnt vmcnt\((\d+)\)", t)
                if w and int(w.group(1)) <= MAX_COVERING:
                    break
                if t and not t.startswith(".") and reg in _regs(t):
                    bad.append((i0, reg, t))
                if t.startswith("s_endpgm"):
                    break
                m = re.match(r"s_(c?)branch\w*\s+(\.LBB\w+)", t)
                if m:
                    todo.append(labels[m.group(2)])
                    if not m.group(1):
                        break
                i += 1
    return loads, bad


@pytest.mark.skipif(shutil.which(build_lib.HIPCC) is None and not os.path.exists(build_lib.HIPCC),
                    reason="hipcc not available")
def test_scale_load_registers_untouched_until_covered(tmp_path):
    src = os.path.join(build_lib.CSRC, "moe_fp8.hip")
    out = tmp_path / "moe_fp8.s"
    r = subprocess.run([build_lib.HIPCC, *[f for f in build_lib.FLAGS if f != "-fPIC"],
                        "--cuda-device-only", "-S", src, "-o", str(out)],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr
    s = out.read_text()
    body = s[s.index(KERNEL + ":"):]
    body = body[:body.index("s_endpgm") + len("s_endpgm")]
    loads, bad = _check(body.split("\n"))
    assert len(loads) >= 4, "expected the scale loads of the prologue and of the K loop"
    assert not bad, bad[:5]
