"""The int8 ring kernel issues its main MFMAs as inline asm (so the accumulators
stay in place across the K loop), and the compiler does not insert the wait
states an MFMA needs after a VALU write of one of its source VGPRs when that
MFMA is asm.  The kernel places its own s_nop after the VALU writes it makes;
this test checks, on the AMD assembly of this repository's own build, that the
compiler added none of its own (a register copy or a rematerialised constant
right before an asm MFMA gives wrong sums with no error).

Every asm MFMA of gemm_i8.hip (gfx950, the library's flags) is scanned back
over its 8 preceding instructions, stopping at an s_nop; a v_* instruction
other than an MFMA whose destination overlaps the MFMA's sources fails.  The
scan is checked on a planted case: a VALU copy of a source right before an
asm MFMA is found, and an s_nop in between clears it."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RT = os.path.join(ROOT, "simplang_amd", "runtime")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
WINDOW = 8


def _vregs(tok):
    tok = tok.strip().rstrip(",")
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def asm_mfma_hazards(text, window=WINDOW):
    """(number of asm MFMAs, [(function, VALU instruction, MFMA)] hazards)."""
    lines = text.split("\n")
    func, found, n_asm = None, [], 0
    for i, line in enumerate(lines):
        if re.match(r"^_Z\S*:", line):
            func = line.split(":")[0]
        t = line.strip()
        if not (t.startswith("v_mfma") and i > 0 and lines[i - 1].strip() == ";;#ASMSTART"):
            continue
        n_asm += 1
        ops = t.split(None, 1)[1].split(",")
        srcs = set().union(*[_vregs(o) for o in ops[1:]])
        j, seen = i - 2, 0
        while j >= 0 and seen < window:
            u = lines[j].strip()
            j -= 1
            if not u or u.startswith((";", ".")) or u.endswith(":"):
                continue
            seen += 1
            parts = u.split(None, 1)
            if parts[0].startswith("s_nop"):
                break
            if parts[0].startswith("v_") and not parts[0].startswith("v_mfma") and len(parts) > 1:
                if _vregs(parts[1].split(",")[0]) & srcs:
                    found.append((func, u, t))
    return n_asm, found


def test_scanner_finds_a_planted_hazard():
    planted = "\n".join([
        "_Zfoo:",
        "\tv_mov_b64_e32 v[24:25], s[38:39]",
        "\t;;#ASMSTART",
        "\tv_mfma_i32_16x16x64_i8 v[18:21], v[34:37], v[22:25], v[18:21]",
        "\t;;#ASMEND"])
    n, found = asm_mfma_hazards(planted)
    assert n == 1 and len(found) == 1
    cleared = planted.replace("\t;;#ASMSTART", "\ts_nop 7\n\t;;#ASMSTART")
    assert asm_mfma_hazards(cleared)[1] == []
    # a copy into an unrelated register is no hazard
    assert asm_mfma_hazards(planted.replace("v[24:25]", "v[60:61]"))[1] == []


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc absent")
def test_gemm_i8_asm_mfmas_have_no_valu_source_writes(tmp_path):
    out = tmp_path / "gemm_i8.s"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17",
                    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                    "-I" + os.path.join(ROOT, "include"), "-I" + RT,
                    os.path.join(RT, "gemm_i8.hip"), "--cuda-device-only", "-S", "-o", str(out)],
                   check=True, capture_output=True, timeout=600)
    n, found = asm_mfma_hazards(out.read_text())
    assert n > 0
    assert found == [], found[:5]
