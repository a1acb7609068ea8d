"""CPU check of the streamed GEMV's untracked x loads in the gfx950 assembly.

k_gemv_sdig loads its activations with inline-assembly global_load_dwordx4
that the compiler does not track (so that its own wait before the first use
would not be a vmcnt(0) over the ring's direct-to-LDS copies as well), then
waits for them with an explicit s_waitcnt vmcnt(n).  The compiler treats the
destination registers as written when the asm statement issues, so any
instruction it places between a load and that wait which reads those
registers reads them before the data lands, and any instruction that writes
them is overwritten when the data lands (an address register reused that
way turns the loaded x into an address).  This test compiles kq_gemv.hip to
gfx950 assembly with the library's own flags and checks, for every such
load, that nothing between it and the next vmcnt wait names its registers.
"""
import re
import shutil
import subprocess

import pytest

from inferno_hip import build


def _vregs(token):
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", token)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", token)
    return {int(m.group(1))} if m else set()


def _operands(line):
    parts = line.split(None, 1)
    regs = set()
    for tok in re.findall(r"v\[\d+:\d+\]|v\d+\b", parts[1] if len(parts) > 1 else ""):
        regs |= _vregs(tok)
    return regs


def untracked_load_hazards(asm_lines):
    """(loads checked, [(kernel, line number, text)]) for the assembly of one
    translation unit."""
    kernel, checked, found = "", 0, []
    for i, line in enumerate(asm_lines):
        m = re.match(r"^(_Z\S+):", line)
        if m:
            kernel = m.group(1)
        if ("global_load_dwordx4" not in line or "lds" in line or i == 0
                or "ASMSTART" not in asm_lines[i - 1]):
            continue
        dst = _vregs(line.split()[1].rstrip(","))
        checked += 1
        for j in range(i + 1, len(asm_lines)):
            t = asm_lines[j].strip()
            if (re.search(r"s_waitcnt\s+vmcnt", t) or t.startswith("_Z") or "s_endpgm" in t):
                break
            if not t or t.startswith((";", ".")) or "global_load_dwordx4" in t:
                continue
            if _operands(t) & dst:
                found.append((kernel, j + 1, t))
    return checked, found


def test_checker_flags_a_reused_destination():
    # the pattern the check exists for: a copy of an in-flight destination
    # and a write of a register the load will still fill
    bad = [
        "_Zk:",
        "\t;;#ASMSTART",
        "\tglobal_load_dwordx4 v[2:5], v[6:7], off",
        "\t;;#ASMEND",
        "\tv_mov_b64_e32 v[98:99], v[2:3]",
        "\tv_lshl_add_u64 v[4:5], s[6:7], 0, v[8:9]",
        "\ts_waitcnt vmcnt(2)",
        "\tv_add_f32_e32 v10, v2, v3",
    ]
    checked, found = untracked_load_hazards(bad)
    assert checked == 1 and [f[1] for f in found] == [5, 6]
    good = bad[:4] + ["\tglobal_load_lds_dwordx4 v40, s[4:5]", "\ts_waitcnt vmcnt(2)", bad[7]]
    assert untracked_load_hazards(good) == (1, [])


@pytest.mark.skipif(shutil.which(build.HIPCC) is None and not build.Path(build.HIPCC).exists(),
                    reason="hipcc not available")
def test_streamed_gemv_untracked_loads_are_waited_before_use(tmp_path):
    out = tmp_path / "kq_gemv.s"
    flags = [f for f in build.FLAGS if f not in ("-shared", "-fPIC")]
    cmd = [build.HIPCC, *flags, f"-I{build.INCLUDE}", f"-I{build.CSRC}", "--cuda-device-only", "-S",
           "-o", str(out), str(build.CSRC / "kq_gemv.hip")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    checked, found = untracked_load_hazards(out.read_text().split("\n"))
    assert checked > 0, "no untracked x loads found: the check no longer sees the kernel's loads"
    assert not found, f"{len(found)} instructions touch in-flight registers, first: {found[:3]}"
