"""The rotated decode's prologue loads R with loads the compiler does not track.

``decode_packed_kernel<..., ROT=true>`` issues this wave's R rows with
inline-asm ``global_load_dwordx4`` ahead of the first two tile loads, waits for
them with its own ``s_waitcnt`` (which also covers the query), and only then
reads the registers, behind an empty asm that redefines them.  That is sound
only if the compiled code neither reads nor moves those registers between the
loads and that point.  This test compiles the kernel to gfx950 assembly and
checks exactly that for every rotated instance (CPU only: hipcc cross-compiles).
"""

import os
import re
import subprocess

import pytest

HIPCC = "/opt/rocm/bin/hipcc"
CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "fade_amd", "csrc")

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="needs hipcc")

_LOAD = re.compile(r"global_load_dwordx4 v\[(\d+):(\d+)\], v\[\d+:\d+\], off$")


def _regs(line: str) -> set[int]:
    out = set()
    for m in re.finditer(r"v\[(\d+):(\d+)\]", line):
        out |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"(?<![\w\[:])v(\d+)\b", line):
        out.add(int(m.group(1)))
    return out


@pytest.mark.parametrize("source", ["decode_int4.hip", "decode_int4_bf16.hip"])  # fp16 and bf16 instances
def test_rotated_prologue_registers_untouched_until_the_wait(tmp_path, source):
    out = tmp_path / (source[:-4] + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "--cuda-device-only", "-S", "-O3", "-std=c++17",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-fast-math", "-Wno-inline-asm",
           "-I", CSRC, os.path.join(CSRC, source), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    lines = out.read_text().split("\n")
    starts = [i for i, l in enumerate(lines)
              if re.match(r"^_ZN4fade6decode12_GLOBAL__N_120decode_packed_kernelIL.*Lb1ELi\d+EEEvNS0_6ParamsE:", l)
              and "ELi0ELi" in l]
    assert len(starts) == 8, "expected the 8 rotated instances (4/2-bit x DET x two passes)"
    for s in starts:
        body = lines[s : s + 4000]
        loads = [i for i, l in enumerate(body[:1000]) if _LOAD.search(l.strip())]
        assert loads, f"no untracked R loads in {lines[s][:100]}"
        regs = set()
        for i in loads:
            m = _LOAD.search(body[i].strip())
            regs |= set(range(int(m.group(1)), int(m.group(2)) + 1))
        last = max(loads)
        # the register laundering: the first empty inline-asm block after the loads
        lau = next(i for i in range(last + 1, len(body) - 1)
                   if body[i].strip() == ";;#ASMSTART" and body[i + 1].strip() == ";;#ASMEND")
        assert any("s_waitcnt vmcnt" in body[i] for i in range(last + 1, lau)), "no wait before the registers are used"
        early = [body[i].strip() for i in range(last + 1, lau)
                 if not body[i].strip().startswith(";") and _regs(body[i]) & regs]
        assert not early, f"R registers touched before the wait in {lines[s][:100]}: {early[:3]}"
