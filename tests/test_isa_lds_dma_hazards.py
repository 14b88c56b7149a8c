"""Every LDS DMA in the built kernels respects the two GFX9-family issue hazards
that the hardware does not interlock and that the compiler cannot see inside
inline asm:

- an SALU write of m0 needs one wait state before an LDS DMA reads m0 (else
  the DMA may take the previous base and land in the previous load's slot);
- a VALU write of an SGPR (``v_readfirstlane_b32``) needs five wait states
  before a VMEM instruction reads it as its scalar base.

For its own LDS DMAs the compiler inserts ``s_nop`` for both on gfx950; the
kernels' DMAs are inline asm (``fade_amd/csrc/lds_dma.h``), so this test
compiles every source that issues them to gfx950 assembly and scans each
``global_load_lds_*`` backwards over its straight-line predecessors (CPU only:
hipcc cross-compiles).
"""

import os
import re
import subprocess

import pytest

HIPCC = "/opt/rocm/bin/hipcc"
CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "fade_amd", "csrc")
SOURCES = ("decode_int4.hip", "decode_int4_bf16.hip", "decode_mfma.hip", "prefill.hip")
FLAGS = ["--offload-arch=gfx950", "--cuda-device-only", "-S", "-O3", "-std=c++17", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-fast-math",
         "-Wno-inline-asm", "-I", CSRC]

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="needs hipcc")


def _sregs(text: str) -> set[int]:
    out = set()
    for m in re.finditer(r"\bs\[(\d+):(\d+)\]", text):
        out |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"(?<![\w\[:])s(\d+)\b", text):
        out.add(int(m.group(1)))
    return out


def hazards(asm: str) -> tuple[int, list[str]]:
    """(LDS DMAs seen, descriptions of the hazards among them)."""
    items = []  # ("L", label) or ("I", instruction)
    for line in asm.split("\n"):
        s = line.split(";")[0].strip()
        if not s or s.startswith("."):
            continue
        items.append(("L", s) if s.endswith(":") else ("I", s))
    found, bad = 0, []
    for i, (kind, ins) in enumerate(items):
        if kind != "I" or not ins.startswith("global_load_lds"):
            continue
        found += 1
        ops = ins.split(None, 1)[1].split(",")
        sbase = _sregs(ops[1]) if len(ops) > 1 and ops[1].strip() != "off" else set()
        waits, m0_done = 0, False
        for kind2, prev in reversed(items[:i]):
            if kind2 == "L" or waits >= 5:
                break  # a branch target or enough wait states: nothing earlier can reach
            op = prev.split()[0]
            dst = prev.split(None, 1)[1].split(",")[0].strip() if " " in prev else ""
            if not m0_done and op.startswith("s_") and dst == "m0":
                m0_done = True
                if waits < 1:
                    bad.append(f"m0 written right before `{ins}`")
            if op.startswith("v_") and sbase and _sregs(dst) & sbase:
                bad.append(f"`{prev}` {waits} wait states before `{ins}`")
                break
            waits += int(prev.split()[1]) + 1 if op == "s_nop" else 1
    return found, bad


def test_scanner_flags_the_unsafe_forms():
    unsafe = "\n".join([
        "v_readfirstlane_b32 s2, v2",
        "s_mov_b32 m0, s4",
        "global_load_lds_dwordx4 v1, s[2:3]",
    ])
    n, bad = hazards(unsafe)
    assert n == 1 and len(bad) == 2
    safe = "\n".join([
        "v_readfirstlane_b32 s2, v2",
        "s_mov_b32 m0, s4",
        "s_nop 3",
        "global_load_lds_dwordx4 v1, s[2:3]",
        "s_mov_b32 m0, s5",
        "s_nop 0",
        "global_load_lds_dwordx4 v[4:5], off",
    ])
    assert hazards(safe) == (2, [])


@pytest.mark.parametrize("src", SOURCES)
def test_lds_dma_hazard_free(tmp_path, src):
    out = tmp_path / (src + ".s")
    subprocess.run([HIPCC, *FLAGS, os.path.join(CSRC, src), "-o", str(out)], check=True, capture_output=True,
                   timeout=900)
    n, bad = hazards(out.read_text())
    assert n > 0, f"no LDS DMA found in {src}"
    assert not bad, f"{len(bad)} of {n} LDS DMAs in {src} break an issue hazard, e.g. {bad[:3]}"
