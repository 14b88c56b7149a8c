"""The C-ABI library loads and exports every symbol include/fade_hip.h declares (no GPU calls)."""

import ctypes
import os
import re
import subprocess

import pytest

from fade_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fade_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(fade_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_binding_table():
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    assert sorted(_lib.EXPORTED_SYMBOLS) == declared


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} missing: run __graft_entry__.build()")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.fade_hip_abi_version() == 1


def test_ctypes_struct_layout_matches_c(tmp_path):
    """sizeof/offsetof of the argument structs, compiled by gcc from the header."""
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "fade_hip.h"\n'
        "int main(void){printf(\"%zu %zu %zu %zu %zu %zu %zu\\n\", sizeof(fade_fp16_tier), sizeof(fade_mid_tier),"
        " sizeof(fade_decode_args), offsetof(fade_decode_args, sm_scale), offsetof(fade_decode_args, mid),"
        " offsetof(fade_decode_args, n_splits), offsetof(fade_decode_args, workspace_bytes)); return 0;}\n"
    )
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    A = _lib.DecodeArgs
    want = [
        ctypes.sizeof(_lib.Fp16Tier),
        ctypes.sizeof(_lib.MidTier),
        ctypes.sizeof(A),
        A.sm_scale.offset,
        A.mid.offset,
        A.n_splits.offset,
        A.workspace_bytes.offset,
    ]
    assert got == want


def test_prefill_struct_layout_matches_c(tmp_path):
    src = tmp_path / "layout_p.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "fade_hip.h"\n'
        "int main(void){printf(\"%zu %zu %zu %zu %zu %zu\\n\", sizeof(fade_prefill_args),"
        " offsetof(fade_prefill_args, sm_scale), offsetof(fade_prefill_args, lens), offsetof(fade_prefill_args, sink),"
        " offsetof(fade_prefill_args, mid), offsetof(fade_prefill_args, chunk)); return 0;}\n"
    )
    exe = tmp_path / "layout_p"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    A = _lib.PrefillArgs
    assert got == [ctypes.sizeof(A), A.sm_scale.offset, A.lens.offset, A.sink.offset, A.mid.offset, A.chunk.offset]


def test_prefill_argument_errors():
    lib = _lib.load()
    a = _lib.PrefillArgs()
    a.B, a.Hq, a.Hkv, a.D, a.Sq = 2, 36, 4, 128, 16
    assert lib.fade_tiered_prefill_attn(ctypes.byref(a), None) == _lib.FADE_EINVAL
    assert b"Hq/Hkv <= 8" in lib.fade_hip_last_error()
    a.Hq, a.Hkv = 32, 8
    assert lib.fade_tiered_prefill_attn(ctypes.byref(a), None) == _lib.FADE_EINVAL
    assert b"null q, out or lens" in lib.fade_hip_last_error()


def test_argument_errors_come_back_as_value_errors():
    """Validation runs before any GPU work, so it is testable without a device."""
    lib = _lib.load()
    a = _lib.DecodeArgs()
    a.B, a.Hq, a.Hkv, a.D = 1, 32, 8, 96
    rc = lib.fade_tiered_decode_attn(ctypes.byref(a), None)
    assert rc == _lib.FADE_EINVAL
    assert b"head_dim must be 32, 64, 128 or 256" in lib.fade_hip_last_error()
    with pytest.raises(ValueError, match="head_dim"):
        _lib.check(rc, "fade_tiered_decode_attn")
    a.D, a.Hq = 128, 30
    assert lib.fade_tiered_decode_attn(ctypes.byref(a), None) == _lib.FADE_EINVAL
    assert b"not a multiple" in lib.fade_hip_last_error()
    rc = lib.fade_quant_int2_grouped(None, 1, 1, 100, 100, 128, 0, 0, 0, 64, None, None, None)
    assert rc == _lib.FADE_EINVAL and b"must be divisible by group_size" in lib.fade_hip_last_error()
