"""The C-ABI library loads and exports every symbol include/fade_hip.h declares (no GPU calls)."""

import ctypes
import os
import re
import struct
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
    assert lib.fade_hip_abi_version() == 2


def _elf_sections(data: bytes):
    """{name: (offset, size, link)} of an ELF64 little-endian image."""
    shoff = struct.unpack_from("<Q", data, 0x28)[0]
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", data, 0x3A)
    hdrs = [struct.unpack_from("<IIQQQQIIQQ", data, shoff + i * shentsize) for i in range(shnum)]
    stro = hdrs[shstrndx][4]
    out = {}
    for h in hdrs:
        name = data[stro + h[0] : data.index(b"\0", stro + h[0])].decode()
        out[name] = (h[4], h[5], h[6], hdrs)
    return out


def _elf_symbols(data: bytes) -> set[str]:
    secs = _elf_sections(data)
    off, size, link, hdrs = secs[".symtab"]
    stroff = hdrs[link][4]
    names = set()
    for i in range(size // 24):
        st_name = struct.unpack_from("<I", data, off + 24 * i)[0]
        if st_name:
            names.add(data[stroff + st_name : data.index(b"\0", stroff + st_name)].decode())
    return names


def _device_symbols(lib: bytes) -> set[str]:
    """Symbols of every gfx950 code object in the library's offload bundles."""
    off, size, _, _ = _elf_sections(lib)[".hip_fatbin"]
    fat = lib[off : off + size]
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    names: set[str] = set()
    starts = [m.start() for m in re.finditer(re.escape(magic), fat)]
    assert starts, "no offload bundle in .hip_fatbin"
    for b in starts:
        (n,) = struct.unpack_from("<Q", fat, b + len(magic))
        p = b + len(magic) + 8
        for _ in range(n):
            eoff, esize, tlen = struct.unpack_from("<QQQ", fat, p)
            triple = fat[p + 24 : p + 24 + tlen].decode()
            p += 24 + tlen
            if "gfx950" in triple:
                names |= _elf_symbols(fat[b + eoff : b + eoff + esize])
    return names


def test_every_launched_kernel_is_in_the_code_object():
    """Each kernel the host side launches (one ``__device_stub__`` per kernel)
    names a symbol of the gfx950 code object.  A kernel whose signature the
    host and device passes mangle differently (e.g. an expression over an
    unnamed enum) builds and links, then aborts at its first launch."""
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} missing: run __graft_entry__.build()")
    lib = open(_lib.LIB_PATH, "rb").read()
    host = _elf_symbols(lib)
    stub = re.compile(r"(\d+)__device_stub__")
    kernels = set()
    for name in host:
        m = stub.search(name)
        if m:  # mangled: <len>__device_stub__<id> -> <len-15><id>
            kernels.add(name[: m.start()] + str(int(m.group(1)) - 15) + name[m.end() :])
        elif name.startswith("__device_stub__"):
            kernels.add(name[len("__device_stub__") :])
    assert len(kernels) > 50
    missing = sorted(kernels - _device_symbols(lib))
    assert not missing, f"{len(missing)} launched kernels absent from the code object: {missing[:3]}"


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
    a.D = 264
    assert lib.fade_tiered_prefill_attn(ctypes.byref(a), None) == _lib.FADE_EINVAL
    assert b"head_dim must be a multiple of 8 in [8, 256]" in lib.fade_hip_last_error()
    a.D = 256  # taken: the next check is the pointers
    assert lib.fade_tiered_prefill_attn(ctypes.byref(a), None) == _lib.FADE_EINVAL
    assert b"null q, out or lens" in lib.fade_hip_last_error()


def test_argument_errors_come_back_as_value_errors():
    """Validation runs before any GPU work, so it is testable without a device."""
    lib = _lib.load()
    a = _lib.DecodeArgs()
    a.B, a.Hq, a.Hkv, a.D = 1, 32, 8, 100
    rc = lib.fade_tiered_decode_attn(ctypes.byref(a), None)
    assert rc == _lib.FADE_EINVAL
    assert b"head_dim must be a multiple of 8 in [8, 256]" in lib.fade_hip_last_error()
    with pytest.raises(ValueError, match="head_dim"):
        _lib.check(rc, "fade_tiered_decode_attn")
    a.D, a.Hq = 128, 30
    assert lib.fade_tiered_decode_attn(ctypes.byref(a), None) == _lib.FADE_EINVAL
    assert b"not a multiple" in lib.fade_hip_last_error()
    rc = lib.fade_quant_int2_grouped(None, 1, 1, 100, 100, 128, 0, 0, 0, 64, None, None, None)
    assert rc == _lib.FADE_EINVAL and b"must be divisible by group_size" in lib.fade_hip_last_error()
