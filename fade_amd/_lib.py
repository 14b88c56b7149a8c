"""ctypes binding of ``libfade_hip.so`` (the C ABI declared in ``include/fade_hip.h``).

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch already mapped (one runtime per process).  There is no CPU
fallback: every op in this package raises when the library is missing or
when it is handed a CPU tensor.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# FADE_HIP_LIB points at an alternative build of the same library (e.g. an
# installed copy); the default is the in-tree build.
LIB_PATH = os.environ.get("FADE_HIP_LIB") or os.path.join(_HERE, "libfade_hip.so")

FADE_OK = 0
FADE_ERUNTIME = -1
FADE_EINVAL = -22

AXIS_CHANNEL = 0
AXIS_TOKEN = 1

MID_NONE = 0
MID_FP16 = 1
MID_SYM = 2
MID_K4V2G = 3
MID_ASYM = 4

MASK_BOTTOM_RIGHT = 0
MASK_TOP_LEFT = 1
MASK_NONE = 2

_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_p = ctypes.c_void_p
_pi64 = ctypes.POINTER(ctypes.c_int64)


class Fp16Tier(ctypes.Structure):
    _fields_ = [
        ("k", _p),
        ("v", _p),
        ("len", _i64),
        ("k_sb", _i64),
        ("k_sh", _i64),
        ("k_ss", _i64),
        ("v_sb", _i64),
        ("v_sh", _i64),
        ("v_ss", _i64),
    ]


class MidTier(ctypes.Structure):
    _fields_ = [
        ("fmt", _i32),
        ("k_bits", _i32),
        ("v_bits", _i32),
        ("group", _i32),
        ("len", _i64),
        ("v_rows", _i64),
        ("k_codes", _p),
        ("k_scale", _p),
        ("k_zero", _p),
        ("v_codes", _p),
        ("v_scale", _p),
        ("v_zero", _p),
        ("pages", _p),
        ("pages_per_row", _i64),
        ("page_stride", _i64),
    ]


# FADE_ABI_VERSION of include/fade_hip.h that DecodeArgs / PrefillArgs mirror
ABI_VERSION = 2


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("B", _i64),
        ("Hq", _i64),
        ("Hkv", _i64),
        ("D", _i64),
        ("q", _p),
        ("q_sb", _i64),
        ("q_sh", _i64),
        ("out", _p),
        ("o_sb", _i64),
        ("o_sh", _i64),
        ("sm_scale", ctypes.c_float),
        ("sink", Fp16Tier),
        ("mid", MidTier),
        ("recent", Fp16Tier),
        ("n_splits", _i32),
        ("kernel", _i32),
        ("workspace", _p),
        ("workspace_bytes", _i64),
        ("lens", _p),
        ("deterministic", _i32),
        ("rotation", _p),
        ("dtype", _i32),
    ]


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("B", _i64),
        ("Hq", _i64),
        ("Hkv", _i64),
        ("D", _i64),
        ("Sq", _i64),
        ("q", _p),
        ("q_sb", _i64),
        ("q_sh", _i64),
        ("q_ss", _i64),
        ("out", _p),
        ("o_sb", _i64),
        ("o_sh", _i64),
        ("o_ss", _i64),
        ("sm_scale", ctypes.c_float),
        ("lens", _p),
        ("order", _p),
        ("sink", Fp16Tier),
        ("mid", MidTier),
        ("recent", Fp16Tier),
        ("chunk", Fp16Tier),
        ("mask_mode", _i32),
        ("dtype", _i32),
    ]


class ReassignArgs(ctypes.Structure):
    """``FadeReassignArgs`` of include/fade_hip.h."""

    _fields_ = [
        ("B", _i64), ("H", _i64), ("D", _i64), ("S", _i64),
        ("n_sink_old", _i64), ("n_mid_old", _i64),
        ("src_lens", _p), ("plan_rows", _i64), ("pos_old_rs", _i64), ("n_rec_cap", _i64),
        ("sink_k", _p), ("sink_v", _p), ("sink_sb", _i64), ("sink_sh", _i64), ("sink_ss", _i64),
        ("mid_kq", _p), ("mid_ks", _p), ("mid_vq", _p), ("mid_vs", _p),
        ("rec_k", _p), ("rec_v", _p), ("rec_sb", _i64), ("rec_sh", _i64), ("rec_ss", _i64),
        ("dst", _p), ("newpos", _p), ("src_of", _p), ("rows", _i64), ("counts", _p), ("pos_old", _p),
        ("cos_tab", _p), ("sin_tab", _p), ("table_rows", _i64),
        ("out_sink_k", _p), ("out_sink_v", _p), ("cap_sink", _i64),
        ("out_rec_k", _p), ("out_rec_v", _p), ("out_rec_sb", _i64), ("out_rec_sh", _i64), ("out_rec_ss", _i64),
        ("cap_rec", _i64),
        ("out_mid_k", _p), ("out_mid_v", _p), ("cap_mid", _i64),
        ("mid_colmax", _p), ("colmax_parts", _i64),
    ]


# name -> argtypes; every function returns int (status) unless listed in _RESTYPES.
_SIGNATURES: dict[str, list] = {
    "fade_hip_abi_version": [],
    "fade_hip_last_error": [],
    "fade_pack_codes": [_p, _i64, _i64, _i32, _p, _p],
    "fade_unpack_codes": [_p, _i64, _i64, _i32, _p, _p],
    "fade_quant_k_int4_workspace_bytes": [_i64, _i64, _i64, _i64, _pi64],
    "fade_quant_k_int4": [_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _p],
    "fade_quant_k_int4_from_colmax": [_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p, _p, _p],
    "fade_quant_v_int4": [_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p],
    "fade_dequant_sym": [_p, _p, _i32, _i32, _i64, _i64, _i64, _i64, _p, _p],
    "fade_quant_rotated_dtype": [_p, _i64, _i64, _i64, _i64, _i32, _i32, _p, _p, _i32, _p, _i64, _p],
    "fade_quant_k_int4_dtype": [_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _i64, _p],
    "fade_quant_v_int4_dtype": [_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p],
    "fade_dequant_sym_dtype": [_p, _p, _i32, _i32, _i32, _i64, _i64, _i64, _i64, _p, _p],
    "fade_quant_int2_grouped": [_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p],
    "fade_dequant_int2_grouped": [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p],
    "fade_quant_int2_grouped_dtype": [_p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p],
    "fade_dequant_int2_grouped_dtype": [_p, _p, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p],
    "fade_quant_rotated_workspace_bytes": [_i64, _i64, _i64, _i64, _i32, _pi64],
    "fade_quant_rotated": [_p, _i64, _i64, _i64, _i64, _i32, _i32, _p, _p, _p, _i64, _p],
    "fade_rotate_quant_workspace_bytes": [_i64, _i64, _i64, _i64, _i32, _pi64],
    "fade_rotate_quant": [_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i32, _i32, _p, _p, _p, _i64, _p],
    "fade_quant_asym": [_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _p, _p, _p, _p],
    "fade_dequant_asym": [_p, _p, _p, _i32, _i32, _i64, _i64, _i64, _i64, _p, _p],
    "fade_rerope_gather": [
        _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        _p, _i64, _p, _p, _p, _p, _p, _p, _p,
    ],
    "fade_rerope_gather_dtype": [
        _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
        _p, _i64, _p, _p, _p, _p, _p, _p, _i32, _p,
    ],
    "fade_tiered_decode_workspace_bytes": [ctypes.POINTER(DecodeArgs), _pi64],
    "fade_tiered_decode_attn": [ctypes.POINTER(DecodeArgs), _p],
    "fade_tiered_decode_attn_noalloc": [ctypes.POINTER(DecodeArgs), _p],
    "fade_reassign_plan": [_p, _i64, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _p],
    "fade_reassign_gather": [ctypes.POINTER(ReassignArgs), _p],
    "fade_tiered_prefill_attn": [ctypes.POINTER(PrefillArgs), _p],
}
_RESTYPES = {"fade_hip_last_error": ctypes.c_char_p}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def library_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"fade_amd: HIP library not found at {LIB_PATH}; build it with "
                    "`python -c 'import __graft_entry__ as g; g.build()'` or "
                    "`make -C fade_amd/csrc`"
                )
            lib = ctypes.CDLL(LIB_PATH)
            for name, argtypes in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            if lib.fade_hip_abi_version() != ABI_VERSION:  # the argument structs below match this version only
                raise RuntimeError(
                    f"fade_amd: {LIB_PATH} has ABI version {lib.fade_hip_abi_version()}, this package needs "
                    f"{ABI_VERSION}; rebuild it (`make -C fade_amd/csrc`)"
                )
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc == FADE_OK:
        return
    msg = load().fade_hip_last_error()
    msg = msg.decode() if msg else what
    if rc == FADE_EINVAL:
        raise ValueError(msg)
    raise RuntimeError(f"{what}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream_handle(device: torch.device) -> int:
    """The current stream of ``device`` as a raw handle (the fast accessor when torch has it)."""
    if _RAW_STREAM is not None:
        return int(_RAW_STREAM(device.index if device.index is not None else torch.cuda.current_device()))
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors: torch.Tensor | None, op: str = "fade_amd") -> None:
    """Reject CPU tensors: the hot path has no CPU implementation."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                f"{op}: the MI355X kernels need GPU tensors (got a tensor on {t.device}); "
                "fade_amd has no CPU fallback"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{op}: tensors are on different devices ({dev} vs {t.device})")


# FADE_DTYPE_* of the dtype-tagged quantizer entry points
DTYPE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def require_f16(t: torch.Tensor, op: str) -> None:
    if t.dtype != torch.float16:
        raise ValueError(f"{op}: expected a float16 tensor, got {t.dtype}")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Scratch for one kernel family; zero-filled (the decode split counters start at zero)."""
    return torch.zeros(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def scratch(nbytes: int, device: torch.device) -> torch.Tensor:
    """Uninitialized scratch, for kernels that write every byte of it they read."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


_STREAM_WS: dict = {}  # (device, stream, counter slots) -> the current zero-filled buffer
_STREAM_WS_OUTGROWN: list = []  # replaced buffers, kept alive for graphs that captured them


def stream_workspace(nbytes: int, device: torch.device, stream: int, pairs: int) -> torch.Tensor:
    """Zero-filled decode workspace shared by the calls on one stream.

    The decode workspace holds the split counters in its first
    round256(4 * pairs) bytes (pairs = B * Hkv * ceil((Hq / Hkv) / 4), one per
    kv pair and head pass) and the partial results right after them.  Every
    call leaves its counters at zero, so calls with the same ``pairs`` can
    share one buffer whatever their other sizes: their partials never reach
    the counter region.  Calls with another ``pairs`` get another
    buffer (their partials could land where these counters sit).  Calls on one
    stream run in order; different streams get different buffers.  A buffer
    too small for a call is replaced by a zero-filled one of at least twice
    its size; the old one is kept for the life of the process, as every buffer
    is (a graph that captured one keeps a valid address).  The zero fill runs on
    ``stream`` itself, so the first kernel on that stream sees it done; a buffer
    is never created or grown while a HIP graph is being captured (the fill
    would only be recorded in the graph): run the same call once before
    capturing.
    """
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, int(stream), int(pairs))
    need = max(int(nbytes), 1)
    ws = _STREAM_WS.get(key)
    if ws is None or ws.numel() < need:
        target = torch.cuda.ExternalStream(int(stream), device=torch.device("cuda", idx))
        with torch.cuda.stream(target):
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(
                    "tiered decode: its shared workspace would be created or grown during HIP-graph capture; "
                    "run the same call once on this stream before capturing"
                )
            if ws is not None:
                _STREAM_WS_OUTGROWN.append(ws)
                need = max(need, 2 * ws.numel())
            ws = torch.zeros(need, dtype=torch.uint8, device=torch.device("cuda", idx))
        _STREAM_WS[key] = ws
    return ws
