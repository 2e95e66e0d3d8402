"""ctypes binding of include/padra_hip.h (libpadra_hip.so).

The library is loaded lazily on first use and must exist: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# PADRA_HIP_LIB selects another build of the same library (the host-sanitizer build of
# padra_amd/build.py --asan); it must exist like the default one.
library_path = os.environ.get("PADRA_HIP_LIB") or os.path.join(_HERE, "libpadra_hip.so")

# Status codes (mellum16::StatusCode numbering, include/mellum16/status.h:11-21).
OK, INVALID_ARGUMENT, UNSUPPORTED, INTERNAL = 0, 1, 5, 8
_STATUS = {INVALID_ARGUMENT: "invalid argument", UNSUPPORTED: "unsupported shape",
           INTERNAL: "internal (launch failed)"}

ACT_BF16, ACT_F32 = 0, 1
TREE_128, TREE_256 = 128, 256
KV_BF16, KV_Q8, KV_Q8_0, KV_Q8_0_NOROT = 0, 1, 2, 3
POS_BASE, POS_PREFILL, POS_DECODE = 0, 1, 2


class PadraError(RuntimeError):
    """A nonzero status from the C-ABI (nothing was launched)."""

    def __init__(self, fn: str, status: int):
        super().__init__(f"{fn}: {_STATUS.get(status, 'status')} ({status})")
        self.status = status


class DecodeState(ctypes.Structure):
    """decode_control.cuh:3-6 (32 bytes)."""
    _fields_ = [(n, ctypes.c_int32) for n in (
        "token", "position", "capacity", "remaining", "global_valid", "local_valid", "eos",
        "stopped")]


class PrefillState(ctypes.Structure):
    """src/runtime/prefill_state.h:8-11 (32 bytes)."""
    _fields_ = [("base", ctypes.c_int32), ("prompt_offset", ctypes.c_int32),
                ("tokens", ctypes.c_int32), ("capacity", ctypes.c_int32),
                ("committed", ctypes.c_int32), ("binding_epoch", ctypes.c_uint32),
                ("request_epoch", ctypes.c_uint32), ("valid", ctypes.c_uint32)]


class Positions(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int32), ("base", ctypes.c_int32),
                ("prefill", ctypes.c_void_p), ("decode", ctypes.c_void_p),
                ("maximum", ctypes.c_int32), ("vocab", ctypes.c_int32),
                ("binding_epoch", ctypes.c_uint32)]


class KVCache(ctypes.Structure):
    _fields_ = [("format", ctypes.c_int32), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
                ("scales", ctypes.c_void_p), ("cap", ctypes.c_int32), ("first", ctypes.c_int32),
                ("seq_stride", ctypes.c_int64)]


assert ctypes.sizeof(DecodeState) == 32 and ctypes.sizeof(PrefillState) == 32

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float

# name -> argtypes (restype int unless listed otherwise)
# Floats of padra_DecodeAttentionNoAlloc's fixed device workspace (padra_hip.h).
DECODE_ATTENTION_STATIC_FLOATS = 4718592

SIGNATURES = {
    "padra_ResidualPostNorm": [_P, _P, _P, _P, _P, _I, _I, _F, _I, _P, _P, _I],
    "padra_RopeTable": [_P, _I, _I, _F, _I, _F, _I],
    "padra_QKNormRopeStore": [_P, _P, _P, _P, _P, _P, _P, _I, ctypes.POINTER(Positions), _I, _I,
                              _I, _I, _F, ctypes.POINTER(KVCache), _P, _I],
    "padra_ResidualNormQKRopeStore": [_P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I,
                                      ctypes.POINTER(Positions), _I, _I, _I, _I, _F,
                                      ctypes.POINTER(KVCache), _P, _I],
    "padra_EmbedResidualNormQKRopeStore": [_P, _P, _I, _P, _P, _P, _P, _P, _I, _I, _P, _P, _P,
                                           _P, _P, _P, _P, _I, ctypes.POINTER(Positions), _I,
                                           _I, _I, _I, _F, ctypes.POINTER(KVCache), _P],
    "padra_KVStore": [_P, _P, _P, ctypes.POINTER(Positions), _I, _I, _I, ctypes.POINTER(KVCache),
                      _P, _I],
    "padra_KVCommit": [_P, ctypes.POINTER(KVCache), ctypes.POINTER(KVCache),
                       ctypes.POINTER(Positions), _I, _I, _P],
    "padra_KvQ8_0Dequantize": [_P, _P, _P, _P, _P, ctypes.c_longlong, _I, _P, _I],
    "padra_KvQ8_0DequantizePrefix": [_P, _P, _P, _P, _P, ctypes.POINTER(Positions), _I, _I, _I,
                                     _P],
    "padra_CheckFP8Paths": [_P, _P],
    "padra_CheckQ8Path": [_P, _P],
    "padra_DecodeAttentionScratch": [_I, _I, _I, _I],
    "padra_DecodeAttentionSplits": [ctypes.POINTER(KVCache), _I, _I, _I, _I],
    "padra_DecodeAttention": [_P, _P, ctypes.POINTER(KVCache), _P, ctypes.POINTER(Positions), _I,
                              _I, _I, _I, _I, _P, ctypes.c_longlong, _P, _I],
    "padra_DecodeAttentionNoAlloc": [_P, _P, ctypes.POINTER(KVCache), _P,
                                     ctypes.POINTER(Positions), _I, _I, _I, _I, _I, _P, _I],
    "padra_DecodeAttentionFP8": [_P, _P, ctypes.POINTER(KVCache), _P, _P, _P,
                                 ctypes.POINTER(Positions), _I, _I, _I, _I, _I, _P,
                                 ctypes.c_longlong, _P, _I],
    "padra_KVCheckpointCapture": [_P, ctypes.POINTER(KVCache), ctypes.POINTER(KVCache),
                                  ctypes.POINTER(KVCache), ctypes.POINTER(Positions), _I, _I, _I,
                                  _P],
    "padra_Combine": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _I],
    "padra_QuantizeFP8": [_P, _P, _P, _P, _I, _I, _P, _I],
    "padra_CombineNorm": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, ctypes.c_float, _P, _P,
                          _I],
    "padra_NormFP8": [_P, _P, _P, _P, _P, _P, _I, _I, ctypes.c_float, _P, _P, _I],
    "padra_RotateRows": [_P, _P, ctypes.c_longlong, _I, _P, _I],
    "padra_SiluTableBuild": [_P, _P],
    "padra_SwiGLU": [_P, _P, _P, _P, ctypes.c_longlong, _P, _P, _I],
    "padra_Embed": [_P, _P, _I, _I, _P, ctypes.POINTER(Positions), _I, _P, _P, _I],
    "padra_StreamCopy": [_P, _P, _P, ctypes.c_longlong],
    "padra_version": [],
}
RESTYPES = {"padra_version": ctypes.c_char_p, "padra_DecodeAttentionScratch": ctypes.c_longlong}

_lib = None


def lib() -> ctypes.CDLL:
    """Loads libpadra_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(library_path):
            raise RuntimeError(
                f"{library_path} is missing: build it with `python -m padra_amd.build` "
                "(hipcc, gfx950).  There is no CPU fallback.")
        handle = ctypes.CDLL(library_path)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        _lib = handle
    return _lib


def call(name: str, *args) -> None:
    status = getattr(lib(), name)(*args)
    if status != OK:
        raise PadraError(name, status)
