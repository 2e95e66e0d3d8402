"""ctypes binding of the CPU parity oracle (oracle/libpadra_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker.  The product (padra_amd) never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# PADRA_ORACLE_LIB selects another build of the same source (the sanitizer build of
# `make -C oracle asan`).
LIB = os.environ.get("PADRA_ORACLE_LIB") or os.path.join(HERE, "libpadra_oracle.so")


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = ctypes.CDLL(LIB)
        P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        sig = {
            "po_bf16_round": ([F], F), "po_f32_to_f16": ([F], ctypes.c_uint16),
            "po_f16_to_f32": ([ctypes.c_uint16], F),
            "po_sumsq_tree": ([P, I, I], F),
            "po_residual_rmsnorm": ([P, P, P, P, I, I, F, I, P, P], None),
            "po_rmsnorm": ([P, P, P, I, I, F, I, P, P], None),
            "po_e4m3": ([F], ctypes.c_uint8),
            "po_fp8_needs_division": ([ctypes.c_uint32], I),
            "po_fp8_encode": ([F, F, F], ctypes.c_uint8),
            "po_norm_fp8": ([P, P, P, P, P, I, I, F, P, P], None),
            "po_combine": ([P, P, P, I, I, I, I, P], None),
            "po_quantize_fp8": ([P, P, P, I, I, P], None),
            "po_round_away_mismatches": ([ctypes.c_uint64, ctypes.c_uint64], ctypes.c_ulonglong),
            "po_decode_attention": ([P, P, P, I, I, I, I, I, I, P, P], I),
            "po_decode_attention_q8_0": ([P, P, P, I, I, I, I, I, I, P, P], I),
            "po_kv_checkpoint_plane": ([P, P, P, I, I, I], None),
            "po_kv_checkpoint_admitted": ([P, I, I, ctypes.c_uint32, I], I),
            "po_combine_norm": ([P, P, P, P, P, P, P, I, I, I, F, P, P], None),
            "po_rope_table": ([P, I, I, F, I, F, I], None),
            "po_qk_norm_rope": ([P, P, P, P, P, P, I, I, I, I, F, P], None),
            "po_kv_store_bf16": ([P, P, P, P, P, I, I, I, I], None),
            "po_kv_q8_encode": ([P, P, P, P, P, P, I, I, I, I, I, P], None),
            "po_hadamard": ([P, I, F], None),
            "po_q8_0_row_bytes": ([I], I),
            "po_kv_q8_0_encode": ([P, P, P, P, P, I, I, I, I, I, I, P], None),
            "po_kv_q8_0_dequantize": ([P, P, P, P, I, I, P], None),
            "po_silu_bf16": ([ctypes.c_uint16], ctypes.c_uint16),
            "po_silu_table": ([P], None),
            "po_swiglu": ([P, P, P, ctypes.c_longlong, P], None),
            "po_embed": ([P, P, P, I, I, I, P], None),
            "po_decode_ready": ([P, I, I], I),
            "po_valid_prefill_state": ([P, I, I, ctypes.c_uint32, I], I),
        }
        for name, (args, res) in sig.items():
            fn = getattr(_lib, name)
            fn.argtypes = args
            fn.restype = res
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


class Bad:
    def __init__(self):
        self.v = ctypes.c_int(0)

    @property
    def ptr(self):
        return ctypes.byref(self.v)

    def __bool__(self):
        return bool(self.v.value)


def residual_rmsnorm(x, residual, gamma, eps=1e-6, threads=128):
    """Returns (x_new, y, stats, bad) for BF16-bit arrays x, residual [rows][H]."""
    x = np.array(x, dtype=np.uint16, copy=True, order="C")
    rows, hidden = x.shape
    y = np.empty_like(x)
    stats = np.empty((rows, 2), np.float32)
    bad = Bad()
    lib().po_residual_rmsnorm(_p(x), _p(np.ascontiguousarray(residual, np.uint16)), _p(y),
                              _p(np.ascontiguousarray(gamma, np.uint16)), rows, hidden, eps,
                              threads, _p(stats), bad.ptr)
    return x, y, stats, bool(bad)


def rmsnorm(x, gamma, eps=1e-6, threads=128):
    x = np.ascontiguousarray(x, np.uint16)
    rows, hidden = x.shape
    y = np.empty_like(x)
    stats = np.empty((rows, 2), np.float32)
    bad = Bad()
    lib().po_rmsnorm(_p(x), _p(y), _p(np.ascontiguousarray(gamma, np.uint16)), rows, hidden,
                     eps, threads, _p(stats), bad.ptr)
    return y, stats, bool(bad)


def norm_fp8(x, gamma, eps=1e-6):
    """Returns (normalized, packed u8, scales [rows], stats [2] of row 0, bad)."""
    x = np.ascontiguousarray(x, np.uint16)
    rows, hidden = x.shape
    y = np.empty_like(x)
    packed = np.empty((rows, hidden), np.uint8)
    scales = np.empty(rows, np.float32)
    stats = np.empty(2, np.float32)
    bad = Bad()
    lib().po_norm_fp8(_p(x), _p(y), _p(np.ascontiguousarray(gamma, np.uint16)), _p(packed),
                      _p(scales), rows, hidden, eps, _p(stats), bad.ptr)
    return y, packed, scales, stats, bool(bad)


def combine(x, down, weights, residual=True):
    """x [rows][H] BF16 bits, down [rows][E][H] BF16 bits, weights [rows][E] f32.
    Returns (x_new, bad)."""
    x = np.array(x, dtype=np.uint16, copy=True, order="C")
    rows, hidden = x.shape
    experts = down.shape[1]
    bad = Bad()
    lib().po_combine(_p(x), _p(np.ascontiguousarray(down, np.uint16)),
                     _p(np.ascontiguousarray(weights, np.float32)), rows, hidden, experts,
                     int(bool(residual)), bad.ptr)
    return x, bool(bad)


def combine_norm(x, down, weights, gamma, fp8=True, eps=1e-6):
    """Returns (x_new, normalized, packed or None, scales or None, stats [2], bad)."""
    x = np.array(x, dtype=np.uint16, copy=True, order="C")
    rows, hidden = x.shape
    experts = down.shape[1]
    y = np.empty_like(x)
    packed = np.empty((rows, hidden), np.uint8) if fp8 else None
    scales = np.empty(rows, np.float32) if fp8 else None
    stats = np.empty(2, np.float32)
    bad = Bad()
    lib().po_combine_norm(_p(x), _p(np.ascontiguousarray(down, np.uint16)),
                          _p(np.ascontiguousarray(weights, np.float32)), _p(y),
                          _p(np.ascontiguousarray(gamma, np.uint16)), _p(packed), _p(scales),
                          rows, hidden, experts, eps, _p(stats), bad.ptr)
    return x, y, packed, scales, stats, bool(bad)


def kv_checkpoint(old_planes, current_planes, state, tokens, anchor, epoch=1, maximum=131072):
    """Snapshot of a 1024-row local ring.  old_planes / current_planes: lists of 2-D byte
    arrays (rows x row_bytes; old: 1024 rows, current: `tokens` rows), one per plane (K, V
    and, for q8, the scale pairs).  state: int32[8] PrefillState.  Returns the saved planes,
    or None when the capture is not admitted."""
    st = np.ascontiguousarray(state, np.int32)
    if not lib().po_kv_checkpoint_admitted(_p(st), tokens, anchor, epoch, maximum):
        return None
    out = []
    for old, cur in zip(old_planes, current_planes):
        old = np.ascontiguousarray(old).view(np.uint8).reshape(1024, -1)
        cur = np.ascontiguousarray(cur).view(np.uint8).reshape(cur.shape[0], -1)
        saved = np.empty_like(old)
        lib().po_kv_checkpoint_plane(_p(old), _p(cur), _p(saved), old.shape[1], int(st[0]),
                                     anchor)
        out.append(saved)
    return out


def decode_attention(q, kc, vc, position, local=False, splits=0):
    """q [hq][128] BF16 bits, kc / vc [cap][hkv*128] BF16 bits.  Returns (out [hq][128]
    BF16 bits, splits used, bad)."""
    q = np.ascontiguousarray(q, np.uint16)
    kc = np.ascontiguousarray(kc, np.uint16)
    vc = np.ascontiguousarray(vc, np.uint16)
    hq = q.shape[0]
    cap, features = kc.shape
    out = np.empty((hq, 128), np.uint16)
    bad = Bad()
    used = lib().po_decode_attention(_p(q), _p(kc), _p(vc), cap, int(position), int(bool(local)),
                                     hq, features // 128, int(splits), _p(out), bad.ptr)
    return out, used, bool(bad)


def decode_attention_q8_0(q, rows_k, rows_v, position, local=False, splits=0, hkv=4):
    """q [hq][128] BF16 bits, rows_k / rows_v [cap][544] q8_0 rows.  Returns (out [hq][128]
    BF16 bits, splits used, bad)."""
    q = np.ascontiguousarray(q, np.uint16)
    rows_k = np.ascontiguousarray(rows_k, np.uint8)
    rows_v = np.ascontiguousarray(rows_v, np.uint8)
    hq = q.shape[0]
    out = np.zeros((hq, 128), np.uint16)
    bad = Bad()
    used = lib().po_decode_attention_q8_0(_p(q), _p(rows_k), _p(rows_v), rows_k.shape[0],
                                          int(position), int(bool(local)), hq, hkv, int(splits),
                                          _p(out), bad.ptr)
    return out, used, bool(bad)


def round_away_mismatches(lo=0, hi=1 << 32):
    """Floats in bit range [lo, hi) where the GPU's three-instruction roundf differs."""
    return int(lib().po_round_away_mismatches(lo, hi))


def quantize_fp8(x):
    """x fp32 [rows][cols].  Returns (packed u8, scales [rows], bad)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    packed = np.empty((rows, cols), np.uint8)
    scales = np.empty(rows, np.float32)
    bad = Bad()
    lib().po_quantize_fp8(_p(x), _p(packed), _p(scales), rows, cols, bad.ptr)
    return packed, scales, bool(bad)


def e4m3(values) -> np.ndarray:
    f = lib().po_e4m3
    return np.array([f(float(v)) for v in np.asarray(values, np.float32)], np.uint8)


def rope_table(positions, head_dim=128, theta=1e6, yarn=False, factor=16.0,
               original_context=8192) -> np.ndarray:
    """float32 [positions][head_dim] (BF16-exact values)."""
    t = np.empty((positions, head_dim), np.float32)
    lib().po_rope_table(_p(t), positions, head_dim, theta, int(yarn), factor, original_context)
    return t


def qk_norm_rope(q, k, qn, kn, table_bits, positions, eps=1e-6):
    q = np.array(q, dtype=np.uint16, copy=True, order="C")
    k = np.array(k, dtype=np.uint16, copy=True, order="C")
    tokens, hq, d = q.shape
    hkv = k.shape[1]
    pos = np.ascontiguousarray(positions, np.int32)
    bad = Bad()
    lib().po_qk_norm_rope(_p(q), _p(k), _p(np.ascontiguousarray(qn, np.uint16)),
                          _p(np.ascontiguousarray(kn, np.uint16)),
                          _p(np.ascontiguousarray(table_bits, np.uint16)), _p(pos), tokens, hq,
                          hkv, d, eps, bad.ptr)
    return q, k, bool(bad)


def kv_store_bf16(k, v, kc, vc, positions, cap, first=0):
    tokens = k.shape[0]
    features = int(np.prod(k.shape[1:]))
    lib().po_kv_store_bf16(_p(np.ascontiguousarray(k, np.uint16)),
                           _p(np.ascontiguousarray(v, np.uint16)), _p(kc), _p(vc),
                           _p(np.ascontiguousarray(positions, np.int32)), tokens, features, cap,
                           first)


def kv_q8_encode(k, v, codes_k, codes_v, scales, positions, cap, first=0):
    tokens, hkv, d = k.shape
    bad = Bad()
    lib().po_kv_q8_encode(_p(np.ascontiguousarray(k, np.uint16)),
                          _p(np.ascontiguousarray(v, np.uint16)), _p(codes_k), _p(codes_v),
                          _p(scales), _p(np.ascontiguousarray(positions, np.int32)), tokens,
                          hkv, d, cap, first, bad.ptr)
    return bool(bad)


def kv_q8_0_encode(k, v, rows_k, rows_v, positions, cap, first=0, rotate=True):
    tokens, hkv, d = k.shape
    bad = Bad()
    lib().po_kv_q8_0_encode(_p(np.ascontiguousarray(k, np.uint16)),
                            _p(np.ascontiguousarray(v, np.uint16)), _p(rows_k), _p(rows_v),
                            _p(np.ascontiguousarray(positions, np.int32)), tokens, hkv, d, cap,
                            first, int(rotate), bad.ptr)
    return bool(bad)


def kv_q8_0_dequantize(rows_k, rows_v, rows, features):
    out_k = np.empty((rows, features), np.uint16)
    out_v = np.empty((rows, features), np.uint16)
    bad = Bad()
    lib().po_kv_q8_0_dequantize(_p(rows_k), _p(rows_v), _p(out_k), _p(out_v), rows, features,
                                bad.ptr)
    return out_k, out_v, bool(bad)


def hadamard(x, scale):
    x = np.array(x, dtype=np.float32, copy=True)
    lib().po_hadamard(_p(x), x.size, scale)
    return x


def silu_table() -> np.ndarray:
    t = np.empty(65536, np.uint16)
    lib().po_silu_table(_p(t))
    return t


def swiglu(gate, up):
    gate = np.ascontiguousarray(gate, np.uint16)
    out = np.zeros_like(gate)
    bad = Bad()
    lib().po_swiglu(_p(gate), _p(np.ascontiguousarray(up, np.uint16)), _p(out), gate.size,
                    bad.ptr)
    return out, bool(bad)


def embed(table, ids, vocab=None):
    ids = np.ascontiguousarray(ids, np.int32)
    vocab = table.shape[0] if vocab is None else vocab
    out = np.zeros((ids.size, table.shape[1]), np.uint16)
    bad = Bad()
    lib().po_embed(_p(np.ascontiguousarray(table, np.uint16)), _p(ids), _p(out), ids.size,
                   table.shape[1], vocab, bad.ptr)
    return out, bool(bad)
