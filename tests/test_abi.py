"""The C-ABI library loads, exports every entry point include/padra_hip.h declares, and
rejects bad host arguments with a status before any GPU work (CPU-only tests)."""
import ctypes
import os
import re

import numpy as np
import pytest

from padra_amd import abi, ops, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "padra_hip.h")).read()
    return sorted(set(re.findall(r"\b(padra_[A-Za-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declaration():
    lib = abi.lib()
    names = declared()
    assert len(names) >= 4
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) <= set(abi.SIGNATURES)


def test_version():
    assert b"gfx950" in abi.lib().padra_version()


def test_host_validation_returns_status_without_launch():
    lib = abi.lib()
    bad = ctypes.c_void_p(16)
    # null x
    st = lib.padra_ResidualPostNorm(None, None, None, ctypes.c_void_p(16), ctypes.c_void_p(16),
                                    1, 2048, 1e-6, 128, None, bad, 0)
    assert st == abi.INVALID_ARGUMENT
    # hidden not a multiple of the tree
    st = lib.padra_ResidualPostNorm(None, ctypes.c_void_p(16), None, ctypes.c_void_p(32),
                                    ctypes.c_void_p(48), 1, 2000, 1e-6, 128, None, bad, 0)
    assert st == abi.UNSUPPORTED
    # misaligned pointer
    st = lib.padra_ResidualPostNorm(None, ctypes.c_void_p(18), None, ctypes.c_void_p(32),
                                    ctypes.c_void_p(48), 1, 2048, 1e-6, 128, None, bad, 0)
    assert st == abi.INVALID_ARGUMENT
    # head_dim other than 128
    pos = ops.positions_base(0)
    st = lib.padra_QKNormRopeStore(None, ctypes.c_void_p(16), ctypes.c_void_p(32), None,
                                   ctypes.c_void_p(48), ctypes.c_void_p(64), ctypes.c_void_p(80),
                                   10, ctypes.byref(pos), 1, 16, 4, 64, 1e-6, None, bad, 0)
    assert st == abi.UNSUPPORTED
    # a local ring cannot hold more than cap rows of one chunk
    kv = abi.KVCache(format=abi.KV_BF16, k=16, v=32, scales=None, cap=4, first=0, seq_stride=0)
    st = lib.padra_QKNormRopeStore(None, ctypes.c_void_p(16), ctypes.c_void_p(32),
                                   ctypes.c_void_p(96), ctypes.c_void_p(48), ctypes.c_void_p(64),
                                   ctypes.c_void_p(80), 10, ctypes.byref(pos), 8, 16, 4, 128,
                                   1e-6, ctypes.byref(kv), bad, 0)
    assert st == abi.INVALID_ARGUMENT
    with pytest.raises(abi.PadraError):
        abi.call("padra_RopeTable", None, 1, 128, 1e6, 0, 16.0, 8192)


@pytest.mark.parametrize("theta,yarn", [(1e6, False), (5e5, False), (5e5, True)])
def test_rope_table_host_matches_oracle(oracle, theta, yarn):
    got = ops.RopeTable(3000, 128, theta, yarn=yarn).view(__import__("torch").int16).numpy()
    want = synth.bf16_bits(oracle.rope_table(3000, 128, theta, yarn=yarn))
    assert np.array_equal(got.view(np.uint16), want)
