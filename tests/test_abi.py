"""The C-ABI library loads, exports every entry point include/padra_hip.h (the drop-in
surface) and include/padra_hip_diag.h (self-checks, the benchmark's copy) declare, and
rejects bad host arguments with a status before any GPU work (CPU-only tests)."""
import ctypes
import os
import re

import numpy as np
import pytest

from padra_amd import abi, ops, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header="padra_hip.h"):
    text = open(os.path.join(ROOT, "include", header)).read()
    return sorted(set(re.findall(r"\b(padra_[A-Za-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declaration():
    lib = abi.lib()
    names = declared()
    diag = declared("padra_hip_diag.h")
    assert len(names) >= 4
    assert diag == ["padra_CheckFP8Paths", "padra_CheckQ8Path", "padra_StreamCopy"]
    assert not set(diag) & set(names)  # the drop-in header carries no diagnostics
    for name in names + diag:
        assert hasattr(lib, name), name
    assert set(names + diag) <= set(abi.SIGNATURES)


def test_static_workspace_size_matches_header():
    text = open(os.path.join(ROOT, "include", "padra_hip.h")).read()
    m = re.search(r"#define PADRA_DECODE_ATTENTION_STATIC_FLOATS (\d+)", text)
    assert m and int(m.group(1)) == abi.DECODE_ATTENTION_STATIC_FLOATS


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


def _p(v):
    return ctypes.c_void_p(v)


def test_host_validation_newer_entry_points():
    """Argument checks of the FP8 norm, combine, checkpoint, q8_0 prefix decode and decode
    attention entry points: each returns its status and launches nothing."""
    lib = abi.lib()
    bad = _p(16)
    # FP8 norm: packed must be given and 16-byte aligned; hidden from the supported set
    assert lib.padra_NormFP8(None, _p(16), _p(32), _p(48), None, _p(64), 4, 2048, 1e-6, None, bad,
                             0) == abi.INVALID_ARGUMENT
    assert lib.padra_NormFP8(None, _p(16), _p(32), _p(48), _p(72), _p(64), 4, 2048, 1e-6, None,
                             bad, 0) == abi.INVALID_ARGUMENT
    assert lib.padra_NormFP8(None, _p(16), _p(32), _p(48), _p(64), _p(64), 4, 1536, 1e-6, None,
                             bad, 0) == abi.UNSUPPORTED
    # combine: the reference's top-8 only
    assert lib.padra_Combine(None, _p(16), _p(32), _p(48), 4, 2048, 6, 1, bad, 0) == \
        abi.UNSUPPORTED
    assert lib.padra_Combine(None, _p(16), _p(32), _p(48), 4, 2044, 8, 1, bad, 0) == \
        abi.INVALID_ARGUMENT
    # combine + norm: normalized may not alias x; scales required with packed
    assert lib.padra_CombineNorm(None, _p(16), _p(32), _p(48), _p(16), _p(64), None, None, 1,
                                 2304, 8, 1e-6, None, bad, 0) == abi.INVALID_ARGUMENT
    assert lib.padra_CombineNorm(None, _p(16), _p(32), _p(48), _p(80), _p(64), _p(96), None, 1,
                                 2304, 8, 1e-6, None, bad, 0) == abi.INVALID_ARGUMENT
    # checkpoint: formats must agree, the snapshot may not alias a source
    ring = abi.KVCache(format=abi.KV_BF16, k=16, v=32, scales=None, cap=1024, first=0,
                       seq_stride=0)
    chunk = abi.KVCache(format=abi.KV_BF16, k=48, v=64, scales=None, cap=16, first=0,
                        seq_stride=0)
    other = abi.KVCache(format=abi.KV_Q8_0, k=80, v=96, scales=None, cap=1024, first=0,
                        seq_stride=0)
    alias = abi.KVCache(format=abi.KV_BF16, k=48, v=96, scales=None, cap=1024, first=0,
                        seq_stride=0)
    good = abi.KVCache(format=abi.KV_BF16, k=80, v=96, scales=None, cap=1024, first=0,
                       seq_stride=0)
    state = np.zeros(8, np.int32)
    pre = abi.Positions(mode=abi.POS_PREFILL, base=0, prefill=state.ctypes.data, decode=None,
                        maximum=4096, vocab=1, binding_epoch=1)
    for saved, want in ((other, abi.INVALID_ARGUMENT), (alias, abi.INVALID_ARGUMENT)):
        assert lib.padra_KVCheckpointCapture(None, ctypes.byref(ring), ctypes.byref(chunk),
                                             ctypes.byref(saved), ctypes.byref(pre), 16, 8, 4,
                                             bad) == want
    base = abi.Positions(mode=abi.POS_BASE, base=0, prefill=None, decode=None, maximum=4096,
                         vocab=1, binding_epoch=1)
    assert lib.padra_KVCheckpointCapture(None, ctypes.byref(ring), ctypes.byref(chunk),
                                         ctypes.byref(good), ctypes.byref(base), 16, 8, 4,
                                         bad) == abi.INVALID_ARGUMENT
    # q8_0 prefix decode needs a PrefillState
    assert lib.padra_KvQ8_0DequantizePrefix(None, _p(16), _p(32), _p(48), _p(64),
                                            ctypes.byref(base), 8, 64, 4, bad) == \
        abi.INVALID_ARGUMENT
    # decode attention: a BF16 cache, decode states, enough scratch, supported head groups
    dec = abi.Positions(mode=abi.POS_DECODE, base=0, prefill=None, decode=state.ctypes.data,
                        maximum=4096, vocab=98304, binding_epoch=1)
    kv = abi.KVCache(format=abi.KV_BF16, k=16, v=32, scales=None, cap=4096, first=0,
                     seq_stride=4096)
    need = lib.padra_DecodeAttentionScratch(abi.KV_BF16, 2, 16, 32)
    assert need == 2 * 32 * 16 * 129 + 4  # partials and lse, then the dispatch order
    assert lib.padra_DecodeAttentionScratch(abi.KV_Q8_0, 2, 16, 32) == need + 2 * 16 * 36
    assert lib.padra_DecodeAttentionScratch(abi.KV_BF16, 2, 16, 33) == -1
    assert lib.padra_DecodeAttentionScratch(abi.KV_Q8, 2, 16, 32) == need
    assert lib.padra_DecodeAttentionScratch(abi.KV_Q8_0_NOROT, 2, 16, 32) == -1
    # the lse ends on a 16-byte boundary before the q8_0 query region; the dispatch order
    # (one int per sequence) is last, rounded up to 16 bytes
    assert lib.padra_DecodeAttentionScratch(abi.KV_BF16, 1, 1, 1) == 132 + 4
    assert lib.padra_DecodeAttentionScratch(abi.KV_Q8_0, 1, 1, 1) == 132 + 36 + 4
    assert lib.padra_DecodeAttentionScratch(abi.KV_BF16, 5, 1, 1) == 5 * 129 + 3 + 8
    assert lib.padra_DecodeAttention(None, _p(16), ctypes.byref(kv), _p(32), ctypes.byref(dec), 2,
                                     16, 4, 0, 0, _p(64), need - 1, bad, 0) == abi.INVALID_ARGUMENT
    assert lib.padra_DecodeAttention(None, _p(16), ctypes.byref(kv), _p(32), ctypes.byref(dec), 2,
                                     24, 4, 0, 0, _p(64), need * 2, bad, 0) == abi.UNSUPPORTED
    q8 = abi.KVCache(format=abi.KV_Q8, k=16, v=32, scales=None, cap=4096, first=0,
                     seq_stride=4096)
    assert lib.padra_DecodeAttention(None, _p(16), ctypes.byref(q8), _p(32), ctypes.byref(dec), 2,
                                     16, 4, 0, 0, _p(64), need, bad, 0) == abi.INVALID_ARGUMENT
    norot = abi.KVCache(format=abi.KV_Q8_0_NOROT, k=16, v=32, scales=None, cap=4096, first=0,
                        seq_stride=4096)
    assert lib.padra_DecodeAttention(None, _p(16), ctypes.byref(norot), _p(32), ctypes.byref(dec),
                                     2, 16, 4, 0, 0, _p(64), need, bad, 0) == abi.UNSUPPORTED
    assert lib.padra_DecodeAttention(None, _p(16), ctypes.byref(kv), _p(32), ctypes.byref(base),
                                     2, 16, 4, 0, 0, _p(64), need, bad, 0) == abi.INVALID_ARGUMENT
    # the entry point without a workspace argument refuses launches its fixed array cannot
    # hold (64 sequences x 64 query heads x 32 splits), before touching a device
    assert lib.padra_DecodeAttentionScratch(abi.KV_BF16, 64, 64, 32) > \
        abi.DECODE_ATTENTION_STATIC_FLOATS
    assert lib.padra_DecodeAttentionNoAlloc(None, _p(16), ctypes.byref(kv), _p(32),
                                            ctypes.byref(dec), 64, 64, 8, 0, 32, bad, 0) == \
        abi.INVALID_ARGUMENT
    assert lib.padra_DecodeAttentionNoAlloc(None, _p(16), None, _p(32), ctypes.byref(dec), 2,
                                            16, 4, 0, 0, bad, 0) == abi.INVALID_ARGUMENT
    # the FP8 merge: both outputs required and aligned, at most 32 query heads, no q8_0
    fp8 = lib.padra_DecodeAttentionFP8
    assert fp8(None, _p(16), ctypes.byref(kv), _p(32), None, _p(96), ctypes.byref(dec), 2, 16,
               4, 0, 0, _p(64), need, bad, 0) == abi.INVALID_ARGUMENT
    assert fp8(None, _p(16), ctypes.byref(kv), _p(32), _p(80), None, ctypes.byref(dec), 2, 16,
               4, 0, 0, _p(64), need, bad, 0) == abi.INVALID_ARGUMENT
    assert fp8(None, _p(16), ctypes.byref(kv), _p(32), _p(81), _p(96), ctypes.byref(dec), 2, 16,
               4, 0, 0, _p(64), need, bad, 0) == abi.INVALID_ARGUMENT
    big = lib.padra_DecodeAttentionScratch(abi.KV_BF16, 2, 64, 32)
    assert fp8(None, _p(16), ctypes.byref(kv), _p(32), _p(80), _p(96), ctypes.byref(dec), 2, 64,
               8, 0, 0, _p(64), big, bad, 0) == abi.INVALID_ARGUMENT
    q8_0 = abi.KVCache(format=abi.KV_Q8_0, k=16, v=32, scales=None, cap=4096, first=0,
                       seq_stride=4096)
    assert fp8(None, _p(16), ctypes.byref(q8_0), _p(32), _p(80), _p(96), ctypes.byref(dec), 2,
               16, 4, 0, 0, _p(64), need * 2, bad, 0) == abi.UNSUPPORTED
    # the self-checks need their count buffers; the streaming copy whole 16-byte units
    assert lib.padra_CheckQ8Path(None, None) == abi.INVALID_ARGUMENT
    assert lib.padra_CheckFP8Paths(None, None) == abi.INVALID_ARGUMENT
    # fused gather + chain: the embedding table is required
    base = abi.Positions(mode=abi.POS_BASE, base=0, prefill=None, decode=None, maximum=4096,
                         vocab=1000, binding_epoch=1)
    assert lib.padra_EmbedResidualNormQKRopeStore(
        None, None, 1000, _p(160), _p(16), _p(32), _p(48), _p(64), 2048, 256, None, _p(80),
        _p(96), None, _p(112), _p(128), _p(144), 4096, ctypes.byref(base), 1, 16, 4, 128, 1e-6,
        None, bad) == abi.INVALID_ARGUMENT
    assert lib.padra_StreamCopy(None, _p(16), _p(32), 24) == abi.INVALID_ARGUMENT
    assert lib.padra_StreamCopy(None, _p(16), _p(40), 32) == abi.INVALID_ARGUMENT


def test_decode_attention_split_counts():
    """padra_DecodeAttentionSplits: 0 gives the reference's count, -1 the tuned count for a
    local ring (a global window keeps the reference's), 1..32 as given, anything else -1."""
    lib = abi.lib()

    def splits(fmt, cap, seqs, local, s, kv_heads=4):
        kv = abi.KVCache(fmt, None, None, None, cap, 0, 0)
        return lib.padra_DecodeAttentionSplits(ctypes.byref(kv), seqs, kv_heads, local, s)

    bf16, q8, q8_0 = abi.KV_BF16, abi.KV_Q8, abi.KV_Q8_0
    # reference counts: min(ceil(cap / 32), 16 local / 32 global); q8_0 always 16 / 32
    assert splits(bf16, 4096, 64, 1, 0) == 16 and splits(bf16, 4096, 64, 0, 0) == 32
    assert splits(bf16, 100, 64, 0, 0) == 4 and splits(q8_0, 100, 64, 0, 0) == 32
    assert splits(q8_0, 4096, 1, 1, 0) == 16
    # tuned, local: ~1,024 resident waves (BF16, q8_0 by sequences alone), ~2,048 for q8
    assert [splits(bf16, 4096, n, 1, -1) for n in (1, 8, 40, 64, 512)] == [16, 16, 6, 4, 2]
    assert [splits(q8, 4096, n, 1, -1) for n in (1, 8, 40, 64, 512)] == [32, 32, 12, 8, 2]
    assert [splits(q8_0, 4096, n, 1, -1) for n in (1, 8, 40, 64, 512)] == [16, 16, 6, 4, 4]
    assert splits(bf16, 100, 1, 1, -1) == 4 and splits(bf16, 64, 64, 1, -1) == 2
    assert splits(bf16, 4096, 64, 1, -1, kv_heads=1) == 16
    # tuned, global: the reference's count
    for fmt in (bf16, q8, q8_0):
        assert splits(fmt, 4096, 64, 0, -1) == splits(fmt, 4096, 64, 0, 0)
    # explicit counts pass through; out of range is invalid
    assert splits(bf16, 4096, 64, 1, 7) == 7 and splits(q8, 4096, 64, 0, 32) == 32
    assert splits(bf16, 4096, 64, 1, 33) == -1 and splits(bf16, 4096, 64, 1, -2) == -1
