"""The library called at run time from C++ (tests/cpp/padra_caller.cpp): a C++20 program
that includes only include/padra_hip.h and links libpadra_hip.so, fills the device
PrefillState and DecodeStates as Padra's runtime does, and runs the config-1 chain (eager,
then a captured HIP graph replayed after the state moves to the next chunk) and the
config-4 fused decode step (embedding gather + chain, 64 sequences).  Its outputs are
compared with the oracle bit for bit.  The program is built with the library
(padra_amd/build.py build_caller) and started as a child process."""
import os
import subprocess

import numpy as np
import pytest

from padra_amd import synth

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
CALLER = os.path.join(HERE, "cpp", "padra_caller")


def _write(d, name, a):
    np.ascontiguousarray(a).tofile(os.path.join(d, name))


def _read(d, name, dtype=np.uint16):
    return np.fromfile(os.path.join(d, name), dtype=dtype)


def test_cpp_caller(oracle, tmp_path):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert os.path.exists(CALLER), "build the C++ caller first: python -m padra_amd.build"
    d = str(tmp_path)
    # config 1: a 2048-token chunk at base 1000 of an 8192-row BF16 cache
    tokens, hidden, hq, hkv, cap, base = 2048, 2048, 16, 4, 8192, 1000
    c = synth.chain_inputs(tokens, hidden, hq, hkv, 128, outliers=True, seed=21)
    _write(d, "chain_meta.i32", np.array([tokens, hidden, hq, hkv, cap, base], np.int32))
    for key in ("x", "residual", "gamma", "q", "k", "v", "qn", "kn"):
        _write(d, "chain_" + ("r" if key == "residual" else key), c[key])
    # config 4: 64 sequences, ragged positions in 4096-row caches, Zipf tokens of an
    # 8192-row embedding table
    seqs, dcap, vocab = 64, 4096, 8192
    e = synth.chain_inputs(vocab, hidden, hq, hkv, 128, outliers=False, seed=22)
    dd = synth.chain_inputs(seqs, hidden, hq, hkv, 128, outliers=False, seed=23)
    rng = np.random.default_rng(24)
    positions = rng.integers(0, dcap, seqs).astype(np.int32)
    positions[0] = 0
    ids = synth.zipf_ids(seqs, vocab, s=1.1, seed=25)
    states = np.zeros((seqs, 8), np.int32)
    for s in range(seqs):
        p = int(positions[s])
        states[s] = [ids[s], p, dcap, 10, p, min(p, 1024), 0, 0]
    _write(d, "decode_meta.i32", np.array([seqs, hidden, hq, hkv, dcap, vocab], np.int32))
    _write(d, "decode_embed", e["x"])
    _write(d, "decode_states.i32", states)
    for key in ("residual", "gamma", "q", "k", "v", "qn", "kn"):
        _write(d, "decode_" + ("r" if key == "residual" else key), dd[key])

    print("[case] C++ caller: config-1 chunk (eager and graph replay), config-4 step", flush=True)
    res = subprocess.run([CALLER, d], capture_output=True, text=True, timeout=180)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip().endswith("ok")

    # the chunk, eagerly and replayed at base + tokens
    table = synth.bf16_bits(oracle.rope_table(cap, 128, 1e6))
    for prefix, b in (("chain_out_", base), ("replay_out_", base + tokens)):
        pos = np.arange(tokens, dtype=np.int32) + b
        wx, wy, _, _ = oracle.residual_rmsnorm(c["x"], c["residual"], c["gamma"], threads=128)
        wq, wk, _ = oracle.qk_norm_rope(c["q"], c["k"], c["qn"], c["kn"], table, pos)
        kc = np.zeros((cap, hkv * 128), np.uint16)
        vc = np.zeros_like(kc)
        oracle.kv_store_bf16(wk, c["v"], kc, vc, pos, cap)
        assert _read(d, prefix + "bad", np.int32)[0] == 0, prefix
        assert np.array_equal(_read(d, prefix + "x").reshape(wx.shape), wx), prefix
        assert np.array_equal(_read(d, prefix + "y").reshape(wy.shape), wy), prefix
        assert np.array_equal(_read(d, prefix + "q").reshape(wq.shape), wq), prefix
        assert np.array_equal(_read(d, prefix + "k").reshape(wk.shape), wk), prefix
        assert np.array_equal(_read(d, prefix + "kc").reshape(tokens, -1), kc[b:b + tokens])
        assert np.array_equal(_read(d, prefix + "vc").reshape(tokens, -1), vc[b:b + tokens])

    # the decode step: x = embed[token], the 256-thread tree, one cache row per sequence
    dtable = synth.bf16_bits(oracle.rope_table(dcap, 128, 1e6))
    x0 = e["x"][ids]
    wx, wy, _, _ = oracle.residual_rmsnorm(x0, dd["residual"], dd["gamma"], threads=256)
    wq, wk, _ = oracle.qk_norm_rope(dd["q"], dd["k"], dd["qn"], dd["kn"], dtable, positions)
    assert _read(d, "decode_out_bad", np.int32)[0] == 0
    assert np.array_equal(_read(d, "decode_out_x").reshape(wx.shape), wx)
    assert np.array_equal(_read(d, "decode_out_y").reshape(wy.shape), wy)
    assert np.array_equal(_read(d, "decode_out_q").reshape(wq.shape), wq)
    assert np.array_equal(_read(d, "decode_out_k").reshape(wk.shape), wk)
    assert np.array_equal(_read(d, "decode_out_kc").reshape(seqs, -1), wk.reshape(seqs, -1))
    assert np.array_equal(_read(d, "decode_out_vc").reshape(seqs, -1), dd["v"].reshape(seqs, -1))
