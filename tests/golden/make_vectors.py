"""Writes tests/golden/op_vectors.npz: a few rows per op per BASELINE config, inputs and
expected outputs, computed by the C oracle (oracle/padra_oracle.c), so that a later change
of the oracle, or a caller without Python, can check outputs against stored bytes.

  chain_<fmt>  config 1/2: 4 tokens of the fused residual+RMSNorm+QK-norm+RoPE+KV store
               (128-thread tree, outlier channels), positions 4097..4100 of an 8192-row
               cache, for BF16, q8, q8_0 (rotated) and q8_0 (unrotated) caches; the cache
               rows the tokens write are stored (BF16 / int8 codes / 544-byte rows; q8
               scale pairs)
  decode       config 0/4: 3 sequences of the decode step (gather from a 16-row embedding
               table, 256-thread tree, ragged positions, BF16 cache rows)
  swiglu       config 3: 4 rows x 1024 of silu(gate) * up (gate, up N(0, 2))
  table        RoPE rows 0, 1, 4097 and 131071 (theta 1e6)

Run: python tests/golden/make_vectors.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle  # noqa: E402
from padra_amd import synth  # noqa: E402

CAP, BASE, TOKENS = 8192, 4097, 4
TABLE_ROWS = (0, 1, 4097, 131071)


def chain_vectors(out):
    d = synth.chain_inputs(TOKENS, outliers=True, seed=901)
    table = synth.bf16_bits(oracle.rope_table(CAP, 128, 1e6))
    pos = np.arange(TOKENS, dtype=np.int32) + BASE
    wx, wy, wst, bad = oracle.residual_rmsnorm(d["x"], d["residual"], d["gamma"], threads=128)
    assert not bad
    wq, wk, bad = oracle.qk_norm_rope(d["q"], d["k"], d["qn"], d["kn"], table, pos)
    assert not bad
    for key in ("x", "residual", "gamma", "q", "k", "v", "qn", "kn"):
        out[f"chain_in_{key}"] = d[key]
    out["chain_positions"] = pos
    out["chain_out_x"], out["chain_out_y"], out["chain_out_stats"] = wx, wy, wst
    out["chain_out_q"], out["chain_out_k"] = wq, wk
    rows = slice(BASE, BASE + TOKENS)
    kc = np.zeros((CAP, 512), np.uint16)
    vc = np.zeros_like(kc)
    oracle.kv_store_bf16(wk, d["v"], kc, vc, pos, CAP)
    out["chain_bf16_kc"], out["chain_bf16_vc"] = kc[rows], vc[rows]
    ck = np.zeros((CAP, 512), np.int8)
    cv = np.zeros_like(ck)
    sc = np.zeros((CAP, 4, 2), np.float32)
    assert not oracle.kv_q8_encode(wk, d["v"], ck, cv, sc, pos, CAP)
    out["chain_q8_kc"], out["chain_q8_vc"], out["chain_q8_scales"] = ck[rows], cv[rows], sc[rows]
    for name, rotate in (("q8_0", True), ("q8_0_norot", False)):
        rk = np.zeros((CAP, 544), np.uint8)
        rv = np.zeros_like(rk)
        assert not oracle.kv_q8_0_encode(wk, d["v"], rk, rv, pos, CAP, rotate=rotate)
        out[f"chain_{name}_kc"], out[f"chain_{name}_vc"] = rk[rows], rv[rows]


def decode_vectors(out):
    seqs, vocab, cap = 3, 16, 8192
    e = synth.chain_inputs(vocab, outliers=False, seed=902)["x"]
    d = synth.chain_inputs(seqs, outliers=False, seed=903)
    ids = np.array([5, 15, 0], np.int32)
    pos = np.array([4097, 0, 8191], np.int32)
    table = synth.bf16_bits(oracle.rope_table(cap, 128, 1e6))
    x0, bad = oracle.embed(e, ids)
    assert not bad
    wx, wy, wst, bad = oracle.residual_rmsnorm(x0, d["residual"], d["gamma"], threads=256)
    assert not bad
    wq, wk, bad = oracle.qk_norm_rope(d["q"], d["k"], d["qn"], d["kn"], table, pos)
    assert not bad
    out["decode_in_embed"], out["decode_in_ids"], out["decode_positions"] = e, ids, pos
    for key in ("residual", "gamma", "q", "k", "v", "qn", "kn"):
        out[f"decode_in_{key}"] = d[key]
    out["decode_out_x"], out["decode_out_y"], out["decode_out_stats"] = wx, wy, wst
    out["decode_out_q"], out["decode_out_k"] = wq, wk
    out["decode_out_krow"] = wk.reshape(seqs, -1)  # each sequence's cache row: rotated K
    out["decode_out_vrow"] = d["v"].reshape(seqs, -1)


def swiglu_vectors(out):
    rng = np.random.default_rng(904)
    gate = synth.bf16_bits((rng.standard_normal((4, 1024)) * 2).astype(np.float32))
    up = synth.bf16_bits((rng.standard_normal((4, 1024)) * 2).astype(np.float32))
    o, bad = oracle.swiglu(gate, up)
    assert not bad
    out["swiglu_in_gate"], out["swiglu_in_up"], out["swiglu_out"] = gate, up, o


def table_vectors(out):
    t = synth.bf16_bits(oracle.rope_table(131072, 128, 1e6))
    out["table_rows"] = np.array(TABLE_ROWS, np.int32)
    out["table_out"] = t[list(TABLE_ROWS)]


def build() -> dict:
    out = {}
    chain_vectors(out)
    decode_vectors(out)
    swiglu_vectors(out)
    table_vectors(out)
    return out


def main():
    out = build()
    np.savez_compressed(os.path.join(HERE, "op_vectors.npz"), **out)
    print({k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
