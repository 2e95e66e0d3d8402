"""The per-op golden vectors of tests/golden/op_vectors.npz (written by
tests/golden/make_vectors.py from the oracle): the oracle re-derives every stored output
on the CPU, and the HIP path reproduces the stored bytes on the GPU (chain in each KV
format, the decode step with the gather, SwiGLU, RoPE table rows)."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_vectors  # noqa: E402

from padra_amd import abi, synth  # noqa: E402


def stored():
    with np.load(os.path.join(HERE, "golden", "op_vectors.npz")) as f:
        return {k: f[k] for k in f.files}


def test_vectors_rederived_by_oracle(oracle):
    want = stored()
    got = make_vectors.build()
    assert sorted(got) == sorted(want)
    for key in want:
        assert got[key].dtype == want[key].dtype and np.array_equal(got[key], want[key]), key


def test_vector_layouts():
    """Byte layouts the stored rows follow (src/runtime/kv_cache_layout.h:12-33,
    docs/kv-cache.md): a BF16 row of 4 KV heads is 512 values; a q8 row 512 codes with one
    (k, v) fp32 scale pair per head; a q8_0 row 544 bytes, 16 fp16 block scales then 512
    codes, each block scale the largest |code x scale| of its 32 values over 127."""
    v = stored()
    assert v["chain_bf16_kc"].shape == (4, 512) and v["chain_q8_kc"].shape == (4, 512)
    assert v["chain_q8_scales"].shape == (4, 4, 2)
    row = v["chain_q8_0_norot_vc"][0]
    d = row[:32].view(np.float16).astype(np.float32)
    codes = row[32:].view(np.int8).astype(np.float32).reshape(16, 32)
    vals = synth.bf16_to_f32(v["chain_in_v"][0].reshape(16, 32))
    # unrotated q8_0: d = half(amax / 127), codes within 1 of value / d
    assert np.array_equal(d, (np.abs(vals).max(axis=1) / np.float32(127)).astype(np.float16)
                          .astype(np.float32))
    assert np.all(np.abs(codes - vals / d[:, None]) <= 0.6)  # d is the fp16 of the fp32 scale


@pytest.mark.gpu
def test_vectors_on_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from padra_amd import ops
    v = stored()
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(
        np.int16 if a.dtype == np.uint16 else a.dtype)).cuda()
    h16 = lambda t: t.cpu().numpy().view(np.uint16)
    cap, base = make_vectors.CAP, make_vectors.BASE
    table = ops.RopeTable(cap, 128, 1e6).view(torch.int16).cuda()
    # chain in every KV format
    for fmt, name in ((abi.KV_BF16, "bf16"), (abi.KV_Q8, "q8"), (abi.KV_Q8_0, "q8_0"),
                      (abi.KV_Q8_0_NOROT, "q8_0_norot")):
        print(f"[case] op vectors chain {name}", flush=True)
        x, r, g = dev(v["chain_in_x"]), dev(v["chain_in_residual"]), dev(v["chain_in_gamma"])
        y = torch.empty_like(x)
        st = torch.empty((4, 2), dtype=torch.float32, device="cuda")
        q, k, vv = dev(v["chain_in_q"]), dev(v["chain_in_k"]), dev(v["chain_in_v"])
        if fmt == abi.KV_BF16:
            kc = torch.zeros((cap, 512), dtype=torch.int16, device="cuda")
            sc = None
        elif fmt == abi.KV_Q8:
            kc = torch.zeros((cap, 512), dtype=torch.int8, device="cuda")
            sc = torch.zeros((cap, 4, 2), dtype=torch.float32, device="cuda")
        else:
            kc = torch.zeros((cap, 544), dtype=torch.uint8, device="cuda")
            sc = None
        vc = torch.zeros_like(kc)
        bad = torch.zeros(1, dtype=torch.int32, device="cuda")
        ops.ResidualNormQKRopeStore(x, r, y, g, q, k, vv, dev(v["chain_in_qn"]),
                                    dev(v["chain_in_kn"]), table, ops.positions_base(base),
                                    ops.kv_cache(fmt, kc, vc, cap, scales=sc), bad,
                                    statistics=st)
        torch.cuda.synchronize()
        assert bad.item() == 0
        assert np.array_equal(h16(x), v["chain_out_x"]) and np.array_equal(h16(y), v["chain_out_y"])
        assert np.array_equal(st.cpu().numpy(), v["chain_out_stats"])
        assert np.array_equal(h16(q), v["chain_out_q"]) and np.array_equal(h16(k), v["chain_out_k"])
        rows = slice(base, base + 4)
        view = h16 if fmt == abi.KV_BF16 else (lambda t: t.cpu().numpy())
        assert np.array_equal(view(kc)[rows], v[f"chain_{name}_kc"]), name
        assert np.array_equal(view(vc)[rows], v[f"chain_{name}_vc"]), name
        if sc is not None:
            assert np.array_equal(sc.cpu().numpy()[rows], v["chain_q8_scales"])
    # the decode step: gather + chain, 256-thread tree, one BF16 row per sequence
    print("[case] op vectors decode step", flush=True)
    seqs, dcap = 3, 8192
    pos = v["decode_positions"]
    states = np.zeros((seqs, 8), np.int32)
    for s in range(seqs):
        p = int(pos[s])
        states[s] = [v["decode_in_ids"][s], p, dcap, 10, p, min(p, 1024), 0, 0]
    x = torch.zeros((seqs, 2048), dtype=torch.int16, device="cuda")
    y = torch.empty_like(x)
    q, k = dev(v["decode_in_q"]), dev(v["decode_in_k"])
    kc = torch.zeros((seqs * dcap, 512), dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.EmbedResidualNormQKRopeStore(
        dev(v["decode_in_embed"]), None, x, dev(v["decode_in_residual"]), y,
        dev(v["decode_in_gamma"]), q, k, dev(v["decode_in_v"]), dev(v["decode_in_qn"]),
        dev(v["decode_in_kn"]), table, ops.positions_decode(dev(states), maximum=dcap, vocab=16),
        ops.kv_cache(abi.KV_BF16, kc, vc, dcap, seq_stride=dcap), bad)
    torch.cuda.synchronize()
    assert bad.item() == 0
    assert np.array_equal(h16(x), v["decode_out_x"]) and np.array_equal(h16(y), v["decode_out_y"])
    assert np.array_equal(h16(q), v["decode_out_q"]) and np.array_equal(h16(k), v["decode_out_k"])
    slots = np.arange(seqs) * dcap + pos % dcap
    assert np.array_equal(h16(kc)[slots], v["decode_out_krow"])
    assert np.array_equal(h16(vc)[slots], v["decode_out_vrow"])
    # SwiGLU through the LUT
    print("[case] op vectors SwiGLU", flush=True)
    lut = torch.empty(65536, dtype=torch.int16, device="cuda")
    ops.SiluTableBuild(lut)
    out = torch.empty_like(dev(v["swiglu_in_gate"]))
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    ops.SwiGLU(dev(v["swiglu_in_gate"]), dev(v["swiglu_in_up"]), out, lut, bad)
    torch.cuda.synchronize()
    assert bad.item() == 0 and np.array_equal(h16(out), v["swiglu_out"])
    # the host RoPE table builder's rows
    t = ops.RopeTable(131072, 128, 1e6).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(t[v["table_rows"]], v["table_out"])
