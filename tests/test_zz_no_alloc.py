"""padra_DecodeAttentionNoAlloc (the decode attention entry point whose workspace is the
library's fixed device array) against padra_DecodeAttention with a caller workspace:
identical outputs and flags, through the C-ABI, on two calls in a row, the second with a
smaller input, for BF16, q8 and q8_0 caches."""
import ctypes

import numpy as np
import pytest
import torch

from padra_amd import abi, ops, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    abi.lib()
    yield
    torch.cuda.synchronize()


def _case(oracle, fmt, seqs, hq, cap, seed):
    """Inputs of one decode batch: queries, a cache binding, decode states (the last
    sequence stopped, so it writes nothing and raises the flag)."""
    rng = np.random.default_rng(seed)
    hkv = 4
    q = torch.from_numpy(synth.bf16_bits(rng.standard_normal((seqs, hq, 128))
                                         .astype(np.float32)).view(np.int16)).cuda()
    scales = None
    if fmt == abi.KV_BF16:
        mk = lambda: torch.from_numpy(synth.bf16_bits(rng.standard_normal((seqs * cap, 512))
                                                      .astype(np.float32)).view(np.int16)).cuda()
        kc, vc = mk(), mk()
    elif fmt == abi.KV_Q8:
        mk = lambda: torch.from_numpy(rng.integers(-127, 128, (seqs * cap, 512))
                                      .astype(np.int8)).cuda()
        kc, vc = mk(), mk()
        scales = torch.from_numpy(rng.uniform(0.005, 0.02, (seqs * cap, hkv, 2))
                                  .astype(np.float32)).cuda()
    else:
        rk = np.zeros((seqs * cap, 544), np.uint8)
        rv = np.zeros((seqs * cap, 544), np.uint8)
        d = synth.chain_inputs(seqs * cap, outliers=True, seed=seed)
        oracle.kv_q8_0_encode(d["k"], d["v"], rk, rv, np.arange(seqs * cap, dtype=np.int32),
                              seqs * cap)
        kc, vc = torch.from_numpy(rk).cuda(), torch.from_numpy(rv).cuda()
    kv = ops.kv_cache(fmt, kc, vc, cap, scales=scales, seq_stride=cap)
    positions = rng.integers(0, cap, seqs).astype(np.int32)
    positions[0] = 0
    states = np.zeros((seqs, 8), np.int32)
    for s, p in enumerate(positions):
        states[s] = [5, p, cap, 10, p, min(p, 1024), 0, 0]
    states[-1, 7] = 1  # stopped
    pos = ops.positions_decode(torch.from_numpy(states).cuda(), maximum=cap)
    return q, kv, pos


def _no_alloc(q, kv, out, pos, bad):
    seqs, hq = q.shape[0], q.shape[1]
    return abi.lib().padra_DecodeAttentionNoAlloc(
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), ctypes.c_void_p(q.data_ptr()),
        ctypes.byref(kv), ctypes.c_void_p(out.data_ptr()), ctypes.byref(pos), seqs, hq, 4, 0, 0,
        ctypes.c_void_p(bad.data_ptr()), 0)


@pytest.mark.parametrize("fmt", [abi.KV_BF16, abi.KV_Q8, abi.KV_Q8_0])
def test_decode_attention_no_alloc_matches(oracle, fmt):
    print(f"[case] decode attention no-alloc fmt={fmt}", flush=True)
    for seqs, hq, cap, seed in ((6, 16, 2048, 300 + fmt), (3, 8, 1024, 310 + fmt)):
        q, kv, pos = _case(oracle, fmt, seqs, hq, cap, seed)
        want = torch.full((seqs, hq, 128), 0x1234, dtype=torch.int16, device="cuda")
        got = torch.full_like(want, 0x1234)
        wbad = torch.zeros(1, dtype=torch.int32, device="cuda")
        gbad = torch.zeros_like(wbad)
        ops.DecodeAttention(q, kv, want, pos, wbad)
        assert _no_alloc(q, kv, got, pos, gbad) == abi.OK
        torch.cuda.synchronize()
        assert wbad.item() == 1 and gbad.item() == 1  # the stopped sequence
        assert torch.equal(got, want), (seqs, hq)
