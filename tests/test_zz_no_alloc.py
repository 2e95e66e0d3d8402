"""padra_DecodeAttentionNoAlloc (the decode attention entry point whose workspace is the
library's fixed device array) against padra_DecodeAttention with a caller workspace:
identical outputs and flags, through the C-ABI, on two calls in a row, the second with a
smaller input, for BF16, q8 and q8_0 caches, global windows and 1024-row local rings, the
reference's split count and the MI355X one (splits = -1); the batch the array is sized for
(64 sequences x 16 query heads x 32 splits); and the process's first call made under HIP
graph capture, replayed at new device-side positions."""
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


def _case(oracle, fmt, seqs, hq, cap, seed, local=False):
    """Inputs of one decode batch: queries, a cache binding, decode states (the last
    sequence stopped, so it writes nothing and raises the flag).  local: 1024-row rings,
    positions up to 4 x the ring (cap is then the ring's 1024 rows)."""
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
    capacity = 4 * cap if local else cap
    positions = rng.integers(0, capacity, seqs).astype(np.int32)
    positions[0] = 0
    states = np.zeros((seqs, 8), np.int32)
    for s, p in enumerate(positions):
        states[s] = [5, p, capacity, 10, p, min(p, 1024), 0, 0]
    states[-1, 7] = 1  # stopped
    st = torch.from_numpy(states).cuda()
    pos = ops.positions_decode(st, maximum=capacity)
    return q, kv, pos, st


def _no_alloc(q, kv, out, pos, bad, local=0, splits=0):
    seqs, hq = q.shape[0], q.shape[1]
    return abi.lib().padra_DecodeAttentionNoAlloc(
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), ctypes.c_void_p(q.data_ptr()),
        ctypes.byref(kv), ctypes.c_void_p(out.data_ptr()), ctypes.byref(pos), seqs, hq, 4,
        int(local), int(splits), ctypes.c_void_p(bad.data_ptr()), 0)


def test_no_alloc_first_call_under_capture(oracle):
    """Collected first in this file: run alone, the capture holds the process's first call
    (the workspace address is looked up inside capture).  The graph is replayed three times,
    each after eager work that moves the decode positions on the device, and every replay
    equals padra_DecodeAttention at those positions."""
    print("[case] decode attention no-alloc under graph capture", flush=True)
    seqs, hq, cap = 5, 16, 2048
    q, kv, pos, st = _case(oracle, abi.KV_BF16, seqs, hq, cap, 333)
    got = torch.zeros((seqs, hq, 128), dtype=torch.int16, device="cuda")
    gbad = torch.zeros(1, dtype=torch.int32, device="cuda")
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            status = _no_alloc(q, kv, got, pos, gbad)
    torch.cuda.synchronize()
    assert status == abi.OK
    for step in range(3):
        # eager work between replays: new positions (and their valid counts) on the device
        p = (st[:, 1] + 97 * (step + 1)) % cap
        st[:, 1] = p
        st[:, 4] = p
        st[:, 5] = torch.clamp(p, max=1024)
        gbad.zero_()
        torch.cuda.synchronize()
        graph.replay()
        want = torch.zeros_like(got)  # the stopped sequence's rows stay as `got` began
        wbad = torch.zeros_like(gbad)
        ops.DecodeAttention(q, kv, want, pos, wbad)
        torch.cuda.synchronize()
        assert gbad.item() == wbad.item() == 1  # the stopped sequence
        assert torch.equal(got, want), step


@pytest.mark.parametrize("local,splits", [(0, 0), (1, 0), (1, -1)])
@pytest.mark.parametrize("fmt", [abi.KV_BF16, abi.KV_Q8, abi.KV_Q8_0])
def test_decode_attention_no_alloc_matches(oracle, fmt, local, splits):
    print(f"[case] decode attention no-alloc fmt={fmt} local={local} splits={splits}",
          flush=True)
    cases = ((40, 16, 1024, 300 + fmt), (6, 8, 1024, 310 + fmt)) if local else \
        ((6, 16, 2048, 300 + fmt), (3, 8, 1024, 310 + fmt))
    for seqs, hq, cap, seed in cases:
        q, kv, pos, _ = _case(oracle, fmt, seqs, hq, cap, seed, local=bool(local))
        want = torch.full((seqs, hq, 128), 0x1234, dtype=torch.int16, device="cuda")
        got = torch.full_like(want, 0x1234)
        wbad = torch.zeros(1, dtype=torch.int32, device="cuda")
        gbad = torch.zeros_like(wbad)
        ops.DecodeAttention(q, kv, want, pos, wbad, local=bool(local), splits=splits)
        assert _no_alloc(q, kv, got, pos, gbad, local, splits) == abi.OK
        torch.cuda.synchronize()
        assert wbad.item() == 1 and gbad.item() == 1  # the stopped sequence
        assert torch.equal(got, want), (seqs, hq)


def test_decode_attention_no_alloc_sizing_batch(oracle):
    """The batch the fixed array is sized for: 64 sequences x 16 query heads x 32 splits
    (global windows of a 2048-row cache, the reference's split count), then the smallest
    batch of that shape that does not fit, which the entry point refuses without writing."""
    print("[case] decode attention no-alloc sizing batch", flush=True)
    seqs, hq, cap = 64, 16, 2048
    used = abi.lib().padra_DecodeAttentionSplits(
        ctypes.byref(abi.KVCache(abi.KV_BF16, None, None, None, cap, 0, 0)), seqs, 4, 0, 0)
    assert used == 32
    q, kv, pos, _ = _case(oracle, abi.KV_BF16, seqs, hq, cap, 350)
    want = torch.full((seqs, hq, 128), 0x1234, dtype=torch.int16, device="cuda")
    got = torch.full_like(want, 0x1234)
    wbad = torch.zeros(1, dtype=torch.int32, device="cuda")
    gbad = torch.zeros_like(wbad)
    ops.DecodeAttention(q, kv, want, pos, wbad)
    assert _no_alloc(q, kv, got, pos, gbad) == abi.OK
    torch.cuda.synchronize()
    assert torch.equal(got, want) and gbad.item() == wbad.item() == 1
    # the smallest batch of this shape whose workspace exceeds the array
    lib = abi.lib()
    big = seqs
    while lib.padra_DecodeAttentionScratch(abi.KV_BF16, big, hq, 32) <= \
            abi.DECODE_ATTENTION_STATIC_FLOATS:
        big += 1
    q2, kv2, pos2, _ = _case(oracle, abi.KV_BF16, big, hq, cap, 351)
    out = torch.full((big, hq, 128), 0x1234, dtype=torch.int16, device="cuda")
    assert _no_alloc(q2, kv2, out, pos2, gbad) == abi.INVALID_ARGUMENT
    torch.cuda.synchronize()
    assert bool((out == 0x1234).all())
