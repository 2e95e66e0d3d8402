"""GPU parity of the KV store/commit/decode, row rotation, SwiGLU and embedding gather
kernels against the CPU oracle, through the C-ABI.  Exact equality throughout."""
import ctypes

import numpy as np
import pytest
import torch

from padra_amd import abi, ops, synth

from attn_tolerance import attn_close as _attn_close, bound_bf16, bound_q8_0

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    abi.lib()
    yield
    torch.cuda.synchronize()


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


def host16(t):
    return t.cpu().numpy().view(np.uint16)


def flag():
    return torch.zeros(1, dtype=torch.int32, device="cuda")


def _cache(fmt, rows):
    if fmt == abi.KV_BF16:
        mk = lambda: torch.zeros((rows, 512), dtype=torch.int16, device="cuda")
        return mk(), mk(), None
    if fmt == abi.KV_Q8:
        mk = lambda: torch.zeros((rows, 512), dtype=torch.int8, device="cuda")
        return mk(), mk(), torch.zeros((rows, 4, 2), dtype=torch.float32, device="cuda")
    mk = lambda: torch.zeros((rows, 544), dtype=torch.uint8, device="cuda")
    return mk(), mk(), None


def _expected(oracle, fmt, k, v, positions, cap, first):
    if fmt == abi.KV_BF16:
        kc = np.zeros((cap, 512), np.uint16)
        vc = np.zeros((cap, 512), np.uint16)
        oracle.kv_store_bf16(k, v, kc, vc, positions, cap, first)
        return kc, vc, None
    if fmt == abi.KV_Q8:
        kc = np.zeros((cap, 512), np.int8)
        vc = np.zeros((cap, 512), np.int8)
        sc = np.zeros((cap, 4, 2), np.float32)
        oracle.kv_q8_encode(k, v, kc, vc, sc, positions, cap, first)
        return kc, vc, sc
    kc = np.zeros((cap, 544), np.uint8)
    vc = np.zeros((cap, 544), np.uint8)
    oracle.kv_q8_0_encode(k, v, kc, vc, positions, cap, first, rotate=fmt == abi.KV_Q8_0)
    return kc, vc, None


def _np(t, fmt):
    a = t.cpu().numpy()
    return a.view(np.uint16) if fmt == abi.KV_BF16 else a


FORMATS = [abi.KV_BF16, abi.KV_Q8, abi.KV_Q8_0, abi.KV_Q8_0_NOROT]


@pytest.mark.parametrize("fmt", FORMATS)
def test_kv_store_then_commit(oracle, fmt):
    """Prefill encode into a chunk buffer (cap = T, positions 0..), then commit of the last
    `cap` rows into a local ring at base 700 (the reference's local-layer sequence)."""
    print(f"[case] kv store+commit fmt={fmt}", flush=True)
    tokens, base, cap, capacity = 1500, 700, 1024, 4096
    d = synth.chain_inputs(tokens, outliers=True, seed=50 + fmt)
    first = max(0, tokens - cap)
    ck, cv, cs = _cache(fmt, tokens)
    bad = flag()
    ops.KVStore(dev(d["k"]), dev(d["v"]), ops.positions_base(0),
                ops.kv_cache(fmt, ck, cv, tokens, scales=cs), bad)
    torch.cuda.synchronize()
    assert bad.item() == 0
    ek, ev, es = _expected(oracle, fmt, d["k"], d["v"], np.arange(tokens, dtype=np.int32),
                           tokens, 0)
    assert np.array_equal(_np(ck, fmt), ek) and np.array_equal(_np(cv, fmt), ev)
    if es is not None:
        assert np.array_equal(cs.cpu().numpy(), es)
    rk, rv, rs = _cache(fmt, cap)
    state = torch.tensor([base, base, tokens, capacity, base, 1, 1, 1], dtype=torch.int32,
                         device="cuda")
    ops.KVCommit(ops.kv_cache(fmt, ck, cv, tokens, scales=cs),
                 ops.kv_cache(fmt, rk, rv, cap, scales=rs, first=first),
                 ops.positions_prefill(state, maximum=capacity), tokens, 4, bad)
    torch.cuda.synchronize()
    assert bad.item() == 0
    slots = (base + np.arange(first, tokens)) % cap
    assert np.array_equal(_np(rk, fmt)[slots], ek[first:])
    assert np.array_equal(_np(rv, fmt)[slots], ev[first:])
    if es is not None:
        assert np.array_equal(rs.cpu().numpy()[slots], es[first:])


@pytest.mark.parametrize("fmt", [abi.KV_Q8, abi.KV_Q8_0, abi.KV_Q8_0_NOROT])
def test_kv_store_nonfinite_pairs(oracle, fmt):
    """The store-only encoder writes a (token, head) pair's K and V rows together or not
    at all (kv_q8.cuh:49-54, kv_q8_native.cuh:70-92): a NaN in K only (token 2 head 1),
    an infinity in V only (token 9 head 3), and a V value of 1e9 whose q8_0 block scale
    overflows fp16 (token 20 head 0, block 2: blocks 0-1 of both written, 2-3 of
    neither).  Caches start filled with a pattern; every byte is compared with the
    oracle's encoders, which follow the reference."""
    print(f"[case] kv store nonfinite pairs fmt={fmt}", flush=True)
    tokens = 37
    d = synth.chain_inputs(tokens, outliers=True, seed=61 + fmt)
    k, v = d["k"].view(np.uint16).copy(), d["v"].view(np.uint16).copy()
    k[2, 1, 40] = 0x7FC0
    v[9, 3, 3] = 0x7F80
    v[20, 0, 70] = 0x4E6E
    ek, ev, es = (np.full_like(a, 0x5A) if a is not None else None
                  for a in _expected(oracle, fmt, k, v, np.arange(tokens, dtype=np.int32),
                                     tokens, 0))
    if es is not None:
        es[:] = 7.0
    pos = np.arange(tokens, dtype=np.int32)
    if fmt == abi.KV_Q8:
        assert oracle.kv_q8_encode(k, v, ek, ev, es, pos, tokens, 0)
    else:
        assert oracle.kv_q8_0_encode(k, v, ek, ev, pos, tokens, 0, rotate=fmt == abi.KV_Q8_0)
    ck, cv, cs = _cache(fmt, tokens)
    ck.fill_(0x5A)
    cv.fill_(0x5A)
    if cs is not None:
        cs.fill_(7.0)
    bad = flag()
    ops.KVStore(dev(k), dev(v), ops.positions_base(0), ops.kv_cache(fmt, ck, cv, tokens, scales=cs),
                bad)
    torch.cuda.synchronize()
    assert bad.item() == 1
    assert np.array_equal(_np(ck, fmt), ek) and np.array_equal(_np(cv, fmt), ev)
    if es is not None:
        assert np.array_equal(cs.cpu().numpy(), es)


def test_kv_store_decode_states(oracle):
    seqs, cap = 8, 128
    rng = np.random.default_rng(3)
    positions = rng.integers(0, cap, seqs).astype(np.int32)
    states = np.zeros((seqs, 8), np.int32)
    for s, p in enumerate(positions):
        states[s] = [1, p, cap, 5, p, min(p, 1024), 0, 0]
    d = synth.chain_inputs(seqs, seed=4)
    kc, vc, _ = _cache(abi.KV_BF16, seqs * cap)
    bad = flag()
    ops.KVStore(dev(d["k"]), dev(d["v"]), ops.positions_decode(torch.from_numpy(states).cuda(),
                                                               maximum=cap),
                ops.kv_cache(abi.KV_BF16, kc, vc, cap, seq_stride=cap), bad)
    torch.cuda.synchronize()
    assert bad.item() == 0
    k3, v3 = host16(kc).reshape(seqs, cap, 512), host16(vc).reshape(seqs, cap, 512)
    for s in range(seqs):
        assert np.array_equal(k3[s, positions[s]], d["k"][s].reshape(-1))
        assert np.array_equal(v3[s, positions[s]], d["v"][s].reshape(-1))


@pytest.mark.parametrize("act", ["bf16", "f32"])
def test_q8_0_dequantize(oracle, act):
    tokens = 300
    d = synth.chain_inputs(tokens, outliers=True, seed=60)
    rk = np.zeros((tokens, 544), np.uint8)
    rv = np.zeros((tokens, 544), np.uint8)
    oracle.kv_q8_0_encode(d["k"], d["v"], rk, rv, np.arange(tokens, dtype=np.int32), tokens)
    wk, wv, _ = oracle.kv_q8_0_dequantize(rk, rv, tokens, 512)
    if act == "bf16":
        ok = torch.empty((tokens, 512), dtype=torch.int16, device="cuda")
    else:
        ok = torch.empty((tokens, 512), dtype=torch.float32, device="cuda")
    ov = torch.empty_like(ok)
    bad = flag()
    ops.KvQ8_0Dequantize(dev(rk), dev(rv), ok, ov, bad)
    torch.cuda.synchronize()
    assert bad.item() == 0
    gk = host16(ok) if act == "bf16" else synth.bf16_bits(ok.cpu().numpy())
    gv = host16(ov) if act == "bf16" else synth.bf16_bits(ov.cpu().numpy())
    assert np.array_equal(gk, wk) and np.array_equal(gv, wv)
    bad_rows = rk.copy()
    bad_rows[5, 32 + 7] = 0x80  # code -128
    ops.KvQ8_0Dequantize(dev(bad_rows), dev(rv), ok, ov, bad)
    torch.cuda.synchronize()
    assert bad.item() == 1


def test_q8_0_dequantize_prefix(oracle):
    """Ring of 64 rows, PrefillState base 40: rows 0..39 decoded, the rest untouched; an
    invalid state writes nothing."""
    cap, base = 64, 40
    d = synth.chain_inputs(cap, seed=61)
    rk = np.zeros((cap, 544), np.uint8)
    rv = np.zeros((cap, 544), np.uint8)
    oracle.kv_q8_0_encode(d["k"], d["v"], rk, rv, np.arange(cap, dtype=np.int32), cap)
    wk, wv, _ = oracle.kv_q8_0_dequantize(rk, rv, cap, 512)
    ok = torch.full((cap, 512), 7, dtype=torch.int16, device="cuda")
    ov = torch.full((cap, 512), 7, dtype=torch.int16, device="cuda")
    state = torch.tensor([base, base, 8, cap, base, 1, 1, 1], dtype=torch.int32, device="cuda")
    bad = flag()
    ops.KvQ8_0DequantizePrefix(dev(rk), dev(rv), ok, ov, ops.positions_prefill(state, maximum=cap),
                               8, bad)
    torch.cuda.synchronize()
    assert bad.item() == 0
    assert np.array_equal(host16(ok)[:base], wk[:base]) and np.array_equal(host16(ov)[:base], wv[:base])
    assert np.all(host16(ok)[base:] == 7)
    bad_state = torch.tensor([base, base, 8, cap, base + 1, 1, 1, 1], dtype=torch.int32,
                             device="cuda")
    ok.fill_(7)
    ops.KvQ8_0DequantizePrefix(dev(rk), dev(rv), ok, ov,
                               ops.positions_prefill(bad_state, maximum=cap), 8, bad)
    torch.cuda.synchronize()
    assert bad.item() == 1 and np.all(host16(ok) == 7)


@pytest.mark.parametrize("value", [False, True])
def test_rotate_rows(oracle, value):
    rows = 96
    rng = np.random.default_rng(7)
    x = synth.bf16_bits(rng.standard_normal((rows, 128)))
    want = []
    for r in range(rows):
        xf = synth.bf16_to_f32(x[r])
        if value:
            out = np.concatenate([oracle.hadamard(xf[:64], .125), oracle.hadamard(xf[64:], .125)])
        else:
            out = oracle.hadamard(xf, .08838834764831845)
        want.append(synth.bf16_bits(out))
    t = dev(x)
    bad = flag()
    ops.RotateRows(t, bad, value=value)
    torch.cuda.synchronize()
    assert np.array_equal(host16(t), np.stack(want))


def test_silu_table_exhaustive(oracle):
    table = torch.empty(65536, dtype=torch.int16, device="cuda")
    ops.SiluTableBuild(table)
    torch.cuda.synchronize()
    got = host16(table)
    want = oracle.silu_table()
    g = synth.bf16_to_f32(np.arange(65536, dtype=np.uint16))
    finite = np.isfinite(g)
    assert np.array_equal(got[finite], want[finite])


@pytest.mark.parametrize("act", ["bf16", "f32"])
def test_swiglu_all_gates(oracle, act):
    """Every BF16 gate value (finite ones), each with four up values, plus the config-3
    distribution; the kernel's closed forms outside the staged table span included."""
    table = torch.empty(65536, dtype=torch.int16, device="cuda")
    ops.SiluTableBuild(table)
    gates = np.arange(65536, dtype=np.uint16)
    gates = gates[np.isfinite(synth.bf16_to_f32(gates))]
    rng = np.random.default_rng(11)
    gate = np.repeat(gates, 4)
    up = synth.bf16_bits(rng.standard_normal(gate.size) * 4)
    n = gate.size // 8 * 8
    gate, up = gate[:n], up[:n]
    want, wbad = oracle.swiglu(gate, up)
    if act == "bf16":
        tg, tu = dev(gate), dev(up)
    else:
        tg = torch.from_numpy(synth.bf16_to_f32(gate)).cuda()
        tu = torch.from_numpy(synth.bf16_to_f32(up)).cuda()
    out = torch.empty_like(tg)
    bad = flag()
    ops.SwiGLU(tg, tu, out, table, bad)
    torch.cuda.synchronize()
    got = host16(out) if act == "bf16" else synth.bf16_bits(out.cpu().numpy())
    assert np.array_equal(got, want)
    assert bool(bad.item()) == wbad


def test_swiglu_config3_shape_in_place(oracle):
    d = synth.swiglu_inputs(tokens=256, seed=0)  # 2048 rows x 1024, expert-permuted
    want, _ = oracle.swiglu(d["gate"], d["up"])
    table = torch.empty(65536, dtype=torch.int16, device="cuda")
    ops.SiluTableBuild(table)
    g = dev(d["gate"])
    bad = flag()
    ops.SwiGLU(g, dev(d["up"]), g, table, bad)  # in place over gate, as the reference
    torch.cuda.synchronize()
    assert np.array_equal(host16(g), want) and bad.item() == 0
    gate = d["gate"].copy()
    gate[3, 5] = 0x7FC0  # NaN gate: flag raised, element left as it was
    g = dev(gate)
    ops.SwiGLU(g, dev(d["up"]), g, table, bad)
    torch.cuda.synchronize()
    assert bad.item() == 1 and host16(g)[3, 5] == 0x7FC0


def test_embed_sources(oracle):
    rng = np.random.default_rng(12)
    vocab, hidden = 5000, 2048
    table_bits = synth.bf16_bits(rng.standard_normal((vocab, hidden)) * 0.02)
    table = dev(table_bits)
    ids = synth.zipf_ids(64, vocab, seed=1)
    # ids
    out = torch.empty((64, hidden), dtype=torch.int16, device="cuda")
    bad = flag()
    ops.Embed(table, out, bad, ids=torch.from_numpy(ids).cuda())
    torch.cuda.synchronize()
    want, _ = oracle.embed(table_bits, ids)
    assert np.array_equal(host16(out), want) and bad.item() == 0
    # prompt through a PrefillState (prompt_offset 10)
    prompt = np.concatenate([np.zeros(10, np.int32), ids])
    state = torch.tensor([10, 10, 64, 4096, 10, 1, 1, 1], dtype=torch.int32, device="cuda")
    out.zero_()
    ops.Embed(table, out, bad, ids=torch.from_numpy(prompt).cuda(),
              positions=ops.positions_prefill(state, maximum=4096), tokens=64)
    torch.cuda.synchronize()
    assert np.array_equal(host16(out), want) and bad.item() == 0
    # decode states, one token out of range: that row is left untouched, flag raised
    states = np.zeros((64, 8), np.int32)
    for s in range(64):
        states[s] = [ids[s], 7, 64, 3, 7, 7, 0, 0]
    states[9, 0] = vocab + 3
    out32 = torch.full((64, hidden), 9.0, dtype=torch.float32, device="cuda")
    ops.Embed(table, out32, bad, positions=ops.positions_decode(torch.from_numpy(states).cuda(),
                                                                 maximum=64, vocab=vocab * 2))
    torch.cuda.synchronize()
    got = out32.cpu().numpy()
    assert bad.item() == 1
    assert np.all(got[9] == 9.0)
    keep = [s for s in range(64) if s != 9]
    assert np.array_equal(synth.bf16_bits(got[keep]), want[keep])


# ---- expert combine ----------------------------------------------------------------------

def _combine_inputs(rows, hidden, seed):
    rng = np.random.default_rng(seed)
    d = synth.chain_inputs(rows, hidden=hidden, outliers=True, seed=seed)
    down = synth.bf16_bits((rng.standard_normal((rows, 8, hidden)) * 0.5).astype(np.float32))
    w = rng.dirichlet(np.ones(8), rows).astype(np.float32)
    return d, down, w


@pytest.mark.parametrize("residual", [True, False])
@pytest.mark.parametrize("act", ["bf16", "f32"])
def test_combine(oracle, residual, act):
    print(f"[case] combine residual={residual} act={act}", flush=True)
    rows, hidden = 300, 2304
    d, down, w = _combine_inputs(rows, hidden, 31)
    want, want_bad = oracle.combine(d["x"], down, w, residual=residual)
    if act == "bf16":
        x, dn = dev(d["x"]), dev(down)
    else:
        x = torch.from_numpy(synth.bf16_to_f32(d["x"])).cuda()
        dn = torch.from_numpy(synth.bf16_to_f32(down)).cuda()
    bad = flag()
    ops.Combine(x, dn, torch.from_numpy(w).cuda(), bad, residual=residual)
    torch.cuda.synchronize()
    got = host16(x) if act == "bf16" else synth.bf16_bits(x.cpu().numpy())
    assert np.array_equal(got, want)
    assert bool(bad.item()) == want_bad


@pytest.mark.parametrize("hidden,rows", [(2048, 67), (2304, 67), (4608, 67), (1024, 5), (2048, 2048)])
@pytest.mark.parametrize("fp8", [True, False])
def test_combine_norm(oracle, hidden, rows, fp8):
    """Combine + RMSNorm (+ FP8) against the oracle bit for bit; 2048 x 2048 is the size the
    bench times."""
    print(f"[case] combine norm hidden={hidden} rows={rows} fp8={fp8}", flush=True)
    d, down, w = _combine_inputs(rows, hidden, 32 + hidden)
    want_x, want_y, want_p, want_s, want_st, want_bad = oracle.combine_norm(
        d["x"], down, w, d["gamma"], fp8=fp8)
    x = dev(d["x"])
    y = torch.empty_like(x)
    packed = torch.empty((rows, hidden), dtype=torch.uint8, device="cuda") if fp8 else None
    scales = torch.empty(rows, dtype=torch.float32, device="cuda") if fp8 else None
    st = torch.empty(2, dtype=torch.float32, device="cuda")
    bad = flag()
    ops.CombineNorm(x, dev(down), torch.from_numpy(w).cuda(), y, dev(d["gamma"]), bad,
                    packed=packed, scales=scales, statistics=st)
    torch.cuda.synchronize()
    assert np.array_equal(host16(x), want_x) and np.array_equal(host16(y), want_y)
    assert np.array_equal(st.cpu().numpy(), want_st)
    if fp8:
        assert np.array_equal(packed.cpu().numpy(), want_p)
        assert np.array_equal(scales.cpu().numpy(), want_s)
    assert bool(bad.item()) == want_bad


def test_combine_nonfinite_sets_bad(oracle):
    rows, hidden = 4, 2304
    d, down, w = _combine_inputs(rows, hidden, 33)
    down = down.copy()
    down[2, 3, 17] = 0x7F80
    want_x, want_bad = oracle.combine(d["x"], down, w)
    assert want_bad
    x = dev(d["x"])
    bad = flag()
    ops.Combine(x, dev(down), torch.from_numpy(w).cuda(), bad)
    torch.cuda.synchronize()
    assert bad.item() == 1 and np.array_equal(host16(x), want_x)
    y = torch.empty_like(x)
    bad2 = flag()
    ops.CombineNorm(dev(d["x"]), dev(down), torch.from_numpy(w).cuda(), y, dev(d["gamma"]), bad2)
    torch.cuda.synchronize()
    assert bad2.item() == 1


# ---- local-ring checkpoint capture ----------------------------------------------------------

@pytest.mark.parametrize("fmt", FORMATS)
def test_kv_checkpoint_capture(oracle, fmt):
    """Snapshot of a 1024-row ring before a 600-row chunk at base 700, anchor 1250: slots
    from the chunk, from the old ring and (positions < 0 never occur here) bit copies."""
    print(f"[case] checkpoint fmt={fmt}", flush=True)
    base, tokens, anchor, capacity = 700, 600, 1250, 4096
    rng = np.random.default_rng(70 + fmt)
    def planes(rows):
        if fmt == abi.KV_BF16:
            return [rng.integers(0, 65536, (rows, 512), dtype=np.uint16) for _ in range(2)]
        if fmt == abi.KV_Q8:
            return [rng.integers(-127, 128, (rows, 512), dtype=np.int8) for _ in range(2)] + \
                [rng.standard_normal((rows, 4, 2)).astype(np.float32)]
        return [rng.integers(0, 256, (rows, 544), dtype=np.uint8) for _ in range(2)]
    old, cur = planes(1024), planes(tokens)
    state = np.array([base, base, tokens, capacity, base, 1, 1, 1], np.int32)
    want = oracle.kv_checkpoint(old, cur, state, tokens, anchor)
    todev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.uint8)).cuda()
    o, c = [todev(a) for a in old], [todev(a) for a in cur]
    sv = [torch.full_like(t, 0xAB) for t in o]
    sc = lambda lst: lst[2] if len(lst) > 2 else None
    ring = ops.kv_cache(fmt, o[0], o[1], 1024, scales=sc(o))
    chunk = ops.kv_cache(fmt, c[0], c[1], tokens, scales=sc(c))
    saved = ops.kv_cache(fmt, sv[0], sv[1], 1024, scales=sc(sv))
    st = torch.from_numpy(state).cuda()
    bad = flag()
    ops.KVCheckpointCapture(ring, chunk, saved, ops.positions_prefill(st, maximum=capacity),
                            tokens, anchor, bad)
    torch.cuda.synchronize()
    assert bad.item() == 0
    for got, w in zip(sv, want):
        assert np.array_equal(got.cpu().numpy().reshape(w.shape), w)
    # a capture whose anchor lies outside the chunk writes nothing and raises the flag
    for t in sv:
        t.fill_(0xAB)
    ops.KVCheckpointCapture(ring, chunk, saved, ops.positions_prefill(st, maximum=capacity),
                            tokens, base, bad)
    torch.cuda.synchronize()
    assert bad.item() == 1 and all(bool((t == 0xAB).all()) for t in sv)
    # with the flag already raised, a valid capture copies nothing
    ops.KVCheckpointCapture(ring, chunk, saved, ops.positions_prefill(st, maximum=capacity),
                            tokens, anchor, bad)
    torch.cuda.synchronize()
    assert all(bool((t == 0xAB).all()) for t in sv)


# ---- decode attention --------------------------------------------------------------------

@pytest.mark.parametrize("hq,local,splits", [(16, False, 0), (32, False, 0), (16, True, 0),
                                             (16, False, 5), (4, False, 0), (8, True, 0)])
def test_decode_attention(oracle, hq, local, splits):
    """Ragged decode batch against the oracle's attention at each sequence's position,
    within the _attn_close tolerance (the reference's tensor-core order and CUDA expf/logf
    differ from any other implementation by fp32 ulps before the BF16 roundings)."""
    print(f"[case] decode attention hq={hq} local={local} splits={splits}", flush=True)
    seqs, hkv, capacity = 6, 4, 4096
    cap = 1024 if local else capacity
    rng = np.random.default_rng(90 + hq + local + splits)
    positions = rng.integers(0, capacity, seqs).astype(np.int32)
    positions[0], positions[1] = 0, 33
    q = synth.bf16_bits((rng.standard_normal((seqs, hq, 128)) * 2).astype(np.float32))
    kc = synth.bf16_bits(rng.standard_normal((seqs, cap, hkv * 128)).astype(np.float32))
    vc = synth.bf16_bits(rng.standard_normal((seqs, cap, hkv * 128)).astype(np.float32))
    states = np.zeros((seqs, 8), np.int32)
    for s, p in enumerate(positions):
        states[s] = [5, p, capacity, 10, p, min(p, 1024), 0, 0]
    out = torch.empty((seqs, hq, 128), dtype=torch.int16, device="cuda")
    bad = flag()
    kv = ops.kv_cache(abi.KV_BF16, dev(kc.reshape(seqs * cap, -1)), dev(vc.reshape(seqs * cap, -1)),
                      cap, seq_stride=cap)
    st = torch.from_numpy(states).cuda()
    ops.DecodeAttention(dev(q), kv, out, ops.positions_decode(st, maximum=capacity), bad,
                        kv_heads=hkv, local=local, splits=splits)
    torch.cuda.synchronize()
    assert bad.item() == 0
    got = host16(out)
    worst = 0
    for s in range(seqs):
        want, used, wbad = oracle.decode_attention(q[s], kc[s], vc[s], positions[s],
                                                   local=local, splits=splits)
        assert not wbad
        close, d = _attn_close(got[s], want,
                               bound_bf16(q[s], kc[s], vc[s], positions[s], local, used))
        assert close.all(), s
        worst = max(worst, int(d.max()))
        if d.max() > 1:
            i = np.unravel_index(np.argmax(d), d.shape)
            gv, wv = synth.bf16_to_f32(got[s])[i], synth.bf16_to_f32(want)[i]
            hm = np.abs(synth.bf16_to_f32(want)[i[0]]).max()
            print(f"  seq {s} pos {positions[s]} at {i}: got {gv} want {wv} head max {hm} "
                  f"count>1: {(d > 1).sum()}", flush=True)
    print(f"  max BF16 ulp difference {worst}", flush=True)


def test_decode_attention_f32_and_invalid(oracle):
    seqs, hq, hkv, cap = 3, 16, 4, 512
    rng = np.random.default_rng(97)
    positions = np.array([100, 511, 7], np.int32)
    q = synth.bf16_bits(rng.standard_normal((seqs, hq, 128)).astype(np.float32))
    kc = synth.bf16_bits(rng.standard_normal((seqs, cap, hkv * 128)).astype(np.float32))
    vc = synth.bf16_bits(rng.standard_normal((seqs, cap, hkv * 128)).astype(np.float32))
    states = np.zeros((seqs, 8), np.int32)
    for s, p in enumerate(positions):
        states[s] = [5, p, cap, 10, p, min(p, 1024), 0, 0]
    states[2, 6] = 1  # eos: not admitted, nothing written, flag raised
    out = torch.full((seqs, hq, 128), 7.0, dtype=torch.float32, device="cuda")
    bad = flag()
    kv = ops.kv_cache(abi.KV_BF16, dev(kc.reshape(seqs * cap, -1)), dev(vc.reshape(seqs * cap, -1)),
                      cap, seq_stride=cap)
    ops.DecodeAttention(torch.from_numpy(synth.bf16_to_f32(q)).cuda(), kv, out,
                        ops.positions_decode(torch.from_numpy(states).cuda(), maximum=cap), bad)
    torch.cuda.synchronize()
    assert bad.item() == 1
    got = out.cpu().numpy()
    assert np.all(got[2] == 7.0)
    for s in range(2):
        want, used, _ = oracle.decode_attention(q[s], kc[s], vc[s], positions[s])
        assert _attn_close(synth.bf16_bits(got[s]), want,
                           bound_bf16(q[s], kc[s], vc[s], positions[s], False, used))[0].all()



@pytest.mark.parametrize("fmt", [abi.KV_BF16, abi.KV_Q8, abi.KV_Q8_0])
def test_decode_attention_tuned_splits(oracle, fmt):
    """splits = -1 on a local ring of 40 sequences runs the MI355X count (6 / 12 / 6 splits
    for BF16 / q8 / q8_0, against the reference's 16): the result is the oracle's at that
    count, within the _attn_close tolerance."""
    seqs, hq, hkv, capacity, cap = 40, 16, 4, 4096, 1024
    kv_probe = abi.KVCache(fmt, None, None, None, cap, 0, 0)
    used = abi.lib().padra_DecodeAttentionSplits(ctypes.byref(kv_probe), seqs, hkv, 1, -1)
    print(f"[case] decode attention tuned splits fmt={fmt} -> {used}", flush=True)
    assert used == (12 if fmt == abi.KV_Q8 else 6)
    rng = np.random.default_rng(150 + fmt)
    positions = rng.integers(0, capacity, seqs).astype(np.int32)
    positions[0], positions[1], positions[2] = 0, 33, 1023
    q = synth.bf16_bits((rng.standard_normal((seqs, hq, 128)) * 2).astype(np.float32))
    states = np.zeros((seqs, 8), np.int32)
    for s, p in enumerate(positions):
        states[s] = [5, p, capacity, 10, p, min(p, 1024), 0, 0]
    if fmt == abi.KV_Q8_0:
        rk = np.zeros((seqs, cap, 544), np.uint8)
        rv = np.zeros((seqs, cap, 544), np.uint8)
        for s in range(seqs):
            d = synth.chain_inputs(cap, outliers=True, seed=300 + s)
            oracle.kv_q8_0_encode(d["k"], d["v"], rk[s], rv[s], np.arange(cap, dtype=np.int32),
                                  cap)
        kv = ops.kv_cache(fmt, dev(rk.reshape(seqs * cap, 544)), dev(rv.reshape(seqs * cap, 544)),
                          cap, seq_stride=cap)
    elif fmt == abi.KV_Q8:
        codes_k = rng.integers(-127, 128, (seqs, cap, hkv * 128)).astype(np.int8)
        codes_v = rng.integers(-127, 128, (seqs, cap, hkv * 128)).astype(np.int8)
        scales = rng.uniform(0.005, 0.02, (seqs, cap, hkv, 2)).astype(np.float32)
        kc = synth.bf16_bits(codes_k.reshape(seqs, cap, hkv, 128).astype(np.float32) *
                             scales[..., 0:1]).reshape(seqs, cap, -1)
        vc = synth.bf16_bits(codes_v.reshape(seqs, cap, hkv, 128).astype(np.float32) *
                             scales[..., 1:2]).reshape(seqs, cap, -1)
        kv = ops.kv_cache(fmt, torch.from_numpy(codes_k.reshape(seqs * cap, -1)).cuda(),
                          torch.from_numpy(codes_v.reshape(seqs * cap, -1)).cuda(), cap,
                          scales=torch.from_numpy(scales.reshape(seqs * cap, hkv, 2)).cuda(),
                          seq_stride=cap)
    else:
        kc = synth.bf16_bits(rng.standard_normal((seqs, cap, hkv * 128)).astype(np.float32))
        vc = synth.bf16_bits(rng.standard_normal((seqs, cap, hkv * 128)).astype(np.float32))
        kv = ops.kv_cache(fmt, dev(kc.reshape(seqs * cap, -1)), dev(vc.reshape(seqs * cap, -1)),
                          cap, seq_stride=cap)
    out = torch.empty((seqs, hq, 128), dtype=torch.int16, device="cuda")
    bad = flag()
    ops.DecodeAttention(dev(q), kv, out, ops.positions_decode(torch.from_numpy(states).cuda(),
                                                              maximum=capacity),
                        bad, kv_heads=hkv, local=True, splits=-1)
    torch.cuda.synchronize()
    assert bad.item() == 0
    got = host16(out)
    worst = 0
    for s in range(seqs):
        if fmt == abi.KV_Q8_0:
            want, wsplits, wbad = oracle.decode_attention_q8_0(q[s], rk[s], rv[s], positions[s],
                                                               local=True, splits=used)
        else:
            want, wsplits, wbad = oracle.decode_attention(q[s], kc[s], vc[s], positions[s],
                                                          local=True, splits=used)
        # the splits the oracle ran: the count, capped by the window's tiles (32 keys; 128
        # for q8_0)
        tile = 128 if fmt == abi.KV_Q8_0 else 32
        assert not wbad and wsplits == min(used, (min(positions[s] + 1, cap) + tile - 1) // tile)
        if fmt == abi.KV_Q8_0:
            b = bound_q8_0(q[s], rk[s], rv[s], positions[s], True, wsplits)
        else:
            b = bound_bf16(q[s], kc[s], vc[s], positions[s], True, wsplits)
        close, d = _attn_close(got[s], want, b)
        worst = max(worst, int(d.max()))
        assert close.all(), (s, int(d.max()))
    print(f"  max BF16 ulp difference {worst}", flush=True)


@pytest.mark.parametrize("hq,local", [(16, False), (32, False), (16, True), (4, False),
                                      (8, True)])
def test_decode_attention_q8_0(oracle, hq, local):
    """q8_0 caches (rotated v2) against the oracle's EncodeQuery/Split/Merge, within the
    _attn_close tolerance (CUDA expf/logf against any other implementation)."""
    print(f"[case] decode attention q8_0 hq={hq} local={local}", flush=True)
    seqs, hkv, capacity = 5, 4, 4096
    cap = 1024 if local else capacity
    rng = np.random.default_rng(110 + hq + local)
    positions = rng.integers(0, capacity, seqs).astype(np.int32)
    positions[0], positions[1] = 0, 200
    q = synth.bf16_bits((rng.standard_normal((seqs, hq, 128)) * 2).astype(np.float32))
    rk = np.zeros((seqs, cap, 544), np.uint8)
    rv = np.zeros((seqs, cap, 544), np.uint8)
    for s in range(seqs):
        d = synth.chain_inputs(cap, outliers=True, seed=200 + s)
        oracle.kv_q8_0_encode(d["k"], d["v"], rk[s], rv[s], np.arange(cap, dtype=np.int32), cap)
    states = np.zeros((seqs, 8), np.int32)
    for s, p in enumerate(positions):
        states[s] = [5, p, capacity, 10, p, min(p, 1024), 0, 0]
    out = torch.empty((seqs, hq, 128), dtype=torch.int16, device="cuda")
    bad = flag()
    kv = ops.kv_cache(abi.KV_Q8_0, dev(rk.reshape(seqs * cap, 544)), dev(rv.reshape(seqs * cap, 544)),
                      cap, seq_stride=cap)
    ops.DecodeAttention(dev(q), kv, out, ops.positions_decode(torch.from_numpy(states).cuda(),
                                                              maximum=capacity),
                        bad, kv_heads=hkv, local=local)
    torch.cuda.synchronize()
    assert bad.item() == 0
    got = host16(out)
    worst = 0
    for s in range(seqs):
        want, used, wbad = oracle.decode_attention_q8_0(q[s], rk[s], rv[s], positions[s],
                                                        local=local)
        assert not wbad
        close, d = _attn_close(got[s], want,
                               bound_q8_0(q[s], rk[s], rv[s], positions[s], local, used))
        worst = max(worst, int(d.max()))
        assert close.all(), (s, int(d.max()))
    print(f"  max BF16 ulp difference {worst}", flush=True)


@pytest.mark.parametrize("hq,local", [(16, False), (16, True), (4, False), (8, True)])
def test_decode_attention_q8(oracle, hq, local):
    """q8 caches (per-head fp32 scale): the split reads bf16(code * scale) rows
    (kv_q8::Decode), so the oracle is the BF16 attention over the decoded cache; within the
    _attn_close tolerance."""
    print(f"[case] decode attention q8 hq={hq} local={local}", flush=True)
    seqs, hkv, capacity = 4, 4, 4096
    cap = 1024 if local else capacity
    rng = np.random.default_rng(130 + local)
    positions = rng.integers(0, capacity, seqs).astype(np.int32)
    positions[0] = 3
    q = synth.bf16_bits((rng.standard_normal((seqs, hq, 128)) * 2).astype(np.float32))
    codes_k = rng.integers(-127, 128, (seqs, cap, hkv * 128)).astype(np.int8)
    codes_v = rng.integers(-127, 128, (seqs, cap, hkv * 128)).astype(np.int8)
    scales = (rng.uniform(0.005, 0.02, (seqs, cap, hkv, 2))).astype(np.float32)
    dk = synth.bf16_bits(codes_k.reshape(seqs, cap, hkv, 128).astype(np.float32) *
                         scales[..., 0:1]).reshape(seqs, cap, -1)
    dv = synth.bf16_bits(codes_v.reshape(seqs, cap, hkv, 128).astype(np.float32) *
                         scales[..., 1:2]).reshape(seqs, cap, -1)
    states = np.zeros((seqs, 8), np.int32)
    for s, p in enumerate(positions):
        states[s] = [5, p, capacity, 10, p, min(p, 1024), 0, 0]
    out = torch.empty((seqs, hq, 128), dtype=torch.int16, device="cuda")
    bad = flag()
    kv = ops.kv_cache(abi.KV_Q8, torch.from_numpy(codes_k.reshape(seqs * cap, -1)).cuda(),
                      torch.from_numpy(codes_v.reshape(seqs * cap, -1)).cuda(), cap,
                      scales=torch.from_numpy(scales.reshape(seqs * cap, hkv, 2)).cuda(),
                      seq_stride=cap)
    ops.DecodeAttention(dev(q), kv, out, ops.positions_decode(torch.from_numpy(states).cuda(),
                                                              maximum=capacity),
                        bad, kv_heads=hkv, local=local)
    torch.cuda.synchronize()
    assert bad.item() == 0
    got = host16(out)
    for s in range(seqs):
        want, used, wbad = oracle.decode_attention(q[s], dk[s], dv[s], positions[s], local=local)
        assert not wbad
        close, d = _attn_close(got[s], want,
                               bound_bf16(q[s], dk[s], dv[s], positions[s], local, used))
        assert close.all(), (s, int(d.max()))
    # a -128 code inside the window raises the flag: in the window's first tile (whole,
    # for a window of 32 keys or more) and at the current position
    if not local and positions[1] >= 64:
        codes_k[1, 0, 5] = -128
        kv1 = ops.kv_cache(abi.KV_Q8, torch.from_numpy(codes_k.reshape(seqs * cap, -1)).cuda(),
                           torch.from_numpy(codes_v.reshape(seqs * cap, -1)).cuda(), cap,
                           scales=torch.from_numpy(scales.reshape(seqs * cap, hkv, 2)).cuda(),
                           seq_stride=cap)
        bad.zero_()
        ops.DecodeAttention(dev(q), kv1, out,
                            ops.positions_decode(torch.from_numpy(states).cuda(),
                                                 maximum=capacity), bad, kv_heads=hkv)
        torch.cuda.synchronize()
        assert bad.item() == 1
        codes_k[1, 0, 5] = 0
        bad.zero_()
    codes_k[1, positions[1] % cap, 5] = -128
    kv2 = ops.kv_cache(abi.KV_Q8, torch.from_numpy(codes_k.reshape(seqs * cap, -1)).cuda(),
                       torch.from_numpy(codes_v.reshape(seqs * cap, -1)).cuda(), cap,
                       scales=torch.from_numpy(scales.reshape(seqs * cap, hkv, 2)).cuda(),
                       seq_stride=cap)
    ops.DecodeAttention(dev(q), kv2, out, ops.positions_decode(torch.from_numpy(states).cuda(),
                                                               maximum=capacity),
                        bad, kv_heads=hkv, local=local)
    torch.cuda.synchronize()
    assert bad.item() == 1


@pytest.mark.parametrize("fmt,seqs", [(abi.KV_BF16, 7), (abi.KV_Q8, 7), (abi.KV_Q8_0, 7),
                                      (abi.KV_BF16, 512), (abi.KV_BF16, 513),
                                      (abi.KV_Q8_0, 513)])
def test_decode_attention_dispatch_order(fmt, seqs):
    """Several sequences on a global cache run their split waves longest window first (up
    to 512 sequences; more run in sequence order); every output equals the same sequence
    decoded alone, bit for bit.  7 sequences: windows of 1, 6, 101, 2048 and twice 3001
    keys (a tie) plus one at the last row of 4096; 512 and 513: random windows of a
    64-row cache, every sequence with position 10 (ties), each sixteenth checked alone."""
    print(f"[case] decode attention dispatch order fmt={fmt} seqs={seqs}", flush=True)
    hq, hkv = 16, 4
    rng = np.random.default_rng(150 + fmt + seqs)
    if seqs == 7:
        cap = 4096
        positions = np.array([5, 3000, 100, 3000, 0, 2047, cap - 1], np.int32)
        check = range(seqs)
    else:
        cap = 64
        positions = rng.integers(0, cap, seqs).astype(np.int32)
        positions[::5] = 10
        check = range(0, seqs, 16)
    q = synth.bf16_bits((rng.standard_normal((seqs, hq, 128)) * 2).astype(np.float32))
    if fmt == abi.KV_BF16:
        kc = synth.bf16_bits(rng.standard_normal((seqs * cap, hkv * 128)).astype(np.float32))
        vc = synth.bf16_bits(rng.standard_normal((seqs * cap, hkv * 128)).astype(np.float32))
        kc, vc, sc = kc.view(np.int16), vc.view(np.int16), None
    elif fmt == abi.KV_Q8:
        kc = rng.integers(-127, 128, (seqs * cap, hkv * 128)).astype(np.int8)
        vc = rng.integers(-127, 128, (seqs * cap, hkv * 128)).astype(np.int8)
        sc = rng.uniform(0.005, 0.02, (seqs * cap, hkv, 2)).astype(np.float32)
    else:
        kc = rng.integers(-127, 128, (seqs * cap, 544)).astype(np.int8)
        vc = rng.integers(-127, 128, (seqs * cap, 544)).astype(np.int8)
        kc[:, :32].view(np.int16)[:] = 0x2400  # block scales 1/64 (fp16)
        vc[:, :32].view(np.int16)[:] = 0x2400
        sc = None
    states = np.zeros((seqs, 8), np.int32)
    for i, p in enumerate(positions):
        states[i] = [5, p, cap, 10, p, min(p, 1024), 0, 0]
    kd, vd = torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda()
    sd = torch.from_numpy(sc).cuda() if sc is not None else None
    qd = dev(q)
    out = torch.empty((seqs, hq, 128), dtype=torch.int16, device="cuda")
    bad = flag()
    ops.DecodeAttention(qd, ops.kv_cache(fmt, kd, vd, cap, scales=sd, seq_stride=cap), out,
                        ops.positions_decode(torch.from_numpy(states).cuda(), maximum=cap),
                        bad, kv_heads=hkv)
    torch.cuda.synchronize()
    assert bad.item() == 0
    for i in check:
        one = torch.empty((1, hq, 128), dtype=torch.int16, device="cuda")
        rows = slice(i * cap, (i + 1) * cap)
        kv = ops.kv_cache(fmt, kd[rows], vd[rows], cap,
                          scales=sd[rows] if sd is not None else None)
        ops.DecodeAttention(qd[i:i + 1], kv, one,
                            ops.positions_decode(torch.from_numpy(states[i:i + 1]).cuda(),
                                                 maximum=cap), bad, kv_heads=hkv)
        torch.cuda.synchronize()
        assert bad.item() == 0
        assert torch.equal(one[0], out[i]), i


@pytest.mark.parametrize("fmt", [abi.KV_BF16, abi.KV_Q8])
@pytest.mark.parametrize("hq", [16, 32])
def test_decode_attention_fp8_merge(fmt, hq):
    """The merge with the FP8 output (MergeQuantize): out identical to padra_DecodeAttention's
    and the codes and scales identical to padra_QuantizeFP8 of that output (both pinned by
    their own tests), for BF16 and q8 caches; a zero query row gives scale 1 and zero
    codes; a q8_0 cache is refused."""
    print(f"[case] decode attention fp8 merge fmt={fmt} hq={hq}", flush=True)
    seqs, hkv, capacity = 5, 4, 4096
    rng = np.random.default_rng(150 + hq + fmt)
    positions = rng.integers(0, capacity, seqs).astype(np.int32)
    positions[0] = 0
    q = synth.bf16_bits((rng.standard_normal((seqs, hq, 128)) * 2).astype(np.float32))
    if fmt == abi.KV_BF16:
        kc = dev(synth.bf16_bits(rng.standard_normal((seqs * capacity, hkv * 128)).astype(np.float32)))
        vc = dev(synth.bf16_bits(rng.standard_normal((seqs * capacity, hkv * 128)).astype(np.float32)))
        vc[capacity * 2:capacity * 3] = 0  # sequence 2: all-zero values, a zero output row
        kv = ops.kv_cache(fmt, kc, vc, capacity, seq_stride=capacity)
    else:
        codes_k = torch.from_numpy(rng.integers(-127, 128, (seqs * capacity, hkv * 128)).astype(np.int8)).cuda()
        codes_v = torch.from_numpy(rng.integers(-127, 128, (seqs * capacity, hkv * 128)).astype(np.int8)).cuda()
        codes_v[capacity * 2:capacity * 3] = 0
        sc = torch.from_numpy(rng.uniform(0.005, 0.02, (seqs * capacity, hkv, 2)).astype(np.float32)).cuda()
        kv = ops.kv_cache(fmt, codes_k, codes_v, capacity, scales=sc, seq_stride=capacity)
    states = np.zeros((seqs, 8), np.int32)
    for s, p in enumerate(positions):
        states[s] = [5, p, capacity, 10, p, min(p, 1024), 0, 0]
    pos = ops.positions_decode(torch.from_numpy(states).cuda(), maximum=capacity)
    out_a = torch.empty((seqs, hq, 128), dtype=torch.int16, device="cuda")
    out_b = torch.empty_like(out_a)
    packed_a = torch.empty((seqs, hq * 128), dtype=torch.uint8, device="cuda")
    packed_b = torch.empty_like(packed_a)
    scales_a = torch.empty(seqs, dtype=torch.float32, device="cuda")
    scales_b = torch.empty_like(scales_a)
    bad = flag()
    ops.DecodeAttention(dev(q), kv, out_a, pos, bad, kv_heads=hkv)
    ops.QuantizeFP8(out_a.view(seqs, hq * 128), packed_a, scales_a, bad)
    ops.DecodeAttention(dev(q), kv, out_b, pos, bad, kv_heads=hkv, packed=packed_b,
                        scales=scales_b)
    torch.cuda.synchronize()
    assert bad.item() == 0
    assert torch.equal(out_a, out_b)
    assert torch.equal(packed_a, packed_b)
    assert torch.equal(scales_a, scales_b)
    assert scales_b[2].item() == 1.0 and not packed_b[2].any().item()
    q8_0 = ops.kv_cache(abi.KV_Q8_0, torch.zeros((seqs * capacity, 544), dtype=torch.uint8,
                                                 device="cuda"),
                        torch.zeros((seqs * capacity, 544), dtype=torch.uint8, device="cuda"),
                        capacity, seq_stride=capacity)
    with pytest.raises(abi.PadraError):
        ops.DecodeAttention(dev(q), q8_0, out_b, pos, bad, kv_heads=hkv, packed=packed_b,
                            scales=scales_b)


def test_decode_attention_q8_scales(oracle):
    """kv_q8::Decode's checks (kv_q8.cuh:15-27) on the rows the split reads: a scale whose
    127 * scale overflows BF16 decodes its smaller codes to finite values (no flag) and its
    overflowing ones to a flag; a zero scale in the window is flagged; a NaN scale outside
    the window is never read."""
    print("[case] decode attention q8 scales", flush=True)
    seqs, hq, hkv, cap = 2, 16, 4, 1024
    rng = np.random.default_rng(141)
    positions = np.array([3, 700], np.int32)
    q = synth.bf16_bits((rng.standard_normal((seqs, hq, 128)) * 2).astype(np.float32))
    codes_k = rng.integers(-127, 128, (seqs, cap, hkv * 128)).astype(np.int8)
    codes_v = rng.integers(-127, 128, (seqs, cap, hkv * 128)).astype(np.int8)
    scales = (rng.uniform(0.005, 0.02, (seqs, cap, hkv, 2))).astype(np.float32)
    # sequence 1, row 17, V of every head: scale 3e36, codes within +-100 (3e38 < BF16 max)
    codes_v[1, 17] = rng.integers(-100, 101, hkv * 128)
    scales[1, 17, :, 1] = 3e36
    scales[0, 500, :, 0] = np.nan  # outside sequence 0's window (positions 0..3)
    states = np.zeros((seqs, 8), np.int32)
    for s, p in enumerate(positions):
        states[s] = [5, p, cap, 10, p, min(p, 1024), 0, 0]

    def run(ck, sc):
        out = torch.empty((seqs, hq, 128), dtype=torch.int16, device="cuda")
        bad = flag()
        kv = ops.kv_cache(abi.KV_Q8, torch.from_numpy(ck.reshape(seqs * cap, -1)).cuda(),
                          torch.from_numpy(codes_v.reshape(seqs * cap, -1)).cuda(), cap,
                          scales=torch.from_numpy(sc.reshape(seqs * cap, hkv, 2)).cuda(),
                          seq_stride=cap)
        ops.DecodeAttention(dev(q), kv, out,
                            ops.positions_decode(torch.from_numpy(states).cuda(), maximum=cap),
                            bad, kv_heads=hkv)
        torch.cuda.synchronize()
        return host16(out), bad.item()

    got, bad = run(codes_k, scales)
    assert bad == 0
    with np.errstate(over="ignore", invalid="ignore"):
        dk = synth.bf16_bits(codes_k.reshape(seqs, cap, hkv, 128).astype(np.float32) *
                             scales[..., 0:1]).reshape(seqs, cap, -1)
        dv = synth.bf16_bits(codes_v.reshape(seqs, cap, hkv, 128).astype(np.float32) *
                             scales[..., 1:2]).reshape(seqs, cap, -1)
    for s in range(seqs):
        want, used, wbad = oracle.decode_attention(q[s], dk[s], dv[s], positions[s])
        assert not wbad
        with np.errstate(over="ignore", invalid="ignore"):
            b = bound_bf16(q[s], dk[s], dv[s], positions[s], False, used)
        close, d = _attn_close(got[s], want, b)
        assert close.all(), (s, int(d.max()))
    # code 127 at scale 3e36 rounds to a BF16 infinity
    codes_v[1, 17, 3] = 127
    assert run(codes_k, scales)[1] == 1
    codes_v[1, 17, 3] = 0
    sc = scales.copy()
    sc[1, 650, 2, 0] = 0.0  # zero K scale inside sequence 1's window
    assert run(codes_k, sc)[1] == 1


def test_stream_copy():
    """The bench's ceiling kernel copies exactly (whole and partial last workgroups) and
    refuses misaligned sizes."""
    print("[case] stream copy", flush=True)
    for n in (16, 16 * 1023, 16 * 1024 * 5 + 48):
        src = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda")
        dst = torch.zeros_like(src)
        abi.call("padra_StreamCopy", None, dst.data_ptr(), src.data_ptr(), n)
        torch.cuda.synchronize()
        assert torch.equal(src, dst), n
    with pytest.raises(abi.PadraError):
        abi.call("padra_StreamCopy", None, dst.data_ptr(), src.data_ptr(), 24)


@pytest.mark.parametrize("mode,fmt", [("decode", abi.KV_BF16), ("decode", abi.KV_Q8_0),
                                      ("base", abi.KV_BF16), ("prefill", abi.KV_Q8)])
def test_embed_chain_matches_gather_then_chain(oracle, mode, fmt):
    """padra_EmbedResidualNormQKRopeStore against padra_Embed followed by
    padra_ResidualNormQKRopeStore on the same inputs: x, normalized, q, k, the caches and
    the flag bit-identical; x and normalized also against the oracle's residual norm of the
    gathered rows.  Decode: 64 sequences at ragged positions with per-sequence caches, one
    of them holding a token outside the vocabulary (the flag is raised and that row reads
    x as it was); base: token ids from an array; prefill: the prompt ids from the
    PrefillState's prompt offset."""
    print(f"[case] embed chain mode={mode} fmt={fmt}", flush=True)
    seqs, capacity, vocab, hidden = 64, 2048, 1000, 2048
    rng = np.random.default_rng(123)
    d = synth.chain_inputs(seqs, outliers=True, seed=124)
    emb = synth.bf16_bits((rng.standard_normal((vocab, hidden)) * 0.5).astype(np.float32))
    offset = 7 if mode == "prefill" else 0
    prompt = rng.integers(0, vocab, seqs + offset).astype(np.int32)
    ids = prompt[offset:]
    positions = rng.integers(0, capacity, seqs).astype(np.int32)
    tb = ops.RopeTable(capacity, 128, 1e6).view(torch.int16).numpy().view(np.uint16)
    states = np.zeros((seqs, 8), np.int32)
    for i, p in enumerate(positions):
        states[i] = [ids[i], p, capacity, 10, p, min(int(p), 1024), 0, 0]
    invalid = 5 if mode == "decode" else None
    if invalid is not None:
        states[invalid, 0] = vocab  # outside [0, vocab)

    def run(fused):
        x, r, y = dev(d["x"]), dev(d["residual"]), torch.empty((seqs, hidden), dtype=torch.int16, device="cuda")
        q, k = dev(d["q"]), dev(d["k"])
        rows = seqs * capacity if mode == "decode" else capacity
        kc, vc, sc = _cache(fmt, rows)
        st = dev(states)
        bad = flag()
        if mode == "decode":
            pos = ops.positions_decode(st, maximum=capacity, vocab=vocab)
            kv = ops.kv_cache(fmt, kc, vc, capacity, scales=sc, seq_stride=capacity)
        elif mode == "prefill":
            pst = torch.tensor([100, offset, seqs, capacity, 100, 1, 1, 1], dtype=torch.int32,
                               device="cuda")
            pos = ops.positions_prefill(pst, maximum=capacity)
            kv = ops.kv_cache(fmt, kc, vc, capacity, scales=sc)
        else:
            pos = ops.positions_base(100)
            kv = ops.kv_cache(fmt, kc, vc, capacity, scales=sc)
        args = (x, dev(d["residual"]), y, dev(d["gamma"]), q, k, dev(d["v"]), dev(d["qn"]),
                dev(d["kn"]), dev(tb), pos, kv, bad)
        table, idt = dev(emb), dev(prompt if mode == "prefill" else ids)
        if fused:
            ops.EmbedResidualNormQKRopeStore(table, idt, *args, tree=abi.TREE_256)
        else:
            ops.Embed(table, x, bad, ids=idt, positions=pos)
            ops.ResidualNormQKRopeStore(*args, tree=abi.TREE_256)
        torch.cuda.synchronize()
        out = [host16(x), host16(y), host16(q), host16(k), kc.cpu().numpy(), vc.cpu().numpy(),
               int(bad.item())]
        if sc is not None:
            out.append(sc.cpu().numpy())
        return out

    fused, split = run(True), run(False)
    for a, b in zip(fused, split):
        assert np.array_equal(a, b)
    assert fused[6] == (1 if invalid is not None else 0)
    xin = emb[ids].copy()
    if invalid is not None:
        xin[invalid] = d["x"].reshape(seqs, hidden)[invalid]
    wx, wy, _, _ = oracle.residual_rmsnorm(xin, d["residual"].reshape(seqs, hidden),
                                           d["gamma"], threads=256)
    assert np.array_equal(fused[0], wx) and np.array_equal(fused[1], wy)


@pytest.mark.parametrize("fmt,fp8", [(abi.KV_BF16, False), (abi.KV_Q8, False),
                                     (abi.KV_Q8_0, False), (abi.KV_BF16, True),
                                     (abi.KV_Q8, True)])
def test_decode_attention_scratch_bounds(oracle, fmt, fp8):
    """The split and merge kernels stay inside the padra_DecodeAttentionScratch floats: a
    scratch of exactly that size followed by sentinel floats keeps every sentinel, and the
    output equals the one computed with an oversized scratch."""
    print(f"[case] decode attention scratch bounds fmt={fmt} fp8={fp8}", flush=True)
    seqs, hq, hkv, cap, splits = 3, 4, 4, 512, 5
    rng = np.random.default_rng(150 + fmt)
    positions = np.array([0, 300, 511], np.int32)
    q = dev(synth.bf16_bits(rng.standard_normal((seqs, hq, 128)).astype(np.float32)))
    scales = None
    if fmt == abi.KV_BF16:
        kc = dev(synth.bf16_bits(rng.standard_normal((seqs * cap, 512)).astype(np.float32)))
        vc = dev(synth.bf16_bits(rng.standard_normal((seqs * cap, 512)).astype(np.float32)))
    elif fmt == abi.KV_Q8:
        kc = torch.from_numpy(rng.integers(-127, 128, (seqs * cap, 512)).astype(np.int8)).cuda()
        vc = torch.from_numpy(rng.integers(-127, 128, (seqs * cap, 512)).astype(np.int8)).cuda()
        scales = torch.from_numpy(rng.uniform(0.005, 0.02, (seqs * cap, hkv, 2))
                                  .astype(np.float32)).cuda()
    else:
        rk = np.zeros((seqs * cap, 544), np.uint8)
        rv = np.zeros((seqs * cap, 544), np.uint8)
        d = synth.chain_inputs(seqs * cap, outliers=True, seed=151)
        oracle.kv_q8_0_encode(d["k"], d["v"], rk, rv, np.arange(seqs * cap, dtype=np.int32),
                              seqs * cap)
        kc, vc = dev(rk), dev(rv)
    kv = ops.kv_cache(fmt, kc, vc, cap, scales=scales, seq_stride=cap)
    states = np.zeros((seqs, 8), np.int32)
    for s, p in enumerate(positions):
        states[s] = [5, p, cap, 10, p, min(p, 1024), 0, 0]
    pos = ops.positions_decode(torch.from_numpy(states).cuda(), maximum=cap)
    need = abi.lib().padra_DecodeAttentionScratch(fmt, seqs, hq, splits)
    assert need > 0 and need % 4 == 0
    guard = 4096
    sentinel = -12345.678
    outs = []
    for extra in (guard, 1 << 20):
        scratch = torch.full((need + extra,), sentinel, dtype=torch.float32, device="cuda")
        out = torch.empty((seqs, hq, 128), dtype=torch.int16, device="cuda")
        bad = flag()
        packed = scl = None
        if fp8:
            packed = torch.empty((seqs, hq * 128), dtype=torch.uint8, device="cuda")
            scl = torch.empty(seqs, dtype=torch.float32, device="cuda")
        ops.DecodeAttention(q, kv, out, pos, bad, kv_heads=hkv, splits=splits,
                            scratch=scratch[:need], packed=packed, scales=scl)
        torch.cuda.synchronize()
        assert bad.item() == 0
        tail = scratch[need:].cpu().numpy()
        assert np.all(tail == np.float32(sentinel)), int(np.argmax(tail != np.float32(sentinel)))
        outs.append(host16(out))
    assert np.array_equal(outs[0], outs[1])
