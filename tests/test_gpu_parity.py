"""GPU parity: the HIP library (through its C-ABI) against the CPU oracle, bit for bit.

Every output here is BF16, integer codes or fp16/fp32 scales: the bar is exact equality.
The reduction-order golden rows (tests/golden/reduction_order.npz) make the tree order
observable, so a GPU tree that differs from the reference's fails here.
"""
import os

import numpy as np
import pytest
import torch

from padra_amd import abi, ops, synth

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


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


def table_bits(oracle, n, theta=1e6):
    return synth.bf16_bits(oracle.rope_table(n, 128, theta))


# ---- residual + RMSNorm ------------------------------------------------------------------

@pytest.mark.parametrize("tree", [128, 256])
@pytest.mark.parametrize("hidden", [2048, 2304])
@pytest.mark.parametrize("rows", [1, 5, 37])
@pytest.mark.parametrize("residual", [True, False])
def test_residual_norm_bf16(oracle, tree, hidden, rows, residual):
    print(f"[case] norm tree={tree} hidden={hidden} rows={rows} residual={residual}", flush=True)
    d = synth.chain_inputs(rows, hidden=hidden, outliers=True, seed=rows + hidden + tree)
    if residual:
        want_x, want_y, want_st, want_bad = oracle.residual_rmsnorm(d["x"], d["residual"],
                                                                    d["gamma"], threads=tree)
    else:
        want_y, want_st, want_bad = oracle.rmsnorm(d["x"], d["gamma"], threads=tree)
        want_x = d["x"]
    x, r, g = dev(d["x"]), dev(d["residual"]), dev(d["gamma"])
    y = torch.empty_like(x)
    st = torch.empty((rows, 2), dtype=torch.float32, device="cuda")
    bad = flag()
    ops.ResidualPostNorm(x, r if residual else None, y, g, bad, tree=tree, statistics=st)
    torch.cuda.synchronize()
    assert np.array_equal(host16(x), want_x)
    assert np.array_equal(host16(y), want_y)
    assert np.array_equal(st.cpu().numpy(), want_st)
    assert bool(bad.item()) == want_bad


@pytest.mark.parametrize("tree", [128, 256])
def test_residual_norm_f32_activations(oracle, tree):
    print(f"[case] norm f32 tree={tree}", flush=True)
    d = synth.chain_inputs(9, outliers=True, seed=77)
    want_x, want_y, want_st, _ = oracle.residual_rmsnorm(d["x"], d["residual"], d["gamma"],
                                                         threads=tree)
    x = torch.from_numpy(synth.bf16_to_f32(d["x"])).cuda()
    r = torch.from_numpy(synth.bf16_to_f32(d["residual"])).cuda()
    y = torch.empty_like(x)
    bad = flag()
    ops.ResidualPostNorm(x, r, y, dev(d["gamma"]), bad, tree=tree)
    torch.cuda.synchronize()
    assert np.array_equal(x.cpu().numpy(), synth.bf16_to_f32(want_x))
    assert np.array_equal(y.cpu().numpy(), synth.bf16_to_f32(want_y))
    assert not bad.item()


def test_residual_norm_golden_order_rows(oracle):
    """Rows built from the order-sensitive golden vector: the two trees give different
    variances, and the GPU must give each tree's own."""
    g = np.load(os.path.join(HERE, "golden", "reduction_order.npz"))
    row = np.zeros(2048, np.float32)
    row[:512] = g["v512"]
    bits = synth.bf16_bits(np.stack([row, row * 0.5]))
    gamma = synth.bf16_bits(np.ones(2048))
    for tree, key in ((128, "v512_tree128"), (256, "v512_tree256")):
        print(f"[case] golden order tree={tree}", flush=True)
        x = dev(bits)
        y = torch.empty_like(x)
        st = torch.empty((2, 2), dtype=torch.float32, device="cuda")
        ops.ResidualPostNorm(x, None, y, dev(gamma), flag(), tree=tree, statistics=st)
        torch.cuda.synchronize()
        assert st[0, 0].item() == np.float32(g[key] / np.float32(2048))
        want_y, want_st, _ = oracle.rmsnorm(bits, gamma, threads=tree)
        assert np.array_equal(host16(y), want_y)
        assert np.array_equal(st.cpu().numpy(), want_st)


def test_residual_norm_nonfinite_sets_bad():
    d = synth.chain_inputs(4, seed=3)
    xb = d["x"].copy()
    xb[2, 100] = 0x7F80
    x = dev(xb)
    y = torch.empty_like(x)
    bad = flag()
    ops.ResidualPostNorm(x, dev(d["residual"]), y, dev(d["gamma"]), bad)
    torch.cuda.synchronize()
    assert bad.item() == 1


# ---- RMSNorm + FP8 E4M3 row encoding ---------------------------------------------------------

@pytest.mark.parametrize("hidden,rows", [(2048, 1), (2048, 37), (2048, 512), (2048, 2048),
                                         (2304, 1), (2304, 37), (2304, 512), (1024, 9),
                                         (1152, 9), (4096, 9), (4608, 9)])
@pytest.mark.parametrize("act", ["bf16", "f32"])
def test_norm_fp8(oracle, hidden, rows, act):
    print(f"[case] norm fp8 hidden={hidden} rows={rows} act={act}", flush=True)
    d = synth.chain_inputs(rows, hidden=hidden, outliers=True, seed=rows + hidden)
    xb = d["x"].copy()
    if rows > 1:
        xb[rows // 2] = 0  # all-zero row: scale 1
    want_y, want_p, want_s, want_st, want_bad = oracle.norm_fp8(xb, d["gamma"])
    if act == "bf16":
        x = dev(xb)
    else:
        x = torch.from_numpy(synth.bf16_to_f32(xb)).cuda()
    y = torch.empty_like(x)
    packed = torch.empty((rows, hidden), dtype=torch.uint8, device="cuda")
    scales = torch.empty(rows, dtype=torch.float32, device="cuda")
    st = torch.full((2,), -1.0, dtype=torch.float32, device="cuda")
    bad = flag()
    ops.NormFP8(x, y, dev(d["gamma"]), packed, scales, bad, statistics=st)
    torch.cuda.synchronize()
    got_y = host16(y) if act == "bf16" else synth.bf16_bits(y.cpu().numpy())
    assert np.array_equal(got_y, want_y)
    assert np.array_equal(scales.cpu().numpy(), want_s)
    assert np.array_equal(packed.cpu().numpy(), want_p)
    assert np.array_equal(st.cpu().numpy(), want_st)
    assert bool(bad.item()) == want_bad


def test_fp8_fast_path_identities_exhaustive():
    """The two identities the FP8 fast path rests on, over their whole domains: the hardware
    E4M3 conversion equals the format-defined encoder on every float up to 480, and the
    reciprocal-plus-correction quotient gives the correctly rounded quotient's code for
    every BF16 (maximum, value) pair the fast path admits."""
    print("[case] fp8 fast-path identities", flush=True)
    counts = torch.full((2,), -1, dtype=torch.int64, device="cuda")
    abi.call("padra_CheckFP8Paths", None, counts.data_ptr())
    torch.cuda.synchronize()
    assert counts.tolist() == [0, 0]


def test_q8_reciprocal_code_exhaustive():
    """The q8 KV code through the scale's reciprocal (the store kernels' form) equals the
    code of the correctly rounded division for every BF16 (maximum, value) pair whose scale
    is at least 2^-100."""
    print("[case] q8 reciprocal code", flush=True)
    counts = torch.full((1,), -1, dtype=torch.int64, device="cuda")
    abi.call("padra_CheckQ8Path", None, counts.data_ptr())
    torch.cuda.synchronize()
    assert counts.tolist() == [0]


@pytest.mark.parametrize("act", ["bf16", "f32"])
def test_quantize_fp8(oracle, act):
    """E4M3 row encoding of activations (the attention output): BF16 rows (fast path),
    fp32 rows that are not BF16-exact (division path), a zero row and a NaN row."""
    print(f"[case] quantize fp8 act={act}", flush=True)
    rng = np.random.default_rng(140)
    rows, cols = 40, 4096
    xf = (rng.standard_normal((rows, cols)) * np.exp2(rng.integers(-8, 8, (rows, 1)))).astype(
        np.float32)
    xf[3] = 0
    if act == "bf16":
        xb = synth.bf16_bits(xf)
        xf = synth.bf16_to_f32(xb)
        x = dev(xb)
    else:
        x = torch.from_numpy(xf).cuda()
    want_p, want_s, want_bad = oracle.quantize_fp8(xf)
    packed = torch.empty((rows, cols), dtype=torch.uint8, device="cuda")
    scales = torch.empty(rows, dtype=torch.float32, device="cuda")
    bad = flag()
    ops.QuantizeFP8(x, packed, scales, bad)
    torch.cuda.synchronize()
    assert not want_bad and bad.item() == 0
    assert np.array_equal(scales.cpu().numpy(), want_s)
    assert np.array_equal(packed.cpu().numpy(), want_p)


def test_norm_fp8_nonfinite_and_extremes(oracle):
    """A NaN and an infinite input row (flag raised; bytes as the reference writes them), a
    row of tiny values (scale near the fp32 minimum) and a row whose sum of squares
    overflows (inv = 0, so y = 0 and scale 1)."""
    print("[case] norm fp8 extremes", flush=True)
    hidden, rows = 2304, 6
    d = synth.chain_inputs(rows, hidden=hidden, outliers=True, seed=91)
    xb = d["x"].copy()
    xb[1, 5] = 0x7FC0  # NaN
    xb[2, 9] = 0x7F80  # +inf
    xb[3] = synth.bf16_bits(synth.bf16_to_f32(xb[3]) * np.float32(2.0**-120))
    xb[4] = synth.bf16_bits(synth.bf16_to_f32(xb[4]) * np.float32(2.0**100))
    want_y, want_p, want_s, _, want_bad = oracle.norm_fp8(xb, d["gamma"])
    assert want_bad
    x = dev(xb)
    y = torch.empty_like(x)
    packed = torch.empty((rows, hidden), dtype=torch.uint8, device="cuda")
    scales = torch.empty(rows, dtype=torch.float32, device="cuda")
    bad = flag()
    ops.NormFP8(x, y, dev(d["gamma"]), packed, scales, bad)
    torch.cuda.synchronize()
    assert bad.item() == 1
    # NaN signs and payloads are platform-defined (x86 and gfx950 make different default
    # NaNs): NaN outputs match as NaN, every other bit exactly.
    got_y = host16(y)
    nan_w = (want_y & 0x7FFF) > 0x7F80
    nan_g = (got_y & 0x7FFF) > 0x7F80
    assert np.array_equal(nan_g, nan_w) and nan_w.any()
    assert np.array_equal(got_y[~nan_w], want_y[~nan_w])
    assert np.array_equal(scales.cpu().numpy(), want_s)
    assert np.array_equal(packed.cpu().numpy(), want_p)


# ---- Q/K norm + RoPE + KV store -------------------------------------------------------------

def _qk_oracle(oracle, d, tb, positions):
    return oracle.qk_norm_rope(d["q"], d["k"], d["qn"], d["kn"], tb, positions)


@pytest.mark.parametrize("tokens,base", [(1, 4097), (7, 0), (300, 123)])
def test_qk_rope_no_store(oracle, tokens, base):
    print(f"[case] qk tokens={tokens} base={base}", flush=True)
    d = synth.chain_inputs(tokens, outliers=True, seed=tokens)
    tb = table_bits(oracle, base + tokens)
    wq, wk, _ = _qk_oracle(oracle, d, tb, np.arange(base, base + tokens, dtype=np.int32))
    q, k = dev(d["q"]), dev(d["k"])
    bad = flag()
    ops.QKNormRopeStore(q, k, dev(d["qn"]), dev(d["kn"]), dev(tb), ops.positions_base(base), bad)
    torch.cuda.synchronize()
    assert np.array_equal(host16(q), wq) and np.array_equal(host16(k), wk)
    assert not bad.item()


def test_qk_rope_golden_order_heads(oracle):
    g = np.load(os.path.join(HERE, "golden", "reduction_order.npz"))
    heads = synth.bf16_bits(g["head128"])  # [2][128]
    q = np.ascontiguousarray(np.repeat(heads[:, None, :], 16, axis=1))
    k = np.ascontiguousarray(np.repeat(heads[:, None, :], 4, axis=1))
    ones = synth.bf16_bits(np.ones(128))
    tb = table_bits(oracle, 4)
    wq, wk, _ = oracle.qk_norm_rope(q, k, ones, ones, tb, np.array([1, 2], np.int32))
    tq, tk = dev(q), dev(k)
    ops.QKNormRopeStore(tq, tk, dev(ones), dev(ones), dev(tb), ops.positions_base(1), flag())
    torch.cuda.synchronize()
    assert np.array_equal(host16(tq), wq) and np.array_equal(host16(tk), wk)


def _prefill_state(base, tokens, capacity, overrides=None):
    s = dict(base=base, prompt_offset=base, tokens=tokens, capacity=capacity, committed=base,
             binding_epoch=1, request_epoch=1, valid=1)
    s.update(overrides or {})
    return torch.tensor([s[k] for k in ("base", "prompt_offset", "tokens", "capacity",
                                        "committed", "binding_epoch", "request_epoch", "valid")],
                        dtype=torch.int32, device="cuda")


def _expected_cache(oracle, fmt, wk, v, positions, cap, first):
    tokens = wk.shape[0]
    if fmt == abi.KV_BF16:
        kc = np.zeros((cap, 512), np.uint16)
        vc = np.zeros((cap, 512), np.uint16)
        oracle.kv_store_bf16(wk, v, kc, vc, positions, cap, first)
        return kc, vc, None
    if fmt == abi.KV_Q8:
        kc = np.zeros((cap, 512), np.int8)
        vc = np.zeros((cap, 512), np.int8)
        sc = np.zeros((cap, 4, 2), np.float32)
        assert not oracle.kv_q8_encode(wk, v, kc, vc, sc, positions, cap, first)
        return kc, vc, sc
    kc = np.zeros((cap, 544), np.uint8)
    vc = np.zeros((cap, 544), np.uint8)
    assert not oracle.kv_q8_0_encode(wk, v, kc, vc, positions, cap, first,
                                     rotate=(fmt == abi.KV_Q8_0))
    return kc, vc, None


def _alloc_cache(fmt, rows):
    if fmt == abi.KV_BF16:
        return (torch.zeros((rows, 512), dtype=torch.int16, device="cuda"),
                torch.zeros((rows, 512), dtype=torch.int16, device="cuda"), None)
    if fmt == abi.KV_Q8:
        return (torch.zeros((rows, 512), dtype=torch.int8, device="cuda"),
                torch.zeros((rows, 512), dtype=torch.int8, device="cuda"),
                torch.zeros((rows, 4, 2), dtype=torch.float32, device="cuda"))
    return (torch.zeros((rows, 544), dtype=torch.uint8, device="cuda"),
            torch.zeros((rows, 544), dtype=torch.uint8, device="cuda"), None)


def _np(t, fmt):
    a = t.cpu().numpy()
    return a.view(np.uint16) if fmt == abi.KV_BF16 else a


FORMATS = [abi.KV_BF16, abi.KV_Q8, abi.KV_Q8_0, abi.KV_Q8_0_NOROT]


# A 64-row ring exists for the BF16 cache only: a quantized ring is the capacity or the
# 1024-row local ring (test_quantized_ring_rule_writes_nothing covers the rejection).
@pytest.mark.parametrize("fmt,tokens,base,cap",
                         [(f, t, b, c) for f in FORMATS
                          for t, b, c in [(64, 0, 4096), (100, 5, 64), (300, 1000, 4096),
                                          (1500, 100, 1024)]
                          if c != 64 or f == abi.KV_BF16])
def test_qk_rope_store_prefill(oracle, fmt, tokens, base, cap):
    print(f"[case] store fmt={fmt} tokens={tokens} base={base} cap={cap}", flush=True)
    d = synth.chain_inputs(tokens, outliers=True, seed=fmt * 7 + tokens)
    capacity = 4096
    first = 0 if cap == capacity else max(0, tokens - cap)
    tb = table_bits(oracle, capacity)
    positions = np.arange(base, base + tokens, dtype=np.int32)
    wq, wk, _ = _qk_oracle(oracle, d, tb, positions)
    ek, ev, es = _expected_cache(oracle, fmt, wk, d["v"], positions, cap, first)
    kc, vc, sc = _alloc_cache(fmt, cap)
    q, k = dev(d["q"]), dev(d["k"])
    state = _prefill_state(base, tokens, capacity)
    bad = flag()
    kv = ops.kv_cache(fmt, kc, vc, cap, scales=sc, first=first)
    ops.QKNormRopeStore(q, k, dev(d["qn"]), dev(d["kn"]), dev(tb),
                        ops.positions_prefill(state, maximum=capacity), bad, v=dev(d["v"]), kv=kv)
    torch.cuda.synchronize()
    assert not bad.item()
    assert np.array_equal(host16(q), wq) and np.array_equal(host16(k), wk)
    assert np.array_equal(_np(kc, fmt), ek)
    assert np.array_equal(_np(vc, fmt), ev)
    if es is not None:
        assert np.array_equal(sc.cpu().numpy(), es)


@pytest.mark.parametrize("fmt", [abi.KV_Q8, abi.KV_Q8_0, abi.KV_Q8_0_NOROT])
@pytest.mark.parametrize("tokens", [48, 400])
def test_store_extreme_value_scales(oracle, fmt, tokens):
    """V heads of tiny and huge magnitude (q8: scales below 2^-100, where the store takes
    the division instead of the reciprocal form, and near the top of the fp32 range; q8_0:
    fp16 block scales from subnormal to near their top), bit-exact against the oracle's
    codes and scales, in both launch shapes (48 tokens: a wave per (token, KV head) pair;
    400: four lanes per head)."""
    print(f"[case] store extreme scales fmt={fmt} tokens={tokens}", flush=True)
    capacity = 4096
    d = synth.chain_inputs(tokens, outliers=False, seed=77 + fmt)
    v = d["v"].view(np.uint16).reshape(tokens, -1).astype(np.uint32) << 16
    vf = v.view(np.float32).copy()
    # q8_0 scales are fp16 (amax / 127 must stay finite there), q8 scales fp32
    # q8_0 also takes subnormal V heads (1e-39): their block's 1 / ad overflows to
    # infinity, the one case whose codes need the clamp
    factors = np.array([1e-36, 3e-33, 1e-30, 1.0, 1e30, 1e36] if fmt == abi.KV_Q8 else
                       [1e-36, 1e-20, 1e-6, 1.0, 1e3, 1e5, 1e-39, 1.0], np.float32)
    vf *= factors[np.arange(tokens) % len(factors)][:, None]
    d["v"] = synth.bf16_bits(vf).reshape(d["v"].shape)
    tb = table_bits(oracle, capacity)
    positions = np.arange(tokens, dtype=np.int32)
    wq, wk, _ = _qk_oracle(oracle, d, tb, positions)
    ek, ev, es = _expected_cache(oracle, fmt, wk, d["v"], positions, capacity, 0)
    kc, vc, sc = _alloc_cache(fmt, capacity)
    q, k = dev(d["q"]), dev(d["k"])
    bad = flag()
    kv = ops.kv_cache(fmt, kc, vc, capacity, scales=sc)
    ops.QKNormRopeStore(q, k, dev(d["qn"]), dev(d["kn"]), dev(tb), ops.positions_base(0), bad,
                        v=dev(d["v"]), kv=kv)
    torch.cuda.synchronize()
    assert not bad.item()
    assert np.array_equal(_np(kc, fmt), ek)
    assert np.array_equal(_np(vc, fmt), ev)
    if es is not None:
        assert np.array_equal(sc.cpu().numpy(), es)
        small = es[..., 1][es[..., 1] > 0]
        assert small.min() < 2.0 ** -100  # the division path ran


@pytest.mark.parametrize("act", ["bf16", "f32"])
@pytest.mark.parametrize("fmt", [abi.KV_Q8, abi.KV_Q8_0, abi.KV_Q8_0_NOROT])
@pytest.mark.parametrize("tokens", [40, 400])
def test_store_nonfinite_heads(oracle, fmt, act, tokens):
    """Non-finite K and V heads in the quantized stores (kv_q8.cuh:49-54,
    kv_q8_native.cuh:70-79): the flag is raised and the head's codes and scales are not
    written.  Token 3 head 1 has a NaN in K and V, token 10 head 2 infinities in both,
    token 17 head 0 a NaN in V only: as in the reference, which encodes K and V of a head
    together, neither the K nor the V row of that head is written.  Token 25 head 3 has a
    V value of 1e9, whose q8_0 block scale overflows fp16 (block 2, both rotations): blocks
    0 and 1 of K and V are written, blocks 2 and 3 of neither (kv_q8_native.cuh:84-92).
    The caches start filled with a pattern, so that a row written with zero codes and
    scales differs from a row left alone; a second launch with only the V head of token
    17 invalid must raise the flag by itself.  Every byte of both caches is compared, in
    both launch shapes (40 tokens: a wave per (token, KV head) pair; 400: four lanes per
    head)."""
    print(f"[case] store nonfinite fmt={fmt} act={act} tokens={tokens}", flush=True)
    capacity = 4096
    d0 = synth.chain_inputs(tokens, outliers=False, seed=91 + fmt)
    tb = table_bits(oracle, capacity)
    positions = np.arange(tokens, dtype=np.int32)
    conv = (lambda a: torch.from_numpy(synth.bf16_to_f32(a)).cuda()) if act == "f32" else dev
    fill_code, fill_scale = 0x5A, 7.0

    def run(both):
        d = dict(d0)
        k, v = d0["k"].view(np.uint16).copy(), d0["v"].view(np.uint16).copy()
        if both:
            k[3, 1, 5], v[3, 1, 77] = 0x7FC0, 0x7FC0
            k[10, 2, 0], v[10, 2, 127] = 0x7F80, 0xFF80
        v[17, 0, 64] = 0x7FC0
        v[25, 3, 70] = 0x4E6E  # bf16(1e9)
        d["k"], d["v"] = k.view(d0["k"].dtype), v.view(d0["v"].dtype)
        _, wk, _ = _qk_oracle(oracle, d, tb, positions)
        width = 512 if fmt == abi.KV_Q8 else 544
        kind = np.int8 if fmt == abi.KV_Q8 else np.uint8
        ek, ev = np.full((capacity, width), fill_code, kind), np.full((capacity, width), fill_code, kind)
        es = None
        if fmt == abi.KV_Q8:
            es = np.full((capacity, 4, 2), fill_scale, np.float32)
            assert oracle.kv_q8_encode(wk, d["v"], ek, ev, es, positions, capacity, 0)
        else:
            assert oracle.kv_q8_0_encode(wk, d["v"], ek, ev, positions, capacity, 0,
                                         rotate=(fmt == abi.KV_Q8_0))
        kc, vc, sc = _alloc_cache(fmt, capacity)
        kc.fill_(fill_code)
        vc.fill_(fill_code)
        if sc is not None:
            sc.fill_(fill_scale)
        bad = flag()
        kv = ops.kv_cache(fmt, kc, vc, capacity, scales=sc)
        ops.QKNormRopeStore(conv(d["q"]), conv(d["k"]), dev(d["qn"]), dev(d["kn"]), dev(tb),
                            ops.positions_base(0), bad, v=conv(d["v"]), kv=kv)
        torch.cuda.synchronize()
        assert bad.item()
        assert np.array_equal(_np(vc, fmt), ev)
        assert np.array_equal(_np(kc, fmt), ek)
        # head 0 of token 17 (q8: codes 0-127; q8_0: scales d[0..3] and codes qs[0..127])
        head0 = np.r_[0:128] if fmt == abi.KV_Q8 else np.r_[0:8, 32:160]
        for c in (kc, vc):
            assert np.all(_np(c, fmt)[17, head0] == kind(fill_code))
        if es is not None:
            assert np.array_equal(sc.cpu().numpy(), es)

    run(True)
    run(False)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("tokens,base,cap", [(300, 1000, 4096), (1500, 100, 1024)])
def test_qk_rope_store_f32_activations(oracle, fmt, tokens, base, cap):
    """The reference's own activation form (fp32 buffers of BF16-exact values) through the
    Q/K path, every KV format, a global cache and a local ring narrower than the chunk:
    q and k in place, cache rows, codes and scales bit-exact against the oracle."""
    print(f"[case] store f32 fmt={fmt} tokens={tokens} cap={cap}", flush=True)
    d = synth.chain_inputs(tokens, outliers=True, seed=fmt * 11 + tokens)
    capacity = 4096
    first = 0 if cap == capacity else max(0, tokens - cap)
    tb = table_bits(oracle, capacity)
    positions = np.arange(base, base + tokens, dtype=np.int32)
    wq, wk, _ = _qk_oracle(oracle, d, tb, positions)
    ek, ev, es = _expected_cache(oracle, fmt, wk, d["v"], positions, cap, first)
    kc, vc, sc = _alloc_cache(fmt, cap)
    f32 = lambda a: torch.from_numpy(synth.bf16_to_f32(a)).cuda()
    q, k, v = f32(d["q"]), f32(d["k"]), f32(d["v"])
    state = _prefill_state(base, tokens, capacity)
    bad = flag()
    kv = ops.kv_cache(fmt, kc, vc, cap, scales=sc, first=first)
    ops.QKNormRopeStore(q, k, dev(d["qn"]), dev(d["kn"]), dev(tb),
                        ops.positions_prefill(state, maximum=capacity), bad, v=v, kv=kv)
    torch.cuda.synchronize()
    assert not bad.item()
    assert np.array_equal(q.cpu().numpy(), synth.bf16_to_f32(wq))
    assert np.array_equal(k.cpu().numpy(), synth.bf16_to_f32(wk))
    assert np.array_equal(_np(kc, fmt), ek)
    assert np.array_equal(_np(vc, fmt), ev)
    if es is not None:
        assert np.array_equal(sc.cpu().numpy(), es)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("act", ["bf16", "f32"])
@pytest.mark.parametrize("seqs", [16, 400])
def test_qk_rope_store_decode_batch(oracle, fmt, act, seqs):
    """Ragged positions, one token per sequence, per-sequence caches (seq_stride rows), on
    BF16 activations and on fp32 activations holding BF16-exact values (whose outputs must
    stay BF16-exact), with 16 sequences (a wave per head vector) and 400 (four lanes per
    head)."""
    print(f"[case] decode batch fmt={fmt} act={act} seqs={seqs}", flush=True)
    if act == "f32":
        conv = lambda a: torch.from_numpy(synth.bf16_to_f32(a)).cuda()

        def back(t):
            w = t.cpu().numpy().view(np.uint32)
            assert not (w & 0xFFFF).any()
            return (w >> 16).astype(np.uint16)
    else:
        conv, back = dev, host16
    cap, capacity = 256, 256
    rng = np.random.default_rng(fmt)
    positions = rng.integers(0, capacity, seqs).astype(np.int32)
    d = synth.chain_inputs(seqs, outliers=True, seed=40 + fmt)
    tb = table_bits(oracle, capacity)
    states = np.zeros((seqs, 8), np.int32)
    for s, p in enumerate(positions):
        states[s] = [5, p, capacity, 10, p, min(p, 1024), 0, 0]
    states[3, 7] = 1  # stopped: this sequence must write nothing and raise the flag
    wq, wk, _ = _qk_oracle(oracle, d, tb, positions)
    kc, vc, sc = _alloc_cache(fmt, seqs * cap)
    q, k = conv(d["q"]), conv(d["k"])
    bad = flag()
    kv = ops.kv_cache(fmt, kc, vc, cap, scales=sc, seq_stride=cap)
    ops.QKNormRopeStore(q, k, dev(d["qn"]), dev(d["kn"]), dev(tb),
                        ops.positions_decode(torch.from_numpy(states).cuda(), maximum=capacity),
                        bad, v=conv(d["v"]), kv=kv)
    torch.cuda.synchronize()
    assert bad.item() == 1
    gq, gk = back(q).copy(), back(k).copy()
    assert np.array_equal(gq[3], d["q"][3]) and np.array_equal(gk[3], d["k"][3])
    keep = [s for s in range(seqs) if s != 3]
    assert np.array_equal(gq[keep], wq[keep]) and np.array_equal(gk[keep], wk[keep])
    kca, vca = _np(kc, fmt).reshape(seqs, cap, -1), _np(vc, fmt).reshape(seqs, cap, -1)
    sca = None if sc is None else sc.cpu().numpy().reshape(seqs, cap, 4, 2)
    for s in range(seqs):
        ek, ev, es = _expected_cache(oracle, fmt, wk[s:s + 1], d["v"][s:s + 1],
                                     positions[s:s + 1], cap, 0)
        if s == 3:
            assert not kca[s].any() and not vca[s].any()
            continue
        assert np.array_equal(kca[s], ek) and np.array_equal(vca[s], ev)
        if es is not None:
            assert np.array_equal(sca[s], es)


def test_invalid_prefill_state_writes_nothing(oracle):
    d = synth.chain_inputs(8, seed=9)
    tb = table_bits(oracle, 64)
    for field in ({"committed": 1}, {"valid": 0}, {"tokens": 7}, {"base": 60}):
        q, k = dev(d["q"]), dev(d["k"])
        kc, vc, _ = _alloc_cache(abi.KV_BF16, 64)
        state = _prefill_state(0, 8, 64, overrides=field)
        bad = flag()
        ops.QKNormRopeStore(q, k, dev(d["qn"]), dev(d["kn"]), dev(tb),
                            ops.positions_prefill(state, maximum=64), bad, v=dev(d["v"]),
                            kv=ops.kv_cache(abi.KV_BF16, kc, vc, 64))
        torch.cuda.synchronize()
        assert bad.item() == 1, field
        assert np.array_equal(host16(q), d["q"]) and not kc.any().item(), field


@pytest.mark.parametrize("fmt", [abi.KV_Q8, abi.KV_Q8_0])
@pytest.mark.parametrize("tokens", [8, 400])
def test_quantized_ring_rule_writes_nothing(oracle, fmt, tokens):
    """A quantized cache binding whose capacity is neither the state's capacity nor the
    1024-row local ring (kv_q8.cuh:36-38): every token fails, so the flag is raised and no
    Q, K or cache byte is written, in the per-head launch (8 tokens) and the quad launch
    (400 tokens) alike."""
    print(f"[case] quantized ring rule fmt={fmt} tokens={tokens}", flush=True)
    d = synth.chain_inputs(tokens, seed=19)
    tb = table_bits(oracle, 4096)
    q, k = dev(d["q"]), dev(d["k"])
    kc, vc, sc = _alloc_cache(fmt, 512)
    state = _prefill_state(0, tokens, 4096)
    bad = flag()
    ops.QKNormRopeStore(q, k, dev(d["qn"]), dev(d["kn"]), dev(tb),
                        ops.positions_prefill(state, maximum=4096), bad, v=dev(d["v"]),
                        kv=ops.kv_cache(fmt, kc, vc, 512, scales=sc))
    torch.cuda.synchronize()
    assert bad.item() == 1
    assert np.array_equal(host16(q), d["q"]) and np.array_equal(host16(k), d["k"])
    assert not kc.any().item() and not vc.any().item()
    if sc is not None:
        assert not sc.any().item()


# ---- fused chain -----------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("tree", [128, 256])
@pytest.mark.parametrize("tokens", [333, 321, 193, 192, 37])
def test_fused_chain_matches_oracle(oracle, fmt, tree, tokens):
    """Both launch shapes of the chain on each side of their thresholds: up to 192 tokens
    (BF16 cache) or 320 (quantized caches) a wave per Q/K head, which with a quantized
    cache also encodes the K/V pair, and with the 256-thread tree a workgroup per norm
    row; above, four lanes per head."""
    print(f"[case] chain fmt={fmt} tree={tree} tokens={tokens}", flush=True)
    capacity = 4096
    d = synth.chain_inputs(tokens, outliers=True, seed=fmt + tree)
    tb = table_bits(oracle, capacity)
    positions = np.arange(tokens, dtype=np.int32) + 17
    wx, wy, wst, _ = oracle.residual_rmsnorm(d["x"], d["residual"], d["gamma"], threads=tree)
    wq, wk, _ = _qk_oracle(oracle, d, tb, positions)
    ek, ev, es = _expected_cache(oracle, fmt, wk, d["v"], positions, capacity, 0)
    x, r, g = dev(d["x"]), dev(d["residual"]), dev(d["gamma"])
    y = torch.empty_like(x)
    st = torch.empty((tokens, 2), dtype=torch.float32, device="cuda")
    q, k = dev(d["q"]), dev(d["k"])
    kc, vc, sc = _alloc_cache(fmt, capacity)
    bad = flag()
    ops.ResidualNormQKRopeStore(x, r, y, g, q, k, dev(d["v"]), dev(d["qn"]), dev(d["kn"]),
                                dev(tb), ops.positions_base(17),
                                ops.kv_cache(fmt, kc, vc, capacity, scales=sc), bad, tree=tree,
                                statistics=st)
    torch.cuda.synchronize()
    assert not bad.item()
    assert np.array_equal(host16(x), wx) and np.array_equal(host16(y), wy)
    assert np.array_equal(st.cpu().numpy(), wst)
    assert np.array_equal(host16(q), wq) and np.array_equal(host16(k), wk)
    assert np.array_equal(_np(kc, fmt), ek) and np.array_equal(_np(vc, fmt), ev)
    if es is not None:
        assert np.array_equal(sc.cpu().numpy(), es)


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("tree,tokens", [(128, 300), (256, 64), (128, 385), (256, 384),
                                         (256, 700)])
def test_fused_chain_f32_activations(oracle, fmt, tree, tokens):
    """The fused chain on fp32 activations holding BF16-exact values (the reference's
    buffers): every output equal to the oracle's, as floats, on both launch shapes (one
    launch with a wave per head vector up to 384 tokens with a BF16 cache and 320 with a
    quantized one; above, the norm launch and the four-lanes-per-head Q/K launch)."""
    print(f"[case] chain f32 fmt={fmt} tree={tree} tokens={tokens}", flush=True)
    capacity = 4096
    d = synth.chain_inputs(tokens, outliers=True, seed=300 + fmt + tree)
    tb = table_bits(oracle, capacity)
    positions = np.arange(tokens, dtype=np.int32) + 9
    wx, wy, wst, _ = oracle.residual_rmsnorm(d["x"], d["residual"], d["gamma"], threads=tree)
    wq, wk, _ = _qk_oracle(oracle, d, tb, positions)
    ek, ev, es = _expected_cache(oracle, fmt, wk, d["v"], positions, capacity, 0)
    f32 = lambda a: torch.from_numpy(synth.bf16_to_f32(a)).cuda()
    x, r, q, k = f32(d["x"]), f32(d["residual"]), f32(d["q"]), f32(d["k"])
    y = torch.empty_like(x)
    st = torch.empty((tokens, 2), dtype=torch.float32, device="cuda")
    kc, vc, sc = _alloc_cache(fmt, capacity)
    bad = flag()
    ops.ResidualNormQKRopeStore(x, r, y, dev(d["gamma"]), q, k, f32(d["v"]), dev(d["qn"]),
                                dev(d["kn"]), dev(tb), ops.positions_base(9),
                                ops.kv_cache(fmt, kc, vc, capacity, scales=sc), bad, tree=tree,
                                statistics=st)
    torch.cuda.synchronize()
    assert not bad.item()
    as_f32 = lambda t: t.cpu().numpy()
    assert np.array_equal(as_f32(x), synth.bf16_to_f32(wx))
    assert np.array_equal(as_f32(y), synth.bf16_to_f32(wy))
    assert np.array_equal(st.cpu().numpy(), wst)
    assert np.array_equal(as_f32(q), synth.bf16_to_f32(wq))
    assert np.array_equal(as_f32(k), synth.bf16_to_f32(wk))
    assert np.array_equal(_np(kc, fmt), ek) and np.array_equal(_np(vc, fmt), ev)
    if es is not None:
        assert np.array_equal(sc.cpu().numpy(), es)


def test_config1_full_chunk(oracle):
    """Config 1 at full size: 2048-token prefill chunk, BF16 KV, cap 131072, outliers."""
    print("[case] config1 full", flush=True)
    tokens, capacity = 2048, 131072
    d = synth.chain_inputs(tokens, outliers=True, seed=0)
    tb = table_bits(oracle, tokens)
    positions = np.arange(tokens, dtype=np.int32)
    wx, wy, _, _ = oracle.residual_rmsnorm(d["x"], d["residual"], d["gamma"], threads=128)
    wq, wk, _ = _qk_oracle(oracle, d, tb, positions)
    x, r, g = dev(d["x"]), dev(d["residual"]), dev(d["gamma"])
    y = torch.empty_like(x)
    q, k = dev(d["q"]), dev(d["k"])
    kc = torch.zeros((capacity, 512), dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    state = _prefill_state(0, tokens, capacity)
    bad = flag()
    ops.ResidualNormQKRopeStore(x, r, y, g, q, k, dev(d["v"]), dev(d["qn"]), dev(d["kn"]),
                                dev(tb), ops.positions_prefill(state),
                                ops.kv_cache(abi.KV_BF16, kc, vc, capacity), bad)
    torch.cuda.synchronize()
    assert not bad.item()
    assert np.array_equal(host16(x), wx) and np.array_equal(host16(y), wy)
    assert np.array_equal(host16(q), wq) and np.array_equal(host16(k), wk)
    assert np.array_equal(host16(kc[:tokens]), wk.reshape(tokens, -1))
    assert np.array_equal(host16(vc[:tokens]), d["v"].reshape(tokens, -1))
    assert not kc[tokens:].any().item()


@pytest.mark.parametrize("fmt", [abi.KV_Q8, abi.KV_Q8_0, abi.KV_Q8_0_NOROT])
def test_config2_full_chunk(oracle, fmt):
    """Config 2 at full size: the 2048-token chunk with quantized KV (q8, q8_0 rotated and
    unrotated), cap 131072, outliers in K and V; every output and code bit-exact."""
    print(f"[case] config2 full fmt={fmt}", flush=True)
    tokens, capacity = 2048, 131072
    d = synth.chain_inputs(tokens, outliers=True, seed=2)
    tb = table_bits(oracle, tokens)
    positions = np.arange(tokens, dtype=np.int32)
    wx, wy, _, _ = oracle.residual_rmsnorm(d["x"], d["residual"], d["gamma"], threads=128)
    wq, wk, _ = _qk_oracle(oracle, d, tb, positions)
    # slots of positions < tokens: the expected rows of a cache `tokens` rows long
    ek, ev, es = _expected_cache(oracle, fmt, wk, d["v"], positions, tokens, 0)
    x, r, g = dev(d["x"]), dev(d["residual"]), dev(d["gamma"])
    y = torch.empty_like(x)
    q, k = dev(d["q"]), dev(d["k"])
    kc, vc, sc = _alloc_cache(fmt, capacity)
    state = _prefill_state(0, tokens, capacity)
    bad = flag()
    ops.ResidualNormQKRopeStore(x, r, y, g, q, k, dev(d["v"]), dev(d["qn"]), dev(d["kn"]),
                                dev(tb), ops.positions_prefill(state),
                                ops.kv_cache(fmt, kc, vc, capacity, scales=sc), bad)
    torch.cuda.synchronize()
    assert not bad.item()
    assert np.array_equal(host16(x), wx) and np.array_equal(host16(y), wy)
    assert np.array_equal(host16(q), wq) and np.array_equal(host16(k), wk)
    assert np.array_equal(_np(kc[:tokens], fmt), ek) and np.array_equal(_np(vc[:tokens], fmt), ev)
    assert not kc[tokens:].any().item() and not vc[tokens:].any().item()
    if es is not None:
        assert np.array_equal(sc[:tokens].cpu().numpy(), es)
        assert not sc[tokens:].any().item()


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("tree", [128, 256])
@pytest.mark.parametrize("tokens", [97, 400])
def test_reference_geometry_chain(oracle, fmt, tree, tokens):
    """The reference model's own shapes: hidden 2304, 32 Q heads, 4 KV heads
    (inference.cu:184-186, qk_rope_store_exact.cuh:23-26), ragged token counts on each
    launch shape (97: a wave per head vector; 400: four lanes per head)."""
    print(f"[case] reference geometry fmt={fmt} tree={tree} tokens={tokens}", flush=True)
    capacity, hidden, hq = 2048, 2304, 32
    d = synth.chain_inputs(tokens, hidden=hidden, q_heads=hq, outliers=True, seed=70 + fmt)
    tb = table_bits(oracle, capacity, theta=5e5)
    positions = np.arange(tokens, dtype=np.int32) + 1000
    wx, wy, wst, _ = oracle.residual_rmsnorm(d["x"], d["residual"], d["gamma"], threads=tree)
    wq, wk, _ = _qk_oracle(oracle, d, tb, positions)
    ek, ev, es = _expected_cache(oracle, fmt, wk, d["v"], positions, capacity, 0)
    x, r, g = dev(d["x"]), dev(d["residual"]), dev(d["gamma"])
    y = torch.empty_like(x)
    st = torch.empty((tokens, 2), dtype=torch.float32, device="cuda")
    q, k = dev(d["q"]), dev(d["k"])
    kc, vc, sc = _alloc_cache(fmt, capacity)
    state = _prefill_state(1000, tokens, capacity)
    bad = flag()
    ops.ResidualNormQKRopeStore(x, r, y, g, q, k, dev(d["v"]), dev(d["qn"]), dev(d["kn"]),
                                dev(tb), ops.positions_prefill(state, maximum=capacity),
                                ops.kv_cache(fmt, kc, vc, capacity, scales=sc), bad, tree=tree,
                                statistics=st)
    torch.cuda.synchronize()
    assert not bad.item()
    assert np.array_equal(host16(x), wx) and np.array_equal(host16(y), wy)
    assert np.array_equal(st.cpu().numpy(), wst)
    assert np.array_equal(host16(q), wq) and np.array_equal(host16(k), wk)
    assert np.array_equal(_np(kc, fmt), ek) and np.array_equal(_np(vc, fmt), ev)
    if es is not None:
        assert np.array_equal(sc.cpu().numpy(), es)


# ---- graph capture ----------------------------------------------------------------------------

@pytest.mark.parametrize("fmt", [abi.KV_BF16, abi.KV_Q8, abi.KV_Q8_0])
def test_decode_chain_graph_replays(oracle, fmt):
    """The decode step (residual norm, 256-thread tree, + Q/K norm/RoPE + KV store at each
    sequence's DecodeState position; BF16, or a quantized cache through the per-pair
    encoder) captured once into a graph and replayed at new positions: positions are read
    on the device, so each replay must match the oracle at the positions the state held
    when it ran.  Eager work and synchronizations run between the replays (state updates,
    input and cache resets)."""
    print(f"[case] decode chain graph replays fmt={fmt}", flush=True)
    seqs, capacity = 8, 512
    d = synth.chain_inputs(seqs, outliers=True, seed=81)
    tb = table_bits(oracle, capacity)
    x0, q0, k0 = dev(d["x"]), dev(d["q"]), dev(d["k"])
    x, q, k = x0.clone(), q0.clone(), k0.clone()
    r, g, v = dev(d["residual"]), dev(d["gamma"]), dev(d["v"])
    qn, kn, table = dev(d["qn"]), dev(d["kn"]), dev(tb)
    y = torch.empty_like(x)
    kc, vc, sc = _alloc_cache(fmt, seqs * capacity)
    states = torch.zeros((seqs, 8), dtype=torch.int32, device="cuda")
    bad = flag()
    pos = ops.positions_decode(states, maximum=capacity)
    kv = ops.kv_cache(fmt, kc, vc, capacity, scales=sc, seq_stride=capacity)

    def set_positions(p):
        host = np.zeros((seqs, 8), np.int32)
        for s, ps in enumerate(p):
            host[s] = [5, ps, capacity, 10, ps, min(int(ps), 1024), 0, 0]
        states.copy_(torch.from_numpy(host))

    rng = np.random.default_rng(82)
    set_positions(rng.integers(0, capacity, seqs))
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        ops.ResidualNormQKRopeStore(x, r, y, g, q, k, v, qn, kn, table, pos, kv, bad, tree=256)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            ops.ResidualNormQKRopeStore(x, r, y, g, q, k, v, qn, kn, table, pos, kv, bad,
                                        tree=256)
    torch.cuda.synchronize()
    wx, wy, _, _ = oracle.residual_rmsnorm(d["x"], d["residual"], d["gamma"], threads=256)
    for replay in range(4):
        p = rng.integers(0, capacity, seqs).astype(np.int32)
        set_positions(p)
        x.copy_(x0), q.copy_(q0), k.copy_(k0)
        kc.zero_(), vc.zero_()
        if sc is not None:
            sc.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert not bad.item(), replay
        wq, wk, _ = _qk_oracle(oracle, d, tb, p)
        assert np.array_equal(host16(x), wx) and np.array_equal(host16(y), wy), replay
        assert np.array_equal(host16(q), wq) and np.array_equal(host16(k), wk), replay
        kca = _np(kc, fmt).reshape(seqs, capacity, -1)
        vca = _np(vc, fmt).reshape(seqs, capacity, -1)
        sca = None if sc is None else sc.cpu().numpy().reshape(seqs, capacity, 4, 2)
        for s in range(seqs):
            ek, ev, es = _expected_cache(oracle, fmt, wk[s:s + 1], d["v"][s:s + 1],
                                         p[s:s + 1], capacity, 0)
            assert np.array_equal(kca[s], ek) and np.array_equal(vca[s], ev), (replay, s)
            if es is not None:
                assert np.array_equal(sca[s], es), (replay, s)


def _cancelling_heads(rng, tokens):
    """[tokens][4][128] floats whose rotation cancels: pattern (t * 4 + h) % 5 is
    0: features 32-63 equal 0-31 and 96-127 equal 64-95 (the bit-5 stage's differences
    are exact zeros), 1: every feature equal (every output but the first is zero),
    2: features 64-127 equal 0-63 (the K bit-6 stage's differences), 3: features 32-63
    the negation of 0-31 and 96-127 of 64-95 (zero sums), 4: unstructured."""
    x = rng.standard_normal((tokens, 4, 128)).astype(np.float32)
    kind = (np.arange(tokens)[:, None] * 4 + np.arange(4)[None, :]) % 5
    for t in range(tokens):
        for h in range(4):
            r = x[t, h]
            if kind[t, h] == 0:
                r[32:64], r[96:128] = r[0:32], r[64:96]
            elif kind[t, h] == 1:
                r[:] = r[0]
            elif kind[t, h] == 2:
                r[64:] = r[:64]
            elif kind[t, h] == 3:
                r[32:64], r[96:128] = -r[0:32], -r[64:96]
    return synth.bf16_bits(x)


@pytest.mark.parametrize("fmt", [abi.KV_Q8_0, abi.KV_Q8_0_NOROT])
@pytest.mark.parametrize("path", ["store", "chain"])
@pytest.mark.parametrize("tokens", [40, 400])
def test_q8_0_cancelling_heads(oracle, fmt, path, tokens):
    """K and V heads whose rotation stages produce exact zeros (equal or opposite halves):
    the cross-lane stages hold the upper lane's value negated and fold the signs into the
    scale multiply, so a zero there is -0 before the codes; the codes and scales must
    still equal the oracle's byte for byte.  Both the store-only encoder and the fused
    Q/K store (there the table is cos 1, sin 0 and the K norm weight 1, so K keeps its
    structure through the norm and RoPE), in both launch shapes."""
    print(f"[case] q8_0 cancelling heads fmt={fmt} path={path} tokens={tokens}", flush=True)
    capacity = 4096
    rng = np.random.default_rng(1234 + tokens)
    d = synth.chain_inputs(tokens, outliers=False, seed=5 + tokens)
    d["k"] = _cancelling_heads(rng, tokens).reshape(d["k"].shape)
    d["v"] = _cancelling_heads(rng, tokens).reshape(d["v"].shape)
    positions = np.arange(tokens, dtype=np.int32)
    kc, vc, _ = _alloc_cache(fmt, capacity)
    bad = flag()
    kv = ops.kv_cache(fmt, kc, vc, capacity)
    if path == "store":
        wk = d["k"]
        ops.KVStore(dev(d["k"]), dev(d["v"]), ops.positions_base(0), kv, bad)
    else:
        d["kn"] = np.full_like(d["kn"], 0x3F80)
        tb = np.zeros((capacity, 128), np.uint16)
        tb[:, :64] = 0x3F80
        wq, wk, _ = _qk_oracle(oracle, d, tb, positions)
        q, k = dev(d["q"]), dev(d["k"])
        ops.QKNormRopeStore(q, k, dev(d["qn"]), dev(d["kn"]), dev(tb), ops.positions_base(0),
                            bad, v=dev(d["v"]), kv=kv)
    torch.cuda.synchronize()
    assert not bad.item()
    ek, ev, _ = _expected_cache(oracle, fmt, wk, d["v"], positions, capacity, 0)
    if fmt == abi.KV_Q8_0:
        # the structure reaches the codes: most rotated codes of patterns 0-3 are zero
        assert (ek[:tokens, 32:] == 0).mean() > 0.3 and (ev[:tokens, 32:] == 0).mean() > 0.3
    if path == "chain":
        assert np.array_equal(host16(q), wq) and np.array_equal(host16(k), wk)
    assert np.array_equal(_np(kc, fmt), ek)
    assert np.array_equal(_np(vc, fmt), ev)
