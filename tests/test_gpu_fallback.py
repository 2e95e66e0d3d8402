"""GPU parity where the order-free sum of squares must give way to the reference tree.

Rows and heads built to put their exact sum of squares within 2^-58 of an fp32 rounding
midpoint (tests/tierows.py) fail the kernels' certificate, so every kernel that takes the
fp64 sum replays the reference's ordered tree for them.  They are mixed with ordinary
rows and heads in one launch, so waves that take the fallback and waves that do not run
side by side, and every output is compared with the oracle bit for bit.  The launch
shapes covered: the residual norm (a wave per row; a workgroup per row for the 256-thread
tree at few rows), the FP8 norm, the expert combine + norm, the Q/K launch (four lanes per head; a wave per head),
and the fused chain in each of its shapes.
"""
import numpy as np
import pytest
import torch

from padra_amd import abi, ops, synth
from tierows import certified, margin, near_midpoint_row

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    abi.lib()
    yield
    torch.cuda.synchronize()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()


def host16(t):
    return t.cpu().numpy().view(np.uint16)


def flag():
    return torch.zeros(1, dtype=torch.int32, device="cuda")


def _tie(rng, n):
    row = near_midpoint_row(rng, n, 2.0**-58, bool(rng.integers(2)))
    # any margin the kernels use refuses it (their largest depth term is far below 2^-58)
    assert not certified(float(np.sum(row.astype(np.float64) ** 2)), margin(1, 1))[0]
    return row


def tie_inputs(tokens, hidden=2048, seed=0):
    """Chain inputs in which every other row of x (residual zero there, so v = x) and
    every third Q head and every other K head sit next to an fp32 midpoint."""
    rng = np.random.default_rng(seed)
    d = synth.chain_inputs(tokens, hidden=hidden, outliers=True, seed=seed)
    zero = synth.bf16_bits(np.zeros(hidden))
    for t in range(0, tokens, 2):
        d["x"][t] = synth.bf16_bits(_tie(rng, hidden))
        d["residual"][t] = zero
    for t in range(tokens):
        for h in range(d["q"].shape[1]):
            if (t * d["q"].shape[1] + h) % 3 == 0:
                d["q"][t, h] = synth.bf16_bits(_tie(rng, 128))
        for h in range(d["k"].shape[1]):
            if (t + h) % 2 == 0:
                d["k"][t, h] = synth.bf16_bits(_tie(rng, 128))
    return d


@pytest.mark.parametrize("tree,rows", [(128, 3), (128, 70), (256, 3), (256, 160)])
def test_fallback_residual_norm(oracle, tree, rows):
    print(f"[case] fallback residual norm tree={tree} rows={rows}", flush=True)
    d = tie_inputs(rows, seed=rows + tree)
    want_x, want_y, want_st, _ = oracle.residual_rmsnorm(d["x"], d["residual"], d["gamma"],
                                                         threads=tree)
    x, y = dev(d["x"]), torch.empty_like(dev(d["x"]))
    st = torch.empty((rows, 2), dtype=torch.float32, device="cuda")
    bad = flag()
    ops.ResidualPostNorm(x, dev(d["residual"]), y, dev(d["gamma"]), bad, tree=tree,
                         statistics=st)
    torch.cuda.synchronize()
    assert not bad.item()
    assert np.array_equal(host16(x), want_x) and np.array_equal(host16(y), want_y)
    assert np.array_equal(st.cpu().numpy(), want_st)


def test_fallback_norm_fp8(oracle):
    print("[case] fallback FP8 norm", flush=True)
    rows = 40
    d = tie_inputs(rows, seed=5)
    want_y, want_codes, want_scales, _, _ = oracle.norm_fp8(d["x"], d["gamma"])
    y = torch.empty_like(dev(d["x"]))
    packed = torch.zeros((rows, 2048), dtype=torch.uint8, device="cuda")
    scales = torch.zeros(rows, dtype=torch.float32, device="cuda")
    bad = flag()
    ops.NormFP8(dev(d["x"]), y, dev(d["gamma"]), packed, scales, bad)
    torch.cuda.synchronize()
    assert np.array_equal(host16(y), want_y)
    assert np.array_equal(packed.cpu().numpy(), want_codes)
    assert np.array_equal(scales.cpu().numpy(), want_scales)


@pytest.mark.parametrize("hidden", [2048, 2304, 4608])
@pytest.mark.parametrize("fp8", [True, False])
def test_fallback_combine_norm(oracle, hidden, fp8):
    """Expert combine + norm (+ FP8), four waves per row: every other row's expert rows are
    zero, so its combined row is x, a row next to an fp32 midpoint."""
    print(f"[case] fallback combine norm hidden={hidden} fp8={fp8}", flush=True)
    rows = 40
    d = tie_inputs(rows, hidden=hidden, seed=hidden + fp8)
    rng = np.random.default_rng(hidden)
    down = synth.bf16_bits((rng.standard_normal((rows, 8, hidden)) * 0.5).astype(np.float32))
    down[0::2] = 0
    w = rng.dirichlet(np.ones(8), rows).astype(np.float32)
    want_x, want_y, want_p, want_s, want_st, want_bad = oracle.combine_norm(
        d["x"], down, w, d["gamma"], fp8=fp8)
    assert not want_bad
    x = dev(d["x"])
    y = torch.empty_like(x)
    packed = torch.zeros((rows, hidden), dtype=torch.uint8, device="cuda") if fp8 else None
    scales = torch.zeros(rows, dtype=torch.float32, device="cuda") if fp8 else None
    st = torch.empty(2, dtype=torch.float32, device="cuda")
    bad = flag()
    ops.CombineNorm(x, dev(down), torch.from_numpy(w).cuda(), y, dev(d["gamma"]), bad,
                    packed=packed, scales=scales, statistics=st)
    torch.cuda.synchronize()
    assert not bad.item()
    assert np.array_equal(host16(x), want_x) and np.array_equal(host16(y), want_y)
    assert np.array_equal(st.cpu().numpy(), want_st)
    if fp8:
        assert np.array_equal(packed.cpu().numpy(), want_p)
        assert np.array_equal(scales.cpu().numpy(), want_s)


@pytest.mark.parametrize("tokens", [24, 400])
def test_fallback_qk(oracle, tokens):
    print(f"[case] fallback Q/K tokens={tokens}", flush=True)
    d = tie_inputs(tokens, seed=tokens)
    tb = synth.bf16_bits(oracle.rope_table(tokens + 8, 128, 1e6))
    positions = np.arange(tokens, dtype=np.int32) + 3
    wq, wk, _ = oracle.qk_norm_rope(d["q"], d["k"], d["qn"], d["kn"], tb, positions)
    q, k = dev(d["q"]), dev(d["k"])
    bad = flag()
    ops.QKNormRopeStore(q, k, dev(d["qn"]), dev(d["kn"]), dev(tb), ops.positions_base(3), bad)
    torch.cuda.synchronize()
    assert not bad.item()
    assert np.array_equal(host16(q), wq) and np.array_equal(host16(k), wk)


@pytest.mark.parametrize("tree,tokens", [(128, 40), (256, 40), (128, 400), (256, 400)])
@pytest.mark.parametrize("fmt", [abi.KV_BF16, abi.KV_Q8_0])
def test_fallback_chain(oracle, tree, tokens, fmt):
    """The fused chain in each launch shape: per-head waves with norm-row waves (128 tree)
    or norm-row workgroups (256 tree) at 40 tokens, four lanes per head at 400.  The
    quantized cache keeps the ordered tree throughout; it is here as the control."""
    print(f"[case] fallback chain tree={tree} tokens={tokens} fmt={fmt}", flush=True)
    cap = 1024
    d = tie_inputs(tokens, seed=tree + tokens + fmt)
    tb = synth.bf16_bits(oracle.rope_table(cap, 128, 1e6))
    positions = np.arange(tokens, dtype=np.int32) + 9
    wx, wy, wst, _ = oracle.residual_rmsnorm(d["x"], d["residual"], d["gamma"], threads=tree)
    wq, wk, _ = oracle.qk_norm_rope(d["q"], d["k"], d["qn"], d["kn"], tb, positions)
    if fmt == abi.KV_BF16:
        ek = np.zeros((cap, 512), np.uint16)
        ev = np.zeros((cap, 512), np.uint16)
        oracle.kv_store_bf16(wk, d["v"], ek, ev, positions, cap, 0)
        kc = torch.zeros((cap, 512), dtype=torch.int16, device="cuda")
        vc = torch.zeros_like(kc)
    else:
        ek = np.zeros((cap, 544), np.uint8)
        ev = np.zeros((cap, 544), np.uint8)
        assert not oracle.kv_q8_0_encode(wk, d["v"], ek, ev, positions, cap, 0, rotate=True)
        kc = torch.zeros((cap, 544), dtype=torch.uint8, device="cuda")
        vc = torch.zeros_like(kc)
    x, q, k = dev(d["x"]), dev(d["q"]), dev(d["k"])
    y = torch.empty_like(x)
    st = torch.empty((tokens, 2), dtype=torch.float32, device="cuda")
    bad = flag()
    ops.ResidualNormQKRopeStore(x, dev(d["residual"]), y, dev(d["gamma"]), q, k, dev(d["v"]),
                                dev(d["qn"]), dev(d["kn"]), dev(tb), ops.positions_base(9),
                                ops.kv_cache(fmt, kc, vc, cap), bad, tree=tree, statistics=st)
    torch.cuda.synchronize()
    assert not bad.item()
    assert np.array_equal(host16(x), wx) and np.array_equal(host16(y), wy)
    assert np.array_equal(st.cpu().numpy(), wst)
    assert np.array_equal(host16(q), wq) and np.array_equal(host16(k), wk)
    view = (lambda t: host16(t)) if fmt == abi.KV_BF16 else (lambda t: t.cpu().numpy())
    assert np.array_equal(view(kc), ek) and np.array_equal(view(vc), ev)
