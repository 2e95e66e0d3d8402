"""Pins the CPU oracle (oracle/padra_oracle.c) against things other than itself.

Per oracle function, what checks it:
  po_f32_to_bf16 / po_bf16_round  torch's RNE float->bfloat16 cast, specials
  po_f32_to_f16                   numpy's float32->float16 cast (RNE, subnormals), all
                                  2^16 half values round trip
  po_accumulate / po_sumsq_tree   tests/refsim.py (thread-level simulation of the CUDA
                                  kernels) on order-sensitive golden inputs and random
                                  rows; exact rational sums (|error| <= 1 ulp)
  po_rms_inv                      numpy float32 arithmetic (correctly rounded)
  po_residual_rmsnorm/po_rmsnorm  refsim rows (bitwise), closed forms (zero row,
                                  constant row), float64 formula within 1 BF16 ulp
  po_rope_table                   identity row at p=0, float64 cos/sin of the same
                                  float32 angle, YaRN ramp constants of the reference
  po_qk_norm_rope                 pos 0 = plain norm, float64 rotation within 1 ulp,
                                  refsim norm of a head (bitwise)
  po_kv_store_bf16                ring addressing: last `cap` rows win, rows < first skipped
  po_kv_q8_encode                 numpy float32 division + rint, |code|<=127, max 127
  po_hadamard                     scipy.linalg.hadamard on integer inputs (exact)
  po_kv_q8_0_encode               roundf half-away ties, fp16 scale via numpy, decode error
                                  bound, rotation self-inverse
  po_kv_q8_0_dequantize           bf16(code * fp16 d) via torch
  po_silu_table                   all 65536 gates against a long-double evaluation
  po_embed / state predicates     numpy indexing; reference truth tables
  po_e4m3                         torch float8_e4m3fn (RNE) on every finite BF16 value and
                                  random float32 below 464; saturation and NaN by the OCP
                                  format definition
  po_fp8_encode                   equals the code of a correctly rounded division (numpy
                                  float32 + torch) on values aimed at every E4M3 midpoint
  po_norm_fp8                     y = po_rmsnorm's, scale = max|y|/448, codes = torch
                                  float8 of y/scale, zero row, non-finite row
  po_quantize_fp8                 scale = max|x|/448, codes = torch float8 of numpy's x/scale
  po_combine                      one-hot weights give B(x + down_e); power-of-two weights
                                  on small integers are exact; float64 weighted sum within
                                  the rounding bound; the expert order of the accumulation
  po_combine_norm                 = po_combine, then po_norm_fp8 / po_rmsnorm of the new x
  po_kv_checkpoint_*              slot contents by search over positions (the newest p <
                                  anchor with p = slot mod 1024), admission truth table
  po_decode_attention             float64 softmax attention over the same keys (global and
                                  local ring) within the BF16-probability error bound; the
                                  split count changes results only within that bound
  po_decode_attention_q8_0        float64 attention of the original query over the cache's
                                  decoded rows rotated back, within the query-coding bound
"""
import numpy as np
import pytest
import torch
from fractions import Fraction

from padra_amd import synth

import refsim

F32 = np.float32


def f32bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


# ---- A1 -------------------------------------------------------------------------------

def test_bf16_round_matches_torch(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.exp2(rng.integers(-130, 127, 20000)),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.3895314e38, 3.3961514e38, 3.39615e38,
                  1e-40, -1e-41, 1.0 + 2**-8, 1.0 + 3 * 2**-8], np.float32)]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = synth.bf16_bits(x)
    assert np.array_equal(got, ref)
    lib = oracle.lib()
    for v in x[::97]:
        assert F32(lib.po_bf16_round(float(v))).tobytes() == synth.bf16_to_f32(
            synth.bf16_bits(np.array([v])))[0].tobytes()


def test_f16_conversion_matches_numpy(oracle):
    lib = oracle.lib()
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(5000).astype(np.float32) * np.exp2(rng.integers(-30, 18, 5000)),
        np.array([65504, 65519.99, 65520, 2**-24, 2**-25, 3 * 2**-26, 2**-14, 0.0, -0.0],
                 np.float32)]).astype(np.float32)
    for v in x:
        assert lib.po_f32_to_f16(float(v)) == int(np.float16(v).view(np.uint16)), v
    halves = np.arange(65536, dtype=np.uint16).view(np.float16)
    finite = np.isfinite(halves)
    for h, v in zip(np.nonzero(finite)[0][::7], halves[finite][::7]):
        assert F32(lib.po_f16_to_f32(int(h))) == F32(v)


# ---- reduction order ----------------------------------------------------------------

def test_sumsq_tree_golden_order_sensitive(oracle):
    g = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                           "reduction_order.npz"))
    lib = oracle.lib()
    v = np.ascontiguousarray(g["v512"])
    ptr = v.ctypes.data_as(__import__("ctypes").c_void_p)
    t128, t256 = F32(lib.po_sumsq_tree(ptr, 512, 128)), F32(lib.po_sumsq_tree(ptr, 512, 256))
    assert t128 == g["v512_tree128"] and t256 == g["v512_tree256"]
    assert t128 != t256  # the fixture separates the two trees
    # the 128-thread tree is the correctly rounded one here; the 256 tree drops 2^-18
    exact = sum(Fraction(float(x)) ** 2 for x in v)
    assert abs(Fraction(float(t128)) - exact) < abs(Fraction(float(t256)) - exact)
    for h, want in zip(g["head128"], g["head128_tree128"]):
        h = np.ascontiguousarray(h)
        assert F32(lib.po_sumsq_tree(h.ctypes.data_as(__import__("ctypes").c_void_p), 128,
                                     128)) == want


@pytest.mark.parametrize("threads", [128, 256])
def test_sumsq_tree_matches_refsim_random(oracle, threads):
    import ctypes
    lib = oracle.lib()
    rng = np.random.default_rng(threads)
    for n in (256, 512, 768):
        v = synth.bf16_to_f32(synth.bf16_bits(rng.standard_normal(n) * np.exp2(
            rng.integers(-8, 8, n))))
        got = F32(lib.po_sumsq_tree(v.ctypes.data_as(ctypes.c_void_p), n, threads))
        assert got == refsim.block_sumsq(v, threads)
        exact = sum(Fraction(float(x)) ** 2 for x in v)
        ulp = np.spacing(got)
        assert abs(Fraction(float(got)) - exact) <= Fraction(float(ulp))


def test_rms_inv_numpy(oracle):
    import ctypes
    lib = oracle.lib()
    rng = np.random.default_rng(3)
    _, st, _ = oracle.rmsnorm(np.zeros((1, 128), np.uint16), np.zeros(128, np.uint16))
    assert st[0, 0] == 0 and st[0, 1] == F32(F32(1) / np.sqrt(F32(1e-6)))
    # direct: variance and inv of a random row follow numpy float32 arithmetic
    x = synth.bf16_bits(rng.standard_normal((4, 2048)))
    _, st, _ = oracle.rmsnorm(x, synth.bf16_bits(np.ones(2048)))
    for r in range(4):
        xv = synth.bf16_to_f32(x[r])
        s = F32(lib.po_sumsq_tree(np.ascontiguousarray(xv).ctypes.data_as(ctypes.c_void_p),
                                  2048, 128))
        var = F32(s / F32(2048))
        assert st[r, 0] == var
        assert st[r, 1] == F32(F32(1) / np.sqrt(F32(var + F32(1e-6))))


# ---- A2 / A3 -------------------------------------------------------------------------

@pytest.mark.parametrize("threads", [128, 256])
def test_residual_norm_matches_refsim(oracle, threads):
    rng = np.random.default_rng(10 + threads)
    hidden = 512
    x = synth.bf16_bits(rng.standard_normal((2, hidden)))
    r = synth.bf16_bits(rng.standard_normal((2, hidden)) * 3)
    g = synth.bf16_bits(rng.uniform(0.5, 1.5, hidden))
    xn, y, st, bad = oracle.residual_rmsnorm(x, r, g, threads=threads)
    assert not bad
    for row in range(2):
        v = [refsim.bf16(F32(a + b)) for a, b in zip(synth.bf16_to_f32(x[row]),
                                                    synth.bf16_to_f32(r[row]))]
        assert np.array_equal(synth.bf16_to_f32(xn[row]), np.array(v, np.float32))
        want, var, inv = refsim.norm_row(v, synth.bf16_to_f32(g), threads)
        assert np.array_equal(synth.bf16_to_f32(y[row]), np.array(want, np.float32))
        assert st[row, 0] == var and st[row, 1] == inv


def test_residual_norm_closed_forms(oracle):
    hidden = 2048
    zero = np.zeros((1, hidden), np.uint16)
    g = synth.bf16_bits(np.linspace(0.5, 1.5, hidden))
    xn, y, st, bad = oracle.residual_rmsnorm(zero, zero, g)
    assert not bad and not y.any() and st[0, 0] == 0
    c = F32(0.75)
    row = synth.bf16_bits(np.full((1, hidden), c))
    ones = synth.bf16_bits(np.ones(hidden))
    y, st, _ = oracle.rmsnorm(row, ones)
    inv = F32(F32(1) / np.sqrt(F32(F32(c * c) + F32(1e-6))))  # S/H = c^2 exactly
    assert st[0, 1] == inv
    assert np.all(synth.bf16_to_f32(y) == refsim.bf16(F32(c * inv)))


@pytest.mark.parametrize("threads", [128, 256])
def test_residual_norm_float64_within_1p5_ulp(oracle, threads):
    d = synth.chain_inputs(64, outliers=True, seed=4)
    xn, y, st, bad = oracle.residual_rmsnorm(d["x"], d["residual"], d["gamma"], threads=threads)
    assert not bad
    v = (synth.bf16_to_f32(d["x"]).astype(np.float64) + synth.bf16_to_f32(d["residual"]))
    v = synth.bf16_to_f32(synth.bf16_bits(v.astype(np.float32))).astype(np.float64)
    inv = 1 / np.sqrt((v * v).mean(axis=1, keepdims=True) + 1e-6)
    ref = v * inv * synth.bf16_to_f32(d["gamma"])
    got = synth.bf16_to_f32(y).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
    # two BF16 roundings (B(v*inv), then B(.*gamma)): within 1.5 ulp of the exact value
    assert np.all(np.abs(got - ref) <= 1.5 * ulp)


def test_residual_norm_nonfinite_sets_bad(oracle):
    d = synth.chain_inputs(2, seed=5)
    x = d["x"].copy()
    x[1, 7] = 0x7F80  # +inf
    _, _, _, bad = oracle.residual_rmsnorm(x, d["residual"], d["gamma"])
    assert bad


# ---- A3 FP8 ----------------------------------------------------------------------------

def torch_e4m3(values):
    return torch.from_numpy(np.ascontiguousarray(values, np.float32)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_matches_torch(oracle):
    bf = np.arange(65536, dtype=np.uint32)
    vals = (bf << 16).view(np.float32)
    vals = vals[np.isfinite(vals) & (np.abs(vals) < 464)]
    rng = np.random.default_rng(11)
    rand = rng.integers(0, 2**32, 60000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    rand = rand[np.isfinite(rand) & (np.abs(rand) < 464)]
    for v in (vals, rand):
        assert np.array_equal(oracle.e4m3(v), torch_e4m3(v))


def test_e4m3_saturation_and_nan(oracle):
    big = np.array([464, 480, 1e6, 3e38, np.inf], np.float32)
    assert np.all(oracle.e4m3(big) == 0x7E) and np.all(oracle.e4m3(-big) == 0xFE)
    assert oracle.e4m3([np.nan])[0] == 0x7F and oracle.e4m3([-np.nan])[0] == 0x7F
    # the 127 finite positive codes decode to k * 2^-9 (subnormal) or 2^(e-7) (1 + m/8)
    for code in range(0x7F):
        e, m = code >> 3, code & 7
        value = m * 2.0**-9 if e == 0 else 2.0**(e - 7) * (1 + m / 8)
        assert oracle.e4m3([value])[0] == code


def test_fp8_encode_equals_division(oracle):
    """The cached-reciprocal path with its midpoint fallback gives the code of the correctly
    rounded quotient, on BF16 values aimed at E4M3 rounding midpoints."""
    rng = np.random.default_rng(12)
    amax = synth.bf16_to_f32(synth.bf16_bits(np.exp2(rng.uniform(-30, 30, 120)).astype(F32)))
    codes = np.arange(0x7E, dtype=np.float64)
    grid = np.where(codes < 8, codes * 2.0**-9, 2.0**((codes // 8) - 7) * (1 + (codes % 8) / 8))
    mids = (grid[:-1] + grid[1:]) / 2
    enc = oracle.lib().po_fp8_encode
    checked = 0
    for a in amax:
        scale = F32(a / F32(448))
        inverse = F32(F32(1) / scale)
        target = synth.bf16_bits((mids * np.float64(scale)).astype(F32)).astype(np.int64)
        vals = np.concatenate([target + d for d in (-2, -1, 0, 1, 2)])
        vals = synth.bf16_to_f32(np.clip(vals, 0, 0x7F7F).astype(np.uint16))
        vals = vals[np.abs(vals) <= a]
        vals = np.concatenate([vals, -vals])
        want = torch_e4m3(vals / scale)
        got = np.array([enc(float(v), float(scale), float(inverse)) for v in vals], np.uint8)
        assert np.array_equal(got, want), a
        checked += len(vals)
    assert checked > 100000


def test_norm_fp8(oracle):
    d = synth.chain_inputs(12, hidden=2304, outliers=True, seed=13)
    x = d["x"].copy()
    x[3] = 0  # all-zero row: scale 1, codes 0
    y, packed, scales, stats, bad = oracle.norm_fp8(x, d["gamma"])
    assert not bad
    y_ref, st_ref, _ = oracle.rmsnorm(x, d["gamma"], threads=128)
    assert np.array_equal(y, y_ref) and np.array_equal(stats, st_ref[0])
    yf = synth.bf16_to_f32(y)
    amax = np.abs(yf).max(axis=1)
    want_scale = np.where(amax == 0, F32(1), (amax / F32(448)).astype(F32))
    assert np.array_equal(scales, want_scale) and scales[3] == 1
    assert np.array_equal(packed, torch_e4m3(yf / scales[:, None]))
    x[5, 9] = 0x7FC0  # NaN input
    *_, bad = oracle.norm_fp8(x, d["gamma"])
    assert bad


def test_quantize_fp8(oracle):
    rng = np.random.default_rng(25)
    x = (rng.standard_normal((6, 4096)) * np.exp2(rng.integers(-20, 20, (6, 1)))).astype(F32)
    x[2] = 0
    packed, scales, bad = oracle.quantize_fp8(x)
    assert not bad and scales[2] == 1 and not packed[2].any()
    amax = np.abs(x).max(axis=1)
    want = np.where(amax == 0, F32(1), (amax / F32(448)).astype(F32))
    assert np.array_equal(scales, want)
    assert np.array_equal(packed, torch_e4m3(x / scales[:, None]))
    x[4, 9] = np.inf
    assert oracle.quantize_fp8(x)[2]


# ---- Expert combine ---------------------------------------------------------------------

def test_combine_closed_forms(oracle):
    rng = np.random.default_rng(21)
    rows, experts, hidden = 3, 8, 256
    x = synth.bf16_bits(rng.standard_normal((rows, hidden)).astype(F32))
    down = synth.bf16_bits(rng.standard_normal((rows, experts, hidden)).astype(F32))
    onehot = np.zeros((rows, experts), F32)
    onehot[np.arange(rows), [0, 5, 7]] = 1
    got, bad = oracle.combine(x, down, onehot)
    pick = down[np.arange(rows), [0, 5, 7]]
    want = synth.bf16_bits(synth.bf16_to_f32(x) + synth.bf16_to_f32(pick))
    assert not bad and np.array_equal(got, want)
    got, _ = oracle.combine(x, down, onehot, residual=False)
    assert np.array_equal(got, pick)
    # small integers times powers of two: every step exact
    ints = rng.integers(-8, 9, (rows, experts, hidden)).astype(F32)
    w = np.exp2(-rng.integers(0, 4, (rows, experts))).astype(F32)
    got, _ = oracle.combine(np.zeros((rows, hidden), np.uint16), synth.bf16_bits(ints), w,
                            residual=False)
    assert np.array_equal(synth.bf16_to_f32(got), (ints * w[:, :, None]).sum(axis=1))


def test_combine_rounding_bound_and_order(oracle):
    rng = np.random.default_rng(22)
    rows, experts, hidden = 4, 8, 512
    down = synth.bf16_bits(rng.standard_normal((rows, experts, hidden)).astype(F32))
    w = rng.dirichlet(np.ones(experts), rows).astype(F32)
    got, _ = oracle.combine(np.zeros((rows, hidden), np.uint16), down, w, residual=False)
    exact = (synth.bf16_to_f32(down).astype(np.float64) * w[:, :, None]).sum(axis=1)
    # 16 BF16 roundings of partial sums bounded by sum |d w|
    bound = 16 * 2.0**-8 * (np.abs(synth.bf16_to_f32(down)) * w[:, :, None]).sum(axis=1)
    assert np.all(np.abs(synth.bf16_to_f32(got) - exact) <= bound + 1e-30)
    # the accumulation runs e = 0..7: reversing the experts changes some results
    rev, _ = oracle.combine(np.zeros((rows, hidden), np.uint16), down[:, ::-1].copy(),
                            w[:, ::-1].copy(), residual=False)
    assert not np.array_equal(rev, got)
    seq = np.zeros((rows, hidden), F32)
    for e in range(experts):
        prod = synth.bf16_to_f32(synth.bf16_bits(synth.bf16_to_f32(down[:, e]) * w[:, e:e + 1]))
        seq = synth.bf16_to_f32(synth.bf16_bits(seq + prod))
    assert np.array_equal(synth.bf16_to_f32(got), seq)


def test_combine_norm_composition(oracle):
    rng = np.random.default_rng(23)
    rows, experts, hidden = 5, 8, 2304
    d = synth.chain_inputs(rows, hidden=hidden, outliers=True, seed=24)
    down = synth.bf16_bits(rng.standard_normal((rows, experts, hidden)).astype(F32))
    w = rng.dirichlet(np.ones(experts), rows).astype(F32)
    xn, y, packed, scales, stats, bad = oracle.combine_norm(d["x"], down, w, d["gamma"])
    assert not bad
    want_x, _ = oracle.combine(d["x"], down, w)
    assert np.array_equal(xn, want_x)
    y2, p2, s2, st2, _ = oracle.norm_fp8(want_x, d["gamma"])
    assert np.array_equal(y, y2) and np.array_equal(packed, p2) and np.array_equal(scales, s2)
    assert np.array_equal(stats, st2)
    _, y3, none_p, none_s, _, _ = oracle.combine_norm(d["x"], down, w, d["gamma"], fp8=False)
    assert none_p is None and np.array_equal(y3, y)


# ---- A5 --------------------------------------------------------------------------------

def test_rope_table_plain(oracle):
    t = oracle.rope_table(4096, 128, 1e6)
    assert np.all(t[0, :64] == 1) and np.all(t[0, 64:] == 0)
    i = np.arange(64)
    freq = (F32(1) / np.power(F32(1e6), (2 * i).astype(np.float32) / F32(128))).astype(np.float32)
    mismatch = 0
    for p in (1, 7, 4097 % 4096, 4095):
        ang = (F32(p) * freq).astype(np.float32).astype(np.float64)
        c = synth.bf16_to_f32(synth.bf16_bits(np.cos(ang).astype(np.float32)))
        s = synth.bf16_to_f32(synth.bf16_bits(np.sin(ang).astype(np.float32)))
        mismatch += int((t[p, :64] != c).sum() + (t[p, 64:] != s).sum())
        assert np.all(np.abs(t[p, :64] - c) <= 2 ** -8) and np.all(np.abs(t[p, 64:] - s) <= 2 ** -8)
    assert mismatch <= 2
    norm = t[:, :64].astype(np.float64) ** 2 + t[:, 64:].astype(np.float64) ** 2
    assert np.all(np.abs(norm - 1) < 2 ** -6)


def test_rope_table_yarn_ramp(oracle):
    # reference constants: theta 5e5, factor 16, original context 8192 -> low 18, high 35
    t = oracle.rope_table(2, 128, 5e5, yarn=True, factor=16.0, original_context=8192)
    scale = F32(1 + 0.1 * np.log(16.0))
    i = np.arange(64)
    freq = np.power(F32(5e5), (2 * i).astype(np.float32) / F32(128)).astype(np.float32)
    ramp = np.clip((i - 18.0) / (35.0 - 18.0), 0, 1)
    f = (1 / (16 * freq.astype(np.float64))) * ramp + (1 / freq.astype(np.float64)) * (1 - ramp)
    c = np.cos(f) * scale
    assert np.all(np.abs(t[1, :64] - c) <= np.abs(c) * 2 ** -7 + 1e-6)
    assert np.all(t[0, :64] == synth.bf16_to_f32(synth.bf16_bits(np.full(64, scale))))


# ---- A4 / A6 ----------------------------------------------------------------------------

def _table_bits(oracle, n, theta=1e6):
    return synth.bf16_bits(oracle.rope_table(n, 128, theta))


def test_qk_rope_position_zero_is_norm(oracle):
    d = synth.chain_inputs(3, seed=6)
    tb = _table_bits(oracle, 8)
    q, k, bad = oracle.qk_norm_rope(d["q"], d["k"], d["qn"], d["kn"], tb, np.zeros(3, np.int32))
    assert not bad
    yq, _, _ = oracle.rmsnorm(d["q"].reshape(-1, 128), d["qn"])
    yk, _, _ = oracle.rmsnorm(d["k"].reshape(-1, 128), d["kn"])
    assert np.array_equal(q.reshape(-1, 128), yq) and np.array_equal(k.reshape(-1, 128), yk)


def test_qk_rope_head_refsim_and_float64(oracle):
    d = synth.chain_inputs(4, seed=7, outliers=True)
    tb = _table_bits(oracle, 5000)
    pos = np.array([0, 1, 4097, 4999], np.int32)
    q, k, bad = oracle.qk_norm_rope(d["q"], d["k"], d["qn"], d["kn"], tb, pos)
    assert not bad
    tf = synth.bf16_to_f32(tb)
    for t in range(4):
        head = synth.bf16_to_f32(d["k"][t, 2])
        o, _, _ = refsim.norm_row(head, synth.bf16_to_f32(d["kn"]), 128)
        o = np.array(o, np.float32)
        c, s = tf[pos[t], :64], tf[pos[t], 64:]
        lo = [refsim.bf16(F32(refsim.bf16(F32(a * cc)) + refsim.bf16(F32(-b * ss))))
              for a, b, cc, ss in zip(o[:64], o[64:], c, s)]
        hi = [refsim.bf16(F32(refsim.bf16(F32(b * cc)) + refsim.bf16(F32(a * ss))))
              for a, b, cc, ss in zip(o[:64], o[64:], c, s)]
        assert np.array_equal(synth.bf16_to_f32(k[t, 2]), np.array(lo + hi, np.float32))
        # float64 rotation of the normalized head agrees to BF16 rounding
        ref = np.concatenate([o[:64] * c - o[64:] * s, o[64:] * c + o[:64] * s]).astype(np.float64)
        got = synth.bf16_to_f32(k[t, 2])
        # each product is rounded to BF16 before the add: bound by the term magnitudes
        terms = np.concatenate([np.abs(o[:64] * c) + np.abs(o[64:] * s),
                                np.abs(o[64:] * c) + np.abs(o[:64] * s)]).astype(np.float64)
        assert np.all(np.abs(got - ref) <= 2 ** -8 * terms + 2 ** -8 * 1.01 * np.abs(ref) + 1e-30)


def test_qk_head_golden_order(oracle):
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "reduction_order.npz"))
    for h, want in zip(g["head128"], g["head128_tree128"]):
        bits = synth.bf16_bits(h).reshape(1, 1, 128)
        ones = synth.bf16_bits(np.ones(128))
        tb = _table_bits(oracle, 1)
        q, _, _ = oracle.qk_norm_rope(bits, bits.copy(), ones, ones, tb, np.zeros(1, np.int32))
        var = F32(want / F32(128))
        inv = F32(F32(1) / np.sqrt(F32(var + F32(1e-6))))
        exp = np.array([refsim.bf16(F32(refsim.bf16(F32(x * inv)))) for x in h], np.float32)
        assert np.array_equal(synth.bf16_to_f32(q[0, 0]), exp)


def test_kv_store_ring(oracle):
    d = synth.chain_inputs(10, seed=8)
    cap = 4
    kc = np.zeros((cap, 512), np.uint16)
    vc = np.zeros((cap, 512), np.uint16)
    pos = np.arange(100, 110, dtype=np.int32)
    oracle.kv_store_bf16(d["k"], d["v"], kc, vc, pos, cap, first=10 - cap)
    for t in range(6, 10):
        assert np.array_equal(kc[pos[t] % cap], d["k"][t].reshape(-1))
        assert np.array_equal(vc[pos[t] % cap], d["v"][t].reshape(-1))


# ---- A7 ---------------------------------------------------------------------------------

def test_kv_q8_codes(oracle):
    d = synth.chain_inputs(6, seed=9, outliers=True)
    cap = 8
    ck = np.zeros((cap, 512), np.int8)
    cv = np.zeros((cap, 512), np.int8)
    sc = np.zeros((cap, 4, 2), np.float32)
    pos = np.arange(6, dtype=np.int32) + 3
    assert not oracle.kv_q8_encode(d["k"], d["v"], ck, cv, sc, pos, cap)
    for t in range(6):
        for h in range(4):
            for src, codes, j in ((d["k"], ck, 0), (d["v"], cv, 1)):
                x = synth.bf16_to_f32(src[t, h])
                am = np.abs(x).max()
                s = F32(am / F32(127)) if am else F32(1)
                assert sc[pos[t] % cap, h, j] == s
                want = np.clip(np.rint(x / s), -127, 127).astype(np.int8)
                got = codes[pos[t] % cap, h * 128:(h + 1) * 128]
                assert np.array_equal(got, want)
                assert np.abs(got).max() == 127
                assert np.all(np.abs(got * s - x) <= s / 2 * (1 + 2 ** -20))


# ---- A8 ---------------------------------------------------------------------------------

def test_hadamard_matches_sylvester(oracle):
    from scipy.linalg import hadamard
    rng = np.random.default_rng(11)
    for n, scale in ((128, 1.0), (64, 1.0)):
        x = rng.integers(-50, 50, n).astype(np.float32)
        assert np.array_equal(oracle.hadamard(x, scale), (hadamard(n) @ x).astype(np.float32))
    x = rng.standard_normal(128).astype(np.float32)
    twice = oracle.hadamard(oracle.hadamard(x, .08838834764831845), .08838834764831845)
    assert np.allclose(twice, x, atol=1e-5)


def _row_fields(rows, features=512):
    nd = features // 32
    d = rows[:, :2 * nd].copy().view(np.float16)
    qs = rows[:, 2 * nd:2 * nd + features].view(np.int8)
    return d, qs


@pytest.mark.parametrize("rotate", [True, False])
def test_kv_q8_0_encode(oracle, rotate):
    d = synth.chain_inputs(5, seed=12, outliers=True)
    cap = 8
    rb = 544
    rk = np.zeros((cap, rb), np.uint8)
    rv = np.zeros((cap, rb), np.uint8)
    pos = np.arange(5, dtype=np.int32)
    assert not oracle.kv_q8_0_encode(d["k"], d["v"], rk, rv, pos, cap, rotate=rotate)
    dk, qk = _row_fields(rk)
    for t in range(5):
        for h in range(4):
            x = synth.bf16_to_f32(d["k"][t, h])
            if rotate:
                x = oracle.hadamard(x, .08838834764831845)
            for r in range(4):
                blk = x[32 * r:32 * r + 32]
                ad = F32(np.abs(blk).max() / F32(127))
                assert dk[t, h * 4 + r] == np.float16(ad)
                inv = F32(F32(1) / ad)
                prod = (blk * inv).astype(np.float32)
                want = np.clip(np.sign(prod) * np.floor(np.abs(prod) + 0.5), -127, 127)
                got = qk[t, h * 128 + 32 * r:h * 128 + 32 * r + 32]
                assert np.array_equal(got, want.astype(np.int8))
                assert np.abs(got).max() == 127
    # decode error bound on K: |code*d - x| <= d/2 (+ fp16 scale rounding)
    out_k, out_v, bad = oracle.kv_q8_0_dequantize(rk, rv, 5, 512)
    assert not bad
    ref = torch.from_numpy(qk[:5].astype(np.float32) *
                           np.repeat(dk[:5].astype(np.float32), 32, axis=1))
    assert np.array_equal(out_k, ref.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))


def test_q8_0_roundf_ties_away():
    # roundf, not rint: 2.5 -> 3, -2.5 -> -3 (kv_q8_native.cuh:46-48)
    from oracle import oracle as o
    # block with amax 127 -> ad = 1, inverse = 1, so codes are roundf of the values
    vals = np.zeros((1, 4, 128), np.float32)
    vals[0, 0, 0] = 127
    vals[0, 0, 1] = 2.5
    vals[0, 0, 2] = -2.5
    vals[0, 0, 3] = 0.5
    bits = synth.bf16_bits(vals)
    rk = np.zeros((1, 544), np.uint8)
    rv = np.zeros((1, 544), np.uint8)
    o.kv_q8_0_encode(bits, bits, rk, rv, np.zeros(1, np.int32), 1, rotate=False)
    _, qk = _row_fields(rk)
    assert list(qk[0, :4]) == [127, 3, -3, 1]


def test_q8_0_layout_bytes(oracle):
    assert oracle.lib().po_q8_0_row_bytes(512) == 544
    from padra_amd import ops, abi
    assert ops.kv_cache_layout(abi.KV_Q8_0, 131072)["v_offset"] == 131072 * 544
    assert ops.kv_cache_layout(abi.KV_Q8_0, 131072)["bytes"] == 131072 * 1088
    q8 = ops.kv_cache_layout(abi.KV_Q8, 8192)
    assert (q8["v_offset"], q8["scales_offset"], q8["bytes"]) == (8192 * 512, 8192 * 1024,
                                                                 8192 * 1056)
    assert ops.kv_cache_layout(abi.KV_BF16, 1024)["bytes"] == 1024 * 2048


# ---- A10 --------------------------------------------------------------------------------

def test_silu_table_exhaustive_long_double(oracle):
    table = oracle.silu_table()
    g = synth.bf16_to_f32(np.arange(65536, dtype=np.uint16))
    finite = np.isfinite(g)
    gl = g[finite].astype(np.longdouble)
    e = np.exp(-gl)  # 64-bit mantissa
    with np.errstate(over="ignore"):
        e32 = e.astype(np.float32)  # one rounding from extended precision
    den = (F32(1) + e32).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        s = (g[finite] / den).astype(np.float32)
    want = synth.bf16_bits(s)
    got = table[finite]
    assert np.array_equal(got, want)


def test_swiglu(oracle):
    d = synth.swiglu_inputs(tokens=4, width=64, seed=13)
    out, bad = oracle.swiglu(d["gate"], d["up"])
    assert not bad
    table = oracle.silu_table()
    want = synth.bf16_bits(synth.bf16_to_f32(table[d["gate"]]) * synth.bf16_to_f32(d["up"]))
    assert np.array_equal(out, want)
    g = d["gate"].copy()
    g[0, 0] = 0x7FC0
    assert oracle.swiglu(g, d["up"])[1]


# ---- A11 / A12 ----------------------------------------------------------------------------

def test_embed(oracle):
    rng = np.random.default_rng(14)
    table = synth.bf16_bits(rng.standard_normal((100, 64)) * 0.02)
    ids = np.array([0, 99, 5, 5], np.int32)
    out, bad = oracle.embed(table, ids)
    assert not bad and np.array_equal(out, table[ids])
    _, bad = oracle.embed(table, np.array([100], np.int32))
    assert bad


def test_state_predicates(oracle):
    import ctypes
    from padra_amd.abi import DecodeState, PrefillState
    lib = oracle.lib()
    s = DecodeState(token=5, position=2000, capacity=4096, remaining=3, global_valid=2000,
                    local_valid=1024, eos=0, stopped=0)
    assert lib.po_decode_ready(ctypes.byref(s), 8192, 98304)
    for field, value in (("local_valid", 2000), ("stopped", 1), ("remaining", 0),
                         ("position", 4096), ("token", 98304)):
        bad = DecodeState.from_buffer_copy(s)
        setattr(bad, field, value)
        if field == "position":
            bad.global_valid = 4096
        assert not lib.po_decode_ready(ctypes.byref(bad), 8192, 98304), field
    assert not lib.po_decode_ready(ctypes.byref(s), 2048, 98304)  # capacity above maximum
    p = PrefillState(base=0, prompt_offset=0, tokens=2048, capacity=131072, committed=0,
                     binding_epoch=1, request_epoch=1, valid=1)
    assert lib.po_valid_prefill_state(ctypes.byref(p), 2048, 131072, 1, 131072)
    for field, value in (("committed", 1), ("valid", 0), ("tokens", 2047), ("request_epoch", 0),
                         ("base", 131072 - 2047)):
        bad = PrefillState.from_buffer_copy(p)
        setattr(bad, field, value)
        assert not lib.po_valid_prefill_state(ctypes.byref(bad), 2048, 131072, 1, 131072), field


# ---- local-ring checkpoint capture ---------------------------------------------------------

@pytest.mark.parametrize("base,tokens,anchor", [(0, 300, 200), (700, 600, 1300),
                                                (3000, 2048, 5048), (1500, 100, 1501)])
def test_kv_checkpoint_plane(oracle, base, tokens, anchor):
    rng = np.random.default_rng(base + anchor)
    old = rng.integers(0, 256, (1024, 48), dtype=np.uint8)
    cur = rng.integers(0, 256, (tokens, 48), dtype=np.uint8)
    state = np.array([base, base, tokens, 8192, base, 1, 1, 1], np.int32)
    (saved,) = oracle.kv_checkpoint([old], [cur], state, tokens, anchor)
    for slot in range(1024):
        p = max(q for q in range(anchor - 1024, anchor) if q % 1024 == slot)
        if p >= base:
            want = cur[p - base]
        elif p >= 0:
            want = old[slot]
        else:
            want = np.zeros(48, np.uint8)
        assert np.array_equal(saved[slot], want), slot


def test_kv_checkpoint_admission(oracle):
    old = np.zeros((1024, 16), np.uint8)
    cur = np.zeros((10, 16), np.uint8)
    good = np.array([100, 100, 10, 2048, 100, 1, 1, 1], np.int32)
    assert oracle.kv_checkpoint([old], [cur], good, 10, 105) is not None
    assert oracle.kv_checkpoint([old], [cur], good, 10, 110) is not None
    assert oracle.kv_checkpoint([old], [cur], good, 10, 100) is None   # anchor <= base
    assert oracle.kv_checkpoint([old], [cur], good, 10, 111) is None   # past the chunk
    small = good.copy()
    small[3] = 512                                                     # capacity < 1024
    assert oracle.kv_checkpoint([old], [cur], small, 10, 105) is None
    stale = good.copy()
    stale[4] = 99                                                      # committed != base
    assert oracle.kv_checkpoint([old], [cur], stale, 10, 105) is None
    assert oracle.kv_checkpoint([old], [cur], good, 10, 105, epoch=2) is None


# ---- decode attention -------------------------------------------------------------------------

def _attn_inputs(cap, hq, hkv, seed):
    rng = np.random.default_rng(seed)
    q = synth.bf16_bits((rng.standard_normal((hq, 128)) * 2).astype(F32))
    kc = synth.bf16_bits(rng.standard_normal((cap, hkv * 128)).astype(F32))
    vc = synth.bf16_bits(rng.standard_normal((cap, hkv * 128)).astype(F32))
    return q, kc, vc


def _attn_float64(q, kc, vc, rows, hkv):
    hq = q.shape[0]
    g = hq // hkv
    qf = synth.bf16_to_f32(q).astype(np.float64)
    out = np.empty((hq, 128))
    for h in range(hq):
        kv = h // g
        k = synth.bf16_to_f32(kc[rows, kv * 128:(kv + 1) * 128]).astype(np.float64)
        v = synth.bf16_to_f32(vc[rows, kv * 128:(kv + 1) * 128]).astype(np.float64)
        s = k @ qf[h] / np.sqrt(128.0)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ v
    return out


@pytest.mark.parametrize("position,local,cap", [(0, False, 256), (77, False, 256),
                                                (4000, False, 4096), (3000, True, 1024)])
def test_decode_attention_float64(oracle, position, local, cap):
    hq, hkv = 16, 4
    q, kc, vc = _attn_inputs(cap, hq, hkv, position)
    out, used, bad = oracle.decode_attention(q, kc, vc, position, local=local)
    assert not bad
    n = min(position + 1, 1024) if local else position + 1
    rows = np.arange(position + 1 - n, position + 1) % cap
    ref = _attn_float64(q, kc, vc, rows, hkv)
    got = synth.bf16_to_f32(out).astype(np.float64)
    # BF16 probabilities (relative 2^-9 each) and the final BF16 rounding
    vmax = np.abs(synth.bf16_to_f32(vc)).max()
    assert np.all(np.abs(got - ref) <= 2.0**-8 * np.abs(ref) + 2.0**-8 * vmax)
    if not local and cap == 4096:
        other, used2, _ = oracle.decode_attention(q, kc, vc, position, splits=7)
        assert used2 == 7 and used == 32
        assert np.all(np.abs(synth.bf16_to_f32(other) - got) <= 2.0**-7 * vmax)


@pytest.mark.parametrize("position,local", [(5, False), (700, False), (3000, True)])
def test_decode_attention_q8_0_float64(oracle, position, local):
    """Against float64 attention of the original query over the cache's decoded rows (codes
    times scale, rotated back): the query's own int8 coding (relative 1/254 per block)
    bounds the difference."""
    hq, hkv = 16, 4
    cap = 1024 if local else 4096
    rng = np.random.default_rng(position)
    q = synth.bf16_bits(rng.standard_normal((hq, 128)).astype(F32))
    k = synth.bf16_bits(rng.standard_normal((cap, hkv, 128)).astype(F32))
    v = synth.bf16_bits(rng.standard_normal((cap, hkv, 128)).astype(F32))
    rk = np.zeros((cap, 544), np.uint8)
    rv = np.zeros((cap, 544), np.uint8)
    oracle.kv_q8_0_encode(k, v, rk, rv, np.arange(cap, dtype=np.int32), cap)
    out, used, bad = oracle.decode_attention_q8_0(q, rk, rv, position, local=local)
    assert not bad and used == min(16 if local else 32, (min(position + 1, 1024 if local else 10**9) + 127) // 128)
    # decoded rows in the original basis
    dk, dv, _ = oracle.kv_q8_0_dequantize(rk, rv, cap, 512)
    kf = synth.bf16_to_f32(dk).reshape(cap, hkv, 128).astype(np.float64)
    vf = synth.bf16_to_f32(dv).reshape(cap, hkv, 128).astype(np.float64)
    h128 = __import__("scipy").linalg.hadamard(128) / np.sqrt(128)
    h64 = __import__("scipy").linalg.hadamard(64) / 8.0
    kf = kf @ h128.T  # inverse rotation (symmetric, orthonormal)
    vf = np.concatenate([vf[..., :64] @ h64.T, vf[..., 64:] @ h64.T], axis=-1)
    n = min(position + 1, 1024) if local else position + 1
    rows = np.arange(position + 1 - n, position + 1) % cap
    g = hq // hkv
    qf = synth.bf16_to_f32(q).astype(np.float64)
    got = synth.bf16_to_f32(out).astype(np.float64)
    for h in range(hq):
        s = kf[rows, h // g] @ qf[h] / np.sqrt(128)
        w = np.exp(s - s.max())
        ref = (w / w.sum()) @ vf[rows, h // g]
        assert np.max(np.abs(got[h] - ref)) <= 0.02 * np.abs(vf).max(), h


def test_round_away_identity(oracle):
    """The GPU rounds q8_0 codes as (int)(v + copysign(0.49999997, v)) in place of roundf:
    equal on every finite float with |v| < 2^23 (all 2^32 bit patterns scanned, ~10 s), and
    the plain v + 0.5 it avoids is not (0.49999997 + 0.5 rounds up to 1)."""
    assert oracle.round_away_mismatches() == 0
    assert np.float32(0.49999997) + np.float32(0.5) == np.float32(1.0)
