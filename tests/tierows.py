"""Rows whose sum of squares sits at a chosen distance from an fp32 rounding midpoint, and
the kernels' certificate for the order-free sum (padra_amd/csrc/common.h: sumsq_margin,
certified_sum) restated for the tests.  Rows close to a midpoint are the ones the kernels
must send to the reference's ordered tree.
"""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np

from padra_amd import synth

F32 = np.float32


def margin(m: int, depth: int) -> float:
    """sumsq_margin(m, depth) of common.h (test_margin_formula_matches_source keeps the two
    in step)."""
    return 1.01 * (1.003 * (m + 20.0) * (m + 20.0) * 2.0**-48 + 1.001 * depth * 2.0**-53) + 2.0**-51


def certified(s64: float, c: float):
    """certified_sum of common.h: the fma ends computed exactly, then rounded once to fp64
    (what v_fma_f64 does) and converted to fp32 (v_cvt_f32_f64, RNE)."""
    s = Fraction(s64)
    lo = F32(float(s - Fraction(c) * s))  # float(Fraction) is RN64; F32(.) is RN32
    hi = F32(float(s + Fraction(c) * s))
    ok = bool(lo == hi) and 2.0**-60 <= s64 < 2.0**126
    return ok, hi


def bf16_floor(x: float) -> float:
    """Largest BF16 value <= x (x > 0)."""
    b = int(np.array([x], np.float32).view(np.uint32)[0]) & 0xFFFF0000
    f = float(np.array([b], np.uint32).view(np.float32)[0])
    while f > x:
        b -= 0x10000
        f = float(np.array([b], np.uint32).view(np.float32)[0])
    return f


def near_midpoint_row(rng, n, rel_distance, above):
    """A BF16 row (length n) whose exact sum of squares lies about rel_distance * S from
    an fp32 rounding midpoint, on the chosen side: n - 6 random values, then greedy tiny
    values whose squares walk the sum onto the target."""
    base = synth.bf16_to_f32(synth.bf16_bits(rng.standard_normal(n - 6)))
    s = sum(Fraction(float(x)) ** 2 for x in base)
    f = F32(float(s))  # RN32 or its neighbour: either one's midpoint will do
    ulp = Fraction(float(np.spacing(np.float32(f))))
    mid = Fraction(float(f)) + ulp / 2
    if mid <= s:
        mid += ulp
    target = mid + (1 if above else -1) * Fraction(rel_distance) * mid
    extra = []
    r = target - s
    for _ in range(6):
        if r <= 0:
            extra.append(0.0)
            continue
        t = bf16_floor(math.sqrt(float(r)))
        if t <= 0 or not np.isfinite(t):
            extra.append(0.0)
            continue
        extra.append(t)
        r -= Fraction(t) ** 2
    row = np.concatenate([base, np.array(extra, np.float32)])
    return row[rng.permutation(n)].astype(np.float32)
