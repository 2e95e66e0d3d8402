"""The order-free sum of squares and its certificate (padra_amd/csrc/common.h,
sumsq_margin / certified_sum) against the reference's compensated tree.

The kernels sum the squares of a row or head in fp64, in an order of their own, and take
RN32 of that sum only when both ends of [S64 (1 - c), S64 (1 + c)] round to the same
float; otherwise they replay the reference tree (AccurateReduce, inference.cu:103-135;
residual_norm_wide_exact.cuh:24-63).  The claim is that a certified value always equals
the tree's RN32(s + e).  These tests check it against the oracle's tree
(po_sumsq_tree, itself pinned to tests/refsim.py) on:
  - the golden order-sensitive vectors: the trees disagree there, so the certificate must
    refuse them (it would otherwise prove two different values equal);
  - rows built to put the exact sum at a chosen distance from an fp32 rounding midpoint
    (2^-58 .. 2^-26 of the sum), where trees and the fp64 sum can round apart;
  - random rows of the benchmark's shapes (outlier channels), counting the refusals.
"""
from __future__ import annotations

import ctypes
import math
import os
import re
from fractions import Fraction

import numpy as np
import pytest

from padra_amd import synth
from tierows import certified, margin, near_midpoint_row

F32 = np.float32
HERE = os.path.dirname(os.path.abspath(__file__))
COMMON_H = os.path.join(os.path.dirname(HERE), "padra_amd", "csrc", "common.h")


def test_margin_formula_matches_source():
    src = open(COMMON_H).read()
    body = re.search(r"constexpr double sumsq_margin\(int m, int depth\) \{\s*return (.*?);", src,
                     re.S).group(1)
    body = " ".join(body.split())
    assert body == ("1.01 * (1.003 * (m + 20.0) * (m + 20.0) * 0x1p-48 + 1.001 * depth * 0x1p-53) "
                    "+ 0x1p-51")


def tree(lib, v: np.ndarray, threads: int) -> F32:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return F32(lib.po_sumsq_tree(v.ctypes.data_as(ctypes.c_void_p), len(v), threads))


def fp64_sum(v: np.ndarray, rng) -> float:
    """The squares summed in fp64 in a shuffled order (any order's error is inside the
    margin's depth term for these sizes)."""
    sq = v.astype(np.float64) ** 2
    return float(np.sum(sq[rng.permutation(len(sq))]))


def test_golden_vectors_are_refused(oracle):
    g = np.load(os.path.join(HERE, "golden", "reduction_order.npz"))
    lib = oracle.lib()
    rng = np.random.default_rng(0)
    v = g["v512"]
    for threads in (128, 256):
        ok, _ = certified(fp64_sum(v, rng), margin(512 // threads, 512 // 64 + 6))
        assert not ok, "a vector on which the trees disagree must take the ordered tree"
    assert tree(lib, v, 128) != tree(lib, v, 256)
    for h in g["head128"]:
        ok, val = certified(fp64_sum(h, rng), margin(1, 34))
        # the heads separate the tree from a sequential compensated sum; where the
        # certificate holds, the tree must give its value
        if ok:
            assert val == tree(lib, h, 128)


@pytest.mark.parametrize("n,threads", [(128, 128), (2048, 128), (2048, 256), (2304, 128)])
def test_certified_equals_tree_near_midpoints(oracle, n, threads):
    lib = oracle.lib()
    rng = np.random.default_rng(n + threads)
    m = n // threads
    c = margin(m, (n // 64 if n > 128 else 32) + 6)
    refused = {}
    trials = 6 if n > 128 else 12
    for k in range(26, 60, 2):
        for above in (False, True):
            for _ in range(trials):
                row = near_midpoint_row(rng, n, 2.0**-k, above)
                ok, val = certified(fp64_sum(row, rng), c)
                if ok:
                    assert val == tree(lib, row, threads), (k, above)
                else:
                    refused[k] = refused.get(k, 0) + 1
    # close to a midpoint the certificate must refuse; far from it, accept
    assert refused.get(58, 0) == 2 * trials
    assert refused.get(26, 0) == 0


@pytest.mark.parametrize("n,threads", [(2048, 128), (2048, 256), (128, 128)])
def test_random_rows_refusal_rate(oracle, n, threads):
    """Rows like the benchmark's (N(0,1), 1% of channels x20): every certified value equals
    the tree's, and the refusals are few: about 2c / 2^-23.5 of rows for sums spread
    evenly between floats, plus sums that fall exactly on a midpoint (squares of BF16
    values sit on a coarse grid, so a 128-feature head's sum is a tie now and then)."""
    lib = oracle.lib()
    rng = np.random.default_rng(7)
    m = n // threads
    c = margin(m, (n // 64 if n > 128 else 32) + 6)
    rows = 4000 if n > 128 else 20000
    scale = np.ones(n)
    scale[rng.choice(n, max(1, n // 100), replace=False)] = 20.0
    refused = 0
    for _ in range(rows):
        row = synth.bf16_to_f32(synth.bf16_bits(rng.standard_normal(n) * scale))
        ok, val = certified(fp64_sum(row, rng), c)
        if ok:
            assert val == tree(lib, row, threads)
        else:
            refused += 1
    expected = rows * 2 * c / 2.0**-23.5
    print(f"n={n} threads={threads}: {refused} of {rows} rows refused (about {expected:.1f} expected)")
    assert refused <= max(4 * expected + 5, rows // 1000)
