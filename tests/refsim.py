"""Thread-level simulation of the reference's CUDA reduction kernels, in numpy float32.

A second, independent restatement used to pin the C oracle: it keeps the reference's
own structure (per-thread registers, __shfl_down_sync with its lane-bound condition,
the shared scratch array, the warp-0 second pass) instead of the oracle's array form.
Small inputs only (pure Python loops).
"""
from __future__ import annotations

import numpy as np

f32 = np.float32


def accumulate(value, s, e):
    """inference.cu:103-109."""
    value, s, e = f32(value), f32(s), f32(e)
    nxt = f32(s + value)
    if abs(s) >= abs(value):
        residual = f32(f32(s - nxt) + value)
    else:
        residual = f32(f32(value - nxt) + s)
    return nxt, f32(e + residual)


def _shfl_down_tree(sums, errs, lanes):
    """One warp: for d = 16..1, every lane with (lane & 31) + d < 32 folds the value the
    source lane held when the shuffle executed."""
    for d in (16, 8, 4, 2, 1):
        src_s = list(sums)
        src_e = list(errs)
        for lane in range(lanes):
            if (lane & 31) + d < 32:
                other, low = src_s[lane + d], src_e[lane + d]
                sums[lane], errs[lane] = accumulate(other, sums[lane], errs[lane])
                sums[lane], errs[lane] = accumulate(low, sums[lane], errs[lane])
    return sums, errs


def block_sumsq(values, threads):
    """AccurateReduce (threads=128, inference.cu:110-135) and the wide variant
    (threads=256, residual_norm_wide_exact.cuh:24-63) over `values`."""
    values = [f32(v) for v in values]
    sums, errs = [], []
    for t in range(threads):
        s, e = f32(0), f32(0)
        i = t
        while i < len(values):
            s, e = accumulate(f32(values[i] * values[i]), s, e)
            i += threads
        sums.append(s)
        errs.append(e)
    scratch_s, scratch_e = [], []
    for w in range(threads // 32):
        ws, we = _shfl_down_tree(sums[32 * w:32 * w + 32], errs[32 * w:32 * w + 32], 32)
        scratch_s.append(ws[0])
        scratch_e.append(we[0])
    s2 = [scratch_s[t] if t < len(scratch_s) else f32(0) for t in range(32)]
    e2 = [scratch_e[t] if t < len(scratch_e) else f32(0) for t in range(32)]
    s2, e2 = _shfl_down_tree(s2, e2, 32)
    return f32(s2[0] + e2[0])


def bf16(x):
    b = np.array([x], dtype=np.float32).view(np.uint32)[0]
    b = (int(b) + 0x7FFF + ((int(b) >> 16) & 1)) & 0xFFFF0000
    return np.array([b], dtype=np.uint32).view(np.float32)[0]


def norm_row(values, gamma, threads, eps=1e-6):
    """Norm (inference.cu:188-214) on one row of BF16-exact float32 values."""
    s = block_sumsq(values, threads)
    var = f32(s / f32(len(values)))
    inv = f32(f32(1) / f32(np.sqrt(f32(var + f32(eps)))))
    return [bf16(f32(bf16(f32(v * inv)) * g)) for v, g in zip(values, gamma)], var, inv
