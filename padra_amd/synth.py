"""Seeded synthetic inputs for the five workloads of the per-token layer path.

numpy PCG64 with seed 0; normals via Generator.standard_normal; every tensor is
rounded to BF16 (round-to-nearest-even) before use, so the same bits feed the GPU
kernels and the CPU checker.  Outlier channels (config 1/2): 1% of the channels of each
activation, chosen by a seeded permutation, scaled x20 before rounding.
"""
from __future__ import annotations

import numpy as np


def bf16_bits(a) -> np.ndarray:
    """float32 -> BF16 bit patterns (uint16), RNE; NaN -> 0x7fff."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = a.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        r[nan] = 0x7FFF
    return r


def bf16_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def outlier_channels(rng: np.random.Generator, n: int, frac: float = 0.01) -> np.ndarray:
    return np.sort(rng.permutation(n)[: max(1, int(round(n * frac)))])


def _normal(rng, shape, sigma=1.0, outliers=None, scale=20.0):
    x = rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma)
    if outliers is not None:
        x[..., outliers] *= np.float32(scale)
    return x


def chain_inputs(tokens: int, hidden: int = 2048, q_heads: int = 16, kv_heads: int = 4,
                 head_dim: int = 128, outliers: bool = False, seed: int = 0) -> dict:
    """x, residual [T][H]; q [T][Hq][D]; k, v [T][Hkv][D]; gamma [H]; qn, kn [D] (BF16 bits)."""
    rng = np.random.default_rng(seed)
    oh = outlier_channels(rng, hidden) if outliers else None
    oq = outlier_channels(rng, q_heads * head_dim) if outliers else None
    okv = outlier_channels(rng, kv_heads * head_dim) if outliers else None
    x = _normal(rng, (tokens, hidden), outliers=oh)
    r = _normal(rng, (tokens, hidden), outliers=oh)
    q = _normal(rng, (tokens, q_heads * head_dim), outliers=oq)
    k = _normal(rng, (tokens, kv_heads * head_dim), outliers=okv)
    v = _normal(rng, (tokens, kv_heads * head_dim), outliers=okv)
    gamma = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
    qn = rng.uniform(0.5, 1.5, head_dim).astype(np.float32)
    kn = rng.uniform(0.5, 1.5, head_dim).astype(np.float32)
    return {
        "x": bf16_bits(x), "residual": bf16_bits(r),
        "q": bf16_bits(q).reshape(tokens, q_heads, head_dim),
        "k": bf16_bits(k).reshape(tokens, kv_heads, head_dim),
        "v": bf16_bits(v).reshape(tokens, kv_heads, head_dim),
        "gamma": bf16_bits(gamma), "qn": bf16_bits(qn), "kn": bf16_bits(kn),
    }


def swiglu_inputs(tokens: int = 2048, top_k: int = 8, width: int = 1024, experts: int = 64,
                  sigma: float = 2.0, seed: int = 0) -> dict:
    """gate, up [rows][W] with rows = tokens*top_k, stably sorted by a uniform random expert
    id (ragged expert segments); offsets[e] = first row of expert e."""
    rng = np.random.default_rng(seed)
    rows = tokens * top_k
    expert = rng.integers(0, experts, rows)
    order = np.argsort(expert, kind="stable")
    gate = _normal(rng, (rows, width), sigma)[order]
    up = _normal(rng, (rows, width), sigma)[order]
    offsets = np.searchsorted(expert[order], np.arange(experts + 1)).astype(np.int32)
    return {"gate": bf16_bits(gate), "up": bf16_bits(up), "offsets": offsets}


def zipf_ids(n: int, vocab: int, s: float = 1.1, seed: int = 0) -> np.ndarray:
    """Token ids ~ Zipf(s) over [0, vocab) by inverse CDF (rank 1 -> id 0)."""
    rng = np.random.default_rng(seed)
    w = 1.0 / np.arange(1, vocab + 1, dtype=np.float64) ** s
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    return np.minimum(np.searchsorted(cdf, rng.random(n)), vocab - 1).astype(np.int32)
