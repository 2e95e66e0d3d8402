"""The decode attention tolerance of the GPU tests (BF16 outputs against the oracle)."""
import numpy as np

from padra_amd import synth


def ulp_diff(got_bits, want_bits):
    """Distance in BF16 ulps (ordered bit patterns, both signs)."""
    def ordered(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + b)
    return np.abs(ordered(got_bits) - ordered(want_bits))


def attn_close(got_bits, want_bits):
    """Per element: within 1 BF16 ulp of the oracle, or within 2^-10 of the head's largest
    |output|.  The second bound covers near-cancelling sums, where a BF16 probability that
    rounds the other way (the score's fp32 sum order differs) moves the output by a
    fraction of one term (2^-8 x p x |v|), not of the small result: p ~ 0.015 against
    |v| ~ 2 moves an output of 0.003 by 4 ulps.  Over 82k outputs per format (40 local-ring
    sequences x 16 heads, 6 / 12 / 16 splits) the largest such move was 2^-10.9 of the head
    maximum.  Returns (mask, ulp distances)."""
    d = ulp_diff(got_bits, want_bits)
    g, w = synth.bf16_to_f32(got_bits), synth.bf16_to_f32(want_bits)
    head_max = np.abs(w).max(axis=-1, keepdims=True)
    return (d <= 1) | (np.abs(g - w) <= 2.0**-10 * head_max), d
