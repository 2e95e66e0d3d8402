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
    """Per element: within 1 BF16 ulp of the oracle, or within 2^-12 of the head's largest
    |output|.  The second bound covers near-cancelling sums, where a BF16 probability that
    rounds the other way (the score's fp32 sum order differs) moves the output by a
    fraction of one term, not of the small result.  Returns (mask, ulp distances)."""
    d = ulp_diff(got_bits, want_bits)
    g, w = synth.bf16_to_f32(got_bits), synth.bf16_to_f32(want_bits)
    head_max = np.abs(w).max(axis=-1, keepdims=True)
    return (d <= 1) | (np.abs(g - w) <= 2.0**-12 * head_max), d
