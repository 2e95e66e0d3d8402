"""Writes tests/golden/reduction_order.npz: inputs on which the compensated sum of squares
depends on the reduction tree, with the expected results computed by tests/refsim.py
(a thread-level simulation of the reference's CUDA reduction, independent of the C
oracle).  The sparse inputs were found by a seeded random search over values
{+-2^15, +-2^12, +-8, +-2^-9}; only their nonzero entries are listed here.

Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import refsim  # noqa: E402

# (length, [(index, value)]) -- the 512-vector separates the 128- and 256-thread trees;
# the 128-vectors separate the 128-thread tree from a sequential compensated sum.
SPARSE = [
    (512, [(18, 2**-9), (104, -4096.0), (158, 8.0), (226, -2**-9), (259, 16384.0),
           (262, 4096.0), (280, 32768.0), (351, 2**-9), (410, -2**-9), (470, 4096.0)]),
    (128, [(23, -2**-9), (26, 4096.0), (80, -32768.0), (98, -2**-9), (102, -8.0),
           (114, -4096.0)]),
    (128, [(7, 8.0), (13, -2**-9), (73, 2**-9), (77, 32768.0), (81, -4096.0)]),
]


def dense(n, entries):
    v = np.zeros(n, np.float32)
    for i, x in entries:
        v[i] = x
    return v


def main():
    v512 = dense(*SPARSE[0])
    h128 = np.stack([dense(*s) for s in SPARSE[1:]])
    out = {
        "v512": v512,
        "v512_tree128": np.float32(refsim.block_sumsq(v512, 128)),
        "v512_tree256": np.float32(refsim.block_sumsq(v512, 256)),
        "head128": h128,
        "head128_tree128": np.array([refsim.block_sumsq(h, 128) for h in h128], np.float32),
    }
    np.savez(os.path.join(HERE, "reduction_order.npz"), **out)
    print({k: (v if np.ndim(v) == 0 else v.shape) for k, v in out.items()})


if __name__ == "__main__":
    main()
