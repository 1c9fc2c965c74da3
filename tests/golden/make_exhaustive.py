"""Writes tests/golden/exhaustive_small.npz: tiny encode problems with their exhaustive answers.

The reference ships no golden vectors for its encoder (its tests compare paths with each other),
so these fixtures come from mathematics instead: for each vector, every code tuple is scored by
its exact least-squares reconstruction error in fp64 (numpy lstsq), and the minimum is kept.
A prefix-LS beam whose width is at least prod(h_vec[1:]) keeps every prefix, so it must return
an optimal tuple (BeamSearchPrefixLS, src/quantizer/beam_search.cpp:196-422).

Run:  python tests/golden/make_exhaustive.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from helpers import exhaustive  # noqa: E402

CASES = [
    # (seed, n, d, h_vec)
    (101, 40, 6, [8, 8, 8]),
    (202, 40, 5, [16, 16]),
    (303, 30, 8, [4, 4, 4, 4]),
    (404, 40, 3, [6, 5, 7]),
]


def main():
    out = {}
    for ci, (seed, n, d, h_vec) in enumerate(CASES):
        rng = np.random.default_rng(seed)
        C = rng.standard_normal((sum(h_vec), d)).astype(np.float32)
        X = (rng.standard_normal((n, d)) * 1.5).astype(np.float32)
        codes, cost = exhaustive(X, C, h_vec)
        out[f"c{ci}_X"] = X
        out[f"c{ci}_C"] = C
        out[f"c{ci}_h"] = np.array(h_vec, np.int32)
        out[f"c{ci}_codes"] = codes
        out[f"c{ci}_cost"] = cost
    out["ncases"] = np.array(len(CASES))
    np.savez_compressed(os.path.join(HERE, "exhaustive_small.npz"), **out)


if __name__ == "__main__":
    main()
