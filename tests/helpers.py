"""Problem builders and the parity protocol shared by the tests."""
from __future__ import annotations

import numpy as np

from stlq_amd import workloads


def offsets(h_vec):
    return np.concatenate([[0], np.cumsum(h_vec)[:-1]]).astype(np.int64)


def random_problem(seed, n, d, h_vec, scale=1.0, x_scale=None):
    rng = np.random.default_rng(seed)
    C = (rng.standard_normal((int(sum(h_vec)), d)) * scale).astype(np.float32)
    X = (rng.standard_normal((n, d)) * (scale if x_scale is None else x_scale)).astype(np.float32)
    return X, C


def rvq_problem(seed, n, d, m, K, kind="gauss", n_comp=64, train_n=4000, iters=6):
    mix = workloads.Mixture(kind, d, n_comp, seed)
    Xtr = mix.sample(1_000_000, train_n)
    C = workloads.residual_codebooks(Xtr, m, K, iters, seed + 3, spherical=(kind == "sphere"))
    X = mix.sample(0, n)
    return X, C


def exhaustive(X, C, h_vec):
    """Exhaustive LS-optimal code tuples in fp64 (ties -> lexicographically first tuple)."""
    import itertools

    off = offsets(h_vec)
    C64 = C.astype(np.float64)
    tuples = list(itertools.product(*[range(k) for k in h_vec]))
    best_codes = np.zeros((X.shape[0], len(h_vec)), np.uint8)
    best_cost = np.zeros(X.shape[0])
    for i in range(X.shape[0]):
        x = X[i].astype(np.float64)
        bc, bt = None, None
        for tup in tuples:
            Cs = C64[[off[l] + t for l, t in enumerate(tup)]]
            a, *_ = np.linalg.lstsq(Cs.T, x, rcond=None)
            e = float(np.sum((x - Cs.T @ a) ** 2))
            if bc is None or e < bc:
                bc, bt = e, tup
        best_codes[i] = bt
        best_cost[i] = bc
    return best_codes, best_cost


def parity(orc, X, C, h_vec, codes_ref, codes_test, max_frac=1e-3, tie_rel=1e-5, mse_rel=1e-5):
    """North-star parity protocol: codes may differ on at most max_frac of the vectors, only where
    the two code tuples' costs tie within tie_rel (relative), and per-vector reconstruction MSE
    (fp64 LS refit + explicit reconstruction, applied to both code sets) agrees within mse_rel.
    Returns a report dict; `ok` says whether the protocol passes."""
    diff = np.any(codes_ref != codes_test, axis=1)
    n = X.shape[0]
    rep = {"n": n, "n_diff": int(diff.sum()), "frac_diff": float(diff.mean()) if n else 0.0,
           "max_rel_mse": 0.0, "ok": True}
    if diff.any():
        idx = np.nonzero(diff)[0]
        ma = orc.mse_fp64_refit(X[idx], C, h_vec, codes_ref[idx])
        mb = orc.mse_fp64_refit(X[idx], C, h_vec, codes_test[idx])
        rel = np.abs(ma - mb) / np.maximum(np.abs(ma), 1e-30)
        rep["max_rel_mse"] = float(rel.max())
        rep["ok"] = rep["frac_diff"] <= max_frac and rep["max_rel_mse"] <= max(tie_rel, mse_rel)
    return rep
