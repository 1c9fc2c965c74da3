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


BEAM_CASES = [
    # name, seed, n, d, h_vec, H_beam, kind
    ("m2_K16_b4", 10, 800, 12, [16, 16], 4, "gauss"),
    ("m4_K32_b1", 11, 800, 24, [32] * 4, 1, "gauss"),
    ("m4_K256_b4_c1", 12, 600, 128, [256] * 4, 4, "gauss"),
    ("m8_K256_b16_c2", 13, 500, 128, [256] * 8, 16, "desc"),
    ("m8_K256_b16_sphere", 14, 400, 96, [256] * 8, 16, "sphere"),
    ("m5_K100_b64", 15, 300, 20, [100, 90, 80, 70, 60], 64, "gauss"),
    ("m3_K7_b40", 16, 500, 6, [7, 9, 5], 40, "gauss"),
    ("m10_K64_b8", 17, 300, 40, [64] * 10, 8, "gauss"),
    ("m16_K256_b8_decay", 18, 120, 64, [256] * 16, 8, "decay"),
    ("m1_K200_b3", 19, 500, 16, [200], 3, "gauss"),
    ("m6_K65_b33", 20, 300, 30, [65, 130, 200, 3, 256, 64], 33, "gauss"),
    # the deepest prefixes (kMaxM = 20: layers up to 19, past the scalar-register budget)
    ("m20_K256_b8_decay", 21, 80, 64, [256] * 20, 8, "decay"),
    ("m20_K24_b33", 22, 200, 24, [24] * 20, 33, "gauss"),
]


def beam_case(seed, n, d, h, kind):
    if kind == "gauss" and max(h) < 100:
        return random_problem(seed, n, d, h, x_scale=2.0)
    if len(set(h)) == 1:
        return rvq_problem(seed, n, d, len(h), h[0], kind=kind, train_n=max(2000, 4 * h[0]), iters=4)
    return random_problem(seed, n, d, h, x_scale=2.0)


DEGENERATE = ["dup_within_layer", "dup_across_layers", "zero_codeword", "zero_layer", "zero_root_layer",
              "tiny_codebook", "scaled_copies", "nan_codeword"]


def degenerate_problem(case):
    """Exact ties, zero codewords/layers, tiny codebooks: (X, C, h_vec) for one named case."""
    rng = np.random.default_rng(100 + DEGENERATE.index(case))
    d, h = 10, [12, 12, 12, 12]
    C = rng.standard_normal((48, d)).astype(np.float32)
    X = (rng.standard_normal((400, d)) * 2).astype(np.float32)
    if case == "dup_within_layer":
        C[3] = C[7]
        C[12 + 5] = C[12 + 1]
        C[24 + 0] = C[24 + 11]
    elif case == "dup_across_layers":
        C[12 + 4] = C[2]
        C[24 + 4] = C[2]
        C[36 + 9] = C[12 + 4]
    elif case == "zero_codeword":
        C[5] = 0
        C[12 + 0] = 0
        C[36 + 11] = 0
    elif case == "zero_layer":
        C[24:36] = 0
    elif case == "zero_root_layer":
        C[0:12] = 0
    elif case == "tiny_codebook":
        h = [2, 1, 3, 2]
        C = C[:8]
    elif case == "scaled_copies":
        C[12 + 3] = 2.0 * C[1]
        C[24 + 6] = -0.5 * C[12 + 8]
    elif case == "nan_codeword":
        # Layer-2 code 7 and layer-3 code 2 give NaN candidate errors (NaN and inf Gram entries);
        # a NaN enters the beam (NaN >= worst is false) and pins RecomputeWorst while finite
        # candidates keep the beam alive. Zero vectors add exact ties at error 0. (Vectors whose
        # whole beam turns non-finite reach the all-skipped fallback, which reads the reference's
        # stale per-thread workspace, so no case here produces them.)
        C[24 + 7, 1] = np.nan
        C[36 + 2, 4] = np.inf
        X[38:45] = 0
    return X, C, h


def large_root_problem(orc, seed, n, d, h0, K, m, H_beam=4, root_mode=1, kind="gauss"):
    """A large-root problem (root codebook of h0 codewords + m-1 residual books of K) with the
    oracle's precomp, xC_small, and the oracle's large-root beam codes as the starting point."""
    from stlq_amd import workloads

    mix = workloads.Mixture(kind, d, 128, seed)
    rng = np.random.default_rng(seed)
    C0 = mix.sample(5_000_000, h0)
    Xtr = mix.sample(1_000_000, 2000)
    Cs = workloads.residual_codebooks(Xtr - C0[rng.integers(0, h0, 2000)], m - 1, K, 3, seed + 1)
    X = mix.sample(0, n)
    h = [h0] + [K] * (m - 1)
    norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs)
    invs = orc.invnorm_small(Cs)
    nx2 = orc.xnorm2(X)
    xs = orc.gemm_xc(Cs, X, mode=1)
    cid, Bs, _ = orc.beam_search_large_root(X, nx2, C0, norm0, xs, Gs, G0S, h, H_beam, root_mode=root_mode)
    return dict(X=X, C0=C0, Cs=Cs, h=h, norm0=norm0, Gs=Gs, G0S=G0S, invs=invs, nx2=nx2, xs=xs, cid=cid, Bs=Bs)
