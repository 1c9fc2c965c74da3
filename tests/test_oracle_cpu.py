"""Pins the CPU oracle (oracle/stlq_oracle.cpp) against answers fixed by mathematics.

The reference holds no golden vectors for its encoder, so each oracle routine is checked
against an independent answer: exhaustive search, closed forms, fp64 linear algebra and
invariants of the algorithm. Each check is chosen so that a plausible restatement mistake
(wrong sign, dropped term, transposed G index, wrong slot rule) fails it.
"""
import os

import numpy as np
import pytest

from tests.helpers import exhaustive, offsets, random_problem, rvq_problem

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "exhaustive_small.npz")


def _prep(orc, X, C, h):
    G, inv = orc.build_precomp(C, h)
    nx2 = orc.xnorm2(X)
    xC = orc.gemm_xc(C, X)
    return G, inv, nx2, xC


def test_precomp_matches_fp64(orc):
    X, C = random_problem(1, 10, 17, [5, 7, 3])
    G, inv = orc.build_precomp(C, [5, 7, 3])
    C64 = C.astype(np.float64)
    np.testing.assert_allclose(G, C64 @ C64.T, rtol=1e-5, atol=1e-5)
    assert np.array_equal(G, G.T), "sequential Gram must be exactly symmetric"
    np.testing.assert_allclose(inv, 1.0 / np.linalg.norm(C64, axis=1), rtol=1e-6)
    Cz = C.copy()
    Cz[3] = 0.0
    _, invz = orc.build_precomp(Cz, [5, 7, 3])
    assert invz[3] == 0.0  # encoder_precomp.inc:37: zero codeword -> 0


def test_xnorm_and_gemm(orc):
    X, C = random_problem(2, 33, 19, [4, 4])
    np.testing.assert_allclose(orc.xnorm2(X), np.sum(X.astype(np.float64) ** 2, axis=1), rtol=1e-6)
    xC = orc.gemm_xc(C, X)
    np.testing.assert_allclose(xC, X.astype(np.float64) @ C.astype(np.float64).T, rtol=1e-5, atol=1e-5)
    # sequential order: the first element equals a plain left-to-right float32 loop
    s = np.float32(0)
    for t in range(X.shape[1]):
        s = np.float32(s + np.float32(C[2, t] * X[5, t]))
    assert xC[5, 2] == s


def test_beam_exhaustive_golden(orc):
    """Full-width beam == exhaustive LS search (committed fixtures)."""
    z = np.load(GOLDEN)
    for ci in range(int(z["ncases"])):
        X, C, h = z[f"c{ci}_X"], z[f"c{ci}_C"], z[f"c{ci}_h"]
        want_cost = z[f"c{ci}_cost"]
        G, inv, nx2, xC = _prep(orc, X, C, h)
        width = int(np.prod(h[1:])) if len(h) > 1 else 1
        codes, err = orc.beam_search(nx2, xC, G, h, min(64, width))
        got_cost = orc.mse_fp64_refit(X, C, h, codes)
        np.testing.assert_allclose(got_cost, want_cost, rtol=1e-6, atol=1e-9)
        if want_cost.min() > 1e-6:  # case 3 has d == m: every tuple reconstructs exactly
            agree = np.mean(np.all(codes == z[f"c{ci}_codes"], axis=1))
            assert agree >= 0.97, (ci, agree)


def test_beam_exhaustive_random(orc):
    X, C = random_problem(3, 30, 7, [6, 6, 6], x_scale=2.0)
    h = [6, 6, 6]
    G, inv, nx2, xC = _prep(orc, X, C, h)
    codes, err = orc.beam_search(nx2, xC, G, h, 36)
    ex_codes, ex_cost = exhaustive(X, C, h)
    got = orc.mse_fp64_refit(X, C, h, codes)
    np.testing.assert_allclose(got, ex_cost, rtol=1e-6, atol=1e-9)


def test_m1_closed_form(orc):
    """m = 1: the single code maximises gamma^2/alpha (first maximum), e = ||x||^2 - gamma^2/alpha."""
    X, C = random_problem(4, 200, 9, [40])
    G, inv, nx2, xC = _prep(orc, X, C, [40])
    codes, err = orc.beam_search(nx2, xC, G, [40], 3)
    score = (X.astype(np.float64) @ C.astype(np.float64).T) ** 2 / np.sum(C.astype(np.float64) ** 2, axis=1)
    want = np.argmax(score, axis=1)
    assert np.mean(codes[:, 0] == want) == 1.0
    ref_err = np.sum(X.astype(np.float64) ** 2, axis=1) - score.max(axis=1)
    np.testing.assert_allclose(err, ref_err, rtol=1e-4, atol=1e-4)


def test_beam_err_is_ls_cost(orc):
    """The selected beam error equals the LS-refit cost of the returned codes
    (mirrors tests/test_beam_large_root_best_err_matches_cost.cpp:102-131)."""
    X, C = rvq_problem(5, 500, 24, 5, 32)
    h = [32] * 5
    G, inv, nx2, xC = _prep(orc, X, C, h)
    codes, err = orc.beam_search(nx2, xC, G, h, 8)
    a, fails = orc.solve_ls_all(xC, G, h, codes)
    cost = orc.compute_costs(xC, G, h, codes, a, nx2)
    assert fails == 0
    np.testing.assert_allclose(err, cost, rtol=2e-3, atol=1e-3 * float(np.mean(nx2)))
    ex = orc.mse_fp64_refit(X, C, h, codes)
    np.testing.assert_allclose(err, ex, rtol=2e-3, atol=1e-3 * float(np.mean(nx2)))


def test_beam_wider_is_not_worse_on_average(orc):
    X, C = rvq_problem(6, 400, 16, 4, 16)
    h = [16] * 4
    G, inv, nx2, xC = _prep(orc, X, C, h)
    e1 = orc.mse_fp64_refit(X, C, h, orc.beam_search(nx2, xC, G, h, 1)[0]).mean()
    e4 = orc.mse_fp64_refit(X, C, h, orc.beam_search(nx2, xC, G, h, 4)[0]).mean()
    e16 = orc.mse_fp64_refit(X, C, h, orc.beam_search(nx2, xC, G, h, 16)[0]).mean()
    assert e16 <= e4 * (1 + 1e-6) and e4 <= e1 * (1 + 1e-6)


def test_beam_tie_first_slot(orc):
    """Duplicate codewords give exactly tied candidates: the streaming rule keeps the first
    scanned one (strict '<' insertion), so the lower code index wins at the boundary."""
    rng = np.random.default_rng(7)
    d = 8
    C = rng.standard_normal((12, d)).astype(np.float32)
    C[5] = C[2]          # layer 0: codes 2 and 5 identical
    C[6 + 4] = C[6 + 1]  # layer 1: codes 1 and 4 identical
    h = [6, 6]
    X = rng.standard_normal((300, d)).astype(np.float32)
    G, inv, nx2, xC = _prep(orc, X, C, h)
    codes, err = orc.beam_search(nx2, xC, G, h, 1)
    assert not np.any(codes[:, 0] == 5)
    assert not np.any(codes[:, 1] == 4)


def test_ls_orthogonal_closed_form(orc):
    """Orthogonal codewords: G is diagonal and a_l = <x, c_l> / ||c_l||^2."""
    d, h = 12, [4, 4, 4]
    Q, _ = np.linalg.qr(np.random.default_rng(8).standard_normal((d, d)))
    C = (Q.T * np.linspace(0.5, 3.0, d)[:, None]).astype(np.float32)  # 12 mutually orthogonal rows
    X = np.random.default_rng(9).standard_normal((50, d)).astype(np.float32)
    G, inv, nx2, xC = _prep(orc, X, C, h)
    codes = np.random.default_rng(10).integers(0, 4, size=(50, 3)).astype(np.uint8)
    a, fails = orc.solve_ls_all(xC, G, h, codes)
    assert fails == 0
    flat = codes + offsets(h)[None, :]
    C64 = C.astype(np.float64)
    want = np.take_along_axis(X.astype(np.float64) @ C64.T, flat, 1) / np.sum(C64 ** 2, axis=1)[flat]
    np.testing.assert_allclose(a, want, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("m", [3, 5, 8, 10])
def test_ls_matches_fp64(orc, m):
    X, C = random_problem(11 + m, 80, 20, [8] * m)
    h = [8] * m
    G, inv, nx2, xC = _prep(orc, X, C, h)
    codes = np.random.default_rng(m).integers(0, 8, size=(80, m)).astype(np.uint8)
    a, fails = orc.solve_ls_all(xC, G, h, codes)
    assert fails == 0
    flat = codes + offsets(h)[None, :]
    C64 = C.astype(np.float64)
    for i in range(0, 80, 7):
        Cs = C64[flat[i]]
        want = np.linalg.solve(Cs @ Cs.T, Cs @ X[i].astype(np.float64))
        np.testing.assert_allclose(a[i], want, rtol=2e-3, atol=2e-3 * np.abs(want).max())
    cost = orc.compute_costs(xC, G, h, codes, a, nx2)
    ex = orc.mse_fp64_refit(X, C, h, codes)
    np.testing.assert_allclose(cost, ex, rtol=1e-3, atol=1e-3 * float(nx2.mean()))


def test_ls_retry_bumps_and_failure(orc):
    """least_squares.cpp:112-128: a zero codeword in the tuple fails the plain Cholesky; the
    retries add 1e-6, 1e-5, 1e-4 to the diagonal. With the m in {5,10} test (pivot <= 1e-6) the
    first success is at 1e-5; with LAPACK's test (pivot <= 0) it is at 1e-6. A NaN codeword
    fails every retry under LAPACK's test and yields zero coefficients."""
    rng = np.random.default_rng(12)
    d = 9
    for m, bump in ((5, np.float32(1e-6) * np.float32(10.0)), (4, np.float32(1e-6))):
        h = [4] * m
        C = rng.standard_normal((4 * m, d)).astype(np.float32)
        C[4 + 1] = 0.0
        X = rng.standard_normal((2, d)).astype(np.float32)
        G, inv, nx2, xC = _prep(orc, X, C, h)
        codes = np.array([[2, 1] + [0] * (m - 2), [0, 0] + [1] * (m - 2)], np.uint8)
        a, fails = orc.solve_ls_all(xC, G, h, codes)
        assert fails == 0
        flat = codes[0] + offsets(h)
        Gs = G[np.ix_(flat, flat)].astype(np.float64) + float(bump) * np.eye(m)
        want = np.linalg.solve(Gs, xC[0, flat].astype(np.float64))
        np.testing.assert_allclose(a[0], want, rtol=1e-3)
        assert a[0, 1] == 0.0
    C[4 + 1, 0] = np.nan
    G, inv, nx2, xC = _prep(orc, X, C, h)
    a, fails = orc.solve_ls_all(xC, G, h, codes)
    assert fails == 1 and np.all(a[0] == 0.0) and np.all(np.isfinite(a[1]))


def test_icm_monotone_and_fixed_point(orc):
    X, C = rvq_problem(13, 600, 16, 6, 32)
    h = [32] * 6
    G, inv, nx2, xC = _prep(orc, X, C, h)
    codes0, _ = orc.beam_search(nx2, xC, G, h, 2)
    a0, _ = orc.solve_ls_all(xC, G, h, codes0)
    cost0 = orc.compute_costs(xC, G, h, codes0, a0, nx2)
    codes1, a1, cost1, _ = orc.icm(xC, G, inv, h, nx2, codes0, 4, True, 38251450)
    assert np.all(cost1 <= cost0 + 1e-3)
    assert np.all(codes1[:, 0] == codes0[:, 0]), "layer 0 is frozen in RunIcm"
    changed = np.any(codes1 != codes0, axis=1)
    assert np.all(cost1[changed] + 1e-6 < cost0[changed])  # acceptance rule icm.cpp:321
    assert changed.any()
    # a and cost returned are the LS refit / SampleCost of the final codes
    a_chk, _ = orc.solve_ls_all(xC, G, h, codes1)
    np.testing.assert_array_equal(a_chk, a1)
    np.testing.assert_array_equal(orc.compute_costs(xC, G, h, codes1, a1, nx2), cost1)
    # Converged codes are a fixed point: more sweeps from there change nothing.
    codes2, _, _, _ = orc.icm(xC, G, inv, h, nx2, codes1, 30, True, 1)
    codes3, _, _, _ = orc.icm(xC, G, inv, h, nx2, codes2, 30, True, 2)
    assert np.array_equal(codes2, codes3)


def test_icm_orders_are_permutations(orc):
    o = orc.icm_orders(8, 5, 38251450)
    assert o.shape == (5, 8)
    for row in o:
        assert sorted(row.tolist()) == list(range(8))
    assert np.array_equal(o, orc.icm_orders(8, 5, 38251450))
    assert not np.array_equal(o, orc.icm_orders(8, 5, 1))


def test_large_root_full_width_is_exhaustive(orc):
    """Large-root beam with every root candidate kept equals exhaustive search."""
    rng = np.random.default_rng(14)
    d, h = 6, [12, 5, 5]  # 12 roots x 5 = 60 <= 64 prefixes kept after layer 1
    C0 = rng.standard_normal((12, d)).astype(np.float32)
    Cs = rng.standard_normal((10, d)).astype(np.float32)
    X = (rng.standard_normal((30, d)) * 1.3).astype(np.float32)
    norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs)
    nx2 = orc.xnorm2(X)
    xs = orc.gemm_xc(Cs, X)
    cid, Bs, err = orc.beam_search_large_root(X, nx2, C0, norm0, xs, Gs, G0S, h, 64)
    codes = np.concatenate([cid[:, None].astype(np.int64), Bs.astype(np.int64)], axis=1)
    C_all = np.concatenate([C0, Cs], axis=0)
    _, ex_cost = exhaustive(X, C_all, h)
    got = orc.mse_fp64_refit(X, C_all, h, codes.astype(np.uint8))
    np.testing.assert_allclose(got, ex_cost, rtol=1e-6, atol=1e-9)


def test_large_root_matches_full_precomp_semantics(orc):
    """With a root layer small enough for the full precomp, the large-root beam returns the
    same codes as the full beam (same candidate order; only 1/diag scaling differs), except on
    near-ties."""
    X, C = rvq_problem(15, 400, 12, 4, 16)
    h = [16] * 4
    G, inv, nx2, xC = _prep(orc, X, C, h)
    full, _ = orc.beam_search(nx2, xC, G, h, 4)
    C0, Cs = C[:16], C[16:]
    norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs)
    xs = orc.gemm_xc(Cs, X)
    cid, Bs, _ = orc.beam_search_large_root(X, nx2, C0, norm0, xs, Gs, G0S, h, 4)
    lr = np.concatenate([cid[:, None], Bs], axis=1).astype(np.uint8)
    assert np.mean(np.all(lr == full, axis=1)) >= 0.99


def test_forced_root(orc):
    X, C = rvq_problem(16, 300, 12, 4, 16)
    h = [16] * 4
    C0, Cs = C[:16], C[16:]
    norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs)
    nx2 = orc.xnorm2(X)
    xs = orc.gemm_xc(Cs, X)
    forced = np.random.default_rng(1).integers(0, 16, size=300).astype(np.uint32)
    cid, Bs, err = orc.beam_search_large_root(X, nx2, C0, norm0, xs, Gs, G0S, h, 4, forced_root=forced)
    assert np.array_equal(cid, forced)
    # nearest-root forcing picks argmin of ||x||^2 - gamma^2/alpha
    cid1, _, _ = orc.beam_search_large_root(X, nx2, C0, norm0, xs, Gs, G0S, h, 4, root_mode=1)
    g = X.astype(np.float64) @ C0.astype(np.float64).T
    want = np.argmax(g * g / np.sum(C0.astype(np.float64) ** 2, axis=1), axis=1)
    assert np.mean(cid1 == want) >= 0.99


def test_ils_never_worse_and_shard_invariant(orc):
    """ILS only accepts strict improvements, so every vector's cost is at most its ICM-only cost;
    perturbations are keyed by the global sample id, so two shards with their offsets reproduce
    the whole set exactly."""
    h = [32] * 6
    X, C = rvq_problem(61, 1200, 24, 6, 32, train_n=2000, iters=3)
    G, inv, nx2, xC = _prep(orc, X, C, h)
    codes, _ = orc.beam_search(nx2, xC, G, h, 4)
    k0, a0, c0, _ = orc.icm(xC, G, inv, h, nx2, codes, 2, True, 9)
    k1, a1, c1, _ = orc.icm_ils(xC, G, inv, h, nx2, codes, 2, 4, 3, True, 9)
    assert np.all(c1 <= c0)
    assert np.any(k1 != k0)  # the rounds did move some vectors
    ka, aa, ca, _ = orc.icm_ils(xC[:700], G, inv, h, nx2[:700], codes[:700], 2, 4, 3, True, 9, 0)
    kb, ab, cb, _ = orc.icm_ils(xC[700:], G, inv, h, nx2[700:], codes[700:], 2, 4, 3, True, 9, 700)
    assert np.array_equal(np.concatenate([ka, kb]), k1)
    assert np.array_equal(np.concatenate([ca, cb]).view(np.uint32), c1.view(np.uint32))
    # ils_iters = 0 is the plain ICM
    k2, _, c2, _ = orc.icm_ils(xC, G, inv, h, nx2, codes, 2, 0, 3, True, 9)
    assert np.array_equal(k2, k0) and np.array_equal(c2.view(np.uint32), c0.view(np.uint32))
