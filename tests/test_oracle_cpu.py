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


# ---------------------------------------------------------------------------------------------
# Root scan of the large-root beam (beam_search.cpp:686-705; RecomputeWorst :101-113). Roots are
# scaled unit vectors s e_j with s a power of two and x has small integer entries, so every
# quantity of the scan is exact in fp32: gamma = s x_j, a0 = x_j / s, e = |x|^2 - x_j^2, r00 = s.

def _unit_roots(spec, d):
    """spec: list of (axis, scale) -> C0 rows (scale 0: a zero root)."""
    C0 = np.zeros((len(spec), d), np.float32)
    for c, (j, s) in enumerate(spec):
        C0[c, j] = s
    return C0


def _scan(orc, x, C0, H, root_mode=0, norm0=None, forced=None):
    X = np.asarray(x, np.float32)[None, :]
    nx2 = orc.xnorm2(X)
    if norm0 is None:
        norm0 = np.sum(C0.astype(np.float64) ** 2, axis=1).astype(np.float32)
    fr = None if forced is None else np.array([forced], np.uint32)
    e, c, a0, r00 = orc.large_root_candidates(X, nx2, C0, norm0, H, forced_root=fr, root_mode=root_mode)
    return e[0], c[0], a0[0], r00[0]


X_ROOT = [3.0, 1.0, 2.0, 0.0]  # |x|^2 = 14; a root on axis 0/1/2/3 leaves 5/13/10/14


def test_root_scan_duplicates_lower_code_wins(orc):
    """Equal errors never displace a kept root (the e >= worst skip), so among duplicates the
    lowest code is kept; with two slots, the replaced slot is the first one holding the worst."""
    C0 = _unit_roots([(1, 1.0), (0, 2.0), (2, 1.0), (0, 4.0), (0, 2.0)], 4)  # errors 13, 5, 10, 5, 5
    e, c, a0, r00 = _scan(orc, X_ROOT, C0, 1, root_mode=1)
    assert (c[0], e[0], a0[0], r00[0]) == (1, 5.0, 1.5, 2.0)
    e, c, a0, r00 = _scan(orc, X_ROOT, C0, 2)
    # slots: [13,inf] -> [13,5] -> [10,5] -> [5(code 3),5(code 1)]; code 4 (5 >= 5) is skipped
    assert list(c) == [3, 1] and list(e) == [5.0, 5.0] and list(a0) == [0.75, 1.5] and list(r00) == [4.0, 2.0]
    # equal errors in both slots: a better root replaces slot 0, evicting code 0 and keeping code 1
    x = [2.0, 1.0, 3.0, 0.0]  # |x|^2 = 14: errors 10, 10, 5
    e, c, _, _ = _scan(orc, x, _unit_roots([(0, 1.0), (0, 2.0), (2, 1.0)], 4), 2)
    assert list(c) == [2, 1] and list(e) == [5.0, 10.0]


def test_root_scan_zero_norm_roots_are_skipped(orc):
    """alpha == 0 roots never enter (their 0/0 would be NaN), also under a forced root; with
    every root zero, all slots keep the initial (+inf, code 0, 0, 0)."""
    C0 = _unit_roots([(1, 1.0), (0, 0.0), (2, 1.0)], 4)  # the zero root would otherwise be free
    e, c, _, _ = _scan(orc, X_ROOT, C0, 1, root_mode=1)
    assert (c[0], e[0]) == (2, 10.0)
    e, c, a0, r00 = _scan(orc, X_ROOT, _unit_roots([(0, 0.0)] * 3, 4), 2)
    assert np.all(np.isinf(e)) and not c.any() and not a0.any() and not r00.any()
    e, c, _, _ = _scan(orc, X_ROOT, C0, 2, forced=1)
    assert np.isinf(e[0]) and np.isinf(e[1])
    e, c, a0, r00 = _scan(orc, X_ROOT, C0, 2, forced=2)
    assert (c[0], e[0], a0[0], r00[0]) == (2, 10.0, 2.0, 1.0) and np.isinf(e[1])


def test_root_scan_nan_root_enters_and_is_replaced(orc):
    """A NaN error passes the e >= worst skip, so it enters; RecomputeWorst's e > we never selects
    it unless it sits in slot 0, where it is the worst and the next root replaces it. Elsewhere
    it stays. norm0 is handed in, so a NaN norm gives the NaN error."""
    C0 = _unit_roots([(1, 1.0), (0, 1.0), (2, 1.0), (0, 1.0)], 4)  # errors 13, 5, NaN, 5
    norm0 = np.array([1.0, 1.0, np.nan, 1.0], np.float32)
    e, c, _, _ = _scan(orc, X_ROOT, C0, 1, root_mode=1, norm0=norm0)
    assert (c[0], e[0]) == (3, 5.0)  # NaN replaced code 1, then code 3 (5 >= NaN is false) replaced it
    C0 = _unit_roots([(0, 1.0), (1, 1.0), (2, 1.0), (2, 1.0), (3, 2.0)], 4)  # errors 5, 13, NaN, 10, 14
    norm0 = np.array([1.0, 1.0, np.nan, 1.0, 4.0], np.float32)
    X2 = [2.0, 1.0, 2.0, 3.0]  # |x|^2 = 18: errors 14, 17, NaN, 14, 9
    e, c, _, _ = _scan(orc, X2, C0, 2, norm0=norm0)
    # [14,inf] -> [14,17] -> [14,NaN] (worst slot 1 held 17) -> code 3 (14 >= 14) skipped ->
    # code 4 (9 < 14) takes slot 0; the NaN in slot 1 is never the worst again
    assert c[0] == 4 and e[0] == 9.0 and c[1] == 2 and np.isnan(e[1])


def test_root_scan_keeps_h_smallest_errors(orc):
    """Without NaN the kept errors are the H smallest errors (a strict-improvement top-H), each
    with its own code; which of several equal errors survives depends on the slot order (the
    first slot holding the worst is replaced, so an equal later code can outlive an earlier one).
    Brute force over many ties."""
    rng = np.random.default_rng(21)
    d, h0 = 5, 40
    for trial in range(60):
        axes = rng.integers(0, d, h0)
        scales = 2.0 ** rng.integers(-2, 3, h0)
        scales[rng.random(h0) < 0.1] = 0.0
        C0 = _unit_roots(list(zip(axes, scales)), d)
        x = rng.integers(-3, 4, d).astype(np.float32)
        H = int(rng.integers(1, 9))
        e, c, _, _ = _scan(orc, x, C0, H)
        err = np.array([np.sum(x ** 2) - x[j] ** 2 if s else np.inf for j, s in zip(axes, scales)])
        live = [k for k in range(h0) if scales[k] != 0.0]
        want = sorted(err[k] for k in live)[:H]
        kept = [(int(k), float(ek)) for k, ek in zip(c, e) if np.isfinite(ek)]
        assert sorted(ek for _, ek in kept) == want, (trial, kept, want)
        assert len({k for k, _ in kept}) == len(kept)
        for k, ek in kept:
            assert scales[k] != 0.0 and ek == err[k]


def test_precomp_large_root_exact_on_integers(orc):
    """Integer codebooks: every sum is exact in fp32, so norm0, G_small and G0S equal the integer
    products whatever the summation order; d = 37 exercises the 4-lane tail. Pins the layouts
    (G0S[flat, root] = <C_small[flat], C0[root]>, G_small symmetric)."""
    rng = np.random.default_rng(5)
    d, h0, Hs = 37, 23, 19
    C0 = rng.integers(-8, 9, (h0, d)).astype(np.float32)
    Cs = rng.integers(-8, 9, (Hs, d)).astype(np.float32)
    norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs)
    C0i, Csi = C0.astype(np.int64), Cs.astype(np.int64)
    assert np.array_equal(norm0.astype(np.int64), np.sum(C0i * C0i, axis=1))
    assert np.array_equal(Gs.astype(np.int64), Csi @ Csi.T)
    assert np.array_equal(G0S.astype(np.int64), Csi @ C0i.T)


def test_precomp_large_root_fp64_bound(orc):
    """Random codebooks: each entry within the fp32 dot-product bound gamma_d sum |a_i b_i| of the
    fp64 product (Higham Thm 3.1)."""
    rng = np.random.default_rng(6)
    d, h0, Hs = 96, 50, 40
    C0 = rng.standard_normal((h0, d)).astype(np.float32)
    Cs = (rng.standard_normal((Hs, d)) * 0.3).astype(np.float32)
    norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs)
    gam = d * 2.0 ** -24 / (1 - d * 2.0 ** -24)
    A0, As = C0.astype(np.float64), Cs.astype(np.float64)
    for got, exact, mag in ((norm0, np.sum(A0 * A0, 1), np.sum(A0 * A0, 1)),
                            (Gs, As @ As.T, np.abs(As) @ np.abs(As).T),
                            (G0S, As @ A0.T, np.abs(As) @ np.abs(A0).T)):
        assert np.all(np.abs(got.astype(np.float64) - exact) <= gam * mag)
