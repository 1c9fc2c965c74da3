"""HIP encoder vs the CPU oracle, through the C ABI.

Bar: bit-exact wherever both sides see the same inputs (precomp, ||x||^2, beam codes and
selected errors given the same xC/G/||x||^2, LS coefficients, costs, ICM); for the end-to-end
encode, whose xC comes from fp32 MFMA on the GPU and from a sequential CPU dot product in the
oracle: codes differ on at most 0.1% of vectors, only where the two
code tuples' fp64 costs tie within 1e-5 relative, and per-vector fp64 MSE within 1e-5 relative.
"""
import numpy as np
import pytest

from stlq_amd.encoder import EncodeConfig
from tests.helpers import BEAM_CASES, DEGENERATE, beam_case, degenerate_problem, parity, random_problem, rvq_problem

pytestmark = pytest.mark.gpu


def _set(ctx, C, h):
    ctx.set_codebooks(C, h)
    return ctx.get_precomp()


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def test_precomp_bit_exact(ctx, orc):
    X, C = rvq_problem(1, 100, 37, 3, 40)
    h = [40, 40, 40]
    G, inv = _set(ctx, C, h)
    Go, invo = orc.build_precomp(C, h)
    assert np.array_equal(_bits(G), _bits(Go))
    assert np.array_equal(_bits(inv), _bits(invo))


@pytest.mark.parametrize("d", [1, 3, 13, 37, 96, 128, 130, 960])
def test_xnorm_bit_exact(ctx, orc, d):
    """||x||^2 in the reference build's OpenMP-simd order, aligned and ragged d."""
    X, C = random_problem(2 + d, 3001, d, [8, 8], x_scale=50.0)
    ctx.set_codebooks(C, [8, 8])
    assert np.array_equal(_bits(ctx.xnorm2(X)), _bits(orc.xnorm2(X)))


@pytest.mark.parametrize("n,d,H", [(1000, 128, 2048), (777, 96, 300), (130, 7, 48), (257, 960, 512)])
def test_gemm_xc_close(ctx, orc, n, d, H):
    rng = np.random.default_rng(n + d)
    X = (rng.standard_normal((n, d)) * 3).astype(np.float32)
    C = rng.standard_normal((H, d)).astype(np.float32)
    ctx.set_codebooks(C, [256] * (H // 256) + ([H % 256] if H % 256 else []))
    xg = ctx.gemm_xc(X)
    x64 = X.astype(np.float64) @ C.astype(np.float64).T
    scale = np.sqrt(np.sum(X.astype(np.float64) ** 2, 1))[:, None] * np.sqrt(np.sum(C.astype(np.float64) ** 2, 1))[None, :]
    assert np.max(np.abs(xg - x64) / scale) < 4 * d * 2.0 ** -24


@pytest.mark.parametrize("name,seed,n,d,h,Hb,kind", BEAM_CASES, ids=[c[0] for c in BEAM_CASES])
def test_beam_bit_exact_given_same_inputs(ctx, orc, name, seed, n, d, h, Hb, kind):
    X, C = beam_case(seed, n, d, h, kind)
    G, inv = _set(ctx, C, h)
    nx2 = orc.xnorm2(X)
    xC = orc.gemm_xc(C, X)
    codes_o, err_o = orc.beam_search(nx2, xC, G, h, Hb)
    codes_g, err_g = ctx.beam_search(xC, Hb, nx2=nx2)
    bad = np.nonzero(np.any(codes_o != codes_g, axis=1))[0]
    assert bad.size == 0, (name, bad[:10], codes_o[bad[:3]], codes_g[bad[:3]])
    assert np.array_equal(_bits(err_o), _bits(err_g))


def test_beam_from_gpu_xc_bit_exact(ctx, orc):
    """The oracle fed the GPU's own xC, G and ||x||^2 reproduces the GPU encode exactly."""
    X, C = rvq_problem(21, 2000, 128, 8, 256, kind="desc", train_n=3000, iters=4)
    h = [256] * 8
    G, inv = _set(ctx, C, h)
    xg = ctx.gemm_xc(X)
    nx = ctx.xnorm2(X)
    codes_g, _, _, _ = ctx.encode(X, EncodeConfig(H_beam=16, icm_iters=0, want_coeffs=False))
    codes_o, _ = orc.beam_search(nx, xg, G, h, 16)
    assert np.array_equal(codes_g, codes_o)


@pytest.mark.parametrize("case", DEGENERATE)
def test_beam_degenerate_bit_exact(ctx, orc, case):
    """Exact ties, skipped candidates (alpha == 0, denom == 0), non-finite beam errors and the
    all-skipped fallback follow the reference's slot rules bit for bit."""
    X, C, h = degenerate_problem(case)
    G, inv = _set(ctx, C, h)
    nx2 = orc.xnorm2(X)
    xC = orc.gemm_xc(C, X)
    for Hb in (1, 2, 5, 16):
        codes_o, err_o = orc.beam_search(nx2, xC, G, h, Hb)
        codes_g, err_g = ctx.beam_search(xC, Hb, nx2=nx2)
        assert np.array_equal(codes_o, codes_g), (case, Hb)
        # bit for bit, except that a NaN's payload is the platform's (x86 and gfx950 differ)
        same = (_bits(err_o) == _bits(err_g)) | (np.isnan(err_o) & np.isnan(err_g))
        assert np.all(same), (case, Hb, np.nonzero(~same)[0][:10])


def _beam_both_orders(ctx, xC, Hb, nx2, monkeypatch):
    """Beam codes, errors and re-run count with the default best-first pass, then in the
    reference order throughout."""
    monkeypatch.delenv("STLQ_MI355_BEAM_ORDER", raising=False)
    codes_b, err_b = ctx.beam_search(xC, Hb, nx2=nx2)
    reruns = ctx.last_timings().beam_reruns
    monkeypatch.setenv("STLQ_MI355_BEAM_ORDER", "reference")
    codes_r, err_r = ctx.beam_search(xC, Hb, nx2=nx2)
    assert ctx.last_timings().beam_reruns == 0
    monkeypatch.delenv("STLQ_MI355_BEAM_ORDER")
    return codes_b, err_b, codes_r, err_r, reruns


def test_best_first_beam_equals_reference_order(ctx, orc, monkeypatch):
    """The best-first pass plus the re-run of its flagged vectors returns the reference order's
    codes and errors bit for bit, and on descriptor-like data re-runs only a small fraction."""
    X, C = rvq_problem(31, 20000, 128, 8, 256, kind="desc", train_n=4000, iters=4)
    h = [256] * 8
    G, inv = _set(ctx, C, h)
    nx2 = orc.xnorm2(X)
    xC = ctx.gemm_xc(X)
    for Hb in (4, 16):
        codes_b, err_b, codes_r, err_r, reruns = _beam_both_orders(ctx, xC, Hb, nx2, monkeypatch)
        assert np.array_equal(codes_b, codes_r), Hb
        assert np.array_equal(_bits(err_b), _bits(err_r)), Hb
        assert reruns <= 0.01 * X.shape[0], (Hb, reruns)
    codes_o, err_o = orc.beam_search(nx2, xC, G, h, 16)
    assert np.array_equal(codes_b, codes_o)


@pytest.mark.parametrize("case", ["dup_within_layer", "dup_across_layers", "scaled_copies", "nan_codeword"])
def test_best_first_beam_reruns_ties(ctx, orc, monkeypatch, case):
    """Ties at the top-H boundary (duplicate or zero codewords) and NaN errors send vectors to the
    reference-order re-run; the results stay the reference's."""
    X, C, h = degenerate_problem(case)
    G, inv = _set(ctx, C, h)
    nx2 = orc.xnorm2(X)
    xC = orc.gemm_xc(C, X)
    for Hb in (2, 5, 16):
        codes_b, err_b, codes_r, err_r, reruns = _beam_both_orders(ctx, xC, Hb, nx2, monkeypatch)
        assert np.array_equal(codes_b, codes_r), (case, Hb)
        same = (_bits(err_b) == _bits(err_r)) | (np.isnan(err_b) & np.isnan(err_r))
        assert np.all(same), (case, Hb)
        codes_o, _ = orc.beam_search(nx2, xC, G, h, Hb)
        assert np.array_equal(codes_b, codes_o), (case, Hb)
        if case == "nan_codeword":  # every vector meets a NaN candidate at layer 2
            assert reruns == X.shape[0], (case, Hb, reruns)


def test_beam_user_precomp_nonsymmetric(ctx, orc):
    """set_precomp with a caller's G: every read uses the reference's G(row, col) element."""
    X, C = random_problem(22, 500, 16, [20, 20, 20], x_scale=2.0)
    h = [20, 20, 20]
    G, inv = orc.build_precomp(C, h)
    Gp = G.copy()
    rng = np.random.default_rng(3)
    Gp += (rng.standard_normal(G.shape) * 1e-3).astype(np.float32)  # no longer symmetric
    ctx.set_precomp(C, h, Gp, inv)
    G2, _ = ctx.get_precomp()
    assert np.array_equal(G2, Gp)
    nx2 = orc.xnorm2(X)
    xC = orc.gemm_xc(C, X)
    codes_o, err_o = orc.beam_search(nx2, xC, Gp, h, 6)
    codes_g, err_g = ctx.beam_search(xC, 6, nx2=nx2)
    assert np.array_equal(codes_o, codes_g)
    assert np.array_equal(_bits(err_o), _bits(err_g))
    codes_i, a_i, cost_i, _ = orc.icm(xC, Gp, inv, h, nx2, codes_o, 2, True, 5)
    codes_j, a_j, cost_j = ctx.icm(xC, codes_o, 2, True, 5, nx2=nx2)
    assert np.array_equal(codes_i, codes_j)
    assert np.array_equal(_bits(a_i), _bits(a_j))


@pytest.mark.parametrize("m", [1, 3, 4, 5, 8, 10, 16, 20])
def test_ls_and_costs_bit_exact(ctx, orc, m):
    h = [32] * m
    X, C = random_problem(30 + m, 1500, 24, h, x_scale=2.0)
    G, inv = _set(ctx, C, h)
    nx2 = orc.xnorm2(X)
    xC = orc.gemm_xc(C, X)
    codes = np.random.default_rng(m).integers(0, 32, size=(1500, m)).astype(np.uint8)
    codes[7, :] = codes[7, 0]  # tuples that need the retry bumps: same code index in every layer
    a_o, f_o = orc.solve_ls_all(xC, G, h, codes)
    a_g, f_g = ctx.solve_ls_all(xC, codes)
    assert f_o == f_g
    assert np.array_equal(_bits(a_o), _bits(a_g))
    c_o = orc.compute_costs(xC, G, h, codes, a_o, nx2)
    c_g = ctx.compute_costs(xC, codes, a_o, nx2)
    assert np.array_equal(_bits(c_o), _bits(c_g))


@pytest.mark.parametrize("use_abs", [True, False])
@pytest.mark.parametrize("m,K,d,iters", [(8, 256, 96, 2), (5, 64, 32, 4), (10, 32, 40, 3), (16, 64, 48, 1),
                                         (20, 24, 24, 2)])
def test_icm_bit_exact(ctx, orc, use_abs, m, K, d, iters):
    h = [K] * m
    X, C = rvq_problem(40 + m, 1200, d, m, K, kind="sphere" if d == 96 else "gauss", train_n=max(2000, 4 * K), iters=4)
    G, inv = _set(ctx, C, h)
    nx2 = orc.xnorm2(X)
    xC = orc.gemm_xc(C, X)
    codes0, _ = orc.beam_search(nx2, xC, G, h, 2)
    seed = 38251450
    co, ao, so, fo = orc.icm(xC, G, inv, h, nx2, codes0, iters, use_abs, seed)
    cg, ag, sg = ctx.icm(xC, codes0, iters, use_abs, seed, nx2=nx2)
    assert np.any(co != codes0)
    assert np.array_equal(co, cg)
    assert np.array_equal(_bits(ao), _bits(ag))
    assert np.array_equal(_bits(so), _bits(sg))


@pytest.mark.parametrize("m,K,d,icm,ils,pk,off", [(4, 64, 32, 2, 3, 2, 0), (5, 64, 32, 1, 4, 3, 5000),
                                                  (8, 256, 96, 2, 2, 3, 0), (10, 32, 40, 0, 3, 10, 77)])
def test_ils_bit_exact(ctx, orc, m, K, d, icm, ils, pk, off):
    """ICM + ILS rounds (perturbation stream keyed by global sample id, continuing layer-order
    stream, accept-if-better) match the oracle bit for bit."""
    h = [K] * m
    X, C = rvq_problem(60 + m, 1500, d, m, K, kind="sphere" if d == 96 else "gauss", train_n=max(2000, 4 * K),
                       iters=4)
    G, inv = _set(ctx, C, h)
    nx2 = orc.xnorm2(X)
    xC = orc.gemm_xc(C, X)
    codes0, _ = orc.beam_search(nx2, xC, G, h, 2)
    seed = 38251450
    for use_abs in (True, False):
        co, ao, so, _ = orc.icm_ils(xC, G, inv, h, nx2, codes0, icm, ils, pk, use_abs, seed, off)
        cg, ag, sg = ctx.icm_ils(xC, codes0, icm, ils, pk, use_abs, seed, nx2=nx2, sample_id_offset=off)
        if icm > 0:  # (without ICM sweeps a random perturbation is hardly ever an improvement)
            ci, _, _, _ = orc.icm(xC, G, inv, h, nx2, codes0, icm, use_abs, seed)
            assert np.any(co != ci)  # the ILS rounds moved some vectors
        assert np.array_equal(co, cg), (use_abs, np.nonzero(np.any(co != cg, axis=1))[0][:10])
        assert np.array_equal(_bits(ao), _bits(ag))
        assert np.array_equal(_bits(so), _bits(sg))


def _oracle_encode(orc, X, C, h, Hb, icm_iters=0, use_abs=True, seed=38251450, gemm_mode=1, ils_iters=0,
                   perturb_k=3):
    G, inv = orc.build_precomp(C, h)
    nx2 = orc.xnorm2(X)
    xC = orc.gemm_xc(C, X, mode=gemm_mode)
    codes, err = orc.beam_search(nx2, xC, G, h, Hb)
    if ils_iters:
        codes, a, cost, _ = orc.icm_ils(xC, G, inv, h, nx2, codes, icm_iters, ils_iters, perturb_k, use_abs, seed)
    elif icm_iters:
        codes, a, cost, _ = orc.icm(xC, G, inv, h, nx2, codes, icm_iters, use_abs, seed)
    else:
        a, _ = orc.solve_ls_all(xC, G, h, codes)
        cost = orc.compute_costs(xC, G, h, codes, a, nx2)
    return codes, a, cost


def _scaled_config(cfg, n=None):
    from stlq_amd import workloads

    w = workloads.CONFIGS[cfg]
    n = n or {"C1": 20000, "C2": 4000, "C3": 4000, "C4": 1000}[cfg]
    mix = workloads.Mixture(w.kind, w.d, w.n_comp, w.seed)
    Xtr = mix.sample(10_000_000, 4000 if w.d < 900 else 2000)
    C = workloads.residual_codebooks(Xtr, w.m, w.K, 4, w.seed + 5, spherical=(w.kind == "sphere"))
    X = mix.sample(0, n)
    return w, X, C, [w.K] * w.m


@pytest.mark.parametrize("cfg", ["C1", "C2", "C3", "C4"])
def test_encode_end_to_end_bit_exact(ctx, orc, cfg):
    """Scaled-down benchmark configurations, GPU end to end (MFMA xC, beam, [ICM], LS, cost)
    vs the oracle end to end with xC accumulated in the device GEMM's fused k order:
    codes, coefficients and costs are identical."""
    w, X, C, h = _scaled_config(cfg)
    ctx.set_codebooks(C, h)
    cfgc = EncodeConfig(H_beam=w.H_beam, icm_iters=w.icm_iters, want_coeffs=True)
    codes_g, a_g, cost_g, (bm, fm) = ctx.encode(X, cfgc, want_mse=True)
    codes_o, a_o, cost_o = _oracle_encode(orc, X, C, h, w.H_beam, w.icm_iters, gemm_mode=1)
    bad = np.nonzero(np.any(codes_o != codes_g, axis=1))[0]
    assert bad.size == 0, (cfg, bad.size, bad[:10])
    assert np.array_equal(_bits(a_o), _bits(a_g))
    assert np.array_equal(_bits(cost_o), _bits(cost_g))
    assert np.isfinite(bm) and np.isfinite(fm) and fm <= bm * (1 + 1e-6)
    want_fm = np.mean(np.maximum(cost_o.astype(np.float64), 0.0))
    assert abs(fm - want_fm) <= 1e-9 * abs(want_fm)


def test_encode_with_ils_end_to_end(ctx, orc, monkeypatch):
    """EncodeBase with the production ILS defaults (4 ICM sweeps, 32 ILS rounds, 3 perturbed
    codes): GPU end to end equals the oracle; tiled encodes (global sample ids per tile), the
    device entry point and the stream agree with it too."""
    X, C = rvq_problem(53, 3000, 32, 6, 64, train_n=2000, iters=3)
    h = [64] * 6
    ctx.set_codebooks(C, h)
    cfg = EncodeConfig(H_beam=4, icm_iters=4, ils_iters=32, perturb_k=3, want_coeffs=True)
    codes_g, a_g, cost_g, (bm, fm) = ctx.encode(X, cfg, want_mse=True)
    codes_o, a_o, cost_o = _oracle_encode(orc, X, C, h, 4, icm_iters=4, ils_iters=32, perturb_k=3)
    assert np.array_equal(codes_o, codes_g)
    assert np.array_equal(_bits(a_o), _bits(a_g))
    assert np.array_equal(_bits(cost_o), _bits(cost_g))
    assert fm <= bm
    monkeypatch.setenv("STLQ_MI355_WORKSPACE_GB", "0.0005")  # ~1k-vector tiles
    codes_t, _, cost_t, _ = ctx.encode(X, cfg)
    assert np.array_equal(codes_t, codes_g) and np.array_equal(_bits(cost_t), _bits(cost_g))
    monkeypatch.delenv("STLQ_MI355_WORKSPACE_GB")
    got = {}

    def fill(first, count, dst):
        dst[:] = X[first:first + count]

    def sink(first, count, res):
        got[first] = (res["codes"].copy(), res["cost"].copy())

    ctx.encode_stream(X.shape[0], 700, cfg, fill, sink)
    codes_s = np.concatenate([got[k][0] for k in sorted(got)])
    cost_s = np.concatenate([got[k][1] for k in sorted(got)])
    assert np.array_equal(codes_s, codes_g) and np.array_equal(_bits(cost_s), _bits(cost_g))


@pytest.mark.parametrize("cfg", ["C1", "C2", "C3"])
def test_encode_parity_unfused_oracle_xc(ctx, orc, cfg):
    """Sensitivity to the GEMM summation order (the reference's BLAS order is unpinned): against
    an oracle whose xC is a non-fused sequential dot, the codes differ only on cost ties —
    every differing vector's two tuples have fp64 LS costs equal within 1e-5 relative — and on
    at most 0.1% of the vectors."""
    w, X, C, h = _scaled_config(cfg)
    print(f"unfused parity {cfg} n={X.shape[0]}", flush=True)
    ctx.set_codebooks(C, h)
    cfgc = EncodeConfig(H_beam=w.H_beam, icm_iters=w.icm_iters, want_coeffs=True)
    codes_g, _, _, _ = ctx.encode(X, cfgc)
    codes_o, _, _ = _oracle_encode(orc, X, C, h, w.H_beam, w.icm_iters, gemm_mode=0)
    rep = parity(orc, X, C, h, codes_o, codes_g, max_frac=1e-3)
    print(rep, flush=True)
    assert rep["ok"], rep


def test_encode_parity_c4_10k(ctx, orc):
    """C4 (d=960, M=16, K=256, beam 8) on 10,000 vectors. With the oracle's xC in the device GEMM's
    fused k order the whole encode is bit-exact: codes, coefficients and costs, 0 of 10,000
    differing. Against an xC summed in the other (non-fused, sequential) order, the ulp-level
    differences of 960-term dot products change the beam's choices on a few tenths of a percent of
    the vectors, with real fp64-MSE differences (the beam is discontinuous in its inputs), so the
    per-vector tie rule cannot hold across summation orders. There the test bounds the share of
    differing vectors (< 1%) and the mean fp64 MSE (within 1e-4 relative, either direction)."""
    w, X, C, h = _scaled_config("C4", n=10_000)
    print(f"c4 10k: n={X.shape[0]}", flush=True)
    ctx.set_codebooks(C, h)
    cfgc = EncodeConfig(H_beam=w.H_beam, icm_iters=w.icm_iters, want_coeffs=True)
    codes_g, a_g, cost_g, _ = ctx.encode(X, cfgc)
    codes_f, a_f, cost_f = _oracle_encode(orc, X, C, h, w.H_beam, w.icm_iters, gemm_mode=1)
    bad = np.nonzero(np.any(codes_f != codes_g, axis=1))[0]
    assert bad.size == 0, (bad.size, bad[:10])
    assert np.array_equal(_bits(a_f), _bits(a_g))
    assert np.array_equal(_bits(cost_f), _bits(cost_g))
    codes_o, _, _ = _oracle_encode(orc, X, C, h, w.H_beam, w.icm_iters, gemm_mode=0)
    diff = np.any(codes_o != codes_g, axis=1)
    mse_g = orc.mse_fp64_refit(X, C, h, codes_g)
    mse_o = orc.mse_fp64_refit(X, C, h, codes_o)
    rel = (mse_g.sum() - mse_o.sum()) / mse_o.sum()
    print(f"c4 10k vs the non-fused xC order: {diff.sum()} differ, mean fp64 MSE rel diff {rel:.2e}", flush=True)
    assert diff.mean() < 1e-2
    assert abs(rel) <= 1e-4


def test_encode_device_matches_host(ctx, orc):
    X, C = rvq_problem(50, 3000, 64, 6, 128, train_n=2000, iters=3)
    h = [128] * 6
    ctx.set_codebooks(C, h)
    cfg = EncodeConfig(H_beam=8, icm_iters=1, want_coeffs=True)
    codes_h, a_h, cost_h, _ = ctx.encode(X, cfg)
    n, d, m = X.shape[0], X.shape[1], 6
    dX = ctx.dev_alloc(X.nbytes)
    dc = ctx.dev_alloc(n * m)
    da = ctx.dev_alloc(n * m * 4)
    ds = ctx.dev_alloc(n * 4)
    try:
        ctx.h2d(dX, X)
        ctx.encode_device(dX, n, cfg, dc, da, ds)
        ctx.synchronize()
        codes_d = ctx.d2h(np.empty((n, m), np.uint8), dc)
        a_d = ctx.d2h(np.empty((n, m), np.float32), da)
        cost_d = ctx.d2h(np.empty(n, np.float32), ds)
    finally:
        for p in (dX, dc, da, ds):
            ctx.dev_free(p)
    assert np.array_equal(codes_h, codes_d)
    assert np.array_equal(_bits(a_h), _bits(a_d))
    assert np.array_equal(_bits(cost_h), _bits(cost_d))
    t = ctx.last_timings()
    assert t.n == n and t.gemm_ms > 0 and t.beam_ms > 0


def test_tiled_encode_matches_single_tile(ctx, orc, monkeypatch):
    """Splitting the encode into workspace-bounded tiles does not change any result
    (mirrors tests/test_streaming_encode_base.cpp:253-268)."""
    X, C = rvq_problem(51, 5000, 32, 4, 64, train_n=2000, iters=3)
    h = [64] * 4
    ctx.set_codebooks(C, h)
    cfg = EncodeConfig(H_beam=4, icm_iters=2, want_coeffs=True)
    codes1, a1, cost1, _ = ctx.encode(X, cfg)
    monkeypatch.setenv("STLQ_MI355_WORKSPACE_GB", "0.0005")  # ~1k-vector tiles
    codes2, a2, cost2, _ = ctx.encode(X, cfg)
    assert np.array_equal(codes1, codes2)
    assert np.array_equal(_bits(a1), _bits(a2))
    assert np.array_equal(_bits(cost1), _bits(cost2))


@pytest.mark.parametrize("sub", [700, 2500])
def test_overlapped_subtiles_match_single_tile(ctx, orc, monkeypatch, sub):
    """Sub-tiles whose xC GEMM overlaps the previous sub-tile's beam (two streams, alternating
    buffers) give the same codes, coefficients, costs and MSE as one tile, with and without ICM."""
    X, C = rvq_problem(52, 6001, 32, 4, 64, train_n=2000, iters=3)
    h = [64] * 4
    ctx.set_codebooks(C, h)
    for icm in (2, 0):
        cfg = EncodeConfig(H_beam=4, icm_iters=icm, want_coeffs=True)
        want_mse = icm == 0  # (beam MSE before ICM keeps the whole tile's xC: no overlap there)
        monkeypatch.setenv("STLQ_MI355_PIPE_SUB", "0")
        codes1, a1, cost1, mse1 = ctx.encode(X, cfg, want_mse=want_mse)
        monkeypatch.setenv("STLQ_MI355_PIPE_SUB", str(sub))
        codes2, a2, cost2, mse2 = ctx.encode(X, cfg, want_mse=want_mse)
        t = ctx.last_timings()
        assert t.n == X.shape[0] and t.gemm_launches == -(-X.shape[0] // sub)
        assert np.array_equal(codes1, codes2), icm
        assert np.array_equal(_bits(a1), _bits(a2))
        assert np.array_equal(_bits(cost1), _bits(cost2))
        assert mse1 == mse2
        codes3, _, _, _ = ctx.encode(X, cfg)  # again, reusing the buffers and events
        assert np.array_equal(codes1, codes3)


@pytest.mark.parametrize("chunk", [1000, 1777, 5000])
def test_stream_matches_in_memory(ctx, chunk):
    from stlq_amd import workloads

    mix = workloads.Mixture("desc", 32, 64, 9)
    X = mix.sample(0, 5000)
    C = workloads.residual_codebooks(mix.sample(1_000_000, 2000), 4, 64, 3, 4)
    h = [64] * 4
    ctx.set_codebooks(C, h)
    cfg = EncodeConfig(H_beam=4, icm_iters=1, want_coeffs=True)
    codes, a, cost, _ = ctx.encode(X, cfg)
    got_c = np.zeros_like(codes)
    got_a = np.zeros_like(a)
    got_s = np.zeros_like(cost)
    seen = []

    def fill(first, count, out):
        out[:] = X[first:first + count]

    def sink(first, count, res):
        seen.append(first)
        got_c[first:first + count] = res["codes"]
        got_a[first:first + count] = res["a"]
        got_s[first:first + count] = res["cost"]

    st = ctx.encode_stream(X.shape[0], chunk, cfg, fill, sink)
    assert seen == sorted(seen) and len(seen) == -(-5000 // chunk)
    assert st.chunks == len(seen)
    assert np.array_equal(codes, got_c)
    assert np.array_equal(_bits(a), _bits(got_a))
    assert np.array_equal(_bits(cost), _bits(got_s))


def test_errors_are_reported(ctx):
    from stlq_amd._lib import StlqError

    X, C = random_problem(60, 10, 8, [4, 4])
    ctx.set_codebooks(C, [4, 4])
    with pytest.raises(StlqError, match="H_beam"):
        ctx.beam_search(np.zeros((10, 8), np.float32), 65, nx2=np.ones(10, np.float32))
    with pytest.raises(StlqError, match="ils_iters"):
        ctx.encode(X, EncodeConfig(H_beam=2, icm_iters=0, ils_iters=-1))
    with pytest.raises(StlqError):
        ctx.set_codebooks(np.zeros((300, 8), np.float32), [300])


LARGE_ROOT_CASES = [
    # name, seed, n, d, h0, small layers, H_beam, mode ("forced" | "nearest" | "topH")
    ("lr_topH_small", 70, 600, 24, 300, [64, 64, 64], 8, "topH"),
    ("lr_nearest", 71, 600, 32, 1000, [128, 128, 128, 128], 16, "nearest"),
    ("lr_forced", 72, 600, 32, 1000, [256, 256, 256], 32, "forced"),
    ("lr_c5_shape", 73, 300, 128, 4096, [256] * 6, 32, "nearest"),
    ("lr_m1", 74, 400, 16, 500, [], 4, "topH"),
    ("lr_m20", 75, 200, 32, 700, [64] * 19, 16, "nearest"),
]


@pytest.mark.parametrize("name,seed,n,d,h0,small,Hb,mode", LARGE_ROOT_CASES, ids=[c[0] for c in LARGE_ROOT_CASES])
def test_large_root_bit_exact(ctx, orc, name, seed, n, d, h0, small, Hb, mode):
    """BeamSearchPrefixLSLargeRoot (beam_search.cpp:579-992): root candidates from the MFMA score
    GEMM (or a forced root), expansion with reciprocal-scaled solves; cluster ids, small codes
    and selected errors are identical to the oracle's."""
    from stlq_amd import workloads

    mix = workloads.Mixture("desc" if d >= 32 else "gauss", d, 256, seed)
    rng = np.random.default_rng(seed)
    C0 = mix.sample(5_000_000, h0)
    Xtr = mix.sample(1_000_000, 3000)
    Cs = workloads.residual_codebooks(Xtr - C0[rng.integers(0, h0, 3000)], len(small), small[0], 3, seed + 1) \
        if small else np.zeros((0, d), np.float32)
    X = mix.sample(0, n)
    h = [h0] + small
    ctx.set_large_root(C0, Cs, h)
    forced = rng.integers(0, h0, n).astype(np.uint32) if mode == "forced" else None
    root_mode = 1 if mode == "nearest" else 0
    cid_g, Bs_g, err_g = ctx.beam_search_large_root(X, Hb, forced_root=forced, root_mode=root_mode)
    norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs if small else np.zeros((1, d), np.float32))
    nx2 = orc.xnorm2(X)
    xs = orc.gemm_xc(Cs, X, mode=1) if small else np.zeros((n, 1), np.float32)
    cid_o, Bs_o, err_o = orc.beam_search_large_root(X, nx2, C0, norm0, xs, Gs, G0S, h, Hb, forced_root=forced,
                                                    root_mode=root_mode)
    assert np.array_equal(cid_o, cid_g), (name, np.nonzero(cid_o != cid_g)[0][:10])
    assert np.array_equal(Bs_o, Bs_g)
    assert np.array_equal(_bits(err_o), _bits(err_g))
    if mode == "forced":
        assert np.array_equal(cid_g, forced)


@pytest.mark.parametrize("case", ["plain", "dup_small", "nan_small"])
def test_large_root_best_first_equals_reference_order(ctx, orc, monkeypatch, case):
    """The large-root expansion's best-first pass (one root slot per vector, nearest or forced;
    full small layers) plus the re-seeded reference-order re-run of the vectors it flags returns
    the reference order's cluster ids, small codes and errors bit for bit, and the oracle's.
    dup_small: duplicate small codewords within and across layers (boundary ties, re-runs);
    nan_small: a small codeword with a NaN entry (NaN candidate errors, re-runs)."""
    from stlq_amd import workloads

    seed, d, h0, K, ms, Hb, n = 76, 64, 512, 256, 5, 32, 1500
    mix = workloads.Mixture("desc", d, 256, seed)
    rng = np.random.default_rng(seed)
    C0 = mix.sample(5_000_000, h0)
    Xtr = mix.sample(1_000_000, 3000)
    Cs = workloads.residual_codebooks(Xtr - C0[rng.integers(0, h0, 3000)], ms, K, 3, seed + 1)
    X = mix.sample(0, n)
    if case == "dup_small":
        Cs[5] = Cs[9]
        Cs[K + 17] = Cs[K + 3]
        Cs[2 * K + 100] = Cs[3 * K + 7]
    elif case == "nan_small":
        Cs[2 * K + 7, 1] = np.nan
    h = [h0] + [K] * ms
    ctx.set_large_root(C0, Cs, h)
    norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs)
    nx2 = orc.xnorm2(X)
    xs = orc.gemm_xc(Cs, X, mode=1)
    for mode in ("nearest", "forced"):
        forced = rng.integers(0, h0, n).astype(np.uint32) if mode == "forced" else None
        rm = 1 if mode == "nearest" else 0
        monkeypatch.delenv("STLQ_MI355_BEAM_ORDER", raising=False)
        cid_b, Bs_b, err_b = ctx.beam_search_large_root(X, Hb, forced_root=forced, root_mode=rm)
        reruns = ctx.last_timings().beam_reruns
        monkeypatch.setenv("STLQ_MI355_BEAM_ORDER", "reference")
        cid_r, Bs_r, err_r = ctx.beam_search_large_root(X, Hb, forced_root=forced, root_mode=rm)
        assert ctx.last_timings().beam_reruns == 0
        monkeypatch.delenv("STLQ_MI355_BEAM_ORDER")
        print(f"{case}/{mode}: {reruns} of {n} vectors re-run", flush=True)
        assert np.array_equal(cid_b, cid_r), (case, mode)
        assert np.array_equal(Bs_b, Bs_r), (case, mode, np.nonzero(np.any(Bs_b != Bs_r, axis=1))[0][:10])
        same = (_bits(err_b) == _bits(err_r)) | (np.isnan(err_b) & np.isnan(err_r))
        assert np.all(same), (case, mode)
        cid_o, Bs_o, err_o = orc.beam_search_large_root(X, nx2, C0, norm0, xs, Gs, G0S, h, Hb, forced_root=forced,
                                                        root_mode=rm)
        assert np.array_equal(cid_o, cid_b) and np.array_equal(Bs_o, Bs_b), (case, mode)
        if case == "plain":
            assert reruns <= 0.02 * n, (mode, reruns)
        else:
            assert reruns > 0, (case, mode)


def _crafted_roots(variant, seed=90, n=500, d=32, h0=300, K=16, m=4):
    """Root codebooks built to hit the root scan's corner cases (beam_search.cpp:686-705):
    ties: exact duplicate roots (adjacent and far apart; the lower code must win), zero roots
    (skipped) and a root that the first 40 vectors are orthogonal to (gamma = 0 exactly: the
    quotient's range check sends the column to IEEE division);
    scaled: roots scaled by 2^40 and 2^-40 (alpha outside [2^-60, 2^60]: the IEEE division path)
    and by 2^64 (alpha overflows to +inf: a0 = 0, error ||x||^2);
    nan: a root with an infinite entry (alpha = +inf, gamma infinite or NaN, a NaN error that
    enters the scan and is then replaced or stays, per the slot rule)."""
    from stlq_amd import workloads

    mix = workloads.Mixture("desc", d, 128, seed)
    rng = np.random.default_rng(seed)
    C0 = mix.sample(5_000_000, h0)
    Xtr = mix.sample(1_000_000, 2000)
    Cs = workloads.residual_codebooks(Xtr - C0[rng.integers(0, h0, 2000)], m - 1, K, 3, seed + 1)
    X = mix.sample(0, n)
    if variant == "ties":
        for dst in (11, 50, 120, 299):
            C0[dst] = C0[10]
        C0[[5, 77, 200]] = 0.0
        C0[3] = 0.0
        C0[3, 0] = 1.5
        X[:40, 0] = 0.0
        # make the duplicated root the nearest one for some vectors
        X[40:80] = C0[10] + 0.01 * X[40:80]
    elif variant == "scaled":
        C0[30] *= np.float32(2.0 ** 40)
        C0[31] *= np.float32(2.0 ** -40)
        C0[32] *= np.float32(2.0 ** 64)
        X[:30] = C0[31] * np.float32(2.0 ** 40) + 0.01 * X[:30]  # near the tiny root's direction
    else:
        C0[250, 0] = np.inf
        X[:20, 0] = 0.0  # 0 * inf: a NaN gamma
    return X.astype(np.float32), C0.astype(np.float32), Cs, [h0] + [K] * (m - 1)


@pytest.mark.parametrize("variant", ["ties", "scaled", "nan"])
@pytest.mark.parametrize("root_mode", [1, 0], ids=["nearest", "topH"])
def test_large_root_crafted_roots(ctx, orc, variant, root_mode):
    """Device root scans (the nearest-root GEMM with its NaN fixup, and the top-H seed) on
    crafted root codebooks equal the oracle's cluster ids, small codes and errors bit for bit."""
    X, C0, Cs, h = _crafted_roots(variant)
    Hb = 4
    print(f"crafted roots {variant} root_mode={root_mode} n={X.shape[0]} h={h} beam={Hb}", flush=True)
    ctx.set_large_root(C0, Cs, h)
    cid_g, Bs_g, err_g = ctx.beam_search_large_root(X, Hb, root_mode=root_mode)
    with np.errstate(all="ignore"):
        norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs)
    nx2 = orc.xnorm2(X)
    xs = orc.gemm_xc(Cs, X, mode=1)
    cid_o, Bs_o, err_o = orc.beam_search_large_root(X, nx2, C0, norm0, xs, Gs, G0S, h, Hb, root_mode=root_mode)
    assert np.array_equal(cid_o, cid_g), (variant, np.nonzero(cid_o != cid_g)[0][:10])
    assert np.array_equal(Bs_o, Bs_g)
    # IEEE 754 leaves the sign and payload of a generated NaN to the platform (x86 SSE: 0xFFC00000,
    # CDNA: 0x7FC00000), so NaN errors match as NaN; every other error bit for bit.
    nan_o, nan_g = np.isnan(err_o), np.isnan(err_g)
    assert np.array_equal(nan_o, nan_g)
    assert np.array_equal(_bits(err_o)[~nan_o], _bits(err_g)[~nan_g])
    if variant == "ties":
        assert not np.isin(cid_g, [5, 77, 200]).any()  # zero roots never enter
        if root_mode == 1:  # one slot: a later duplicate never displaces the first
            assert not np.isin(cid_g, [11, 50, 120, 299]).any() and np.any(cid_g == 10)
    if variant == "nan" and root_mode == 1:
        assert np.all(cid_g > 250)  # the NaN entered at 250 and the next root replaced it


@pytest.mark.parametrize("chunk", [700, 2500])
def test_stream_large_root_u8_matches_in_memory(ctx, chunk):
    """Streaming large-root encode of uint8 chunks (EncodeBaseStreaming's u8 path) equals the
    in-memory large-root beam on the widened vectors."""
    from stlq_amd import workloads

    mix = workloads.Mixture("desc", 64, 128, 81)
    X = mix.sample(0, 4000)
    Xu8 = X.astype(np.uint8)
    rng = np.random.default_rng(5)
    C0 = mix.sample(5_000_000, 2048)
    Cs = workloads.residual_codebooks(mix.sample(1_000_000, 3000) - C0[rng.integers(0, 2048, 3000)], 5, 256, 3, 7)
    h = [2048] + [256] * 5
    ctx.set_large_root(C0, Cs, h)
    cid, Bs, err = ctx.beam_search_large_root(Xu8.astype(np.float32), 8, root_mode=1)
    got = {"cluster_id": np.zeros_like(cid), "B_small": np.zeros_like(Bs), "best_err": np.zeros_like(err)}

    def fill(first, count, out):
        out[:] = Xu8[first:first + count]

    def sink(first, count, res):
        for k in got:
            got[k][first:first + count] = res[k]

    st = ctx.encode_stream(4000, chunk, EncodeConfig(H_beam=8, icm_iters=0), fill, sink, input_u8=True,
                           large_root=True, root_mode=1)
    assert st.chunks == -(-4000 // chunk) and st.h2d_bytes == 4000 * 64
    assert np.array_equal(got["cluster_id"], cid)
    assert np.array_equal(got["B_small"], Bs)
    assert np.array_equal(_bits(got["best_err"]), _bits(err))


def test_stream_chunk_larger_than_workspace(ctx, monkeypatch):
    """A streamed chunk bigger than the workspace budget is encoded in tiles, with identical results."""
    from stlq_amd import workloads

    mix = workloads.Mixture("desc", 32, 64, 91)
    X = mix.sample(0, 6000)
    C = workloads.residual_codebooks(mix.sample(1_000_000, 2000), 4, 64, 3, 4)
    ctx.set_codebooks(C, [64] * 4)
    cfg = EncodeConfig(H_beam=4, icm_iters=1, want_coeffs=True)
    codes, a, cost, _ = ctx.encode(X, cfg)
    monkeypatch.setenv("STLQ_MI355_WORKSPACE_GB", "0.0005")
    got = np.zeros_like(codes)

    def fill(first, count, out):
        out[:] = X[first:first + count]

    def sink(first, count, res):
        got[first:first + count] = res["codes"]

    ctx.encode_stream(6000, 6000, cfg, fill, sink)
    assert np.array_equal(codes, got)


def _lr_refit_problem(ctx, orc, m, seed, n=2000, d=32, h0=1500, K=64):
    from tests.helpers import large_root_problem

    p = large_root_problem(orc, seed, n, d, h0, K, m, H_beam=4, root_mode=1, kind="desc" if d >= 32 else "gauss")
    ctx.set_large_root(p["C0"], p["Cs"], p["h"])
    return p


@pytest.mark.parametrize("m", [2, 5, 8, 11, 17, 20])
def test_large_root_ls_costs_bit_exact(ctx, orc, m):
    """SolveLeastSquaresAllLargeRoot + ComputeCostsLargeRoot on the device: b0 = <C0[:,root], x> in
    the omp-simd order, the root row of the system from norm0/G0S, the reference's cost order."""
    p = _lr_refit_problem(ctx, orc, m, 300 + m)
    print(f"lr refit m={m} n={p['X'].shape[0]}", flush=True)
    a_o, _ = orc.solve_ls_all_large_root(p["X"], p["C0"], p["norm0"], p["xs"], p["Gs"], p["G0S"], p["h"], p["cid"],
                                         p["Bs"])
    c_o = orc.compute_costs_large_root(p["X"], p["C0"], p["norm0"], p["xs"], p["Gs"], p["G0S"], p["h"], p["cid"],
                                       p["Bs"], a_o, p["nx2"])
    for xs in (p["xs"], None):  # given xC_small, or the device GEMM (same fused order as the oracle's mode 1)
        a_g, fails = ctx.solve_ls_all_large_root(p["X"], p["cid"], p["Bs"], xC_small=xs)
        assert fails == 0
        assert np.array_equal(_bits(a_g), _bits(a_o))
        c_g = ctx.compute_costs_large_root(p["X"], p["cid"], p["Bs"], a_o, xC_small=xs)
        assert np.array_equal(_bits(c_g), _bits(c_o))


@pytest.mark.parametrize("m,icm,ils,pk,off,use_abs", [(5, 2, 0, 3, 0, True), (5, 1, 3, 2, 777, False),
                                                      (8, 2, 2, 3, 10_000, True), (3, 0, 3, 3, 5, True),
                                                      (17, 1, 1, 3, 0, True), (20, 2, 0, 2, 0, False)])
def test_large_root_icm_ils_bit_exact(ctx, orc, m, icm, ils, pk, off, use_abs):
    """DynamicIcmWithIls*NoNormalLargeRoot on the device: roots fixed, ICM over layers 1..m-1
    with the root's G0S row, ILS rounds keyed by the global id; codes, a and cost identical."""
    p = _lr_refit_problem(ctx, orc, m, 400 + m + icm + ils)
    print(f"lr icm m={m} icm={icm} ils={ils} pk={pk} off={off} abs={use_abs}", flush=True)
    B_o, a_o, c_o, _ = orc.icm_ils_large_root(p["X"], p["C0"], p["norm0"], p["xs"], p["Gs"], p["G0S"], p["invs"],
                                              p["h"], p["cid"], p["nx2"], p["Bs"], icm, ils, pk, use_abs, 38251450,
                                              off)
    B_g, a_g, c_g = ctx.icm_ils_large_root(p["X"], p["cid"], p["Bs"], icm, ils, pk, use_abs, 38251450,
                                           sample_id_offset=off)
    if icm > 0:
        assert np.any(B_o != p["Bs"])
    assert np.array_equal(B_g, B_o), np.nonzero(np.any(B_g != B_o, axis=1))[0][:10]
    assert np.array_equal(_bits(a_g), _bits(a_o))
    assert np.array_equal(_bits(c_g), _bits(c_o))


@pytest.mark.parametrize("icm,ils", [(0, 0), (1, 2)])
def test_stream_large_root_refit(ctx, orc, icm, ils):
    """The large-root streaming encode with the refit (encode_base_streaming.cpp:1117-1210): per
    chunk cluster ids and codes of the beam, then LS/ICM/ILS with sample_id_offset = the chunk's
    global start; equal to the in-memory beam followed by the oracle's refit over all vectors."""
    m, n, chunk = 6, 5000, 1700
    p = _lr_refit_problem(ctx, orc, m, 500 + icm, n=n, d=64, h0=2048, K=128)
    Xu8 = np.clip(np.rint(p["X"]), 0, 255).astype(np.uint8)
    Xf = Xu8.astype(np.float32)
    cid, Bs, _ = ctx.beam_search_large_root(Xf, 8, root_mode=1)
    nx2 = orc.xnorm2(Xf)
    xs = orc.gemm_xc(p["Cs"], Xf, mode=1)
    B_o, a_o, c_o, _ = orc.icm_ils_large_root(Xf, p["C0"], p["norm0"], xs, p["Gs"], p["G0S"], p["invs"], p["h"], cid,
                                              nx2, Bs, icm, ils, 3, True, 38251450, 0)
    got = {"cluster_id": np.zeros_like(cid), "B_small": np.zeros_like(Bs), "a": np.zeros_like(a_o),
           "cost": np.zeros_like(c_o)}

    def fill(first, count, out):
        out[:] = Xu8[first:first + count]

    def sink(first, count, res):
        for k in got:
            got[k][first:first + count] = res[k]

    cfg = EncodeConfig(H_beam=8, icm_iters=icm, ils_iters=ils, perturb_k=3, want_coeffs=True)
    ctx.encode_stream(n, chunk, cfg, fill, sink, input_u8=True, large_root=True, root_mode=1)
    assert np.array_equal(got["cluster_id"], cid)
    assert np.array_equal(got["B_small"], B_o)
    assert np.array_equal(_bits(got["a"]), _bits(a_o))
    assert np.array_equal(_bits(got["cost"]), _bits(c_o))


def _orthogonal(d, seed):
    q, r = np.linalg.qr(np.random.default_rng(seed).standard_normal((d, d)))
    return (q * np.sign(np.diag(r))).astype(np.float32)


@pytest.mark.parametrize("d", [96, 100, 128])
def test_convert_u8_rotate(ctx, orc, d):
    """ConvertU8ToF32AndRotatePtr (kernel_provider.h:44-52): widening is exact; R X on the MFMA
    GEMM equals the oracle's fused k-ascending product bit for bit (the reference's BLAS order is
    unpinned); R = I returns the widened input unchanged; a column stride ld_in > d is honoured."""
    import ctypes

    from stlq_amd import _lib

    rng = np.random.default_rng(d)
    Xu8 = rng.integers(0, 256, (3001, d), dtype=np.uint8)
    Xf = Xu8.astype(np.float32)
    assert np.array_equal(_bits(ctx.convert_u8_rotate(Xu8)), _bits(Xf))
    assert np.array_equal(_bits(ctx.convert_u8_rotate(Xu8, np.eye(d, dtype=np.float32))), _bits(Xf))
    R = _orthogonal(d, d + 1)
    got = ctx.convert_u8_rotate(Xu8, R)
    assert np.array_equal(_bits(got), _bits(orc.gemm_xc(R, Xf, mode=1)))
    ld = d + 7
    padded = np.zeros((Xu8.shape[0], ld), np.uint8)
    padded[:, :d] = Xu8
    out = np.empty_like(Xf)
    Rc = np.ascontiguousarray(R.T)
    _lib.check(ctx.lib.stlq_mi355_convert_u8_rotate(ctx.h, padded.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), ld, d,
                                                    Xu8.shape[0], Rc.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                                    out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
    assert np.array_equal(_bits(out), _bits(got))


def test_stream_rotation_full_precomp(ctx, orc):
    """EncodeBaseStreamingF32 with a rotation (encode_base_streaming.cpp:1367-1390): every chunk is
    rotated on the device before the encode; identical to the in-memory encode of the oracle-
    rotated vectors. R = I gives the unrotated stream's results."""
    X, C = rvq_problem(95, 5000, 64, 4, 64, kind="desc", train_n=2000, iters=3)
    h = [64] * 4
    ctx.set_codebooks(C, h)
    R = _orthogonal(64, 7)
    cfg = EncodeConfig(H_beam=4, icm_iters=1, ils_iters=1, want_coeffs=True)
    Xr = orc.gemm_xc(R, X, mode=1)
    codes, a, cost, _ = ctx.encode(Xr, cfg)

    def run(Rm):
        got = {"codes": np.zeros_like(codes), "a": np.zeros_like(a), "cost": np.zeros_like(cost)}

        def fill(first, count, out):
            out[:] = X[first:first + count]

        def sink(first, count, res):
            for k in got:
                got[k][first:first + count] = res[k]

        ctx.encode_stream(X.shape[0], 1800, cfg, fill, sink, R=Rm)
        return got

    g = run(R)
    assert np.array_equal(g["codes"], codes)
    assert np.array_equal(_bits(g["a"]), _bits(a))
    assert np.array_equal(_bits(g["cost"]), _bits(cost))
    g_id, g_none = run(np.eye(64, dtype=np.float32)), run(None)
    for k in g_id:  # byte-for-byte equal
        assert np.array_equal(np.ascontiguousarray(g_id[k]).view(np.uint8), np.ascontiguousarray(g_none[k]).view(np.uint8))


def test_stream_rotation_large_root_u8(ctx, orc):
    """EncodeBaseStreaming's uint8 path with a rotation (encode_base_streaming.cpp:817-833): widen,
    rotate, large-root beam and refit; identical to the in-memory large-root encode of the
    oracle-rotated vectors."""
    m, n = 5, 3000
    p = _lr_refit_problem(ctx, orc, m, 611, n=n, d=64, h0=1024, K=64)
    Xu8 = np.clip(np.rint(p["X"]), 0, 255).astype(np.uint8)
    R = _orthogonal(64, 11)
    Xr = orc.gemm_xc(R, Xu8.astype(np.float32), mode=1)
    cid, Bs, err = ctx.beam_search_large_root(Xr, 8, root_mode=1)
    B_g, a_g, c_g = ctx.icm_ils_large_root(Xr, cid, Bs, 0, 0, 3, True, 38251450)
    got = {"cluster_id": np.zeros_like(cid), "B_small": np.zeros_like(Bs), "best_err": np.zeros_like(err),
           "a": np.zeros_like(a_g), "cost": np.zeros_like(c_g)}

    def fill(first, count, out):
        out[:] = Xu8[first:first + count]

    def sink(first, count, res):
        for k in got:
            got[k][first:first + count] = res[k]

    cfg = EncodeConfig(H_beam=8, icm_iters=0, want_coeffs=True)
    ctx.encode_stream(n, 1100, cfg, fill, sink, input_u8=True, large_root=True, root_mode=1, R=R)
    assert np.array_equal(got["cluster_id"], cid)
    assert np.array_equal(got["B_small"], B_g)
    assert np.array_equal(_bits(got["best_err"]), _bits(err))
    assert np.array_equal(_bits(got["a"]), _bits(a_g))
    assert np.array_equal(_bits(got["cost"]), _bits(c_g))


@pytest.mark.parametrize("nan_roots", [0, 3])
def test_large_root_nearest_nan_roots(ctx, orc, nan_roots):
    """Nearest-root mode with root codewords that give NaN errors for every vector: the fused
    first-minimum GEMM flags those vectors and the exact scan redoes them (a NaN enters the
    one-slot scan and the next candidate replaces it), matching the oracle's streaming scan."""
    from stlq_amd import workloads

    n, d, h0, K = 700, 32, 700, 64
    mix = workloads.Mixture("gauss", d, 128, 97)
    rng = np.random.default_rng(97)
    C0 = mix.sample(5_000_000, h0)
    Cs = workloads.residual_codebooks(mix.sample(1_000_000, 2000) - C0[rng.integers(0, h0, 2000)], 3, K, 3, 98)
    for r in rng.choice(h0, nan_roots, replace=False):
        C0[r, 5] = np.nan
    X = mix.sample(0, n)
    h = [h0] + [K] * 3
    print(f"lr nearest nan_roots={nan_roots} n={n} h0={h0}", flush=True)
    ctx.set_large_root(C0, Cs, h)
    cid_g, Bs_g, err_g = ctx.beam_search_large_root(X, 8, root_mode=1)
    norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs)
    nx2 = orc.xnorm2(X)
    xs = orc.gemm_xc(Cs, X, mode=1)
    cid_o, Bs_o, err_o = orc.beam_search_large_root(X, nx2, C0, norm0, xs, Gs, G0S, h, 8, root_mode=1)
    assert np.array_equal(cid_o, cid_g), np.nonzero(cid_o != cid_g)[0][:10]
    assert np.array_equal(Bs_o, Bs_g)
    same = (_bits(err_o) == _bits(err_g)) | (np.isnan(err_o) & np.isnan(err_g))
    assert np.all(same)


@pytest.mark.parametrize("large_root", [False, True])
def test_stream_resume_start_id(ctx, orc, large_root):
    """EncodeBaseStreaming from a start_id (encode_base_streaming.cpp:1913-1936, :874): two resumed
    half-streams (the second at start_id = n/2) give exactly the whole stream's codes, coefficients
    and costs, with ILS perturbations keyed by the global id, and both equal the oracle with
    sample_id_offset 0 over all n; fill and sink see global ids."""
    n, half, chunk = 4000, 2000, 700
    cfg = EncodeConfig(H_beam=4, icm_iters=1, ils_iters=3, perturb_k=3, want_coeffs=True)
    print(f"stream resume large_root={large_root}", flush=True)
    if large_root:
        p = _lr_refit_problem(ctx, orc, 5, 811, n=n, d=64, h0=1024, K=64)
        X = p["X"]
        cid, Bs, _ = ctx.beam_search_large_root(X, 4, root_mode=1)
        nx2 = orc.xnorm2(X)
        xs = orc.gemm_xc(p["Cs"], X, mode=1)
        B_o, a_o, c_o, _ = orc.icm_ils_large_root(X, p["C0"], p["norm0"], xs, p["Gs"], p["G0S"], p["invs"], p["h"],
                                                  cid, nx2, Bs, 1, 3, 3, True, 38251450, 0)
        want = {"cluster_id": cid, "B_small": B_o, "a": a_o, "cost": c_o}
        kw = dict(large_root=True, root_mode=1)
    else:
        X, C = rvq_problem(812, n, 32, 5, 64, train_n=2000, iters=3)
        h = [64] * 5
        ctx.set_codebooks(C, h)
        codes_o, a_o, cost_o = _oracle_encode(orc, X, C, h, 4, icm_iters=1, ils_iters=3, perturb_k=3)
        want = {"codes": codes_o, "a": a_o, "cost": cost_o}
        kw = {}

    def run(start, count):
        got = {k: np.zeros((count,) + v.shape[1:], v.dtype) for k, v in want.items()}
        seen = []

        def fill(first, cnt, out):
            assert start <= first and first + cnt <= start + count
            out[:] = X[first:first + cnt]

        def sink(first, cnt, res):
            seen.append(first)
            for k in got:
                got[k][first - start:first - start + cnt] = res[k]

        ctx.encode_stream(count, chunk, cfg, fill, sink, start_id=start, **kw)
        assert seen[0] == start and seen == sorted(seen)
        return got

    whole = run(0, n)
    first, second = run(0, half), run(half, n - half)
    for k in want:
        joined = np.concatenate([first[k], second[k]])
        assert np.array_equal(np.ascontiguousarray(joined).view(np.uint8),
                              np.ascontiguousarray(whole[k]).view(np.uint8)), k
        assert np.array_equal(np.ascontiguousarray(whole[k]).view(np.uint8),
                              np.ascontiguousarray(want[k]).view(np.uint8)), k


def test_stream_large_root_c5_shape(ctx, orc):
    """The C5 workload's shape on a 2,048-vector sample: uint8 descriptor-like vectors streamed in
    chunks, nearest of h0 = 65,536 root codewords (the fused root GEMM sweeps all 512 root tiles),
    16 residual codebooks of 256 (layers 1..16, the deep large-root kernels), beam 32, then the
    large-root LS refit and costs (encode_base_streaming.cpp:1117-1210). Cluster ids, B_small,
    coefficients and costs are identical to the oracle's."""
    from stlq_amd import workloads

    w = workloads.CONFIGS["C5"]
    n, h0, msmall, K, Hb = 2048, 65536, 16, 256, 32
    mix = workloads.Mixture(w.kind, w.d, w.n_comp, w.seed)
    C0 = mix.sample(20_000_000, h0)
    Xtr = mix.sample(10_000_000, 4000)
    lab = np.argmax(2.0 * (Xtr @ C0.T) - np.sum(C0 * C0, axis=1)[None, :], axis=1)
    Cs = workloads.residual_codebooks(Xtr - C0[lab], msmall, K, 2, w.seed + 77)
    Xu8 = mix.sample(0, n).astype(np.uint8)  # clipped, rounded to [0, 255]: exact as uint8
    Xf = Xu8.astype(np.float32)
    h = [h0] + [K] * msmall
    print(f"c5 shape: n={n} h0={h0} small={msmall}x{K} beam={Hb}", flush=True)
    ctx.set_large_root(C0, Cs, h)
    got = {"cluster_id": np.zeros(n, np.uint32), "B_small": np.zeros((n, msmall), np.uint8),
           "a": np.zeros((n, msmall + 1), np.float32), "cost": np.zeros(n, np.float32)}

    def fill(first, count, out):
        out[:] = Xu8[first:first + count]

    def sink(first, count, res):
        for k in got:
            got[k][first:first + count] = res[k]

    cfg = EncodeConfig(H_beam=Hb, icm_iters=0, want_coeffs=True)
    ctx.encode_stream(n, 700, cfg, fill, sink, input_u8=True, large_root=True, root_mode=1)
    print("c5 shape: device stream done", flush=True)
    norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs)
    invs = orc.invnorm_small(Cs)
    nx2 = orc.xnorm2(Xf)
    xs = orc.gemm_xc(Cs, Xf, mode=1)
    cid, Bs, _ = orc.beam_search_large_root(Xf, nx2, C0, norm0, xs, Gs, G0S, h, Hb, root_mode=1)
    B_o, a_o, c_o, _ = orc.icm_ils_large_root(Xf, C0, norm0, xs, Gs, G0S, invs, h, cid, nx2, Bs, 0, 0, 3, True,
                                              38251450, 0)
    assert np.array_equal(got["cluster_id"], cid), np.nonzero(got["cluster_id"] != cid)[0][:10]
    assert np.array_equal(got["B_small"], B_o), np.nonzero(np.any(got["B_small"] != B_o, axis=1))[0][:10]
    assert np.array_equal(_bits(got["a"]), _bits(a_o))
    assert np.array_equal(_bits(got["cost"]), _bits(c_o))
