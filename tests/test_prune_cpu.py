"""The beam's candidate pruning (stlq_amd/csrc/prune_bound.hpp) rejects only candidates the
reference rejects (src/quantizer/beam_search.cpp:320): tests/prune_check.cpp replays the reference
beam in its slot order with the device's pruning constants and test (the product header, built
with hipcc as host code) on samples of the benchmark workloads and on ill-conditioned codebooks,
and requires
  * no pruned candidate the reference would have inserted,
  * every candidate kept when the threshold is its own error (a strict lower bound),
  * the beam that skips the pruned candidates equal to the full beam, codes and errors bit for bit,
  * on the benchmark samples, most candidates pruned (the bound is tight enough to matter),
  * the last layer's minimum rule (LastPick in beam_kernels.hpp: parents in ascending error order, each
    candidate bound-tested against the running minimum, only the minimum kept) picking the
    reference's codes and error bit for bit on every vector it does not flag for a re-run."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from stlq_amd import workloads
from tests.helpers import rvq_problem

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("prune") / "libprune_check.so")
    cmd = ["/opt/rocm/bin/hipcc", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
           f"-I{os.path.join(ROOT, 'stlq_amd', 'csrc')}", os.path.join(HERE, "prune_check.cpp"), "-o", out]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    lib = ctypes.CDLL(out)
    f32p = ctypes.POINTER(ctypes.c_float)
    lib.prune_check.argtypes = [f32p, f32p, f32p, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                ctypes.c_int64, ctypes.c_int, ctypes.POINTER(ctypes.c_int64)]
    return lib


def _run(checker, orc, X, C, h, Hb):
    G, _ = orc.build_precomp(C, h)
    xC = np.ascontiguousarray(orc.gemm_xc(C, X))
    nx2 = np.ascontiguousarray(orc.xnorm2(X))
    hv = (ctypes.c_int * len(h))(*h)
    st = (ctypes.c_int64 * 12)()
    f32p = ctypes.POINTER(ctypes.c_float)
    G = np.ascontiguousarray(G)
    assert checker.prune_check(G.ctypes.data_as(f32p), xC.ctypes.data_as(f32p), nx2.ctypes.data_as(f32p),
                               int(sum(h)), len(h), hv, X.shape[0], Hb, st) == 0
    keys = ["candidates", "tested", "pruned", "violations", "self_kept_fail", "mismatches", "lp_decided",
            "lp_flagged", "lp_mismatches", "lp_candidates", "lp_pruned", "last_pruned_worst"]
    rep = dict(zip(keys, list(st)))
    # the minimum rule decides or flags every vector, and never disagrees with the reference
    assert rep["lp_decided"] + rep["lp_flagged"] == X.shape[0], rep
    assert rep["lp_mismatches"] == 0, rep
    return rep


@pytest.mark.parametrize("cfg,n,Hb", [("C2", 400, 16), ("C4", 60, 8), ("C3", 300, 16)])
def test_pruning_never_drops_an_entrant(checker, orc, cfg, n, Hb):
    w = workloads.CONFIGS[cfg]
    mix = workloads.Mixture(w.kind, w.d, w.n_comp, w.seed)
    Xtr = mix.sample(10_000_000, 3000 if w.d < 900 else 1500)
    C = workloads.residual_codebooks(Xtr, w.m, w.K, 3, w.seed + 5, spherical=(w.kind == "sphere"))
    X = mix.sample(0, n)
    rep = _run(checker, orc, X, C, [w.K] * w.m, Hb)
    print(cfg, rep)
    assert rep["violations"] == 0 and rep["self_kept_fail"] == 0 and rep["mismatches"] == 0, rep
    assert rep["pruned"] >= 0.75 * rep["candidates"], rep  # tight enough to matter (reference scan order)
    # the minimum rule decides most vectors (C4's deep near-zero codewords leave ties for the
    # minimum, which the best-first pass flags in any case) and prunes more of the last layer than
    # the top-H bound does
    assert rep["lp_flagged"] <= 0.2 * n, rep
    assert rep["lp_pruned"] > rep["last_pruned_worst"], rep


@pytest.mark.parametrize("kind", ["near_dependent", "scaled", "tiny"])
def test_pruning_safe_on_ill_conditioned_codebooks(checker, orc, kind):
    """Codebooks whose prefixes are nearly linearly dependent (Cholesky pivots near zero), span
    many orders of magnitude, or are tiny: the constants grow or leave their ranges, pruning backs
    off, and nothing the reference inserts is ever skipped."""
    rng = np.random.default_rng(7)
    X, C = rvq_problem(77, 200, 16, 5, 32, train_n=1500, iters=3)
    if kind == "near_dependent":
        C[32:64] = C[0:32] * 1.0001 + 1e-4 * rng.standard_normal((32, 16)).astype(np.float32)
        C[96:128] = C[64:96] + 1e-3 * rng.standard_normal((32, 16)).astype(np.float32)
    elif kind == "scaled":
        C[32:64] *= 1e4
        C[64:96] *= 1e-4
    else:
        C *= 1e-12
        X *= 1e-12
    rep = _run(checker, orc, X, C, [32] * 5, 8)
    print(kind, rep)
    assert rep["violations"] == 0 and rep["self_kept_fail"] == 0 and rep["mismatches"] == 0, rep


def test_pruning_deep_layers_beam32(checker, orc):
    """A 17-layer, beam-32 encode of d=128 descriptors (the depth and width of the large-root
    stream): past layer 10 the prefix codewords are far from orthogonal and the Frobenius bound
    kap ||b||^2 alone prunes almost nothing; with the diagonal split most candidates are still
    pruned, and none that the reference would insert."""
    w = workloads.CONFIGS["C2"]
    mix = workloads.Mixture(w.kind, w.d, w.n_comp, w.seed)
    C = workloads.residual_codebooks(mix.sample(10_000_000, 3000), 17, w.K, 3, w.seed + 5)
    X = mix.sample(0, 10)
    rep = _run(checker, orc, X, C, [w.K] * 17, 32)
    print(rep)
    assert rep["violations"] == 0 and rep["self_kept_fail"] == 0 and rep["mismatches"] == 0, rep
    assert rep["pruned"] >= 0.8 * rep["candidates"], rep
