"""ctypes wrapper of the CPU oracle (oracle/stlq_oracle.cpp) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, and
only as the checker (or the timed CPU baseline). The product (stlq_amd/) never imports it.

Array conventions follow the reference's column-major matrices
(include/stlq/common/types.h:35-51) viewed from numpy as C-contiguous row-major arrays:
  X      (n, d)  float32      vector i = X[i]
  C_all  (H, d)  float32      codeword f = C_all[f]
  G      (H, H)  float32      G[col, row] in numpy == reference G(row, col)
  xC     (n, H)  float32
  codes  (n, m)  uint8
  a      (n, m)  float32
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# STLQ_ORACLE_LIB selects another build of the same source (the sanitizer test loads an
# AddressSanitizer/UBSan build through it).
_LIB_PATH = os.environ.get("STLQ_ORACLE_LIB") or os.path.join(_HERE, "_build", "libstlq_oracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i64 = ctypes.c_int64
_int = ctypes.c_int


def build() -> str:
    """Compile the oracle with its Makefile (g++, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_build_precomp.argtypes = [_int, _int, _i32p, _f32p, _f32p, _f32p, _int]
        L.orc_xnorm2.argtypes = [_f32p, _int, _i64, _f32p, _int]
        L.orc_gemm_xc.argtypes = [_f32p, _int, _int, _f32p, _i64, _f32p, _int, _int]
        L.orc_beam_search.argtypes = [_f32p, _f32p, _f32p, _int, _int, _i32p, _int, _i64, _u8p, _f32p, _int]
        L.orc_solve_ls_all.argtypes = [_f32p, _f32p, _int, _int, _i32p, _u8p, _i64, _f32p, _int]
        L.orc_solve_ls_all.restype = _i64
        L.orc_compute_costs.argtypes = [_f32p, _f32p, _int, _int, _i32p, _u8p, _f32p, _f32p, _i64, _f32p, _int]
        L.orc_icm.argtypes = [_f32p, _f32p, _f32p, _int, _int, _i32p, _f32p, _i64, _int, _int,
                              ctypes.c_uint32, _u8p, _f32p, _f32p, _int]
        L.orc_icm.restype = _i64
        L.orc_icm_ils.argtypes = [_f32p, _f32p, _f32p, _int, _int, _i32p, _f32p, _i64, _int, _int, _int, _int,
                                  ctypes.c_uint32, ctypes.c_uint64, _u8p, _f32p, _f32p, _int]
        L.orc_icm_ils.restype = _i64
        L.orc_icm_orders.argtypes = [_int, _int, ctypes.c_uint32, _i32p]
        L.orc_mse_from_precomp.argtypes = [_f32p, _int, _f32p, _f32p, _int, _int, _i32p, _u8p, _f32p, _i64, _f64p, _int]
        L.orc_mse_fp64_refit.argtypes = [_f32p, _int, _f32p, _int, _int, _i32p, _u8p, _i64, _f64p, _int]
        L.orc_build_precomp_large_root.argtypes = [_int, _int, _int, _f32p, _f32p, _f32p, _f32p, _f32p, _int]
        L.orc_beam_search_large_root.argtypes = [_f32p, _int, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
                                                 _int, _int, _int, _i32p, _int, _i64, _u32p, _int,
                                                 _u32p, _u8p, _f32p, _int]
        L.orc_large_root_candidates.argtypes = [_f32p, _int, _f32p, _f32p, _f32p, _int, _int, _i64, _u32p, _int,
                                                _f32p, _i32p, _f32p, _f32p, _int]
        L.orc_invnorm_small.argtypes = [_f32p, _int, _int, _f32p]
        L.orc_solve_ls_all_large_root.argtypes = [_f32p, _int, _f32p, _f32p, _int, _f32p, _f32p, _f32p, _int, _int,
                                                  _i32p, _u32p, _u8p, _i64, _f32p, _int]
        L.orc_solve_ls_all_large_root.restype = _i64
        L.orc_compute_costs_large_root.argtypes = [_f32p, _int, _f32p, _f32p, _int, _f32p, _f32p, _f32p, _int, _int,
                                                   _i32p, _u32p, _u8p, _f32p, _f32p, _i64, _f32p, _int]
        L.orc_icm_ils_large_root.argtypes = [_f32p, _int, _f32p, _f32p, _int, _f32p, _f32p, _f32p, _f32p, _int, _int,
                                             _i32p, _u32p, _f32p, _i64, _int, _int, _int, _int, ctypes.c_uint32,
                                             ctypes.c_uint64, _u8p, _f32p, _f32p, _int]
        L.orc_icm_ils_large_root.restype = _i64
        _lib = L
    return _lib


def _p(a, t):
    return a.ctypes.data_as(t) if a is not None else None


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def build_precomp(C_all, h_vec, nthreads=0):
    C_all = _c(C_all, np.float32)
    H, d = C_all.shape
    hv = _c(h_vec, np.int32)
    G = np.empty((H, H), np.float32)
    inv = np.empty(H, np.float32)
    lib().orc_build_precomp(d, len(hv), _p(hv, _i32p), _p(C_all, _f32p), _p(G, _f32p), _p(inv, _f32p), nthreads)
    return G, inv


def xnorm2(X, nthreads=0):
    X = _c(X, np.float32)
    n, d = X.shape
    out = np.empty(n, np.float32)
    lib().orc_xnorm2(_p(X, _f32p), d, n, _p(out, _f32p), nthreads)
    return out


def gemm_xc(C_all, X, mode=0, nthreads=0):
    C_all = _c(C_all, np.float32)
    X = _c(X, np.float32)
    H, d = C_all.shape
    n = X.shape[0]
    xC = np.empty((n, H), np.float32)
    lib().orc_gemm_xc(_p(C_all, _f32p), d, H, _p(X, _f32p), n, _p(xC, _f32p), mode, nthreads)
    return xC


def beam_search(nx2, xC, G, h_vec, H_beam, nthreads=0):
    nx2 = _c(nx2, np.float32)
    xC = _c(xC, np.float32)
    G = _c(G, np.float32)
    hv = _c(h_vec, np.int32)
    n, H = xC.shape
    m = len(hv)
    codes = np.empty((n, m), np.uint8)
    err = np.empty(n, np.float32)
    lib().orc_beam_search(_p(nx2, _f32p), _p(xC, _f32p), _p(G, _f32p), H, m, _p(hv, _i32p), H_beam, n,
                          _p(codes, _u8p), _p(err, _f32p), nthreads)
    return codes, err


def solve_ls_all(xC, G, h_vec, codes, nthreads=0):
    xC = _c(xC, np.float32)
    G = _c(G, np.float32)
    hv = _c(h_vec, np.int32)
    codes = _c(codes, np.uint8)
    n, H = xC.shape
    m = len(hv)
    a = np.empty((n, m), np.float32)
    fails = lib().orc_solve_ls_all(_p(xC, _f32p), _p(G, _f32p), H, m, _p(hv, _i32p), _p(codes, _u8p), n,
                                   _p(a, _f32p), nthreads)
    return a, int(fails)


def compute_costs(xC, G, h_vec, codes, a, nx2, nthreads=0):
    xC = _c(xC, np.float32)
    G = _c(G, np.float32)
    hv = _c(h_vec, np.int32)
    codes = _c(codes, np.uint8)
    a = _c(a, np.float32)
    nx2 = _c(nx2, np.float32)
    n, H = xC.shape
    cost = np.empty(n, np.float32)
    lib().orc_compute_costs(_p(xC, _f32p), _p(G, _f32p), H, len(hv), _p(hv, _i32p), _p(codes, _u8p),
                            _p(a, _f32p), _p(nx2, _f32p), n, _p(cost, _f32p), nthreads)
    return cost


def icm(xC, G, invnorm, h_vec, nx2, codes, icm_iters, use_abs, seed, nthreads=0):
    xC = _c(xC, np.float32)
    G = _c(G, np.float32)
    inv = _c(invnorm, np.float32)
    hv = _c(h_vec, np.int32)
    nx2 = _c(nx2, np.float32)
    codes = np.array(codes, dtype=np.uint8, copy=True, order="C")
    n, H = xC.shape
    m = len(hv)
    a = np.empty((n, m), np.float32)
    cost = np.empty(n, np.float32)
    fails = lib().orc_icm(_p(xC, _f32p), _p(G, _f32p), _p(inv, _f32p), H, m, _p(hv, _i32p), _p(nx2, _f32p), n,
                          icm_iters, int(bool(use_abs)), seed & 0xFFFFFFFF, _p(codes, _u8p), _p(a, _f32p),
                          _p(cost, _f32p), nthreads)
    return codes, a, cost, int(fails)


def icm_ils(xC, G, invnorm, h_vec, nx2, codes, icm_iters, ils_iters, perturb_k, use_abs, seed,
            sample_id_offset=0, nthreads=0):
    """ICM with the ILS outer loop; returns (codes, a, cost, ls_fails)."""
    xC = _c(xC, np.float32)
    G = _c(G, np.float32)
    inv = _c(invnorm, np.float32)
    hv = _c(h_vec, np.int32)
    nx2 = _c(nx2, np.float32)
    codes = np.array(codes, dtype=np.uint8, copy=True, order="C")
    n, H = xC.shape
    m = len(hv)
    a = np.empty((n, m), np.float32)
    cost = np.empty(n, np.float32)
    fails = lib().orc_icm_ils(_p(xC, _f32p), _p(G, _f32p), _p(inv, _f32p), H, m, _p(hv, _i32p), _p(nx2, _f32p), n,
                              icm_iters, ils_iters, perturb_k, int(bool(use_abs)), seed & 0xFFFFFFFF,
                              int(sample_id_offset), _p(codes, _u8p), _p(a, _f32p), _p(cost, _f32p), nthreads)
    return codes, a, cost, int(fails)


def icm_orders(m, icm_iters, seed):
    out = np.empty((max(icm_iters, 0), m), np.int32)
    lib().orc_icm_orders(m, icm_iters, seed & 0xFFFFFFFF, _p(out, _i32p))
    return out


def mse_from_precomp(X, xC, G, h_vec, codes, a, nthreads=0):
    X = _c(X, np.float32)
    xC = _c(xC, np.float32)
    G = _c(G, np.float32)
    hv = _c(h_vec, np.int32)
    codes = _c(codes, np.uint8)
    a = _c(a, np.float32)
    n, d = X.shape
    out = np.empty(n, np.float64)
    lib().orc_mse_from_precomp(_p(X, _f32p), d, _p(xC, _f32p), _p(G, _f32p), xC.shape[1], len(hv), _p(hv, _i32p),
                               _p(codes, _u8p), _p(a, _f32p), n, _p(out, _f64p), nthreads)
    return out


def mse_fp64_refit(X, C_all, h_vec, codes, nthreads=0):
    X = _c(X, np.float32)
    C_all = _c(C_all, np.float32)
    hv = _c(h_vec, np.int32)
    codes = _c(codes, np.uint8)
    n, d = X.shape
    out = np.empty(n, np.float64)
    lib().orc_mse_fp64_refit(_p(X, _f32p), d, _p(C_all, _f32p), C_all.shape[0], len(hv), _p(hv, _i32p),
                             _p(codes, _u8p), n, _p(out, _f64p), nthreads)
    return out


def build_precomp_large_root(C0, C_small, nthreads=0):
    C0 = _c(C0, np.float32)
    C_small = _c(C_small, np.float32)
    h0, d = C0.shape
    Hs = C_small.shape[0]
    norm0 = np.empty(h0, np.float32)
    G_small = np.empty((Hs, Hs), np.float32)
    G0S = np.empty((Hs, h0), np.float32)  # numpy [flat, root] == reference G0S(root, flat)
    lib().orc_build_precomp_large_root(d, h0, Hs, _p(C0, _f32p), _p(C_small, _f32p), _p(norm0, _f32p),
                                       _p(G_small, _f32p), _p(G0S, _f32p), nthreads)
    return norm0, G_small, G0S


def beam_search_large_root(X, nx2, C0, norm0, xC_small, G_small, G0S, h_vec, H_beam,
                           forced_root=None, root_mode=0, nthreads=0):
    X = _c(X, np.float32)
    nx2 = _c(nx2, np.float32)
    C0 = _c(C0, np.float32)
    norm0 = _c(norm0, np.float32)
    xC_small = _c(xC_small, np.float32)
    G_small = _c(G_small, np.float32)
    G0S = _c(G0S, np.float32)
    hv = _c(h_vec, np.int32)
    n, d = X.shape
    h0 = C0.shape[0]
    Hs = G_small.shape[0]
    m = len(hv)
    fr = _c(forced_root, np.uint32) if forced_root is not None else None
    cid = np.empty(n, np.uint32)
    Bs = np.empty((n, max(m - 1, 0)), np.uint8)
    err = np.empty(n, np.float32)
    lib().orc_beam_search_large_root(_p(X, _f32p), d, _p(nx2, _f32p), _p(C0, _f32p), _p(norm0, _f32p),
                                     _p(xC_small, _f32p), _p(G_small, _f32p), _p(G0S, _f32p), h0, Hs, m,
                                     _p(hv, _i32p), H_beam, n, _p(fr, _u32p), root_mode, _p(cid, _u32p),
                                     _p(Bs, _u8p), _p(err, _f32p), nthreads)
    return cid, Bs, err


def large_root_candidates(X, nx2, C0, norm0, H_beam, forced_root=None, root_mode=0, nthreads=0):
    """Root stage of the large-root beam: [n, H_beam] arrays (errs, codes, a0, r00) in the
    layout of ExpandFromRootCandidates; unused slots have error +inf."""
    X = _c(X, np.float32)
    nx2 = _c(nx2, np.float32)
    C0 = _c(C0, np.float32)
    norm0 = _c(norm0, np.float32)
    n, d = X.shape
    fr = _c(forced_root, np.uint32) if forced_root is not None else None
    errs = np.empty((n, H_beam), np.float32)
    codes = np.empty((n, H_beam), np.int32)
    a0 = np.empty((n, H_beam), np.float32)
    r00 = np.empty((n, H_beam), np.float32)
    lib().orc_large_root_candidates(_p(X, _f32p), d, _p(nx2, _f32p), _p(C0, _f32p), _p(norm0, _f32p), C0.shape[0],
                                    H_beam, n, _p(fr, _u32p), root_mode, _p(errs, _f32p), _p(codes, _i32p),
                                    _p(a0, _f32p), _p(r00, _f32p), nthreads)
    return errs, codes, a0, r00


def invnorm_small(C_small):
    """invnorm_small_flat of BuildPrecompLargeRoot (precomp_large_root.cpp:101-114)."""
    C_small = _c(C_small, np.float32)
    Hs, d = C_small.shape
    out = np.empty(Hs, np.float32)
    lib().orc_invnorm_small(_p(C_small, _f32p), d, Hs, _p(out, _f32p))
    return out


def _lr_args(X, C0, norm0, xC_small, G_small, G0S, h_vec, cluster_id):
    X = _c(X, np.float32)
    C0 = _c(C0, np.float32)
    n, d = X.shape
    return (X, d, C0, _c(norm0, np.float32), C0.shape[0], _c(xC_small, np.float32), _c(G_small, np.float32),
            _c(G0S, np.float32), _c(h_vec, np.int32), _c(cluster_id, np.uint32), n)


def solve_ls_all_large_root(X, C0, norm0, xC_small, G_small, G0S, h_vec, cluster_id, B_small, nthreads=0):
    """SolveLeastSquaresAllLargeRoot; returns (a (n, m), ls_fails). B_small is (n, m-1)."""
    X, d, C0, norm0, h0, xs, Gs, G0S, hv, cid, n = _lr_args(X, C0, norm0, xC_small, G_small, G0S, h_vec, cluster_id)
    Bs = _c(B_small, np.uint8)
    m = len(hv)
    a = np.empty((n, m), np.float32)
    fails = lib().orc_solve_ls_all_large_root(_p(X, _f32p), d, _p(C0, _f32p), _p(norm0, _f32p), h0, _p(xs, _f32p),
                                              _p(Gs, _f32p), _p(G0S, _f32p), Gs.shape[0], m, _p(hv, _i32p),
                                              _p(cid, _u32p), _p(Bs, _u8p), n, _p(a, _f32p), nthreads)
    return a, int(fails)


def compute_costs_large_root(X, C0, norm0, xC_small, G_small, G0S, h_vec, cluster_id, B_small, a, nx2, nthreads=0):
    """ComputeCostsLargeRoot; returns cost (n,)."""
    X, d, C0, norm0, h0, xs, Gs, G0S, hv, cid, n = _lr_args(X, C0, norm0, xC_small, G_small, G0S, h_vec, cluster_id)
    Bs = _c(B_small, np.uint8)
    a = _c(a, np.float32)
    nx2 = _c(nx2, np.float32)
    cost = np.empty(n, np.float32)
    lib().orc_compute_costs_large_root(_p(X, _f32p), d, _p(C0, _f32p), _p(norm0, _f32p), h0, _p(xs, _f32p),
                                       _p(Gs, _f32p), _p(G0S, _f32p), Gs.shape[0], len(hv), _p(hv, _i32p),
                                       _p(cid, _u32p), _p(Bs, _u8p), _p(a, _f32p), _p(nx2, _f32p), n,
                                       _p(cost, _f32p), nthreads)
    return cost


def icm_ils_large_root(X, C0, norm0, xC_small, G_small, G0S, invs, h_vec, cluster_id, nx2, B_small, icm_iters,
                       ils_iters, perturb_k, use_abs, seed, sample_id_offset=0, nthreads=0):
    """DynamicIcmWithIls{Abs,NoAbs}NoNormalLargeRoot; returns (B_small, a, cost, ls_fails)."""
    X, d, C0, norm0, h0, xs, Gs, G0S, hv, cid, n = _lr_args(X, C0, norm0, xC_small, G_small, G0S, h_vec, cluster_id)
    Bs = np.array(B_small, dtype=np.uint8, copy=True, order="C")
    invs = _c(invs, np.float32)
    nx2 = _c(nx2, np.float32)
    m = len(hv)
    a = np.empty((n, m), np.float32)
    cost = np.empty(n, np.float32)
    fails = lib().orc_icm_ils_large_root(_p(X, _f32p), d, _p(C0, _f32p), _p(norm0, _f32p), h0, _p(xs, _f32p),
                                         _p(Gs, _f32p), _p(G0S, _f32p), _p(invs, _f32p), Gs.shape[0], m,
                                         _p(hv, _i32p), _p(cid, _u32p), _p(nx2, _f32p), n, icm_iters, ils_iters,
                                         perturb_k, int(bool(use_abs)), seed & 0xFFFFFFFF, int(sample_id_offset),
                                         _p(Bs, _u8p), _p(a, _f32p), _p(cost, _f32p), nthreads)
    return Bs, a, cost, int(fails)
