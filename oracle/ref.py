"""ctypes access to the reference's own CPU encoder functions, compiled from the reference
sources in place by `make -C oracle ref` into oracle/_ref/libstlq_ref.so (see ref_driver.cpp).

TEST INFRASTRUCTURE ONLY: tests use it to check the oracle restatement against the reference;
the product never loads it. Where the reference sources are absent the library cannot be built
and available() is False.

Array conventions follow the oracle's: numpy row-major (n, d) == the reference's column-major
d x n, (n, H) == H x n, codes (n, m) == m x n.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_ref", "libstlq_ref.so")
REF_ROOT = os.environ.get("STLQ_REFERENCE_ROOT", "/root/reference")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_int = ctypes.c_int


def sources_present() -> bool:
    return os.path.exists(os.path.join(REF_ROOT, "src", "quantizer", "beam_search.cpp"))


def build() -> str:
    """make -C oracle ref (g++ on the reference's own translation units)."""
    subprocess.run(["make", "-s", "-C", _HERE, "ref", f"REF={REF_ROOT}"], check=True)
    return _LIB_PATH


def available() -> bool:
    """True when the reference library is built and loads (its MKL dependency included)."""
    if not os.path.exists(_LIB_PATH):
        return False
    try:
        lib()
    except OSError:
        return False
    return True


def lib():
    global _lib
    if _lib is None:
        # MKL's sequential layer for the LAPACK calls (read by mkl_rt when it first initialises):
        # its threaded layer inside the reference's OpenMP loops left results depending on
        # earlier calls in the process.
        os.environ.setdefault("MKL_THREADING_LAYER", "SEQUENTIAL")
        # Lazy binding: GemmRaw/BlasSetThreads (blas.cpp, not buildable here) stay unresolved and
        # are never reached by the driver's entry points.
        L = ctypes.CDLL(_LIB_PATH, mode=os.RTLD_LAZY)
        L.ref_xnorm2.argtypes = [_f32p, _int, _int, _f32p]
        L.ref_beam_search.argtypes = [_f32p, _int, _int, _f32p, _f32p, _int, _i32p, _int, _int, _u8p]
        L.ref_compute_costs.argtypes = [_f32p, _f32p, _int, _i32p, _int, _u8p, _f32p, _f32p, _int, _f32p]
        L.ref_expand_large_root.argtypes = [_f32p, _int, _f32p, _int, _i32p, _int, _f32p, _int, _int, _f32p,
                                            _i32p, _f32p, _f32p, _u32p, _u8p]
        L.ref_solve_ls_all.argtypes = [_f32p, _f32p, _int, _i32p, _int, _u8p, _int, _f32p]
        L.ref_icm.argtypes = [_f32p, _int, _int, _f32p, _f32p, _f32p, _int, _i32p, _int, _int, _int, _int, _int,
                              ctypes.c_uint32, ctypes.c_uint64, _u8p, _f32p, _f32p]
        L.ref_solve_ls_all_large_root.argtypes = [_f32p, _int, _int, _f32p, _f32p, _f32p, _int, _f32p, _i32p, _int,
                                                  _f32p, _u32p, _u8p, _f32p]
        L.ref_compute_costs_large_root.argtypes = [_f32p, _int, _int, _f32p, _f32p, _f32p, _int, _f32p, _i32p, _int,
                                                   _f32p, _u32p, _u8p, _f32p, _f32p, _f32p]
        L.ref_icm_large_root.argtypes = [_f32p, _int, _int, _f32p, _f32p, _f32p, _int, _f32p, _f32p, _i32p, _int,
                                         _f32p, _u32p, _int, _int, _int, _int, ctypes.c_uint32, ctypes.c_uint64,
                                         _u8p, _f32p, _f32p]
        for f in (L.ref_xnorm2, L.ref_beam_search, L.ref_compute_costs, L.ref_expand_large_root, L.ref_solve_ls_all,
                  L.ref_icm, L.ref_solve_ls_all_large_root, L.ref_compute_costs_large_root, L.ref_icm_large_root):
            f.restype = None
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _p(a, t):
    return a.ctypes.data_as(t)


def xnorm2(X):
    X = _c(X, np.float32)
    n, d = X.shape
    out = np.empty(n, np.float32)
    lib().ref_xnorm2(_p(X, _f32p), d, n, _p(out, _f32p))
    return out


def beam_search(X, xC, G, h_vec, H_beam):
    """stlq::BeamSearchPrefixLS; ||x||^2 is formed inside from X."""
    X = _c(X, np.float32)
    xC = _c(xC, np.float32)
    G = _c(G, np.float32)
    hv = _c(h_vec, np.int32)
    n, d = X.shape
    H = G.shape[0]
    m = len(hv)
    codes = np.empty((n, m), np.uint8)
    lib().ref_beam_search(_p(X, _f32p), d, n, _p(xC, _f32p), _p(G, _f32p), H, _p(hv, _i32p), m, H_beam,
                          _p(codes, _u8p))
    return codes


def compute_costs(xC, G, h_vec, codes, a, nx2):
    xC = _c(xC, np.float32)
    G = _c(G, np.float32)
    hv = _c(h_vec, np.int32)
    codes = _c(codes, np.uint8)
    a = _c(a, np.float32)
    nx2 = _c(nx2, np.float32)
    n, H = xC.shape
    cost = np.empty(n, np.float32)
    lib().ref_compute_costs(_p(xC, _f32p), _p(G, _f32p), H, _p(hv, _i32p), len(hv), _p(codes, _u8p), _p(a, _f32p),
                            _p(nx2, _f32p), n, _p(cost, _f32p))
    return cost


def solve_ls_all(xC, G, h_vec, codes):
    """stlq::SolveLeastSquaresAll (hand Cholesky for m in {5, 10}, LAPACK spotrf/spotrs otherwise)."""
    xC = _c(xC, np.float32)
    G = _c(G, np.float32)
    hv = _c(h_vec, np.int32)
    codes = _c(codes, np.uint8)
    n, H = xC.shape
    a = np.empty((n, len(hv)), np.float32)
    lib().ref_solve_ls_all(_p(xC, _f32p), _p(G, _f32p), H, _p(hv, _i32p), len(hv), _p(codes, _u8p), n, _p(a, _f32p))
    return a


def icm(X, xC, G, invnorm, h_vec, codes, icm_iters, use_abs, seed, ils_iters=0, perturb_k=3, sample_id_offset=0):
    """stlq::DynamicIcmWithIls{Abs,NoAbs}NoNormal; returns (codes, a, cost)."""
    X = _c(X, np.float32)
    xC = _c(xC, np.float32)
    G = _c(G, np.float32)
    inv = _c(invnorm, np.float32)
    hv = _c(h_vec, np.int32)
    codes = np.array(codes, dtype=np.uint8, copy=True, order="C")
    n, d = X.shape
    H = G.shape[0]
    m = len(hv)
    a = np.empty((n, m), np.float32)
    cost = np.empty(n, np.float32)
    lib().ref_icm(_p(X, _f32p), d, n, _p(xC, _f32p), _p(G, _f32p), _p(inv, _f32p), H, _p(hv, _i32p), m, icm_iters,
                  ils_iters, perturb_k, int(bool(use_abs)), seed & 0xFFFFFFFF, int(sample_id_offset),
                  _p(codes, _u8p), _p(a, _f32p), _p(cost, _f32p))
    return codes, a, cost


def expand_large_root(G_small, G0S, h_vec, xC_small, H_beam, root_errs, root_codes, root_a0, root_r00):
    """stlq::BeamSearchPrefixLSLargeRootExpandFromRootCandidates over all vectors.
    G0S as the oracle returns it: numpy (Hs, h0) == the reference's h0 x Hs column-major."""
    G_small = _c(G_small, np.float32)
    G0S = _c(G0S, np.float32)
    hv = _c(h_vec, np.int32)
    xs = _c(xC_small, np.float32)
    n, Hs = xs.shape
    h0 = G0S.shape[1]
    m = len(hv)
    cid = np.empty(n, np.uint32)
    Bs = np.empty((n, m - 1), np.uint8)
    lib().ref_expand_large_root(_p(G_small, _f32p), Hs, _p(G0S, _f32p), h0, _p(hv, _i32p), m, _p(xs, _f32p), n,
                                H_beam, _p(_c(root_errs, np.float32), _f32p), _p(_c(root_codes, np.int32), _i32p),
                                _p(_c(root_a0, np.float32), _f32p), _p(_c(root_r00, np.float32), _f32p),
                                _p(cid, _u32p), _p(Bs, _u8p))
    return cid, Bs


def _lr(X, C0, norm0, G_small, G0S, h_vec, xC_small, cluster_id):
    X = _c(X, np.float32)
    n, d = X.shape
    return (X, d, n, _c(C0, np.float32), _c(norm0, np.float32), _c(G_small, np.float32), _c(G0S, np.float32),
            _c(h_vec, np.int32), _c(xC_small, np.float32), _c(cluster_id, np.uint32))


def solve_ls_all_large_root(X, C0, norm0, G_small, G0S, h_vec, xC_small, cluster_id, B_small):
    """stlq::SolveLeastSquaresAllLargeRoot. G0S as the oracle returns it (numpy (Hs, h0))."""
    X, d, n, C0, norm0, Gs, G0S, hv, xs, cid = _lr(X, C0, norm0, G_small, G0S, h_vec, xC_small, cluster_id)
    a = np.empty((n, len(hv)), np.float32)
    lib().ref_solve_ls_all_large_root(_p(X, _f32p), d, n, _p(C0, _f32p), _p(norm0, _f32p), _p(Gs, _f32p),
                                      Gs.shape[0], _p(G0S, _f32p), _p(hv, _i32p), len(hv), _p(xs, _f32p),
                                      _p(cid, _u32p), _p(_c(B_small, np.uint8), _u8p), _p(a, _f32p))
    return a


def compute_costs_large_root(X, C0, norm0, G_small, G0S, h_vec, xC_small, cluster_id, B_small, a, nx2):
    """stlq::ComputeCostsLargeRoot."""
    X, d, n, C0, norm0, Gs, G0S, hv, xs, cid = _lr(X, C0, norm0, G_small, G0S, h_vec, xC_small, cluster_id)
    cost = np.empty(n, np.float32)
    lib().ref_compute_costs_large_root(_p(X, _f32p), d, n, _p(C0, _f32p), _p(norm0, _f32p), _p(Gs, _f32p),
                                       Gs.shape[0], _p(G0S, _f32p), _p(hv, _i32p), len(hv), _p(xs, _f32p),
                                       _p(cid, _u32p), _p(_c(B_small, np.uint8), _u8p), _p(_c(a, np.float32), _f32p),
                                       _p(_c(nx2, np.float32), _f32p), _p(cost, _f32p))
    return cost


def icm_large_root(X, C0, norm0, G_small, G0S, invs, h_vec, xC_small, cluster_id, B_small, icm_iters, use_abs, seed,
                   ils_iters=0, perturb_k=3, sample_id_offset=0):
    """stlq::DynamicIcmWithIls{Abs,NoAbs}NoNormalLargeRoot; returns (B_small, a, cost)."""
    X, d, n, C0, norm0, Gs, G0S, hv, xs, cid = _lr(X, C0, norm0, G_small, G0S, h_vec, xC_small, cluster_id)
    Bs = np.array(B_small, dtype=np.uint8, copy=True, order="C")
    m = len(hv)
    a = np.empty((n, m), np.float32)
    cost = np.empty(n, np.float32)
    lib().ref_icm_large_root(_p(X, _f32p), d, n, _p(C0, _f32p), _p(norm0, _f32p), _p(Gs, _f32p), Gs.shape[0],
                             _p(G0S, _f32p), _p(_c(invs, np.float32), _f32p), _p(hv, _i32p), m, _p(xs, _f32p),
                             _p(cid, _u32p), icm_iters, ils_iters, perturb_k, int(bool(use_abs)), seed & 0xFFFFFFFF,
                             int(sample_id_offset), _p(Bs, _u8p), _p(a, _f32p), _p(cost, _f32p))
    return Bs, a, cost


def _store_lib():
    L = lib()
    if not getattr(L, "_store_declared", False):
        _u64p = ctypes.POINTER(ctypes.c_uint64)
        _i64p = ctypes.POINTER(ctypes.c_int64)
        L.ref_store_write.argtypes = [ctypes.c_char_p, _int, _int, _i32p, _int, _int, _int, _int, _int, _int, _int,
                                      _int, ctypes.c_uint64, _u64p, _int, _int, _u64p, _i64p, _u32p, _u8p, _f32p,
                                      _int, ctypes.c_void_p, ctypes.c_char_p, _u64p, ctypes.c_char_p, _int]
        L.ref_store_write.restype = _int
        L.ref_store_truncate.argtypes = [ctypes.c_char_p, _int, _i32p, _int, _int, _int, ctypes.c_char_p, _u64p,
                                         _u64p, _int, ctypes.POINTER(_int), ctypes.c_char_p, _int]
        L.ref_store_truncate.restype = _int
        L._store_declared = True
    return L


def store_write(dir, d, m, h_vec, blocks, raw_kind=0, shard_size=2000000, bucket_size=256, bucket_flush_mb=256,
                write_vector_bucket=True, write_basic_to_bucket=True, raw_bytes_per_vec=0, resume_start=None,
                bucket_sizes=None, ckpt_path=None):
    """Writes a store with the reference's io::BaseBasicWriter. blocks: list of
    (start_id, cluster_id (n,), B_small (n, m-1), a (n, m), raw (n, d) or None). raw_kind 0 AppendBlock
    without vectors, 1 AppendBlockRawU8, 2 AppendBlockRawF32, 3 AppendBlock with a uint8 matrix.
    resume_start (with bucket_sizes) opens with OpenResume; ckpt_path commits after every block.
    Returns (ok, err, bucket_file_bytes)."""
    L = _store_lib()
    hv = _c(h_vec, np.int32)
    starts = np.array([b[0] for b in blocks], dtype=np.uint64)
    counts = np.array([len(b[1]) for b in blocks], dtype=np.int64)
    cid = _c(np.concatenate([np.asarray(b[1], np.uint32) for b in blocks]) if blocks else np.zeros(0), np.uint32)
    mc = max(0, m - 1)
    Bs = _c(np.concatenate([np.asarray(b[2], np.uint8).reshape(len(b[1]), mc) for b in blocks]) if blocks
            else np.zeros((0, mc)), np.uint8)
    A = _c(np.concatenate([np.asarray(b[3], np.float32).reshape(len(b[1]), m) for b in blocks]) if blocks
           else np.zeros((0, m)), np.float32)
    raw = None
    if blocks and blocks[0][4] is not None:
        raw = np.ascontiguousarray(np.concatenate([np.asarray(b[4]) for b in blocks]))
    h0 = int(hv[0]) if len(hv) else 0
    nlayout = (h0 + max(1, bucket_size) - 1) // max(1, bucket_size) if h0 > 0 else 0
    # A fresh Open ignores bucket_sizes; their count then only caps the bucket bytes read back.
    sizes = _c(bucket_sizes if resume_start is not None else np.zeros(max(nlayout, 1)), np.uint64)
    out = np.zeros(len(sizes), np.uint64)
    err = ctypes.create_string_buffer(512)
    _u64p = ctypes.POINTER(ctypes.c_uint64)
    ok = L.ref_store_write(dir.encode(), d, m, _p(hv, _i32p), len(hv), shard_size, bucket_size, bucket_flush_mb,
                           int(bool(write_vector_bucket)), int(bool(write_basic_to_bucket)), raw_bytes_per_vec,
                           int(resume_start is not None), int(resume_start or 0), _p(sizes, _u64p), len(sizes),
                           len(blocks), _p(starts, _u64p), _p(counts, ctypes.POINTER(ctypes.c_int64)),
                           _p(cid, _u32p), _p(Bs, _u8p), _p(A, _f32p), raw_kind,
                           None if raw is None else raw.ctypes.data_as(ctypes.c_void_p),
                           ckpt_path.encode() if ckpt_path else None, _p(out, _u64p), err, 512)
    return bool(ok), err.value.decode(), out[:nlayout]


def store_truncate(dir, m, h_vec, ckpt_path, shard_size=2000000, bucket_size=256):
    """app::ReadBaseBasicCheckpoint + app::TruncateBaseBasicToCheckpoint; returns (ok, err, next_id, sizes)."""
    L = _store_lib()
    hv = _c(h_vec, np.int32)
    nid = ctypes.c_uint64()
    sizes = np.zeros(1 << 16, np.uint64)
    nb = ctypes.c_int()
    err = ctypes.create_string_buffer(512)
    ok = L.ref_store_truncate(dir.encode(), m, _p(hv, _i32p), len(hv), shard_size, bucket_size, ckpt_path.encode(),
                              ctypes.byref(nid), _p(sizes, ctypes.POINTER(ctypes.c_uint64)), len(sizes),
                              ctypes.byref(nb), err, 512)
    return bool(ok), err.value.decode(), int(nid.value), sizes[:nb.value].copy()
