"""Python host mirror of STLQ's encoder interface, backed by libstlq_mi355 (HIP, gfx950).

The free functions carry the reference's names (namespace stlq, src/quantizer/*) and argument
meaning; arrays are numpy views of the reference's column-major matrices
(include/stlq/common/types.h:35-51):

    X      (n, d)  float32     == ColMajorMatrix<float> d x n
    C_all  (H, d)  float32     == Precomp::C_all d x H
    G      (H, H)  float32     numpy G[col, row] == reference G(row, col)
    xC     (n, H)  float32     == xC H x n
    codes  (n, m)  uint8       == ColMajorMatrix<FullCode> m x n
    a      (n, m)  float32

Every call runs on the GPU through the C ABI; errors raise StlqError with the library's
message (the reference returns false / throws std::runtime_error on its CUDA paths).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import EncodeParams, StreamStats, Timings, check

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i64p = ctypes.POINTER(ctypes.c_int64)


def _p(a, t):
    return a.ctypes.data_as(t) if a is not None else None


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


@dataclass
class EncodeConfig:
    """base.encode.* (include/stlq/common/config.h:473-482)."""

    H_beam: int = 2
    icm_iters: int = 4
    ils_iters: int = 0
    perturb_k: int = 3
    use_abs: bool = True
    seed: int = 38251450
    want_coeffs: bool = True

    def to_c(self) -> EncodeParams:
        return EncodeParams(int(self.H_beam), int(self.icm_iters), int(self.ils_iters), int(self.perturb_k),
                            int(bool(self.use_abs)), int(self.seed) & 0xFFFFFFFF, int(bool(self.want_coeffs)))


@dataclass
class BaseEncoding:
    """include/stlq/common/types.h:77-80."""

    B: np.ndarray
    a: np.ndarray | None


class Context:
    """One device context (stream + device buffers). Not thread-safe; one per host thread."""

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        h = ctypes.c_void_p()
        check(self.lib.stlq_mi355_ctx_create(int(device), ctypes.byref(h)))
        self.h = h
        self.d = self.m = self.H = 0
        self.h_vec: list[int] = []
        self.lr = None

    def close(self):
        if self.h:
            self.lib.stlq_mi355_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- precomp -------------------------------------------------------------------------
    def set_codebooks(self, C_all, h_vec):
        """BuildPrecomp (src/quantizer/encoder_precomp.inc:1-53) on the device."""
        C_all = _c(C_all, np.float32)
        hv = _c(h_vec, np.int32)
        H, d = C_all.shape
        if int(hv.sum()) != H:
            raise ValueError("sum(h_vec) must equal the number of codewords")
        check(self.lib.stlq_mi355_set_codebooks(self.h, d, len(hv), _p(hv, _i32p), _p(C_all, _f32p)))
        self.d, self.m, self.H, self.h_vec = d, len(hv), H, [int(x) for x in hv]

    def set_precomp(self, C_all, h_vec, G, invnorm):
        """Caller-built Precomp (include/stlq/common/types.h:62-75)."""
        C_all = _c(C_all, np.float32)
        hv = _c(h_vec, np.int32)
        G = _c(G, np.float32)
        inv = _c(invnorm, np.float32)
        H, d = C_all.shape
        check(self.lib.stlq_mi355_set_precomp(self.h, d, len(hv), _p(hv, _i32p), _p(C_all, _f32p), _p(G, _f32p),
                                              _p(inv, _f32p)))
        self.d, self.m, self.H, self.h_vec = d, len(hv), H, [int(x) for x in hv]

    def get_precomp(self):
        G = np.empty((self.H, self.H), np.float32)
        inv = np.empty(self.H, np.float32)
        check(self.lib.stlq_mi355_get_precomp(self.h, _p(G, _f32p), _p(inv, _f32p)))
        return G, inv

    # ---- building blocks -----------------------------------------------------------------
    def xnorm2(self, X):
        X = _c(X, np.float32)
        out = np.empty(X.shape[0], np.float32)
        check(self.lib.stlq_mi355_xnorm2(self.h, _p(X, _f32p), X.shape[1], X.shape[0], _p(out, _f32p)))
        return out

    def gemm_xc(self, X):
        X = _c(X, np.float32)
        xC = np.empty((X.shape[0], self.H), np.float32)
        check(self.lib.stlq_mi355_gemm_xc(self.h, _p(X, _f32p), X.shape[0], _p(xC, _f32p)))
        return xC

    def beam_search(self, xC, H_beam, X=None, nx2=None):
        xC = _c(xC, np.float32)
        n = xC.shape[0]
        Xc = _c(X, np.float32) if X is not None else None
        nx = _c(nx2, np.float32) if nx2 is not None else None
        codes = np.empty((n, self.m), np.uint8)
        err = np.empty(n, np.float32)
        check(self.lib.stlq_mi355_beam_search(self.h, _p(Xc, _f32p), _p(nx, _f32p), _p(xC, _f32p), n, int(H_beam),
                                              _p(codes, _u8p), _p(err, _f32p)))
        return codes, err

    def solve_ls_all(self, xC, codes):
        xC = _c(xC, np.float32)
        codes = _c(codes, np.uint8)
        n = xC.shape[0]
        a = np.empty((n, self.m), np.float32)
        fails = ctypes.c_int64(0)
        check(self.lib.stlq_mi355_solve_ls_all(self.h, _p(xC, _f32p), _p(codes, _u8p), n, _p(a, _f32p),
                                               ctypes.byref(fails)))
        return a, int(fails.value)

    def compute_costs(self, xC, codes, a, nx2):
        xC = _c(xC, np.float32)
        codes = _c(codes, np.uint8)
        a = _c(a, np.float32)
        nx2 = _c(nx2, np.float32)
        cost = np.empty(xC.shape[0], np.float32)
        check(self.lib.stlq_mi355_compute_costs(self.h, _p(xC, _f32p), _p(codes, _u8p), _p(a, _f32p), _p(nx2, _f32p),
                                                xC.shape[0], _p(cost, _f32p)))
        return cost

    def icm(self, xC, codes, icm_iters, use_abs, seed, X=None, nx2=None):
        xC = _c(xC, np.float32)
        codes = np.array(codes, dtype=np.uint8, order="C", copy=True)
        n = xC.shape[0]
        Xc = _c(X, np.float32) if X is not None else None
        nx = _c(nx2, np.float32) if nx2 is not None else None
        a = np.empty((n, self.m), np.float32)
        cost = np.empty(n, np.float32)
        check(self.lib.stlq_mi355_icm(self.h, _p(Xc, _f32p), _p(nx, _f32p), _p(xC, _f32p), n, int(icm_iters),
                                      int(bool(use_abs)), int(seed) & 0xFFFFFFFF, _p(codes, _u8p), _p(a, _f32p),
                                      _p(cost, _f32p)))
        return codes, a, cost

    def icm_ils(self, xC, codes, icm_iters, ils_iters, perturb_k, use_abs, seed, X=None, nx2=None,
                sample_id_offset=0):
        """ICM followed by the ILS outer loop (icm.cpp:872-1003); returns (codes, a, cost)."""
        xC = _c(xC, np.float32)
        codes = np.array(codes, dtype=np.uint8, order="C", copy=True)
        n = xC.shape[0]
        Xc = _c(X, np.float32) if X is not None else None
        nx = _c(nx2, np.float32) if nx2 is not None else None
        a = np.empty((n, self.m), np.float32)
        cost = np.empty(n, np.float32)
        check(self.lib.stlq_mi355_icm_ils(self.h, _p(Xc, _f32p), _p(nx, _f32p), _p(xC, _f32p), n, int(icm_iters),
                                          int(ils_iters), int(perturb_k), int(bool(use_abs)), int(seed) & 0xFFFFFFFF,
                                          int(sample_id_offset), _p(codes, _u8p), _p(a, _f32p), _p(cost, _f32p)))
        return codes, a, cost

    def encode(self, X, cfg: EncodeConfig, want_mse=False):
        X = _c(X, np.float32)
        n = X.shape[0]
        codes = np.empty((n, self.m), np.uint8)
        want = cfg.want_coeffs or cfg.icm_iters > 0 or cfg.ils_iters > 0
        a = np.empty((n, self.m), np.float32) if want else None
        cost = np.empty(n, np.float32) if want else None
        bm, fm = ctypes.c_double(0), ctypes.c_double(0)
        p = cfg.to_c()
        check(self.lib.stlq_mi355_encode(self.h, _p(X, _f32p), n, ctypes.byref(p), _p(codes, _u8p), _p(a, _f32p),
                                         _p(cost, _f32p), ctypes.byref(bm) if want_mse else None,
                                         ctypes.byref(fm) if want_mse else None))
        return codes, a, cost, (bm.value, fm.value)

    def last_timings(self) -> Timings:
        t = Timings()
        check(self.lib.stlq_mi355_last_timings(self.h, ctypes.byref(t)))
        return t

    # ---- device buffers (bench / FFI callers) ----------------------------------------------
    def dev_alloc(self, nbytes):
        p = ctypes.c_void_p()
        check(self.lib.stlq_mi355_dev_alloc(self.h, int(nbytes), ctypes.byref(p)))
        return p.value

    def dev_free(self, p):
        check(self.lib.stlq_mi355_dev_free(self.h, ctypes.c_void_p(p)))

    def h2d(self, dptr, arr):
        arr = np.ascontiguousarray(arr)
        check(self.lib.stlq_mi355_copy_h2d(self.h, ctypes.c_void_p(dptr), arr.ctypes.data_as(ctypes.c_void_p),
                                           arr.nbytes))

    def d2h(self, arr, dptr):
        check(self.lib.stlq_mi355_copy_d2h(self.h, arr.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(dptr),
                                           arr.nbytes))
        return arr

    def synchronize(self):
        check(self.lib.stlq_mi355_synchronize(self.h))

    def encode_device(self, dX, n, cfg: EncodeConfig, dcodes, da=None, dcost=None, stream=None):
        p = cfg.to_c()
        check(self.lib.stlq_mi355_encode_device(self.h, ctypes.c_void_p(dX), int(n), ctypes.byref(p),
                                                ctypes.c_void_p(dcodes), ctypes.c_void_p(da) if da else None,
                                                ctypes.c_void_p(dcost) if dcost else None,
                                                ctypes.c_void_p(stream) if stream else None))

    def encode_device_noalloc(self, dX, n, cfg: EncodeConfig, dcodes, da=None, dcost=None, stream=None):
        """encode_device without any device allocation (static per-device scratch; one tile)."""
        p = cfg.to_c()
        check(self.lib.stlq_mi355_encode_device_noalloc(self.h, ctypes.c_void_p(dX), int(n), ctypes.byref(p),
                                                        ctypes.c_void_p(dcodes), ctypes.c_void_p(da) if da else None,
                                                        ctypes.c_void_p(dcost) if dcost else None,
                                                        ctypes.c_void_p(stream) if stream else None))

    def device_info(self):
        buf = ctypes.create_string_buffer(128)
        cu = ctypes.c_int(0)
        check(self.lib.stlq_mi355_device_info(self.h, buf, 128, ctypes.byref(cu)))
        return buf.value.decode(), cu.value

    # ---- streaming -----------------------------------------------------------------------
    def encode_stream(self, n_total, chunk, cfg: EncodeConfig, fill, sink, input_u8=False, large_root=False,
                      root_mode=1, R=None, start_id=0):
        """Streaming encode of the vectors with global ids start_id .. start_id + n_total - 1.
        fill(first, count, out) fills `out` ((count, d) float32, or uint8 when input_u8) with the
        vectors from global id `first`. sink(first, count, result) receives a dict of numpy copies:
        full precomp -> codes; large root -> cluster_id, B_small, best_err; both with a and cost
        when coefficients or ICM/ILS are asked for. ILS perturbations are keyed by the global ids."""
        if large_root:
            d, m = self.lr[0], len(self.lr[1])
        else:
            d, m = self.d, self.m
        want = cfg.want_coeffs or cfg.icm_iters > 0 or cfg.ils_iters > 0
        dt = np.uint8 if input_u8 else np.float32
        ctype = ctypes.c_uint8 if input_u8 else ctypes.c_float
        err = []

        def _fill(user, first, count, dst):
            try:
                buf = ctypes.cast(dst, ctypes.POINTER(ctype))
                view = np.ctypeslib.as_array(buf, shape=(count * d,)).reshape(count, d)
                assert view.dtype == dt
                fill(int(first), int(count), view)
                return 0
            except Exception as e:  # surfaced after the call
                err.append(e)
                return 1

        def _sink(user, first, count, outp):
            try:
                o = outp.contents
                res = {}
                if large_root:
                    res["cluster_id"] = np.ctypeslib.as_array(o.cluster_id, shape=(count,)).copy()
                    res["B_small"] = (np.ctypeslib.as_array(o.B_small, shape=(count * (m - 1),)).reshape(count, m - 1).copy()
                                      if m > 1 else np.zeros((count, 0), np.uint8))
                    res["best_err"] = np.ctypeslib.as_array(o.best_err, shape=(count,)).copy()
                    if want:
                        res["a"] = np.ctypeslib.as_array(o.a, shape=(count * m,)).reshape(count, m).copy()
                        res["cost"] = np.ctypeslib.as_array(o.cost, shape=(count,)).copy()
                else:
                    res["codes"] = np.ctypeslib.as_array(o.codes, shape=(count * m,)).reshape(count, m).copy()
                    if want:
                        res["a"] = np.ctypeslib.as_array(o.a, shape=(count * m,)).reshape(count, m).copy()
                        res["cost"] = np.ctypeslib.as_array(o.cost, shape=(count,)).copy()
                sink(int(first), int(count), res)
                return 0
            except Exception as e:
                err.append(e)
                return 1

        f, s = _lib.FILL_FN(_fill), _lib.SINK_FN(_sink)
        st = StreamStats()
        Rc = None
        if R is not None:  # numpy (d, d) matrix R[r, k]; the C ABI takes the reference's column-major array
            Rc = np.ascontiguousarray(np.asarray(R, dtype=np.float32).T)
            if Rc.shape != (d, d):
                raise ValueError(f"R must be {d} x {d}")
        p = _lib.StreamParams(cfg.to_c(), int(bool(input_u8)), int(bool(large_root)), int(root_mode), _p(Rc, _f32p),
                              int(start_id))
        rc = self.lib.stlq_mi355_encode_stream(self.h, int(n_total), int(chunk), ctypes.byref(p), f, s, None,
                                               ctypes.byref(st))
        if err:
            raise err[0]
        check(rc)
        return st

    # ---- large root ----------------------------------------------------------------------
    def set_large_root(self, C0, C_small, h_vec):
        """BuildPrecompLargeRoot (src/quantizer/precomp_large_root.cpp:27-157) on the device."""
        C0 = _c(C0, np.float32)
        Cs = _c(C_small, np.float32)
        hv = _c(h_vec, np.int32)
        check(self.lib.stlq_mi355_set_large_root(self.h, C0.shape[1], len(hv), _p(hv, _i32p), _p(C0, _f32p),
                                                 _p(Cs, _f32p)))
        self.lr = (C0.shape[1], [int(x) for x in hv])

    def beam_search_large_root(self, X, H_beam, xC_small=None, forced_root=None, root_mode=0):
        X = _c(X, np.float32)
        n = X.shape[0]
        m = len(self.lr[1])
        xs = _c(xC_small, np.float32) if xC_small is not None else None
        fr = _c(forced_root, np.uint32) if forced_root is not None else None
        cid = np.empty(n, np.uint32)
        Bs = np.empty((n, max(m - 1, 0)), np.uint8)
        err = np.empty(n, np.float32)
        check(self.lib.stlq_mi355_beam_search_large_root(self.h, _p(X, _f32p), _p(xs, _f32p), n, int(H_beam),
                                                         _p(fr, _u32p), int(root_mode), _p(cid, _u32p), _p(Bs, _u8p),
                                                         _p(err, _f32p)))
        return cid, Bs, err

    def convert_u8_rotate(self, X_u8, R=None):
        """ConvertU8ToF32AndRotatePtr (kernel_provider.h:44-52) on row-major (n, d) uint8 vectors:
        returns float32 (n, d) with row i = R @ x_i (R a numpy (d, d) matrix; None = identity)."""
        X_u8 = np.ascontiguousarray(X_u8, dtype=np.uint8)
        n, d = X_u8.shape
        Rc = np.ascontiguousarray(np.asarray(R, dtype=np.float32).T) if R is not None else None
        out = np.empty((n, d), np.float32)
        check(self.lib.stlq_mi355_convert_u8_rotate(self.h, _p(X_u8, _u8p), d, d, n, _p(Rc, _f32p), _p(out, _f32p)))
        return out

    def _lr_inputs(self, X, cluster_id, B_small, xC_small):
        X = _c(X, np.float32)
        n = X.shape[0]
        m = len(self.lr[1])
        cid = _c(cluster_id, np.uint32)
        Bs = np.array(B_small, dtype=np.uint8, order="C", copy=True).reshape(n, max(m - 1, 0))
        xs = _c(xC_small, np.float32) if xC_small is not None else None
        return X, n, m, cid, Bs, xs

    def solve_ls_all_large_root(self, X, cluster_id, B_small, xC_small=None):
        """SolveLeastSquaresAllLargeRoot (least_squares.cpp:667-745); returns (a, fail_count)."""
        X, n, m, cid, Bs, xs = self._lr_inputs(X, cluster_id, B_small, xC_small)
        a = np.empty((n, m), np.float32)
        fails = ctypes.c_int64(0)
        check(self.lib.stlq_mi355_solve_ls_all_large_root(self.h, _p(X, _f32p), _p(xs, _f32p), n, _p(cid, _u32p),
                                                          _p(Bs, _u8p), _p(a, _f32p), ctypes.byref(fails)))
        return a, int(fails.value)

    def compute_costs_large_root(self, X, cluster_id, B_small, a, nx2=None, xC_small=None):
        """ComputeCostsLargeRoot (cost_utils.cpp:211-233)."""
        X, n, m, cid, Bs, xs = self._lr_inputs(X, cluster_id, B_small, xC_small)
        a = _c(a, np.float32)
        nx = _c(nx2, np.float32) if nx2 is not None else None
        cost = np.empty(n, np.float32)
        check(self.lib.stlq_mi355_compute_costs_large_root(self.h, _p(X, _f32p), _p(xs, _f32p), n, _p(cid, _u32p),
                                                           _p(Bs, _u8p), _p(a, _f32p), _p(nx, _f32p), _p(cost, _f32p)))
        return cost

    def icm_ils_large_root(self, X, cluster_id, B_small, icm_iters, ils_iters, perturb_k, use_abs, seed,
                           nx2=None, xC_small=None, sample_id_offset=0):
        """DynamicIcmWithIls{Abs,NoAbs}NoNormalLargeRoot (icm.cpp:1005-1120); returns (B_small, a, cost)."""
        X, n, m, cid, Bs, xs = self._lr_inputs(X, cluster_id, B_small, xC_small)
        nx = _c(nx2, np.float32) if nx2 is not None else None
        a = np.empty((n, m), np.float32)
        cost = np.empty(n, np.float32)
        check(self.lib.stlq_mi355_icm_ils_large_root(self.h, _p(X, _f32p), _p(nx, _f32p), _p(xs, _f32p), n,
                                                     _p(cid, _u32p), int(icm_iters), int(ils_iters), int(perturb_k),
                                                     int(bool(use_abs)), int(seed) & 0xFFFFFFFF, int(sample_id_offset),
                                                     _p(Bs, _u8p), _p(a, _f32p), _p(cost, _f32p)))
        return Bs, a, cost


# ---- reference-named free functions ----------------------------------------------------------
def BuildPrecomp(ctx: Context, C_all, h_vec):
    """src/quantizer/encoder_precomp.inc:1-53. Returns (G, invnorm) as computed on the device."""
    ctx.set_codebooks(C_all, h_vec)
    return ctx.get_precomp()


def ComputeXNorm2(ctx: Context, X):
    """src/quantizer/cost_utils.cpp:88-110."""
    return ctx.xnorm2(X)


def BeamSearchPrefixLS(ctx: Context, X, xC, H_beam):
    """src/quantizer/beam_search.cpp:196-422: codes (n, m) uint8."""
    return ctx.beam_search(xC, max(1, int(H_beam)), X=X)[0]


def SolveLeastSquaresAll(ctx: Context, xC, B):
    """src/quantizer/least_squares.cpp:406-565: a (n, m); failed vectors get zero coefficients."""
    return ctx.solve_ls_all(xC, B)[0]


def ComputeCosts(ctx: Context, xC, B, a, X_norm2):
    """src/quantizer/cost_utils.cpp:139-158."""
    return ctx.compute_costs(xC, B, a, X_norm2)


def _dynamic_icm(ctx, X, xC, icm_iters, ils_iters, perturb_k, seed, B, use_abs, sample_id_offset):
    return ctx.icm_ils(xC, B, icm_iters, ils_iters, perturb_k, use_abs, seed, X=X, sample_id_offset=sample_id_offset)


def DynamicIcmWithIlsAbsNoNormal(ctx: Context, X, xC, icm_iters, ils_iters, perturb_k, seed, B,
                                 print_progress=True, sample_id_offset=0):
    """src/quantizer/icm.cpp:1153-1170 (icm.h:33-43): returns (B, a, cost)."""
    return _dynamic_icm(ctx, X, xC, icm_iters, ils_iters, perturb_k, seed, B, True, sample_id_offset)


def DynamicIcmWithIlsNoAbsNoNormal(ctx: Context, X, xC, icm_iters, ils_iters, perturb_k, seed, B,
                                   print_progress=True, sample_id_offset=0):
    """src/quantizer/icm.cpp:1132-1151 (icm.h:15-31): returns (B, a, cost)."""
    return _dynamic_icm(ctx, X, xC, icm_iters, ils_iters, perturb_k, seed, B, False, sample_id_offset)


def EncodeBase(ctx: Context, X, cfg: EncodeConfig):
    """src/quantizer/encoder_encode_base.inc:1-106: (BaseEncoding, beam_mse, final_mse)."""
    if X.shape[0] == 0 or X.shape[1] == 0:
        raise ValueError("Empty base dataset.")
    if X.shape[1] != ctx.d:
        raise ValueError("Precomp dimensions do not match codebooks or dataset.")
    codes, a, _, (bm, fm) = ctx.encode(X, cfg, want_mse=True)
    return BaseEncoding(codes, a), bm, fm


def EncodeBaseStreamingF32(ctx: Context, n_total, chunk, cfg: EncodeConfig, fill, sink, start_id=0):
    """src/quantizer/encode_base_streaming.cpp:4544-4579: fp32 chunks, double-buffered H2D; ids
    start at start_id (a resumed stream)."""
    return ctx.encode_stream(n_total, chunk, cfg, fill, sink, start_id=start_id)


def EncodeBaseStreaming(ctx: Context, n_total, chunk, cfg: EncodeConfig, fill, sink, root_mode=1, start_id=0):
    """src/quantizer/encode_base_streaming.cpp:1913 (large pipeline): uint8 chunks widened on the
    device, large-root beam, then the large-root refit (:1117-1210) when cfg asks for
    coefficients or ICM/ILS; sink gets cluster_id, B_small, best_err (and a, cost) per chunk."""
    return ctx.encode_stream(n_total, chunk, cfg, fill, sink, input_u8=True, large_root=True, root_mode=root_mode,
                             start_id=start_id)


def BuildPrecompLargeRoot(ctx: Context, C0, C_small, h_vec):
    """src/quantizer/precomp_large_root.cpp:27-157."""
    ctx.set_large_root(C0, C_small, h_vec)


def BeamSearchPrefixLSLargeRoot(ctx: Context, X, xC_small, H_beam, forced_root=None):
    """src/quantizer/beam_search.cpp:579-726: (cluster_id, B_small)."""
    cid, Bs, _ = ctx.beam_search_large_root(X, H_beam, xC_small=xC_small, forced_root=forced_root)
    return cid, Bs


def SolveLeastSquaresAllLargeRoot(ctx: Context, X, xC_small, cluster_id, B_small):
    """src/quantizer/least_squares.cpp:667-745: a (n, m); failed vectors get zero coefficients."""
    return ctx.solve_ls_all_large_root(X, cluster_id, B_small, xC_small=xC_small)[0]


def ComputeCostsLargeRoot(ctx: Context, X, xC_small, cluster_id, B_small, a, X_norm2):
    """src/quantizer/cost_utils.cpp:211-233."""
    return ctx.compute_costs_large_root(X, cluster_id, B_small, a, nx2=X_norm2, xC_small=xC_small)


def DynamicIcmWithIlsAbsNoNormalLargeRoot(ctx: Context, X, xC_small, icm_iters, ils_iters, perturb_k, seed,
                                          cluster_id, B_small, print_progress=True, sample_id_offset=0):
    """src/quantizer/icm.cpp:1005-1120 (icm.h:62-75), |score|: returns (B_small, a, cost)."""
    return ctx.icm_ils_large_root(X, cluster_id, B_small, icm_iters, ils_iters, perturb_k, True, seed,
                                  xC_small=xC_small, sample_id_offset=sample_id_offset)


def DynamicIcmWithIlsNoAbsNoNormalLargeRoot(ctx: Context, X, xC_small, icm_iters, ils_iters, perturb_k, seed,
                                            cluster_id, B_small, print_progress=True, sample_id_offset=0):
    """src/quantizer/icm.cpp:1005-1120 (icm.h:47-60), signed score: returns (B_small, a, cost)."""
    return ctx.icm_ils_large_root(X, cluster_id, B_small, icm_iters, ils_iters, perturb_k, False, seed,
                                  xC_small=xC_small, sample_id_offset=sample_id_offset)
