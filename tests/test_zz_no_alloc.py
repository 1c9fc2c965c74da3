"""stlq_mi355_encode_device_noalloc: the device encode with every work buffer in the static
per-device scratch. Called through the C ABI and compared bit for bit with
stlq_mi355_encode_device (codes, coefficients, costs) on two calls in a row, the second with a
smaller input, so stale scratch contents from the first call must not leak into the second."""
import ctypes

import numpy as np
import pytest

from stlq_amd import _lib
from stlq_amd.encoder import EncodeConfig
from tests.helpers import rvq_problem

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


class _Dev:
    """Device buffers for one encode: X, codes, a, cost."""

    def __init__(self, ctx, X, m):
        n = X.shape[0]
        self.ctx, self.n, self.m = ctx, n, m
        self.X = ctx.dev_alloc(X.nbytes)
        self.codes = ctx.dev_alloc(n * m)
        self.a = ctx.dev_alloc(n * m * 4)
        self.cost = ctx.dev_alloc(n * 4)
        ctx.h2d(self.X, X)

    def results(self):
        c = self.ctx
        c.synchronize()
        codes = c.d2h(np.empty((self.n, self.m), np.uint8), self.codes)
        a = c.d2h(np.empty((self.n, self.m), np.float32), self.a)
        cost = c.d2h(np.empty(self.n, np.float32), self.cost)
        return codes, a, cost

    def free(self):
        for p in (self.X, self.codes, self.a, self.cost):
            self.ctx.dev_free(p)


def _noalloc(ctx, dev, cfg, with_coeffs=True):
    p = cfg.to_c()
    rc = ctx.lib.stlq_mi355_encode_device_noalloc(ctx.h, ctypes.c_void_p(dev.X), dev.n, ctypes.byref(p),
                                                 ctypes.c_void_p(dev.codes),
                                                 ctypes.c_void_p(dev.a) if with_coeffs else None,
                                                 ctypes.c_void_p(dev.cost) if with_coeffs else None, None)
    _lib.check(rc)


def _alloc(ctx, dev, cfg):
    p = cfg.to_c()
    _lib.check(ctx.lib.stlq_mi355_encode_device(ctx.h, ctypes.c_void_p(dev.X), dev.n, ctypes.byref(p),
                                                ctypes.c_void_p(dev.codes), ctypes.c_void_p(dev.a),
                                                ctypes.c_void_p(dev.cost), None))


@pytest.mark.parametrize("cfg", [EncodeConfig(H_beam=16, icm_iters=0, want_coeffs=True),
                                 EncodeConfig(H_beam=8, icm_iters=2, ils_iters=2, perturb_k=3, want_coeffs=True)],
                         ids=["beam16_ls", "beam8_icm_ils"])
def test_noalloc_matches_encode_device_two_calls(ctx, cfg):
    X, C = rvq_problem(901, 6000, 64, 8, 256, kind="desc", train_n=3000, iters=3)
    h = [256] * 8
    ctx.set_codebooks(C, h)
    print(f"noalloc cfg H_beam={cfg.H_beam} icm={cfg.icm_iters} ils={cfg.ils_iters}", flush=True)
    for n in (6000, 1700):  # second call smaller: the scratch still holds the first call's bytes
        Xn = np.ascontiguousarray(X[:n])
        ref, got = _Dev(ctx, Xn, 8), _Dev(ctx, Xn, 8)
        try:
            _alloc(ctx, ref, cfg)
            want = ref.results()
            _noalloc(ctx, got, cfg)
            have = got.results()
        finally:
            ref.free()
            got.free()
        assert np.array_equal(want[0], have[0]), (n, np.nonzero(np.any(want[0] != have[0], axis=1))[0][:10])
        assert np.array_equal(_bits(want[1]), _bits(have[1])), n
        assert np.array_equal(_bits(want[2]), _bits(have[2])), n


def test_noalloc_codes_only_and_capacity_error(ctx):
    """Without coefficient outputs the LS buffers come from the scratch too; an n beyond the
    scratch capacity for the shape is refused with a message naming the capacity."""
    X, C = rvq_problem(902, 3000, 128, 8, 256, kind="desc", train_n=3000, iters=3)
    h = [256] * 8
    ctx.set_codebooks(C, h)
    cfg = EncodeConfig(H_beam=16, icm_iters=1, want_coeffs=True)
    ref, got = _Dev(ctx, X, 8), _Dev(ctx, X, 8)
    try:
        _alloc(ctx, ref, cfg)
        want = ref.results()
        _noalloc(ctx, got, cfg, with_coeffs=False)
        have = got.results()
    finally:
        ref.free()
        got.free()
    assert np.array_equal(want[0], have[0])
    # capacity: at this shape each vector needs ~16 KB of the 256 MiB scratch, so 40k is too many
    # (real buffers of the full size all the same, so nothing could read out of bounds)
    big = _Dev(ctx, np.zeros((40_000, 128), np.float32), 8)
    try:
        p = cfg.to_c()
        rc = ctx.lib.stlq_mi355_encode_device_noalloc(ctx.h, ctypes.c_void_p(big.X), 40_000, ctypes.byref(p),
                                                     ctypes.c_void_p(big.codes), None, None, None)
    finally:
        big.free()
    assert rc == 4, rc  # STLQ_MI355_ERR_UNSUPPORTED, refused before any launch
    msg = ctx.lib.stlq_mi355_last_error().decode()
    assert "no-allocation capacity" in msg, msg
