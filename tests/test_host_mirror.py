"""The C++ host mirror of the reference's encoder interface (stlq_amd/host/stlq_mi355.hpp).

tests/host_mirror_check.cpp drives the reference-named functions (BuildPrecomp, BeamSearchPrefixLS,
ComputeXNorm2, DynamicIcmWithIls*NoNormal, EncodeBase, BuildPrecompLargeRoot,
BeamSearchPrefixLSLargeRoot, EncodeBaseStreamingF32 over a reader/writer pair) on arrays handed
over from here; the GPU tests compare what they
return with the oracle, bit for bit, so a transposed operand or a misplaced argument in the
mirror's plumbing fails them.
"""
import ctypes
import os

import numpy as np
import pytest

from tests.helpers import rvq_problem

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOSTCHECK = os.path.join(ROOT, "stlq_amd", "lib", "libstlq_mi355_hostcheck.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i32p = ctypes.POINTER(ctypes.c_int32)


def _lib():
    if not os.path.exists(HOSTCHECK):
        pytest.fail(f"{HOSTCHECK} is not built (python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(HOSTCHECK)
    lib.mirror_encode.restype = ctypes.c_int
    lib.mirror_encode.argtypes = [ctypes.c_int, ctypes.c_int, _i32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, ctypes.c_int, ctypes.c_uint32, _f32p, _u8p, _u8p, _f32p, _f32p,
                                  _f32p, ctypes.c_char_p, ctypes.c_int]
    lib.mirror_large_root.restype = ctypes.c_int
    lib.mirror_large_root.argtypes = [ctypes.c_int, ctypes.c_int, _i32p, _f32p, _f32p, _f32p, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, _u32p, _u8p, _f32p, _f32p,
                                      ctypes.c_char_p, ctypes.c_int]
    lib.mirror_stream.restype = ctypes.c_int
    lib.mirror_stream.argtypes = [ctypes.c_int, ctypes.c_int, _i32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint64,
                                  ctypes.c_int, ctypes.c_int, _u32p, _u8p, _f32p, _f32p, _f32p, _i32p,
                                  ctypes.c_char_p, ctypes.c_int]
    return lib


def _p(a, t):
    return a.ctypes.data_as(t)


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def test_hostcheck_library_loads():
    lib = _lib()
    assert lib.mirror_encode is not None and lib.mirror_large_root is not None and lib.mirror_stream is not None


def _stream(d, m, h, C_all, X, n, large, Hb, icm, ils, block, start_id, write_raw, use_hook):
    cid = np.full(n, 0xFFFFFFFF, np.uint32)
    Bs = np.zeros((n, max(m - 1, 0)), np.uint8)
    a = np.zeros((n, m), np.float32)
    raw = np.zeros((n, d), np.float32)
    mse = np.zeros(2, np.float32)
    calls = np.zeros(1, np.int32)
    err = ctypes.create_string_buffer(512)
    rc = _lib().mirror_stream(d, m, _p(h, _i32p), _p(C_all, _f32p), _p(X, _f32p), n, large, Hb, icm, ils, block,
                              start_id, write_raw, use_hook, _p(cid, _u32p), _p(Bs, _u8p), _p(a, _f32p),
                              _p(raw, _f32p), _p(mse, _f32p), _p(calls, _i32p), err, 512)
    return rc, err.value.decode(), dict(cid=cid, Bs=Bs, a=a, raw=raw, mse=mse, calls=int(calls[0]))


@pytest.mark.parametrize("start_id,block,hook,msg", [(101, 50, 0, "start_id out of range"),
                                                     (30, 50, 1, "multiple of large.base_block")])
def test_mirror_stream_rejects_bad_start(start_id, block, hook, msg):
    """EncodeBaseStreamingF32's argument checks (encode_base_streaming.cpp:4551-4579) run before
    any device work: m = 0 here builds no precomp."""
    d, n = 8, 100
    h = np.zeros(1, np.int32)
    C = np.zeros(1, np.float32)
    X = np.zeros((n, d), np.float32)
    rc, err, _ = _stream(d, 0, h, C, X, n, 1, 4, 0, 0, block, start_id, 1, hook)
    assert rc == 1 and msg in err, (rc, err)


@pytest.mark.gpu
@pytest.mark.parametrize("icm_iters,use_abs", [(0, 1), (2, 1), (2, 0)])
def test_mirror_encode_matches_oracle(orc, icm_iters, use_abs):
    n, d, m, K, Hb, seed = 3000, 48, 5, 64, 6, 38251450
    X, C = rvq_problem(71 + icm_iters + use_abs, n, d, m, K)
    h = np.full(m, K, np.int32)
    G = np.empty((C.shape[0], C.shape[0]), np.float32)
    cb = np.empty((n, m), np.uint8)
    cf = np.empty((n, m), np.uint8)
    a = np.empty((n, m), np.float32)
    cost = np.empty(n, np.float32)
    mse = np.empty(2, np.float32)
    err = ctypes.create_string_buffer(512)
    C = np.ascontiguousarray(C, np.float32)
    X = np.ascontiguousarray(X, np.float32)
    print(f"mirror_encode n={n} d={d} m={m} K={K} beam={Hb} icm={icm_iters} abs={use_abs}", flush=True)
    rc = _lib().mirror_encode(d, m, _p(h, _i32p), _p(C, _f32p), _p(X, _f32p), n, Hb, icm_iters, use_abs, seed,
                              _p(G, _f32p), _p(cb, _u8p), _p(cf, _u8p), _p(a, _f32p), _p(cost, _f32p),
                              _p(mse, _f32p), err, 512)
    assert rc == 0, err.value.decode()
    G_o, inv_o = orc.build_precomp(C, h)
    assert np.array_equal(_bits(G_o), _bits(G))
    nx2 = orc.xnorm2(X)
    xC = orc.gemm_xc(C, X, mode=1)
    codes_o, _ = orc.beam_search(nx2, xC, G_o, h, Hb)
    assert np.array_equal(codes_o, cb)
    codes_f, a_o, cost_o, _ = orc.icm(xC, G_o, inv_o, h, nx2, codes_o, icm_iters, use_abs, seed)
    assert np.array_equal(codes_f, cf)
    assert np.array_equal(_bits(a_o), _bits(a))
    assert np.array_equal(_bits(cost_o), _bits(cost))
    want = np.float32(np.mean(np.maximum(cost_o.astype(np.float64), 0.0)))
    assert abs(mse[1] - want) <= 1e-6 * abs(want)


@pytest.mark.gpu
def test_mirror_large_root_matches_oracle(orc):
    from stlq_amd import workloads

    n, d, h0, K, m, Hb, seed = 2000, 32, 1500, 64, 4, 8, 93
    mix = workloads.Mixture("desc", d, 256, seed)
    rng = np.random.default_rng(seed)
    C0 = mix.sample(5_000_000, h0)
    Xtr = mix.sample(1_000_000, 3000)
    Cs = workloads.residual_codebooks(Xtr - C0[rng.integers(0, h0, 3000)], m - 1, K, 3, seed + 1)
    X = mix.sample(0, n)
    h = np.array([h0] + [K] * (m - 1), np.int32)
    cid = np.empty(n, np.uint32)
    Bs = np.empty((n, m - 1), np.uint8)
    err = ctypes.create_string_buffer(512)
    print(f"mirror_large_root n={n} d={d} h0={h0} K={K} m={m} beam={Hb}", flush=True)
    a = np.empty((n, m), np.float32)
    cost = np.empty(n, np.float32)
    rc = _lib().mirror_large_root(d, m, _p(h, _i32p), _p(C0, _f32p), _p(Cs, _f32p), _p(X, _f32p), n, Hb, 1, 2,
                                  _p(cid, _u32p), _p(Bs, _u8p), _p(a, _f32p), _p(cost, _f32p), err, 512)
    assert rc == 0, err.value.decode()
    norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs)
    nx2 = orc.xnorm2(X)
    xs = orc.gemm_xc(Cs, X, mode=1)
    cid_o, Bs_o, _ = orc.beam_search_large_root(X, nx2, C0, norm0, xs, Gs, G0S, list(h), Hb)
    assert np.array_equal(cid_o, cid)
    B_o, a_o, c_o, _ = orc.icm_ils_large_root(X, C0, norm0, xs, Gs, G0S, orc.invnorm_small(Cs), list(h), cid_o, nx2,
                                              Bs_o, 1, 2, 3, True, 38251450, 0)
    assert np.array_equal(B_o, Bs)
    assert np.array_equal(_bits(a_o), _bits(a))
    assert np.array_equal(_bits(c_o), _bits(cost))


def _stream_problem(large):
    from stlq_amd import workloads

    n, d, K, m, seed = 1800, 32, 64, 4, 95
    mix = workloads.Mixture("desc", d, 256, seed)
    rng = np.random.default_rng(seed)
    if large:
        h0 = 1200
        C0 = mix.sample(5_000_000, h0)
        Xtr = mix.sample(1_000_000, 3000)
        Cs = workloads.residual_codebooks(Xtr - C0[rng.integers(0, h0, 3000)], m - 1, K, 3, seed + 1)
        C_all = np.ascontiguousarray(np.concatenate([C0, Cs]), np.float32)
        h = np.array([h0] + [K] * (m - 1), np.int32)
    else:
        C_all = np.ascontiguousarray(workloads.residual_codebooks(mix.sample(1_000_000, 3000), m, K, 3, seed + 1),
                                     np.float32)
        h = np.full(m, K, np.int32)
    X = np.ascontiguousarray(mix.sample(0, n), np.float32)
    return n, d, m, h, C_all, X


@pytest.mark.gpu
@pytest.mark.parametrize("large", [1, 0], ids=["large_root", "full_precomp"])
def test_mirror_stream_matches_oracle_and_resumes(orc, large):
    """EncodeBaseStreamingF32 through the mirror: blocks reach the writer in id order with the raw
    tiles, the commit hook sees every block, the records equal the oracle's encode (large root:
    beam + ICM + ILS keyed by global id; full precomp: layer 0's code as the cluster id), and a run
    resumed at start_id = 2 blocks writes the same records for the ids it covers."""
    n, d, m, h, C_all, X = _stream_problem(large)
    Hb, icm, ils, block = 8, 1, (2 if large else 0), 400
    print(f"mirror_stream large={large} n={n} d={d} h={list(h)} beam={Hb} icm={icm} ils={ils}", flush=True)
    rc, err, full = _stream(d, m, h, C_all, X, n, large, Hb, icm, ils, block, 0, 1, 1)
    assert rc == 0, err
    assert full["calls"] == (n + block - 1) // block
    assert np.array_equal(full["raw"], X)
    nx2 = orc.xnorm2(X)
    if large:
        C0, Cs = C_all[:h[0]], C_all[h[0]:]
        norm0, Gs, G0S = orc.build_precomp_large_root(C0, Cs)
        xs = orc.gemm_xc(Cs, X, mode=1)
        # the streamed beam forces the nearest root (root_mode 1), as the reference's device beams do
        cid_o, Bs_o, _ = orc.beam_search_large_root(X, nx2, C0, norm0, xs, Gs, G0S, list(h), Hb, root_mode=1)
        B_o, a_o, c_o, _ = orc.icm_ils_large_root(X, C0, norm0, xs, Gs, G0S, orc.invnorm_small(Cs), list(h), cid_o,
                                                  nx2, Bs_o, icm, ils, 3, True, 38251450, 0)
        assert np.array_equal(cid_o, full["cid"])
        assert np.array_equal(B_o, full["Bs"])
    else:
        G_o, inv_o = orc.build_precomp(C_all, h)
        xC = orc.gemm_xc(C_all, X, mode=1)
        codes_o, _ = orc.beam_search(nx2, xC, G_o, h, Hb)
        codes_f, a_o, c_o, _ = orc.icm(xC, G_o, inv_o, h, nx2, codes_o, icm, True, 38251450)
        assert np.array_equal(codes_f[:, 0].astype(np.uint32), full["cid"])
        assert np.array_equal(codes_f[:, 1:], full["Bs"])
    assert np.array_equal(_bits(a_o), _bits(full["a"]))
    want = np.float32(np.mean(np.maximum(c_o.astype(np.float64), 0.0)))
    assert abs(full["mse"][1] - want) <= 1e-6 * abs(want)

    start = 2 * block
    rc, err, part = _stream(d, m, h, C_all, X, n, large, Hb, icm, ils, block, start, 0, 1)
    assert rc == 0, err
    assert part["calls"] == (n - start + block - 1) // block
    assert np.all(part["cid"][:start] == 0xFFFFFFFF)
    for key in ("cid", "Bs", "a"):
        assert np.array_equal(part[key][start:], full[key][start:]), key
    assert not part["raw"].any()  # write_vector_bucket off: AppendBlock without the raw tile


def _stream_store(root, d, m, h, C_all, X, u8, n, large, Hb, icm, ils, block, shard, bucket, resume=0, stop_at=0):
    lib = _lib()
    lib.mirror_stream_store.restype = ctypes.c_int
    lib.mirror_stream_store.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, _i32p, _f32p, ctypes.c_void_p] + \
        [ctypes.c_int] * 14 + [ctypes.c_char_p, ctypes.c_int]
    err = ctypes.create_string_buffer(512)
    rc = lib.mirror_stream_store(str(root).encode(), d, m, _p(h, _i32p), _p(C_all, _f32p),
                                 X.ctypes.data_as(ctypes.c_void_p), int(u8), n, large, Hb, icm, ils, block, shard,
                                 bucket, 1, 1, 1, resume, stop_at, err, 512)
    return rc, err.value.decode()


def _tree(root):
    out = {}
    for dp, _, fns in os.walk(root):
        for f in fns:
            out[os.path.relpath(os.path.join(dp, f), root)] = open(os.path.join(dp, f), "rb").read()
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("large", [1, 0], ids=["large_root_u8", "full_precomp_f32"])
def test_mirror_stream_store_matches_c_abi_and_resumes(ctx, tmp_path, large):
    """EncodeBaseStreaming[F32] through the mirror into io::BaseBasicWriter with the pipeline's
    checkpoint hook writes the same store, byte for byte, as stlq_mi355_encode_stream_store; a run
    stopped after two blocks, resumed through ReadBaseBasicCheckpoint + TruncateBaseBasicToCheckpoint
    + OpenResume, ends with the same files as the uninterrupted one (checkpoint included)."""
    from stlq_amd import store as S
    from stlq_amd.encoder import EncodeConfig

    n, d, m, h, C_all, X = _stream_problem(large)
    Hb, icm, ils, block, shard, bucket = 8, 1, 2, 400, 800, 300
    if large:
        X = np.clip(np.rint(X), 0, 255).astype(np.uint8)
    print(f"mirror stream store large={large} n={n}", flush=True)
    rc, err = _stream_store(tmp_path / "mirror", d, m, h, C_all, X, large, n, large, Hb, icm, ils, block, shard, bucket)
    assert rc == 0, err
    if large:
        ctx.set_large_root(C_all[:h[0]], C_all[h[0]:], list(h))
    else:
        ctx.set_codebooks(C_all, list(h))
    cfg = S.BaseBasicStoreConfig(dir=str(tmp_path / "abi"), d=d, m=m, h_vec=list(h), shard_size=shard,
                                 bucket_size=bucket, bucket_flush_mb=1,
                                 raw_bytes_per_vec=d if large else 4 * d)
    w = S.BaseBasicWriter()
    assert w.Open(cfg), w.err

    def fill(first, cnt, out):
        out[:] = X[first:first + cnt]

    S.encode_stream_store(ctx, w, n, block, EncodeConfig(H_beam=Hb, icm_iters=icm, ils_iters=ils), fill,
                          input_u8=bool(large), large_root=bool(large), root_mode=1,
                          checkpoint_path=S.BaseBasicCheckpointPath(str(tmp_path / "abi")))
    assert w.Close(), w.err
    a, b = _tree(tmp_path / "mirror"), _tree(tmp_path / "abi")
    assert sorted(a) == sorted(b)
    for k in a:
        assert a[k] == b[k], k
    root = tmp_path / "resumed"
    rc, err = _stream_store(root, d, m, h, C_all, X, large, n, large, Hb, icm, ils, block, shard, bucket,
                            stop_at=2 * block)
    assert rc == 0, err
    with open(root / "cluster_id.u32", "ab") as fh:
        fh.write(b"\x01" * 40)
    rc, err = _stream_store(root, d, m, h, C_all, X, large, n, large, Hb, icm, ils, block, shard, bucket, resume=1)
    assert rc == 0, err
    c = _tree(root)
    assert sorted(a) == sorted(c)
    for k in a:
        assert a[k] == c[k], k
