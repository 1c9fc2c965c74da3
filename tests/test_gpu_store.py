"""The streaming encode writing its BaseBasicStore on the device path
(stlq_mi355_encode_stream_store), against the reference's own io::BaseBasicWriter and checkpoint
hook (oracle/_ref) fed the oracle's encode of the same vectors in the same blocks: the store
files and the checkpoint are identical byte for byte. A run stopped after a committed block, cut
back to its checkpoint and resumed from it gives the same files as one uninterrupted run
(EncodeBaseStreaming's start_id + StreamingBasicCommitHook, encode_base_streaming.cpp:1913-2060;
stlq_large_base_stages.cpp:321-406)."""
import os

import numpy as np
import pytest

from oracle import ref
from stlq_amd import store as S
from stlq_amd.encoder import EncodeConfig
from tests.helpers import rvq_problem
from tests.test_gpu_parity import _lr_refit_problem, _oracle_encode

pytestmark = pytest.mark.gpu


def _files(root):
    out = {}
    for dp, _, fns in os.walk(root):
        for f in fns:
            p = os.path.join(dp, f)
            out[os.path.relpath(p, root)] = open(p, "rb").read()
    return out


def _same_tree(a, b):
    fa, fb = _files(a), _files(b)
    assert sorted(fa) == sorted(fb)
    for k in fa:
        assert fa[k] == fb[k], k


def _problem(ctx, orc, large_root, n):
    """Device codebooks set; returns (stream input, oracle blocks source, store cfg kwargs, stream kw)."""
    if large_root:
        p = _lr_refit_problem(ctx, orc, 5, 901, n=n, d=64, h0=1024, K=64)
        Xu8 = np.clip(np.rint(p["X"]), 0, 255).astype(np.uint8)
        Xf = Xu8.astype(np.float32)
        nx2 = orc.xnorm2(Xf)
        xs = orc.gemm_xc(p["Cs"], Xf, mode=1)
        cid, Bs, _ = orc.beam_search_large_root(Xf, nx2, p["C0"], p["norm0"], xs, p["Gs"], p["G0S"], p["h"], 4,
                                                root_mode=1)
        B_o, a_o, _, _ = orc.icm_ils_large_root(Xf, p["C0"], p["norm0"], xs, p["Gs"], p["G0S"], p["invs"], p["h"],
                                                cid, nx2, Bs, 1, 2, 3, True, 38251450, 0)
        res = (cid.astype(np.uint32), B_o, a_o, Xu8)
        store = dict(d=64, m=5, h_vec=list(p["h"]), shard_size=1400, bucket_flush_mb=1)
        kw = dict(input_u8=True, large_root=True, root_mode=1)
        return Xu8, res, store, kw, 1
    X, C = rvq_problem(902, n, 32, 5, 64, train_n=2000, iters=3)
    h = [64] * 5
    ctx.set_codebooks(C, h)
    codes, a, _ = _oracle_encode(orc, X, C, h, 4, icm_iters=1, ils_iters=2, perturb_k=3)
    res = (codes[:, 0].astype(np.uint32), codes[:, 1:], a, X)
    store = dict(d=32, m=5, h_vec=h, shard_size=1400, bucket_size=16, bucket_flush_mb=1, raw_bytes_per_vec=128)
    return X, res, store, {}, 2


CFG = EncodeConfig(H_beam=4, icm_iters=1, ils_iters=2, perturb_k=3, want_coeffs=True)


def _stream(ctx, root, X, store, kw, start, count, chunk, ckpt=True, resume=None):
    cfg = S.BaseBasicStoreConfig(dir=root, **store)
    w = S.BaseBasicWriter()
    assert (w.OpenResume(cfg, resume[0], resume[1]) if resume else w.Open(cfg)), w.err

    def fill(first, cnt, out):
        out[:] = X[first:first + cnt]

    S.encode_stream_store(ctx, w, count, chunk, CFG, fill, start_id=start,
                          checkpoint_path=S.BaseBasicCheckpointPath(root) if ckpt else None, **kw)
    assert w.Close(), w.err
    return cfg


@pytest.mark.skipif(not ref.available(), reason="reference build (oracle/_ref) not available")
@pytest.mark.parametrize("large_root", [False, True], ids=["full_precomp_f32", "large_root_u8"])
def test_stream_store_equals_reference_writer(ctx, orc, tmp_path, large_root):
    n, chunk = 4000, 700
    print(f"stream store vs reference writer large_root={large_root}", flush=True)
    X, (cid, Bs, a, raw), store, kw, raw_kind = _problem(ctx, orc, large_root, n)
    _stream(ctx, str(tmp_path / "ours"), X, store, kw, 0, n, chunk)
    blocks = [(s, cid[s:s + chunk], Bs[s:s + chunk], a[s:s + chunk], raw[s:s + chunk]) for s in range(0, n, chunk)]
    opts = {k: v for k, v in store.items() if k not in ("d", "m", "h_vec")}
    root = str(tmp_path / "ref")
    ok, err, _ = ref.store_write(root, store["d"], store["m"], store["h_vec"], blocks, raw_kind=raw_kind,
                                 ckpt_path=S.BaseBasicCheckpointPath(root), **opts)
    assert ok, err
    _same_tree(tmp_path / "ref", tmp_path / "ours")
    ck = S.ReadBaseBasicCheckpoint(S.BaseBasicCheckpointPath(root))
    assert ck.next_id == n and int(ck.bucket_sizes.sum()) == os.path.getsize(tmp_path / "ours" / "cluster_id.u32") \
        // 4 * (8 + (store.get("raw_bytes_per_vec") or store["d"]) + (store["m"] - 1) + 4 * store["m"])


@pytest.mark.parametrize("large_root", [False, True], ids=["full_precomp_f32", "large_root_u8"])
def test_stream_store_resume_after_stop(ctx, orc, tmp_path, large_root):
    n, chunk = 4000, 700
    print(f"stream store resume large_root={large_root}", flush=True)
    X, _, store, kw, _ = _problem(ctx, orc, large_root, n)
    _stream(ctx, str(tmp_path / "whole"), X, store, kw, 0, n, chunk)
    root = str(tmp_path / "resumed")
    cfg = _stream(ctx, root, X, store, kw, 0, 3 * chunk, chunk)  # stops after three committed blocks
    for f in ("cluster_id.u32", "codes_shard_0001.bin", "coeffs_shard_0001.bin", "bucket_0001.bin"):
        with open(os.path.join(root, f), "ab") as fh:  # a torn fourth block
            fh.write(b"\x5a" * 53)
    ck = S.ReadBaseBasicCheckpoint(S.BaseBasicCheckpointPath(root))
    assert ck.next_id == 3 * chunk
    S.TruncateBaseBasicToCheckpoint(cfg, ck)
    _stream(ctx, root, X, store, kw, ck.next_id, n - ck.next_id, chunk, resume=(ck.next_id, ck.bucket_sizes))
    _same_tree(tmp_path / "whole", tmp_path / "resumed")


def test_stream_store_refuses_mismatched_store(ctx, orc, tmp_path):
    X, _, store, kw, _ = _problem(ctx, orc, False, 700)
    bad = dict(store, m=4)
    cfg = S.BaseBasicStoreConfig(dir=str(tmp_path / "bad"), **bad)
    w = S.BaseBasicWriter()
    assert w.Open(cfg), w.err
    with pytest.raises(RuntimeError, match="differ from the codebooks"):
        S.encode_stream_store(ctx, w, 700, 700, CFG, lambda f, c, o: None, **kw)
    with pytest.raises(RuntimeError, match="multiple of large.base_block"):
        w2 = S.BaseBasicWriter()
        assert w2.Open(S.BaseBasicStoreConfig(dir=str(tmp_path / "b2"), **store))
        S.encode_stream_store(ctx, w2, 700, 700, CFG, lambda f, c, o: None, start_id=5,
                              checkpoint_path=str(tmp_path / "ck.bin"), **kw)
    w.Close()
