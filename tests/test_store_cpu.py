"""The BaseBasicStore writer and checkpoint helpers (host code, no GPU) against the reference's own
io::BaseBasicWriter (src/io/base_store.cpp) and app checkpoint helpers
(src/pipeline/main_virtual_helpers.cpp:100-297), compiled into oracle/_ref: the same blocks
written by both must give the same files, byte for byte, and the same committed bucket bytes."""
import filecmp
import os

import numpy as np
import pytest

from oracle import ref
from stlq_amd import store as S

pytestmark = pytest.mark.skipif(not ref.available(), reason="reference build (oracle/_ref) not available")


def _files(root):
    out = {}
    for dp, _, fns in os.walk(root):
        for f in fns:
            p = os.path.join(dp, f)
            out[os.path.relpath(p, root)] = open(p, "rb").read()
    return out


def _blocks(seed, n, d, m, cid_hi, block, start=0, raw="u8"):
    rng = np.random.default_rng(seed)
    cid = rng.integers(0, cid_hi, n).astype(np.uint32)
    B = rng.integers(0, 256, (n, max(0, m - 1))).astype(np.uint8)
    a = rng.standard_normal((n, m)).astype(np.float32)
    X = (rng.integers(0, 256, (n, d)).astype(np.uint8) if raw == "u8"
         else rng.standard_normal((n, d)).astype(np.float32) if raw == "f32" else None)
    out = []
    for s in range(0, n, block):
        e = min(n, s + block)
        out.append((start + s, cid[s:e], B[s:e], a[s:e], None if X is None else X[s:e]))
    return out


def _ours(dir, d, m, h_vec, blocks, kind, resume=None, ckpt=None, **cfg):
    c = S.BaseBasicStoreConfig(dir=dir, d=d, m=m, h_vec=list(h_vec), **cfg)
    w = S.BaseBasicWriter()
    ok = w.OpenResume(c, resume[0], resume[1]) if resume else w.Open(c)
    assert ok, w.err
    for (start, cid, B, a, X) in blocks:
        fn = {0: lambda: w.AppendBlock(start, cid, B, a),
              1: lambda: w.AppendBlockRawU8(start, cid, B, a, X),
              2: lambda: w.AppendBlockRawF32(start, cid, B, a, X),
              3: lambda: w.AppendBlock(start, cid, B, a, X)}[kind]
        if not fn():
            return False, w.err, None
        if ckpt:
            assert w.Flush(), w.err
            S.WriteBaseBasicCheckpointAtomic(ckpt, S.BaseBasicCheckpoint(start + len(cid), w.bucket_file_bytes()))
    assert w.Close(), w.err
    return True, "", w.bucket_file_bytes()


# name: d, m, h_vec, n, block, kind (0 none, 1 u8, 2 f32, 3 u8 matrix), cid range, start id, store options
CASES = [
    ("u8_default", 16, 4, [1000, 16, 16, 16], 2100, 300, 1, 1000, 0, dict(shard_size=600)),
    ("u8_matrix", 16, 4, [1000, 16, 16, 16], 900, 300, 3, 1000, 0, dict(shard_size=600)),
    ("f32_raw", 24, 5, [700, 8, 8, 8, 8], 1500, 250, 2, 700, 0, dict(shard_size=500, raw_bytes_per_vec=96)),
    ("no_buckets", 16, 4, [1000, 16, 16, 16], 1200, 300, 0, 1000, 0,
     dict(write_vector_bucket=False, write_basic_to_bucket=False)),
    ("basic_only", 16, 4, [1000, 16, 16, 16], 1200, 300, 0, 1000, 0, dict(write_vector_bucket=False)),
    ("vector_only", 16, 4, [1000, 16, 16, 16], 1200, 300, 1, 1000, 0, dict(write_basic_to_bucket=False)),
    ("shard_crossing", 16, 4, [1000, 16, 16, 16], 2000, 300, 1, 1000, 0, dict(shard_size=500)),
    ("flush_mid_stream", 128, 4, [1024, 16, 16, 16], 12000, 3000, 2, 1024, 0,
     dict(bucket_flush_mb=1, raw_bytes_per_vec=512)),
    ("ids_beyond_layout", 16, 4, [1000, 16, 16, 16], 1200, 300, 1, 1600, 0, {}),
    ("bucket_size_zero", 8, 3, [20, 16, 16], 600, 200, 1, 20, 0, dict(bucket_size=0)),
    ("empty_h_vec", 8, 3, [], 600, 200, 1, 700, 0, {}),
    ("m1_root_only", 8, 1, [300], 600, 200, 1, 300, 0, dict(bucket_size=100)),
    ("start_id_offset", 16, 4, [1000, 16, 16, 16], 900, 300, 1, 1000, 5_000_000, {}),
]


@pytest.mark.parametrize("name,d,m,h_vec,n,block,kind,cid_hi,start,opts", CASES, ids=[c[0] for c in CASES])
def test_store_bytes_match_reference(tmp_path, name, d, m, h_vec, n, block, kind, cid_hi, start, opts):
    raw = {0: None, 1: "u8", 2: "f32", 3: "u8"}[kind]
    blocks = _blocks(hash(name) & 0xFFFF, n, d, m, cid_hi, block, start, raw)
    ok_r, err_r, sizes_r = ref.store_write(str(tmp_path / "ref"), d, m, h_vec, blocks, raw_kind=kind, **opts)
    assert ok_r, err_r
    ok_o, err_o, sizes_o = _ours(str(tmp_path / "ours"), d, m, h_vec, blocks, kind, **opts)
    assert ok_o, err_o
    fr, fo = _files(tmp_path / "ref"), _files(tmp_path / "ours")
    assert sorted(fr) == sorted(fo)
    for k in fr:
        assert fr[k] == fo[k], k
    assert np.array_equal(sizes_r, sizes_o)
    if kind and opts.get("write_vector_bucket", True):  # the records hold the raw vectors
        assert sum(len(v) for k, v in fo.items() if k.startswith("bucket_")) >= n * d


def test_checkpoint_resume_matches_reference_and_one_shot(tmp_path):
    d, m, h_vec = 16, 4, [1000, 16, 16, 16]
    blocks = _blocks(7, 3000, d, m, 1000, 250, 0, "u8")
    opts = dict(shard_size=1000, bucket_flush_mb=1)
    # one-shot stores
    assert ref.store_write(str(tmp_path / "ref_full"), d, m, h_vec, blocks, raw_kind=1, **opts)[0]
    assert _ours(str(tmp_path / "ours_full"), d, m, h_vec, blocks, 1, **opts)[0]
    k = 5  # blocks 0..k-1 committed, block k half-written when the run stops
    for who in ("ref", "ours"):
        root = str(tmp_path / who)
        ck = S.BaseBasicCheckpointPath(root)
        if who == "ref":
            assert ref.store_write(root, d, m, h_vec, blocks[:k], raw_kind=1, ckpt_path=ck, **opts)[0]
        else:
            assert _ours(root, d, m, h_vec, blocks[:k], 1, ckpt=ck, **opts)[0]
        for f in ("cluster_id.u32", "codes_shard_0001.bin", "coeffs_shard_0001.bin", "bucket_0002.bin"):
            with open(os.path.join(root, f), "ab") as fh:  # torn writes past the checkpoint
                fh.write(b"\xa5" * 37)
        if who == "ref":
            ok, err, nid, sizes = ref.store_truncate(root, m, h_vec, ck, shard_size=opts["shard_size"])
            assert ok, err
            ok, err, _ = ref.store_write(root, d, m, h_vec, blocks[k:], raw_kind=1, resume_start=nid,
                                         bucket_sizes=sizes, ckpt_path=ck, **opts)
            assert ok, err
        else:
            c = S.BaseBasicStoreConfig(dir=root, d=d, m=m, h_vec=h_vec, **opts)
            got = S.ReadBaseBasicCheckpoint(ck)
            S.TruncateBaseBasicToCheckpoint(c, got)
            assert _ours(root, d, m, h_vec, blocks[k:], 1, resume=(got.next_id, got.bucket_sizes), ckpt=ck, **opts)[0]
        assert S.ReadBaseBasicCheckpoint(ck).next_id == 3000
    fr, fo = _files(tmp_path / "ref"), _files(tmp_path / "ours")
    assert sorted(fr) == sorted(fo)
    for key in fr:
        assert fr[key] == fo[key], key
    full = _files(tmp_path / "ours_full")
    resumed = {k2: v for k2, v in fo.items() if not k2.startswith("checkpoint")}
    assert sorted(full) == sorted(resumed)
    for key in full:
        assert full[key] == resumed[key], key
    assert filecmp.cmp(tmp_path / "ref_full" / "meta.bin", tmp_path / "ours" / "meta.bin", shallow=False)


def test_checkpoint_file_format(tmp_path):
    p = str(tmp_path / "x" / "ckpt.bin")
    sizes = np.array([0, 5, 1 << 40, 7], np.uint64)
    S.WriteBaseBasicCheckpointAtomic(p, S.BaseBasicCheckpoint(123456789012, sizes))
    raw = open(p, "rb").read()
    head = np.frombuffer(raw[:16], np.uint32)
    assert head.tolist() == [0x544B4342, 1, 4, 0]  # "BCKT", version 1, nbucket, reserved
    assert np.frombuffer(raw[16:24], np.uint64)[0] == 123456789012
    assert np.array_equal(np.frombuffer(raw[24:], np.uint64), sizes)
    back = S.ReadBaseBasicCheckpoint(p)
    assert back.next_id == 123456789012 and np.array_equal(back.bucket_sizes, sizes)
    assert not os.path.exists(p + ".tmp")
    with open(p, "r+b") as fh:
        fh.write(b"XXXX")
    with pytest.raises(RuntimeError, match="magic"):
        S.ReadBaseBasicCheckpoint(p)


def test_store_errors_match_reference(tmp_path):
    d, m, h_vec = 8, 3, [512, 16, 16]
    good = _blocks(3, 100, d, m, 512, 100, 0, "u8")
    # raw vectors required but not given (AppendBlock without x): both write the block's ids,
    # codes and coefficients, then fail.
    ok_r, err_r, _ = ref.store_write(str(tmp_path / "r1"), d, m, h_vec, good, raw_kind=0)
    ok_o, err_o, _ = _ours(str(tmp_path / "o1"), d, m, h_vec, good, 0)
    assert not ok_r and not ok_o and "write_vector_bucket" in err_r and "write_vector_bucket" in err_o
    for f in ("cluster_id.u32", "codes_shard_0000.bin", "coeffs_shard_0000.bin"):
        assert os.path.getsize(tmp_path / "r1" / f) == os.path.getsize(tmp_path / "o1" / f) > 0
    # raw bytes of float records, uint8 append: both refuse before writing anything.
    ok_r, err_r, _ = ref.store_write(str(tmp_path / "r2"), d, m, h_vec, good, raw_kind=1, raw_bytes_per_vec=4 * d)
    ok_o, err_o, _ = _ours(str(tmp_path / "o2"), d, m, h_vec, good, 1, raw_bytes_per_vec=4 * d)
    assert not ok_r and not ok_o
    for f in ("cluster_id.u32",):
        assert os.path.getsize(tmp_path / "r2" / f) == os.path.getsize(tmp_path / "o2" / f) == 0
    # wrong coefficient rows (the reference's B/a shape check, base_store.cpp:424-430)
    bad = [(0, good[0][1], good[0][2], good[0][3][:, :2], good[0][4])]
    ok_o, err_o, _ = _ours(str(tmp_path / "o3"), d, m, h_vec, bad, 1)
    assert not ok_o and "shape" in err_o
    assert os.path.getsize(tmp_path / "o3" / "cluster_id.u32") == 0
    # resume with the wrong bucket count
    c = S.BaseBasicStoreConfig(dir=str(tmp_path / "o1"), d=d, m=m, h_vec=h_vec)
    w = S.BaseBasicWriter()
    assert not w.OpenResume(c, 100, [0, 0, 0]) and "bucket_sizes" in w.err
    ok_r, err_r, _ = ref.store_write(str(tmp_path / "r1"), d, m, h_vec, good, raw_kind=1, resume_start=100,
                                     bucket_sizes=np.zeros(3, np.uint64))
    assert not ok_r and "bucket_sizes" in err_r
    # invalid config
    assert not w.Open(S.BaseBasicStoreConfig(dir="", d=d, m=m, h_vec=h_vec))
    assert not w.Open(S.BaseBasicStoreConfig(dir=str(tmp_path / "o4"), d=0, m=m, h_vec=h_vec))
