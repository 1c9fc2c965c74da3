"""The BaseBasicStore output of the streaming encode, over the C ABI of include/stlq_mi355_store.h.

Mirrors the reference's io::BaseBasicWriter (include/stlq/io/base_store.h:28-100) and the
pipeline's checkpoint helpers (include/stlq/pipeline/main_virtual_helpers.h:35-69): the same
names, argument meaning and failure behaviour (methods return False and set `err`), writing the
same files byte for byte.

Array conventions: numpy row-major (n, k) is the reference's column-major k x n, so
cluster_id (n,), B_small (n, m-1), a (n, m) and raw vectors (n, d).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import StoreConfig, StreamParams, StreamStats, check

_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int)


@dataclass
class BaseBasicStoreConfig:
    """io::BaseBasicStoreConfig (include/stlq/io/base_store.h:12-25), with its defaults."""

    dir: str = ""
    d: int = 0
    m: int = 0
    h_vec: list = field(default_factory=list)
    shard_size: int = 2000000
    bucket_size: int = 256
    bucket_flush_mb: int = 256
    write_vector_bucket: bool = True
    write_basic_to_bucket: bool = True
    raw_bytes_per_vec: int = 0

    def to_c(self):
        hv = np.ascontiguousarray(self.h_vec, dtype=np.int32)
        c = StoreConfig(self.dir.encode(), int(self.d), int(self.m), hv.ctypes.data_as(_i32p), len(hv),
                        int(self.shard_size), int(self.bucket_size), int(self.bucket_flush_mb),
                        int(bool(self.write_vector_bucket)), int(bool(self.write_basic_to_bucket)),
                        int(self.raw_bytes_per_vec))
        return c, hv  # hv keeps the h_vec buffer alive while c is used


def _err():
    return _lib.load().stlq_mi355_last_error().decode(errors="replace")


def _ptr(a, t):
    return None if a is None else a.ctypes.data_as(t)


class BaseBasicWriter:
    """io::BaseBasicWriter. After a False return, `err` holds the message."""

    def __init__(self):
        self.lib = _lib.load()
        self.h = None
        self.err = ""
        self._closed_bytes = np.zeros(0, np.uint64)

    def _ok(self, rc):
        if rc != 0:
            self.err = _err()
            return False
        return True

    def Open(self, cfg: BaseBasicStoreConfig) -> bool:
        self.Close()
        c, _hv = cfg.to_c()
        h = ctypes.c_void_p()
        ok = self._ok(self.lib.stlq_mi355_store_open(ctypes.byref(c), ctypes.byref(h)))
        self.h = h.value if ok else None
        return ok

    def OpenResume(self, cfg: BaseBasicStoreConfig, start_id: int, bucket_sizes) -> bool:
        self.Close()
        c, _hv = cfg.to_c()
        sizes = np.ascontiguousarray(bucket_sizes, dtype=np.uint64)
        h = ctypes.c_void_p()
        ok = self._ok(self.lib.stlq_mi355_store_open_resume(ctypes.byref(c), int(start_id), _ptr(sizes, _u64p),
                                                            len(sizes), ctypes.byref(h)))
        self.h = h.value if ok else None
        return ok

    def _append(self, start_id, cluster_id, B_small, a, kind, raw):
        cid = np.ascontiguousarray(cluster_id, dtype=np.uint32)
        n = len(cid)
        B = np.ascontiguousarray(B_small, dtype=np.uint8)
        A = np.ascontiguousarray(a, dtype=np.float32)
        if B.ndim != 2 or A.ndim != 2 or B.shape[0] != n or A.shape[0] != n:
            self.err = "AppendBlock: B/a shape mismatch."
            return False
        rawp, ld = None, 0
        if raw is not None:
            raw = np.ascontiguousarray(raw)
            rawp, ld = raw.ctypes.data_as(ctypes.c_void_p), raw.shape[1]
        return self._ok(self.lib.stlq_mi355_store_append(self.h, int(start_id), n, _ptr(cid, _u32p), B.shape[1],
                                                         _ptr(B, _u8p), A.shape[1], _ptr(A, _f32p), kind, rawp, ld))

    def AppendBlock(self, start_id, cluster_id, B_small, a, x_u8_optional=None) -> bool:
        if x_u8_optional is None:
            return self._append(start_id, cluster_id, B_small, a, _lib_raw("NONE"), None)
        x = np.asarray(x_u8_optional, dtype=np.uint8)
        if x.shape != (len(cluster_id), x.shape[1]):
            self.err = "AppendBlock: x_u8 shape mismatch."
            return False
        return self._append(start_id, cluster_id, B_small, a, _lib_raw("U8"), x)

    def AppendBlockRawU8(self, start_id, cluster_id, B_small, a, x_u8) -> bool:
        return self._append(start_id, cluster_id, B_small, a, _lib_raw("U8"),
                            None if x_u8 is None else np.asarray(x_u8, dtype=np.uint8))

    def AppendBlockRawF32(self, start_id, cluster_id, B_small, a, x_f32) -> bool:
        return self._append(start_id, cluster_id, B_small, a, _lib_raw("F32"),
                            None if x_f32 is None else np.asarray(x_f32, dtype=np.float32))

    def Flush(self) -> bool:
        return self._ok(self.lib.stlq_mi355_store_flush(self.h))

    def bucket_file_bytes(self):
        if self.h is None:  # after Close: the bytes committed when it closed
            return self._closed_bytes.copy()
        nb = ctypes.c_int64()
        check(self.lib.stlq_mi355_store_bucket_bytes(self.h, None, 0, ctypes.byref(nb)))
        out = np.zeros(nb.value, np.uint64)
        check(self.lib.stlq_mi355_store_bucket_bytes(self.h, _ptr(out, _u64p), nb.value, ctypes.byref(nb)))
        return out

    def Close(self) -> bool:
        if self.h is None:
            return True
        # Writing out the bucket buffers first (what Close does itself) keeps the committed bytes
        # readable after the store is freed, as the reference's writer object keeps them.
        ok = self._ok(self.lib.stlq_mi355_store_flush(self.h))
        if ok:
            self._closed_bytes = self.bucket_file_bytes()
        h, self.h = self.h, None
        return self._ok(self.lib.stlq_mi355_store_close(h)) and ok

    def __del__(self):
        try:
            self.Close()
        except Exception:
            pass


def _lib_raw(kind):
    return {"NONE": 0, "U8": 1, "F32": 2}[kind]


# ---- checkpoint helpers (src/pipeline/main_virtual_helpers.cpp:100-297) ----

@dataclass
class BaseBasicCheckpoint:
    next_id: int = 0
    bucket_sizes: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint64))

    @property
    def nbucket(self):
        return len(self.bucket_sizes)


def ComputeNbucketsForBasic(cfg: BaseBasicStoreConfig) -> int:
    h0 = cfg.h_vec[0] if len(cfg.h_vec) else 0
    bs = max(1, cfg.bucket_size)
    return (h0 + bs - 1) // bs if h0 > 0 else 0


def BaseBasicCheckpointPath(base_basic_dir: str) -> str:
    return os.path.join(base_basic_dir, "checkpoint", "base_basic", "ckpt.bin")


def WriteBaseBasicCheckpointAtomic(path: str, ck: BaseBasicCheckpoint):
    sizes = np.ascontiguousarray(ck.bucket_sizes, dtype=np.uint64)
    check(_lib.load().stlq_mi355_checkpoint_write(path.encode(), int(ck.next_id), _ptr(sizes, _u64p), len(sizes)))


def ReadBaseBasicCheckpoint(path: str) -> BaseBasicCheckpoint:
    lib = _lib.load()
    nid, nb = ctypes.c_uint64(), ctypes.c_int64()
    check(lib.stlq_mi355_checkpoint_read(path.encode(), ctypes.byref(nid), None, 0, ctypes.byref(nb)))
    sizes = np.zeros(nb.value, np.uint64)
    check(lib.stlq_mi355_checkpoint_read(path.encode(), ctypes.byref(nid), _ptr(sizes, _u64p), nb.value,
                                         ctypes.byref(nb)))
    return BaseBasicCheckpoint(int(nid.value), sizes)


def TruncateBaseBasicToCheckpoint(cfg: BaseBasicStoreConfig, ck: BaseBasicCheckpoint):
    c, _hv = cfg.to_c()
    sizes = np.ascontiguousarray(ck.bucket_sizes, dtype=np.uint64)
    check(_lib.load().stlq_mi355_store_truncate_to_checkpoint(ctypes.byref(c), int(ck.next_id),
                                                              _ptr(sizes, _u64p), len(sizes)))


def encode_stream_store(ctx, writer: BaseBasicWriter, n_total, chunk, cfg, fill, input_u8=False,
                        large_root=False, root_mode=1, R=None, start_id=0, checkpoint_path=None):
    """EncodeBaseStreaming[F32] into `writer` (stlq_mi355_encode_stream_store): each chunk of
    `chunk` vectors is one block, committed (flush + checkpoint) when checkpoint_path is set.
    fill(first, count, out) as in Context.encode_stream. Returns the stream statistics."""
    d = ctx.lr[0] if large_root else ctx.d
    dt = np.uint8 if input_u8 else np.float32
    ctype = ctypes.c_uint8 if input_u8 else ctypes.c_float
    err = []

    def _fill(user, first, count, dst):
        try:
            view = np.ctypeslib.as_array(ctypes.cast(dst, ctypes.POINTER(ctype)), shape=(count * d,)).reshape(count, d)
            assert view.dtype == dt
            fill(int(first), int(count), view)
            return 0
        except Exception as e:
            err.append(e)
            return 1

    f = _lib.FILL_FN(_fill)
    Rc = None
    if R is not None:
        Rc = np.ascontiguousarray(np.asarray(R, dtype=np.float32).T)
    p = StreamParams(cfg.to_c(), int(bool(input_u8)), int(bool(large_root)), int(root_mode), _ptr(Rc, _f32p),
                     int(start_id))
    st = StreamStats()
    rc = ctx.lib.stlq_mi355_encode_stream_store(ctx.h, int(n_total), int(chunk), ctypes.byref(p), f, None, writer.h,
                                                checkpoint_path.encode() if checkpoint_path else None,
                                                ctypes.byref(st))
    if err:
        raise err[0]
    check(rc)
    return st
