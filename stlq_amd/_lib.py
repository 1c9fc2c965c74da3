"""Loads libstlq_mi355.so (built in-tree by stlq_amd/build.py) and declares its C ABI.

The library is the product: there is no CPU fallback. If the shared object is missing the
import of this module raises, naming the build command.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libstlq_mi355.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int


class EncodeParams(ctypes.Structure):
    """stlq_mi355_encode_params (base.encode.* knobs, include/stlq/common/config.h:473-482)."""

    _fields_ = [
        ("H_beam", ctypes.c_int),
        ("icm_iters", ctypes.c_int),
        ("ils_iters", ctypes.c_int),
        ("perturb_k", ctypes.c_int),
        ("use_abs", ctypes.c_int),
        ("seed", ctypes.c_uint32),
        ("want_coeffs", ctypes.c_int),
    ]


class Timings(ctypes.Structure):
    _fields_ = [
        ("xnorm_ms", ctypes.c_double),
        ("gemm_ms", ctypes.c_double),
        ("beam_ms", ctypes.c_double),
        ("ls_ms", ctypes.c_double),
        ("icm_ms", ctypes.c_double),
        ("total_ms", ctypes.c_double),
        ("n", ctypes.c_int64),
        ("gemm_launches", ctypes.c_int),
        ("beam_launches", ctypes.c_int),
        ("layer_ms", ctypes.c_double * 20),
        ("beam_reruns", ctypes.c_int64),
    ]


class StreamParams(ctypes.Structure):
    _fields_ = [
        ("encode", EncodeParams),
        ("input_u8", ctypes.c_int),
        ("large_root", ctypes.c_int),
        ("root_mode", ctypes.c_int),
        ("R", ctypes.POINTER(ctypes.c_float)),
        ("start_id", ctypes.c_uint64),
    ]


class ChunkOut(ctypes.Structure):
    _fields_ = [
        ("codes", _u8p),
        ("a", _f32p),
        ("cost", _f32p),
        ("cluster_id", _u32p),
        ("B_small", _u8p),
        ("best_err", _f32p),
        ("input", _vp),
    ]


class StoreConfig(ctypes.Structure):
    """stlq_mi355_store_config (io::BaseBasicStoreConfig, include/stlq/io/base_store.h:12-25)."""

    _fields_ = [
        ("dir", ctypes.c_char_p),
        ("d", ctypes.c_int),
        ("m", ctypes.c_int),
        ("h_vec", _i32p),
        ("h_len", ctypes.c_int),
        ("shard_size", ctypes.c_int),
        ("bucket_size", ctypes.c_int),
        ("bucket_flush_mb", ctypes.c_int),
        ("write_vector_bucket", ctypes.c_int),
        ("write_basic_to_bucket", ctypes.c_int),
        ("raw_bytes_per_vec", ctypes.c_int),
    ]


class StreamStats(ctypes.Structure):
    _fields_ = [
        ("wall_ms", ctypes.c_double),
        ("h2d_ms", ctypes.c_double),
        ("compute_ms", ctypes.c_double),
        ("fill_ms", ctypes.c_double),
        ("sink_ms", ctypes.c_double),
        ("h2d_bytes", ctypes.c_double),
        ("chunks", ctypes.c_int64),
    ]


FILL_FN = ctypes.CFUNCTYPE(ctypes.c_int, _vp, ctypes.c_int64, ctypes.c_int64, _vp)
SINK_FN = ctypes.CFUNCTYPE(ctypes.c_int, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.POINTER(ChunkOut))

# Every symbol the public headers declare, with its (argtypes, restype).
SIGNATURES = {
    "stlq_mi355_last_error": ([], ctypes.c_char_p),
    "stlq_mi355_version": ([], ctypes.c_char_p),
    "stlq_mi355_ctx_create": ([_int, ctypes.POINTER(_vp)], _int),
    "stlq_mi355_ctx_destroy": ([_vp], _int),
    "stlq_mi355_set_codebooks": ([_vp, _int, _int, _i32p, _f32p], _int),
    "stlq_mi355_set_precomp": ([_vp, _int, _int, _i32p, _f32p, _f32p, _f32p], _int),
    "stlq_mi355_get_precomp": ([_vp, _f32p, _f32p], _int),
    "stlq_mi355_xnorm2": ([_vp, _f32p, _int, _i64, _f32p], _int),
    "stlq_mi355_gemm_xc": ([_vp, _f32p, _i64, _f32p], _int),
    "stlq_mi355_beam_search": ([_vp, _f32p, _f32p, _f32p, _i64, _int, _u8p, _f32p], _int),
    "stlq_mi355_solve_ls_all": ([_vp, _f32p, _u8p, _i64, _f32p, _i64p], _int),
    "stlq_mi355_compute_costs": ([_vp, _f32p, _u8p, _f32p, _f32p, _i64, _f32p], _int),
    "stlq_mi355_icm": ([_vp, _f32p, _f32p, _f32p, _i64, _int, _int, ctypes.c_uint32, _u8p, _f32p, _f32p], _int),
    "stlq_mi355_icm_ils": ([_vp, _f32p, _f32p, _f32p, _i64, _int, _int, _int, _int, ctypes.c_uint32, ctypes.c_uint64,
                            _u8p, _f32p, _f32p], _int),
    "stlq_mi355_encode": ([_vp, _f32p, _i64, ctypes.POINTER(EncodeParams), _u8p, _f32p, _f32p, _f64p, _f64p], _int),
    "stlq_mi355_encode_device": ([_vp, _vp, _i64, ctypes.POINTER(EncodeParams), _vp, _vp, _vp, _vp], _int),
    "stlq_mi355_encode_device_noalloc": ([_vp, _vp, _i64, ctypes.POINTER(EncodeParams), _vp, _vp, _vp, _vp], _int),
    "stlq_mi355_encode_stream": ([_vp, _i64, _i64, ctypes.POINTER(StreamParams), FILL_FN, SINK_FN, _vp,
                                  ctypes.POINTER(StreamStats)], _int),
    "stlq_mi355_last_timings": ([_vp, ctypes.POINTER(Timings)], _int),
    "stlq_mi355_set_large_root": ([_vp, _int, _int, _i32p, _f32p, _f32p], _int),
    "stlq_mi355_beam_search_large_root": ([_vp, _f32p, _f32p, _i64, _int, _u32p, _int, _u32p, _u8p, _f32p], _int),
    "stlq_mi355_convert_u8_rotate": ([_vp, _u8p, _int, _int, _int, _f32p, _f32p], _int),
    "stlq_mi355_solve_ls_all_large_root": ([_vp, _f32p, _f32p, _i64, _u32p, _u8p, _f32p, _i64p], _int),
    "stlq_mi355_compute_costs_large_root": ([_vp, _f32p, _f32p, _i64, _u32p, _u8p, _f32p, _f32p, _f32p], _int),
    "stlq_mi355_icm_ils_large_root": ([_vp, _f32p, _f32p, _f32p, _i64, _u32p, _int, _int, _int, _int, ctypes.c_uint32,
                                       ctypes.c_uint64, _u8p, _f32p, _f32p], _int),
    "stlq_mi355_dev_alloc": ([_vp, ctypes.c_size_t, ctypes.POINTER(_vp)], _int),
    "stlq_mi355_dev_free": ([_vp, _vp], _int),
    "stlq_mi355_copy_h2d": ([_vp, _vp, _vp, ctypes.c_size_t], _int),
    "stlq_mi355_copy_d2h": ([_vp, _vp, _vp, ctypes.c_size_t], _int),
    "stlq_mi355_synchronize": ([_vp], _int),
    "stlq_mi355_dev_copy_kernel": ([_vp, _vp, _vp, ctypes.c_size_t], _int),
    "stlq_mi355_device_info": ([_vp, ctypes.c_char_p, _int, _i32p], _int),
    # include/stlq_mi355_store.h
    "stlq_mi355_store_config_init": ([ctypes.POINTER(StoreConfig)], None),
    "stlq_mi355_store_open": ([ctypes.POINTER(StoreConfig), ctypes.POINTER(_vp)], _int),
    "stlq_mi355_store_open_resume": ([ctypes.POINTER(StoreConfig), ctypes.c_uint64, _u64p, _i64,
                                      ctypes.POINTER(_vp)], _int),
    "stlq_mi355_store_append": ([_vp, ctypes.c_uint64, _i64, _u32p, _int, _u8p, _int, _f32p, _int, _vp, _i64], _int),
    "stlq_mi355_store_flush": ([_vp], _int),
    "stlq_mi355_store_bucket_bytes": ([_vp, _u64p, _i64, _i64p], _int),
    "stlq_mi355_store_info": ([_vp, _i32p, _i32p, _i32p, _i32p, _i32p], _int),
    "stlq_mi355_store_close": ([_vp], _int),
    "stlq_mi355_checkpoint_write": ([ctypes.c_char_p, ctypes.c_uint64, _u64p, _i64], _int),
    "stlq_mi355_checkpoint_read": ([ctypes.c_char_p, _u64p, _u64p, _i64, _i64p], _int),
    "stlq_mi355_store_truncate_to_checkpoint": ([ctypes.POINTER(StoreConfig), ctypes.c_uint64, _u64p, _i64], _int),
    "stlq_mi355_encode_stream_store": ([_vp, _i64, _i64, ctypes.POINTER(StreamParams), FILL_FN, _vp, _vp,
                                        ctypes.c_char_p, ctypes.POINTER(StreamStats)], _int),
}

_lib = None


def load():
    """Returns the loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python stlq_amd/build.py`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


class StlqError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"stlq_mi355 error {code}: {msg}")
        self.code = code


def check(rc):
    if rc != 0:
        raise StlqError(rc, load().stlq_mi355_last_error().decode(errors="replace"))
    return rc
