"""The C-ABI library loads and exports every symbol the public headers declare (no GPU calls)."""
import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(stlq_mi355_\w+)\s*\(", re.M)


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"typedef[^;]*;", "", text)
        names.update(DECL.findall(text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    from stlq_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        from stlq_amd import build

        build.build()
    return ctypes.CDLL(_lib.LIB_PATH)


def test_headers_declare_the_api():
    names = declared_symbols()
    for must in ("stlq_mi355_ctx_create", "stlq_mi355_set_codebooks", "stlq_mi355_beam_search",
                 "stlq_mi355_encode", "stlq_mi355_encode_stream", "stlq_mi355_icm",
                 "stlq_mi355_beam_search_large_root"):
        assert must in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_the_headers():
    from stlq_amd import _lib

    assert set(declared_symbols()) == set(_lib.SIGNATURES)


def test_version_string(lib):
    lib.stlq_mi355_version.restype = ctypes.c_char_p
    assert b"gfx950" in lib.stlq_mi355_version()


def test_null_context_is_an_error_not_a_crash(lib):
    lib.stlq_mi355_ctx_destroy.argtypes = [ctypes.c_void_p]
    assert lib.stlq_mi355_ctx_destroy(None) == 0
    lib.stlq_mi355_set_codebooks.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                             ctypes.c_void_p]
    assert lib.stlq_mi355_set_codebooks(None, 4, 2, None, None) == 1  # STLQ_MI355_ERR_INVALID
    lib.stlq_mi355_last_error.restype = ctypes.c_char_p
    assert b"null context" in lib.stlq_mi355_last_error()


def test_package_refuses_to_run_without_library(monkeypatch, tmp_path):
    from stlq_amd import _lib

    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="missing"):
        _lib.load()
