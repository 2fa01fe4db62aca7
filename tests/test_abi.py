"""The C-ABI library loads and exports every function ``include/rune_hip.h`` declares."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "rune_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rune_[a-z_]+)\s*\(", text)))


def test_header_declares_the_api():
    names = declared_functions()
    for required in ("rune_nlist_build", "rune_nlist_from_padded", "rune_model_create",
                     "rune_model_set_tensor", "rune_model_finalize", "rune_model_compute",
                     "rune_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from rune_amd import _native
    if not _native.LIB_PATH.exists():
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_error_text_without_gpu():
    from rune_amd import _native
    if not _native.LIB_PATH.exists():
        pytest.skip("library not built")
    assert "gfx950" in _native.version()
    lib = _native.library()
    h = ctypes.c_void_p()
    assert lib.rune_model_create(None, ctypes.byref(h)) == _native.ERR_ARGUMENT
    assert b"null" in lib.rune_last_error()
