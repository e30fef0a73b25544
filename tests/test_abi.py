"""The C-ABI library loads and exports every function include/gofann_hip.h
declares (no compute call: this runs without a GPU)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def declared_functions():
    text = (ROOT / "include" / "gofann_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gofann_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(hip_lib_path):
    lib = ctypes.CDLL(str(hip_lib_path))
    names = declared_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header():
    from gofann_amd import _lib
    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_null_context_is_rejected(hip_lib_path):
    lib = ctypes.CDLL(str(hip_lib_path))
    lib.gofann_synchronize.argtypes = [ctypes.c_void_p]
    assert lib.gofann_synchronize(None) == -1
    lib.gofann_last_error.restype = ctypes.c_char_p
    lib.gofann_last_error.argtypes = [ctypes.c_void_p]
    assert lib.gofann_last_error(None) == b"null context"
