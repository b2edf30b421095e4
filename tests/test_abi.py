"""The C-ABI library loads on the CPU and exports every declared entry point."""

import ctypes
import re
from pathlib import Path

from loopspec_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "loopspec_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ls_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "ls_greedy_verify" in names and "ls_last_error" in names
    assert len(names) >= 7


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"missing exports: {missing}"


def test_every_declared_symbol_has_a_python_signature():
    missing = [n for n in declared_symbols() if n not in _lib.SIGNATURES]
    assert not missing, f"no ctypes signature for: {missing}"


def test_version_options_and_errors_without_gpu():
    lib = _lib.load()
    assert lib.ls_abi_version() >= 1
    assert lib.ls_set_option(b"greedy_splits", 0) == _lib.LS_OK
    assert lib.ls_set_option(b"no_such_option", 1) == _lib.LS_ERR_VALUE
    assert b"unknown option" in lib.ls_last_error()
    # argument validation happens before any device call
    assert lib.ls_greedy_verify(None, 0, 0, None, 0, 0, None, 1, 1, 0, 10, None, None, None, None, 0, None) \
        == _lib.LS_ERR_VALUE
    assert lib.ls_argmax_rows(None, 7, 1, 10, 10, None, None, 0, None) == _lib.LS_ERR_VALUE
