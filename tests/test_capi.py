"""The C-ABI library loads and exports every entry point include/drama3_moe.h declares (no GPU needed: nothing is
launched), and the Python binding knows each of them."""
import ctypes
import pathlib
import re

import pytest

from drama3 import _lib

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "drama3_moe.h"


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(d3_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "d3_moe_a8" in names and "d3_last_error" in names


def test_library_exports_every_declared_symbol():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert sorted(set(declared()) - set(_lib.SIGNATURES)) == []


def test_host_only_calls():
    lib = _lib.lib()
    assert lib.d3_version() >= 1
    assert lib.d3_moe_a8_workspace_bytes(16, 8, 2048, 768) > 0
    # argument errors come back as D3_EINVAL with a message, without touching a device
    rc = lib.d3_moe_a8(None, None)
    assert rc == -1 and b"null" in lib.d3_last_error()
