"""The C ABI surface on the CPU: the library loads, and it exports exactly the entry points include/wdl.h declares
(no compute calls: there is no GPU here)."""

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def declared():
    text = (ROOT / "include" / "wdl.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(wdl_\w+)\(", text, re.M)))


def test_header_declares_entry_points():
    assert "wdl_kv_append_fp8" in declared()
    assert "wdl_last_error" in declared()


def test_library_loads_and_exports_every_declared_symbol():
    from wdl import _lib

    lib = _lib.library()
    for name in declared():
        assert hasattr(lib, name), name
    assert set(declared()) == set(_lib.SIGNATURES)
    assert lib.wdl_abi_version() == 1
    assert lib.wdl_last_error() == b""


def test_invalid_call_reports_error_without_launch():
    from wdl import _lib

    lib = _lib.library()
    strides = _lib.i64s([1, 1, 1, 1])
    # at + n beyond capacity: rejected on the host, before any launch (null pointers are never dereferenced)
    rc = lib.wdl_kv_append_fp8(None, 2, strides, None, 2, strides, 1, 4, 1, 8, None, None, None, None, 3, 0, None)
    assert rc == 1
    assert b"exceeds capacity" in lib.wdl_last_error()
