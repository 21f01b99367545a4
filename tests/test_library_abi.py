"""The C ABI library: it loads, exports exactly what include/moba_hip.h
declares, and rejects bad arguments on the host before touching a GPU."""

import ctypes
import re
from pathlib import Path

import pytest

from moba import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "moba_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moba_[a-z0-9_]+)\s*\(", text)))


def test_library_loads():
    lib = _lib.load()
    assert lib.moba_abi_version() == 6


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 13
    for name in names:
        assert hasattr(lib, name), f"{name} missing from {_lib.LIB_PATH}"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert sorted(_lib.SIGNATURES) == names


def test_status_strings():
    lib = _lib.load()
    assert lib.moba_status_string(0) == b"ok"
    assert lib.moba_status_string(1) == b"invalid argument"


def test_invalid_arguments_fail_on_the_host():
    lib = _lib.load()
    rc = lib.moba_pool(None, None, None, 0, 0, 0, 0, 0, 0, 0, 0, None)
    assert rc == _lib.MOBA_ERR_INVALID
    assert b"non-positive" in lib.moba_last_error()
    rc = lib.moba_gate(None, None, None, None, 1, 128, 128, 3, 2, 64, 1, 128, 8, 7, 1, 0,
                       None, 0, None)
    assert rc == _lib.MOBA_ERR_INVALID
    assert b"divisible" in lib.moba_last_error()
    with pytest.raises(ValueError, match="divisible"):
        _lib.call("moba_gate", None, None, None, None, 1, 128, 128, 3, 2, 64, 1, 128, 8, 7,
                  1, 0, None, 0, None)


def test_workspace_queries_are_host_only():
    lib = _lib.load()
    assert lib.moba_gate_workspace_size(1, 65536, 4) >= 8 * 65536 * 4
    # 1024-query tiles would give 4 x 64 = 256 units (< 512), so the build
    # takes 256-query tiles. Count table: 4 heads x 256 tiles x 512 columns;
    # chunk sums: 4 kv heads x 16 chunks (256 units in chunks of 16) x 512.
    assert lib.moba_csc_workspace_size(1, 65536, 4, 4, 512, 8) == 4 * (4 * 256 + 4 * 16) * 512
    # 512K: 4 x 512 units at 1024 queries each. Chunk sums: 32 chunks of 16.
    assert lib.moba_csc_workspace_size(1, 524288, 4, 4, 4096, 8) == 4 * (4 * 512 + 4 * 32) * 4096
    # past 16384 columns: the table of one 16384-column window
    tiles = (1 << 22) // 1024
    chunk = -(-2 * tiles // 64)
    assert lib.moba_csc_workspace_size(2, 1 << 22, 4, 2, 32768, 8) == \
        4 * 2 * 16384 * (4 * tiles + 2 * (-(-2 * tiles // chunk)))


def test_noalloc_gate_rejects_sizes_past_its_static_scratch():
    lib = _lib.load()
    # [1, 524288 + 256, 4, 64]: 2^21 + 1024 query rows, past the 2^21 limit;
    # rejected on the host before any device call.
    rc = lib.moba_gate_noalloc(None, None, None, None, 1, 524288 + 256, 524288 + 256, 4, 4,
                               64, 4099, 128, 8, 7, 1, 0, None)
    assert rc == _lib.MOBA_ERR_WORKSPACE
    assert b"static scratch limit" in lib.moba_last_error()
