"""The C-ABI library loads and exports every entry point include/kvssd_hip.h
declares; argument errors surface without any GPU work."""

import ctypes
import re
from pathlib import Path

import pytest

from kvssd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "kvssd_hip.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(kvssd_hip_\w+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    names = declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert set(_native.SIGNATURES) == names
    assert lib.kvssd_hip_abi_version() == _native.ABI_VERSION


def test_argument_errors_are_negative_with_messages():
    lib = _native.load()
    desc = _native.DecodeDesc(32, 8, 128, 4, 128, 3, 32, 0, 0, 0, 0.1)
    n = ctypes.c_size_t(0)
    rc = lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n))
    assert rc < 0 and "bits must be 2 or 4" in _native.last_error()
    with pytest.raises(ValueError, match="bits"):
        _native.check(rc, "workspace")
    desc.bits, desc.query_heads = 4, 30
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) < 0
    assert "divisible" in _native.last_error()
    desc.query_heads, desc.head_dim = 32, 512
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) < 0
    desc.head_dim, desc.group_size = 128, 48
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) < 0
    assert "group_size" in _native.last_error()
    desc.group_size = 32
    assert lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(n)) == 0 and n.value > 0
    assert lib.kvssd_hip_unpack_codes(None, 3, 4, None, None) < 0
    assert lib.kvssd_hip_merge_chunks(0, 8, None, None, None, None, None) < 0


def test_kernel_choice_is_reported():
    lib = _native.load()
    k = ctypes.c_int(-1)
    desc = _native.DecodeDesc(4, 2, 32, 2, 8, 4, 16, 2, 0, 0, 0.1)
    assert lib.kvssd_hip_decode_kernel(ctypes.byref(desc), ctypes.byref(k)) == 0
    assert k.value == _native.KERNEL_GENERAL
    desc.kernel = _native.KERNEL_GENERAL
    assert lib.kvssd_hip_decode_kernel(ctypes.byref(desc), ctypes.byref(k)) == 0
