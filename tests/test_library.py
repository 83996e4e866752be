"""The C-ABI library: it is built, loads, and exports every declared symbol.

Loading needs no GPU; nothing here launches a kernel.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

from tklab import _hip

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "tklab_hip.h"


def _declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^(?:int|const char\*)\s+(tk_\w+)\(", text, flags=re.MULTILINE))


def test_header_and_binding_agree() -> None:
    assert _declared_functions() == set(_hip.EXPORTED_SYMBOLS)


def test_library_loads_and_exports_every_declared_symbol() -> None:
    lib = _hip.load_library()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.tk_abi_version() == _hip.ABI_VERSION
    assert lib.tk_last_error() == b""


def test_library_has_gfx950_code_only() -> None:
    data = _hip.LIBRARY_PATH.read_bytes()
    assert b"gfx950" in data
    for other in (b"gfx942", b"gfx90a", b"gfx1100"):
        assert other not in data


def test_invalid_arguments_fail_before_any_launch() -> None:
    lib = _hip.load_library()
    status = lib.tk_softmax_fwd(0, None, None, 4, 4, 4, 4, None)
    assert status != 0
    assert b"null pointer" in lib.tk_last_error()
    status = lib.tk_softmax_fwd(7, ctypes.c_void_p(16), ctypes.c_void_p(16), 4, 4, 4, 4, None)
    assert status != 0
    assert b"dtype" in lib.tk_last_error()


def test_elementwise_limit_is_the_int32_extent() -> None:
    """Any int32-addressable problem passes the size check (unaligned data takes the
    one-element-per-chunk path, so chunks == elements); one element more is rejected
    before any launch."""
    import torch

    lib = _hip.load_library()
    unaligned = ctypes.c_void_p(2)
    too_big = ctypes.c_int64(2**31)
    status = lib.tk_swiglu_fwd(1, unaligned, unaligned, unaligned, ctypes.c_int64(1), too_big,
                               too_big, too_big, too_big, None)
    assert status != 0 and b"problem too large" in lib.tk_last_error()
    if torch.cuda.is_available():
        return  # the accepted size would launch on the fake pointers below
    largest = ctypes.c_int64(2**31 - 1)
    status = lib.tk_swiglu_fwd(1, unaligned, unaligned, unaligned, ctypes.c_int64(1), largest,
                               largest, largest, largest, None)
    assert status != 0 and b"problem too large" not in lib.tk_last_error()


def test_gqa_decode_rejects_row_strides_past_its_32_bit_tile_offsets() -> None:
    """The decode kernel addresses a 32-key tile (or the G query heads) through 32-bit buffer
    offsets, so key and head strides of 2^24 elements or more are rejected before any launch."""
    import pytest

    p = 1 << 20  # 16-byte aligned; never dereferenced
    ok = _hip.int64_array([32 * 128, 128])
    kv = _hip.int64_array([8 * 1024 * 128, 1024 * 128, 128])
    big = _hip.int64_array([0, 0, 1 << 24])
    with pytest.raises(_hip.HipLibraryError, match="below 2"):
        _hip.call("tk_gqa_decode", 2, p, p, p, p, None, p, None, 1, 32, 8, 1024, 128, 64, ok, big,
                  kv, ok, 0.1, None)


def test_online_softmax_rejects_a_misaligned_workspace() -> None:
    """The single-read kernel publishes each chunk's partial as one 64-bit word."""
    import pytest

    p = 1 << 20  # 16-byte aligned; never dereferenced
    with pytest.raises(_hip.HipLibraryError, match="8-byte aligned"):
        _hip.call("tk_softmax_online_fwd", 0, p, p, p + 4, 2, 100000, 100000, 100000, None)
