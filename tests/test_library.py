"""The C-ABI library: it is built, loads, and exports every declared symbol.

Loading needs no GPU; nothing here launches a kernel.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

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
    p = 1 << 20  # 16-byte aligned; never dereferenced
    ok = _hip.int64_array([32 * 128, 128])
    kv = _hip.int64_array([8 * 1024 * 128, 1024 * 128, 128])
    big = _hip.int64_array([0, 0, 1 << 24])
    with pytest.raises(_hip.HipLibraryError, match="below 2"):
        _hip.call("tk_gqa_decode", 2, p, p, p, p, None, p, None, 1, 32, 8, 1024, 128, 64, ok, big,
                  kv, ok, 0.1, None)


def test_online_softmax_rejects_a_misaligned_workspace() -> None:
    """The single-read kernel publishes each chunk's partial as one 64-bit word."""
    p = 1 << 20  # 16-byte aligned; never dereferenced
    with pytest.raises(_hip.HipLibraryError, match="8-byte aligned"):
        _hip.call("tk_softmax_online_fwd", 0, p, p, p + 4, 2, 100000, 100000, 100000, None)


def _probe_args(name: str, *, dtype: int, pointer, size: int, stride: int, array: list[int]):
    """Arguments for entry point ``name`` from its signature: the first int32 is the dtype
    code (the activation kind follows it), pointers, the leading int64 values sizes (two,
    or three for the GEMMs' m, n, k and RoPE's rows, seq, half_dim), the later int64 values
    strides, int64 arrays stride tables, floats 0.1."""
    values, ints, n64 = [], 0, 0
    sizes = _SIZE_ARGS.get(name, 2)
    for kind in _hip._SIGNATURES[name]:
        if kind is _hip._I32:
            values.append(dtype if ints == 0 else 0)
            ints += 1
        elif kind is _hip._P:
            values.append(pointer)
        elif kind is _hip._I64:
            n64 += 1
            values.append(size if n64 <= sizes else stride)
        elif kind is _hip._F32:
            values.append(0.1)
        else:
            values.append(_hip.int64_array(array))
    return values


_COMPUTE = sorted(n for n in _hip._SIGNATURES if not n.startswith("tk_roof"))
_SIZE_ARGS = {"tk_gemm": 3, "tk_gemm_rowscale": 3, "tk_gemm_swiglu": 3, "tk_rope_positions": 3}
_NO_STRIDES = {"tk_rmsnorm_bwd_stage2", "tk_layernorm_bwd_stage2"}


def _rejected_before_launch(name: str, values) -> str:
    with pytest.raises(_hip.HipLibraryError) as info:
        _hip.call(name, *values)
    message = str(info.value)
    assert "launch failed" not in message, message
    return message


def _cpu_only() -> None:
    """These probes pass pointers that are never valid device memory: run them only where
    no GPU could receive a launch."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("argument probes run without a GPU")



@pytest.mark.parametrize("name", _COMPUTE)
def test_every_entry_point_rejects_null_pointers(name: str) -> None:
    _cpu_only()
    values = _probe_args(name, dtype=2, pointer=None, size=64, stride=64,
                         array=[64 * 64 * 128, 64 * 128, 128, 1])
    assert "null pointer" in _rejected_before_launch(name, values)


@pytest.mark.parametrize("name", _COMPUTE)
def test_every_entry_point_rejects_an_unknown_dtype(name: str) -> None:
    _cpu_only()
    values = _probe_args(name, dtype=7, pointer=1 << 20, size=64, stride=64,
                         array=[64 * 64 * 128, 64 * 128, 128, 1])
    assert "dtype" in _rejected_before_launch(name, values)


@pytest.mark.parametrize("name", _COMPUTE)
def test_every_entry_point_rejects_negative_sizes(name: str) -> None:
    """Negative sizes whose product is positive (rows = cols = -1) included: the
    contiguous-row fold of the elementwise kernels once turned them into one element."""
    _cpu_only()
    values = _probe_args(name, dtype=2, pointer=1 << 20, size=-1, stride=-1,
                         array=[64 * 64 * 128, 64 * 128, 128, 1])
    _rejected_before_launch(name, values)


@pytest.mark.parametrize("name", sorted(set(_COMPUTE) - _NO_STRIDES))
def test_every_entry_point_rejects_negative_strides(name: str) -> None:
    """Row strides as int64 arguments, or (attention, decode) stride tables: a negative
    entry is refused with the layout error, not reached by a launch."""
    _cpu_only()
    if _hip._I64P in _hip._SIGNATURES[name]:
        values = _probe_args(name, dtype=2, pointer=1 << 20, size=64, stride=64,
                             array=[-64 * 64 * 128, -64 * 128, -128, 1])
    else:
        values = _probe_args(name, dtype=2, pointer=1 << 20, size=64, stride=-64,
                             array=[64 * 64 * 128, 64 * 128, 128, 1])
    assert "stride" in _rejected_before_launch(name, values)


def test_sizes_whose_product_overflows_are_rejected() -> None:
    """rows * cols past the 64-bit range (the contiguous-row fold) or rows that end past
    2^52 elements are refused, whichever check meets them first."""
    _cpu_only()
    huge = 1 << 40
    for name in ("tk_swiglu_fwd", "tk_swiglu_bwd", "tk_activation_fwd", "tk_activation_bwd",
                 "tk_softmax_fwd", "tk_rmsnorm_fwd", "tk_layernorm_fwd", "tk_vector_add"):
        values = _probe_args(name, dtype=2, pointer=1 << 20, size=huge, stride=huge, array=[1])
        if name.startswith("tk_activation"):
            values[1] = 0  # kind
        message = _rejected_before_launch(name, values)
        assert "too large" in message or "in range" in message or "columns" in message, message
