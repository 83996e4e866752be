"""ctypes boundary to ``libtklab_hip.so`` (declared in ``include/tklab_hip.h``).

The library is loaded on the first launch, never at import, so the package
imports and validates inputs on machines without a GPU. There is no fallback:
if the library is missing or fails to load, every launch raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

ABI_VERSION = 1
LIBRARY_PATH = Path(__file__).resolve().parent / "libtklab_hip.so"

DTYPE_CODES: dict[torch.dtype, int] = {
    torch.float32: 0,
    torch.float16: 1,
    torch.bfloat16: 2,
}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float
_I64P = ctypes.POINTER(ctypes.c_int64)

# name -> argument types, in header order (the return type is always int).
_SIGNATURES: dict[str, list[object]] = {
    "tk_softmax_fwd": [_I32, _P, _P, _I64, _I64, _I64, _I64, _P],
    "tk_softmax_online_fwd": [_I32, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "tk_rmsnorm_fwd": [_I32, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _F32, _P],
    "tk_rmsnorm_bwd_stage1": [
        _I32, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P,
    ],
    "tk_rmsnorm_bwd_stage2": [_I32, _P, _P, _I64, _I64, _P],
    "tk_rmsnorm_bwd_noalloc": [
        _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P,
    ],
    "tk_swiglu_fwd": [_I32, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P],
    "tk_swiglu_bwd": [_I32, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "tk_rope_fwd": [_I32, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "tk_rope_bwd": [
        _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P,
    ],
    "tk_rope_positions": [_I32, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P],
    "tk_gemm": [_I32, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P],
    "tk_gemm_rowscale": [_I32, _P, _P, _P, _P] + [_I64] * 9 + [_P],
    "tk_scale_rows": [_I32, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "tk_gemm_swiglu": [
        _I32, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P,
    ],
    "tk_attn_fwd": [
        _I32, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64P, _I64P, _I64P, _I64P, _F32, _I32, _P,
    ],
    "tk_attn_bwd_preprocess": [_I32, _P, _P, _P, _I64, _I64, _I64, _I64, _I64P, _P],
    "tk_attn_bwd_dkdv": [
        _I32, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64P, _F32, _I32, _P,
    ],
    "tk_attn_bwd_dq": [
        _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64P, _F32, _I32, _P,
    ],
    "tk_attn_fwd_gqa": [
        _I32, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64P, _I64P, _I64P, _I64P, _F32,
        _I32, _P,
    ],
    "tk_attn_fwd_rope": [
        _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I64P,
        _I64P, _I64P, _I64P, _F32, _I32, _P,
    ],
    "tk_attn_bwd_dkdv_gqa": [
        _I32, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64P, _I64P, _F32,
        _I32, _P,
    ],
    "tk_attn_bwd_dq_gqa": [
        _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64P, _I64P, _F32, _I32,
        _P,
    ],
    "tk_attn_fwd_varlen": [
        _I32, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64P, _I64P, _I64P,
        _F32, _I32, _P,
    ],
    "tk_attn_bwd_dkdv_varlen": [
        _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64P,
        _I64P, _F32, _I32, _P,
    ],
    "tk_attn_bwd_dq_varlen": [
        _I32, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64P, _I64P,
        _F32, _I32, _P,
    ],
    "tk_vector_add": [_I32, _P, _P, _P, _I64, _I64, _I64, _I64, _P],
    "tk_activation_fwd": [_I32, _I32, _P, _P, _I64, _I64, _I64, _I64, _P],
    "tk_activation_bwd": [_I32, _I32, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P],
    "tk_layernorm_fwd": [_I32, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _F32, _P],
    "tk_layernorm_bwd_stage1": [
        _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P,
    ],
    "tk_layernorm_bwd_stage2": [_I32, _P, _P, _P, _P, _I64, _I64, _P],
    "tk_gqa_decode": [
        _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64P, _I64P, _I64P,
        _I64P, _F32, _P,
    ],
    "tk_roof_copy": [_P, _P, _I64, _P],
    "tk_roof_stream": [_P, _P, _I64, _I32, _I32, _I32, _I32, _I64, _P],
    "tk_roof_mfma": [_I32, _P, _I64, _I64, _P],
}

EXPORTED_SYMBOLS: tuple[str, ...] = ("tk_abi_version", "tk_last_error", *_SIGNATURES)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class HipLibraryError(RuntimeError):
    """The HIP kernel library is missing, stale, or a launch failed."""


def load_library(path: Path | None = None) -> ctypes.CDLL:
    """Load (once) and return the kernel library with typed entry points."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = Path(os.environ.get("TKLAB_HIP_LIBRARY", LIBRARY_PATH)) if path is None else path
        if not target.is_file():
            raise HipLibraryError(
                f"{target} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `make -C triton-kernel-lab_amd/csrc`"
            )
        lib = ctypes.CDLL(str(target))
        lib.tk_abi_version.restype = ctypes.c_int
        lib.tk_abi_version.argtypes = []
        lib.tk_last_error.restype = ctypes.c_char_p
        lib.tk_last_error.argtypes = []
        version = lib.tk_abi_version()
        if version != ABI_VERSION:
            raise HipLibraryError(f"{target} has ABI {version}, expected {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def dtype_code(dtype: torch.dtype) -> int:
    """Return the ``tk_dtype`` code of a supported storage dtype."""
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def ptr(tensor: torch.Tensor | None) -> int | None:
    """Device address of ``tensor`` (``None`` for an absent optional tensor)."""
    return None if tensor is None else tensor.data_ptr()


def stream_of(tensor: torch.Tensor) -> int:
    """Handle of PyTorch's current stream on ``tensor``'s device."""
    return torch.cuda.current_stream(tensor.device).cuda_stream


def int64_array(values: tuple[int, ...] | list[int]) -> ctypes.Array[ctypes.c_int64]:
    """Pack integers into a C ``int64_t[]``."""
    return (ctypes.c_int64 * len(values))(*values)


_bound: dict[str, ctypes._CFuncPtr] = {}


def _function(name: str) -> ctypes._CFuncPtr:
    """Typed entry point ``name`` of the loaded library."""
    fn = _bound.get(name)
    if fn is None:
        fn = getattr(load_library(), name)
        fn.restype = ctypes.c_int
        fn.argtypes = _SIGNATURES[name]
        _bound[name] = fn
    return fn


def call(name: str, *args: object) -> None:
    """Invoke ``name`` and raise :class:`HipLibraryError` on a non-zero status."""
    fn = _function(name)
    lib = load_library()
    status = fn(*args)
    if status != 0:
        message = lib.tk_last_error().decode(errors="replace")
        raise HipLibraryError(f"{name} failed: {message}")
