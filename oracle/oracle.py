"""numpy/ctypes front end of the C oracle (``oracle/tklab_oracle.c``).

TEST INFRASTRUCTURE ONLY. Imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` as the checker for the HIP
kernels; the product (the ``tklab`` package) never imports it.

Every function takes float32 numpy arrays holding values representable in the
storage dtype ``dtype`` (``"float32"``, ``"float16"`` or ``"bfloat16"``) and
returns float32 arrays rounded to that dtype wherever the reference kernel
stores or casts. Shapes follow the reference's kernels; see the C file for the
reference lines each function restates.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

LIBRARY = Path(__file__).resolve().parent / "_build" / "libtklab_oracle.so"
_DT = {"float32": 0, "float16": 1, "bfloat16": 2}

_lib: ctypes.CDLL | None = None
_F = ctypes.POINTER(ctypes.c_float)
_D = ctypes.POINTER(ctypes.c_double)
_I = ctypes.c_int64


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.is_file():
            raise RuntimeError(f"{LIBRARY} is not built; run `make -C oracle`")
        lib = ctypes.CDLL(str(LIBRARY))
        sigs = {
            "or_round_array": [_F, _I, ctypes.c_int],
            "or_softmax": [_F, _F, _I, _I, ctypes.c_int],
            "or_rmsnorm_fwd": [_F, _F, _F, _F, _F, _F, _I, _I, ctypes.c_float, ctypes.c_int],
            "or_rmsnorm_bwd": [_F, _F, _F, _F, _F, _F, _F, _D, _I, _I, ctypes.c_int],
            "or_swiglu_fwd": [_F, _F, _F, _I, ctypes.c_int],
            "or_swiglu_bwd": [_F, _F, _F, _F, _F, _I, ctypes.c_int],
            "or_rope_fwd": [_F, _F, _F, _F, _I, _I, ctypes.c_int],
            "or_rope_bwd": [_F, _F, _F, _F, _F, _F, _F, _I, _I, ctypes.c_int],
            "or_gemm": [_F, _F, _F, _I, _I, _I, ctypes.c_int],
            "or_attn_fwd": [_F, _F, _F, _F, _F, _I, _I, _I, ctypes.c_float, ctypes.c_int, ctypes.c_int],
            "or_gqa_decode": [
                _F, _F, _F, ctypes.c_void_p, _F, _F, _I, _I, _I, _I, _I, ctypes.c_float,
                ctypes.c_int,
            ],
            "or_attn_bwd": [
                _F, _F, _F, _F, _F, _F, _F, _F, _F, _F, _I, _I, _I, ctypes.c_float, ctypes.c_int,
                ctypes.c_int,
            ],
        }
        for name, argtypes in sigs.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = None
        _lib = lib
    return _lib


def set_threads(count: int) -> None:
    """Set the OpenMP thread count used by later oracle calls."""
    os.environ["OMP_NUM_THREADS"] = str(count)
    try:
        libgomp = ctypes.CDLL("libgomp.so.1")
        libgomp.omp_set_num_threads(ctypes.c_int(count))
    except OSError:
        pass


def _f32(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray | None):  # noqa: ANN202 - ctypes pointer
    return None if a is None else a.ctypes.data_as(_F)


def _dt(dtype: str) -> int:
    return _DT[dtype]


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to nearest-even in ``dtype`` (returned as float32)."""
    out = _f32(x).copy()
    _load().or_round_array(_p(out), out.size, _dt(dtype))
    return out


def softmax(x: np.ndarray, dtype: str) -> np.ndarray:
    """Row-wise softmax of a 2-D array."""
    x = _f32(x)
    y = np.empty_like(x)
    _load().or_softmax(_p(x), _p(y), x.shape[0], x.shape[1], _dt(dtype))
    return y


def rmsnorm_fwd(
    x: np.ndarray, weight: np.ndarray, eps: float, dtype: str, residual: np.ndarray | None = None
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Return ``(residual_sum, y, rstd)``; ``residual_sum`` is ``x`` when no residual."""
    x = _f32(x)
    weight = _f32(weight)
    rows, cols = x.shape
    s = np.empty_like(x)
    y = np.empty_like(x)
    rstd = np.empty(rows, dtype=np.float32)
    r = None if residual is None else _f32(residual)
    _load().or_rmsnorm_fwd(
        _p(x), _p(r), _p(weight), _p(s), _p(y), _p(rstd), rows, cols, eps, _dt(dtype)
    )
    return s, y, rstd


def rmsnorm_bwd(
    dy: np.ndarray,
    x: np.ndarray,
    weight: np.ndarray,
    rstd: np.ndarray,
    dtype: str,
    incoming: np.ndarray | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """Return ``(dx, dweight)``; ``x`` is the normalized input (the residual sum)."""
    dy, x, weight, rstd = _f32(dy), _f32(x), _f32(weight), _f32(rstd)
    rows, cols = x.shape
    dx = np.empty_like(x)
    dw = np.empty(cols, dtype=np.float32)
    acc = np.empty(cols, dtype=np.float64)
    inc = None if incoming is None else _f32(incoming)
    _load().or_rmsnorm_bwd(
        _p(dy), _p(x), _p(weight), _p(rstd), _p(inc), _p(dx), _p(dw),
        acc.ctypes.data_as(_D), rows, cols, _dt(dtype),
    )
    return dx, dw


def swiglu_fwd(value: np.ndarray, gate: np.ndarray, dtype: str) -> np.ndarray:
    """``value * silu(gate)`` elementwise."""
    value, gate = _f32(value), _f32(gate)
    y = np.empty_like(value)
    _load().or_swiglu_fwd(_p(value), _p(gate), _p(y), value.size, _dt(dtype))
    return y


def swiglu_bwd(
    dy: np.ndarray, value: np.ndarray, gate: np.ndarray, dtype: str
) -> tuple[np.ndarray, np.ndarray]:
    """Return ``(dvalue, dgate)``."""
    dy, value, gate = _f32(dy), _f32(value), _f32(gate)
    dv = np.empty_like(value)
    dg = np.empty_like(value)
    _load().or_swiglu_bwd(_p(dy), _p(value), _p(gate), _p(dv), _p(dg), value.size, _dt(dtype))
    return dv, dg


def rope_fwd(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str) -> np.ndarray:
    """Rotate-half RoPE of ``x[rows][2*half]`` with ``[rows][half]`` tables."""
    x, cos, sin = _f32(x), _f32(cos), _f32(sin)
    y = np.empty_like(x)
    _load().or_rope_fwd(_p(x), _p(cos), _p(sin), _p(y), x.shape[0], x.shape[1] // 2, _dt(dtype))
    return y


def rope_bwd(
    dy: np.ndarray, x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Return ``(dx, dcos, dsin)``."""
    dy, x, cos, sin = _f32(dy), _f32(x), _f32(cos), _f32(sin)
    dx = np.empty_like(x)
    dcos = np.empty_like(cos)
    dsin = np.empty_like(sin)
    _load().or_rope_bwd(
        _p(dy), _p(x), _p(cos), _p(sin), _p(dx), _p(dcos), _p(dsin),
        x.shape[0], x.shape[1] // 2, _dt(dtype),
    )
    return dx, dcos, dsin


def gemm(a: np.ndarray, b: np.ndarray, dtype: str) -> np.ndarray:
    """``a @ b`` with a high-precision accumulator, rounded to ``dtype``."""
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    c = np.empty((m, n), dtype=np.float32)
    _load().or_gemm(_p(a), _p(b), _p(c), m, n, k, _dt(dtype))
    return c


def attn_fwd(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal: bool, dtype: str
) -> tuple[np.ndarray, np.ndarray]:
    """Return ``(o, lse)`` for ``[..., seq, d]`` inputs; ``lse`` is base 2."""
    shape = q.shape
    q, k, v = (_f32(t).reshape(-1, shape[-2], shape[-1]) for t in (q, k, v))
    heads, seq, d = q.shape
    o = np.empty_like(q)
    lse = np.empty((heads, seq), dtype=np.float32)
    _load().or_attn_fwd(
        _p(q), _p(k), _p(v), _p(o), _p(lse), heads, seq, d, scale, int(causal), _dt(dtype)
    )
    return o.reshape(shape), lse.reshape(shape[:-1])


def gqa_decode(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    scale: float,
    dtype: str,
    lens: np.ndarray | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """Return ``(o, lse)`` for q ``[B, Hq, d]`` and k, v ``[B, Hkv, L, d]``; lse base 2."""
    q, k, v = (_f32(t) for t in (q, k, v))
    batch, q_heads, d = q.shape
    _, kv_heads, length, _ = k.shape
    o = np.empty_like(q)
    lse = np.empty((batch, q_heads), dtype=np.float32)
    lens_arr = None if lens is None else np.ascontiguousarray(lens, dtype=np.int32)
    lens_p = None if lens_arr is None else lens_arr.ctypes.data_as(ctypes.c_void_p)
    _load().or_gqa_decode(
        _p(q), _p(k), _p(v), lens_p, _p(o), _p(lse), batch, q_heads, kv_heads, length, d,
        scale, _dt(dtype),
    )
    return o, lse


def attn_bwd(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    o: np.ndarray,
    dout: np.ndarray,
    lse: np.ndarray,
    scale: float,
    causal: bool,
    dtype: str,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Return ``(dq, dk, dv)`` from the saved output and base-2 LSE."""
    shape = q.shape
    q, k, v, o, dout = (_f32(t).reshape(-1, shape[-2], shape[-1]) for t in (q, k, v, o, dout))
    heads, seq, d = q.shape
    lse = _f32(lse).reshape(heads, seq)
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    ds = np.empty((heads, seq, seq), dtype=np.float32)
    _load().or_attn_bwd(
        _p(q), _p(k), _p(v), _p(o), _p(dout), _p(lse), _p(dq), _p(dk), _p(dv), _p(ds),
        heads, seq, d, scale, int(causal), _dt(dtype),
    )
    return dq.reshape(shape), dk.reshape(shape), dv.reshape(shape)
