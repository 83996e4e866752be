"""Gate/up GEMM with SwiGLU fused into the epilogue (``tk_gemm_swiglu``).

``matmul_swiglu(x, w_gate, w_up)`` is ``swiglu(value=x @ w_up, gate=x @ w_gate)``
(the reference's ``swiglu(value, gate)``, ``swiglu.py:28-59``, applied to two
``matmul_fp32acc`` products, ``matmul.py:72-164``) computed in one kernel: the
epilogue rounds the two float32 accumulators to the storage dtype, exactly as the
two GEMMs would store them, and writes ``value * gate * sigmoid(gate)``. The two
``[M, N]`` intermediates never reach HBM, and the result is bitwise that of the
unfused composition. Where the fused kernel does not apply (non-unit inner
strides, K not a multiple of 32, N not a multiple of 8, unaligned rows) the same
composition runs on the library's GEMM and SwiGLU kernels. Forward only, like
``matmul_fp32acc``.
"""

from __future__ import annotations

import torch

from tklab import _hip
from tklab.harness.addressing import assert_int32_addressable
from tklab.kernels import matmul, swiglu

# Byte extents at or above 2 GiB fall outside the fused kernel's 32-bit buffer offsets.
_BUFFER_LIMIT = 1 << 31


def matmul_swiglu(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """``(x @ w_up) * silu(x @ w_gate)`` for ``x [M, K]`` and weights ``[K, N]``.

    Raises:
        ValueError: on the GEMM input contract (``matmul_fp32acc``'s messages) or
            mismatched weights.
    """
    matmul._validate(x, w_gate)
    matmul._validate(x, w_up)
    if w_up.shape != w_gate.shape:
        raise ValueError("w_gate and w_up must have identical shapes")
    out = torch.empty((x.shape[0], w_gate.shape[1]), device=x.device, dtype=x.dtype)
    _launch(x, w_gate, w_up, out)
    return out


def fused_applies(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> bool:
    """Whether ``tk_gemm_swiglu`` takes this problem (otherwise the composition runs)."""
    m, k = x.shape
    n = w_gate.shape[1]
    if k % 32 or n % 8 or x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        return False
    if ((m - 1) * x.stride(0) + k) * 2 >= _BUFFER_LIMIT:
        return False
    for w in (w_gate, w_up):
        if w.stride(1) != 1 or w.stride(0) % 8 or w.data_ptr() % 16:
            return False
        if ((k - 1) * w.stride(0) + n) * 2 >= _BUFFER_LIMIT:
            return False
    return True


def _launch(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, out: torch.Tensor) -> None:
    """Run into a preallocated ``[M, N]`` output."""
    if out.shape != (x.shape[0], w_gate.shape[1]) or out.dtype != x.dtype or out.device != x.device:
        raise ValueError("output metadata must match the product")
    if any(s <= 0 for s in out.stride()):
        raise ValueError("output requires strictly positive strides")
    assert_int32_addressable(out, name="output")
    if not fused_applies(x, w_gate, w_up):
        gate = matmul.matmul_fp32acc(x, w_gate)
        value = matmul.matmul_fp32acc(x, w_up)
        swiglu._launch_forward(value, gate, out)
        return
    m, k = x.shape
    n = w_gate.shape[1]
    _hip.call(
        "tk_gemm_swiglu",
        _hip.dtype_code(x.dtype),
        x.data_ptr(),
        w_gate.data_ptr(),
        w_up.data_ptr(),
        out.data_ptr(),
        m,
        n,
        k,
        x.stride(0),
        x.stride(1),
        w_gate.stride(0),
        w_gate.stride(1),
        w_up.stride(0),
        w_up.stride(1),
        out.stride(0),
        out.stride(1),
        _hip.stream_of(x),
    )
