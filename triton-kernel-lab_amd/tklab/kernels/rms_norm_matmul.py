"""Residual-RMSNorm feeding a projection GEMM, without the normalized activations.

``residual_rms_norm_matmul(x, residual, folded_weight)`` returns
``(s, rms_norm(s; w) @ W)`` with ``s = x + residual``: the reference's
``residual_rms_norm`` (``residual_rms_norm.py:28-82``) followed by
``matmul_fp32acc`` (``matmul.py:72-164``), the step in front of a QKV projection.
It uses the identity

    rms_norm(s; w) @ W = diag(rstd) . s . (diag(w) . W)

- ``fold_norm_weight(w, W)`` rounds ``w[k] * W[k, n]`` to the storage dtype once per
  weight version (``tk_scale_rows``; at inference, once at load time);
- the statistics pass (``tk_rmsnorm_fwd`` with no output) reads x and residual and
  writes only s and rstd;
- the GEMM multiplies each float32 accumulator row by rstd before rounding
  (``tk_gemm_rowscale``), so the main loop is the plain GEMM's.

The ``M x K`` normalized tensor is neither written nor read back. Rounding differs
from the composition, which rounds ``y = s * rstd * w`` to the storage dtype before
its GEMM, while here ``w * W`` is rounded instead. Both round once per operand
element on the way in, and the tests hold the fused result to the composition's
error against a float64 product. Forward only, like ``matmul_fp32acc``.
"""

from __future__ import annotations

import torch

from tklab import _hip
from tklab.harness.addressing import assert_int32_addressable
from tklab.kernels import matmul
from tklab.kernels._norm_common import EPS, validate_epsilon

# Byte extents at or above 2 GiB fall outside the GEMM's 32-bit buffer offsets.
_BUFFER_LIMIT = 1 << 31


def fold_norm_weight(norm_weight: torch.Tensor, proj_weight: torch.Tensor) -> torch.Tensor:
    """``diag(norm_weight) @ proj_weight`` rounded to the dtype: ``[K]`` and ``[K, N]`` -> ``[K, N]``."""
    if norm_weight.ndim != 1 or proj_weight.ndim != 2:
        raise ValueError("fold_norm_weight expects a 1D norm weight and a 2D projection")
    if norm_weight.shape[0] != proj_weight.shape[0]:
        raise ValueError("norm weight must match the projection's input dimension")
    if norm_weight.dtype != proj_weight.dtype or norm_weight.device != proj_weight.device:
        raise ValueError("norm weight and projection must share dtype and device")
    if proj_weight.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("fold_norm_weight supports float16 and bfloat16 weights only")
    if proj_weight.device.type != "cuda":
        raise ValueError("fold_norm_weight requires CUDA (ROCm/HIP) tensors")
    if proj_weight.stride(1) != 1:
        raise ValueError("projection requires a contiguous final dimension")
    w = norm_weight.contiguous()
    out = torch.empty(proj_weight.shape, device=proj_weight.device, dtype=proj_weight.dtype)
    assert_int32_addressable(proj_weight, name="projection")
    rows, cols = proj_weight.shape
    _hip.call(
        "tk_scale_rows",
        _hip.dtype_code(proj_weight.dtype),
        proj_weight.data_ptr(),
        w.data_ptr(),
        out.data_ptr(),
        rows,
        cols,
        proj_weight.stride(0),
        out.stride(0),
        _hip.stream_of(proj_weight),
    )
    return out


def rms_norm_matmul(x: torch.Tensor, folded_weight: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """``rms_norm(x; w) @ W`` from ``folded_weight = fold_norm_weight(w, W)``."""
    return _run(x, None, folded_weight, eps)[1]


def residual_rms_norm_matmul(
    x: torch.Tensor, residual: torch.Tensor, folded_weight: torch.Tensor, eps: float = EPS
) -> tuple[torch.Tensor, torch.Tensor]:
    """``(s, rms_norm(s; w) @ W)`` with ``s = x + residual`` rounded to the dtype."""
    if residual.shape != x.shape:
        raise ValueError("residual must match the input shape")
    if residual.device != x.device:
        raise ValueError("input and residual must be on the same device")
    if residual.dtype != x.dtype:
        raise ValueError("input and residual must have the same dtype")
    if residual.stride(1) != 1:
        raise ValueError("residual requires a contiguous final dimension")
    s, out = _run(x, residual, folded_weight, eps)
    assert s is not None
    return s, out


def fused_applies(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Whether ``tk_gemm_rowscale`` takes ``a [M, K] @ b [K, N]`` (row-major DMA GEMM)."""
    m, k = a.shape
    n = b.shape[1]
    if k % 32 or n % 8:
        return False
    for t, rows, cols in ((a, m, k), (b, k, n)):
        if t.stride(1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16:
            return False
        if ((rows - 1) * t.stride(0) + cols) * 2 >= _BUFFER_LIMIT:
            return False
    return True


def _run(
    x: torch.Tensor, residual: torch.Tensor | None, folded_weight: torch.Tensor, eps: float
) -> tuple[torch.Tensor | None, torch.Tensor]:
    matmul._validate(x, folded_weight)
    validate_epsilon(eps)
    if x.stride(1) != 1:
        raise ValueError("input requires a contiguous final dimension")
    m, k = x.shape
    n = folded_weight.shape[1]
    s = torch.empty_like(x, memory_format=torch.contiguous_format) if residual is not None else None
    rstd = torch.empty(m, device=x.device, dtype=torch.float32)
    out = torch.empty((m, n), device=x.device, dtype=x.dtype)
    a = s if s is not None else x
    if not fused_applies(a, folded_weight):
        raise ValueError(
            "rms_norm_matmul needs K % 32 == 0, N % 8 == 0, unit inner strides, "
            "16-byte aligned rows and operands below 2 GiB"
        )
    stream = _hip.stream_of(x)
    _hip.call(
        "tk_rmsnorm_fwd",
        _hip.dtype_code(x.dtype),
        x.data_ptr(),
        residual.data_ptr() if residual is not None else None,
        None,
        s.data_ptr() if s is not None else None,
        None,
        rstd.data_ptr(),
        m,
        k,
        x.stride(0),
        residual.stride(0) if residual is not None else 0,
        s.stride(0) if s is not None else 0,
        0,
        eps,
        stream,
    )
    _hip.call(
        "tk_gemm_rowscale",
        _hip.dtype_code(x.dtype),
        a.data_ptr(),
        folded_weight.data_ptr(),
        rstd.data_ptr(),
        out.data_ptr(),
        m,
        n,
        k,
        a.stride(0),
        a.stride(1),
        folded_weight.stride(0),
        folded_weight.stride(1),
        out.stride(0),
        out.stride(1),
        stream,
    )
    return s, out
