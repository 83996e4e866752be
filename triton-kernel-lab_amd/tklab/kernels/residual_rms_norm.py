"""Fused residual add + RMSNorm with two-output autograd, on the HIP kernels.

Contract of ``src/tklab/kernels/residual_rms_norm.py``: ``residual_rms_norm``
returns ``(x + residual, RMSNorm(x + residual))``. The sum is rounded to the
storage dtype before its statistics are taken (the reference does this for
float16, ``residual_rms_norm.py:63-64``; here for float16 and bfloat16 alike),
so the normalized output is computed from exactly the tensor returned.
The backward reuses the RMSNorm stages and folds the direct gradient of the
sum into stage 1 (``residual_rms_norm.py:201-225``).
"""

from __future__ import annotations

from functools import partial
from typing import Any, cast

import torch
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from tklab import _hip
from tklab.harness.addressing import assert_int32_addressable
from tklab.kernels._norm_common import EPS, validate_epsilon
from tklab.kernels.rms_norm import _launch_backward, _validate
from tklab.registry import BenchmarkCall, BenchmarkScalar, KernelSpec, TensorArgs, register

_ROWS = 4096


def _validate_inputs(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor) -> None:
    """Check the residual contract, then the RMSNorm one (reference ``:85-102``)."""
    if residual.shape != x.shape:
        raise ValueError("residual must match the input shape")
    if residual.device != x.device:
        raise ValueError("input and residual must be on the same device")
    if residual.dtype != x.dtype:
        raise ValueError("input and residual must have the same dtype")
    if residual.ndim != 2:
        raise ValueError("residual_rms_norm expects 2D input tensors")
    if residual.stride(1) != 1:
        raise ValueError("residual requires a contiguous final dimension")
    _validate(x, weight)
    assert_int32_addressable(residual, name="residual")


def _validate_output(output: torch.Tensor, reference: torch.Tensor, *, name: str) -> None:
    """Check one preallocated forward output (reference ``:105-120``)."""
    if (
        output.shape != reference.shape
        or output.device != reference.device
        or output.dtype != reference.dtype
    ):
        raise ValueError(f"{name} metadata must match the input")
    if output.stride(1) != 1:
        raise ValueError(f"{name} requires a contiguous final dimension")
    assert_int32_addressable(output, name=name)


def _launch_forward(
    x: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    residual_sum: torch.Tensor,
    output: torch.Tensor,
    rstd: torch.Tensor,
    *,
    eps: float,
    store_residual: bool,
    store_stats: bool,
) -> None:
    """Fused add + normalize into supplied buffers (reference ``:123-167``)."""
    _validate_inputs(x, residual, weight)
    validate_epsilon(eps)
    _validate_output(output, x, name="output")
    if store_residual:
        _validate_output(residual_sum, x, name="residual_sum")
    rows, columns = x.shape
    if store_stats:
        if rstd.shape != (rows,) or rstd.device != x.device:
            raise ValueError("rstd must contain one value per input row")
        if rstd.dtype != torch.float32:
            raise ValueError("rstd must use float32")
    _hip.call(
        "tk_rmsnorm_fwd",
        _hip.dtype_code(x.dtype),
        x.data_ptr(),
        residual.data_ptr(),
        weight.data_ptr(),
        residual_sum.data_ptr() if store_residual else None,
        output.data_ptr(),
        rstd.data_ptr() if store_stats else None,
        rows,
        columns,
        x.stride(0),
        residual.stride(0),
        residual_sum.stride(0) if store_residual else 0,
        output.stride(0),
        eps,
        _hip.stream_of(x),
    )


class _ResidualRMSNormFunction(torch.autograd.Function):
    """Two-output autograd bridge; both inputs receive the same gradient."""

    @staticmethod
    def forward(
        ctx: Any, x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Return ``(residual_sum, normalized)`` and save the sum, weight and rstd."""
        _validate_inputs(x, residual, weight)
        ctx.set_materialize_grads(False)
        residual_sum = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        output = torch.empty_like(residual_sum)
        rstd = torch.empty(x.shape[0], dtype=torch.float32, device=x.device)
        _launch_forward(
            x, residual, weight, residual_sum, output, rstd,
            eps=eps, store_residual=True, store_stats=True,
        )
        ctx.save_for_backward(residual_sum, weight, rstd)
        return residual_sum, output

    @staticmethod
    @once_differentiable
    def backward(
        ctx: Any,
        incoming_residual_sum: torch.Tensor | None,
        incoming_output: torch.Tensor | None,
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, None]:
        """Sum-only gradients pass straight through; otherwise run both stages."""
        residual_sum, weight, rstd = ctx.saved_tensors
        if incoming_output is None:
            total = (
                torch.zeros_like(residual_sum)
                if incoming_residual_sum is None
                else incoming_residual_sum
            )
            dweight = torch.zeros_like(weight)
        else:
            total, dweight = _launch_backward(
                incoming_output, residual_sum, weight, rstd, incoming_dx=incoming_residual_sum
            )
        return total, total, dweight, None


def residual_rms_norm(
    x: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float = EPS,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Return ``(x + residual, RMSNorm(x + residual))`` with autograd."""
    validate_epsilon(eps)
    _validate_inputs(x, residual, weight)
    needs_grad = torch.is_grad_enabled() and (
        x.requires_grad or residual.requires_grad or weight.requires_grad
    )
    if not needs_grad:
        residual_sum = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        output = torch.empty_like(residual_sum)
        _launch_forward(
            x, residual, weight, residual_sum, output, output,
            eps=eps, store_residual=True, store_stats=False,
        )
        return residual_sum, output
    result = _ResidualRMSNormFunction.apply(x, residual, weight, eps)
    return cast(tuple[torch.Tensor, torch.Tensor], result)


def _registered_residual_rms_norm(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor
) -> torch.Tensor:
    """Normalized output only, for the single-output registry contract."""
    _, output = residual_rms_norm(x, residual, weight)
    return output


def _torch_residual_rms_norm(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor
) -> torch.Tensor:
    """PyTorch reference: add, then ``F.rms_norm``."""
    residual_sum = x + residual
    return F.rms_norm(residual_sum, (x.shape[-1],), weight, EPS)


def _make_inputs(columns: int, device: torch.device, dtype: torch.dtype) -> TensorArgs:
    """``(4096, columns)`` input and residual with a standard-normal weight."""
    x = torch.randn(_ROWS, columns, device=device, dtype=dtype)
    residual = torch.randn_like(x)
    weight = torch.randn(columns, device=device, dtype=dtype)
    return x, residual, weight


def _make_adversarial(device: torch.device) -> TensorArgs:
    """Independently row-strided float32 input and residual, 37 x 1000."""
    rows, columns = 37, 1000
    x_storage = torch.randn(rows * 2, columns, device=device, dtype=torch.float32)
    residual_storage = torch.randn(rows * 3, columns, device=device, dtype=torch.float32)
    weight = torch.randn(columns, device=device, dtype=torch.float32)
    return x_storage[::2], residual_storage[::3], weight


def _make_output(args: TensorArgs) -> torch.Tensor:
    """Normalized output buffer."""
    x = args[0]
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


def _launch(args: TensorArgs, output: torch.Tensor) -> None:
    """Normalized output only, default epsilon."""
    x, residual, weight = args
    _launch_forward(
        x, residual, weight, output, output, output,
        eps=EPS, store_residual=False, store_stats=False,
    )


def _make_benchmark_call(args: TensorArgs, output: torch.Tensor) -> BenchmarkCall:
    """Training-mode forward: sum, output and rstd stored."""
    x, residual, weight = args
    residual_sum = torch.empty_like(output)
    rstd = torch.empty(x.shape[0], dtype=torch.float32, device=x.device)
    return partial(
        _launch_forward, x, residual, weight, residual_sum, output, rstd,
        eps=EPS, store_residual=True, store_stats=True,
    )


def _make_reference_call(args: TensorArgs, output: torch.Tensor) -> BenchmarkCall:
    """Native PyTorch add plus ``F.rms_norm``."""
    x, residual, weight = args

    def launch() -> object:
        residual_sum = x + residual
        return residual_sum, F.rms_norm(residual_sum, (x.shape[-1],), weight, EPS)

    return launch


def _make_naive_call(args: TensorArgs, output: torch.Tensor) -> BenchmarkCall:
    """Separate add, reduction, reciprocal-root and scaling ops."""
    x, residual, weight = args

    def launch() -> object:
        residual_sum = x + residual
        s = residual_sum.float()
        mean_square = torch.mean(s * s, dim=-1, keepdim=True)
        normalized = s * torch.rsqrt(mean_square + EPS)
        return residual_sum, (normalized * weight.float()).to(x.dtype)

    return launch


def _bytes_moved(columns: int, dtype: torch.dtype) -> int:
    """Two reads (x, residual) plus two writes (sum, output)."""
    element_size = torch.empty((), dtype=dtype).element_size()
    return 4 * _ROWS * columns * element_size


def _benchmark_metadata(columns: int, dtype: torch.dtype) -> dict[str, BenchmarkScalar]:
    """Describe the two baselines."""
    del columns, dtype
    return {
        "reference_baseline": "torch.add plus torch.nn.functional.rms_norm",
        "naive_baseline": "manual add, pointwise, and reduction composition",
        "reference_allocates_output": True,
        "naive_allocates_output": True,
    }


RESIDUAL_RMS_NORM = register(
    KernelSpec(
        name="residual_rms_norm_forward",
        description="Fused residual addition and RMSNorm with two-output autograd.",
        triton_fn=_registered_residual_rms_norm,
        launch_fn=_launch,
        ref_fn=_torch_residual_rms_norm,
        make_inputs=_make_inputs,
        make_output=_make_output,
        make_adversarial=_make_adversarial,
        sizes=(128, 256, 512, 1024, 2048, 4096, 8192, 16384),
        correctness_sizes=(128, 1024, 4096),
        bound="memory",
        bytes_moved=_bytes_moved,
        dtypes=(torch.float16, torch.bfloat16),
        benchmark_metadata=_benchmark_metadata,
        benchmark_call_factory=_make_benchmark_call,
        reference_call_factory=_make_reference_call,
        naive_call_factory=_make_naive_call,
        supports_interpreter=False,
    )
)
