"""LayerNorm forward and deterministic two-stage backward (registry kernel).

Contract of ``src/tklab/kernels/layer_norm.py``: 2-D input with unit-stride
rows, contiguous weight and bias of the feature width, float32 statistics,
validation order and messages as in ``layer_norm.py:177-205``. The backward
uses the same lock-free group reduction as RMSNorm (``tklab.kernels.rms_norm``),
so it is bitwise reproducible; under PyTorch's deterministic mode it raises (or warns)
as the reference does (``layer_norm.py:367-375``) unless
``_norm_common.REJECT_DETERMINISTIC_MODE`` is False. ``_BackwardBuffers`` keeps the
reference's fields.
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import partial
from typing import Any, cast

import torch
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from tklab import _hip
from tklab.harness.addressing import assert_int32_addressable
from tklab.kernels._norm_common import (
    EPS,
    MAX_FEATURE_BYTES,
    block_size_and_warps,
    check_deterministic_mode,
    group_size_m,
    validate_epsilon,
)
from tklab.registry import BenchmarkCall, BenchmarkScalar, KernelSpec, TensorArgs, register

_ROWS = 4096
_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _validate(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor) -> None:
    """LayerNorm tensor contract."""
    if x.ndim != 2:
        raise ValueError("layer_norm expects a 2D tensor shaped (rows, columns)")
    rows, columns = x.shape
    if rows == 0 or columns == 0:
        raise ValueError("layer_norm does not support empty dimensions")
    if x.stride(1) != 1:
        raise ValueError("layer_norm requires a contiguous final dimension")
    if weight.ndim != 1 or bias.ndim != 1:
        raise ValueError("weight and bias must be one-dimensional")
    if weight.shape != (columns,) or bias.shape != (columns,):
        raise ValueError("weight and bias must match the final input dimension")
    if weight.stride(0) != 1 or bias.stride(0) != 1:
        raise ValueError("weight and bias must be contiguous")
    if x.device != weight.device or x.device != bias.device:
        raise ValueError("input, weight, and bias must be on the same device")
    if x.device.type != "cuda":
        raise ValueError("layer_norm requires CUDA (ROCm/HIP) tensors")
    if x.dtype != weight.dtype or x.dtype != bias.dtype:
        raise ValueError("input, weight, and bias must have the same dtype")
    if x.dtype not in _DTYPES:
        raise ValueError("layer_norm supports float16, bfloat16 and float32 tensors")
    if columns * x.element_size() > MAX_FEATURE_BYTES:
        raise ValueError(
            f"feature row uses {columns * x.element_size()} bytes; "
            f"the fused limit is {MAX_FEATURE_BYTES}"
        )
    assert_int32_addressable(x, name="input")


@dataclass(frozen=True, slots=True)
class _BackwardBuffers:
    """Outputs and reduction workspace of the backward."""

    dx: torch.Tensor
    partial_dw: torch.Tensor
    partial_db: torch.Tensor
    dw: torch.Tensor
    db: torch.Tensor
    locks: torch.Tensor
    group_size: int
    group_count: int
    block_size: int
    num_warps: int


def _launch_forward(
    x: torch.Tensor,
    weight: torch.Tensor,
    bias: torch.Tensor,
    output: torch.Tensor,
    mean: torch.Tensor,
    rstd: torch.Tensor,
    *,
    eps: float,
    store_stats: bool,
) -> None:
    """Forward into preallocated output (and mean/rstd when ``store_stats``)."""
    _validate(x, weight, bias)
    validate_epsilon(eps)
    if output.shape != x.shape or output.device != x.device or output.dtype != x.dtype:
        raise ValueError("output metadata must match the input")
    if output.stride(1) != 1:
        raise ValueError("layer_norm output requires a contiguous final dimension")
    assert_int32_addressable(output, name="output")
    rows, columns = x.shape
    if store_stats:
        expected = (rows,)
        if mean.shape != expected or rstd.shape != expected:
            raise ValueError("mean and rstd must contain one float32 value per row")
        if mean.dtype != torch.float32 or rstd.dtype != torch.float32:
            raise ValueError("mean and rstd must use float32")
        if mean.device != x.device or rstd.device != x.device:
            raise ValueError("mean and rstd must be on the input device")
    _hip.call(
        "tk_layernorm_fwd", _hip.dtype_code(x.dtype), x.data_ptr(), weight.data_ptr(),
        bias.data_ptr(), output.data_ptr(),
        mean.data_ptr() if store_stats else None, rstd.data_ptr() if store_stats else None,
        rows, columns, x.stride(0), output.stride(0), eps, _hip.stream_of(x),
    )


def _make_backward_buffers(
    x: torch.Tensor, weight: torch.Tensor, *, group_size: int | None = None
) -> _BackwardBuffers:
    """Allocate gradients, float32 partial rows and the lock/count words."""
    rows, columns = x.shape
    block_size, num_warps = block_size_and_warps(columns, x.element_size())
    selected = group_size_m(columns) if group_size is None else group_size
    if selected <= 0:
        raise ValueError("group_size must be positive")
    return _BackwardBuffers(
        dx=torch.empty(x.shape, dtype=x.dtype, device=x.device),
        partial_dw=torch.empty((selected, columns), dtype=torch.float32, device=x.device),
        partial_db=torch.empty((selected, columns), dtype=torch.float32, device=x.device),
        dw=torch.empty_like(weight),
        db=torch.empty_like(weight),
        locks=torch.zeros(2 * selected, dtype=torch.int32, device=x.device),
        group_size=selected,
        group_count=min(selected, rows),
        block_size=block_size,
        num_warps=num_warps,
    )


def _launch_backward_stage1(
    dy: torch.Tensor,
    x: torch.Tensor,
    weight: torch.Tensor,
    mean: torch.Tensor,
    rstd: torch.Tensor,
    buffers: _BackwardBuffers,
) -> None:
    """Per-row dx and one dweight/dbias partial row per group."""
    rows, columns = x.shape
    _hip.call(
        "tk_layernorm_bwd_stage1", _hip.dtype_code(x.dtype), buffers.dx.data_ptr(), dy.data_ptr(),
        buffers.partial_dw.data_ptr(), buffers.partial_db.data_ptr(), x.data_ptr(),
        weight.data_ptr(), mean.data_ptr(), rstd.data_ptr(), buffers.locks.data_ptr(), rows,
        columns, x.stride(0), dy.stride(0), buffers.dx.stride(0), buffers.group_size,
        _hip.stream_of(x),
    )


def _launch_backward_stage2(buffers: _BackwardBuffers, columns: int) -> None:
    """dw, db = fixed-order column sums of the active partial rows."""
    _hip.call(
        "tk_layernorm_bwd_stage2", _hip.dtype_code(buffers.dw.dtype),
        buffers.partial_dw.data_ptr(), buffers.partial_db.data_ptr(), buffers.dw.data_ptr(),
        buffers.db.data_ptr(), buffers.group_count, columns, _hip.stream_of(buffers.dw),
    )


def _launch_backward(
    dy: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, mean: torch.Tensor, rstd: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Both backward stages; returns (dx, dw, db)."""
    if dy.shape != x.shape or dy.device != x.device or dy.dtype != x.dtype:
        raise ValueError("upstream gradient metadata must match the input")
    if dy.stride(1) != 1:
        dy = dy.contiguous()
    assert_int32_addressable(dy, name="upstream gradient")
    check_deterministic_mode("LayerNorm")
    buffers = _make_backward_buffers(x, weight)
    _launch_backward_stage1(dy, x, weight, mean, rstd, buffers)
    _launch_backward_stage2(buffers, x.shape[1])
    return buffers.dx, buffers.dw, buffers.db


class _LayerNormFunction(torch.autograd.Function):
    """Autograd bridge; saves (x, weight, mean, rstd)."""

    @staticmethod
    def forward(
        ctx: Any, x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float
    ) -> torch.Tensor:
        _validate(x, weight, bias)
        output = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        mean = torch.empty(x.shape[0], dtype=torch.float32, device=x.device)
        rstd = torch.empty_like(mean)
        _launch_forward(x, weight, bias, output, mean, rstd, eps=eps, store_stats=True)
        ctx.save_for_backward(x, weight, mean, rstd)
        return output

    @staticmethod
    @once_differentiable
    def backward(
        ctx: Any, dy: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, None]:
        x, weight, mean, rstd = ctx.saved_tensors
        dx, dw, db = _launch_backward(dy, x, weight, mean, rstd)
        return dx, dw, db, None


def layer_norm(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float = EPS
) -> torch.Tensor:
    """LayerNorm over the final dimension with autograd."""
    validate_epsilon(eps)
    _validate(x, weight, bias)
    needs_grad = torch.is_grad_enabled() and (
        x.requires_grad or weight.requires_grad or bias.requires_grad
    )
    if not needs_grad:
        output = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        _launch_forward(x, weight, bias, output, output, output, eps=eps, store_stats=False)
        return output
    return cast(torch.Tensor, _LayerNormFunction.apply(x, weight, bias, eps))


def _torch_layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    return F.layer_norm(x, (x.shape[-1],), weight, bias, EPS)


def _naive_layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    mean = torch.mean(xf, dim=-1, keepdim=True)
    centered = xf - mean
    variance = torch.mean(centered * centered, dim=-1, keepdim=True)
    return (centered * torch.rsqrt(variance + EPS) * weight.float() + bias.float()).to(x.dtype)


def _make_output(args: TensorArgs) -> torch.Tensor:
    x = args[0]
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


def _launch(args: TensorArgs, output: torch.Tensor) -> None:
    x, weight, bias = args
    _launch_forward(x, weight, bias, output, output, output, eps=EPS, store_stats=False)


def _make_benchmark_call(args: TensorArgs, output: torch.Tensor) -> BenchmarkCall:
    x, weight, bias = args
    mean = torch.empty(x.shape[0], dtype=torch.float32, device=x.device)
    rstd = torch.empty_like(mean)
    return partial(_launch_forward, x, weight, bias, output, mean, rstd, eps=EPS, store_stats=True)


def _make_reference_call(args: TensorArgs, output: torch.Tensor) -> BenchmarkCall:
    x, weight, bias = args

    def launch() -> object:
        return F.layer_norm(x, (x.shape[-1],), weight, bias, EPS)

    return launch


def _make_inputs(columns: int, device: torch.device, dtype: torch.dtype) -> TensorArgs:
    x = torch.randn(_ROWS, columns, device=device, dtype=dtype)
    weight = torch.randn(columns, device=device, dtype=dtype)
    bias = torch.randn(columns, device=device, dtype=dtype)
    return x, weight, bias


def _make_adversarial(device: torch.device) -> TensorArgs:
    """Row-strided float32 input, 37 x 1000."""
    storage = torch.randn(74, 1000, device=device, dtype=torch.float32)
    weight = torch.randn(1000, device=device, dtype=torch.float32)
    bias = torch.randn(1000, device=device, dtype=torch.float32)
    return storage[::2], weight, bias


def _benchmark_metadata(columns: int, dtype: torch.dtype) -> dict[str, BenchmarkScalar]:
    del columns, dtype
    return {
        "reference_baseline": "torch.nn.functional.layer_norm",
        "naive_baseline": "explicit FP32 mean, variance, normalize, and affine composition",
        "reference_allocates_output": True,
        "naive_allocates_output": True,
    }


def _bytes_moved(columns: int, dtype: torch.dtype) -> int:
    """Input read plus output write."""
    return 2 * _ROWS * columns * torch.empty((), dtype=dtype).element_size()


LAYER_NORM = register(
    KernelSpec(
        name="layer_norm_forward",
        description="Fused row-wise LayerNorm with FP32 statistics and autograd backward.",
        triton_fn=layer_norm,
        launch_fn=_launch,
        ref_fn=_torch_layer_norm,
        make_inputs=_make_inputs,
        make_output=_make_output,
        make_adversarial=_make_adversarial,
        sizes=(128, 256, 512, 1024, 2048, 4096, 8192, 16384),
        correctness_sizes=(128, 1024, 4096),
        bound="memory",
        bytes_moved=_bytes_moved,
        dtypes=(torch.float16, torch.bfloat16),
        naive_fn=_naive_layer_norm,
        benchmark_metadata=_benchmark_metadata,
        benchmark_call_factory=_make_benchmark_call,
        reference_call_factory=_make_reference_call,
        supports_interpreter=False,
    )
)
