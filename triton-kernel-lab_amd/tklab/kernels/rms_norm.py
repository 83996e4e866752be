"""RMSNorm forward and two-stage backward on the HIP kernels, with autograd.

Public and private API of ``src/tklab/kernels/rms_norm.py``: ``rms_norm``,
``_launch_forward``, ``_make_backward_buffers``, ``_launch_backward_stage1``,
``_launch_backward_stage2``, ``_launch_backward`` and ``_BackwardBuffers``,
with the reference's validation order and messages (``rms_norm.py:176-204``).

Backward. The reference reduces dweight partials under a global spin lock in
a scheduling-dependent order and therefore refuses PyTorch's deterministic
mode (``rms_norm.py:370-378``). Here each of ``min(group_size, rows)``
workgroups is one group and owns the rows ``row % group_size == g`` (the reference's
lock grouping, ``rms_norm.py:134``), accumulates them in increasing row order, writes
one float32 partial row with a plain store, and stage 2 sums the partial rows in a
fixed order. The result is bitwise reproducible. Under deterministic
mode ``_launch_backward`` still raises (or warns) as the reference does, unless
``_norm_common.REJECT_DETERMINISTIC_MODE`` is set to False.
``_BackwardBuffers.locks`` keeps its reference layout (``locks || counts``):
the lock half stays zero and stage 1 sets count ``g`` to 1 for every active
group, the observable state the reference's protocol leaves behind.
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


def _validate(x: torch.Tensor, weight: torch.Tensor) -> None:
    """Check the RMSNorm tensor contract (reference ``rms_norm.py:176-204``)."""
    if x.ndim != 2:
        raise ValueError("rms_norm expects a 2D tensor shaped (rows, columns)")
    rows, columns = x.shape
    if rows == 0 or columns == 0:
        raise ValueError("rms_norm does not support empty dimensions")
    if x.stride(1) != 1:
        raise ValueError("rms_norm requires a contiguous final dimension")
    if weight.ndim != 1:
        raise ValueError("weight must be one-dimensional")
    if weight.shape != (columns,):
        raise ValueError("weight must match the final input dimension")
    if weight.stride(0) != 1:
        raise ValueError("weight must be contiguous")
    if x.device != weight.device:
        raise ValueError("input and weight must be on the same device")
    if x.device.type != "cuda":
        raise ValueError("rms_norm requires CUDA (ROCm/HIP) tensors")
    if x.dtype != weight.dtype:
        raise ValueError("input and weight must have the same dtype")
    if x.dtype not in _DTYPES:
        raise ValueError("rms_norm supports float16, bfloat16 and float32 tensors")
    if columns * x.element_size() > MAX_FEATURE_BYTES:
        raise ValueError(
            f"feature row uses {columns * x.element_size()} bytes; "
            f"the fused limit is {MAX_FEATURE_BYTES}"
        )
    assert_int32_addressable(x, name="input")


@dataclass(frozen=True, slots=True)
class _BackwardBuffers:
    """Outputs and reduction workspace of the backward (reference ``rms_norm.py:207-218``).

    ``block_size`` is the number of columns one row group covers and
    ``num_warps`` the number of 64-lane wavefronts sharing a row.
    """

    dx: torch.Tensor
    partial_dw: torch.Tensor
    dw: torch.Tensor
    locks: torch.Tensor
    group_size: int
    group_count: int
    block_size: int
    num_warps: int


def _launch_forward(
    x: torch.Tensor,
    weight: torch.Tensor,
    output: torch.Tensor,
    rstd: torch.Tensor,
    *,
    eps: float,
    store_stats: bool,
) -> None:
    """Forward into preallocated ``output`` (and ``rstd`` when ``store_stats``)."""
    _validate(x, weight)
    validate_epsilon(eps)
    if output.shape != x.shape or output.device != x.device or output.dtype != x.dtype:
        raise ValueError("output metadata must match the input")
    if output.stride(1) != 1:
        raise ValueError("rms_norm output requires a contiguous final dimension")
    assert_int32_addressable(output, name="output")
    rows, columns = x.shape
    if store_stats:
        if rstd.shape != (rows,):
            raise ValueError("rstd must contain one float32 value per row")
        if rstd.dtype != torch.float32:
            raise ValueError("rstd must use float32")
        if rstd.device != x.device:
            raise ValueError("rstd must be on the input device")
    _hip.call(
        "tk_rmsnorm_fwd",
        _hip.dtype_code(x.dtype),
        x.data_ptr(),
        None,
        weight.data_ptr(),
        None,
        output.data_ptr(),
        rstd.data_ptr() if store_stats else None,
        rows,
        columns,
        x.stride(0),
        0,
        0,
        output.stride(0),
        eps,
        _hip.stream_of(x),
    )


def _make_backward_buffers(
    x: torch.Tensor,
    weight: torch.Tensor,
    *,
    group_size: int | None = None,
) -> _BackwardBuffers:
    """Allocate dx, dw, the float32 partial rows and the zeroed lock/count words."""
    rows, columns = x.shape
    block_size, num_warps = block_size_and_warps(columns, x.element_size())
    selected = group_size_m(columns) if group_size is None else group_size
    if selected <= 0:
        raise ValueError("group_size must be positive")
    return _BackwardBuffers(
        dx=torch.empty(x.shape, dtype=x.dtype, device=x.device),
        partial_dw=torch.empty((selected, columns), dtype=torch.float32, device=x.device),
        dw=torch.empty_like(weight),
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
    rstd: torch.Tensor,
    buffers: _BackwardBuffers,
    *,
    incoming_dx: torch.Tensor | None = None,
) -> None:
    """Per-row dx (plus ``incoming_dx``) and one dweight partial row per group."""
    rows, columns = x.shape
    _hip.call(
        "tk_rmsnorm_bwd_stage1",
        _hip.dtype_code(x.dtype),
        buffers.dx.data_ptr(),
        dy.data_ptr(),
        _hip.ptr(incoming_dx),
        buffers.partial_dw.data_ptr(),
        x.data_ptr(),
        weight.data_ptr(),
        rstd.data_ptr(),
        buffers.locks.data_ptr(),
        rows,
        columns,
        x.stride(0),
        dy.stride(0),
        0 if incoming_dx is None else incoming_dx.stride(0),
        buffers.dx.stride(0),
        buffers.group_size,
        _hip.stream_of(x),
    )


def _launch_backward_stage2(buffers: _BackwardBuffers, columns: int) -> None:
    """dw = fixed-order column sum of the active partial rows."""
    _hip.call(
        "tk_rmsnorm_bwd_stage2",
        _hip.dtype_code(buffers.dw.dtype),
        buffers.partial_dw.data_ptr(),
        buffers.dw.data_ptr(),
        buffers.group_count,
        columns,
        _hip.stream_of(buffers.dw),
    )


def _launch_backward(
    dy: torch.Tensor,
    x: torch.Tensor,
    weight: torch.Tensor,
    rstd: torch.Tensor,
    *,
    incoming_dx: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Both backward stages; returns ``(dx, dw)`` (reference ``rms_norm.py:346-390``)."""
    if dy.shape != x.shape or dy.device != x.device or dy.dtype != x.dtype:
        raise ValueError("upstream gradient metadata must match the input")
    if dy.stride(1) != 1:
        dy = dy.contiguous()
    assert_int32_addressable(dy, name="upstream gradient")
    if incoming_dx is not None:
        if (
            incoming_dx.shape != x.shape
            or incoming_dx.device != x.device
            or incoming_dx.dtype != x.dtype
        ):
            raise ValueError("incoming input gradient metadata must match the input")
        if incoming_dx.stride(1) != 1:
            incoming_dx = incoming_dx.contiguous()
        assert_int32_addressable(incoming_dx, name="incoming input gradient")
    check_deterministic_mode("RMSNorm")
    buffers = _make_backward_buffers(x, weight)
    _launch_backward_stage1(dy, x, weight, rstd, buffers, incoming_dx=incoming_dx)
    _launch_backward_stage2(buffers, x.shape[1])
    return buffers.dx, buffers.dw


class _RMSNormFunction(torch.autograd.Function):
    """Autograd bridge: saves (x, weight, rstd) for the backward."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
        """Forward with float32 rstd saved for backward."""
        _validate(x, weight)
        output = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        rstd = torch.empty(x.shape[0], dtype=torch.float32, device=x.device)
        _launch_forward(x, weight, output, rstd, eps=eps, store_stats=True)
        ctx.save_for_backward(x, weight, rstd)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, dy: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, None]:
        """Input and weight gradients."""
        x, weight, rstd = ctx.saved_tensors
        dx, dw = _launch_backward(dy, x, weight, rstd)
        return dx, dw, None


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = EPS) -> torch.Tensor:
    """RMSNorm over the final dimension with autograd.

    Without gradients the forward skips the statistics store
    (reference ``rms_norm.py:423-442``).
    """
    validate_epsilon(eps)
    _validate(x, weight)
    needs_grad = torch.is_grad_enabled() and (x.requires_grad or weight.requires_grad)
    if not needs_grad:
        output = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        _launch_forward(x, weight, output, output, eps=eps, store_stats=False)
        return output
    return cast(torch.Tensor, _RMSNormFunction.apply(x, weight, eps))


def _torch_rms_norm(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """PyTorch reference with the default epsilon."""
    return F.rms_norm(x, (x.shape[-1],), weight, EPS)


def _naive_rms_norm(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Unfused pointwise and reduction composition."""
    mean_square = torch.mean(x.float() * x.float(), dim=-1, keepdim=True)
    normalized = x.float() * torch.rsqrt(mean_square + EPS)
    return (normalized * weight.float()).to(x.dtype)


def _make_output(args: TensorArgs) -> torch.Tensor:
    """Contiguous forward output."""
    x = args[0]
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


def _launch(args: TensorArgs, output: torch.Tensor) -> None:
    """Output-only forward with the default epsilon."""
    x, weight = args
    _launch_forward(x, weight, output, output, eps=EPS, store_stats=False)


def _make_benchmark_call(args: TensorArgs, output: torch.Tensor) -> BenchmarkCall:
    """Training-mode forward (rstd stored), buffers allocated outside the timed call."""
    x, weight = args
    rstd = torch.empty(x.shape[0], dtype=torch.float32, device=x.device)
    return partial(_launch_forward, x, weight, output, rstd, eps=EPS, store_stats=True)


def _make_reference_call(args: TensorArgs, output: torch.Tensor) -> BenchmarkCall:
    """PyTorch's native RMSNorm (allocates its output)."""
    x, weight = args

    def launch() -> object:
        return F.rms_norm(x, (x.shape[-1],), weight, EPS)

    return launch


def _make_inputs(columns: int, device: torch.device, dtype: torch.dtype) -> TensorArgs:
    """``(4096, columns)`` input and a standard-normal weight."""
    x = torch.randn(_ROWS, columns, device=device, dtype=dtype)
    weight = torch.randn(columns, device=device, dtype=dtype)
    return x, weight


def _make_adversarial(device: torch.device) -> TensorArgs:
    """Row-strided float32 input, 37 x 1000."""
    rows, columns = 37, 1000
    storage = torch.randn(rows * 2, columns, device=device, dtype=torch.float32)
    weight = torch.randn(columns, device=device, dtype=torch.float32)
    return storage[::2], weight


def _bytes_moved(columns: int, dtype: torch.dtype) -> int:
    """Input read plus output write; weight and rstd traffic is excluded."""
    element_size = torch.empty((), dtype=dtype).element_size()
    return 2 * _ROWS * columns * element_size


def _benchmark_metadata(columns: int, dtype: torch.dtype) -> dict[str, BenchmarkScalar]:
    """Describe the two baselines."""
    del columns, dtype
    return {
        "reference_baseline": "torch.nn.functional.rms_norm",
        "naive_baseline": "manual PyTorch pointwise and reduction composition",
        "reference_allocates_output": True,
        "naive_allocates_output": True,
    }


RMS_NORM = register(
    KernelSpec(
        name="rms_norm_forward",
        description="Fused row-wise RMSNorm with FP32 statistics and autograd backward.",
        triton_fn=rms_norm,
        launch_fn=_launch,
        ref_fn=_torch_rms_norm,
        make_inputs=_make_inputs,
        make_output=_make_output,
        make_adversarial=_make_adversarial,
        sizes=(128, 256, 512, 1024, 2048, 4096, 8192, 16384),
        correctness_sizes=(128, 1024, 4096),
        bound="memory",
        bytes_moved=_bytes_moved,
        dtypes=(torch.float16, torch.bfloat16),
        naive_fn=_naive_rms_norm,
        benchmark_metadata=_benchmark_metadata,
        benchmark_call_factory=_make_benchmark_call,
        reference_call_factory=_make_reference_call,
        supports_interpreter=False,
    )
)
