"""Rotate-half RoPE forward and backward on HIP kernels, with autograd.

Contract of ``src/tklab/kernels/rope.py``: ``rope(x, cos, sin)`` for a 2-D
``(rows, D)`` input with even ``D`` and ``(rows, D // 2)`` tables of the same
dtype; validation order and messages as in ``rope.py:163-199``. The backward
applies the inverse rotation and, only when asked, the table gradients.
"""

from __future__ import annotations

from functools import partial
from typing import Any, cast

import torch
from torch.autograd.function import once_differentiable

from tklab import _hip
from tklab.harness.addressing import assert_int32_addressable
from tklab.registry import BenchmarkCall, BenchmarkScalar, KernelSpec, TensorArgs, register

_ROWS = 16_384
_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _validate_inputs(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> None:
    """Shape, table, device, dtype, layout and address-width contract."""
    if x.ndim != 2 or cos.ndim != 2 or sin.ndim != 2:
        raise ValueError("rope expects 2D input and angle-table tensors")
    rows, columns = x.shape
    if rows == 0 or columns == 0:
        raise ValueError("rope does not support empty dimensions")
    if columns % 2 != 0:
        raise ValueError("rope requires an even feature dimension")
    expected_table_shape = (rows, columns // 2)
    if cos.shape != expected_table_shape or sin.shape != expected_table_shape:
        raise ValueError("cos and sin must have shape (rows, columns // 2)")
    if x.device != cos.device or x.device != sin.device:
        raise ValueError("x, cos, and sin must be on the same device")
    if x.dtype != cos.dtype or x.dtype != sin.dtype:
        raise ValueError("x, cos, and sin must have the same dtype")
    if x.device.type != "cuda":
        raise ValueError("rope requires CUDA (ROCm/HIP) tensors")
    if x.dtype not in _DTYPES:
        raise ValueError("rope supports float16, bfloat16 and float32 tensors")
    if x.stride(1) != 1 or cos.stride(1) != 1 or sin.stride(1) != 1:
        raise ValueError("rope requires contiguous final dimensions")
    for name, tensor in (("x", x), ("cos", cos), ("sin", sin)):
        assert_int32_addressable(tensor, name=name)


def _validate_output(output: torch.Tensor, x: torch.Tensor, *, name: str) -> None:
    """A preallocated full-width output."""
    if output.shape != x.shape or output.device != x.device or output.dtype != x.dtype:
        raise ValueError(f"{name} metadata must match x")
    if output.stride(1) != 1:
        raise ValueError(f"{name} requires a contiguous final dimension")
    assert_int32_addressable(output, name=name)


def _launch_forward(
    x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, output: torch.Tensor
) -> None:
    """Forward into a supplied output."""
    _validate_inputs(x, cos, sin)
    _validate_output(output, x, name="output")
    rows, columns = x.shape
    _hip.call(
        "tk_rope_fwd",
        _hip.dtype_code(x.dtype),
        x.data_ptr(),
        cos.data_ptr(),
        sin.data_ptr(),
        output.data_ptr(),
        rows,
        columns // 2,
        x.stride(0),
        cos.stride(0),
        sin.stride(0),
        output.stride(0),
        _hip.stream_of(x),
    )


def _launch_backward_into(
    dy: torch.Tensor,
    x: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    dx: torch.Tensor,
    dcos: torch.Tensor | None,
    dsin: torch.Tensor | None,
) -> None:
    """Backward into supplied buffers; ``dcos``/``dsin`` are optional."""
    rows, columns = x.shape
    _hip.call(
        "tk_rope_bwd",
        _hip.dtype_code(x.dtype),
        dy.data_ptr(),
        x.data_ptr(),
        cos.data_ptr(),
        sin.data_ptr(),
        dx.data_ptr(),
        _hip.ptr(dcos),
        _hip.ptr(dsin),
        rows,
        columns // 2,
        dy.stride(0),
        x.stride(0),
        cos.stride(0),
        sin.stride(0),
        dx.stride(0),
        0 if dcos is None else dcos.stride(0),
        0 if dsin is None else dsin.stride(0),
        _hip.stream_of(x),
    )


def _launch_backward(
    dy: torch.Tensor,
    x: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    *,
    need_dcos: bool = True,
    need_dsin: bool = True,
) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor | None]:
    """Deterministic backward (reference ``rope.py:228-272``)."""
    _validate_inputs(x, cos, sin)
    if dy.shape != x.shape or dy.device != x.device or dy.dtype != x.dtype:
        raise ValueError("upstream gradient metadata must match x")
    if dy.stride(1) != 1:
        dy = dy.contiguous()
    assert_int32_addressable(dy, name="upstream gradient")
    dx = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    dcos = torch.empty(cos.shape, dtype=cos.dtype, device=cos.device) if need_dcos else None
    dsin = torch.empty(sin.shape, dtype=sin.dtype, device=sin.device) if need_dsin else None
    _launch_backward_into(dy, x, cos, sin, dx, dcos, dsin)
    return dx, dcos, dsin


class _RoPEFunction(torch.autograd.Function):
    """Autograd bridge; table gradients only for tables that need them."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        """Forward and save (x, cos, sin)."""
        _validate_inputs(x, cos, sin)
        output = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        _launch_forward(x, cos, sin, output)
        ctx.save_for_backward(x, cos, sin)
        return output

    @staticmethod
    @once_differentiable
    def backward(
        ctx: Any, dy: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor | None]:
        """Gradients for x and, when required, both half-width tables."""
        x, cos, sin = ctx.saved_tensors
        return _launch_backward(
            dy, x, cos, sin,
            need_dcos=ctx.needs_input_grad[1],
            need_dsin=ctx.needs_input_grad[2],
        )


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE with ``(rows, feature_dim // 2)`` tables."""
    return cast(torch.Tensor, _RoPEFunction.apply(x, cos, sin))


def _torch_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """PyTorch rotate-half reference."""
    x_first, x_second = x.chunk(2, dim=-1)
    return torch.cat((x_first * cos - x_second * sin, x_second * cos + x_first * sin), dim=-1)


def _naive_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Materialized full-width tables and rotate-half tensor."""
    x_first, x_second = x.chunk(2, dim=-1)
    rotated = torch.cat((-x_second, x_first), dim=-1)
    cos_full = torch.cat((cos, cos), dim=-1)
    sin_full = torch.cat((sin, sin), dim=-1)
    return x * cos_full + rotated * sin_full


def _make_inputs(columns: int, device: torch.device, dtype: torch.dtype) -> TensorArgs:
    """``(16384, columns)`` input with tables of random angles."""
    x = torch.randn(_ROWS, columns, device=device, dtype=dtype)
    angles = torch.randn(_ROWS, columns // 2, device=device, dtype=torch.float32)
    return x, torch.cos(angles).to(dtype), torch.sin(angles).to(dtype)


def _make_adversarial(device: torch.device) -> TensorArgs:
    """Row-strided float32 input and tables, 37 x 1000."""
    rows, columns = 37, 1000
    x_storage = torch.randn(rows * 2, columns, device=device, dtype=torch.float32)
    angles_storage = torch.randn(rows * 3, columns // 2, device=device, dtype=torch.float32)
    angles = angles_storage[::3]
    return x_storage[::2], torch.cos(angles), torch.sin(angles)


def _make_output(args: TensorArgs) -> torch.Tensor:
    """Contiguous output."""
    x = args[0]
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


def _launch(args: TensorArgs, output: torch.Tensor) -> None:
    """Allocation-free forward."""
    x, cos, sin = args
    _launch_forward(x, cos, sin, output)


def _make_benchmark_call(args: TensorArgs, output: torch.Tensor) -> BenchmarkCall:
    """Allocation-free forward call."""
    x, cos, sin = args
    return partial(_launch_forward, x, cos, sin, output)


def _benchmark_metadata(columns: int, dtype: torch.dtype) -> dict[str, BenchmarkScalar]:
    """Describe the two baselines."""
    del columns, dtype
    return {
        "reference_baseline": "direct half-wise PyTorch rotate-half composition",
        "naive_baseline": "materialized full-width tables and rotate-half tensor",
        "reference_allocates_output": True,
        "naive_allocates_output": True,
    }


def _bytes_moved(columns: int, dtype: torch.dtype) -> int:
    """Input, both half tables and output: 3 * rows * D elements."""
    element_size = torch.empty((), dtype=dtype).element_size()
    return 3 * _ROWS * columns * element_size


ROPE = register(
    KernelSpec(
        name="rope_forward",
        description="Rotate-half rotary embedding with half-dimension angle tables.",
        triton_fn=rope,
        launch_fn=_launch,
        ref_fn=_torch_rope,
        make_inputs=_make_inputs,
        make_output=_make_output,
        make_adversarial=_make_adversarial,
        sizes=(32, 64, 128, 256, 512, 1024, 2048),
        correctness_sizes=(64, 128, 256),
        bound="memory",
        bytes_moved=_bytes_moved,
        dtypes=(torch.float16, torch.bfloat16),
        naive_fn=_naive_rope,
        benchmark_metadata=_benchmark_metadata,
        benchmark_call_factory=_make_benchmark_call,
        supports_interpreter=False,
    )
)
