"""SwiGLU ``value * silu(gate)`` forward and elementwise backward on HIP kernels.

Contract of ``src/tklab/kernels/swiglu.py``: 2-D ``value`` and ``gate`` of one
shape and dtype, unit-stride rows (any row stride), float32 nonlinear math with
the branch-stable sigmoid of ``_elementwise_math.py:12-18``; validation order
and messages as in ``swiglu.py:112-145``. bfloat16 is accepted as well.
"""

from __future__ import annotations

from functools import partial
from typing import Any, cast

import torch
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from tklab import _hip
from tklab.harness.addressing import assert_int32_addressable
from tklab.registry import BenchmarkCall, BenchmarkScalar, KernelSpec, TensorArgs, register

_ROWS = 4096
_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def _validate_inputs(value: torch.Tensor, gate: torch.Tensor) -> None:
    """Shape, device, dtype, layout and address-width contract."""
    if value.ndim != 2 or gate.ndim != 2:
        raise ValueError("swiglu expects 2D tensors shaped (rows, columns)")
    rows, columns = value.shape
    if rows == 0 or columns == 0:
        raise ValueError("swiglu does not support empty dimensions")
    if gate.shape != value.shape:
        raise ValueError("value and gate must have identical shapes")
    if gate.device != value.device:
        raise ValueError("value and gate must be on the same device")
    if gate.dtype != value.dtype:
        raise ValueError("value and gate must have the same dtype")
    if value.device.type != "cuda":
        raise ValueError("swiglu requires CUDA (ROCm/HIP) tensors")
    if value.dtype not in _DTYPES:
        raise ValueError("swiglu supports float16, bfloat16 and float32 tensors")
    if value.stride(1) != 1 or gate.stride(1) != 1:
        raise ValueError("swiglu requires contiguous final dimensions")
    for name, tensor in (("value", value), ("gate", gate)):
        assert_int32_addressable(tensor, name=name)


def _validate_output(output: torch.Tensor, reference: torch.Tensor, *, name: str) -> None:
    """One preallocated output or gradient."""
    if (
        output.shape != reference.shape
        or output.device != reference.device
        or output.dtype != reference.dtype
    ):
        raise ValueError(f"{name} metadata must match the input")
    if output.stride(1) != 1:
        raise ValueError(f"{name} requires a contiguous final dimension")
    assert_int32_addressable(output, name=name)


def _launch_forward(value: torch.Tensor, gate: torch.Tensor, output: torch.Tensor) -> None:
    """Forward into a supplied output."""
    _validate_inputs(value, gate)
    _validate_output(output, value, name="output")
    rows, columns = value.shape
    _hip.call(
        "tk_swiglu_fwd",
        _hip.dtype_code(value.dtype),
        value.data_ptr(),
        gate.data_ptr(),
        output.data_ptr(),
        rows,
        columns,
        value.stride(0),
        gate.stride(0),
        output.stride(0),
        _hip.stream_of(value),
    )


def _launch_backward_into(
    dy: torch.Tensor,
    value: torch.Tensor,
    gate: torch.Tensor,
    dvalue: torch.Tensor,
    dgate: torch.Tensor,
) -> None:
    """Backward into supplied gradient buffers (no allocation)."""
    rows, columns = value.shape
    _hip.call(
        "tk_swiglu_bwd",
        _hip.dtype_code(value.dtype),
        dy.data_ptr(),
        value.data_ptr(),
        gate.data_ptr(),
        dvalue.data_ptr(),
        dgate.data_ptr(),
        rows,
        columns,
        dy.stride(0),
        value.stride(0),
        gate.stride(0),
        dvalue.stride(0),
        dgate.stride(0),
        _hip.stream_of(value),
    )


def _launch_backward(
    dy: torch.Tensor, value: torch.Tensor, gate: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """Deterministic elementwise backward (reference ``swiglu.py:170-200``)."""
    _validate_inputs(value, gate)
    if dy.shape != value.shape or dy.device != value.device or dy.dtype != value.dtype:
        raise ValueError("upstream gradient metadata must match the inputs")
    if dy.stride(1) != 1:
        dy = dy.contiguous()
    assert_int32_addressable(dy, name="upstream gradient")
    dvalue = torch.empty(value.shape, dtype=value.dtype, device=value.device)
    dgate = torch.empty_like(dvalue)
    _launch_backward_into(dy, value, gate, dvalue, dgate)
    return dvalue, dgate


class _SwiGLUFunction(torch.autograd.Function):
    """Autograd bridge; saves both inputs."""

    @staticmethod
    def forward(ctx: Any, value: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        """Forward and save (value, gate)."""
        _validate_inputs(value, gate)
        output = torch.empty(value.shape, dtype=value.dtype, device=value.device)
        _launch_forward(value, gate, output)
        ctx.save_for_backward(value, gate)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, dy: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Gradients for value and gate."""
        value, gate = ctx.saved_tensors
        return _launch_backward(dy, value, gate)


def swiglu(value: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """Return ``value * SiLU(gate)`` with float32 nonlinear intermediates."""
    return cast(torch.Tensor, _SwiGLUFunction.apply(value, gate))


def _torch_swiglu(value: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """PyTorch reference."""
    return value * F.silu(gate)


def _naive_swiglu(value: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """Stable float32 sigmoid composed from PyTorch pointwise ops."""
    gate_float = gate.float()
    exp_negative_abs = torch.exp(-torch.abs(gate_float))
    sigmoid = torch.where(
        gate_float >= 0,
        1.0 / (1.0 + exp_negative_abs),
        exp_negative_abs / (1.0 + exp_negative_abs),
    )
    return (value.float() * gate_float * sigmoid).to(value.dtype)


def _make_inputs(columns: int, device: torch.device, dtype: torch.dtype) -> TensorArgs:
    """``(4096, columns)`` value and gate."""
    value = torch.randn(_ROWS, columns, device=device, dtype=dtype)
    gate = torch.randn_like(value)
    return value, gate


def _make_adversarial(device: torch.device) -> TensorArgs:
    """Independently row-strided float32 inputs, 37 x 1000."""
    rows, columns = 37, 1000
    value_storage = torch.randn(rows * 2, columns, device=device, dtype=torch.float32)
    gate_storage = torch.randn(rows * 3, columns, device=device, dtype=torch.float32)
    return value_storage[::2], gate_storage[::3]


def _make_output(args: TensorArgs) -> torch.Tensor:
    """Contiguous output."""
    value = args[0]
    return torch.empty(value.shape, dtype=value.dtype, device=value.device)


def _launch(args: TensorArgs, output: torch.Tensor) -> None:
    """Allocation-free forward."""
    value, gate = args
    _launch_forward(value, gate, output)


def _make_benchmark_call(args: TensorArgs, output: torch.Tensor) -> BenchmarkCall:
    """Allocation-free forward call."""
    value, gate = args
    return partial(_launch_forward, value, gate, output)


def _benchmark_metadata(columns: int, dtype: torch.dtype) -> dict[str, BenchmarkScalar]:
    """Describe the two baselines."""
    del columns, dtype
    return {
        "reference_baseline": "value * torch.nn.functional.silu(gate)",
        "naive_baseline": "stable FP32 sigmoid and explicit pointwise composition",
        "reference_allocates_output": True,
        "naive_allocates_output": True,
    }


def _bytes_moved(columns: int, dtype: torch.dtype) -> int:
    """Two reads plus one write."""
    element_size = torch.empty((), dtype=dtype).element_size()
    return 3 * _ROWS * columns * element_size


SWIGLU = register(
    KernelSpec(
        name="swiglu_forward",
        description="Fused value-times-SiLU gate with stable FP32 nonlinear math.",
        triton_fn=swiglu,
        launch_fn=_launch,
        ref_fn=_torch_swiglu,
        make_inputs=_make_inputs,
        make_output=_make_output,
        make_adversarial=_make_adversarial,
        sizes=(128, 256, 512, 1024, 2048, 4096, 8192, 16384),
        correctness_sizes=(128, 1024, 4096),
        bound="memory",
        bytes_moved=_bytes_moved,
        dtypes=(torch.float16, torch.bfloat16),
        naive_fn=_naive_swiglu,
        benchmark_metadata=_benchmark_metadata,
        benchmark_call_factory=_make_benchmark_call,
        supports_interpreter=False,
    )
)
