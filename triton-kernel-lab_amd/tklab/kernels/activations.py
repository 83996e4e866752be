"""ReLU, exact GELU, SiLU and tanh with deterministic autograd (registry kernels).

Contract of ``src/tklab/kernels/activations.py``: 2-D input with a unit-stride
final dimension, float32 nonlinear math, one elementwise backward kernel per
activation; validation messages as in ``activations.py:139-164``. tanh is
evaluated as ``2*sigmoid(2x) - 1`` like the reference.
"""

from __future__ import annotations

import math
from functools import partial
from typing import Any, cast

import torch
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from tklab import _hip
from tklab.harness.addressing import assert_int32_addressable
from tklab.registry import BenchmarkCall, BenchmarkScalar, KernelSpec, TensorArgs, TensorFn, register

_ROWS = 4096
_DTYPES = (torch.float16, torch.bfloat16, torch.float32)

# Activation codes of tk_activation_fwd / tk_activation_bwd.
_RELU, _GELU, _SILU, _TANH = 0, 1, 2, 3


def _validate_input(x: torch.Tensor) -> None:
    """Shared elementwise-activation contract."""
    if x.ndim != 2:
        raise ValueError("activation expects a 2D tensor shaped (rows, columns)")
    rows, columns = x.shape
    if rows == 0 or columns == 0:
        raise ValueError("activation does not support empty dimensions")
    if x.device.type != "cuda":
        raise ValueError("activation requires CUDA (ROCm/HIP) tensors")
    if x.dtype not in _DTYPES:
        raise ValueError("activation supports float16, bfloat16 and float32 tensors")
    if x.stride(1) != 1:
        raise ValueError("activation requires a contiguous final dimension")
    assert_int32_addressable(x, name="input")


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


def _launch_forward(x: torch.Tensor, output: torch.Tensor, *, activation: int) -> None:
    """Forward into a supplied output."""
    _validate_input(x)
    _validate_output(output, x, name="output")
    rows, columns = x.shape
    _hip.call(
        "tk_activation_fwd", _hip.dtype_code(x.dtype), activation, x.data_ptr(),
        output.data_ptr(), rows, columns, x.stride(0), output.stride(0), _hip.stream_of(x),
    )


def _launch_backward(dy: torch.Tensor, x: torch.Tensor, *, activation: int) -> torch.Tensor:
    """Deterministic backward; returns dx."""
    _validate_input(x)
    if dy.shape != x.shape or dy.device != x.device or dy.dtype != x.dtype:
        raise ValueError("upstream gradient metadata must match the input")
    if dy.stride(1) != 1:
        dy = dy.contiguous()
    assert_int32_addressable(dy, name="upstream gradient")
    rows, columns = x.shape
    dx = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _hip.call(
        "tk_activation_bwd", _hip.dtype_code(x.dtype), activation, dy.data_ptr(), x.data_ptr(),
        dx.data_ptr(), rows, columns, dy.stride(0), x.stride(0), dx.stride(0), _hip.stream_of(x),
    )
    return dx


class _ActivationFunction(torch.autograd.Function):
    """Autograd bridge shared by the four activations."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, activation: int) -> torch.Tensor:
        _validate_input(x)
        output = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        _launch_forward(x, output, activation=activation)
        ctx.save_for_backward(x)
        ctx.activation = activation
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, dy: torch.Tensor) -> tuple[torch.Tensor, None]:
        (x,) = ctx.saved_tensors
        return _launch_backward(dy, x, activation=ctx.activation), None


def _apply(x: torch.Tensor, activation: int) -> torch.Tensor:
    return cast(torch.Tensor, _ActivationFunction.apply(x, activation))


def relu(x: torch.Tensor) -> torch.Tensor:
    """``max(x, 0)``."""
    return _apply(x, _RELU)


def gelu(x: torch.Tensor) -> torch.Tensor:
    """Exact GELU ``0.5 x (1 + erf(x / sqrt(2)))``."""
    return _apply(x, _GELU)


def silu(x: torch.Tensor) -> torch.Tensor:
    """``x * sigmoid(x)``."""
    return _apply(x, _SILU)


def tanh(x: torch.Tensor) -> torch.Tensor:
    """``tanh(x)``."""
    return _apply(x, _TANH)


def _make_inputs(columns: int, device: torch.device, dtype: torch.dtype) -> TensorArgs:
    return (torch.randn(_ROWS, columns, device=device, dtype=dtype),)


def _make_adversarial(device: torch.device) -> TensorArgs:
    """Row-strided float32 input, 37 x 1000."""
    return (torch.randn(74, 1000, device=device, dtype=torch.float32)[::2],)


def _make_output(args: TensorArgs) -> torch.Tensor:
    x = args[0]
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


def _bytes_moved(columns: int, dtype: torch.dtype) -> int:
    """One read plus one write."""
    return 2 * _ROWS * columns * torch.empty((), dtype=dtype).element_size()


def _naive_relu(x: torch.Tensor) -> torch.Tensor:
    return torch.where(x > 0, x, 0.0)


def _naive_gelu(x: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    return (0.5 * xf * (1.0 + torch.erf(xf / math.sqrt(2.0)))).to(x.dtype)


def _naive_silu(x: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.sigmoid(xf)).to(x.dtype)


def _naive_tanh(x: torch.Tensor) -> torch.Tensor:
    xf = x.float()
    return (2.0 * torch.sigmoid(2.0 * xf) - 1.0).to(x.dtype)


def _register_activation(
    *, name: str, activation: int, triton_fn: TensorFn, ref_fn: TensorFn, naive_fn: TensorFn,
    reference_baseline: str, naive_baseline: str, description: str,
) -> KernelSpec:
    """Register one activation with the shared harness wiring."""

    def launch(args: TensorArgs, output: torch.Tensor) -> None:
        _launch_forward(args[0], output, activation=activation)

    def benchmark_call(args: TensorArgs, output: torch.Tensor) -> BenchmarkCall:
        return partial(_launch_forward, args[0], output, activation=activation)

    def benchmark_metadata(columns: int, dtype: torch.dtype) -> dict[str, BenchmarkScalar]:
        del columns, dtype
        return {
            "reference_baseline": reference_baseline,
            "naive_baseline": naive_baseline,
            "reference_allocates_output": True,
            "naive_allocates_output": True,
        }

    return register(
        KernelSpec(
            name=name,
            description=description,
            triton_fn=triton_fn,
            launch_fn=launch,
            ref_fn=ref_fn,
            make_inputs=_make_inputs,
            make_output=_make_output,
            make_adversarial=_make_adversarial,
            sizes=(128, 256, 512, 1024, 2048, 4096, 8192, 16384),
            correctness_sizes=(128, 1024, 4096),
            bound="memory",
            bytes_moved=_bytes_moved,
            dtypes=(torch.float16, torch.bfloat16),
            naive_fn=naive_fn,
            benchmark_metadata=benchmark_metadata,
            benchmark_call_factory=benchmark_call,
            supports_interpreter=False,
        )
    )


RELU = _register_activation(
    name="relu_forward", activation=_RELU, triton_fn=relu, ref_fn=torch.relu,
    naive_fn=_naive_relu, reference_baseline="torch.relu",
    naive_baseline="torch.where(x > 0, x, 0)",
    description="Elementwise ReLU with deterministic autograd.",
)
GELU = _register_activation(
    name="gelu_forward", activation=_GELU, triton_fn=gelu, ref_fn=F.gelu,
    naive_fn=_naive_gelu, reference_baseline='torch.nn.functional.gelu(approximate="none")',
    naive_baseline="explicit FP32 erf GELU composition",
    description="Elementwise exact (erf) GELU with deterministic autograd.",
)
SILU = _register_activation(
    name="silu_forward", activation=_SILU, triton_fn=silu, ref_fn=F.silu,
    naive_fn=_naive_silu, reference_baseline="torch.nn.functional.silu",
    naive_baseline="explicit FP32 x * sigmoid(x) composition",
    description="Elementwise SiLU/swish with deterministic autograd.",
)
TANH = _register_activation(
    name="tanh_forward", activation=_TANH, triton_fn=tanh, ref_fn=torch.tanh,
    naive_fn=_naive_tanh, reference_baseline="torch.tanh",
    naive_baseline="explicit FP32 2 * sigmoid(2x) - 1 composition",
    description="Elementwise tanh with deterministic autograd.",
)
