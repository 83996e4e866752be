"""Strided 1-D vector addition on ``tk_vector_add`` (registry kernel).

Contract of ``src/tklab/kernels/vector_add.py``: two 1-D tensors of one
shape, device and dtype (float16/float32, here also bfloat16), any strides
including 0, a contiguous output; validation order and messages as in
``vector_add.py:56-74``.
"""

from __future__ import annotations

import torch

from tklab import _hip
from tklab.harness.addressing import assert_int32_addressable
from tklab.registry import BenchmarkScalar, KernelSpec, TensorArgs, register

_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def vector_add(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Elementwise ``x + y`` of two 1-D GPU tensors into a contiguous output."""
    _validate_inputs(x, y)
    output = _make_output((x, y))
    _launch((x, y), output)
    return output


def _validate_inputs(x: torch.Tensor, y: torch.Tensor) -> None:
    """Shape, device, dtype and address-width contract."""
    if x.ndim != 1 or y.ndim != 1:
        raise ValueError("vector_add expects one-dimensional tensors")
    if x.numel() == 0:
        raise ValueError("vector_add does not support empty tensors")
    if x.shape != y.shape:
        raise ValueError(f"shape mismatch: {x.shape} != {y.shape}")
    if x.device != y.device:
        raise ValueError(f"device mismatch: {x.device} != {y.device}")
    if x.dtype != y.dtype:
        raise ValueError(f"dtype mismatch: {x.dtype} != {y.dtype}")
    if x.dtype not in _DTYPES:
        raise ValueError("vector_add supports float16, bfloat16 and float32 tensors")
    if x.device.type != "cuda":
        raise ValueError("vector_add requires CUDA (ROCm/HIP) tensors")
    assert_int32_addressable(x, name="left input")
    assert_int32_addressable(y, name="right input")


def _make_output(args: TensorArgs) -> torch.Tensor:
    """Contiguous output (an expanded input's zero stride must not alias the output)."""
    x = args[0]
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


def _launch(args: TensorArgs, output: torch.Tensor) -> None:
    """Add into a preallocated contiguous output."""
    x, y = args
    _validate_inputs(x, y)
    if output.shape != x.shape or output.device != x.device or output.dtype != x.dtype:
        raise ValueError("output metadata must match the inputs")
    if not output.is_contiguous():
        raise ValueError("vector_add output must be contiguous")
    assert_int32_addressable(output, name="output")
    _hip.call(
        "tk_vector_add", _hip.dtype_code(x.dtype), x.data_ptr(), y.data_ptr(), output.data_ptr(),
        x.numel(), x.stride(0), y.stride(0), output.stride(0), _hip.stream_of(x),
    )


def _launch_reference(args: TensorArgs, output: torch.Tensor) -> None:
    """Allocation-free PyTorch add."""
    x, y = args
    torch.add(x, y, out=output)


def _naive_vector_add(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Copy followed by an in-place add."""
    return x.clone().add_(y)


def _make_inputs(size: int, device: torch.device, dtype: torch.dtype) -> TensorArgs:
    """Two standard-normal vectors."""
    return (
        torch.randn(size, device=device, dtype=dtype),
        torch.randn(size, device=device, dtype=dtype),
    )


def _make_adversarial(device: torch.device) -> TensorArgs:
    """Strided views (steps 2 and 3) of length 1009."""
    size = 1009
    left = torch.randn(size * 2, device=device, dtype=torch.float32)[::2]
    right = torch.randn(size * 3, device=device, dtype=torch.float32)[::3]
    return left, right


def _bytes_moved(size: int, dtype: torch.dtype) -> int:
    """Two reads plus one write."""
    return 3 * size * torch.empty((), dtype=dtype).element_size()


def _benchmark_metadata(size: int, dtype: torch.dtype) -> dict[str, BenchmarkScalar]:
    """Describe the two baselines."""
    del size, dtype
    return {
        "reference_baseline": "torch.add(..., out=preallocated_output)",
        "naive_baseline": "x.clone() followed by in-place add_(y)",
        "reference_allocates_output": False,
        "naive_allocates_output": True,
    }


VECTOR_ADD = register(
    KernelSpec(
        name="vector_add",
        description="Strided elementwise vector addition with masked tails.",
        triton_fn=vector_add,
        launch_fn=_launch,
        ref_fn=torch.add,
        reference_launch_fn=_launch_reference,
        make_inputs=_make_inputs,
        make_output=_make_output,
        sizes=tuple(2**exponent for exponent in range(12, 28)),
        correctness_sizes=(4096, 1 << 20, 1 << 24),
        bound="memory",
        bytes_moved=_bytes_moved,
        dtypes=(torch.float16, torch.float32, torch.bfloat16),
        make_adversarial=_make_adversarial,
        naive_fn=_naive_vector_add,
        benchmark_metadata=_benchmark_metadata,
        supports_interpreter=False,
    )
)
