"""Row-wise single-pass softmax on the HIP ``tk_softmax_fwd`` kernel.

Public contract of ``src/tklab/kernels/fused_softmax.py``: ``softmax(x)`` for a
2-D tensor with a unit-stride final dimension and at most 65 536 columns; the
validation order and messages are the reference's (``fused_softmax.py:68-87``).
bfloat16 is accepted in addition to float16 and float32.

``online_softmax(x)`` is the path the reference's width check names for rows
beyond that limit (``fused_softmax.py:75-79``): the same function of each row,
computed over 16 384-column chunks (``tk_softmax_online_fwd``) for any width up
to 2^31 - 1 columns.
"""

from __future__ import annotations

import torch

from tklab import _hip
from tklab.harness.addressing import assert_int32_addressable
from tklab.registry import BenchmarkScalar, KernelSpec, TensorArgs, register

_ROWS = 4096
_MAX_FUSED_COLUMNS = 1 << 16
_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def softmax(x: torch.Tensor) -> torch.Tensor:
    """Softmax over the final dimension of a 2-D tensor.

    Args:
        x: ``(rows, columns)`` tensor, float16/bfloat16/float32; any row stride,
            unit column stride.

    Returns:
        Probabilities with the shape, dtype and device of ``x``.

    Raises:
        ValueError: on an unsupported shape, dtype, layout or device.
    """
    _validate(x)
    output = _make_output((x,))
    _launch((x,), output)
    return output


def online_softmax(x: torch.Tensor) -> torch.Tensor:
    """Softmax over the final dimension of a 2-D tensor of any width.

    Same contract as :func:`softmax` without the 65 536-column limit. Each row is
    reduced over 16 384-column chunks whose (max, sum of exp) partials are folded
    in a fixed order, so results are deterministic; they match :func:`softmax`
    to float32 rounding of the row sum.

    Raises:
        ValueError: on an unsupported shape, dtype, layout or device.
    """
    _validate(x, single_pass=False)
    output = _make_output((x,))
    _launch_online((x,), output)
    return output


def _launch_online(args: TensorArgs, output: torch.Tensor) -> None:
    """Run the online softmax into a preallocated output."""
    (x,) = args
    _validate(x, single_pass=False)
    if output.shape != x.shape or output.device != x.device or output.dtype != x.dtype:
        raise ValueError("output metadata must match the input")
    if output.stride(1) != 1:
        raise ValueError("softmax output requires a contiguous final dimension")
    assert_int32_addressable(output, name="output")
    rows, columns = x.shape
    chunks = -(-columns // ONLINE_CHUNK_COLUMNS)
    partials = torch.empty(2 * rows * chunks, device=x.device, dtype=torch.float32)
    _hip.call(
        "tk_softmax_online_fwd",
        _hip.dtype_code(x.dtype),
        x.data_ptr(),
        output.data_ptr(),
        partials.data_ptr(),
        rows,
        columns,
        x.stride(0),
        output.stride(0),
        _hip.stream_of(x),
    )


# Columns per chunk of tk_softmax_online_fwd (256 threads x 64 values); the
# workspace holds two floats per chunk.
ONLINE_CHUNK_COLUMNS = 16384


def _validate(x: torch.Tensor, *, single_pass: bool = True) -> None:
    """Check the single-pass softmax contract (reference ``fused_softmax.py:68-87``).

    ``single_pass=False`` drops the width limit (the online path).
    """
    if x.ndim != 2:
        raise ValueError("softmax expects a 2D tensor shaped (rows, columns)")
    rows, columns = x.shape
    if rows == 0 or columns == 0:
        raise ValueError("softmax does not support empty dimensions")
    if single_pass and columns > _MAX_FUSED_COLUMNS:
        raise ValueError(
            f"n_cols={columns} exceeds the {_MAX_FUSED_COLUMNS}-column "
            "single-pass limit; use an online softmax"
        )
    if x.stride(1) != 1:
        raise ValueError("softmax requires a contiguous final dimension")
    if x.dtype not in _DTYPES:
        raise ValueError("softmax supports float16, bfloat16 and float32 tensors")
    if x.device.type != "cuda":
        raise ValueError("softmax requires CUDA (ROCm/HIP) tensors")
    assert_int32_addressable(x, name="input")


def _make_output(args: TensorArgs) -> torch.Tensor:
    """Allocate an output with the input's memory format."""
    return torch.empty_like(args[0])


def _launch(args: TensorArgs, output: torch.Tensor) -> None:
    """Run softmax into a preallocated output (reference ``fused_softmax.py:104-124``)."""
    (x,) = args
    _validate(x)
    if output.shape != x.shape or output.device != x.device or output.dtype != x.dtype:
        raise ValueError("output metadata must match the input")
    if output.stride(1) != 1:
        raise ValueError("softmax output requires a contiguous final dimension")
    assert_int32_addressable(output, name="output")
    rows, columns = x.shape
    _hip.call(
        "tk_softmax_fwd",
        _hip.dtype_code(x.dtype),
        x.data_ptr(),
        output.data_ptr(),
        rows,
        columns,
        x.stride(0),
        output.stride(0),
        _hip.stream_of(x),
    )


def _torch_softmax(x: torch.Tensor) -> torch.Tensor:
    """PyTorch reference."""
    return torch.softmax(x, dim=-1)


def _launch_reference(args: TensorArgs, output: torch.Tensor) -> None:
    """Allocation-free PyTorch softmax."""
    (x,) = args
    torch.softmax(x, dim=-1, out=output)


def _make_inputs(n_cols: int, device: torch.device, dtype: torch.dtype) -> TensorArgs:
    """``(4096, n_cols)`` standard-normal input."""
    return (torch.randn(_ROWS, n_cols, device=device, dtype=dtype),)


def _bytes_moved(n_cols: int, dtype: torch.dtype) -> int:
    """One read plus one write of the matrix."""
    element_size = torch.empty((), dtype=dtype).element_size()
    return 2 * _ROWS * n_cols * element_size


def _make_adversarial(device: torch.device) -> TensorArgs:
    """Row-strided view with a non-power-of-two width (32 x 1000 of a 64 x 1000 draw)."""
    x = torch.randn(64, 1000, device=device, dtype=torch.float32)
    return (x[::2],)


def _naive_softmax(x: torch.Tensor) -> torch.Tensor:
    """Unfused max / subtract / exp / sum / divide composition."""
    shifted = x - x.max(dim=-1, keepdim=True).values
    numerator = shifted.exp()
    return numerator / numerator.sum(dim=-1, keepdim=True)


def _benchmark_metadata(n_cols: int, dtype: torch.dtype) -> dict[str, BenchmarkScalar]:
    """Describe the two baselines."""
    del n_cols, dtype
    return {
        "reference_baseline": "torch.softmax(..., out=preallocated_output)",
        "naive_baseline": "explicit max, subtract, exp, sum, and divide composition",
        "reference_allocates_output": False,
        "naive_allocates_output": True,
    }


SOFTMAX = register(
    KernelSpec(
        name="fused_softmax",
        description="Single-pass row-wise softmax with FP32 reductions.",
        triton_fn=softmax,
        launch_fn=_launch,
        ref_fn=_torch_softmax,
        reference_launch_fn=_launch_reference,
        make_inputs=_make_inputs,
        make_output=_make_output,
        make_adversarial=_make_adversarial,
        sizes=(128, 256, 512, 1024, 2048, 4096, 8192, 16384),
        bound="memory",
        bytes_moved=_bytes_moved,
        dtypes=(torch.float16, torch.float32, torch.bfloat16),
        naive_fn=_naive_softmax,
        benchmark_metadata=_benchmark_metadata,
        supports_interpreter=False,
    )
)
