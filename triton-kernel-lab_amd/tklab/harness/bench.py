"""Registry benchmark runner and roofline metrics.

Contract of ``src/tklab/harness/bench.py``: ``bench_spec`` times every dtype and size
of a :class:`~tklab.registry.KernelSpec` (median and 20th/80th percentiles), its
PyTorch reference and, when the spec has one, its naive decomposition, and
``_add_performance_metrics`` prices the row against the roofs: GB/s and percent of
the bandwidth peak for memory-bound specs; TFLOP/s, the reference's TFLOP/s and
percent of the theoretical ceiling for compute-bound ones, plus percent of the BLAS
library (hipBLASLt here, the ``cublas_*`` names kept) when a BLAS roof is given.
Timing is :func:`tklab.harness.timing.time_ms` (HIP events) in place of Triton's
``do_bench``.
"""

from __future__ import annotations

from collections.abc import Callable
from functools import partial
from typing import TypedDict, cast

import torch
from typing_extensions import NotRequired

from tklab.harness.timing import time_ms
from tklab.registry import KernelSpec


class BenchRow(TypedDict):
    """One serialized benchmark observation (reference ``bench.py:16-50``)."""

    kernel: str
    dtype: str
    size: int
    ms: float
    ms_lo: float
    ms_hi: float
    torch_ms: float
    speedup: float
    gbps: NotRequired[float]
    tflops: NotRequired[float]
    pct_peak: NotRequired[float]
    naive_ms: NotRequired[float]
    speedup_vs_naive: NotRequired[float]
    reference_baseline: NotRequired[str]
    naive_baseline: NotRequired[str]
    reference_allocates_output: NotRequired[bool]
    naive_allocates_output: NotRequired[bool]
    reference_tflops: NotRequired[float]
    pct_cublas_same_size: NotRequired[float]
    pct_cublas_peak: NotRequired[float]
    pct_theoretical: NotRequired[float]
    block_m: NotRequired[int]
    block_n: NotRequired[int]
    block_k: NotRequired[int]
    group_m: NotRequired[int]
    num_warps: NotRequired[int]
    num_stages: NotRequired[int]
    mma_opcode: NotRequired[str]
    heads: NotRequired[int]
    head_dim: NotRequired[int]
    causal: NotRequired[bool]


def bench_spec(
    spec: KernelSpec,
    *,
    peak_bw_gbps: float | None,
    cublas_tflops: float | None,
    theoretical_tflops: float | None,
    device: int = 0,
    warmup_ms: int = 25,
    repetition_ms: int = 100,
) -> list[BenchRow]:
    """Benchmark every dtype and size of ``spec`` (reference ``bench.py:53-153``).

    Args:
        spec: Kernel contract to benchmark.
        peak_bw_gbps: Measured bandwidth roof for memory-bound kernels.
        cublas_tflops: Optional practical BLAS (hipBLASLt) roof.
        theoretical_tflops: Clock-scaled compute ceiling.
        device: GPU index.
        warmup_ms: Approximate warmup duration per timing.
        repetition_ms: Approximate measured duration per timing.

    Raises:
        ValueError: If timing parameters or required roofs are invalid.
        RuntimeError: If the selected GPU is unavailable.
    """
    _validate_benchmark_request(device=device, warmup_ms=warmup_ms, repetition_ms=repetition_ms)
    rows: list[BenchRow] = []
    torch_device = torch.device("cuda", device)
    timing = {"warmup_ms": warmup_ms, "repetition_ms": repetition_ms, "device": torch_device}
    for dtype in spec.dtypes:
        for size in spec.sizes:
            args = spec.make_inputs(size, torch_device, dtype)
            output = spec.make_output(args)
            launch = (
                spec.benchmark_call_factory(args, output)
                if spec.benchmark_call_factory is not None
                else partial(spec.launch_fn, args, output)
            )
            median_ms, low_ms, high_ms = cast(
                list[float], time_ms(launch, quantiles=[0.5, 0.2, 0.8], **timing)
            )
            torch_ms = _benchmark_reference(spec, args=args, output=output, **timing)
            row: BenchRow = {
                "kernel": spec.name,
                "dtype": str(dtype).removeprefix("torch."),
                "size": size,
                "ms": median_ms,
                "ms_lo": low_ms,
                "ms_hi": high_ms,
                "torch_ms": torch_ms,
                "speedup": torch_ms / median_ms,
            }
            if spec.benchmark_metadata is not None:
                row.update(cast(BenchRow, dict(spec.benchmark_metadata(size, dtype))))
            naive_call: Callable[[], object] | None = None
            if spec.naive_call_factory is not None:
                naive_call = spec.naive_call_factory(args, output)
            elif spec.naive_fn is not None:
                naive_call = partial(spec.naive_fn, *args)
            if naive_call is not None:
                naive_ms = cast(float, time_ms(naive_call, **timing))
                row["naive_ms"] = naive_ms
                row["speedup_vs_naive"] = naive_ms / median_ms
            _add_performance_metrics(
                row,
                spec=spec,
                size=size,
                dtype=dtype,
                milliseconds=median_ms,
                peak_bw_gbps=peak_bw_gbps,
                cublas_tflops=cublas_tflops,
                theoretical_tflops=theoretical_tflops,
            )
            rows.append(row)
    return rows


def _benchmark_reference(
    spec: KernelSpec,
    *,
    args: tuple[torch.Tensor, ...],
    output: torch.Tensor,
    warmup_ms: int,
    repetition_ms: int,
    device: torch.device,
) -> float:
    """Median time of the PyTorch reference, without its allocation where the spec
    allows (reference ``bench.py:156-181``)."""
    reference_call: Callable[[], object]
    if spec.reference_call_factory is not None:
        reference_call = spec.reference_call_factory(args, output)
    elif spec.reference_launch_fn is not None:
        reference_call = partial(spec.reference_launch_fn, args, output)
    else:
        reference_call = partial(spec.ref_fn, *args)
    return cast(
        float,
        time_ms(reference_call, warmup_ms=warmup_ms, repetition_ms=repetition_ms, device=device),
    )


def _add_performance_metrics(
    row: BenchRow,
    *,
    spec: KernelSpec,
    size: int,
    dtype: torch.dtype,
    milliseconds: float,
    peak_bw_gbps: float | None,
    cublas_tflops: float | None,
    theoretical_tflops: float | None,
) -> None:
    """Add roofline metrics to ``row`` (reference ``bench.py:184-219``).

    Raises:
        ValueError: If the spec lacks its cost model or the matching roof.
    """
    seconds = milliseconds * 1e-3
    if spec.bound == "memory":
        if spec.bytes_moved is None or peak_bw_gbps is None:
            raise ValueError(f"{spec.name}: missing memory cost model or bandwidth peak")
        gbps = spec.bytes_moved(size, dtype) / seconds / 1e9
        row["gbps"] = gbps
        row["pct_peak"] = 100.0 * gbps / peak_bw_gbps
        return
    if spec.flops is None or theoretical_tflops is None:
        raise ValueError(f"{spec.name}: missing compute cost model or theoretical peak")
    flops = spec.flops(size, dtype)
    tflops = flops / seconds / 1e12
    reference_tflops = flops / (row["torch_ms"] * 1e-3) / 1e12
    row["tflops"] = tflops
    row["reference_tflops"] = reference_tflops
    row["pct_theoretical"] = 100.0 * tflops / theoretical_tflops
    if cublas_tflops is not None:
        row["pct_cublas_same_size"] = 100.0 * tflops / reference_tflops
        row["pct_cublas_peak"] = 100.0 * tflops / cublas_tflops


def _validate_benchmark_request(*, device: int, warmup_ms: int, repetition_ms: int) -> None:
    """Validate runtime parameters (reference ``bench.py:222-243``).

    Raises:
        ValueError: If an index is negative or a duration is not positive.
        RuntimeError: If no GPU or the selected one is unavailable.
    """
    if device < 0:
        raise ValueError("device index must be non-negative")
    if warmup_ms <= 0 or repetition_ms <= 0:
        raise ValueError("warmup and repetition durations must be positive")
    if not torch.cuda.is_available():
        raise RuntimeError("a GPU (ROCm/HIP) is required for GPU benchmarks")
    if device >= torch.cuda.device_count():
        raise RuntimeError(
            f"GPU device {device} is unavailable; found {torch.cuda.device_count()} device(s)"
        )
