"""Registry benchmark runner and roofline metrics.

What stays the reference's contract (``src/tklab/harness/bench.py``): the ``BenchRow``
field names, the ``bench_spec`` signature its CLI calls (``cli.py:153``) and the
formulas of ``_add_performance_metrics`` its tests pin (``tests/test_bench.py:17-44``).

How it runs here. Each (dtype, size) point of a spec is a :class:`_Case`: up to three
zero-argument *subjects* over one set of preallocated inputs and one output — the HIP
kernel, the spec's PyTorch reference and, when the spec has one, its naive
decomposition. One :class:`_Clock` times every subject with HIP events
(:func:`tklab.harness.timing.time_ms`: a warmup of about ``warmup_ms``, then single
launches for about ``repetition_ms``, each after a cache flush). The row is assembled by
:func:`_compose_row`, which lays the spec's benchmark metadata down first and the
identity, timing and roofline fields over it, so no metadata key can rename a row.
"""

from __future__ import annotations

import itertools
from collections.abc import Callable
from dataclasses import dataclass
from typing import TypedDict, cast

import torch
from typing_extensions import NotRequired

from tklab.harness.timing import time_ms
from tklab.registry import KernelSpec, TensorArgs


class BenchRow(TypedDict):
    """One serialized benchmark observation; field names as the reference's
    (``bench.py:16-50``), which its CLI and plotters read."""

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


Subject = Callable[[], object]


@dataclass(frozen=True)
class _Case:
    """The subjects timed at one (dtype, size) point, all over the same tensors.

    ``kernel`` is the spec's benchmark call (or its allocation-free launcher);
    ``reference`` the PyTorch reference without its allocation where the spec offers
    that (a reference call factory or launcher), else ``ref_fn`` itself; ``naive`` the
    naive decomposition, or None.
    """

    kernel: Subject
    reference: Subject
    naive: Subject | None

    @classmethod
    def of(cls, spec: KernelSpec, args: TensorArgs, output: torch.Tensor) -> _Case:
        def pick(factory, launcher, plain) -> Subject | None:
            if factory is not None:
                return factory(args, output)
            if launcher is not None:
                return lambda: launcher(args, output)
            if plain is not None:
                return lambda: plain(*args)
            return None

        kernel = pick(spec.benchmark_call_factory, spec.launch_fn, None)
        reference = pick(spec.reference_call_factory, spec.reference_launch_fn, spec.ref_fn)
        naive = pick(spec.naive_call_factory, None, spec.naive_fn)
        assert kernel is not None and reference is not None  # launch_fn, ref_fn are required
        return cls(kernel=kernel, reference=reference, naive=naive)


@dataclass(frozen=True)
class _Clock:
    """HIP-event timing policy shared by every subject of a benchmark run."""

    device: torch.device
    warmup_ms: int
    repetition_ms: int

    def median(self, subject: Subject) -> float:
        return cast(float, time_ms(subject, warmup_ms=self.warmup_ms,
                                   repetition_ms=self.repetition_ms, device=self.device))

    def median_and_spread(self, subject: Subject) -> tuple[float, float, float]:
        """(median, 20th percentile, 80th percentile) in ms."""
        mid, lo, hi = cast(list[float], time_ms(
            subject, warmup_ms=self.warmup_ms, repetition_ms=self.repetition_ms,
            quantiles=(0.5, 0.2, 0.8), device=self.device))
        return mid, lo, hi


@dataclass(frozen=True)
class _Timings:
    """Measured milliseconds of one case."""

    ms: float
    ms_lo: float
    ms_hi: float
    torch_ms: float
    naive_ms: float | None


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
    """One :class:`BenchRow` per (dtype, size) of ``spec``, dtypes outermost.

    ``peak_bw_gbps`` prices memory-bound specs; ``theoretical_tflops`` (and, when given,
    the BLAS roof ``cublas_tflops``) price compute-bound ones. ``warmup_ms`` and
    ``repetition_ms`` set the timing budget of every subject.

    Raises:
        ValueError: On a negative device or a non-positive duration, or when the spec's
            bound has no cost model or no roof.
        RuntimeError: When the GPU ``device`` is not available.
    """
    _validate_benchmark_request(device=device, warmup_ms=warmup_ms, repetition_ms=repetition_ms)
    clock = _Clock(torch.device("cuda", device), warmup_ms, repetition_ms)
    rows: list[BenchRow] = []
    for dtype, size in itertools.product(spec.dtypes, spec.sizes):
        args = spec.make_inputs(size, clock.device, dtype)
        output = spec.make_output(args)
        case = _Case.of(spec, args, output)
        ms, ms_lo, ms_hi = clock.median_and_spread(case.kernel)
        timings = _Timings(ms=ms, ms_lo=ms_lo, ms_hi=ms_hi,
                           torch_ms=clock.median(case.reference),
                           naive_ms=None if case.naive is None else clock.median(case.naive))
        rows.append(_compose_row(spec, size=size, dtype=dtype, timings=timings,
                                 peak_bw_gbps=peak_bw_gbps, cublas_tflops=cublas_tflops,
                                 theoretical_tflops=theoretical_tflops))
        del case, args, output
    return rows


def _compose_row(
    spec: KernelSpec,
    *,
    size: int,
    dtype: torch.dtype,
    timings: _Timings,
    peak_bw_gbps: float | None,
    cublas_tflops: float | None,
    theoretical_tflops: float | None,
) -> BenchRow:
    """The row of one measured case: metadata, then identity and timings, then metrics.

    The spec's ``benchmark_metadata`` goes in first, so its keys (tile shapes, the MFMA
    opcode, baseline labels) cannot replace ``kernel``, ``dtype``, ``size`` or a timing.
    """
    row = cast(BenchRow, dict(spec.benchmark_metadata(size, dtype))
               if spec.benchmark_metadata is not None else {})
    row.update({
        "kernel": spec.name,
        "dtype": str(dtype).removeprefix("torch."),
        "size": size,
        "ms": timings.ms,
        "ms_lo": timings.ms_lo,
        "ms_hi": timings.ms_hi,
        "torch_ms": timings.torch_ms,
        "speedup": timings.torch_ms / timings.ms,
    })
    if timings.naive_ms is not None:
        row["naive_ms"] = timings.naive_ms
        row["speedup_vs_naive"] = timings.naive_ms / timings.ms
    _add_performance_metrics(row, spec=spec, size=size, dtype=dtype, milliseconds=timings.ms,
                             peak_bw_gbps=peak_bw_gbps, cublas_tflops=cublas_tflops,
                             theoretical_tflops=theoretical_tflops)
    return row


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
    """Price ``row`` against the roofs (the reference's formulas, ``bench.py:184-219``).

    Memory-bound: ``gbps`` = cost-model bytes / time and ``pct_peak`` its share of
    ``peak_bw_gbps``. Compute-bound: ``tflops`` and ``reference_tflops`` (same FLOPs over
    ``torch_ms``), ``pct_theoretical`` against ``theoretical_tflops`` and, when a BLAS roof
    is given, ``pct_cublas_same_size`` (kernel over reference) and ``pct_cublas_peak``.

    Raises:
        ValueError: If the spec lacks its cost model or the matching roof.
    """
    per_second = 1e3 / milliseconds
    if spec.bound == "memory":
        if spec.bytes_moved is None or peak_bw_gbps is None:
            raise ValueError(f"{spec.name}: missing memory cost model or bandwidth peak")
        row["gbps"] = spec.bytes_moved(size, dtype) * per_second / 1e9
        row["pct_peak"] = 100.0 * row["gbps"] / peak_bw_gbps
        return
    if spec.flops is None or theoretical_tflops is None:
        raise ValueError(f"{spec.name}: missing compute cost model or theoretical peak")
    teraflop = spec.flops(size, dtype) / 1e12
    row["tflops"] = teraflop * per_second
    row["reference_tflops"] = teraflop * 1e3 / row["torch_ms"]
    row["pct_theoretical"] = 100.0 * row["tflops"] / theoretical_tflops
    if cublas_tflops is not None:
        row["pct_cublas_same_size"] = 100.0 * row["tflops"] / row["reference_tflops"]
        row["pct_cublas_peak"] = 100.0 * row["tflops"] / cublas_tflops


def _validate_benchmark_request(*, device: int, warmup_ms: int, repetition_ms: int) -> None:
    """Reject a run that cannot produce rows, before any tensor is made.

    Raises:
        ValueError: If ``device`` is negative or a duration is not positive.
        RuntimeError: If this process sees no GPU with index ``device``.
    """
    problems = [f"{name} must be positive (got {value})"
                for name, value in (("warmup_ms", warmup_ms), ("repetition_ms", repetition_ms))
                if not value > 0]
    if device < 0:
        problems.insert(0, f"device index must be non-negative (got {device})")
    if problems:
        raise ValueError("; ".join(problems))
    visible = torch.cuda.device_count() if torch.cuda.is_available() else 0
    if device >= visible:
        raise RuntimeError(f"benchmarks need GPU {device}, but this process sees {visible} "
                           "ROCm/HIP device(s)")
