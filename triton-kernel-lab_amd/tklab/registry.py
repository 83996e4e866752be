"""Kernel registry: one :class:`KernelSpec` per kernel.

Tests, the benchmark harness and ``bench.py`` all consume the same spec, so a
kernel module only declares what to run, how to check it and how to price it.
The field names, the callable signatures and the construction invariants are
the reference's contract (``src/tklab/registry.py:16-186``) because the
reference's tests and tools address specs by those names.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping, Sequence
from dataclasses import dataclass, field
from typing import Literal, TypeAlias

import torch

TensorArgs: TypeAlias = tuple[torch.Tensor, ...]
BenchmarkScalar: TypeAlias = str | int | float | bool
InputFn: TypeAlias = Callable[[int, torch.device, torch.dtype], TensorArgs]
AdversarialFn: TypeAlias = Callable[[torch.device], TensorArgs]
TensorFn: TypeAlias = Callable[..., torch.Tensor]
LaunchFn: TypeAlias = Callable[[TensorArgs, torch.Tensor], None]
OutputFn: TypeAlias = Callable[[TensorArgs], torch.Tensor]
CostFn: TypeAlias = Callable[[int, torch.dtype], int]
AssertFn: TypeAlias = Callable[[torch.Tensor, torch.Tensor], None]
BenchmarkMetadataFn: TypeAlias = Callable[[int, torch.dtype], Mapping[str, BenchmarkScalar]]
BenchmarkCall: TypeAlias = Callable[[], object]
BenchmarkCallFactory: TypeAlias = Callable[[TensorArgs, torch.Tensor], BenchmarkCall]
Bound: TypeAlias = Literal["memory", "compute"]
ComputeMode: TypeAlias = Literal["fp16_fp32acc", "fp16_fp16acc", "attention_fp16_fp32acc"]

_COMPUTE_MODES = frozenset({"fp16_fp32acc", "fp16_fp16acc", "attention_fp16_fp32acc"})


def _check_sizes(sizes: Sequence[int], field_name: str) -> None:
    """Require a non-empty, duplicate-free sequence of positive ``int`` sizes."""
    valid = bool(sizes) and all(
        isinstance(size, int) and not isinstance(size, bool) and size > 0 for size in sizes
    )
    if not valid:
        raise ValueError(f"{field_name} must contain positive integers")
    if len(set(sizes)) != len(sizes):
        raise ValueError(f"{field_name} must not contain duplicates")


@dataclass(frozen=True, slots=True)
class KernelSpec:
    """How to run, check and price one kernel.

    ``triton_fn`` keeps the reference's field name; here it is the allocating
    public entry point whose device work runs in ``libtklab_hip.so``.
    ``launch_fn`` writes into a caller-provided output and allocates nothing.
    ``ref_fn`` is the PyTorch reference, evaluated on float32 upcasts.
    Memory-bound specs price a call with ``bytes_moved``; compute-bound specs
    with ``flops`` plus a ``compute_mode``.

    Raises:
        ValueError: on a malformed or self-contradicting specification.
    """

    name: str
    description: str
    triton_fn: TensorFn
    launch_fn: LaunchFn
    ref_fn: TensorFn
    make_inputs: InputFn
    make_output: OutputFn
    sizes: Sequence[int]
    bound: Bound
    bytes_moved: CostFn | None = None
    flops: CostFn | None = None
    dtypes: Sequence[torch.dtype] = field(default_factory=lambda: (torch.float16,))
    correctness_sizes: Sequence[int] | None = None
    make_adversarial: AdversarialFn | None = None
    naive_fn: TensorFn | None = None
    reference_launch_fn: LaunchFn | None = None
    assert_fn: AssertFn | None = None
    benchmark_metadata: BenchmarkMetadataFn | None = None
    benchmark_call_factory: BenchmarkCallFactory | None = None
    reference_call_factory: BenchmarkCallFactory | None = None
    naive_call_factory: BenchmarkCallFactory | None = None
    compute_mode: ComputeMode | None = None
    supports_interpreter: bool = True
    rtol: float | None = None
    atol: float | None = None

    def __post_init__(self) -> None:
        """Freeze sequences into tuples and enforce the spec invariants."""
        object.__setattr__(self, "sizes", tuple(self.sizes))
        if self.correctness_sizes is not None:
            object.__setattr__(self, "correctness_sizes", tuple(self.correctness_sizes))
        object.__setattr__(self, "dtypes", tuple(self.dtypes))

        if not self.name or not self.name.isidentifier():
            raise ValueError("kernel name must be a non-empty Python identifier")
        if not self.description.strip():
            raise ValueError(f"{self.name}: description must not be empty")
        _check_sizes(self.sizes, "sizes")
        if self.correctness_sizes is not None:
            _check_sizes(self.correctness_sizes, "correctness_sizes")
        if not self.dtypes:
            raise ValueError(f"{self.name}: at least one dtype is required")
        if not all(isinstance(dtype, torch.dtype) for dtype in self.dtypes):
            raise ValueError(f"{self.name}: dtypes must contain torch.dtype values")
        if len(set(self.dtypes)) != len(self.dtypes):
            raise ValueError(f"{self.name}: dtypes must not contain duplicates")

        if self.bound == "memory":
            if self.bytes_moved is None:
                raise ValueError(f"{self.name}: memory-bound kernels require bytes_moved")
            if self.flops is not None or self.compute_mode is not None:
                raise ValueError(f"{self.name}: memory-bound kernels cannot define compute metadata")
        elif self.bound == "compute":
            if self.flops is None or self.compute_mode is None:
                raise ValueError(f"{self.name}: compute-bound kernels require flops and compute_mode")
            if self.compute_mode not in _COMPUTE_MODES:
                raise ValueError(f"{self.name}: unsupported compute mode {self.compute_mode!r}")
        else:
            raise ValueError(f"{self.name}: unsupported bound {self.bound!r}")

    def validation_sizes(self) -> Sequence[int]:
        """Sizes used by correctness tests: the reduced set when one is given."""
        return self.correctness_sizes or self.sizes


REGISTRY: dict[str, KernelSpec] = {}


def register(spec: KernelSpec) -> KernelSpec:
    """Add ``spec`` to :data:`REGISTRY` and return it.

    Raises:
        ValueError: if a spec with the same name is already registered.
    """
    if spec.name in REGISTRY:
        raise ValueError(f"duplicate kernel: {spec.name}")
    REGISTRY[spec.name] = spec
    return spec
