"""Registry invariants (restates the checks of the reference's tests/test_registry.py)."""

from __future__ import annotations

import pytest
import torch

import tklab.kernels  # noqa: F401  (registers every spec)
from tklab.registry import REGISTRY, KernelSpec

EXPECTED_KERNELS = {
    "attention_causal",
    "attention_noncausal",
    "fused_softmax",
    "gelu_forward",
    "layer_norm_forward",
    "matmul_fp16acc",
    "matmul_fp32acc",
    "relu_forward",
    "residual_rms_norm_forward",
    "rms_norm_forward",
    "rope_forward",
    "silu_forward",
    "swiglu_forward",
    "tanh_forward",
    "vector_add",
}


def _spec(**changes: object) -> KernelSpec:
    """A minimal valid memory-bound spec with ``changes`` applied."""
    fields: dict[str, object] = dict(
        name="example_kernel",
        description="Example kernel used by unit tests.",
        triton_fn=lambda x: x,
        launch_fn=lambda args, out: out.copy_(args[0]),
        ref_fn=lambda x: x,
        make_inputs=lambda size, device, dtype: (torch.zeros(size, device=device, dtype=dtype),),
        make_output=lambda args: torch.empty_like(args[0]),
        sizes=(1, 2),
        bound="memory",
        bytes_moved=lambda size, dtype: size * torch.empty((), dtype=dtype).element_size(),
    )
    fields.update(changes)
    return KernelSpec(**fields)  # type: ignore[arg-type]


def test_registry_holds_exactly_the_reference_kernel_names() -> None:
    assert set(REGISTRY) == EXPECTED_KERNELS


@pytest.mark.parametrize(
    ("changes", "fragment"),
    [
        ({"name": ""}, "name"),
        ({"name": "not an identifier"}, "identifier"),
        ({"description": "   "}, "description"),
        ({"sizes": ()}, "sizes"),
        ({"sizes": (4, 4)}, "duplicates"),
        ({"sizes": (True, 2)}, "positive integers"),
        ({"sizes": (0, 2)}, "positive integers"),
        ({"correctness_sizes": (3, 3)}, "duplicates"),
        ({"dtypes": ()}, "at least one dtype"),
        ({"dtypes": (torch.float16, torch.float16)}, "dtypes"),
        ({"dtypes": ("float16",)}, "torch.dtype"),
        ({"bytes_moved": None}, "bytes_moved"),
        ({"compute_mode": "fp16_fp32acc"}, "compute metadata"),
        ({"flops": lambda size, dtype: size}, "compute metadata"),
        ({"bound": "other", "bytes_moved": None}, "unsupported bound"),
        ({"bound": "compute", "bytes_moved": None}, "require flops"),
        (
            {"bound": "compute", "bytes_moved": None, "flops": lambda s, d: s, "compute_mode": "x"},
            "unsupported compute mode",
        ),
    ],
)
def test_malformed_specs_are_rejected(changes: dict[str, object], fragment: str) -> None:
    with pytest.raises(ValueError, match=fragment):
        _spec(**changes)


def test_validation_sizes_fall_back_to_benchmark_sizes() -> None:
    assert tuple(_spec().validation_sizes()) == (1, 2)
    assert tuple(_spec(correctness_sizes=[2]).validation_sizes()) == (2,)


def test_sequences_are_frozen_to_tuples() -> None:
    spec = _spec(sizes=[1, 2], dtypes=[torch.float16], correctness_sizes=[1])
    assert spec.sizes == (1, 2)
    assert spec.dtypes == (torch.float16,)
    assert spec.correctness_sizes == (1,)


def test_duplicate_registration_is_rejected() -> None:
    from tklab.registry import register

    existing = next(iter(REGISTRY.values()))
    with pytest.raises(ValueError, match="duplicate kernel"):
        register(existing)


def test_every_registered_spec_prices_its_sizes() -> None:
    for spec in REGISTRY.values():
        for dtype in spec.dtypes:
            for size in spec.sizes:
                cost = spec.bytes_moved if spec.bound == "memory" else spec.flops
                assert cost is not None
                assert cost(size, dtype) > 0


def test_launch_metadata_names_the_kernels_that_launch() -> None:
    """The GEMM/attention metadata describe the DMA kernels every registry shape takes."""
    import torch

    from tklab.kernels import flash_attention, matmul

    gemm = REGISTRY["matmul_fp32acc"].benchmark_metadata(4096, torch.float16)
    assert gemm["hip_kernel"] == "gemm_dma_kernel"
    assert (gemm["block_k"], gemm["num_warps"], gemm["num_stages"]) == (32, 8, 4)
    assert gemm["mma_opcode"] == "v_mfma_f32_16x16x32_f16"
    attn = REGISTRY["attention_causal"].benchmark_metadata(1024, torch.float16)
    assert attn["hip_kernel"] == "attn_fwd_dma_kernel"
    assert (attn["block_m"], attn["block_n"], attn["num_warps"]) == (256, 64, 8)
    assert attn["mma_opcode"] == "v_mfma_f32_16x16x32_f16"
    a = torch.empty(64, 96, dtype=torch.bfloat16)
    b = torch.empty(96, 64, dtype=torch.bfloat16)
    assert matmul.launch_config(a, b)["hip_kernel"] == "gemm_dma_kernel"
    assert matmul.launch_config(a, b)["mma_opcode"] == "v_mfma_f32_16x16x32_bf16"
    assert matmul.launch_config(a[:, :80], b[:80])["hip_kernel"] == "gemm_kernel"
    assert matmul.launch_config(a, b.t().contiguous().t())["hip_kernel"] == "gemm_kernel"
    assert flash_attention.FORWARD_TILE["num_stages"] == 4
