"""GEMM on CDNA4 MFMA through ``tk_gemm``: ``matmul_fp32acc`` and ``matmul_fp16acc``.

Contract of ``src/tklab/kernels/matmul.py``: two 2-D matrices with matching
inner dimension, same device and dtype, strictly positive strides within the
int32 range, float16 (and here also bfloat16) inputs, a contiguous output of
the input dtype. Validation order and messages follow ``matmul.py:167-186``.

The reference autotunes 25 Triton configurations per shape
(``matmul.py:23-75``); this build has a static choice between two kernels and
reports the one a shape launches in the same metadata keys: row-major operands
with K % 32 == 0 (every registry shape) take ``gemm_dma_kernel`` (256 x 256
tiles, K step 32, eight wave64s, buffer->LDS rings of four 32-wide B stages and
three 64-wide A stages, ``v_mfma_f32_16x16x32``); strided operands or other K take the register-staged
``gemm_kernel`` (256 x 256 x 64, four wave64s, ``v_mfma_f32_32x32x16``).
``matmul_fp16acc`` keeps its registry entry, but gfx950 MFMA
accumulates f16 products in float32 only, so both entry points run the same
FP32-accumulate kernel (its result is at least as accurate as an FP16
accumulation and meets the looser 5e-2 bound the reference sets for it).
"""

from __future__ import annotations

import torch

from tklab import _hip
from tklab.harness.addressing import assert_int32_addressable
from tklab.harness.tolerances import assert_relative_frobenius
from tklab.registry import (
    BenchmarkMetadataFn,
    BenchmarkScalar,
    KernelSpec,
    LaunchFn,
    TensorArgs,
    register,
)

_DTYPES = (torch.float16, torch.bfloat16)

# csrc/gemm_dma.hip (BM, BN, BK, kGroupM, kThreads / 64 waves, kBStages): row-major operands
# with K % 32 == 0. "num_warps" counts wave64s; "num_stages" is the ring of 32-wide K steps
# (the B operand's; A is loaded in 64-wide tiles into a ring of kAStages = 3).
TILE = {"hip_kernel": "gemm_dma_kernel", "block_m": 256, "block_n": 256, "block_k": 32, "group_m": 4,
        "num_warps": 8, "num_stages": 4}
_MFMA = {
    torch.float16: "v_mfma_f32_16x16x32_f16",
    torch.bfloat16: "v_mfma_f32_16x16x32_bf16",
}
# csrc/gemm.hip's register-staged kernel: every other operand layout (double-buffered in registers).
FALLBACK_TILE = {"hip_kernel": "gemm_kernel", "block_m": 256, "block_n": 256, "block_k": 64,
                 "group_m": 4, "num_warps": 4, "num_stages": 2}
_FALLBACK_MFMA = {
    torch.float16: "v_mfma_f32_32x32x16_f16",
    torch.bfloat16: "v_mfma_f32_32x32x16_bf16",
}


def launch_config(a: torch.Tensor, b: torch.Tensor) -> dict[str, BenchmarkScalar]:
    """Tile configuration and MFMA of the kernel ``tk_gemm`` launches for ``a @ b``.

    Mirrors ``gemm_dma_applies`` (csrc/gemm_dma.hip): unit column strides, K % 32 == 0,
    N and both row strides multiples of 8, 16-byte aligned bases and operand extents
    under 2 GiB take the DMA kernel.
    """
    (m, k), n = a.shape, b.shape[1]
    dma = (
        a.stride(1) == 1
        and b.stride(1) == 1
        and k % 32 == 0
        and n % 8 == 0
        and a.stride(0) % 8 == 0
        and b.stride(0) % 8 == 0
        and a.data_ptr() % 16 == 0
        and b.data_ptr() % 16 == 0
        and ((m - 1) * a.stride(0) + k) * 2 < 2**31
        and ((k - 1) * b.stride(0) + n) * 2 < 2**31
    )
    if dma:
        return {**TILE, "mma_opcode": _MFMA.get(a.dtype, _MFMA[torch.float16])}
    return {**FALLBACK_TILE, "mma_opcode": _FALLBACK_MFMA.get(a.dtype, _FALLBACK_MFMA[torch.float16])}


def _validate(a: torch.Tensor, b: torch.Tensor) -> None:
    """GEMM input contract (reference ``matmul.py:167-186``)."""
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError("matmul expects two 2D tensors")
    if a.shape[1] != b.shape[0]:
        raise ValueError(f"incompatible shapes: {a.shape} and {b.shape}")
    if 0 in (*a.shape, *b.shape):
        raise ValueError("matmul does not support empty dimensions")
    if a.device != b.device:
        raise ValueError(f"device mismatch: {a.device} != {b.device}")
    if a.dtype != b.dtype:
        raise ValueError(f"dtype mismatch: {a.dtype} != {b.dtype}")
    if a.dtype not in _DTYPES:
        raise ValueError("matmul supports float16 and bfloat16 inputs only")
    for name, tensor in (("left", a), ("right", b)):
        if any(stride <= 0 for stride in tensor.stride()):
            raise ValueError(f"{name} input requires strictly positive strides")
        assert_int32_addressable(tensor, name=name)
    if a.device.type != "cuda":
        raise ValueError("matmul requires CUDA (ROCm/HIP) tensors")


def _make_output(args: TensorArgs) -> torch.Tensor:
    """Contiguous output of the input dtype."""
    a, b = args
    return torch.empty((a.shape[0], b.shape[1]), device=a.device, dtype=a.dtype)


def _launch_factory(*, fp16_accumulate: bool) -> LaunchFn:
    """Allocation-free launcher for one accumulation mode."""

    def launch(args: TensorArgs, output: torch.Tensor) -> None:
        a, b = args
        _validate(a, b)
        if output.shape != (a.shape[0], b.shape[1]):
            raise ValueError("output shape does not match matmul result")
        if output.device != a.device or output.dtype != a.dtype:
            raise ValueError("output metadata must match the inputs")
        if not output.is_contiguous():
            raise ValueError("matmul output must be contiguous")
        m, k = a.shape
        n = b.shape[1]
        _hip.call(
            "tk_gemm",
            _hip.dtype_code(a.dtype),
            a.data_ptr(),
            b.data_ptr(),
            output.data_ptr(),
            m,
            n,
            k,
            a.stride(0),
            a.stride(1),
            b.stride(0),
            b.stride(1),
            output.stride(0),
            output.stride(1),
            int(fp16_accumulate),
            _hip.stream_of(a),
        )

    return launch


_launch_fp32acc = _launch_factory(fp16_accumulate=False)
_launch_fp16acc = _launch_factory(fp16_accumulate=True)


def matmul_fp32acc(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a @ b`` with float32 MFMA accumulation."""
    _validate(a, b)
    output = _make_output((a, b))
    _launch_fp32acc((a, b), output)
    return output


def matmul_fp16acc(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Registry-compatible FP16-accumulate entry point (runs the FP32-accumulate kernel)."""
    _validate(a, b)
    output = _make_output((a, b))
    _launch_fp16acc((a, b), output)
    return output


def _launch_reference(args: TensorArgs, output: torch.Tensor) -> None:
    """Allocation-free PyTorch GEMM (hipBLASLt)."""
    a, b = args
    torch.mm(a, b, out=output)


def _make_inputs(size: int, device: torch.device, dtype: torch.dtype) -> TensorArgs:
    """Square standard-normal matrices."""
    return (
        torch.randn(size, size, device=device, dtype=dtype),
        torch.randn(size, size, device=device, dtype=dtype),
    )


def _make_adversarial(device: torch.device) -> TensorArgs:
    """Strided 129 x 193 @ 193 x 257: M, N and K tails at once."""
    left = torch.randn(129, 386, device=device, dtype=torch.float16)
    right = torch.randn(386, 257, device=device, dtype=torch.float16)
    return left[:, ::2], right[::2, :]


def _assert_fp32acc(output: torch.Tensor, reference: torch.Tensor) -> None:
    """Relative Frobenius error below 1e-2 (reference ``matmul.py:282-284``)."""
    assert_relative_frobenius(output, reference, max_relative_error=1e-2)


def _assert_fp16acc(output: torch.Tensor, reference: torch.Tensor) -> None:
    """Relative Frobenius error below 5e-2 (reference ``matmul.py:287-289``)."""
    assert_relative_frobenius(output, reference, max_relative_error=5e-2)


def _metadata_factory() -> BenchmarkMetadataFn:
    """Tile configuration in the reference's metadata keys (``matmul.py:292-312``)."""

    def metadata(size: int, dtype: torch.dtype) -> dict[str, BenchmarkScalar]:
        # Registry inputs are contiguous size x size matrices (size % 32 == 0).
        del size
        return {**TILE, "mma_opcode": _MFMA.get(dtype, _MFMA[torch.float16])}

    return metadata


_SIZES = (512, 1024, 2048, 4096, 8192)


def _flops(size: int, _dtype: torch.dtype) -> int:
    """``2 * M * N * K`` for a square problem."""
    return 2 * size**3


MATMUL_FP32ACC = register(
    KernelSpec(
        name="matmul_fp32acc",
        description="FP16/BF16 GEMM with FP32 MFMA accumulation.",
        triton_fn=matmul_fp32acc,
        launch_fn=_launch_fp32acc,
        ref_fn=torch.matmul,
        reference_launch_fn=_launch_reference,
        make_inputs=_make_inputs,
        make_output=_make_output,
        make_adversarial=_make_adversarial,
        sizes=_SIZES,
        correctness_sizes=(512, 1024),
        bound="compute",
        flops=_flops,
        dtypes=(torch.float16, torch.bfloat16),
        assert_fn=_assert_fp32acc,
        benchmark_metadata=_metadata_factory(),
        compute_mode="fp16_fp32acc",
        supports_interpreter=False,
    )
)

MATMUL_FP16ACC = register(
    KernelSpec(
        name="matmul_fp16acc",
        description="FP16 GEMM registry entry; MFMA accumulates in FP32 on gfx950.",
        triton_fn=matmul_fp16acc,
        launch_fn=_launch_fp16acc,
        ref_fn=torch.matmul,
        reference_launch_fn=_launch_reference,
        make_inputs=_make_inputs,
        make_output=_make_output,
        make_adversarial=_make_adversarial,
        sizes=_SIZES,
        correctness_sizes=(512, 1024),
        bound="compute",
        flops=_flops,
        dtypes=(torch.float16,),
        assert_fn=_assert_fp16acc,
        benchmark_metadata=_metadata_factory(),
        compute_mode="fp16_fp16acc",
        supports_interpreter=False,
    )
)
