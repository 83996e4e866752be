"""Pre-launch validation on CPU and meta tensors: no GPU, no library load.

Covers the message fragments the reference's tests pin
(tests/test_kernel_validation.py) for the hot-path entry points, plus the
order in which the checks fire.
"""

from __future__ import annotations

import pytest
import torch

from tklab.kernels.fused_softmax import softmax
from tklab.kernels.residual_rms_norm import residual_rms_norm
from tklab.kernels.rms_norm import _make_backward_buffers, rms_norm
from tklab.kernels.rope import rope
from tklab.kernels.swiglu import swiglu


def test_softmax_rejects_column_strided_rows() -> None:
    with pytest.raises(ValueError, match="contiguous final dimension"):
        softmax(torch.zeros(4, 8)[:, ::2])


def test_softmax_requires_a_gpu_tensor() -> None:
    with pytest.raises(ValueError, match="requires CUDA"):
        softmax(torch.zeros(2, 8))


def test_online_softmax_lifts_only_the_width_limit() -> None:
    from tklab.kernels.fused_softmax import online_softmax

    wide = torch.empty(2, 70000, device="meta")
    with pytest.raises(ValueError, match="use an online softmax"):
        softmax(wide)
    with pytest.raises(ValueError, match="requires CUDA"):
        online_softmax(wide)
    with pytest.raises(ValueError, match="2D tensor"):
        online_softmax(torch.empty(2, 3, 4, device="meta"))
    with pytest.raises(ValueError, match="empty dimensions"):
        online_softmax(torch.empty(0, 70000, device="meta"))
    with pytest.raises(ValueError, match="contiguous final dimension"):
        online_softmax(torch.empty(2, 140000, device="meta")[:, ::2])
    with pytest.raises(ValueError, match="float16, bfloat16 and float32"):
        online_softmax(torch.empty(2, 70000, device="meta", dtype=torch.float64))


@pytest.mark.parametrize(
    ("x", "fragment"),
    [
        (torch.zeros(8), "2D tensor"),
        (torch.zeros(0, 8), "empty"),
        (torch.zeros(2, 65537, device="meta"), "single-pass limit"),
        (torch.zeros(2, 8, dtype=torch.float64), "float16"),
    ],
)
def test_softmax_contract(x: torch.Tensor, fragment: str) -> None:
    with pytest.raises(ValueError, match=fragment):
        softmax(x)


def test_rms_norm_rejects_mismatched_weight() -> None:
    with pytest.raises(ValueError, match="match the final input dimension"):
        rms_norm(torch.zeros(2, 8), torch.ones(7))


@pytest.mark.parametrize("eps", [0.0, -1e-5, float("nan"), float("inf")])
def test_rms_norm_rejects_invalid_epsilon(eps: float) -> None:
    with pytest.raises(ValueError, match="finite and positive"):
        rms_norm(torch.zeros(2, 8), torch.ones(8), eps=eps)


def test_rms_norm_checks_weight_layout_before_device() -> None:
    with pytest.raises(ValueError, match="must be contiguous"):
        rms_norm(torch.zeros(2, 8), torch.ones(16)[::2])
    with pytest.raises(ValueError, match="requires CUDA"):
        rms_norm(torch.zeros(2, 8), torch.ones(8))


def test_rms_norm_rejects_rows_beyond_the_fused_budget() -> None:
    x = torch.zeros(2, 32769, dtype=torch.float16, device="meta")
    w = torch.zeros(32769, dtype=torch.float16, device="meta")
    with pytest.raises(ValueError):
        rms_norm(x, w)


def test_backward_buffers_keep_the_reference_layout() -> None:
    x = torch.zeros(1025, 1000)
    w = torch.zeros(1000)
    buffers = _make_backward_buffers(x, w, group_size=1)
    assert buffers.locks.tolist() == [0, 0]
    assert buffers.partial_dw.shape == (1, 1000)
    assert buffers.group_count == 1
    default = _make_backward_buffers(x, w)
    assert default.group_count == min(default.group_size, 1025)
    assert default.locks.shape == (2 * default.group_size,)
    with pytest.raises(ValueError, match="group_size must be positive"):
        _make_backward_buffers(x, w, group_size=0)


def test_residual_rms_norm_rejects_shape_mismatch() -> None:
    with pytest.raises(ValueError, match="residual must match"):
        residual_rms_norm(torch.zeros(2, 8), torch.zeros(3, 8), torch.ones(8))


def test_residual_rms_norm_rejects_invalid_epsilon() -> None:
    with pytest.raises(ValueError, match="finite and positive"):
        residual_rms_norm(torch.zeros(2, 8), torch.zeros(2, 8), torch.ones(8), eps=float("nan"))


def test_swiglu_rejects_shape_mismatch() -> None:
    with pytest.raises(ValueError, match="identical shapes"):
        swiglu(torch.zeros(2, 8), torch.zeros(3, 8))


def test_swiglu_requires_a_gpu_tensor() -> None:
    with pytest.raises(ValueError, match="requires CUDA"):
        swiglu(torch.zeros(2, 8), torch.zeros(2, 8))


def test_rope_rejects_odd_feature_dimension() -> None:
    with pytest.raises(ValueError, match="even feature dimension"):
        rope(torch.zeros(2, 7), torch.zeros(2, 3), torch.zeros(2, 3))


def test_rope_rejects_full_width_tables() -> None:
    with pytest.raises(ValueError, match="columns // 2"):
        rope(torch.zeros(2, 8), torch.zeros(2, 8), torch.zeros(2, 8))


# ---- registry kernels outside the hot path ---------------------------------

from tklab.kernels.activations import gelu  # noqa: E402
from tklab.kernels.flash_attention import attention_noncausal  # noqa: E402
from tklab.kernels.layer_norm import layer_norm  # noqa: E402
from tklab.kernels.matmul import matmul_fp32acc  # noqa: E402
from tklab.kernels.vector_add import vector_add  # noqa: E402


def test_vector_add_rejects_shape_mismatch() -> None:
    with pytest.raises(ValueError, match="shape mismatch"):
        vector_add(torch.zeros(2), torch.zeros(3))


def test_vector_add_requires_a_gpu_tensor() -> None:
    with pytest.raises(ValueError, match="requires CUDA"):
        vector_add(torch.zeros(2), torch.zeros(2))


def test_activation_contract() -> None:
    with pytest.raises(ValueError, match="2D tensor"):
        gelu(torch.zeros(3))
    with pytest.raises(ValueError, match="requires CUDA"):
        gelu(torch.zeros(2, 3))


def test_layer_norm_rejects_mismatched_parameters() -> None:
    with pytest.raises(ValueError, match="match the final input dimension"):
        layer_norm(torch.zeros(2, 8), torch.zeros(7), torch.zeros(8))


def test_layer_norm_rejects_strided_parameters() -> None:
    with pytest.raises(ValueError, match="must be contiguous"):
        layer_norm(torch.zeros(2, 8), torch.zeros(16)[::2], torch.zeros(16)[::2])


def test_layer_norm_requires_a_gpu_tensor() -> None:
    with pytest.raises(ValueError, match="requires CUDA"):
        layer_norm(torch.zeros(2, 8), torch.ones(8), torch.zeros(8))


@pytest.mark.parametrize("eps", [0.0, -1e-5, float("nan"), float("inf")])
def test_layer_norm_rejects_invalid_epsilon(eps: float) -> None:
    with pytest.raises(ValueError, match="finite and positive"):
        layer_norm(torch.zeros(2, 8), torch.ones(8), torch.zeros(8), eps=eps)


def test_matmul_rejects_incompatible_inner_dimensions() -> None:
    with pytest.raises(ValueError, match="incompatible shapes"):
        matmul_fp32acc(torch.zeros(2, 3, dtype=torch.float16), torch.zeros(4, 2, dtype=torch.float16))


def test_matmul_requires_a_gpu_tensor() -> None:
    with pytest.raises(ValueError, match="requires CUDA"):
        matmul_fp32acc(torch.zeros(2, 3, dtype=torch.float16), torch.zeros(3, 2, dtype=torch.float16))


def test_matmul_rejects_zero_strides() -> None:
    left = torch.empty_strided((2, 3), (0, 1), dtype=torch.float16, device="meta")
    right = torch.empty((3, 2), dtype=torch.float16, device="meta")
    with pytest.raises(ValueError, match="strictly positive strides"):
        matmul_fp32acc(left, right)


def test_matmul_rejects_offsets_outside_int32_range() -> None:
    left = torch.empty_strided((2, 2), (2**31, 1), dtype=torch.float16, device="meta")
    right = torch.empty((2, 2), dtype=torch.float16, device="meta")
    with pytest.raises(ValueError, match="int32 offset"):
        matmul_fp32acc(left, right)


def test_matmul_rejects_float32() -> None:
    with pytest.raises(ValueError, match="float16 and bfloat16"):
        matmul_fp32acc(torch.zeros(2, 3), torch.zeros(3, 2))


def test_attention_rejects_shape_mismatch() -> None:
    q = torch.zeros(1, 2, 8, 64, dtype=torch.float16)
    k = torch.zeros(1, 2, 7, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="identical shapes"):
        attention_noncausal(q, k, torch.zeros_like(q))


@pytest.mark.parametrize(
    ("shape", "dtype", "fragment"),
    [
        ((1, 2, 8, 64), torch.float32, "requires CUDA"),  # device is checked before dtype
        ((2, 8, 64), torch.float16, "batch, heads, sequence, dim"),
        ((1, 2, 0, 64), torch.float16, "empty dimensions"),
    ],
)
def test_attention_contract(shape, dtype, fragment) -> None:
    q = torch.zeros(shape, dtype=dtype, device="meta")
    with pytest.raises(ValueError, match=fragment):
        attention_noncausal(q, q, q)


def test_gqa_decode_contract() -> None:
    from tklab.kernels.gqa_decode import gqa_decode, split_length

    q = torch.empty(2, 8, 128, device="meta", dtype=torch.bfloat16)
    k = torch.empty(2, 2, 100, 128, device="meta", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="expects q"):
        gqa_decode(q[0], k, k)
    with pytest.raises(ValueError, match="identical shapes"):
        gqa_decode(q, k, k[:, :, :50])
    with pytest.raises(ValueError, match="1, 2, 4 or 8 times"):
        gqa_decode(torch.empty(2, 6, 128, device="meta", dtype=torch.bfloat16), k, k)
    with pytest.raises(ValueError, match="head_dim 64 and 128"):
        q96 = torch.empty(2, 8, 96, device="meta", dtype=torch.bfloat16)
        k96 = torch.empty(2, 2, 100, 96, device="meta", dtype=torch.bfloat16)
        gqa_decode(q96, k96, k96)
    with pytest.raises(ValueError, match="float16 or bfloat16"):
        gqa_decode(q.float(), k.float(), k.float())
    with pytest.raises(ValueError, match="requires CUDA"):
        gqa_decode(q, k, k)
    # Splits: multiples of 64 keys, about 512 waves (two per CU), never longer than the cache.
    assert split_length(8, 8, 8192) == 1024
    assert split_length(32, 8, 8192) == 4096
    assert split_length(64, 8, 8192) == 8192
    assert split_length(1, 1, 100) == 64
    assert all(split_length(b, 8, n) % 64 == 0 for b in (1, 7, 64) for n in (1, 999, 70000))
