"""Flash attention forward and recompute backward on the HIP MFMA kernels.

Contract of ``src/tklab/kernels/flash_attention.py``: ``attention_causal`` and
``attention_noncausal`` on contiguous ``(batch, heads, sequence, head_dim)``
Q/K/V of one shape and dtype, scale ``1/sqrt(head_dim)``, base-2 online
softmax, a float32 base-2 log-sum-exp saved for the backward, and a
three-launch backward (delta preprocess, dK/dV, dQ). Validation order and
messages follow ``flash_attention.py:267-288``. Beyond the reference: bfloat16
as well as float16, head_dim 128 as well as 64, and any sequence length
without a per-length recompile.

The registry keeps the reference's spec shape (batch 1, 16 heads, head_dim
64, ``flash_attention.py:27-29``) so its FLOP model and tests carry over.

``grouped_query_attention(q, k, v, *, causal)`` extends the same kernels to K/V
with fewer heads than Q (query head ``h`` uses KV head ``h // (heads //
kv_heads)``), forward and backward; dK/dV sum a KV head's query heads in a fixed
order, so the backward stays deterministic. ``varlen_attention(q, k, v,
cu_seqlens, max_seqlen, *, causal)`` runs them on variable-length batches packed
as ``(total, heads, head_dim)`` with int32 sequence offsets ``cu_seqlens``.
``rope_attention(q, k, v, cos, sin, *, causal)`` applies rotate-half RoPE from
position-indexed tables to Q (in the forward kernel's prologue) and K first.
"""

from __future__ import annotations

import math
from typing import Any, cast

import torch
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from tklab import _hip
from tklab.harness.addressing import assert_int32_addressable
from tklab.harness.tolerances import assert_relative_frobenius
from tklab.registry import (
    BenchmarkMetadataFn,
    BenchmarkScalar,
    CostFn,
    KernelSpec,
    LaunchFn,
    TensorArgs,
    TensorFn,
    register,
)

_BATCH = 1
_HEADS = 16
_HEAD_DIM = 64
_HEAD_DIMS = (64, 128)
_DTYPES = (torch.float16, torch.bfloat16)
_LOG2_E = 1.4426950408889634

# Tile configuration of csrc/attention.hip (forward / backward).
# csrc/attention_fwd.hip (Geo<D>: BM, BN, WAVES, STAGES): 256 queries per workgroup as eight
# wave64s of 32, key blocks of 64, a 4-stage buffer->LDS K/V ring, v_mfma_f32_16x16x32.
# "num_warps" counts wave64s.
FORWARD_TILE = {"hip_kernel": "attn_fwd_dma_kernel", "block_m": 256, "block_n": 64, "num_warps": 8,
                "num_stages": 4}
FORWARD_MFMA = {torch.float16: "v_mfma_f32_16x16x32_f16", torch.bfloat16: "v_mfma_f32_16x16x32_bf16"}
# Backward (csrc/attention_bwd.hip, attention_bwd_dq.hip): dK/dV owns 128 keys per workgroup
# over query blocks of 64; dQ owns 256 queries over key blocks of 64.
BACKWARD_TILE = {"block_m": 128, "block_n": 64}


def _validate(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """Dense self-attention contract (reference ``flash_attention.py:267-288``)."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("attention expects Q, K, and V shaped (batch, heads, sequence, dim)")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("Q, K, and V must have identical shapes")
    if 0 in q.shape:
        raise ValueError("attention does not support empty dimensions")
    if q.device != k.device or q.device != v.device:
        raise ValueError("Q, K, and V must be on the same device")
    if q.device.type != "cuda":
        raise ValueError("attention requires CUDA (ROCm/HIP) tensors")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("Q, K, and V must have the same dtype")
    if q.dtype not in _DTYPES:
        raise ValueError("attention supports float16 and bfloat16 inputs only")
    if q.shape[-1] not in _HEAD_DIMS:
        raise ValueError(f"attention requires head_dim in {_HEAD_DIMS}")
    for name, tensor in (("Q", q), ("K", k), ("V", v)):
        if not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        assert_int32_addressable(tensor, name=name)


def _make_output(args: TensorArgs) -> torch.Tensor:
    """Dense attention output."""
    return torch.empty_like(args[0])


def _strides(t: torch.Tensor) -> Any:
    """(batch, head, sequence) element strides as a C ``int64_t[3]``."""
    return _hip.int64_array(list(t.stride()[:3]))


def _launch_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    output: torch.Tensor,
    softmax_lse: torch.Tensor,
    *,
    causal: bool,
    store_lse: bool,
) -> None:
    """Forward into preallocated buffers; ``softmax_lse`` is written only with ``store_lse``."""
    _validate(q, k, v)
    if output.shape != q.shape or output.device != q.device or output.dtype != q.dtype:
        raise ValueError("attention output metadata must match Q")
    if not output.is_contiguous():
        raise ValueError("attention output must be contiguous")
    batch, heads, n_ctx, head_dim = q.shape
    if store_lse:
        if (
            softmax_lse.shape != (batch, heads, n_ctx)
            or softmax_lse.device != q.device
            or softmax_lse.dtype != torch.float32
            or not softmax_lse.is_contiguous()
        ):
            raise ValueError("attention log-sum-exp buffer must be contiguous float32 BxHxN")
        assert_int32_addressable(softmax_lse, name="log-sum-exp buffer")
    _hip.call(
        "tk_attn_fwd",
        _hip.dtype_code(q.dtype),
        q.data_ptr(),
        k.data_ptr(),
        v.data_ptr(),
        output.data_ptr(),
        softmax_lse.data_ptr() if store_lse else None,
        batch,
        heads,
        n_ctx,
        head_dim,
        _strides(q),
        _strides(k),
        _strides(v),
        _strides(output),
        1.0 / math.sqrt(head_dim),
        int(causal),
        _hip.stream_of(q),
    )


def _launch_factory(*, causal: bool) -> LaunchFn:
    """Allocation-free inference launcher for one masking mode."""

    def launch(args: TensorArgs, output: torch.Tensor) -> None:
        q, k, v = args
        _launch_forward(q, k, v, output, output, causal=causal, store_lse=False)

    return launch


_launch_noncausal = _launch_factory(causal=False)
_launch_causal = _launch_factory(causal=True)


def _launch_backward_into(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    output: torch.Tensor,
    softmax_lse: torch.Tensor,
    do: torch.Tensor,
    delta: torch.Tensor,
    dq: torch.Tensor,
    dk: torch.Tensor,
    dv: torch.Tensor,
    *,
    causal: bool,
) -> None:
    """The three backward launches into caller-provided buffers (all BxHxNxD contiguous)."""
    batch, heads, n_ctx, head_dim = q.shape
    code = _hip.dtype_code(q.dtype)
    strides = _strides(q)
    stream = _hip.stream_of(q)
    scale = 1.0 / math.sqrt(head_dim)
    _hip.call(
        "tk_attn_bwd_preprocess", code, output.data_ptr(), do.data_ptr(), delta.data_ptr(),
        batch, heads, n_ctx, head_dim, strides, stream,
    )
    _hip.call(
        "tk_attn_bwd_dkdv", code, q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(),
        dk.data_ptr(), dv.data_ptr(), softmax_lse.data_ptr(), delta.data_ptr(),
        batch, heads, n_ctx, head_dim, strides, scale, int(causal), stream,
    )
    _hip.call(
        "tk_attn_bwd_dq", code, q.data_ptr(), k.data_ptr(), v.data_ptr(), do.data_ptr(),
        dq.data_ptr(), softmax_lse.data_ptr(), delta.data_ptr(),
        batch, heads, n_ctx, head_dim, strides, scale, int(causal), stream,
    )


def _launch_backward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    output: torch.Tensor,
    softmax_lse: torch.Tensor,
    do: torch.Tensor,
    *,
    causal: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Recompute backward; returns dQ, dK, dV (reference ``flash_attention.py:536-607``)."""
    if do.shape != q.shape or do.device != q.device or do.dtype != q.dtype:
        raise ValueError("attention upstream gradient metadata must match Q")
    do = do.contiguous()
    batch, heads, n_ctx, _ = q.shape
    delta = torch.empty((batch, heads, n_ctx), dtype=torch.float32, device=q.device)
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    _launch_backward_into(q, k, v, output, softmax_lse, do, delta, dq, dk, dv, causal=causal)
    return dq, dk, dv


class _FlashAttentionFunction(torch.autograd.Function):
    """Autograd bridge: saves Q, K, V, O and the base-2 LSE."""

    @staticmethod
    def forward(
        ctx: Any, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool
    ) -> torch.Tensor:
        _validate(q, k, v)
        output = torch.empty_like(q)
        batch, heads, n_ctx, _ = q.shape
        softmax_lse = torch.empty((batch, heads, n_ctx), dtype=torch.float32, device=q.device)
        _launch_forward(q, k, v, output, softmax_lse, causal=causal, store_lse=True)
        ctx.save_for_backward(q, k, v, output, softmax_lse)
        ctx.causal = causal
        return output

    @staticmethod
    @once_differentiable
    def backward(
        ctx: Any, do: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, None]:
        q, k, v, output, softmax_lse = ctx.saved_tensors
        dq, dk, dv = _launch_backward(q, k, v, output, softmax_lse, do, causal=ctx.causal)
        return dq, dk, dv, None


def _attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool) -> torch.Tensor:
    """Inference skips the LSE store; training goes through autograd."""
    _validate(q, k, v)
    needs_grad = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)
    if not needs_grad:
        output = torch.empty_like(q)
        _launch_forward(q, k, v, output, output, causal=causal, store_lse=False)
        return output
    return cast(torch.Tensor, _FlashAttentionFunction.apply(q, k, v, causal))


def attention_noncausal(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Dense non-causal scaled dot-product attention with autograd."""
    return _attention(q, k, v, causal=False)


def attention_causal(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Dense causal scaled dot-product attention with autograd."""
    return _attention(q, k, v, causal=True)


def _validate_gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """Grouped-query contract: the dense one with K/V heads dividing Q heads."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("attention expects Q, K, and V shaped (batch, heads, sequence, dim)")
    if k.shape != v.shape:
        raise ValueError("K and V must have identical shapes")
    if q.shape[0] != k.shape[0] or q.shape[2:] != k.shape[2:]:
        raise ValueError("Q and K/V must agree on batch, sequence and head_dim")
    if 0 in q.shape or 0 in k.shape:
        raise ValueError("attention does not support empty dimensions")
    if q.shape[1] % k.shape[1]:
        raise ValueError("the number of Q heads must be a multiple of the K/V heads")
    if q.device != k.device or q.device != v.device:
        raise ValueError("Q, K, and V must be on the same device")
    if q.device.type != "cuda":
        raise ValueError("attention requires CUDA (ROCm/HIP) tensors")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("Q, K, and V must have the same dtype")
    if q.dtype not in _DTYPES:
        raise ValueError("attention supports float16 and bfloat16 inputs only")
    if q.shape[-1] not in _HEAD_DIMS:
        raise ValueError(f"attention requires head_dim in {_HEAD_DIMS}")
    for name, tensor in (("Q", q), ("K", k), ("V", v)):
        if not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        assert_int32_addressable(tensor, name=name)


def _launch_gqa_forward(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, output: torch.Tensor,
    softmax_lse: torch.Tensor | None, *, causal: bool,
) -> None:
    """Grouped-query forward into preallocated buffers (``softmax_lse`` may be None)."""
    batch, heads, n_ctx, head_dim = q.shape
    _hip.call(
        "tk_attn_fwd_gqa", _hip.dtype_code(q.dtype), q.data_ptr(), k.data_ptr(), v.data_ptr(),
        output.data_ptr(), _hip.ptr(softmax_lse), batch, heads, k.shape[1], n_ctx, head_dim,
        _strides(q), _strides(k), _strides(v), _strides(output), 1.0 / math.sqrt(head_dim),
        int(causal), _hip.stream_of(q),
    )


def _launch_gqa_backward(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, output: torch.Tensor,
    softmax_lse: torch.Tensor, do: torch.Tensor, *, causal: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Grouped-query backward: delta, dK/dV per KV head, dQ per query head."""
    if do.shape != q.shape or do.device != q.device or do.dtype != q.dtype:
        raise ValueError("attention upstream gradient metadata must match Q")
    do = do.contiguous()
    batch, heads, n_ctx, head_dim = q.shape
    kv_heads = k.shape[1]
    code = _hip.dtype_code(q.dtype)
    stream = _hip.stream_of(q)
    scale = 1.0 / math.sqrt(head_dim)
    delta = torch.empty((batch, heads, n_ctx), dtype=torch.float32, device=q.device)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    qs, kvs = _strides(q), _strides(k)
    _hip.call("tk_attn_bwd_preprocess", code, output.data_ptr(), do.data_ptr(), delta.data_ptr(),
              batch, heads, n_ctx, head_dim, qs, stream)
    _hip.call("tk_attn_bwd_dkdv_gqa", code, q.data_ptr(), k.data_ptr(), v.data_ptr(),
              do.data_ptr(), dk.data_ptr(), dv.data_ptr(), softmax_lse.data_ptr(),
              delta.data_ptr(), batch, heads, kv_heads, n_ctx, head_dim, qs, kvs, scale,
              int(causal), stream)
    _hip.call("tk_attn_bwd_dq_gqa", code, q.data_ptr(), k.data_ptr(), v.data_ptr(),
              do.data_ptr(), dq.data_ptr(), softmax_lse.data_ptr(), delta.data_ptr(), batch,
              heads, kv_heads, n_ctx, head_dim, qs, kvs, scale, int(causal), stream)
    return dq, dk, dv


class _GQAFunction(torch.autograd.Function):
    """Autograd bridge of grouped-query attention: saves Q, K, V, O and the LSE."""

    @staticmethod
    def forward(
        ctx: Any, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool
    ) -> torch.Tensor:
        output = torch.empty_like(q)
        batch, heads, n_ctx, _ = q.shape
        softmax_lse = torch.empty((batch, heads, n_ctx), dtype=torch.float32, device=q.device)
        _launch_gqa_forward(q, k, v, output, softmax_lse, causal=causal)
        ctx.save_for_backward(q, k, v, output, softmax_lse)
        ctx.causal = causal
        return output

    @staticmethod
    @once_differentiable
    def backward(
        ctx: Any, do: torch.Tensor
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, None]:
        q, k, v, output, softmax_lse = ctx.saved_tensors
        dq, dk, dv = _launch_gqa_backward(q, k, v, output, softmax_lse, do, causal=ctx.causal)
        return dq, dk, dv, None


def grouped_query_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool
) -> torch.Tensor:
    """Scaled dot-product attention with K/V shared by groups of query heads.

    ``q`` is ``(batch, heads, sequence, head_dim)``, ``k`` and ``v`` are
    ``(batch, kv_heads, sequence, head_dim)`` with ``heads % kv_heads == 0``;
    query head ``h`` attends with KV head ``h // (heads // kv_heads)``. Same
    numerics as :func:`attention_causal` / :func:`attention_noncausal`, with
    autograd (first order).
    """
    _validate_gqa(q, k, v)
    needs_grad = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)
    if not needs_grad:
        output = torch.empty_like(q)
        _launch_gqa_forward(q, k, v, output, None, causal=causal)
        return output
    return cast(torch.Tensor, _GQAFunction.apply(q, k, v, causal))


def _validate_rope_tables(q: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> None:
    """Position-indexed rotate-half tables: (positions >= sequence, head_dim // 2)."""
    for table in (cos, sin):
        if table.ndim != 2 or table.shape[1] != q.shape[-1] // 2:
            raise ValueError("rope tables must be shaped (positions, head_dim // 2)")
        if table.shape[0] < q.shape[2]:
            raise ValueError("rope tables need a row per sequence position")
        if table.dtype != q.dtype or table.device != q.device:
            raise ValueError("rope tables must match Q's dtype and device")
        if table.stride(1) != 1:
            raise ValueError("rope tables require a contiguous final dimension")
    if cos.stride(0) != sin.stride(0):
        raise ValueError("rope tables must share one row stride")


def _rope_positions(
    x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, out: torch.Tensor, *, inverse: bool
) -> None:
    """RoPE (or its input gradient) of contiguous (batch, heads, sequence, dim) rows."""
    batch, heads, n_ctx, head_dim = x.shape
    _hip.call(
        "tk_rope_positions", _hip.dtype_code(x.dtype), x.data_ptr(), cos.data_ptr(),
        sin.data_ptr(), out.data_ptr(), batch * heads * n_ctx, n_ctx, head_dim // 2, head_dim,
        cos.stride(0), head_dim, int(inverse), _hip.stream_of(x),
    )


def _launch_rope_forward(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
    output: torch.Tensor, softmax_lse: torch.Tensor | None, k_rot: torch.Tensor, *, causal: bool,
) -> None:
    """RoPE'd grouped-query forward: Q rotated in the kernel prologue, K into ``k_rot``."""
    batch, heads, n_ctx, head_dim = q.shape
    _hip.call(
        "tk_attn_fwd_rope", _hip.dtype_code(q.dtype), q.data_ptr(), k.data_ptr(), v.data_ptr(),
        output.data_ptr(), _hip.ptr(softmax_lse), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
        cos.stride(0), k_rot.data_ptr(), batch, heads, k.shape[1], n_ctx, head_dim,
        _strides(q), _strides(k), _strides(v), _strides(output), 1.0 / math.sqrt(head_dim),
        int(causal), _hip.stream_of(q),
    )


class _RopeAttentionFunction(torch.autograd.Function):
    """Autograd bridge: saves Q, the rotated K, V, the tables, O and the LSE."""

    @staticmethod
    def forward(
        ctx: Any, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
        sin: torch.Tensor, causal: bool,
    ) -> torch.Tensor:
        output, k_rot = torch.empty_like(q), torch.empty_like(k)
        batch, heads, n_ctx, _ = q.shape
        softmax_lse = torch.empty((batch, heads, n_ctx), dtype=torch.float32, device=q.device)
        _launch_rope_forward(q, k, v, cos, sin, output, softmax_lse, k_rot, causal=causal)
        ctx.save_for_backward(q, k_rot, v, cos, sin, output, softmax_lse)
        ctx.causal = causal
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, do: torch.Tensor) -> tuple[Any, ...]:
        q, k_rot, v, cos, sin, output, softmax_lse = ctx.saved_tensors
        q_rot = torch.empty_like(q)
        _rope_positions(q, cos, sin, q_rot, inverse=False)
        dq_rot, dk_rot, dv = _launch_gqa_backward(
            q_rot, k_rot, v, output, softmax_lse, do, causal=ctx.causal
        )
        dq, dk = torch.empty_like(dq_rot), torch.empty_like(dk_rot)
        _rope_positions(dq_rot, cos, sin, dq, inverse=True)
        _rope_positions(dk_rot, cos, sin, dk, inverse=True)
        return dq, dk, dv, None, None, None


def rope_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
    *, causal: bool,
) -> torch.Tensor:
    """Grouped-query attention on rotate-half RoPE'd Q and K.

    ``attention(rope(q), rope(k), v)`` with position-indexed tables ``cos``/``sin``
    of shape ``(positions >= sequence, head_dim // 2)`` (query and key ``i`` use row
    ``i``; the reference's ``rope`` takes per-row tables, ``rope.py:26-73``). Q is
    rotated in the attention kernel's prologue and never stored rotated; K is rotated
    once into a workspace (every query block re-reads it). Bitwise the composition of
    the RoPE and attention kernels; the tables are constants (no gradient).
    """
    _validate_gqa(q, k, v)
    _validate_rope_tables(q, cos, sin)
    needs_grad = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)
    if not needs_grad:
        output, k_rot = torch.empty_like(q), torch.empty_like(k)
        _launch_rope_forward(q, k, v, cos, sin, output, None, k_rot, causal=causal)
        return output
    return cast(torch.Tensor, _RopeAttentionFunction.apply(q, k, v, cos, sin, causal))


def _validate_varlen(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor, max_seqlen: int
) -> None:
    """Packed variable-length contract: (total, heads, head_dim) tensors and offsets."""
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("varlen attention expects Q, K, and V shaped (total, heads, dim)")
    if k.shape != v.shape:
        raise ValueError("K and V must have identical shapes")
    if q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError("Q and K/V must agree on total tokens and head_dim")
    if 0 in q.shape or 0 in k.shape:
        raise ValueError("attention does not support empty dimensions")
    if q.shape[1] % k.shape[1]:
        raise ValueError("the number of Q heads must be a multiple of the K/V heads")
    if q.device != k.device or q.device != v.device or cu_seqlens.device != q.device:
        raise ValueError("Q, K, V and cu_seqlens must be on the same device")
    if q.device.type != "cuda":
        raise ValueError("attention requires CUDA (ROCm/HIP) tensors")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("Q, K, and V must have the same dtype")
    if q.dtype not in _DTYPES:
        raise ValueError("attention supports float16 and bfloat16 inputs only")
    if q.shape[-1] not in _HEAD_DIMS:
        raise ValueError(f"attention requires head_dim in {_HEAD_DIMS}")
    if cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2 or cu_seqlens.dtype != torch.int32:
        raise ValueError("cu_seqlens must be an int32 vector of batch + 1 offsets")
    if not cu_seqlens.is_contiguous():
        raise ValueError("cu_seqlens must be contiguous")
    if not 1 <= max_seqlen <= q.shape[0]:
        raise ValueError("max_seqlen must be in [1, total]")
    for name, tensor in (("Q", q), ("K", k), ("V", v)):
        if not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        assert_int32_addressable(tensor, name=name)


def _check_offsets(cu_seqlens: torch.Tensor, total: int, max_seqlen: int) -> bool:
    """Validate the offsets table on the host (one small device-to-host copy).

    Offsets must start at 0 or later, never decrease, end at ``total`` or earlier, and no
    sequence may be longer than ``max_seqlen``. Returns True when some token rows lie
    outside every sequence (a padded packing), whose outputs and gradients are then zero.
    """
    offsets = cu_seqlens.tolist()
    if offsets[0] < 0 or offsets[-1] > total:
        raise ValueError("cu_seqlens must lie in [0, total]")
    lengths = [b - a for a, b in zip(offsets, offsets[1:])]
    if min(lengths) < 0:
        raise ValueError("cu_seqlens must be non-decreasing")
    if max(lengths) > max_seqlen:
        raise ValueError("max_seqlen must be at least the longest sequence")
    return offsets[0] > 0 or offsets[-1] < total


def _launch_varlen_forward(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
    max_seqlen: int, output: torch.Tensor, softmax_lse: torch.Tensor | None, *, causal: bool,
) -> None:
    """Varlen forward into preallocated buffers (``softmax_lse`` [heads, total] or None)."""
    total, heads, head_dim = q.shape
    _hip.call(
        "tk_attn_fwd_varlen", _hip.dtype_code(q.dtype), q.data_ptr(), k.data_ptr(),
        v.data_ptr(), output.data_ptr(), _hip.ptr(softmax_lse), cu_seqlens.data_ptr(),
        cu_seqlens.numel() - 1, heads, k.shape[1], max_seqlen, total, head_dim,
        _hip.int64_array(list(q.stride()[:2])), _hip.int64_array(list(k.stride()[:2])),
        _hip.int64_array(list(output.stride()[:2])), 1.0 / math.sqrt(head_dim), int(causal),
        _hip.stream_of(q),
    )


def _launch_varlen_backward(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
    max_seqlen: int, output: torch.Tensor, softmax_lse: torch.Tensor, do: torch.Tensor,
    *, causal: bool, zero_fill: bool = False,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Varlen backward: delta [heads, total], dK/dV per KV head, dQ per query head.

    With ``zero_fill`` the gradients start at zero, so token rows outside every sequence
    (which no kernel writes) read as zero."""
    if do.shape != q.shape or do.device != q.device or do.dtype != q.dtype:
        raise ValueError("attention upstream gradient metadata must match Q")
    do = do.contiguous()
    total, heads, head_dim = q.shape
    batch = cu_seqlens.numel() - 1
    code = _hip.dtype_code(q.dtype)
    stream = _hip.stream_of(q)
    scale = 1.0 / math.sqrt(head_dim)
    delta = torch.empty((heads, total), dtype=torch.float32, device=q.device)
    alloc = torch.zeros_like if zero_fill else torch.empty_like
    dq, dk, dv = alloc(q), alloc(k), alloc(v)
    # delta as one sequence of `total` rows: index head * total + token.
    token, head = q.stride(0), q.stride(1)
    _hip.call("tk_attn_bwd_preprocess", code, output.data_ptr(), do.data_ptr(), delta.data_ptr(),
              1, heads, total, head_dim, _hip.int64_array([total * token, head, token]), stream)
    qs = _hip.int64_array([token, head])
    kvs = _hip.int64_array(list(k.stride()[:2]))
    _hip.call("tk_attn_bwd_dkdv_varlen", code, q.data_ptr(), k.data_ptr(), v.data_ptr(),
              do.data_ptr(), dk.data_ptr(), dv.data_ptr(), softmax_lse.data_ptr(),
              delta.data_ptr(), cu_seqlens.data_ptr(), batch, heads, k.shape[1], max_seqlen,
              total, head_dim, qs, kvs, scale, int(causal), stream)
    _hip.call("tk_attn_bwd_dq_varlen", code, q.data_ptr(), k.data_ptr(), v.data_ptr(),
              do.data_ptr(), dq.data_ptr(), softmax_lse.data_ptr(), delta.data_ptr(),
              cu_seqlens.data_ptr(), batch, heads, k.shape[1], max_seqlen, total, head_dim, qs,
              kvs, scale, int(causal), stream)
    return dq, dk, dv


class _VarlenFunction(torch.autograd.Function):
    """Autograd bridge of varlen attention: saves Q, K, V, O, the offsets and the LSE."""

    @staticmethod
    def forward(
        ctx: Any, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
        max_seqlen: int, causal: bool, zero_fill: bool,
    ) -> torch.Tensor:
        output = (torch.zeros_like if zero_fill else torch.empty_like)(q)
        softmax_lse = torch.empty((q.shape[1], q.shape[0]), dtype=torch.float32,
                                  device=q.device)
        _launch_varlen_forward(q, k, v, cu_seqlens, max_seqlen, output, softmax_lse,
                               causal=causal)
        ctx.save_for_backward(q, k, v, cu_seqlens, output, softmax_lse)
        ctx.max_seqlen = max_seqlen
        ctx.causal = causal
        ctx.zero_fill = zero_fill
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx: Any, do: torch.Tensor) -> tuple[Any, ...]:
        q, k, v, cu_seqlens, output, softmax_lse = ctx.saved_tensors
        dq, dk, dv = _launch_varlen_backward(q, k, v, cu_seqlens, ctx.max_seqlen, output,
                                             softmax_lse, do, causal=ctx.causal,
                                             zero_fill=ctx.zero_fill)
        return dq, dk, dv, None, None, None, None


def varlen_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
    max_seqlen: int, *, causal: bool, check_offsets: bool = True,
) -> torch.Tensor:
    """Attention over a variable-length batch packed along the token axis.

    ``q`` is ``(total, heads, head_dim)``, ``k`` and ``v`` ``(total, kv_heads,
    head_dim)`` (``heads % kv_heads == 0``); sequence ``b`` is tokens
    ``cu_seqlens[b]`` .. ``cu_seqlens[b + 1]`` (int32, on the device) and attends
    only to itself; ``max_seqlen`` is at least the longest sequence. Each sequence
    gets exactly the result :func:`grouped_query_attention` gives it alone, with
    autograd (first order). Token rows outside every sequence (``cu_seqlens[0] > 0``
    or ``cu_seqlens[-1] < total``: a padded packing) get zero output and gradients.

    With ``check_offsets`` (default) the offsets are copied to the host and checked
    (start >= 0, non-decreasing, end <= total, no sequence longer than ``max_seqlen``;
    ``ValueError`` otherwise), which synchronizes with the device. ``check_offsets=False``
    skips the copy (no synchronization, e.g. under graph capture): outputs and gradients
    are then zero-filled before the launch, and offsets that break the rules above give
    unspecified values in the rows they cover (the kernels clamp every offset and length,
    so no access leaves the tensors).
    """
    _validate_varlen(q, k, v, cu_seqlens, max_seqlen)
    zero_fill = _check_offsets(cu_seqlens, q.shape[0], max_seqlen) if check_offsets else True
    needs_grad = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)
    if not needs_grad:
        output = (torch.zeros_like if zero_fill else torch.empty_like)(q)
        _launch_varlen_forward(q, k, v, cu_seqlens, max_seqlen, output, None, causal=causal)
        return output
    return cast(torch.Tensor,
                _VarlenFunction.apply(q, k, v, cu_seqlens, max_seqlen, causal, zero_fill))


def _reference_factory(*, causal: bool) -> TensorFn:
    """PyTorch SDPA reference."""

    def reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        return F.scaled_dot_product_attention(q, k, v, is_causal=causal)

    return reference


def _make_inputs(sequence_length: int, device: torch.device, dtype: torch.dtype) -> TensorArgs:
    """Contiguous (1, 16, N, 64) self-attention inputs."""
    shape = (_BATCH, _HEADS, sequence_length, _HEAD_DIM)
    return tuple(torch.randn(shape, device=device, dtype=dtype) for _ in range(3))


def _make_adversarial(device: torch.device) -> TensorArgs:
    """Sequence length 1000: partial query and key tiles."""
    return _make_inputs(1000, device, torch.float16)


def _assert_attention(output: torch.Tensor, reference: torch.Tensor) -> None:
    """Relative Frobenius error below 2e-2 (reference ``flash_attention.py:732-734``)."""
    assert_relative_frobenius(output, reference, max_relative_error=2e-2)


def attention_flops(batch: int, heads: int, n_ctx: int, head_dim: int, *, causal: bool) -> int:
    """Two matmuls over the attended (query, key) pairs: ``4 * B * H * pairs * D``."""
    pairs = n_ctx * (n_ctx + 1) // 2 if causal else n_ctx * n_ctx
    return 4 * batch * heads * pairs * head_dim


def _flops_factory(*, causal: bool) -> CostFn:
    """FLOP model of the registered (1, 16, N, 64) problem."""

    def flops(sequence_length: int, _dtype: torch.dtype) -> int:
        return attention_flops(_BATCH, _HEADS, sequence_length, _HEAD_DIM, causal=causal)

    return flops


def _metadata_factory(*, causal: bool) -> BenchmarkMetadataFn:
    """Tile configuration and problem constants in the reference's keys."""

    def metadata(_size: int, dtype: torch.dtype) -> dict[str, BenchmarkScalar]:
        return {**FORWARD_TILE, "heads": _HEADS, "head_dim": _HEAD_DIM, "causal": causal,
                "mma_opcode": FORWARD_MFMA.get(dtype, FORWARD_MFMA[torch.float16])}

    return metadata


_SIZES = (512, 1024, 2048, 4096, 8192)

ATTENTION_NONCAUSAL = register(
    KernelSpec(
        name="attention_noncausal",
        description="Flash Attention forward with online softmax and no mask.",
        triton_fn=attention_noncausal,
        launch_fn=_launch_noncausal,
        ref_fn=_reference_factory(causal=False),
        make_inputs=_make_inputs,
        make_output=_make_output,
        make_adversarial=_make_adversarial,
        sizes=_SIZES,
        correctness_sizes=(128, 512),
        bound="compute",
        flops=_flops_factory(causal=False),
        dtypes=(torch.float16, torch.bfloat16),
        assert_fn=_assert_attention,
        benchmark_metadata=_metadata_factory(causal=False),
        compute_mode="attention_fp16_fp32acc",
        supports_interpreter=False,
    )
)

ATTENTION_CAUSAL = register(
    KernelSpec(
        name="attention_causal",
        description="Flash Attention forward with causal masking and heaviest-first blocks.",
        triton_fn=attention_causal,
        launch_fn=_launch_causal,
        ref_fn=_reference_factory(causal=True),
        make_inputs=_make_inputs,
        make_output=_make_output,
        make_adversarial=_make_adversarial,
        sizes=_SIZES,
        correctness_sizes=(128, 512),
        bound="compute",
        flops=_flops_factory(causal=True),
        dtypes=(torch.float16, torch.bfloat16),
        assert_fn=_assert_attention,
        benchmark_metadata=_metadata_factory(causal=True),
        compute_mode="attention_fp16_fp32acc",
        supports_interpreter=False,
    )
)
