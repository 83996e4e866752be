"""Grouped-query attention decode on the HIP ``tk_gqa_decode`` kernels.

One query token per sequence: ``q`` is ``[batch, q_heads, head_dim]`` and the KV
cache ``k_cache``/``v_cache`` is ``[batch, kv_heads, max_len, head_dim]``; query
head ``h`` reads KV head ``h // (q_heads // kv_heads)``, the mapping of the
reference's decode model (``docs/research/gqa_decode_model.md``, "Semantic GQA
mapping"). ``cache_seqlens`` (int32 ``[batch]``) gives each sequence's context
length for variable-length batches. The arithmetic is the reference attention
forward's for one query row (``flash_attention.py:90-117, 248-264``): scores
scaled by ``scale * log2(e)``, P rounded to the storage dtype before the PV
product, base-2 LSE.

The cache may be any strided view with a unit-stride head dimension (e.g. a
``[batch, max_len, kv_heads, head_dim]`` cache permuted to head-major). Decode is
inference only: there is no autograd.
"""

from __future__ import annotations

import math

import torch

from tklab import _hip

_DTYPES = (torch.float16, torch.bfloat16)
_HEAD_DIMS = (64, 128)
_GROUPS = (1, 2, 4, 8)
# Waves the split kernel aims for: two per CU of the 256 CUs (each holds a 64 KiB
# LDS ring of K/V tiles), so splits are as long as possible.
_TARGET_SPLITS = 512


def gqa_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    cache_seqlens: torch.Tensor | None = None,
    *,
    scale: float | None = None,
    return_lse: bool = False,
) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """Attention of one query token per sequence over a grouped KV cache.

    Args:
        q: ``[batch, q_heads, head_dim]`` float16/bfloat16.
        k_cache, v_cache: ``[batch, kv_heads, max_len, head_dim]``, same dtype;
            ``q_heads / kv_heads`` in {1, 2, 4, 8}; head_dim 64 or 128.
        cache_seqlens: optional int32 ``[batch]`` context lengths; values are
            clamped to ``[0, max_len]`` (a length of 0 gives a zero output and an
            LSE of ``-inf``). ``None`` means every sequence has ``max_len`` keys.
        scale: score scale, default ``1 / sqrt(head_dim)``.
        return_lse: also return the float32 base-2 LSE ``[batch, q_heads]``.

    Raises:
        ValueError: on an unsupported shape, dtype, layout or device.
    """
    _validate(q, k_cache, v_cache, cache_seqlens)
    batch, q_heads, head_dim = q.shape
    out = torch.empty((batch, q_heads, head_dim), device=q.device, dtype=q.dtype)
    lse = torch.empty((batch, q_heads), device=q.device, dtype=torch.float32)
    _launch(q, k_cache, v_cache, cache_seqlens, out, lse,
            scale=head_dim ** -0.5 if scale is None else scale)
    return (out, lse) if return_lse else out


def split_length(batch: int, kv_heads: int, max_len: int) -> int:
    """Keys per split-kernel wave: a multiple of 64 giving about _TARGET_SPLITS waves (one
    split per (batch, KV head) once there are that many pairs: the split wave then writes O
    and the LSE itself and no combine pass runs)."""
    per = math.ceil(batch * kv_heads * max_len / _TARGET_SPLITS)
    return min(max(64, -(-per // 64) * 64), max(64, -(-max_len // 64) * 64))


def _launch(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    cache_seqlens: torch.Tensor | None,
    out: torch.Tensor,
    lse: torch.Tensor | None,
    *,
    scale: float,
) -> None:
    """Run the decode into preallocated ``out`` (and ``lse`` when given)."""
    _validate(q, k_cache, v_cache, cache_seqlens)
    batch, q_heads, head_dim = q.shape
    kv_heads, max_len = k_cache.shape[1], k_cache.shape[2]
    if out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
        raise ValueError("output metadata must match q")
    if out.stride(-1) != 1 or out.data_ptr() % 16 or any(s % 8 for s in out.stride()[:2]):
        raise ValueError("output needs a unit-stride head dimension and 16-byte aligned rows")
    if lse is not None and (lse.shape != (batch, q_heads) or lse.dtype != torch.float32
                            or not lse.is_contiguous()):
        raise ValueError("lse must be a contiguous float32 [batch, q_heads] tensor")
    split = split_length(batch, kv_heads, max_len)
    splits = -(-max_len // split)
    partials = torch.empty((batch, q_heads, splits, head_dim + 4), device=q.device,
                           dtype=torch.float32)
    _hip.call(
        "tk_gqa_decode",
        _hip.dtype_code(q.dtype),
        q.data_ptr(),
        k_cache.data_ptr(),
        v_cache.data_ptr(),
        out.data_ptr(),
        _hip.ptr(lse),
        partials.data_ptr(),
        _hip.ptr(cache_seqlens),
        batch,
        q_heads,
        kv_heads,
        max_len,
        head_dim,
        split,
        _hip.int64_array(list(q.stride()[:2])),
        _hip.int64_array(list(k_cache.stride()[:3])),
        _hip.int64_array(list(v_cache.stride()[:3])),
        _hip.int64_array(list(out.stride()[:2])),
        float(scale),
        _hip.stream_of(q),
    )


def _validate(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    cache_seqlens: torch.Tensor | None,
) -> None:
    """Check the decode contract."""
    if q.ndim != 3 or k_cache.ndim != 4:
        raise ValueError("gqa_decode expects q [batch, q_heads, head_dim] and caches "
                         "[batch, kv_heads, max_len, head_dim]")
    if v_cache.shape != k_cache.shape:
        raise ValueError("k_cache and v_cache must have identical shapes")
    batch, q_heads, head_dim = q.shape
    if k_cache.shape[0] != batch or k_cache.shape[3] != head_dim:
        raise ValueError("q and the caches disagree on batch or head_dim")
    kv_heads, max_len = k_cache.shape[1], k_cache.shape[2]
    if min(batch, q_heads, kv_heads, max_len) == 0:
        raise ValueError("gqa_decode does not support empty dimensions")
    if q_heads % kv_heads or q_heads // kv_heads not in _GROUPS:
        raise ValueError("q_heads must be 1, 2, 4 or 8 times kv_heads")
    if head_dim not in _HEAD_DIMS:
        raise ValueError("gqa_decode supports head_dim 64 and 128")
    if q.dtype not in _DTYPES or k_cache.dtype != q.dtype or v_cache.dtype != q.dtype:
        raise ValueError("q, k_cache and v_cache must share a float16 or bfloat16 dtype")
    if q.device.type != "cuda" or k_cache.device != q.device or v_cache.device != q.device:
        raise ValueError("gqa_decode requires CUDA (ROCm/HIP) tensors on one device")
    for name, t, dims in (("q", q, 2), ("k_cache", k_cache, 3), ("v_cache", v_cache, 3)):
        if t.stride(-1) != 1:
            raise ValueError(f"{name} requires a contiguous final dimension")
        if t.data_ptr() % 16 or any(s % 8 or s < 0 for s in t.stride()[:dims]):
            raise ValueError(f"{name} rows must be 16-byte aligned (strides multiples of 8)")
    if cache_seqlens is not None:
        if (cache_seqlens.shape != (batch,) or cache_seqlens.dtype != torch.int32
                or cache_seqlens.device != q.device or not cache_seqlens.is_contiguous()):
            raise ValueError("cache_seqlens must be a contiguous int32 [batch] tensor on q's device")
