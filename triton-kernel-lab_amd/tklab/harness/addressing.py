"""Signed 32-bit element-offset guard.

The HIP kernels compute per-row element offsets in 32-bit registers (row base
pointers are 64-bit), so every launcher rejects a tensor whose largest element
displacement exceeds ``2**31 - 1``. The bound and the message fragment
"int32 offset" are the reference's (``src/tklab/harness/addressing.py:14-48``).
"""

from __future__ import annotations

import torch

MAX_INT32_OFFSET = 2**31 - 1


def max_relative_offset(tensor: torch.Tensor) -> int:
    """Largest element displacement reachable inside ``tensor``.

    ``sum((size - 1) * |stride|)`` over all dimensions; 0 for an empty tensor.
    """
    if tensor.numel() == 0:
        return 0
    total = 0
    for size, stride in zip(tensor.shape, tensor.stride(), strict=True):
        total += (size - 1) * abs(stride)
    return total


def assert_int32_addressable(tensor: torch.Tensor, *, name: str) -> None:
    """Raise ``ValueError`` when ``tensor`` cannot be indexed with int32 offsets."""
    if max_relative_offset(tensor) > MAX_INT32_OFFSET:
        raise ValueError(f"{name} strides exceed the signed int32 offset range")
