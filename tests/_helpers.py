"""Helpers shared by the GPU parity tests (not a test module)."""

from __future__ import annotations

import numpy as np
import torch

DTYPE_NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


def host(t: torch.Tensor) -> np.ndarray:
    """Exact float32 numpy copy of a (device) tensor."""
    return t.detach().float().cpu().numpy()


def dev(a: np.ndarray, like: torch.Tensor) -> torch.Tensor:
    """Device float32 tensor from an oracle result, for comparisons."""
    return torch.from_numpy(np.ascontiguousarray(a)).to(like.device)


def name(dtype: torch.dtype) -> str:
    return DTYPE_NAMES[dtype]


def bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bitwise equality of two same-dtype tensors (NaNs compare by pattern)."""
    if a.dtype != b.dtype or a.shape != b.shape:
        return False
    view = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}
    return bool(torch.equal(a.contiguous().view(view[a.dtype]), b.contiguous().view(view[b.dtype])))


def strided_rows(rows: int, cols: int, step: int, *, dtype=torch.float32, requires_grad=False):
    """Every ``step``-th row of a ``(rows*step, cols)`` standard-normal draw."""
    storage = torch.randn(rows * step, cols, device="cuda", dtype=dtype)
    view = storage[::step]
    if requires_grad:
        view = view.detach().requires_grad_(True)
    return view
