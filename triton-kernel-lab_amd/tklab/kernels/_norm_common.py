"""Launch policy shared by the RMSNorm kernels.

Same role as the reference's ``src/tklab/kernels/_norm_common.py:17-75``: one
place for the epsilon rule, the single-pass row budget, the row launch shape
and the number of dweight partial groups. The shape and group numbers are the
MI355X ones used by ``csrc/rmsnorm.hip``.
"""

from __future__ import annotations

import math
import warnings

import torch

# A normalized row is held in registers by one thread group, so it must fit
# the single-pass budget (reference ``_norm_common.py:17``).
MAX_FEATURE_BYTES = 65_536
EPS = 1e-5

# Tile of the dweight stage-2 reduction (reference ``_norm_common.py:21-22`` names the
# Triton block): a workgroup owns STAGE2_BLOCK_N columns and reads the partial rows in
# STAGE2_BLOCK_M interleaved slices (``kStage2Slices`` x ``kStage2Cols`` in
# csrc/rmsnorm.hip), folding the slices in a fixed order.
STAGE2_BLOCK_M = 32
STAGE2_BLOCK_N = 32

# Groups of the backward dweight reduction: one workgroup per group, one group per
# compute unit (256 CUs). Each streams its rows row % 256 == g with two rows of loads in
# flight, so the 256 groups together walk each tensor through a window of about 256
# neighbouring rows; on the 16384-row bf16 backward of 1024 to 8192 columns this ran
# faster than 384, 512 or 1024 groups, and the float32 partial buffer is 256 x columns.
DEFAULT_GROUPS = 256

# The reference's norm backwards reduce dweight under a spin lock in a scheduling-dependent
# order, so under ``torch.use_deterministic_algorithms(True)`` they raise ``RuntimeError`` (and
# warn with ``RuntimeWarning`` in warn-only mode), reference ``rms_norm.py:370-378`` and
# ``layer_norm.py:367-375``. The reduction here is order-fixed and bitwise reproducible, but the
# drop-in keeps that observable by default so code (and tests) written against the reference
# behave the same. Setting this to False lets deterministic mode run the backward.
REJECT_DETERMINISTIC_MODE = True


def check_deterministic_mode(kernel: str) -> None:
    """Raise or warn like the reference's norm backward under PyTorch's deterministic mode.

    Does nothing when deterministic algorithms are off or ``REJECT_DETERMINISTIC_MODE`` is
    False. The message keeps the reference's "not deterministic" fragment.
    """
    if not REJECT_DETERMINISTIC_MODE or not torch.are_deterministic_algorithms_enabled():
        return
    message = (
        f"{kernel} backward is reported as not deterministic, as the reference's lock "
        "reduction is; this build's fixed-order reduction is bitwise reproducible: set "
        "tklab.kernels._norm_common.REJECT_DETERMINISTIC_MODE = False to run it in "
        "deterministic mode"
    )
    if torch.is_deterministic_algorithms_warn_only_enabled():
        warnings.warn(message, RuntimeWarning, stacklevel=3)
    else:
        raise RuntimeError(message)


def validate_epsilon(eps: float) -> None:
    """Require a finite, strictly positive epsilon (reference ``_norm_common.py:25-38``)."""
    if not math.isfinite(eps) or eps <= 0:
        raise ValueError("eps must be finite and positive")


def row_launch_shape(columns: int, element_size: int) -> tuple[int, int]:
    """Return ``(threads_per_row, values_per_thread)`` for a row width.

    Mirrors ``pick_row_shape`` in ``csrc/rows.hpp`` for aligned rows: the
    smallest group of 64, 256 or 1024 threads whose threads each hold at most
    128 bytes of the row (64 16-bit or 32 float32 values, as 16, 32 or 64).

    Raises:
        ValueError: if the row exceeds the single-pass budget.
    """
    if columns * element_size > MAX_FEATURE_BYTES:
        raise ValueError("feature dimension exceeds the fused normalization limit")
    max_values = 128 // element_size
    for threads in (64, 256, 1024):
        for values in (16, 32, 64):
            if values <= max_values and columns <= threads * values:
                return threads, values
    raise ValueError("feature dimension exceeds the fused normalization limit")


def block_size_and_warps(columns: int, element_size: int) -> tuple[int, int]:
    """Return ``(columns covered per row group, wavefronts per row group)``.

    Keeps the reference's helper name (``_norm_common.py:41-60``); on MI355X
    the "warp" count is the number of 64-lane wavefronts sharing one row.
    """
    threads, values = row_launch_shape(columns, element_size)
    return threads * values, threads // 64


def group_size_m(columns: int) -> int:
    """Number of dweight partial groups for the backward stage 1.

    The reference trades lock contention against stage-two work
    (``_norm_common.py:63-75``). Without locks the only concern is streaming the
    rows at full bandwidth while keeping the float32 partial buffer small, so every
    width uses one group per compute unit (``DEFAULT_GROUPS``).
    """
    del columns
    return DEFAULT_GROUPS
