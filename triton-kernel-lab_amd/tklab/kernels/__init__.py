"""Kernel modules. Importing this package registers every built-in spec."""

from tklab.kernels.fused_softmax import SOFTMAX
from tklab.kernels.residual_rms_norm import RESIDUAL_RMS_NORM
from tklab.kernels.rms_norm import RMS_NORM
from tklab.kernels.rope import ROPE
from tklab.kernels.swiglu import SWIGLU

__all__ = [
    "RESIDUAL_RMS_NORM",
    "RMS_NORM",
    "ROPE",
    "SOFTMAX",
    "SWIGLU",
]
