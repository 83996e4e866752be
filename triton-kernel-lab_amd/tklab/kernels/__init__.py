"""Kernel modules. Importing this package registers every built-in spec."""

from tklab.kernels.flash_attention import ATTENTION_CAUSAL, ATTENTION_NONCAUSAL
from tklab.kernels.fused_softmax import SOFTMAX
from tklab.kernels.matmul import MATMUL_FP16ACC, MATMUL_FP32ACC
from tklab.kernels.residual_rms_norm import RESIDUAL_RMS_NORM
from tklab.kernels.rms_norm import RMS_NORM
from tklab.kernels.rope import ROPE
from tklab.kernels.swiglu import SWIGLU

__all__ = [
    "ATTENTION_CAUSAL",
    "ATTENTION_NONCAUSAL",
    "MATMUL_FP16ACC",
    "MATMUL_FP32ACC",
    "RESIDUAL_RMS_NORM",
    "RMS_NORM",
    "ROPE",
    "SOFTMAX",
    "SWIGLU",
]
