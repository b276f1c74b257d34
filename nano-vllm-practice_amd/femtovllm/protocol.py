"""Enums shared by the operator layer and its callers.

Same names and values as femtovllm/protocol.py:20-32 of the reference, so
engine code that routes on them keeps working.
"""

import enum


class AttentionBackend(str, enum.Enum):
    """Which varlen attention route a model layer takes (protocol.py:20-25)."""

    PYTORCH = "pytorch"
    CUSTOM_GEMM = "custom_gemm"
    CUSTOM_GEMM_GEMV = "custom_gemm_gemv"


class ImplCustomKernel(str, enum.Enum):
    """Kernel family selector kept for signature compatibility (protocol.py:28-32).

    Both members run the same HIP kernels for gfx950; there is no second
    backend behind ``TRITON``.
    """

    CUDA = "cuda"
    TRITON = "triton"
