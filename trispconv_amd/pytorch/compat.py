"""``ConvAlgo`` — accepted for API compatibility, never consulted.

Mirrors trispconv/pytorch/compat.py:4-7 (spconv's enum).  The backend always
runs its one fused implicit-GEMM path, whose accumulation follows the slot
order of ``Native``.
"""
from enum import Enum


class ConvAlgo(Enum):
    Native = 0
    MaskImplicitGemm = 1
    MaskSplitImplicitGemm = 2
