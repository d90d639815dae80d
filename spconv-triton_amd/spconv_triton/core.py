"""Algorithm enums (same members and values as reference ``spconv_triton/core.py:13-23``)."""

from enum import Enum

from .constants import NDIM_DONT_CARE  # noqa: F401  (re-exported like upstream)


class ConvAlgo(Enum):
    Native = 0
    MaskImplicitGemm = 1
    MaskSplitImplicitGemm = 2


class AlgoHint(Enum):
    NoHint = 0
    Fowrard = 1  # upstream spelling, kept for name parity
    BackwardInput = 2
    BackwardWeight = 4
