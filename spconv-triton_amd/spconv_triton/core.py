# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
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
