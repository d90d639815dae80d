# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""spconv_triton for AMD Instinct MI355X (gfx950).

Drop-in for ``spconv_triton`` / ``spconv``: keep ``import spconv_triton.pytorch
as spconv`` and the same modules, rulebook caching and checkpoints work; the
sparse-convolution hot path (pair generation, gather-GEMM, pooling) runs in
the hand-written HIP library ``libspconv_hip.so``.
"""

from . import constants
from .core import AlgoHint, ConvAlgo

__version__ = "0.1.0+gfx950"

# Version of upstream spconv whose behaviour this package reproduces.
SPCONV_VERSION_NUMBERS = [2, 3, 8]

__all__ = ["AlgoHint", "ConvAlgo", "constants", "__version__", "SPCONV_VERSION_NUMBERS"]
