# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Configuration flags, read the same way as reference ``spconv_triton/constants.py``.

Live flags:

* ``SPCONV_SAVED_WEIGHT_LAYOUT`` (env): checkpoint weight layout handled by the
  conv load hook (``KRSC``, ``RSKC`` or ``RSCK``).
* ``SPCONV_FX_TRACE_MODE`` (env, ``1``): skip SparseConvTensor shape asserts.
* ``SPCONV_DO_SORT`` (env, default ``1``): sort igemm mask words.
* ``SPCONV_ALLOW_TF32`` / ``SPCONV_ALLOW_FP16_ACCUM`` (module attributes, read
  per call): accepted; the gfx950 kernels always accumulate in fp32 (see
  ``spconv_triton.pytorch._impl.gemm``).

The remaining names exist so that code importing them from spconv keeps
working; nothing reads them.
"""

import os
from pathlib import Path

PACKAGE_ROOT = Path(__file__).parent.resolve()
PACKAGE_NAME = "spconv_triton"

SAVED_WEIGHT_LAYOUT = os.getenv("SPCONV_SAVED_WEIGHT_LAYOUT", "")
if SAVED_WEIGHT_LAYOUT not in ("", "KRSC", "RSKC", "RSCK"):
    raise AssertionError("please set SAVED_WEIGHT_LAYOUT to KRSC, RSKC or RSCK")

SPCONV_FX_TRACE_MODE = os.getenv("SPCONV_FX_TRACE_MODE", "0") == "1"
SPCONV_DO_SORT = os.getenv("SPCONV_DO_SORT", "1") == "1"
SPCONV_USE_DIRECT_TABLE = True
SPCONV_DEBUG_WEIGHT = False
SPCONV_ALLOW_TF32 = False
SPCONV_ALLOW_FP16_ACCUM = os.getenv("SPCONV_ALLOW_FP16_ACCUM", "0") == "1"
NDIM_DONT_CARE = 3

# import-parity names (unused)
ALL_WEIGHT_IS_KRSC = True
FILTER_HWIO = False
DISABLE_JIT = False
EDITABLE_INSTALLED = False
BOOST_ROOT = None
SPCONV_DEBUG_SAVE_PATH = ""
SPCONV_BWD_SPLITK = [1, 2, 4, 8, 16, 32, 64]
SPCONV_DIRECT_TABLE_HASH_SIZE_SCALE = 1.1
SPCONV_INT8_DEBUG = False
SPCONV_DEBUG_CPP_ONLY = False
SPCONV_DEBUG_NVRTC_KERNELS = False
SPCONV_CPP_INDICE_PAIRS = False
SPCONV_CPP_INDICE_PAIRS_IGEMM = False
SPCONV_CPP_GEMM = False


class AllocKeys:
    """Allocator dictionary keys of upstream spconv (import parity only)."""

    PairBwd = "PairBwd"
    IndiceNumPerLoc = "IndiceNumPerLoc"
    PairMask = "PairMask"
    MaskArgSort = "MaskArgSort"
    OutIndices = "OutIndices"
    PairFwd = "PairFwd"
    PairMaskBwd = "PairMaskBwd"
    MaskArgSortBwd = "MaskArgSortBwd"
    MaskOutputFwd = "MaskOutputFwd"
    OutFeatures = "OutFeatures"
    Features = "Features"
    Filters = "Filters"
    OutBp = "OutBp"
    DIn = "DIn"
    DFilters = "DFilters"
    InpBuffer = "InpBuffer"
    OutBuffer = "OutBuffer"
    IndicePairsUniq = "IndicePairsUniq"
    IndicePairsUniqBackup = "IndicePairsUniqBackup"
    HashKOrKV = "HashKOrKV"
    HashV = "HashV"
    ThrustTemp = "ThrustTemp"
    TightUniqueCount = "TightUniqueCount"
