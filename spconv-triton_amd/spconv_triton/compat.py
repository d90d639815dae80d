# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Stand-in for the ``cumm.tensorview`` activation enum that spconv's API exposes.

``from spconv_triton.compat import tv; tv.gemm.Activation.ReLU`` works as in
spconv, without cumm.
"""

from enum import Enum


class Activation(Enum):
    None_ = 0
    ReLU = 1
    Sigmoid = 2
    LeakyReLU = 3


class _Gemm:
    Activation = Activation


class _TensorView:
    gemm = _Gemm


tv = _TensorView()
