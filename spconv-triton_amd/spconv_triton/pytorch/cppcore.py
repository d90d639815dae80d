# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Stream helper of spconv.pytorch.cppcore (no cumm/tensorview here)."""

import torch


def get_current_stream() -> int:
    if torch.cuda.is_available():
        return torch.cuda.current_stream().cuda_stream
    return 0


def torch_tensor_to_tv(*args, **kwargs):
    raise NotImplementedError("spconv_triton has no cumm/tensorview backend; "
                              "use plain torch tensors.")
