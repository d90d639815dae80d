# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Identity module accepting and ignoring extra arguments (spconv.pytorch.identity)."""

from torch import nn


class Identity(nn.Module):
    def forward(self, input, *args, **kwargs):
        return input
