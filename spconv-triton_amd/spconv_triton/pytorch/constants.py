# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Torch version as a list of ints (spconv.pytorch.constants)."""

import torch


def _parse(version: str) -> list[int]:
    core = version.split("+")[0].split(".dev")[0]
    try:
        return [int(p) for p in core.split(".")[:3]]
    except ValueError:
        return [1, 8, 0]


PYTORCH_VERSION: list[int] = _parse(str(torch.__version__))
