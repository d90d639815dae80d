# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Timer stand-in with spconv's ``CUDAKernelTimer`` interface (records nothing).

Per-kernel timing on MI355X comes from ``rocprofv3 --kernel-trace``.
"""

import contextlib

CPU_ONLY_BUILD = False


class CUDAKernelTimer:
    def __init__(self, enable: bool = True):
        self.enable = enable
        self._timer = None

    @contextlib.contextmanager
    def namespace(self, name: str):
        yield

    @contextlib.contextmanager
    def record(self, name: str, stream: int = 0):
        yield

    def get_all_pair_time(self):
        return {}
