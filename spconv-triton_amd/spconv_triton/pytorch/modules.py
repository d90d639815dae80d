# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Sparse module containers (API of spconv.pytorch.modules).

Plain-Python equivalents of reference ``spconv_triton/pytorch/modules.py``:
``SparseModule``, ``SparseSequential`` (dense modules act on ``features``),
and the BatchNorm/ReLU/Identity wrappers.
"""

from __future__ import annotations

import time
from collections import OrderedDict

import torch
from torch import nn


def _sparse_tensor_cls():
    from spconv_triton.pytorch.core import SparseConvTensor

    return SparseConvTensor


def is_spconv_module(module):
    return isinstance(module, (SparseModule, SparseBatchNorm, SparseReLU))


def is_sparse_conv(module):
    from spconv_triton.pytorch.conv import SparseConvolution

    return isinstance(module, SparseConvolution)


class SparseModule(nn.Module):
    """Marks a module as taking and returning SparseConvTensor."""

    def __init__(self, name=None):
        super().__init__()
        self.name = name
        self._sparse_unique_name = ""


class SparseSequential(SparseModule):
    """Runs children in order; non-sparse children are applied to ``features``
    (skipped for an empty tensor)."""

    def __init__(self, *args, **kwargs):
        super().__init__()
        if len(args) == 1 and isinstance(args[0], OrderedDict):
            for key, module in args[0].items():
                self.add_module(key, module)
        else:
            for i, module in enumerate(args):
                self.add_module(str(i), module)
        for key, module in kwargs.items():
            if key in self._modules:
                raise ValueError("name exists.")
            self.add_module(key, module)

    def __getitem__(self, idx):
        n = len(self)
        if not -n <= idx < n:
            raise IndexError(f"index {idx} is out of range")
        return list(self._modules.values())[idx % n]

    def __len__(self):
        return len(self._modules)

    def add(self, module, name=None):
        if name is None:
            name = str(len(self._modules))
            if name in self._modules:
                raise KeyError("name exists")
        self.add_module(name, module)

    def forward(self, x):
        sct = _sparse_tensor_cls()
        for module in self._modules.values():
            if is_spconv_module(module):
                x = module(x)
            elif isinstance(x, sct):
                if x.indices.shape[0] != 0:
                    x = x.replace_feature(module(x.features))
            else:
                x = module(x)
        return x


def assign_name_for_sparse_modules(module: nn.Module):
    for key, mod in module.named_modules():
        if isinstance(mod, SparseModule):
            mod._sparse_unique_name = key


def _on_features(mod_forward, self, x):
    if isinstance(x, _sparse_tensor_cls()):
        return x.replace_feature(mod_forward(self, x.features))
    return mod_forward(self, x)


class SparseBatchNorm(nn.BatchNorm1d):
    def forward(self, x):
        return _on_features(nn.BatchNorm1d.forward, self, x)


class SparseSyncBatchNorm(nn.SyncBatchNorm):
    def forward(self, x):
        return _on_features(nn.SyncBatchNorm.forward, self, x)


class SparseReLU(nn.ReLU):
    def forward(self, x):
        return _on_features(nn.ReLU.forward, self, x)


class SparseIdentity(nn.Identity):
    def forward(self, x):
        return _on_features(nn.Identity.forward, self, x)


class PrintTensorMeta(nn.Module):
    def forward(self, x):
        t = x.features if isinstance(x, _sparse_tensor_cls()) else x
        if isinstance(t, torch.Tensor):
            print(t.min(), t.max(), t.mean())
        return x


class PrintCurrentTime(nn.Module):
    def __init__(self) -> None:
        super().__init__()
        self.first_time = time.time()

    def forward(self, x, msg="", reset: bool = False):
        if reset:
            self.first_time = time.time()
        torch.cuda.synchronize()
        print(msg, time.time() - self.first_time)
        return x
