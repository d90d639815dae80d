# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Table modules (API of spconv.pytorch.tables): concatenate / add the
features of sparse tensors that share indices, or fan one input out."""

from __future__ import annotations

import torch

from spconv_triton.pytorch.core import SparseConvTensor
from spconv_triton.pytorch.modules import SparseModule


def _check_aligned(inputs, msg):
    first = inputs[0]
    for t in inputs:
        if (t.spatial_shape != first.spatial_shape or t.batch_size != first.batch_size
                or t.features.shape[1] != first.features.shape[1]
                or t.indices.shape[0] != first.indices.shape[0]):
            raise AssertionError(msg)


def _combine(inputs, feats):
    first = inputs[0]
    out = SparseConvTensor(feats, first.indices, first.spatial_shape, first.batch_size,
                           first.grid, first.voxel_num, first.indice_dict)
    out.benchmark_record = inputs[1].benchmark_record
    out.thrust_allocator = inputs[1].thrust_allocator
    out._timer = inputs[1]._timer
    return out


class JoinTable(SparseModule):
    def forward(self, inputs: list[SparseConvTensor]):
        _check_aligned(inputs, "you can't use JoinTable in two sptensor with different indices.")
        return _combine(inputs, torch.cat([t.features for t in inputs], 1))

    def input_spatial_size(self, out_size):
        return out_size


class AddTable(SparseModule):
    def forward(self, inputs: list[SparseConvTensor]):
        _check_aligned(inputs, "you can't use AddTable in two sptensor with different indices. "
                               "use AddTableMisaligned instead.")
        return _combine(inputs, sum(t.features for t in inputs))

    def input_spatial_size(self, out_size):
        return out_size


class AddTableMisaligned(SparseModule):
    """Adds sparse tensors of one shape with different coordinates (reference
    tables.py:78-82)."""

    def forward(self, inputs: list[SparseConvTensor]):
        from spconv_triton.pytorch import functional as F

        return F.sparse_add_hash_based(*inputs)


class ConcatTable(SparseModule):
    def forward(self, x):
        return [module(x) for module in self._modules.values()]

    def add(self, module):
        self._modules[str(len(self._modules))] = module
        return self

    def input_spatial_size(self, out_size):
        return self._modules["0"].input_spatial_size(out_size)
