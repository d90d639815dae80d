# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""SparseConvTensor and the rulebook cache records.

Same public surface as reference ``spconv_triton/pytorch/core.py``:
``SparseConvTensor`` (:181-372), ``IndiceData`` (:47-76),
``ImplicitGemmIndiceData`` (:79-120), ``register_implicit_gemm_indice_data``
(:123-164), ``scatter_nd`` and ``expand_nd``.
"""

from __future__ import annotations

from typing import Any, Union

import numpy as np
import torch

from spconv_triton.constants import SPCONV_FX_TRACE_MODE
from spconv_triton.core import ConvAlgo
from spconv_triton.tools import CUDAKernelTimer

try:  # torch.fx-friendly metaclass, as in spconv
    from torch.fx import ProxyableClassMeta as _TensorMeta
except Exception:  # pragma: no cover
    _TensorMeta = type


class ThrustSortAllocator:
    """Interface stand-in for spconv's thrust scratch allocator (unused: the
    HIP library takes its workspaces from torch's caching allocator)."""

    def __init__(self, device: torch.device) -> None:
        self.alloced_objs: dict = {}
        self.device = device


class IndiceData:
    """Native-algorithm rulebook cached under an ``indice_key``."""

    def __init__(self, out_indices, indices, indice_pairs, indice_pair_num, spatial_shape,
                 out_spatial_shape, is_subm: bool, algo: ConvAlgo, ksize: list[int],
                 stride: list[int], dilation: list[int], padding: list[int],
                 voxel_num: Any | None = None):
        self.out_indices = out_indices
        self.indices = indices
        self.indice_pairs = indice_pairs
        self.indice_pair_num = indice_pair_num
        self.spatial_shape = spatial_shape
        self.out_spatial_shape = out_spatial_shape
        self.is_subm = is_subm
        self.algo = algo
        self.ksize = ksize
        self.stride = stride
        self.dilation = dilation
        self.padding = padding
        self.voxel_num = voxel_num


class ImplicitGemmIndiceData:
    """Implicit-GEMM rulebook (gather tables + sorted masks) cached under a key."""

    def __init__(self, out_indices: torch.Tensor, indices: torch.Tensor, pair_fwd: torch.Tensor,
                 pair_bwd: torch.Tensor, pair_mask_fwd_splits: list[torch.Tensor],
                 pair_mask_bwd_splits: list[torch.Tensor],
                 mask_argsort_fwd_splits: list[torch.Tensor],
                 mask_argsort_bwd_splits: list[torch.Tensor], masks: list[np.ndarray],
                 spatial_shape, out_spatial_shape, is_subm: bool, algo: ConvAlgo,
                 ksize: list[int], stride: list[int], dilation: list[int], padding: list[int],
                 in_voxel_num: Any | None = None, out_voxel_num: Any | None = None,
                 deferred_masks: Any | None = None):
        self.out_indices = out_indices
        self.indices = indices
        self.pair_fwd = pair_fwd
        self.pair_bwd = pair_bwd
        # the four mask-split lists; with deferred_masks (an object whose get()
        # returns them) they are computed the first time one is read
        self._mask_splits = [pair_mask_fwd_splits, pair_mask_bwd_splits,
                             mask_argsort_fwd_splits, mask_argsort_bwd_splits]
        self._deferred_masks = deferred_masks
        self.masks = masks
        self.spatial_shape = spatial_shape
        self.out_spatial_shape = out_spatial_shape
        self.is_subm = is_subm
        self.algo = algo
        self.ksize = ksize
        self.stride = stride
        self.dilation = dilation
        self.padding = padding
        self.in_voxel_num = in_voxel_num
        self.out_voxel_num = out_voxel_num

    def _splits(self) -> list:
        if self._deferred_masks is not None:
            self._mask_splits = list(self._deferred_masks.get())
            self._deferred_masks = None
        return self._mask_splits

    def _set_split(self, i: int, value) -> None:
        self._splits()[i] = value

    pair_mask_fwd_splits = property(lambda self: self._splits()[0],
                                    lambda self, v: self._set_split(0, v))
    pair_mask_bwd_splits = property(lambda self: self._splits()[1],
                                    lambda self, v: self._set_split(1, v))
    mask_argsort_fwd_splits = property(lambda self: self._splits()[2],
                                       lambda self, v: self._set_split(2, v))
    mask_argsort_bwd_splits = property(lambda self: self._splits()[3],
                                       lambda self, v: self._set_split(3, v))


def register_implicit_gemm_indice_data(indice_dict, indice_key, res, indices, *, is_subm,
                                       spatial_shape, out_spatial_shape, algo, ksize, stride,
                                       dilation, padding, deferred_masks=None):
    """Store a ``get_indice_pairs_implicit_gemm`` 9-tuple under ``indice_key``;
    an existing key is an error (reference core.py:123-164).  ``deferred_masks``
    (from ``ops.implicit_gemm_rulebook``) supplies the mask splits on first read."""
    if indice_key in indice_dict:
        raise AssertionError(f"your indice key {indice_key} already exists in this sparse tensor.")
    indice_dict[indice_key] = ImplicitGemmIndiceData(
        res[0], indices, res[2], res[3],
        pair_mask_fwd_splits=res[4], pair_mask_bwd_splits=res[5],
        mask_argsort_fwd_splits=res[6], mask_argsort_bwd_splits=res[7], masks=res[8],
        spatial_shape=spatial_shape, out_spatial_shape=out_spatial_shape, is_subm=is_subm,
        algo=algo, ksize=ksize, stride=stride, dilation=dilation, padding=padding,
        deferred_masks=deferred_masks)


def scatter_nd(indices: torch.Tensor, updates: torch.Tensor, shape):
    """Dense tensor of ``shape`` with ``updates`` written at ``indices``
    (later duplicates overwrite earlier ones, as in spconv)."""
    out = torch.zeros(*shape, dtype=updates.dtype, device=updates.device)
    nd = indices.shape[-1]
    flat = indices.reshape(-1, nd)
    tail = list(shape[nd:])
    out[tuple(flat[:, i] for i in range(nd))] = updates.reshape(-1, *tail)
    return out


def expand_nd(ndim: int, val) -> list[int]:
    if isinstance(val, int):
        vals = [val] * ndim
    else:
        vals = list(val)
    if len(vals) != ndim:
        raise AssertionError
    return [int(v) for v in vals]


class SparseConvTensor(metaclass=_TensorMeta):
    """Features [N, C] + int32 indices [N, ndim + 1] (batch in column 0) + the
    spatial shape, with the rulebooks of earlier layers in ``indice_dict``."""

    def __init__(self, features: torch.Tensor, indices: torch.Tensor,
                 spatial_shape: list[int] | np.ndarray, batch_size: int,
                 grid: torch.Tensor | None = None, voxel_num: torch.Tensor | None = None,
                 indice_dict: dict | None = None, benchmark: bool = False,
                 permanent_thrust_allocator: bool = False, enable_timer: bool = False,
                 force_algo: ConvAlgo | None = None):
        ndim = indices.shape[1] - 1
        if not SPCONV_FX_TRACE_MODE:
            if features.ndim != 2:
                raise AssertionError
            if indices.ndim != 2:
                raise AssertionError
            if len(spatial_shape) != ndim:
                raise AssertionError("spatial shape must equal to ndim")
            if indices.dtype != torch.int32:
                raise AssertionError("only support int32")
            if batch_size <= 0:
                raise AssertionError
        self._features = features
        self.indices = indices
        self.spatial_shape = [int(v) for v in spatial_shape]
        self.batch_size = batch_size
        self.indice_dict = {} if indice_dict is None else indice_dict
        self.grid = torch.Tensor() if grid is None else grid
        self.voxel_num = voxel_num
        self.benchmark = benchmark
        self.benchmark_record: dict = {}
        self.thrust_allocator = (ThrustSortAllocator(features.device)
                                 if permanent_thrust_allocator else None)
        self._timer = CUDAKernelTimer(enable_timer)
        self.force_algo = force_algo
        self.int8_scale: np.ndarray | None = None

    def __repr__(self):
        return f"SparseConvTensor[shape={self._features.shape}]"

    @property
    def is_quantized(self):
        return self.features.dtype == torch.qint8

    def q_scale(self):
        if self.is_quantized:
            return self.features.q_scale()
        raise ValueError("sparse tensor must be quantized")

    def _carry_state(self, other: "SparseConvTensor") -> "SparseConvTensor":
        other.benchmark_record = self.benchmark_record
        other.thrust_allocator = self.thrust_allocator
        other._timer = self._timer
        other.force_algo = self.force_algo
        other.int8_scale = self.int8_scale
        return other

    def replace_feature(self, feature: torch.Tensor) -> "SparseConvTensor":
        new = SparseConvTensor(feature, self.indices, self.spatial_shape, self.batch_size,
                               self.grid, self.voxel_num, self.indice_dict)
        new.benchmark = self.benchmark
        return self._carry_state(new)

    def shadow_copy(self) -> "SparseConvTensor":
        new = SparseConvTensor(self.features, self.indices, self.spatial_shape, self.batch_size,
                               self.grid, self.voxel_num, self.indice_dict, self.benchmark)
        return self._carry_state(new)

    def select_by_index(self, valid_indices: torch.Tensor):
        # spconv assigns to the read-only ``features`` here, so this always raises
        new = self.shadow_copy()
        new.indices = self.indices[valid_indices]
        new.features = self.features[valid_indices]
        new.indice_dict.clear()
        return new

    def minus(self):
        return self.replace_feature(-self.features)

    @property
    def features(self):
        return self._features

    @features.setter
    def features(self, val):
        raise ValueError("you can't set feature directly, use "
                         "'x = x.replace_feature(your_new_feature)' to generate new "
                         "SparseConvTensor instead.")

    @classmethod
    def from_dense(cls, x: torch.Tensor):
        """From a channel-last dense tensor [B, *spatial, C]."""
        sp = x.to_sparse(x.ndim - 1)
        return cls(sp.values(), sp.indices().permute(1, 0).contiguous().int(),
                   list(sp.shape[1:-1]), sp.shape[0])

    def dequantize(self):
        return self.replace_feature(self.features.dequantize())

    @property
    def spatial_size(self):
        return np.prod(self.spatial_shape)

    def find_indice_pair(self, key):
        if key is None:
            return None
        return self.indice_dict.get(key)

    def dense(self, channels_first: bool = True):
        shape = [self.batch_size, *self.spatial_shape, self.features.shape[1]]
        res = scatter_nd(self.indices.to(self.features.device).long(), self.features, shape)
        if not channels_first:
            return res
        nd = len(self.spatial_shape)
        perm = [0, nd + 1, *range(1, nd + 1)]
        return res.permute(*perm).contiguous()

    @staticmethod
    def _other_features(other):
        if not isinstance(other, (SparseConvTensor, torch.Tensor)):
            raise AssertionError
        return other if isinstance(other, torch.Tensor) else other.features

    def __add__(self, other: Union["SparseConvTensor", torch.Tensor]):
        return self.replace_feature(self.features + self._other_features(other))

    def __iadd__(self, other: Union["SparseConvTensor", torch.Tensor]):
        self.features += self._other_features(other)
        return self

    def __radd__(self, other: Union["SparseConvTensor", torch.Tensor]):
        return self.replace_feature(self.features + self._other_features(other))
