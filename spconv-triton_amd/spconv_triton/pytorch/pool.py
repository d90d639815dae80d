# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Sparse pooling modules (API and behaviour of spconv.pytorch.pool).

Mirror of reference ``spconv_triton/pytorch/pool.py``: ``SparseMaxPool``
(:28-235, MaskImplicitGemm for kv <= 128, Native above), ``SparseAvgPool``
(:276-403, implicit GEMM only, kv <= 32) and the global pools (:238-273).
"""

from __future__ import annotations

import time as _time

import numpy as np
import torch

from spconv_triton.core import ConvAlgo
from spconv_triton.pytorch import functional as Fsp
from spconv_triton.pytorch import ops
from spconv_triton.pytorch.conv import _MAX_NUM_VOXELS_DURING_TRAINING
from spconv_triton.pytorch.core import (
    IndiceData,
    SparseConvTensor,
    expand_nd,
    register_implicit_gemm_indice_data,
)
from spconv_triton.pytorch.modules import SparseModule

CPU_ONLY_BUILD = False


class _PoolBase(SparseModule):
    def _init_common(self, ndim, kernel_size, stride, padding, dilation, indice_key, subm,
                     record_voxel_count):
        self.ndim = ndim
        self.kernel_size = expand_nd(ndim, kernel_size)
        self.stride = self.kernel_size.copy() if stride is None else expand_nd(ndim, stride)
        self.padding = expand_nd(ndim, padding)
        self.subm = subm
        if record_voxel_count and not subm:
            self.register_buffer(_MAX_NUM_VOXELS_DURING_TRAINING,
                                 torch.zeros(1, dtype=torch.int32))
        self.record_voxel_count = record_voxel_count
        self.dilation = expand_nd(ndim, dilation)
        self.indice_key = indice_key

    def extra_repr(self):
        s = "kernel_size={kernel_size}, stride={stride}"
        if self.padding != (0,) * len(self.padding):
            s += ", padding={padding}"
        if self.dilation != (1,) * len(self.dilation):
            s += ", dilation={dilation}"
        if self.algo is not None:
            s += f", algo={self.algo}"
        return s.format(**self.__dict__)

    def get_max_num_voxels(self) -> torch.Tensor | None:
        return getattr(self, _MAX_NUM_VOXELS_DURING_TRAINING, None)

    def _out_shape(self, spatial_shape):
        if self.subm:
            return spatial_shape
        return ops.get_conv_output_size(spatial_shape, self.kernel_size, self.stride,
                                        self.padding, self.dilation)

    def _igemm_pairs(self, x: SparseConvTensor, indice_dict, out_spatial_shape):
        # pooling reads the gather tables only: the mask sorts are deferred
        res, deferred = ops.implicit_gemm_rulebook(
            x.indices, x.batch_size, x.spatial_shape, self.algo, ksize=self.kernel_size,
            stride=self.stride, padding=self.padding, dilation=self.dilation,
            out_padding=[0] * self.ndim, subm=self.subm,
            is_train=(not self.subm) or self.training)
        if self.indice_key is not None:
            register_implicit_gemm_indice_data(
                indice_dict, self.indice_key, res, x.indices, is_subm=self.subm,
                spatial_shape=x.spatial_shape, out_spatial_shape=out_spatial_shape,
                algo=self.algo, ksize=self.kernel_size, stride=self.stride,
                dilation=self.dilation, padding=self.padding, deferred_masks=deferred)
        return res

    def _finish(self, out_tensor, outids, indice_dict, out_spatial_shape, out_features):
        if (not self.subm and self.record_voxel_count
                and hasattr(self, _MAX_NUM_VOXELS_DURING_TRAINING)):
            ops.maximum_value_int_(getattr(self, _MAX_NUM_VOXELS_DURING_TRAINING),
                                   outids.shape[0])
        out_tensor = out_tensor.replace_feature(out_features)
        out_tensor.indices = outids
        out_tensor.indice_dict = indice_dict
        out_tensor.spatial_shape = out_spatial_shape
        return out_tensor


class SparseMaxPool(_PoolBase):
    def __init__(self, ndim, kernel_size=3, stride=1, padding=0, dilation=1,
                 indice_key: str | None = None, subm: bool = False,
                 algo: ConvAlgo | None = None, record_voxel_count: bool = False, name=None):
        super().__init__(name=name)
        self._init_common(ndim, kernel_size, stride, padding, dilation, indice_key, subm,
                          record_voxel_count)
        kv = int(np.prod(kernel_size))
        if algo is None:
            algo = ConvAlgo.MaskImplicitGemm if kv <= 128 else ConvAlgo.Native
        if kv > 128 and algo != ConvAlgo.Native:
            raise AssertionError("implicit gemm don't support kv >= 32 for now")
        self.algo = algo

    @torch.compiler.disable
    def forward(self, x: SparseConvTensor):
        if x.is_quantized:
            raise NotImplementedError("int8 is not supported by spconv_triton")
        if not isinstance(x, SparseConvTensor):
            raise AssertionError
        features = x.features
        out_spatial_shape = self._out_shape(x.spatial_shape)
        out_tensor = x.shadow_copy()
        if x.benchmark:
            if self.name is None:
                raise ValueError("you need to assign name to spmodules before benchmark "
                                 "(spconv.utils.bench.assign_name_to_spmod)")
            if self.name not in x.benchmark_record:
                x.benchmark_record[self.name] = {
                    "type": "SparseMaxPool", "indice_gen_time": [], "time": [],
                    "num_points": [], "num_out_points": [],
                    "params": {"kernel_size": self.kernel_size, "stride": self.stride,
                               "padding": self.padding, "dilation": self.dilation,
                               "channels": features.shape[1]},
                }
            torch.cuda.synchronize()
            t0 = _time.time()
        indice_dict = x.indice_dict.copy()
        if self.algo == ConvAlgo.Native:
            outids, pairs, pair_num = ops.get_indice_pairs(
                x.indices, x.batch_size, x.spatial_shape, ConvAlgo.Native, self.kernel_size,
                self.stride, self.padding, self.dilation, [0] * self.ndim, False)
            if x.benchmark:
                torch.cuda.synchronize()
                out_tensor.benchmark_record[self.name]["indice_gen_time"].append(
                    _time.time() - t0)
                t0 = _time.time()
            if self.indice_key is not None:
                if x.find_indice_pair(self.indice_key) is not None:
                    raise ValueError(f"indice key {self.indice_key} exists")
                indice_dict[self.indice_key] = IndiceData(
                    outids, x.indices, pairs, pair_num, x.spatial_shape, out_spatial_shape,
                    is_subm=False, algo=self.algo, ksize=self.kernel_size, stride=self.stride,
                    padding=self.padding, dilation=self.dilation)
            out_features = Fsp.indice_maxpool(features, pairs.to(features.device),
                                              pair_num.to(features.device), outids.shape[0])
        else:
            res = self._igemm_pairs(x, indice_dict, out_spatial_shape)
            outids = res[0]
            out_features = Fsp.indice_maxpool_implicit_gemm(features, res[2], res[3],
                                                            outids.shape[0])
        if x.benchmark:
            torch.cuda.synchronize()
            rec = out_tensor.benchmark_record[self.name]
            rec["time"].append(_time.time() - t0)
            rec["num_points"].append(features.shape[0])
            rec["num_out_points"].append(out_features.shape[0])
        return self._finish(out_tensor, outids, indice_dict, out_spatial_shape, out_features)


class SparseAvgPool(_PoolBase):
    def __init__(self, ndim, kernel_size=3, stride=1, padding=0, dilation=1,
                 indice_key: str | None = None, subm: bool = False,
                 algo: ConvAlgo | None = None, record_voxel_count: bool = False, name=None):
        super().__init__(name=name)
        self._init_common(ndim, kernel_size, stride, padding, dilation, indice_key, subm,
                          record_voxel_count)
        if int(np.prod(kernel_size)) > 32:
            raise AssertionError("avg pool only support implicit-gemm style indice gen with "
                                 "kv <= 32 limit")
        self.algo = ConvAlgo.MaskImplicitGemm

    @torch.compiler.disable
    def forward(self, x: SparseConvTensor):
        if x.is_quantized:
            raise NotImplementedError("int8 is not supported by spconv_triton")
        if not isinstance(x, SparseConvTensor):
            raise AssertionError
        out_spatial_shape = self._out_shape(x.spatial_shape)
        out_tensor = x.shadow_copy()
        indice_dict = x.indice_dict.copy()
        res = self._igemm_pairs(x, indice_dict, out_spatial_shape)
        outids = res[0]
        out_features = Fsp.indice_avgpool_implicit_gemm(x.features, res[2], res[3],
                                                        outids.shape[0], True)
        return self._finish(out_tensor, outids, indice_dict, out_spatial_shape, out_features)


class SparseGlobalMaxOrAvgPool(SparseModule):
    def __init__(self, is_mean: bool, name=None):
        super().__init__(name=name)
        self.is_mean = is_mean

    @torch.compiler.disable
    def forward(self, x: SparseConvTensor):
        if x.is_quantized:
            raise NotImplementedError("int8 is not supported by spconv_triton")
        if not isinstance(x, SparseConvTensor):
            raise AssertionError
        rows, counts = ops.global_pool_rearrange(x.indices, x.batch_size)
        counts = counts.cpu().numpy()
        per_batch = []
        for b in range(x.batch_size):
            feats = x.features[rows[b, :counts[b]].long()]
            if self.is_mean:
                # spconv quirk: [0] picks channel 0 of the mean, giving [batch]
                per_batch.append(torch.mean(feats, dim=0)[0])
            else:
                per_batch.append(torch.max(feats, dim=0)[0])
        return torch.stack(per_batch)


class SparseGlobalAvgPool(SparseGlobalMaxOrAvgPool):
    def __init__(self, name=None):
        super().__init__(is_mean=True, name=name)


class SparseGlobalMaxPool(SparseGlobalMaxOrAvgPool):
    def __init__(self, name=None):
        super().__init__(is_mean=False, name=name)


def _make_pool(base, ndim: int):
    def __init__(self, kernel_size, stride=None, padding=0, dilation=1, indice_key=None,
                 algo: ConvAlgo | None = None, record_voxel_count: bool = False, name=None):
        base.__init__(self, ndim, kernel_size, stride, padding, dilation, indice_key=indice_key,
                      algo=algo, record_voxel_count=record_voxel_count, name=name)
    return __init__


class SparseMaxPool1d(SparseMaxPool):
    __init__ = _make_pool(SparseMaxPool, 1)


class SparseMaxPool2d(SparseMaxPool):
    __init__ = _make_pool(SparseMaxPool, 2)


class SparseMaxPool3d(SparseMaxPool):
    __init__ = _make_pool(SparseMaxPool, 3)


class SparseMaxPool4d(SparseMaxPool):
    __init__ = _make_pool(SparseMaxPool, 4)


class SparseAvgPool1d(SparseAvgPool):
    __init__ = _make_pool(SparseAvgPool, 1)


class SparseAvgPool2d(SparseAvgPool):
    __init__ = _make_pool(SparseAvgPool, 2)


class SparseAvgPool3d(SparseAvgPool):
    __init__ = _make_pool(SparseAvgPool, 3)
