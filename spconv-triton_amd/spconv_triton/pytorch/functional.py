# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Autograd functions over the sparse ops (names of spconv.pytorch.functional).

Mirror of reference ``spconv_triton/pytorch/functional.py:51-414``: each
Function calls the matching op of ``ops`` forward and backward, under AMP's
``custom_fwd(cast_inputs=float16)`` / ``custom_bwd`` like the reference
(:34-48), with ``once_differentiable`` backwards.
"""

from __future__ import annotations

import torch
from torch.autograd import Function
from torch.autograd.function import once_differentiable

from spconv_triton.compat import tv
from spconv_triton.pytorch import ops
from spconv_triton.pytorch.hash import HashTable
from spconv_triton.tools import CUDAKernelTimer

_FWD = torch.amp.custom_fwd(cast_inputs=torch.float16, device_type="cuda")
_BWD = torch.amp.custom_bwd(device_type="cuda")

_NO_ACT = tv.gemm.Activation.None_


def _pad_grads(n_inputs: int, *grads):
    return (*grads, *([None] * (n_inputs - len(grads))))


class _NativeConvBase(Function):
    """Native-algorithm conv: ops.indice_conv / indice_conv_backward with fixed
    (inverse, subm) flags."""

    INVERSE = False
    SUBM = False

    @classmethod
    def _fwd(cls, ctx, features, filters, indice_pairs, indice_pair_num, num_activate_out, algo,
             timer, bias, act_alpha, act_beta, act_type):
        ctx.save_for_backward(indice_pairs, indice_pair_num, features, filters)
        ctx.algo = algo
        ctx.timer = timer
        return ops.indice_conv(features, filters, indice_pairs, indice_pair_num, num_activate_out,
                               cls.INVERSE, cls.SUBM, algo=algo, timer=timer, bias=bias,
                               act_alpha=act_alpha, act_beta=act_beta, act_type=act_type)

    @classmethod
    def _bwd(cls, ctx, grad_output):
        indice_pairs, indice_pair_num, features, filters = ctx.saved_tensors
        din, dw = ops.indice_conv_backward(features, filters, grad_output, indice_pairs,
                                           indice_pair_num, cls.INVERSE, cls.SUBM, algo=ctx.algo,
                                           timer=ctx.timer)
        return _pad_grads(11, din, dw)


class SparseConvFunction(_NativeConvBase):
    @staticmethod
    @_FWD
    def forward(ctx, features, filters, indice_pairs, indice_pair_num, num_activate_out, algo,
                timer: CUDAKernelTimer = CUDAKernelTimer(False), bias=None, act_alpha=0.0,
                act_beta=0.0, act_type=_NO_ACT):
        return SparseConvFunction._fwd(ctx, features, filters, indice_pairs, indice_pair_num,
                                       num_activate_out, algo, timer, bias, act_alpha, act_beta,
                                       act_type)

    @staticmethod
    @once_differentiable
    @_BWD
    def backward(ctx, grad_output):
        return SparseConvFunction._bwd(ctx, grad_output)


class SparseInverseConvFunction(_NativeConvBase):
    INVERSE = True

    @staticmethod
    @_FWD
    def forward(ctx, features, filters, indice_pairs, indice_pair_num, num_activate_out, algo,
                timer: CUDAKernelTimer = CUDAKernelTimer(False), bias=None, act_alpha=0.0,
                act_beta=0.0, act_type=_NO_ACT):
        return SparseInverseConvFunction._fwd(ctx, features, filters, indice_pairs,
                                              indice_pair_num, num_activate_out, algo, timer, bias,
                                              act_alpha, act_beta, act_type)

    @staticmethod
    @once_differentiable
    @_BWD
    def backward(ctx, grad_output):
        return SparseInverseConvFunction._bwd(ctx, grad_output)


class SubMConvFunction(_NativeConvBase):
    SUBM = True

    @staticmethod
    @_FWD
    def forward(ctx, features, filters, indice_pairs, indice_pair_num, num_activate_out, algo,
                timer: CUDAKernelTimer = CUDAKernelTimer(False), bias=None, act_alpha=0.0,
                act_beta=0.0, act_type=_NO_ACT):
        return SubMConvFunction._fwd(ctx, features, filters, indice_pairs, indice_pair_num,
                                     num_activate_out, algo, timer, bias, act_alpha, act_beta,
                                     act_type)

    @staticmethod
    @once_differentiable
    @_BWD
    def backward(ctx, grad_output):
        return SubMConvFunction._bwd(ctx, grad_output)


class SparseImplicitGemmFunction(Function):
    @staticmethod
    @_FWD
    def forward(ctx, features, filters, pair_fwd, pair_bwd, pair_mask_fwd_splits,
                pair_mask_bwd_splits, mask_argsort_fwd_splits, mask_argsort_bwd_splits,
                num_activate_out, masks, is_train, is_subm,
                timer: CUDAKernelTimer = CUDAKernelTimer(False), fp32_accum=None, bias=None,
                act_alpha=0.0, act_beta=0.0, act_type=_NO_ACT):
        out, mask_out, mask_width = ops.implicit_gemm(
            features, filters, pair_fwd, pair_mask_fwd_splits, mask_argsort_fwd_splits,
            num_activate_out, masks, is_train, is_subm, timer, fp32_accum, bias, act_alpha,
            act_beta, act_type)
        ctx.save_for_backward(features, filters, pair_fwd, pair_bwd)
        ctx.mask_out = mask_out
        ctx.mask_width = mask_width
        ctx.timer = timer
        ctx.splits = (pair_mask_fwd_splits, pair_mask_bwd_splits, mask_argsort_fwd_splits,
                      mask_argsort_bwd_splits)
        ctx.masks = masks
        ctx.is_subm = is_subm
        ctx.fp32_accum = fp32_accum
        return out

    @staticmethod
    @once_differentiable
    @_BWD
    def backward(ctx, grad_output):
        features, filters, pair_fwd, pair_bwd = ctx.saved_tensors
        pm_fwd, pm_bwd, ma_fwd, ma_bwd = ctx.splits
        din, dw = ops.implicit_gemm_backward(
            features, filters, grad_output, pair_fwd, pair_bwd, pm_fwd, pm_bwd, ma_fwd, ma_bwd,
            mask_output_fwd=ctx.mask_out, masks=ctx.masks, mask_width=ctx.mask_width,
            is_subm=ctx.is_subm, timer=ctx.timer, fp32_accum=ctx.fp32_accum)
        return _pad_grads(18, din, dw)


class SparseMaxPoolFunction(Function):
    @staticmethod
    @_FWD
    def forward(ctx, features, indice_pairs, indice_pair_num, num_activate_out):
        out = ops.indice_maxpool(features, indice_pairs, indice_pair_num, num_activate_out)
        ctx.save_for_backward(indice_pairs, indice_pair_num, features, out)
        return out

    @staticmethod
    @once_differentiable
    @_BWD
    def backward(ctx, grad_output):
        indice_pairs, indice_pair_num, features, out = ctx.saved_tensors
        din = ops.indice_maxpool_backward(features, out, grad_output, indice_pairs,
                                          indice_pair_num)
        return din, None, None, None


class SparseMaxPoolImplicitGemmFunction(Function):
    @staticmethod
    @_FWD
    def forward(ctx, features, indice_pairs_fwd, indice_pairs_bwd, num_activate_out):
        out = ops.indice_maxpool_implicit_gemm(features, indice_pairs_fwd, num_activate_out)
        ctx.save_for_backward(indice_pairs_bwd, features, out)
        return out

    @staticmethod
    @once_differentiable
    @_BWD
    def backward(ctx, grad_output):
        indice_pairs_bwd, features, out = ctx.saved_tensors
        din = ops.indice_maxpool_implicit_gemm_backward(features, out, grad_output,
                                                        indice_pairs_bwd)
        return din, None, None, None


class SparseAvgPoolImplicitGemmFunction(Function):
    @staticmethod
    @_FWD
    def forward(ctx, features, indice_pairs_fwd, indice_pairs_bwd, num_activate_out, calc_count):
        out, count = ops.indice_avgpool_implicit_gemm(features, indice_pairs_fwd,
                                                      num_activate_out, calc_count)
        ctx.save_for_backward(indice_pairs_bwd, count)
        return out

    @staticmethod
    @once_differentiable
    @_BWD
    def backward(ctx, grad_output):
        indice_pairs_bwd, count = ctx.saved_tensors
        din = ops.indice_avgpool_implicit_gemm_backward(grad_output, indice_pairs_bwd, count)
        return din, None, None, None, None


indice_conv = SparseConvFunction.apply
implicit_gemm = SparseImplicitGemmFunction.apply
indice_inverse_conv = SparseInverseConvFunction.apply
indice_subm_conv = SubMConvFunction.apply
indice_maxpool = SparseMaxPoolFunction.apply
indice_maxpool_implicit_gemm = SparseMaxPoolImplicitGemmFunction.apply
indice_avgpool_implicit_gemm = SparseAvgPoolImplicitGemmFunction.apply


_MAX_INT32 = 2 ** 31 - 1


def _indice_to_scalar(indices: torch.Tensor, shape: list[int]) -> torch.Tensor:
    """Batch-major linear key of [b, c0, c1, ...] rows (reference
    functional.py:417-426)."""
    if indices.shape[1] != len(shape):
        raise AssertionError
    stride = [1] * len(shape)
    for i in range(len(shape) - 2, -1, -1):
        stride[i] = stride[i + 1] * shape[i + 1]
    scalar = indices[:, -1].clone()
    for i in range(len(shape) - 1):
        scalar += stride[i] * indices[:, i]
    return scalar.contiguous()


def _check_same_space(tens):
    first = tens[0]
    for ten in tens:
        if ten.spatial_shape != first.spatial_shape:
            raise AssertionError
        if ten.batch_size != first.batch_size:
            raise AssertionError
        if ten.features.shape[1] != first.features.shape[1]:
            raise AssertionError


def _finish_add(tens, feats, inds):
    from spconv_triton.pytorch.core import SparseConvTensor

    first = tens[0]
    res = SparseConvTensor(feats, inds, first.spatial_shape, first.batch_size,
                           benchmark=first.benchmark)
    largest = max(range(len(tens)), key=lambda i: (tens[i].features.shape[0], -i))
    if feats.shape[0] == tens[largest].features.shape[0]:
        res.indice_dict = tens[largest].indice_dict
    res.benchmark_record = first.benchmark_record
    res._timer = first._timer
    res.thrust_allocator = first.thrust_allocator
    return res


def sparse_add_hash_based(*tens):
    """Sum of sparse tensors with different coordinate sets (reference
    functional.py:429-490): every coordinate's linear key goes into a device
    HashTable, the stored keys are numbered in ascending order
    (assign_arange_), and each input's features are added into the rows of
    its keys, in input order."""
    _check_same_space(tens)
    first = tens[0]
    shape = [first.batch_size, *first.spatial_shape]
    whole = 1
    for v in shape:
        whole *= int(v)
    key64 = whole >= _MAX_INT32
    table = HashTable(first.features.device, torch.int64 if key64 else torch.int32, torch.int32,
                      2 * sum(t.features.shape[0] for t in tens))
    scalars = []
    for ten in tens:
        ind = ten.indices.long() if key64 else ten.indices
        scalar = _indice_to_scalar(ind, shape)
        scalars.append(scalar)
        table.insert(scalar)
    count = int(table.assign_arange_().item())
    feat = first.features
    out_features = torch.zeros([count, feat.shape[1]], dtype=feat.dtype, device=feat.device)
    out_indices = torch.zeros([count, first.indices.shape[1]], dtype=first.indices.dtype,
                              device=first.indices.device)
    for ten, scalar in zip(tens, scalars):
        rows, _ = table.query(scalar)
        rows = rows.long()
        out_features[rows] += ten.features
        out_indices[rows] = ten.indices
    return _finish_add(tens, out_features, out_indices)


def sparse_add(*tens):
    """Sum of sparse tensors (reference functional.py:493-535, a coalesced
    torch.sparse sum): the union of the coordinates in ascending batch-major
    order with the features of equal coordinates added in input order -- the
    same result as sparse_add_hash_based."""
    return sparse_add_hash_based(*tens)
