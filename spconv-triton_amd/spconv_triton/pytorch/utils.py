# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Point-cloud voxelisation, a drop-in for ``spconv_triton.pytorch.utils``
(reference ``spconv_triton/pytorch/utils.py:16-192``).

``PointToVoxel`` keeps the reference's constructor, public metadata (``vsize``,
``grid_size``, ``coors_range`` and ``grid_stride`` in ZYX order) and its
preallocated ``voxels`` / ``indices`` / ``num_per_voxel`` buffers, and fills
them with ``sp_point2voxel`` (csrc/sp_voxel.hip): voxels numbered in order of
their first point ("first come, first served"), at most
``max_num_points_per_voxel`` points per voxel in point order, and the voxel
id of every point (-1 when dropped by the range check or the voxel cap).
Points must be on the GPU; this package has no CPU path.
"""

from __future__ import annotations

import ctypes

import torch

from spconv_triton.pytorch._impl import _lib


class PointToVoxel:
    """WARNING: you MUST construct PointToVoxel AFTER set device."""

    def __init__(self, vsize_xyz: list[float], coors_range_xyz: list[float],
                 num_point_features: int, max_num_voxels: int, max_num_points_per_voxel: int,
                 device: torch.device = torch.device("cpu:0")):
        self.ndim = len(vsize_xyz)
        self.device = device
        self.num_point_features = num_point_features
        self.max_num_voxels = max_num_voxels
        self.max_num_points_per_voxel = max_num_points_per_voxel
        cmin = coors_range_xyz[:self.ndim]
        cmax = coors_range_xyz[self.ndim:]
        grid_size_xyz = [round((cmax[i] - cmin[i]) / vsize_xyz[i]) for i in range(self.ndim)]
        self._vsize_xyz = list(vsize_xyz)
        self._grid_size_xyz = grid_size_xyz
        self._coors_range_xyz = list(coors_range_xyz)
        # public metadata in ZYX order, as spconv stores it
        self.vsize = list(reversed(vsize_xyz))
        self.grid_size = list(reversed(grid_size_xyz))
        self.coors_range = list(reversed(cmin)) + list(reversed(cmax))
        stride = [1] * self.ndim
        for i in range(self.ndim - 2, -1, -1):
            stride[i] = stride[i + 1] * self.grid_size[i + 1]
        self.grid_stride = stride
        self.voxels = torch.zeros([max_num_voxels, max_num_points_per_voxel, num_point_features],
                                  dtype=torch.float32, device=device)
        self.indices = torch.zeros([max_num_voxels, self.ndim], dtype=torch.int32, device=device)
        self.num_per_voxel = torch.zeros([max_num_voxels], dtype=torch.int32, device=device)

    def __call__(self, pc: torch.Tensor, clear_voxels: bool = True, empty_mean: bool = False):
        res = self.generate_voxel_with_id(pc, clear_voxels, empty_mean)
        return res[0], res[1], res[2]

    def generate_voxel_with_id(self, pc: torch.Tensor, clear_voxels: bool = True,
                               empty_mean: bool = False):
        if pc.device.type != self.device.type:
            raise AssertionError("your pc device is wrong")
        _lib.require_gpu(pc, self.voxels)
        if pc.dtype not in (torch.float32, torch.float64):
            raise NotImplementedError(f"PointToVoxel: points of dtype {pc.dtype}")
        if pc.dim() != 2 or pc.shape[1] < max(self.ndim, self.num_point_features):
            raise AssertionError("points must be [N, >= max(ndim, num_point_features)]")
        pc = pc.contiguous()
        n = pc.shape[0]
        pc_voxel_id = torch.empty([n], dtype=torch.int64, device=pc.device)
        L = _lib.lib()
        ws = _lib.workspace(L.sp_point2voxel_workspace_size(n, self.max_num_voxels), pc.device)
        vsize = (ctypes.c_double * 4)(*self._vsize_xyz)
        cmin = (ctypes.c_double * 4)(*self._coors_range_xyz[:self.ndim])
        gsize = (ctypes.c_int64 * 4)(*self._grid_size_xyz)
        nv = ctypes.c_int64(0)
        _lib.check(L.sp_point2voxel(
            _lib.ptr(pc), _lib.dtype_code(pc.dtype), n, pc.shape[1], self.ndim, vsize, cmin, gsize,
            self.num_point_features, self.max_num_voxels, self.max_num_points_per_voxel,
            int(clear_voxels), int(empty_mean), _lib.ptr(self.voxels), _lib.ptr(self.indices),
            _lib.ptr(self.num_per_voxel), _lib.ptr(pc_voxel_id), ctypes.byref(nv), _lib.ptr(ws),
            ws.numel(), _lib.stream_of(pc.device)), "sp_point2voxel")
        k = int(nv.value)
        return (self.voxels[:k].clone(), self.indices[:k].clone(), self.num_per_voxel[:k].clone(),
                pc_voxel_id)


def gather_features_by_pc_voxel_id(seg_res_features: torch.Tensor, pc_voxel_id: torch.Tensor,
                                   invalid_value: int | float = 0):
    """Per-point features from per-voxel results: row pc_voxel_id[i], or
    invalid_value where the point has no voxel (reference utils.py:166-192)."""
    if seg_res_features.device != pc_voxel_id.device:
        pc_voxel_id = pc_voxel_id.to(seg_res_features.device)
    shape = (pc_voxel_id.shape[0], *seg_res_features.shape[1:])
    res = torch.full(shape, invalid_value, dtype=seg_res_features.dtype,
                     device=seg_res_features.device)
    valid = torch.nonzero(pc_voxel_id != -1).view(-1)
    res[valid] = seg_res_features[pc_voxel_id[valid]]
    return res
