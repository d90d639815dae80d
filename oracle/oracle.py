"""CPU oracle for the sparse-convolution hot path -- TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py``, always as the checker.  The product package never imports
it (the HIP library must carry every result it returns).

It restates the reference's host flow in numpy around the C kernels of
``spconv_oracle.c`` (built by the Makefile beside this file):

* ``igemm_pairs``  follows ``spconv_triton/pytorch/_impl/pairs.py:281-426``
* ``native_pairs`` follows ``pairs.py:242-278``
* ``compute_candidates`` follows ``pairs.py:126-220``
* ``native_pair_to_tables`` follows ``pairs.py:429-469``
* ``gemm_*`` follow ``_impl/gemm.py:254-321`` (fwd / dgrad) and ``:356-426`` (wgrad)
* ``maxpool_*`` / ``avgpool_*`` follow ``_impl/pool.py:45-257``
* ``point_to_voxel`` follows ``spconv_triton/pytorch/utils.py:16-163``
* ``hash_sparse_add`` follows ``spconv_triton/pytorch/functional.py:417-490``

Every function returns numpy arrays; integer outputs are the exact values the
reference produces (keys are widened to int64, which the reference proves
byte-identical on valid entries, ``pair_kernels.py:12-16``).
"""

from __future__ import annotations

import ctypes
import functools
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libspconv_oracle.so"

_POINT_VANISH_MSG = (
    "Your points vanished here, this usually happens when you provide "
    "conv params that may ignore some input points. Example: "
    "spatial_shape={}, ksize={}, stride={}, padding={}, dilation={}"
)


def build() -> Path:
    """Compile the C oracle (idempotent)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


@functools.lru_cache(maxsize=None)
def lib() -> ctypes.CDLL:
    if not _LIB_PATH.exists():
        build()
    L = ctypes.CDLL(str(_LIB_PATH))
    L.orc_unique_sorted.restype = ctypes.c_int64
    return L


def _p(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else ctypes.c_void_p(0)


def _i64(vals) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(vals, dtype=np.int64))


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(ctypes.c_int(int(n)))


def num_threads() -> int:
    return int(lib().orc_num_threads())


# ---------------------------------------------------------------------------
# shapes (pairs.py:59-88)
# ---------------------------------------------------------------------------

def get_conv_output_size(input_size, kernel_size, stride, padding, dilation):
    out = []
    for i in range(len(input_size)):
        size = (input_size[i] + 2 * padding[i] - dilation[i] * (kernel_size[i] - 1) - 1) // stride[i] + 1
        out.append(1 if kernel_size[i] == -1 else size)
    return out


def get_deconv_output_size(input_size, kernel_size, stride, padding, dilation, output_padding):
    out = []
    for i in range(len(input_size)):
        if kernel_size[i] == -1:
            raise ValueError("deconv don't support kernel_size < 0")
        out.append((input_size[i] - 1) * stride[i] - 2 * padding[i] + kernel_size[i] + output_padding[i])
    return out


def kernel_offsets(ksize) -> np.ndarray:
    kv = int(np.prod(ksize))
    offs = np.empty((kv, len(ksize)), dtype=np.int64)
    ks = _i64(ksize)
    lib().orc_kernel_offsets(ctypes.c_int(len(ksize)), _p(ks), _p(offs))
    return offs


# ---------------------------------------------------------------------------
# candidates (pairs.py:126-220)
# ---------------------------------------------------------------------------

class Candidates:
    def __init__(self, valid, out_row, out_inds, out_shape, n_out, kv, lin_is_int32):
        self.valid = valid          # [kv, N] bool
        self.out_row = out_row      # [kv, N] int32
        self.out_inds = out_inds    # [n_out, ndim+1] int32 or None (subm: input itself)
        self.out_shape = out_shape
        self.n_out = n_out
        self.kv = kv
        self.lin_is_int32 = lin_is_int32


def key_is_int32(batch_size, spatial_shape, out_shape, subm) -> bool:
    """pairs.py:166-171: int32 keys iff batch*volume < 2**31."""
    max_lin = batch_size * int(np.prod(out_shape))
    if subm:
        max_lin = max(max_lin, batch_size * int(np.prod(spatial_shape)))
    return max_lin < 2 ** 31


def compute_candidates(indices, batch_size, spatial_shape, ksize, stride, padding,
                       dilation, out_padding, subm, transpose) -> Candidates:
    indices = np.ascontiguousarray(np.asarray(indices, dtype=np.int32))
    ndim = len(spatial_shape)
    N = indices.shape[0]
    kv = int(np.prod(ksize))
    if N == 0:
        raise ValueError("N > 0 assert: sparse tensor has no points")
    if any(k <= 0 for k in ksize):
        raise ValueError(f"kernel size {ksize} not supported by pair gen")
    if subm:
        if any(k % 2 == 0 for k in ksize):
            raise NotImplementedError("subm convolution requires odd kernel sizes")
        out_shape = list(spatial_shape)
    elif transpose:
        out_shape = get_deconv_output_size(spatial_shape, ksize, stride, padding, dilation, out_padding)
    else:
        out_shape = get_conv_output_size(spatial_shape, ksize, stride, padding, dilation)
    if any(x <= 0 for x in out_shape):
        raise ValueError(f"your out spatial shape {out_shape} reach zero!!! input shape: {spatial_shape}")
    i32 = key_is_int32(batch_size, spatial_shape, out_shape, subm)
    if subm:
        pad = [(ksize[i] // 2) * dilation[i] for i in range(ndim)]
        st = [1] * ndim
    else:
        pad = list(padding)
        st = list(stride)
    strided = any(int(s) != 1 for s in st)
    out_lin = np.empty(kv * N, dtype=np.int64)
    valid = np.empty(kv * N, dtype=np.uint8)
    L = lib()
    a_ks, a_pad, a_st, a_dil, a_os, a_ss = (_i64(ksize), _i64(pad), _i64(st), _i64(dilation),
                                            _i64(out_shape), _i64(spatial_shape))
    L.orc_candidates(_p(indices), ctypes.c_int64(N), ctypes.c_int(ndim), _p(a_ks),
                     _p(a_pad), _p(a_st), _p(a_dil), _p(a_os),
                     ctypes.c_int(int(bool(transpose) and not subm)), ctypes.c_int(int(strided)),
                     _p(out_lin), _p(valid))
    out_row = np.empty(kv * N, dtype=np.int32)
    if subm:
        in_lin = np.empty(N, dtype=np.int64)
        L.orc_linearize(_p(indices), ctypes.c_int64(N), ctypes.c_int(ndim), _p(a_ss), _p(in_lin))
        L.orc_subm_membership(_p(out_lin), _p(valid), ctypes.c_int64(kv), ctypes.c_int64(N), _p(in_lin), _p(out_row))
        return Candidates(valid.reshape(kv, N).astype(bool), out_row.reshape(kv, N), None,
                          out_shape, N, kv, i32)
    uniq = np.empty(kv * N, dtype=np.int64)
    n_out = int(L.orc_unique_sorted(_p(out_lin), _p(valid), ctypes.c_int64(kv * N), _p(uniq)))
    if n_out == 0:
        raise ValueError(_POINT_VANISH_MSG.format(spatial_shape, ksize, stride, padding, dilation))
    uniq = np.ascontiguousarray(uniq[:n_out])
    L.orc_lower_bound_rows(_p(out_lin), _p(valid), ctypes.c_int64(kv * N), _p(uniq), ctypes.c_int64(n_out), _p(out_row))
    out_inds = np.empty((n_out, ndim + 1), dtype=np.int32)
    L.orc_delinearize(_p(uniq), ctypes.c_int64(n_out), ctypes.c_int(ndim), _p(a_os), _p(out_inds))
    return Candidates(valid.reshape(kv, N).astype(bool), out_row.reshape(kv, N), out_inds,
                      out_shape, n_out, kv, i32)


# ---------------------------------------------------------------------------
# masks (pairs.py:344-392)
# ---------------------------------------------------------------------------

def split_masks(kv: int, is_mask_split: bool):
    if is_mask_split:
        kv_div_2 = kv // 2
        remain = kv - kv_div_2
        one = np.array([1], dtype=np.uint64)
        first = (one << np.uint64(remain)) - np.uint64(1)
        second = ((one << np.uint64(kv_div_2)) - np.uint64(1)) << np.uint64(remain)
        return [first.astype(np.uint32), second.astype(np.uint32)]
    return [np.array([0xFFFFFFFF], dtype=np.uint32)]


def mask_splits(pair_table: np.ndarray, masks, do_sort=True):
    kv, n = pair_table.shape
    mic = (kv + 31) // 32
    pair_table = np.ascontiguousarray(pair_table, dtype=np.int32)
    pms, args = [], []
    for m in masks:
        mval = int(m.astype(np.int64)[0])
        pm = np.empty((n, mic), dtype=np.int32)
        ar = np.empty(n, dtype=np.int32)
        lib().orc_mask_split(_p(pair_table), ctypes.c_int64(kv), ctypes.c_int64(n), ctypes.c_int64(mic),
                             ctypes.c_int64(mval), ctypes.c_int(int(bool(do_sort))), _p(pm), _p(ar))
        pms.append(pm)
        args.append(ar)
    return pms, args


# ---------------------------------------------------------------------------
# implicit-gemm / native formats
# ---------------------------------------------------------------------------

def igemm_pairs(indices, batch_size, spatial_shape, ksize, stride, padding, dilation,
                out_padding, subm, transpose, is_train, is_mask_split=False, do_sort=True,
                num_out_act_bound=-1):
    """Restates pairs.py:281-426; returns the same 9-tuple layout (numpy)."""
    indices = np.ascontiguousarray(np.asarray(indices, dtype=np.int32))
    N = indices.shape[0]
    cand = compute_candidates(indices, batch_size, spatial_shape, ksize, stride, padding,
                              dilation, out_padding, subm, transpose)
    kv = cand.kv
    if is_mask_split and kv > 32:
        raise AssertionError("Not Implemented")
    n_out = cand.n_out
    out_inds = cand.out_inds
    if not subm and num_out_act_bound > 0 and n_out > num_out_act_bound:
        n_out = num_out_act_bound
        out_inds = out_inds[:n_out]
    pair_fwd = np.empty((kv, n_out), dtype=np.int32)
    pair_bwd = np.empty((kv, N), dtype=np.int32)
    valid_u8 = np.ascontiguousarray(cand.valid.astype(np.uint8))
    out_row = np.ascontiguousarray(cand.out_row)
    lib().orc_scatter_igemm(_p(valid_u8), _p(out_row), ctypes.c_int64(kv),
                            ctypes.c_int64(N), ctypes.c_int64(n_out), _p(pair_fwd), _p(pair_bwd))
    npl = np.zeros(kv, dtype=np.int32)
    masks = split_masks(kv, is_mask_split)
    pm_fwd, ma_fwd = mask_splits(pair_fwd, masks, do_sort)
    if is_train and not subm:
        pm_bwd, ma_bwd = mask_splits(pair_bwd, masks, do_sort)
    else:
        pm_bwd, ma_bwd = [], []
    pb = pair_bwd if is_train else None
    if subm:
        return (indices, npl, pair_fwd, pb, pm_fwd, [], ma_fwd, [], masks)
    return (out_inds, npl, pair_fwd, pb, pm_fwd, pm_bwd, ma_fwd, ma_bwd, masks)


def native_pairs(indices, batch_size, spatial_shape, ksize, stride, padding, dilation,
                 out_padding, subm, transpose):
    """Restates pairs.py:242-278; returns (out_inds, pair[2,kv,N], npl)."""
    indices = np.ascontiguousarray(np.asarray(indices, dtype=np.int32))
    N = indices.shape[0]
    cand = compute_candidates(indices, batch_size, spatial_shape, ksize, stride, padding,
                              dilation, out_padding, subm, transpose)
    kv = cand.kv
    pair = np.empty((2, kv, N), dtype=np.int32)
    counts = np.empty(kv, dtype=np.int32)
    valid_u8 = np.ascontiguousarray(cand.valid.astype(np.uint8))
    out_row = np.ascontiguousarray(cand.out_row)
    lib().orc_native(_p(valid_u8), _p(out_row), ctypes.c_int64(kv), ctypes.c_int64(N),
                     _p(pair), _p(counts))
    if subm:
        center = kv // 2
        npl = np.where(np.arange(kv) < center, counts, 0).astype(np.int32)
        out_inds = indices
    else:
        npl = counts.astype(np.int32)
        out_inds = cand.out_inds
    return out_inds, pair, npl


def native_pair_to_tables(pair, n_in, n_out, inverse, need_bwd=True):
    pair = np.ascontiguousarray(pair, dtype=np.int32)
    kv, N = pair.shape[1], pair.shape[2]
    pf = np.empty((kv, n_out), dtype=np.int32)
    pb = np.empty((kv, n_in), dtype=np.int32) if need_bwd else None
    lib().orc_native_to_tables(_p(pair), ctypes.c_int64(kv), ctypes.c_int64(N), ctypes.c_int64(n_in),
                               ctypes.c_int64(n_out), ctypes.c_int(int(bool(inverse))), _p(pf), _p(pb))
    return pf, pb


# ---------------------------------------------------------------------------
# GEMM contract (fp64)
# ---------------------------------------------------------------------------

def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def gemm_fwd(X, W_krsc, pf, bias=None) -> np.ndarray:
    """out[m,n] = bias[n] + sum_k sum_c X[pf[k,m],c] * W[n,k,c]  (W: [K, kv, C])."""
    X = _f64(X)
    W = _f64(W_krsc)
    K, kv, C = W.shape
    pf = np.ascontiguousarray(pf, dtype=np.int32)
    n_out = pf.shape[1]
    out = np.empty((n_out, K), dtype=np.float64)
    b = _f64(bias) if bias is not None else None
    lib().orc_gemm_fwd(_p(X), ctypes.c_int64(C), _p(W), ctypes.c_int64(K), ctypes.c_int64(kv),
                       _p(pf), ctypes.c_int64(n_out), _p(b), _p(out))
    return out


def gemm_fwd_f32(X, W_krsc, pf, bias=None) -> np.ndarray:
    X = np.ascontiguousarray(X, dtype=np.float32)
    W = np.ascontiguousarray(W_krsc, dtype=np.float32)
    K, kv, C = W.shape
    pf = np.ascontiguousarray(pf, dtype=np.int32)
    n_out = pf.shape[1]
    out = np.empty((n_out, K), dtype=np.float32)
    b = np.ascontiguousarray(bias, dtype=np.float32) if bias is not None else None
    lib().orc_gemm_fwd_f32(_p(X), ctypes.c_int64(C), _p(W), ctypes.c_int64(K), ctypes.c_int64(kv),
                           _p(pf), ctypes.c_int64(n_out), _p(b), _p(out))
    return out


def gemm_dgrad(G, W_krsc, pb) -> np.ndarray:
    G = _f64(G)
    W = _f64(W_krsc)
    K, kv, C = W.shape
    pb = np.ascontiguousarray(pb, dtype=np.int32)
    n_in = pb.shape[1]
    out = np.empty((n_in, C), dtype=np.float64)
    lib().orc_gemm_dgrad(_p(G), ctypes.c_int64(K), _p(W), ctypes.c_int64(kv), ctypes.c_int64(C),
                         _p(pb), ctypes.c_int64(n_in), _p(out))
    return out


def gemm_wgrad(X, G, pf, K, C) -> np.ndarray:
    X = _f64(X)
    G = _f64(G)
    pf = np.ascontiguousarray(pf, dtype=np.int32)
    kv, n_out = pf.shape
    dW = np.empty((K, kv, C), dtype=np.float64)
    lib().orc_gemm_wgrad(_p(X), ctypes.c_int64(C), _p(G), ctypes.c_int64(K), ctypes.c_int64(kv),
                         _p(pf), ctypes.c_int64(n_out), _p(dW))
    return dW


# ---------------------------------------------------------------------------
# pooling (accumulator fp32 for fp16/fp32 inputs, fp64 for fp64 inputs)
# ---------------------------------------------------------------------------

def _pool_args(dtype):
    if np.dtype(dtype) == np.float64:
        return np.float64, "f64"
    return np.float32, "f32"


def maxpool_fwd(X, pf):
    X = np.asarray(X)
    ft, suf = _pool_args(X.dtype)
    Xw = np.ascontiguousarray(X.astype(ft))
    pf = np.ascontiguousarray(pf, dtype=np.int32)
    kv, n_out = pf.shape
    C = Xw.shape[1]
    out = np.empty((n_out, C), dtype=ft)
    getattr(lib(), f"orc_maxpool_fwd_{suf}")(_p(Xw), ctypes.c_int64(C), _p(pf), ctypes.c_int64(kv),
                                             ctypes.c_int64(n_out), _p(out))
    return out.astype(X.dtype)


def maxpool_bwd(X, OUT, G, pb):
    X = np.asarray(X)
    ft, suf = _pool_args(X.dtype)
    Xw = np.ascontiguousarray(X.astype(ft))
    Ow = np.ascontiguousarray(np.asarray(OUT).astype(ft))
    Gw = np.ascontiguousarray(np.asarray(G).astype(ft))
    pb = np.ascontiguousarray(pb, dtype=np.int32)
    kv, n_in = pb.shape
    C = Xw.shape[1]
    dX = np.empty((n_in, C), dtype=ft)
    getattr(lib(), f"orc_maxpool_bwd_{suf}")(_p(Xw), _p(Ow), _p(Gw), ctypes.c_int64(C), _p(pb),
                                             ctypes.c_int64(kv), ctypes.c_int64(n_in), _p(dX))
    return dX.astype(X.dtype)


def avgpool_fwd(X, pf):
    X = np.asarray(X)
    ft, suf = _pool_args(X.dtype)
    Xw = np.ascontiguousarray(X.astype(ft))
    pf = np.ascontiguousarray(pf, dtype=np.int32)
    kv, n_out = pf.shape
    C = Xw.shape[1]
    out = np.empty((n_out, C), dtype=ft)
    count = np.empty(n_out, dtype=np.int32)
    getattr(lib(), f"orc_avgpool_fwd_{suf}")(_p(Xw), ctypes.c_int64(C), _p(pf), ctypes.c_int64(kv),
                                             ctypes.c_int64(n_out), _p(out), _p(count))
    return out.astype(X.dtype), count


def avgpool_bwd(G, count, pb):
    G = np.asarray(G)
    ft, suf = _pool_args(G.dtype)
    Gw = np.ascontiguousarray(G.astype(ft))
    count = np.ascontiguousarray(count, dtype=np.int32)
    pb = np.ascontiguousarray(pb, dtype=np.int32)
    kv, n_in = pb.shape
    C = Gw.shape[1]
    dX = np.empty((n_in, C), dtype=ft)
    getattr(lib(), f"orc_avgpool_bwd_{suf}")(_p(Gw), _p(count), ctypes.c_int64(C), _p(pb),
                                             ctypes.c_int64(kv), ctypes.c_int64(n_in), _p(dX))
    return dX.astype(G.dtype)


def point_to_voxel(points, vsize_xyz, coors_range_xyz, num_point_features, max_num_voxels,
                   max_num_points_per_voxel, empty_mean=False):
    """First-come-first-served voxelisation (reference utils.py:16-163), in
    numpy.  Quantisation is floor((p - cmin) / vsize) in the points' dtype;
    voxels are numbered by their first point, capped at max_num_voxels; a
    voxel stores up to max_num_points_per_voxel points in point order.
    Returns (voxels [nv, maxpts, F] f32 with zeros in empty slots -- or the
    voxel's mean with empty_mean --, indices [nv, ndim] int32 ZYX,
    num_per_voxel [nv] int32, pc_voxel_id [n] int64)."""
    pts = np.asarray(points)
    ndim = len(vsize_xyz)
    n = pts.shape[0]
    cmin = np.asarray(coors_range_xyz[:ndim], dtype=pts.dtype)
    vsize = np.asarray(vsize_xyz, dtype=pts.dtype)
    grid = [round((coors_range_xyz[ndim + i] - coors_range_xyz[i]) / vsize_xyz[i])
            for i in range(ndim)]
    with np.errstate(invalid="ignore"):
        q = np.floor((pts[:, :ndim] - cmin) / vsize)
        in_range = ((q >= 0) & (q < np.asarray(grid, dtype=pts.dtype))).all(1)
    pc_voxel_id = np.full(n, -1, dtype=np.int64)
    maxpts = max_num_points_per_voxel
    empty = (np.zeros((0, maxpts, num_point_features), np.float32), np.zeros((0, ndim), np.int32),
             np.zeros(0, np.int32), pc_voxel_id)
    valid = np.nonzero(in_range)[0]
    if valid.size == 0:
        return empty
    qv = q[valid].astype(np.int64)
    lin = qv[:, 0].copy()
    for d in range(1, ndim):
        lin = lin * grid[d] + qv[:, d]
    uniq, first, inverse = np.unique(lin, return_index=True, return_inverse=True)
    order = np.argsort(first, kind="stable")          # voxels by first occurrence
    vid_of_uniq = np.empty_like(order)
    vid_of_uniq[order] = np.arange(uniq.size)
    vid = vid_of_uniq[inverse.reshape(-1)]
    nv = min(uniq.size, max_num_voxels)
    kept = vid < nv
    counts = np.bincount(vid[kept], minlength=nv)
    npv = np.minimum(counts, maxpts).astype(np.int32)
    rem = uniq[order][:nv]
    coords = np.empty((nv, ndim), np.int64)
    for d in range(ndim - 1, -1, -1):
        coords[:, d] = rem % grid[d]
        rem = rem // grid[d]
    voxels = np.zeros((nv, maxpts, num_point_features), np.float32)
    slot = np.zeros(nv, np.int64)
    for i, v in zip(valid[kept], vid[kept]):          # point order: arrival order per voxel
        if slot[v] < maxpts:
            voxels[v, slot[v]] = pts[i, :num_point_features].astype(np.float32)
        slot[v] += 1
    pc_voxel_id[valid[kept]] = vid[kept]
    if empty_mean:
        sums = voxels.sum(axis=1, dtype=np.float32)
        means = sums / np.maximum(npv, 1)[:, None].astype(np.float32)
        for v in range(nv):
            voxels[v, npv[v]:] = means[v]
    return voxels, coords[:, ::-1].astype(np.int32), npv, pc_voxel_id


def hash_sparse_add(indices_list, features_list, shape):
    """Union of coordinates in ascending batch-major key order, features of
    equal coordinates summed in input order (reference functional.py:429-490
    with its sorted-array HashTable, hash.py:38-98)."""
    keys = []
    for ind in indices_list:
        ind = np.asarray(ind, dtype=np.int64)
        k = ind[:, 0].copy()
        for d in range(1, ind.shape[1]):
            k = k * int(shape[d]) + ind[:, d]
        keys.append(k)
    uniq = np.unique(np.concatenate(keys))
    C = np.asarray(features_list[0]).shape[1]
    feats = np.zeros((uniq.size, C), dtype=np.asarray(features_list[0]).dtype)
    out_ind = np.zeros((uniq.size, np.asarray(indices_list[0]).shape[1]), np.int32)
    for k, ind, f in zip(keys, indices_list, features_list):
        rows = np.searchsorted(uniq, k)
        feats[rows] += np.asarray(f)
        out_ind[rows] = ind
    return out_ind, feats


if os.environ.get("SPCONV_ORACLE_THREADS"):
    set_num_threads(int(os.environ["SPCONV_ORACLE_THREADS"]))
