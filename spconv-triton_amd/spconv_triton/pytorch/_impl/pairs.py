"""Rulebook (index-pair) generation on the GPU through ``libspconv_hip.so``.

Host-side mirror of ``spconv_triton/pytorch/_impl/pairs.py`` of the reference:
same functions, same argument meaning, same outputs and error types.  The
device work is the library's coordinate-hash pair generator (see
``csrc/sp_pairgen.hip``); results equal the reference's sort/binary-search
construction bit for bit:

* offsets enumerated row-major, last dim fastest, no kernel flip
  (reference ``pairs.py:6-22``, ``:43-48``);
* subm outputs are the input rows and ``indices`` is returned as is
  (``pairs.py:400-401``);
* regular/transpose outputs are the unique candidate keys, ascending
  batch-major (``pairs.py:206-219``);
* Native ``[2, kv, N]`` lists are per offset, ascending input row
  (``pairs.py:223-239``); subm ``indice_num_per_loc`` is zero for
  ``k >= kv // 2`` (``pairs.py:269-275``);
* igemm masks are stably sorted unsigned words (``pairs.py:356-392``).
"""

from __future__ import annotations

import ctypes
import functools

import numpy as np
import torch

from . import _lib

_POINT_VANISH_MSG = (
    "Your points vanished here, this usually happens when you provide "
    "conv params that may ignore some input points. Example: "
    "spatial_shape={}, ksize={}, stride={}, padding={}, dilation={}"
)


def _prod(vals) -> int:
    return functools.reduce(lambda a, b: a * int(b), vals, 1)


def get_conv_output_size(input_size, kernel_size, stride, padding, dilation):
    """Reference ``pairs.py:59-72``."""
    out = []
    for i in range(len(input_size)):
        if kernel_size[i] == -1:
            out.append(1)
            continue
        span = dilation[i] * (kernel_size[i] - 1) + 1
        out.append((input_size[i] + 2 * padding[i] - span) // stride[i] + 1)
    return out


def get_deconv_output_size(input_size, kernel_size, stride, padding, dilation, output_padding):
    """Reference ``pairs.py:75-88`` (dilation does not enter the formula)."""
    out = []
    for i in range(len(input_size)):
        if kernel_size[i] == -1:
            raise ValueError("deconv don't support kernel_size < 0")
        out.append((input_size[i] - 1) * stride[i] - 2 * padding[i] + kernel_size[i]
                   + output_padding[i])
    return out


def _check_and_shape(indices, spatial_shape, ksize, stride, padding, dilation, out_padding,
                     subm, transpose):
    """Validation and output shape, in the order of reference ``pairs.py:137-164``."""
    if indices.shape[0] == 0:
        raise ValueError("N > 0 assert: sparse tensor has no points")
    if any(k <= 0 for k in ksize):
        raise ValueError(f"kernel size {ksize} not supported by pair gen")
    if subm:
        if any(k % 2 == 0 for k in ksize):
            raise NotImplementedError("subm convolution requires odd kernel sizes")
        out_shape = list(spatial_shape)
    elif transpose:
        out_shape = get_deconv_output_size(spatial_shape, ksize, stride, padding, dilation,
                                           out_padding)
    else:
        out_shape = get_conv_output_size(spatial_shape, ksize, stride, padding, dilation)
    if any(x <= 0 for x in out_shape):
        raise ValueError(f"your out spatial shape {out_shape} reach zero!!! "
                         f"input shape: {spatial_shape}")
    return [int(x) for x in out_shape]


def _prepare_indices(indices: torch.Tensor) -> torch.Tensor:
    _lib.require_gpu(indices)
    idx = indices if indices.dtype == torch.int32 else indices.to(torch.int32)
    return idx.contiguous()


def _geom(subm, transpose, batch_size, spatial_shape, out_shape, ksize, stride, padding,
          dilation):
    mode = _lib.SP_PAIR_SUBM if subm else (_lib.SP_PAIR_TRANSPOSE if transpose
                                           else _lib.SP_PAIR_REGULAR)
    ndim = len(spatial_shape)
    st = list(stride) if not subm else [1] * ndim
    pad = list(padding) if not subm else [0] * ndim
    return _lib.make_geom(mode, batch_size, spatial_shape, out_shape, ksize, st, pad, dilation)


def key_is_int64(batch_size, spatial_shape, out_shape, subm) -> bool:
    """int64 linear keys iff batch * volume >= 2^31 (reference ``pairs.py:166-171``)."""
    max_lin = batch_size * _prod(out_shape)
    if subm:
        max_lin = max(max_lin, batch_size * _prod(spatial_shape))
    return max_lin >= 2 ** 31


class _Tables:
    """Raw tables produced by one pair-generation run."""

    def __init__(self, out_inds, pair_fwd, pair_bwd, words_fwd, words_bwd, n_out, npl=None):
        self.out_inds = out_inds
        self.pair_fwd = pair_fwd
        self.pair_bwd = pair_bwd
        self.words_fwd = words_fwd
        self.words_bwd = words_bwd
        self.n_out = n_out
        self.npl = npl  # zeroed indice_num_per_loc, when the build wrote it


#: Dense cell -> row grids kept between subm builds, one per (device, stream):
#: (grid, epoch of its last build).  A grid is zero-filled when created and
#: every 255 builds; in between, each build stamps its cells with a new epoch
#: (``sp_pairgen_subm_grid``), so no build clears it.  Only grids of at most
#: KEEP_GRID_MAX_CELLS int32 cells are kept (a 256^3 volume plus its guard
#: cells, 64 MiB); a build needing a larger one takes a per-build workspace,
#: which the caching allocator can release.  ``release_pairgen_grids()`` drops
#: the kept grids (a grid kept for a stream no longer in use stays until then).
_GRIDS: dict = {}
KEEP_GRID_MAX_CELLS = (1 << 24) + 1024


def _subm_grid(device: torch.device, cells: int):
    """(grid, epoch) for the next subm build on the current stream of ``device``."""
    stream = torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream)
    grid, epoch = _GRIDS.get(key, (None, 255))
    if grid is None or grid.numel() < cells:
        grid = torch.empty((cells,), dtype=torch.int32, device=device)
        epoch = 255
    if epoch >= 255:
        grid.zero_()
        epoch = 0
    epoch += 1
    _GRIDS[key] = (grid, epoch)
    return grid, epoch


def release_pairgen_grids() -> None:
    """Drop the kept subm lookup grids (the next build allocates again)."""
    _GRIDS.clear()


def _attach_coords(table, coords, shape, batch) -> None:
    """Keep the coordinates of a gather table's rows on the table (rows of
    ``coords`` [M, ndim+1] int32 in ``shape``, ``batch`` samples): the GEMM
    may reorder rows by their linear key (``gemm.key_order_variant``)."""
    if table is not None and table.numel() > 0 and coords is not None:
        table._spconv_triton_rowcoords = (coords, tuple(int(v) for v in shape), int(batch))


def _generate(indices, batch_size, spatial_shape, ksize, stride, padding, dilation, out_padding,
              subm, transpose, want_fwd, want_bwd, want_words_fwd, want_words_bwd,
              num_out_act_bound=-1) -> _Tables:
    out_shape = _check_and_shape(indices, spatial_shape, ksize, stride, padding, dilation,
                                 out_padding, subm, transpose)
    idx = _prepare_indices(indices)
    device = idx.device
    N = idx.shape[0]
    kv = _prod(ksize)
    mic = (kv + 31) // 32
    g = _geom(subm, transpose, batch_size, spatial_shape, out_shape, ksize, stride, padding,
              dilation)
    L = _lib.lib()
    stream = _lib.stream_of(device)
    i32 = dict(dtype=torch.int32, device=device)
    if subm:
        pf = torch.empty((kv, N), **i32) if want_fwd else None
        pb = torch.empty((kv, N), **i32) if want_bwd else None
        words = torch.empty((N, mic), **i32) if want_words_fwd else None
        cells = L.sp_pairgen_subm_grid_cells(g, N)
        if (0 < cells <= KEEP_GRID_MAX_CELLS
                and not torch.cuda.is_current_stream_capturing()):
            # a grid kept between builds (a graph replays its kernels with the
            # epoch it was captured with, so captured builds clear their own)
            grid, epoch = _subm_grid(device, cells)
            npl = torch.empty((kv,), **i32)
            _lib.check(L.sp_pairgen_subm_grid(g, _lib.ptr(idx), N, _lib.ptr(pf), _lib.ptr(pb),
                                              _lib.ptr(words), _lib.ptr(npl), _lib.ptr(grid),
                                              grid.numel(), epoch, stream),
                       "sp_pairgen_subm_grid")
        else:
            npl = None
            ws = _lib.workspace(L.sp_pairgen_workspace_size(g, N), device)
            _lib.check(L.sp_pairgen_subm(g, _lib.ptr(idx), N, _lib.ptr(pf), _lib.ptr(pb),
                                         _lib.ptr(words), _lib.ptr(ws), ws.numel(), stream),
                       "sp_pairgen_subm")
        _attach_coords(pf, idx, spatial_shape, batch_size)
        _attach_coords(pb, idx, spatial_shape, batch_size)
        return _Tables(indices, pf, pb, words, None, N, npl)
    ws = _lib.workspace(L.sp_pairgen_workspace_size(g, N), device)
    n_out = ctypes.c_int64(0)
    n_pairs = ctypes.c_int64(0)
    _lib.check(L.sp_pairgen_conv_build(g, _lib.ptr(idx), N, _lib.ptr(ws), ws.numel(), n_out,
                                       n_pairs, stream), "sp_pairgen_conv_build")
    n_out = int(n_out.value)
    if n_out == 0:
        raise ValueError(_POINT_VANISH_MSG.format(spatial_shape, ksize, stride, padding, dilation))
    if num_out_act_bound > 0 and n_out > num_out_act_bound:
        # igemm-only bound: keep the first outputs in canonical order and drop
        # candidates that map beyond them (reference pairs.py:318-323)
        n_out = int(num_out_act_bound)
    out_inds = torch.empty((n_out, len(spatial_shape) + 1), **i32)
    pf = torch.empty((kv, n_out), **i32) if want_fwd else None
    pb = torch.empty((kv, N), **i32) if want_bwd else None
    words_bwd = torch.empty((N, mic), **i32) if want_words_bwd else None
    _lib.check(L.sp_pairgen_conv_fill(g, _lib.ptr(idx), N, _lib.ptr(ws), ws.numel(), n_out,
                                      _lib.ptr(out_inds), _lib.ptr(pf), _lib.ptr(pb),
                                      _lib.ptr(words_bwd), stream), "sp_pairgen_conv_fill")
    words_fwd = None
    if want_words_fwd:
        words_fwd = mask_words(pf)
    for table in (pf, pb):
        if table is not None:
            # the tables' valid entries, known without a further
            # synchronisation: the GEMM's row-order decision reads them
            # (gemm.row_order_variant)
            table._spconv_triton_npairs = int(n_pairs.value)
    _attach_coords(pf, out_inds, out_shape, batch_size)
    _attach_coords(pb, idx, spatial_shape, batch_size)
    return _Tables(out_inds, pf, pb, words_fwd, words_bwd, n_out)


def mask_words(table: torch.Tensor) -> torch.Tensor:
    """Per-row bitmask words of a gather table [kv, n] (reference pair_kernels.py:147-213)."""
    kv, n = table.shape
    words = torch.empty((n, (kv + 31) // 32), dtype=torch.int32, device=table.device)
    _lib.check(_lib.lib().sp_mask_words(_lib.ptr(table.contiguous()), kv, n, _lib.ptr(words),
                                        _lib.stream_of(table.device)), "sp_mask_words")
    return words


def split_masks(kv: int, is_mask_split: bool):
    """Reference ``pairs.py:344-354``: uint32 numpy masks."""
    if is_mask_split:
        half = kv // 2
        remain = kv - half
        one = np.array([1], dtype=np.uint64)
        first = (one << np.uint64(remain)) - np.uint64(1)
        second = ((one << np.uint64(half)) - np.uint64(1)) << np.uint64(remain)
        return [first.astype(np.uint32), second.astype(np.uint32)]
    return [np.array([0xFFFFFFFF], dtype=np.uint32)]


def sort_mask_words(words: torch.Tensor, kv: int, masks, do_sort: bool = True):
    """Mask splits of one table (reference ``make_mask_splits``, ``pairs.py:356-392``)."""
    n, mic = words.shape
    device = words.device
    L = _lib.lib()
    stream = _lib.stream_of(device)
    ws = _lib.workspace(L.sp_mask_sort_workspace_size(n, mic) if do_sort else 1, device)
    pm_splits, arg_splits = [], []
    for m in masks:
        mval = int(m.astype(np.int64)[0]) & 0xFFFFFFFF
        pm = torch.empty((n, mic), dtype=torch.int32, device=device)
        args = torch.empty((n,), dtype=torch.int32, device=device)
        _lib.check(L.sp_mask_sort(_lib.ptr(words), n, mic, kv, mval, int(bool(do_sort)),
                                  _lib.ptr(pm), _lib.ptr(args), _lib.ptr(ws), ws.numel(), stream),
                   "sp_mask_sort")
        pm_splits.append(pm)
        arg_splits.append(args)
    return pm_splits, arg_splits


def native_pairs(indices, batch_size, spatial_shape, ksize, stride, padding, dilation,
                 out_padding, subm, transpose):
    """Native-format pairs (reference ``pairs.py:242-278``): (out_inds, pair[2,kv,N], npl)."""
    t = _generate(indices, batch_size, spatial_shape, ksize, stride, padding, dilation,
                  out_padding, subm, transpose, want_fwd=False, want_bwd=True,
                  want_words_fwd=False, want_words_bwd=False)
    pb = t.pair_bwd
    kv, N = pb.shape
    device = pb.device
    pair = torch.empty((2, kv, N), dtype=torch.int32, device=device)
    npl = torch.empty((kv,), dtype=torch.int32, device=device)
    L = _lib.lib()
    ws = _lib.workspace(L.sp_compact_workspace_size(kv, N), device)
    _lib.check(L.sp_compact_table(_lib.ptr(pb), kv, N, _lib.ptr(pair[0]), _lib.ptr(pair[1]), None,
                                  _lib.ptr(npl), (kv // 2) if subm else kv, _lib.ptr(ws),
                                  ws.numel(), _lib.stream_of(device)), "sp_compact_table")
    out_shape = _check_and_shape(indices, spatial_shape, ksize, stride, padding, dilation,
                                 out_padding, subm, transpose)
    pair._spconv_triton_rowcoords = {
        "in": (_prepare_indices(indices), tuple(spatial_shape), int(batch_size)),
        "out": (t.out_inds if not subm else _prepare_indices(indices), tuple(out_shape),
                int(batch_size))}
    return t.out_inds, pair, npl


class DeferredMaskSplits:
    """The sorted mask splits of one implicit-GEMM rulebook, computed on first use.

    The gather-GEMM skips the offsets a tile has no pair for by itself and never
    reads the masks, so a rulebook that a module builds for its own use keeps
    only what the masks are made from: the mask words where pair generation
    wrote them in passing (subm forward, regular/transposed backward), else the
    gather table.  ``get()`` runs the sorts the first time the values are asked
    for and returns what the eager ``igemm_pairs`` returns.
    """

    def __init__(self, words_fwd: torch.Tensor | None, pair_fwd: torch.Tensor,
                 words_bwd: torch.Tensor | None, kv: int, masks, do_sort: bool):
        self._args = (words_fwd, pair_fwd, words_bwd, kv, masks, do_sort)
        self._stream = torch.cuda.current_stream(pair_fwd.device)
        self._value = None

    def __getstate__(self):
        # pickles and deep copies hold the computed splits: a stream and the
        # pending arguments are not copyable (torch.cuda.Stream does not pickle)
        return {"_value": self.get()}

    def __setstate__(self, state):
        self._args, self._stream = None, None
        self._value = state["_value"]

    def get(self):
        """(pair_mask_fwd_splits, pair_mask_bwd_splits, mask_argsort_fwd_splits,
        mask_argsort_bwd_splits)."""
        if self._value is None:
            words_fwd, pair_fwd, words_bwd, kv, masks, do_sort = self._args
            cur = torch.cuda.current_stream(pair_fwd.device)
            if cur != self._stream:
                # the words and the table were written on the build stream
                cur.wait_stream(self._stream)
                for w in (words_fwd, words_bwd):
                    if w is not None:
                        w.record_stream(cur)
            if words_fwd is None:
                words_fwd = mask_words(pair_fwd)
            pm_fwd, ma_fwd = sort_mask_words(words_fwd, kv, masks, do_sort)
            if words_bwd is not None:
                pm_bwd, ma_bwd = sort_mask_words(words_bwd, kv, masks, do_sort)
            else:
                pm_bwd, ma_bwd = [], []
            self._value = (pm_fwd, pm_bwd, ma_fwd, ma_bwd)
            self._args = None
        return self._value


def igemm_rulebook(indices, batch_size, spatial_shape, ksize, stride, padding, dilation,
                   out_padding, subm, transpose, is_train, is_mask_split, do_sort=True,
                   num_out_act_bound=-1):
    """``igemm_pairs`` with the mask sorts deferred: returns (the 9-tuple with
    empty mask-split lists, a ``DeferredMaskSplits`` that yields them)."""
    kv = _prod(ksize)
    need_bwd = bool(is_train)
    bound = num_out_act_bound if not subm else -1
    if is_mask_split and kv > 32:
        # the reference validates the geometry first, then rejects the split
        _check_and_shape(indices, spatial_shape, ksize, stride, padding, dilation, out_padding,
                         subm, transpose)
        raise AssertionError("Not Implemented")
    t = _generate(indices, batch_size, spatial_shape, ksize, stride, padding, dilation,
                  out_padding, subm, transpose, want_fwd=True, want_bwd=need_bwd,
                  want_words_fwd=subm, want_words_bwd=need_bwd and not subm,
                  num_out_act_bound=bound)
    device = t.pair_fwd.device
    npl = t.npl if t.npl is not None else torch.zeros((kv,), dtype=torch.int32, device=device)
    masks = split_masks(kv, is_mask_split)
    # t.words_bwd exists for a regular/transposed training rulebook only
    deferred = DeferredMaskSplits(t.words_fwd, t.pair_fwd, t.words_bwd, kv, masks, do_sort)
    pb = t.pair_bwd if need_bwd else torch.Tensor()
    if subm:
        return (indices, npl, t.pair_fwd, pb, [], [], [], [], masks), deferred
    return (t.out_inds, npl, t.pair_fwd, pb, [], [], [], [], masks), deferred


def igemm_pairs(indices, batch_size, spatial_shape, ksize, stride, padding, dilation,
                out_padding, subm, transpose, is_train, is_mask_split, do_sort=True,
                num_out_act_bound=-1):
    """Implicit-GEMM tables (reference ``pairs.py:281-426``), the same 9-tuple."""
    res, deferred = igemm_rulebook(indices, batch_size, spatial_shape, ksize, stride, padding,
                                   dilation, out_padding, subm, transpose, is_train,
                                   is_mask_split, do_sort, num_out_act_bound)
    pm_fwd, pm_bwd, ma_fwd, ma_bwd = deferred.get()
    return res[:4] + (pm_fwd, pm_bwd, ma_fwd, ma_bwd) + res[8:]


def native_pair_to_tables(pair: torch.Tensor, indice_pair_num, n_in: int, n_out: int,
                          inverse: bool, need_bwd: bool = True):
    """Native pairs -> gather tables (reference ``pairs.py:429-469``).

    Memoised on the pair tensor keyed by (n_in, n_out, inverse); each table is
    built at most once.  ``indice_pair_num`` is accepted and ignored (validity
    is read from the -1 fill of the pair tensor)."""
    key = (int(n_in), int(n_out), bool(inverse))
    cache = getattr(pair, "_spconv_triton_tables", None)
    if cache is None:
        cache = {}
        pair._spconv_triton_tables = cache
    pf, pb = cache.get(key, (None, None))
    if pf is None or (need_bwd and pb is None):
        _lib.require_gpu(pair)
        pc = pair.contiguous()
        kv, n_pairs = pc.shape[1], pc.shape[2]
        device = pc.device
        pf = torch.empty((kv, int(n_out)), dtype=torch.int32, device=device)
        pb = torch.empty((kv, int(n_in)), dtype=torch.int32, device=device) if need_bwd else pb
        _lib.check(_lib.lib().sp_native_to_tables(
            _lib.ptr(pc), kv, n_pairs, int(bool(inverse)), int(n_in), int(n_out), _lib.ptr(pf),
            _lib.ptr(pb) if need_bwd else None, _lib.stream_of(device)), "sp_native_to_tables")
        coords = getattr(pair, "_spconv_triton_rowcoords", None)
        if coords is not None:
            fwd_rows, bwd_rows = (coords["in"], coords["out"]) if inverse else \
                (coords["out"], coords["in"])
            _attach_coords(pf, *fwd_rows)
            if need_bwd:
                _attach_coords(pb, *bwd_rows)
        cache[key] = (pf, pb)
    return pf, pb
