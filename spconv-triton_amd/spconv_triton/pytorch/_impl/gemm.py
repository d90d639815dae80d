"""Gather-GEMM host wrappers (forward, input gradient, weight gradient).

Host-side mirror of ``spconv_triton/pytorch/_impl/gemm.py`` of the reference
(``conv_forward`` :501-568, ``conv_backward_input`` :571-631,
``conv_backward_weight`` :634-713).  The device work is the MFMA gather-GEMM of
``csrc/sp_gemm.hip``.

Precision: every GEMM accumulates in fp32 on the matrix cores.

* ``SPCONV_ALLOW_TF32`` (read live, fp32 tensors only, like the reference's
  ``_allow_tf32``, gemm.py:456-463): the forward, input-gradient and
  weight-gradient GEMMs run as split-bf16 products on the bf16 matrix cores
  (gfx950 has no xf32 MFMA).  Each fp32 operand x becomes hi = bf16(x) and
  lo = bf16(x - hi), and hi*hi + hi*lo + lo*hi recovers each product to about
  2^-16 relative, tighter than TF32's 2^-11 (Henry, Tang & Heinecke, ARITH
  2019).  Off (the default), fp32 GEMMs are IEEE fp32.
* ``SPCONV_ALLOW_FP16_ACCUM`` / ``fp32_accum=False`` ask for fp16
  accumulation; gfx950 has no fp16-accumulating MFMA, so they are served at
  fp32 accumulation, which is at least as accurate.  The flags are accepted.
"""

from __future__ import annotations

import ctypes
import os
import weakref

import torch

from . import _lib


def _tf32(t: torch.Tensor) -> bool:
    """Split-bf16 products for an fp32 GEMM: live ``SPCONV_ALLOW_TF32`` (reference
    ``_allow_tf32``, gemm.py:460-463)."""
    from spconv_triton import constants

    return t.dtype == torch.float32 and bool(constants.SPCONV_ALLOW_TF32)


def split_bf16(x: torch.Tensor, pattern: int) -> torch.Tensor:
    """bf16 parts of fp32 rows (``sp_split_bf16x3``): pattern 0 = [hi | hi | lo],
    1 = [hi | lo | hi], 2 = [hi | lo]; returns [rows, parts * cols] bf16."""
    x = x.contiguous()
    rows, cols = x.shape
    parts = 2 if pattern == 2 else 3
    out = torch.empty((rows, parts * cols), dtype=torch.bfloat16, device=x.device)
    _lib.check(_lib.lib().sp_split_bf16x3(_lib.ptr(x), rows, cols, pattern, _lib.ptr(out),
                                          _lib.stream_of(x.device)), "sp_split_bf16x3")
    return out


def _should_mask(kv: int, pmask, argsort) -> bool:
    """Masked path applies only to single-word masks, 1 < kv <= 32 (reference gemm.py:486-498)."""
    return pmask is not None and argsort is not None and 1 < kv <= 32


class _PackCache:
    """Packed weights per weight tensor, valid while the tensor's storage,
    version counter (bumped by in-place updates such as optimizer steps) and
    the bias are unchanged.  Keyed by object identity; an entry is dropped
    when its weight tensor is freed."""

    def __init__(self):
        self._store = {}

    @staticmethod
    def _stamp(w: torch.Tensor, bias: torch.Tensor | None):
        bstamp = None if bias is None else (bias.data_ptr(), bias._version, bias.dtype)
        return (w.data_ptr(), w._version, w.dtype, tuple(w.shape), bstamp)

    def get(self, w, bias, dtype, transpose):
        ent = self._store.get(id(w))
        if ent is None or ent[0]() is not w:
            return None
        hit = ent[1].get((dtype, transpose))
        if hit is not None and hit[0] == self._stamp(w, bias):
            return hit[1]
        return None

    def put(self, w, bias, dtype, transpose, packed):
        key = id(w)
        ent = self._store.get(key)
        if ent is None or ent[0]() is not w:
            store = self._store
            ref = weakref.ref(w, lambda _r, k=key, s=store: s.pop(k, None))
            ent = (ref, {})
            store[key] = ent
        ent[1][(dtype, transpose)] = (self._stamp(w, bias), packed)


_PACKED = _PackCache()


def packed_weight(filters: torch.Tensor, bias: torch.Tensor | None, dtype,
                  transpose: bool) -> torch.Tensor:
    """Weights (+ bias) relaid into the MFMA operand layout of ``dtype`` (a torch
    dtype, or "bf16x3": the split-bf16 form of an fp32 weight); see
    ``sp_conv_pack_weight``.  filters is KRSC [K, *ksize, C].

    While the stream is being captured into a graph the cache is bypassed: the
    pack kernel is captured with the GEMM, so every replay reads the weight's
    current values (an optimizer step or ``load_state_dict`` between replays
    updates the weight in place, which no cache stamp can see from inside a
    replay)."""
    capturing = torch.cuda.is_current_stream_capturing()
    hit = None if capturing else _PACKED.get(filters, bias, dtype, transpose)
    if hit is not None:
        return hit
    K, C = filters.shape[0], filters.shape[-1]
    w = filters.detach().reshape(K, -1, C).contiguous()
    kv = w.shape[1]
    b = None if bias is None else bias.detach().contiguous()
    if b is not None and b.dtype != w.dtype:
        b = b.to(w.dtype)
    L = _lib.lib()
    dt = _lib.SP_BF16X3 if dtype == "bf16x3" else _lib.dtype_code(dtype)
    packed = torch.empty(L.sp_conv_packed_bytes(K, kv, C, dt, int(transpose)), dtype=torch.uint8,
                         device=w.device)
    _lib.check(L.sp_conv_pack_weight(_lib.ptr(w), _lib.dtype_code(w.dtype), _lib.ptr(b), K, kv,
                                     C, dt, int(transpose), _lib.ptr(packed),
                                     _lib.stream_of(w.device)), "sp_conv_pack_weight")
    if not capturing:
        _PACKED.put(filters, bias, dtype, transpose, packed)
    return packed


#: Use gather plans (per-tile distinct source rows staged in LDS) for the
#: forward and input-gradient GEMMs: True (always), False (never) or "auto":
#: when rows * max(C, K) >= PLAN_MIN_WORK.  A plan costs a build per table
#: (~25 us, more on large tables) and pays back per GEMM in proportion to the
#: GEMM's size: measured, plans slow a LiDAR encoder whose tables are <= 80k
#: rows of <= 64 channels (1.72 -> 1.78 ms per pass) and speed up the ResUNet
#: training step (88k - 240k rows, up to 256 channels; 10.75 -> 10.60 ms) and
#: the 200k-row 64-channel metric layer (direct kernel ~1.6x slower).
#: Results are bit-identical either way; tests force True / False to compare
#: the two kernels.
USE_GATHER_PLAN = "auto"
PLAN_MIN_WORK = 100_000 * 64


def _use_plan(M: int, C: int, K: int) -> bool:
    if USE_GATHER_PLAN == "auto":
        return M * max(C, K) >= PLAN_MIN_WORK
    return bool(USE_GATHER_PLAN)


def gather_plan(pairs: torch.Tensor, n_src: int, words: torch.Tensor | None = None):
    """Gather plan of a [kv, M] pair table (``sp_gather_plan_build``), or None
    when kv is outside the planned kernel's range.  Memoised on the table
    tensor, like the reference memoises its tables on the indice data
    (pairs.py:429-469); rebuilt if the table is modified in place.  The build
    is asynchronous (no host synchronization).  None as well while the stream
    is being captured and no plan is cached (the GEMM then gathers directly).
    words: the rows' mask words [M, mic] (nullable), which let the build skip
    the entries of offsets a tile's rows do not have (the same plan)."""
    kv, M = pairs.shape
    cached = getattr(pairs, "_spconv_triton_plan", None)
    stamp = (int(n_src), pairs._version, pairs.data_ptr())
    if cached is not None and cached[0] == stamp:
        return cached[1]
    if torch.cuda.is_current_stream_capturing():
        return None  # a build captured into a graph would rerun on every replay
    L = _lib.lib()
    nbytes = L.sp_gather_plan_bytes(M, kv)
    if nbytes == 0:
        return None
    plan = torch.empty(nbytes, dtype=torch.uint8, device=pairs.device)
    plan._spconv_triton_dims = (kv, M)
    _lib.check(L.sp_gather_plan_build(_lib.ptr(pairs), kv, M, int(n_src), _lib.ptr(words),
                                      0 if words is None else words.shape[1], _lib.ptr(plan),
                                      nbytes, None, _lib.stream_of(pairs.device)),
               "sp_gather_plan_build")
    pairs._spconv_triton_plan = (stamp, plan)
    return plan


#: Row order of the forward / input-gradient GEMMs.  "natural": the table's
#: own order, whose 256-row tiles share most of their source rows (staged once
#: per tile in LDS).  "mask": the stable argsort of the rows' masks, the
#: reference's order (gemm.py:282-296), whose tiles hold rows with similar
#: masks and so have fewer live offsets, but more distinct source rows (tiles
#: whose rows do not fit in LDS are gathered directly).  "auto": natural,
#: unless the layer is wide (C * K >= ORDER_MIN_WORK) and the mask order cuts
#: the natural tiles' MFMA work to at most ORDER_MAX_WORK_RATIO of it; only
#: tables that wide layers use more than once are looked at (see
#: row_order_variant).  Before the mask sort, a table whose natural work is
#: under 1 / ORDER_MAX_WORK_RATIO times its pairs is left natural (the mask
#: order's work is at least the pairs): 50k uniform voxels in 41 x 1600 x
#: 1408 (24 % of the natural work on pairs, mask order 28 % of the natural
#: work) take the mask order.  Every order gives bit-identical results.
ROW_ORDER = os.environ.get("SPCONV_GEMM_ROW_ORDER", "auto")
ORDER_MIN_WORK = 128 * 128
ORDER_MAX_WORK_RATIO = 0.35
#: IEEE fp32 operands (no SPCONV_ALLOW_TF32): a 32x32x2 fp32 MFMA does 1/8
#: of a 32x32x16 fp16 one's work in twice the clocks, so the matrix cores are
#: the limit, and the kernels skip the MFMAs of 32-row blocks without a pair.
#: The work is then also counted per live (64-row block, offset) pair, and the
#: mask order is taken when it cuts that work to at most
#: ORDER_MAX_WORK_RATIO_FP32 (or the tile count passes the rule above):
#: the LiDAR-like 50k cloud (natural 64-row work 4.6x the pairs, mask order
#: 49 % of it) 256 -> 256 GEMM 1.08 -> 0.71 ms, 128 -> 128 0.37 -> 0.23 ms,
#: where the 256-row tile count (mask order 50 %) keeps 16-bit layers natural.
ORDER_MAX_WORK_RATIO_FP32 = 0.6
#: Tables of at least ORDER_SPARSE_MIN_KV offsets with at most
#: ORDER_SPARSE_MAX_PAIRS_PER_ROW pairs per row take the mask order up to
#: ORDER_SPARSE_MAX_WORK_RATIO of the natural tile work: their mask-ordered
#: tiles reference few enough distinct rows that about half of them still
#: stage in LDS (the LiDAR-like 50k cloud, 3.27 pairs per row: 95 of 196
#: tiles overflow), where a surface cloud's (10 pairs per row) nearly all
#: overflow.  That cloud's SubMConv3d 256 -> 256 (tile work 50 %): fp16 0.149
#: -> 0.117 ms, TF32-equivalent 0.406 -> 0.342 ms.  The k2 s2 tables of the
#: ResUNet step (kv = 8, 1.7 pairs per row, 42 %; rebuilt every step) paid a
#: mask sort per step for nothing (step +0.1 ms): smaller windows stay out.
ORDER_SPARSE_MIN_KV = 27
ORDER_SPARSE_MAX_PAIRS_PER_ROW = 4.0
ORDER_SPARSE_MAX_WORK_RATIO = 0.5
#: A strided or transposed convolution's rulebook is often used once (rebuilt
#: every pass), so waiting for a second use would never reorder it.  Its pair
#: generation counts the table's pairs in passing; a table with at most
#: FIRST_USE_MAX_PAIRS_PER_ROW pairs per row (a transposed convolution of
#: sparse voxels has one pair per output, while a natural tile of its sorted
#: outputs holds nearly every offset) whose natural GEMM would multiply at
#: least FIRST_USE_MIN_MACS (rows * kv * C * K) is decided at its first wide
#: call instead: the mask sort, the permuted table, its plan and the two
#: statistics read-backs cost ~0.1-0.3 ms, which a smaller GEMM does not
#: repay (measured: the ResUNet step's 151k-row 256 -> 128 k2 s2 inverse
#: convolution, 4e10 MACs, made the step 0.4 ms slower; the transposed k3 s2
#: 256 -> 256 convolution of 50k voxels, 2.4e12 MACs, went 3.1 -> 2.2 ms).
FIRST_USE_MAX_PAIRS_PER_ROW = 1.5
FIRST_USE_MIN_MACS = 2e11
#: With at most SURE_PAIRS_PER_ROW pairs per row the mask order's tiles hold
#: about one offset each, so the statistics are not read back (two
#: synchronisations): the strided k3 s2 256 -> 256 convolution of 50k uniform
#: voxels (1.007 pairs per output) 0.56 -> 0.45 ms.
SURE_PAIRS_PER_ROW = 1.05
#: Mask-ordered tables whose tiles hold at most THIN_MAX_ITEMS_PER_TILE live
#: offsets on average (about one pair per row) run the thin kernel, which
#: loads each reduction chunk three chunks ahead; THIN_TILES forces it on (True)
#: or off (False) for every ordered call ("auto": by that rule).
THIN_MAX_ITEMS_PER_TILE = 1.5
THIN_TILES = "auto"
#: Mask-ordered tables with more items per tile, under IEEE fp32 operands,
#: run the thin kernel's quarter instance with every tile it hands to the
#: direct path spread over four workgroups (thin_tiles 2 of
#: sp_conv_gemm_ordered): the tiles with the most mask bits carry most of the
#: MFMA work (LiDAR-like 50k cloud: 95 of 196 tiles, 82 % of it), and their
#: waves set the kernel's end.  GEMM 256 -> 256 603 -> 483 us (staged ->
#: split), 128 -> 128 229 -> 164 us; for 16-bit operands the staged kernel
#: stays faster (107 against 179 us), and tables of about one pair per row
#: keep the thin kernel's last-16-tiles split (splitting every tile measured
#: 0.101 -> 0.105 ms on the uniform reference-class layer).
THIN_SPLIT_FP32 = True
#: kv range of the gather plans (sp_gather_plan_bytes: 1..1024).  A plan tile
#: holds at most 64 live offsets (more: its rows are gathered directly), so
#: natural-order tables are planned up to kv = 64 only (a 5^3 window's natural
#: tiles hold ~125 live offsets each); mask-ordered tables, whose tiles hold
#: rows of like masks, up to 1024.
_PLAN_MAX_KV = 64
_ORDERED_PLAN_MAX_KV = 1024
#: Above 64 offsets a plan tile also lists only items within one group of 64
#: offsets (the direct kernel's summation groups); a mask-ordered plan with
#: more than ORDERED_PLAN_MAX_OVERFLOW of its tiles gathered directly is
#: dropped at the decision (one more read-back), as the direct kernel with the
#: rows' mask words reads fewer table entries: the 4-D submanifold table of
#: ~500k voxels (time neighbours at offsets 13, 40 and 67 in most tiles) had
#: 1 899 of 1 960 tiles overflow, 289 us planned against 287 us direct.
ORDERED_PLAN_MAX_OVERFLOW = 0.5
_STATS_MAX_KV = 512  # kv range of sp_table_stats


def _launch_table_stats(pairs: torch.Tensor, n_src: int) -> torch.Tensor:
    kv, M = pairs.shape
    stats = torch.zeros(3, dtype=torch.int64, device=pairs.device)
    _lib.check(_lib.lib().sp_table_stats(_lib.ptr(pairs), kv, M, int(n_src), _lib.ptr(stats),
                                         _lib.stream_of(pairs.device)), "sp_table_stats")
    return stats


def table_stats(pairs: torch.Tensor, n_src: int) -> tuple[int, int, int]:
    """(pairs, live (256-row tile, offset) pairs, live (64-row block, offset)
    pairs) of a [kv, M] table in its own row order (``sp_table_stats``).
    Reading them synchronizes."""
    return tuple(int(v) for v in _launch_table_stats(pairs, n_src).cpu())


def mask_order(pairs: torch.Tensor, with_words: bool = False):
    """Stable argsort of the rows' masks of a [kv, M] table, as the reference's
    mask_argsort (pairs.py:356-392) orders them: int32 [M].  with_words: also
    the sorted mask words ([M, ceil(kv/32)], row order[i] at i)."""
    from . import pairs as _pairs
    kv = pairs.shape[0]
    words = _pairs.mask_words(pairs)
    pm, ar = _pairs.sort_mask_words(words, kv, _pairs.split_masks(kv, False), True)
    return (ar[0], pm[0]) if with_words else ar[0]


def permute_table(pairs: torch.Tensor, order: torch.Tensor,
                  order_words: torch.Tensor | None = None) -> torch.Tensor:
    """out[k, i] = pairs[k, order[i]] (``sp_permute_table``); order_words: the
    mask words of the rows in that order (kv <= 32), which lets the kernel
    skip the reads of empty entries."""
    kv, M = pairs.shape
    out = torch.empty_like(pairs)
    _lib.check(_lib.lib().sp_permute_table(_lib.ptr(pairs), kv, M, _lib.ptr(order),
                                           _lib.ptr(order_words), _lib.ptr(out),
                                           _lib.stream_of(pairs.device)), "sp_permute_table")
    return out


def _decide_at_first_use(pairs: torch.Tensor, work: int) -> bool:
    """A table whose pair count (from its pair generation) shows few pairs per
    row, under a large GEMM: see FIRST_USE_MAX_PAIRS_PER_ROW."""
    npairs = getattr(pairs, "_spconv_triton_npairs", None)
    kv, M = pairs.shape
    return (npairs is not None and kv >= 8 and npairs <= FIRST_USE_MAX_PAIRS_PER_ROW * M
            and float(M) * kv * work >= FIRST_USE_MIN_MACS)


def row_order_variant(pairs: torch.Tensor, n_src: int, work: int, plan_ok: bool = True,
                      fp32: bool = False):
    """(order, permuted table, its gather plan or None) when a GEMM of
    ``work`` = C * K on this table should take its rows in mask order (see
    ROW_ORDER), else None.  ``plan_ok``: the call may use a gather plan.
    ``fp32``: the call multiplies IEEE fp32 operands (see
    ORDER_MAX_WORK_RATIO_FP32); the call that makes the decision sets it for
    every layer on the table.

    In auto mode only tables that wide layers use more than once are looked
    at (or, see FIRST_USE_MAX_PAIRS_PER_ROW, tables with few pairs per row):
    the first wide call on a table runs in natural order and launches
    nothing (a table rebuilt every step costs nothing); the second reads the
    table's statistics back (a stream synchronization) and, when they pass,
    sorts the masks, permutes the table and reads the permuted table's
    statistics (a second one).  The outcome is memoised on the table tensor
    (like its plan) and recomputed if the table changes; a reordered table
    keeps the order (M int32), a permuted copy of itself (kv * M int32) and
    that copy's plan.  Calls made while the stream is being captured into a
    graph use a settled order but never advance the decision."""
    mode = ROW_ORDER
    if mode == "natural":
        return None
    if mode not in ("auto", "mask"):
        raise ValueError(f"SPCONV_GEMM_ROW_ORDER must be auto, natural or mask, not {mode!r}")
    kv, M = pairs.shape
    if M == 0:
        return None
    stamp = (int(n_src), pairs._version, pairs.data_ptr(), mode)
    cached = getattr(pairs, "_spconv_triton_order", None)
    step = cached[1] if cached is not None and cached[0] == stamp else "start"
    if isinstance(step, tuple):
        # a settled mask order serves every layer on the table, each with or
        # without the permuted table's gather plan as the call asks (built on
        # the first call that wants it)
        order, perm, plan = step
        if not (plan_ok and kv <= _ORDERED_PLAN_MAX_KV):
            return step if plan is None else (order, perm, None)
        if (plan is None and not getattr(perm, "_spconv_triton_noplan", False)
                and not torch.cuda.is_current_stream_capturing()):
            step = (order, perm, gather_plan(perm, n_src, getattr(perm, "_spconv_triton_words",
                                                                   None)))
            pairs._spconv_triton_order = (stamp, step)
        return step
    if step == "natural" or (mode == "auto" and (work < ORDER_MIN_WORK or kv > _STATS_MAX_KV)):
        return None  # narrow layers never start the decision
    if torch.cuda.is_current_stream_capturing():
        return None  # a graph being captured must not synchronize: decide on a later call
    if mode == "auto" and step == "start" and not _decide_at_first_use(pairs, work):
        pairs._spconv_triton_order = (stamp, "seen")
        return None

    planned = plan_ok and kv <= _ORDERED_PLAN_MAX_KV

    # (rows the GEMM multiplies, bound): per live tile offset (planned) or wave
    # offset; fp32 operands also per live 64-row block offset.  The mask order
    # is taken when one measure passes.  The efficiency test (pairs against
    # the natural work) skips the mask sort only where its work test must
    # fail, as the mask order's work is at least the pairs.
    tests = [((lambda st: 256 * st[1]) if planned else (lambda st: 64 * st[2]),
              ORDER_MAX_WORK_RATIO)]
    if fp32:
        tests.append((lambda st: 64 * st[2], ORDER_MAX_WORK_RATIO_FP32))

    variant = None
    npairs = getattr(pairs, "_spconv_triton_npairs", None)
    sure = mode == "mask" or (npairs is not None and npairs <= SURE_PAIRS_PER_ROW * M)
    natural = table_stats(pairs, n_src) if not sure else None
    if (natural is not None and kv >= ORDER_SPARSE_MIN_KV
            and natural[0] <= ORDER_SPARSE_MAX_PAIRS_PER_ROW * M):
        tests.append((tests[0][0], ORDER_SPARSE_MAX_WORK_RATIO))
    if sure or any(0 < natural[0] < r * f(natural) for f, r in tests):
        order, words = mask_order(pairs, with_words=True)
        perm = permute_table(pairs, order, words if kv <= 32 else None)
        perm._spconv_triton_words = words  # the unplanned kernel reads live offsets only
        masked = table_stats(perm, n_src) if not sure else None
        if sure or any(f(masked) <= r * f(natural) for f, r in tests):
            plan = gather_plan(perm, n_src, words) if planned else None
            tiles = (M + 255) // 256
            if (plan is not None and kv > _PLAN_MAX_KV
                    and plan_overflow_count(plan) > ORDERED_PLAN_MAX_OVERFLOW * tiles):
                plan = None
                perm._spconv_triton_noplan = True
            variant = (order, perm, plan)
            perm._spconv_triton_thin = (
                (mode != "mask" and masked is None)  # about one pair per row
                or (masked is not None and masked[1] <= THIN_MAX_ITEMS_PER_TILE * tiles))
    pairs._spconv_triton_order = (stamp, variant if variant is not None else "natural")
    return variant


#: Key order for planned GEMMs: a table whose natural 256-row tiles mostly
#: overflow LDS (more than KEY_ORDER_MIN_OVERFLOW of its tiles reference more
#: distinct source rows than the plan can stage: rows in no spatial order,
#: e.g. a random permutation of the voxels) takes its rows sorted by their
#: linear coordinate key instead, where a tile's rows are spatial neighbours.
#: The table's rows' coordinates come from pair generation.
KEY_ORDER_MIN_OVERFLOW = 0.25


def key_order(coords) -> torch.Tensor:
    """Stable argsort of rows by batch-major linear key (int32 [M]): the rows'
    coordinates [M, ndim+1], spatial shape and batch size."""
    from . import pairs as _pairs
    idx, shape, batch = coords
    key = idx[:, 0].to(torch.int64)
    for d, n in enumerate(shape):
        key = key * int(n) + idx[:, d + 1].to(torch.int64)
    volume = int(batch)
    for n in shape:
        volume *= int(n)
    bits = max(1, (volume - 1).bit_length())
    if bits <= 32:
        words = key.to(torch.int32).view(-1, 1)
    else:  # two words, the high one most significant
        words = torch.stack([(key & 0xFFFFFFFF).to(torch.int32), (key >> 32).to(torch.int32)], 1)
    _, ar = _pairs.sort_mask_words(words.contiguous(), bits, _pairs.split_masks(bits, False), True)
    return ar[0]


def key_order_variant(pairs: torch.Tensor, n_src: int, plan: torch.Tensor):
    """(order, permuted table, its gather plan) when a planned GEMM on this
    table should take its rows in key order (see KEY_ORDER_MIN_OVERFLOW), else
    None.  Decided on the table's second planned GEMM, like the mask order
    (row_order_variant): the first call launches nothing, the second reads the
    plan's overflow count back (one synchronization) and, when most tiles
    overflow, sorts the rows by key, permutes the table and plans it.  The
    outcome is memoised on the table tensor.  Calls made while the stream is
    being captured into a graph use a settled order but never advance the
    decision."""
    coords = getattr(pairs, "_spconv_triton_rowcoords", None)
    if coords is None or plan is None or coords[0].shape[0] != pairs.shape[1]:
        return None
    stamp = (int(n_src), pairs._version, pairs.data_ptr())
    cached = getattr(pairs, "_spconv_triton_keyorder", None)
    step = cached[1] if cached is not None and cached[0] == stamp else "start"
    if isinstance(step, tuple):
        return step
    if step == "natural" or torch.cuda.is_current_stream_capturing():
        return None
    if step == "start":
        pairs._spconv_triton_keyorder = (stamp, "seen")
        return None
    tiles = (pairs.shape[1] + 255) // 256
    variant = None
    if plan_overflow_count(plan) > KEY_ORDER_MIN_OVERFLOW * tiles:
        order = key_order(coords)
        perm = permute_table(pairs, order)
        variant = (order, perm, gather_plan(perm, n_src))
    pairs._spconv_triton_keyorder = (stamp, variant if variant is not None else "natural")
    return variant


def plan_overflow_count(plan: torch.Tensor) -> int:
    """Number of tiles of a plan (from gather_plan) that the GEMM gathers
    directly (``sp_gather_plan_overflow``: also writes the plan's overflow list;
    synchronizes).  Memoised on the plan tensor, which never changes."""
    n = getattr(plan, "_spconv_triton_novf", None)
    if n is None:
        kv, M = plan._spconv_triton_dims
        out = ctypes.c_int64(0)
        _lib.check(_lib.lib().sp_gather_plan_overflow(_lib.ptr(plan), plan.numel(), kv, M,
                                                      ctypes.byref(out),
                                                      _lib.stream_of(plan.device)),
                   "sp_gather_plan_overflow")
        n = plan._spconv_triton_novf = int(out.value)
    return n


def _gemm(a: torch.Tensor, filters: torch.Tensor, bias, transpose: bool, pairs: torch.Tensor,
          M: int, pm, ar, out: torch.Tensor, split: bool = False):
    """out = gather-GEMM of ``a`` through ``pairs``.  split: ``a`` is the
    [hi | hi | lo] split of an fp32 operand (``split_bf16`` pattern 0) and the
    weight is packed as "bf16x3", so the reduction runs three times as long."""
    K, C = filters.shape[0], filters.shape[-1]
    kv = pairs.shape[0]
    packed = packed_weight(filters, bias, "bf16x3" if split else a.dtype, transpose)
    L = _lib.lib()
    use_plan = _use_plan(M, C, K)
    variant = row_order_variant(pairs, a.shape[0], K * C, use_plan,
                                fp32=a.dtype == torch.float32 and not split)
    if split:  # the GEMM's reduction dimension is tripled
        K, C = (3 * K, C) if transpose else (K, 3 * C)
    if variant is None:
        plan = gather_plan(pairs, a.shape[0]) if use_plan and kv <= _PLAN_MAX_KV else None
        if plan is not None:
            variant = key_order_variant(pairs, a.shape[0], plan)
    if variant is not None:
        order, perm, plan = variant
        thin = THIN_TILES if THIN_TILES != "auto" else getattr(perm, "_spconv_triton_thin", False)
        if (THIN_TILES == "auto" and THIN_SPLIT_FP32 and not thin and plan is not None
                and a.dtype == torch.float32 and not split):
            thin = 2  # see THIN_SPLIT_FP32
        words = getattr(perm, "_spconv_triton_words", None)  # sorted mask words [M, mic]
        _lib.check(L.sp_conv_gemm_ordered(
            _lib.ptr(a), _lib.dtype_code(a.dtype), a.shape[0], _lib.ptr(packed), K, kv, C,
            int(transpose), int(bias is not None), _lib.ptr(perm), M, _lib.ptr(order),
            _lib.ptr(plan), 0 if plan is None else plan.numel(), int(thin),
            _lib.ptr(words), 0 if words is None else words.shape[1], _lib.ptr(out),
            _lib.dtype_code(out.dtype), _lib.stream_of(a.device)), "sp_conv_gemm_ordered")
        return
    if plan is not None:
        # the planned kernel skips empty offsets itself: mask tables are not needed
        _lib.check(L.sp_conv_gemm_planned(
            _lib.ptr(a), _lib.dtype_code(a.dtype), a.shape[0], _lib.ptr(packed), K, kv, C,
            int(transpose), int(bias is not None), _lib.ptr(pairs), M, _lib.ptr(plan),
            plan.numel(), _lib.ptr(out), _lib.dtype_code(out.dtype),
            _lib.stream_of(a.device)), "sp_conv_gemm_planned")
        return
    _lib.check(L.sp_conv_gemm_packed(
        _lib.ptr(a), _lib.dtype_code(a.dtype), a.shape[0], _lib.ptr(packed), K, kv, C,
        int(transpose), int(bias is not None), _lib.ptr(pairs), M, _lib.ptr(pm), _lib.ptr(ar),
        _lib.ptr(out), _lib.dtype_code(out.dtype), _lib.stream_of(a.device)),
        "sp_conv_gemm_packed")


def conv_forward(features: torch.Tensor, filters_krsc: torch.Tensor, pair_fwd: torch.Tensor,
                 n_out: int, bias: torch.Tensor | None = None,
                 out_dtype: torch.dtype | None = None, pair_mask: torch.Tensor | None = None,
                 mask_argsort: torch.Tensor | None = None,
                 fp32_accum: bool | None = None) -> torch.Tensor:
    """Gather-GEMM forward; returns [n_out, K].  filters_krsc is [K, kv, C]
    (or the KRSC parameter [K, *ksize, C] itself, which lets packed weights be
    reused across calls)."""
    _lib.require_gpu(features, pair_fwd)
    K, C = filters_krsc.shape[0], filters_krsc.shape[-1]
    kv = pair_fwd.shape[0]
    if out_dtype is None:
        out_dtype = features.dtype
    out = torch.empty((n_out, K), dtype=out_dtype, device=features.device)
    if n_out == 0:
        return out
    if filters_krsc.numel() != K * kv * C:
        raise AssertionError("filters do not match the pair table's kernel volume")
    x = features.contiguous()
    pf = pair_fwd.contiguous()
    if pf.shape != (kv, n_out):
        raise AssertionError(f"pair_fwd shape {tuple(pf.shape)} != ({kv}, {n_out})")
    if x.shape[1] != C:
        raise AssertionError("channel size mismatch")
    use_mask = _should_mask(kv, pair_mask, mask_argsort)
    pm = pair_mask.contiguous() if use_mask else None
    ar = mask_argsort.contiguous() if use_mask else None
    if use_mask and (pm.numel() != n_out or ar.numel() != n_out):
        raise AssertionError("mask tables do not match the output rows")
    if _tf32(x):
        _gemm(split_bf16(x, 0), filters_krsc, bias, False, pf, n_out, pm, ar, out, split=True)
        return out
    _gemm(x, filters_krsc, bias, False, pf, n_out, pm, ar, out)
    return out


def conv_backward_input(grad_out: torch.Tensor, filters_krsc: torch.Tensor,
                        pair_bwd: torch.Tensor, n_in: int,
                        pair_mask: torch.Tensor | None = None,
                        mask_argsort: torch.Tensor | None = None,
                        fp32_accum: bool | None = None) -> torch.Tensor:
    """din[j, c] = sum_k grad_out[pair_bwd[k, j], :] @ W[k][:, c]; returns [n_in, C]."""
    _lib.require_gpu(grad_out, pair_bwd)
    K, C = filters_krsc.shape[0], filters_krsc.shape[-1]
    kv = pair_bwd.shape[0]
    din = torch.empty((n_in, C), dtype=grad_out.dtype, device=grad_out.device)
    if n_in == 0:
        return din
    g = grad_out.contiguous()
    pb = pair_bwd.contiguous()
    if pb.shape != (kv, n_in):
        raise AssertionError(f"pair_bwd shape {tuple(pb.shape)} != ({kv}, {n_in})")
    if g.shape[1] != K:
        raise AssertionError("grad_out channels do not match the filters")
    use_mask = _should_mask(kv, pair_mask, mask_argsort)
    pm = pair_mask.contiguous() if use_mask else None
    ar = mask_argsort.contiguous() if use_mask else None
    if _tf32(g):
        _gemm(split_bf16(g, 0), filters_krsc, None, True, pb, n_in, pm, ar, din, split=True)
        return din
    _gemm(g, filters_krsc, None, True, pb, n_in, pm, ar, din)
    return din


def compacted_signal(pair_fwd: torch.Tensor):
    """Per-offset (input row, output row) lists of a gather table, output rows
    ascending -- the reference's ``valid_signal`` (gemm.py:661-669) in a
    per-offset slotted layout.  Memoised on the table tensor."""
    cached = getattr(pair_fwd, "_spconv_triton_dw_sig", None)
    if cached is not None:
        return cached
    pf = pair_fwd.contiguous()
    kv, n = pf.shape
    device = pf.device
    out_rows = torch.empty((kv, n), dtype=torch.int32, device=device)
    in_rows = torch.empty((kv, n), dtype=torch.int32, device=device)
    counts = torch.empty((kv,), dtype=torch.int32, device=device)
    L = _lib.lib()
    ws = _lib.workspace(L.sp_compact_workspace_size(kv, n), device)
    _lib.check(L.sp_compact_table(_lib.ptr(pf), kv, n, _lib.ptr(out_rows), _lib.ptr(in_rows),
                                  _lib.ptr(counts), None, kv, _lib.ptr(ws), ws.numel(),
                                  _lib.stream_of(device)), "sp_compact_table")
    sig = (in_rows, out_rows, counts)
    pair_fwd._spconv_triton_dw_sig = sig
    return sig


def conv_backward_weight(features: torch.Tensor, grad_out: torch.Tensor, pair_fwd: torch.Tensor,
                         weight_shape_krsc, fp32_accum: bool | None = None) -> torch.Tensor:
    """dW [K, kv, C] = per-offset X^T G over compacted pairs (deterministic split-P)."""
    _lib.require_gpu(features, grad_out, pair_fwd)
    K, C = int(weight_shape_krsc[0]), int(weight_shape_krsc[-1])
    kv = int(pair_fwd.shape[0])
    n_out = grad_out.shape[0]
    dw = torch.empty((K, kv, C), dtype=grad_out.dtype, device=grad_out.device)
    if n_out == 0 or kv == 0:
        dw.zero_()
        return dw
    x = features.contiguous()
    g = grad_out.contiguous()
    if x.dtype != g.dtype:
        raise AssertionError("features and grad_out dtypes differ")
    in_rows, out_rows, counts = compacted_signal(pair_fwd)
    stride = in_rows.shape[1]
    L = _lib.lib()
    dt = _lib.dtype_code(x.dtype)
    if _tf32(x):  # split-bf16 halves [hi | lo]; the fp32 dW sums their four products
        x, g, dt = split_bf16(x, 2), split_bf16(g, 2), _lib.SP_BF16X3
        ws = _lib.workspace(L.sp_wgrad_workspace_size(2 * K, kv, 2 * C, stride), x.device)
    else:
        ws = _lib.workspace(L.sp_wgrad_workspace_size(K, kv, C, stride), x.device)
    _lib.check(L.sp_conv_wgrad(_lib.ptr(x), x.shape[0], _lib.ptr(g), n_out,
                               dt, C, K, kv, _lib.ptr(in_rows),
                               _lib.ptr(out_rows), _lib.ptr(counts), stride, _lib.ptr(dw),
                               _lib.ptr(ws), ws.numel(), _lib.stream_of(x.device)),
               "sp_conv_wgrad")
    return dw
