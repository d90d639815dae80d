"""Gather plans and the planned gather-GEMM.

A gather plan lists, per tile of 256 consecutive rows of a [kv, M] pair table,
the ascending distinct source rows, and per 64-row wave tile the offsets with
a pair and the staged LDS address of every (offset, row) (csrc/sp_plan.h).
The plan is checked entry by entry against numpy (``np.unique`` /
``np.searchsorted`` per tile).  The planned GEMM stages those
rows in LDS; it must be bit-identical to the unplanned GEMM (same summation
order by construction) on every dtype, on rows whose length is not a multiple
of the vector width, on several column blocks, on the input gradient, and on
tiles with too many distinct rows for LDS (which the kernel gathers directly).
"""

import numpy as np
import pytest
import torch

from test_gpu_gemm import CASES, _q, _tables, rand_indices
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TILE = 256
LDS_ROWS = 896  # kLdsRows of csrc/sp_plan.h
GROUP = 4  # kItemGroup of csrc/sp_plan.h
MAX_ITEMS = 64  # kPlanMaxItems of csrc/sp_plan.h: more live offsets make an overflow tile
GROUP_OFFSETS = 64  # kPlanGroupOffsets: so do live offsets in two groups of 64


def _align(v, a=256):
    return (v + a - 1) // a * a


def _chunk_base(slot):
    """LDS address of a staged row (slot * 64, 16-byte pieces xor-swizzled by slot bits 2-3)."""
    slot = np.asarray(slot, dtype=np.int64)
    return slot * 64 + (((slot >> 2) & 3) << 4)


def _parse(plan, kv, M):
    """Split a plan buffer into its parts (layout of csrc/sp_plan.h).  The
    overflow count and list are written on request only: ask for them first."""
    from spconv_triton.pytorch._impl import gemm

    gemm.plan_overflow_count(plan)
    nt = (max(M, 1) + TILE - 1) // TILE
    E = (min(kv, MAX_ITEMS) + GROUP - 1) // GROUP * GROUP
    buf = plan.cpu().numpy()
    count_off = 256
    ovf_off = _align(count_off + nt * 4)
    rows_off = _align(ovf_off + nt * 4)
    nact_off = _align(rows_off + nt * LDS_ROWS * 4)
    koff_off = _align(nact_off + nt * 4)
    addr_off = _align(koff_off + nt * E * 4)
    n_ovf = int(buf[:4].view(np.int32)[0])
    return {
        "n_ovf": n_ovf,
        "count": buf[count_off:count_off + nt * 4].view(np.int32),
        "ovf": buf[ovf_off:ovf_off + nt * 4].view(np.int32)[:n_ovf],
        "rows": buf[rows_off:rows_off + nt * LDS_ROWS * 4].view(np.int32).reshape(nt, LDS_ROWS),
        "nact": buf[nact_off:nact_off + nt * 4].view(np.int32),
        "koff": buf[koff_off:koff_off + nt * E * 4].view(np.int32).reshape(nt, E),
        # [tile][item][wave][l32][mt] -> [tile][item][row of the tile]
        "addr": buf[addr_off:addr_off + nt * E * TILE * 2].view(np.uint16)
                .reshape(nt, E, 4, 32, 2).transpose(0, 1, 2, 4, 3).reshape(nt, E, TILE),
    }


def _check_plan(pf, n_src, words=None):
    """Every part of the plan against numpy: per tile np.unique of the valid
    sources, the offsets with a pair (ascending) then -1, and per (item, row)
    the staged address of the row's rank in the unique list (np.searchsorted),
    or of the zero row U, up to the end of the tile's last group of items.  A
    tile with more than MAX_ITEMS live offsets is an overflow tile whose count
    reads LDS_ROWS, as does one whose live offsets span two groups of
    GROUP_OFFSETS.  words: build the plan from the rows' mask words too."""
    from spconv_triton.pytorch._impl import gemm

    kv, M = pf.shape
    plan = gemm.gather_plan(pf, n_src, words)
    assert plan is not None
    n_over_host = gemm.plan_overflow_count(plan)
    P = _parse(plan, kv, M)
    p = pf.cpu().numpy()
    overflow = []
    for t in range((M + TILE - 1) // TILE):
        blk = p[:, t * TILE:(t + 1) * TILE]
        valid = (blk >= 0) & (blk < n_src)
        live = np.nonzero(valid.any(axis=1))[0]
        if live.size > MAX_ITEMS or (live.size and live[0] // GROUP_OFFSETS
                                      != live[-1] // GROUP_OFFSETS):
            assert P["count"][t] == LDS_ROWS, f"tile {t}: {live} items, not an overflow tile"
            overflow.append(t)
            continue
        uniq = np.unique(blk[valid])
        U = uniq.size
        assert P["count"][t] == U, f"tile {t}: count {P['count'][t]} != {U}"
        if U >= LDS_ROWS:
            overflow.append(t)
            continue
        np.testing.assert_array_equal(P["rows"][t, :U], uniq)
        assert (P["rows"][t, U:] == -1).all()
        addr = np.where(valid, _chunk_base(np.searchsorted(uniq, np.where(valid, blk, 0))),
                        _chunk_base(U))
        n = live.size
        assert P["nact"][t] == n, f"tile {t}: {P['nact'][t]} items != {n}"
        np.testing.assert_array_equal(P["koff"][t, :n], live)
        assert (P["koff"][t, n:] == -1).all()
        n4 = (n + GROUP - 1) // GROUP * GROUP
        exp = np.full((n4, TILE), _chunk_base(U), dtype=np.int64)
        a = addr[live]
        exp[:n, :a.shape[1]] = a  # rows past M (last tile) keep the zero row
        np.testing.assert_array_equal(P["addr"][t, :n4].astype(np.int64), exp)
    assert n_over_host == P["n_ovf"] == len(overflow)
    np.testing.assert_array_equal(P["ovf"], np.asarray(overflow, dtype=np.int32))
    return len(overflow)


def _random_table(rng, kv, M, n_src, p_valid):
    t = rng.integers(0, n_src, size=(kv, M)).astype(np.int32)
    t[rng.random((kv, M)) > p_valid] = -1
    return torch.from_numpy(t).to(DEV)


def test_plan_layout_limits():
    from spconv_triton.pytorch._impl import _lib

    L = _lib.lib()
    assert L.sp_gather_plan_bytes(1000, 64) > 0
    # above 64 offsets a tile lists at most 64 items: the same size as kv = 64
    assert L.sp_gather_plan_bytes(1000, 1024) == L.sp_gather_plan_bytes(1000, 64)
    assert L.sp_gather_plan_bytes(1000, 1025) == 0  # kv above the planned kernel's range
    assert L.sp_gather_plan_bytes(1000, 0) == 0


@pytest.mark.parametrize("case", ["subm", "strided_fwd", "strided_bwd", "tiny", "exact_tiles",
                                  "overflow", "kv64", "wide_window", "empty_rows"])
def test_plan_matches_numpy(case):
    rng = np.random.default_rng(7)
    if case in ("subm", "strided_fwd", "strided_bwd"):
        idx = rand_indices(rng, 2, [28] * 3, 6000)
        subm = case == "subm"
        res = _tables(idx, 2, [28] * 3, [3] * 3, [1 if subm else 2] * 3, [1] * 3, subm)
        if case == "strided_bwd":
            pf, n_src = res[3], res[2].shape[1]
        else:
            pf, n_src = res[2], idx.shape[0]
    elif case == "tiny":
        idx = rand_indices(rng, 1, [8] * 3, 100)
        pf, n_src = _tables(idx, 1, [8] * 3, [3] * 3, [1] * 3, [1] * 3, True)[2], 100
    elif case == "exact_tiles":
        pf, n_src = _random_table(rng, 27, 512, 800, 0.3), 800
    elif case == "overflow":
        pf, n_src = _random_table(rng, 27, 700, 100_000, 0.7), 100_000
    elif case == "wide_window":
        # sources spread over 5M rows: too wide a window for the bitmap, so the
        # builder sorts
        pf, n_src = _random_table(rng, 27, 600, 5_000_000, 0.05), 5_000_000
    elif case == "empty_rows":
        # tiles without any pair, and out-of-range sources (ignored)
        t = rng.integers(0, 2000, size=(8, 900)).astype(np.int32)
        t[:, 256:600] = -1
        t[0, 700:710] = 5000
        pf, n_src = torch.from_numpy(t).to(DEV), 2000
    else:
        pf, n_src = _random_table(rng, 64, 600, 900, 0.2), 900
    n_over = _check_plan(pf.contiguous(), n_src)
    if case == "overflow":
        assert n_over == 3
    if case == "tiny":
        assert n_over == 0


@pytest.mark.parametrize("kv", [27, 64, 81, 125])
def test_plan_with_row_words_identical(kv):
    """A plan built with the rows' mask words (the build reads only the offsets
    some row of a tile has) equals the plan built from the table alone in
    every part the GEMM reads (counts, overflow list, distinct rows, items and
    their addresses up to the tile's last group), on a mask-ordered sparse
    table (few live offsets per tile) and a denser one."""
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(21)
    M = 5000
    for p_valid in (0.03, 0.5):
        pf = _random_table(rng, kv, M, 20_000, p_valid).contiguous()
        order, words = gemm.mask_order(pf, with_words=True)
        perm = gemm.permute_table(pf, order, words if kv <= 32 else None)
        A = _parse(gemm.gather_plan(perm.clone(), 20_000), kv, M)
        B = _parse(gemm.gather_plan(perm, 20_000, words), kv, M)
        for key in ("count", "ovf"):
            np.testing.assert_array_equal(A[key], B[key], f"{key}, p_valid={p_valid}")
        for t in range(A["count"].shape[0]):
            if A["count"][t] >= LDS_ROWS:
                continue  # an overflow tile: nothing else is written for it
            assert A["nact"][t] == B["nact"][t], f"tile {t} items, p_valid={p_valid}"
            n = int(A["nact"][t])
            n4 = (n + GROUP - 1) // GROUP * GROUP
            np.testing.assert_array_equal(A["rows"][t], B["rows"][t])
            np.testing.assert_array_equal(A["koff"][t], B["koff"][t])
            np.testing.assert_array_equal(A["addr"][t, :n4], B["addr"][t, :n4])


def test_plan_overflow_list_many_tiles():
    """The overflow list of a table with more tiles than one round of the
    listing kernel covers (17 000 tiles, 16 384 per round): every 7th tile
    references 1 024 distinct sources (overflow), the others 64.  Counts and
    the ascending overflow list against numpy."""
    from spconv_triton.pytorch._impl import gemm

    nt, kv = 17_000, 4
    M = nt * TILE
    col = np.arange(M)
    tile, r = col // TILE, col % TILE
    over = np.arange(nt) % 7 == 3
    t = np.empty((kv, M), dtype=np.int32)
    for k in range(kv):
        t[k] = np.where(over[tile], tile * 1024 + k * TILE + r, tile * 1024 + r % 64)
    plan = gemm.gather_plan(torch.from_numpy(t).to(DEV), nt * 1024)
    P = _parse(plan, kv, M)
    np.testing.assert_array_equal(P["count"], np.where(over, 1024, 64))
    assert gemm.plan_overflow_count(plan) == P["n_ovf"] == int(over.sum())
    np.testing.assert_array_equal(P["ovf"], np.nonzero(over)[0].astype(np.int32))


def _both(a, w, bias, transpose, pairs, M, out_dtype=None):
    from spconv_triton.pytorch._impl import gemm

    out_dtype = out_dtype or a.dtype
    N = w.shape[-1] if transpose else w.shape[0]
    res = []
    prev = gemm.USE_GATHER_PLAN
    for use in (True, False):
        gemm.USE_GATHER_PLAN = use
        try:
            out = torch.empty((M, N), dtype=out_dtype, device=DEV)
            gemm._gemm(a, w, bias, transpose, pairs, M, None, None, out)
            res.append(out)
        finally:
            gemm.USE_GATHER_PLAN = prev
    return res


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("ci", range(len(CASES)))
def test_planned_equals_unplanned(ci, dtype):
    C, K, n, subm, stride = CASES[ci]
    rng = np.random.default_rng(90 + ci)
    idx = rand_indices(rng, 2, [28] * 3, n)
    res = _tables(idx, 2, [28] * 3, [3] * 3, [stride] * 3, [1] * 3, subm)
    pf, pb = res[2], res[3]
    torch.manual_seed(ci)
    x, _ = _q(torch.randn(idx.shape[0], C), dtype)
    w, _ = _q(torch.randn(K, 3, 3, 3, C) / np.sqrt(27 * C), dtype)
    b, _ = _q(torch.randn(K) * 0.1, dtype)
    planned, direct = _both(x, w, b, False, pf, pf.shape[1])
    assert torch.equal(planned, direct), "forward: planned != unplanned"
    g, _ = _q(torch.randn(pf.shape[1], K), dtype)
    planned, direct = _both(g, w, None, True, pb, idx.shape[0])
    assert torch.equal(planned, direct), "dgrad: planned != unplanned"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_planned_overflow_tiles(dtype):
    """Tiles with too many distinct rows for LDS take the staged kernel's
    direct path (same launch); mixed with staged tiles the result must not
    change."""
    rng = np.random.default_rng(11)
    kv, M, n_src, C, K = 27, 1500, 50_000, 32, 64
    t = rng.integers(0, n_src, size=(kv, M)).astype(np.int32)
    t[rng.random((kv, M)) > 0.6] = -1
    # tiles 2..5 reference only a narrow window of rows: they fit in LDS
    t[:, 512:] = np.where(t[:, 512:] >= 0, t[:, 512:] % 600, -1)
    pf = torch.from_numpy(t).to(DEV)
    assert _check_plan(pf, n_src) == 2
    torch.manual_seed(5)
    x, _ = _q(torch.randn(n_src, C), dtype)
    w, _ = _q(torch.randn(K, kv, C) * 0.05, dtype)
    planned, direct = _both(x, w, None, False, pf, M)
    assert torch.equal(planned, direct)


@pytest.mark.parametrize("kv", [81, 125, 343])
def test_plan_many_offsets(kv):
    """kv above 64: the build finds a tile's live offsets first (by a scan of
    its entries, or from the rows' mask words) and lists only those, at most
    64; tiles with more are overflow tiles.  The table: every row pairs at
    the centre offset, ~0.3 other pairs per row, and rows 0..299 pair at half
    of all offsets within 700 sources (their tiles: too many offsets, but few
    distinct rows).  Checked against numpy in natural order and in mask order
    (tiles of like masks: most hold one or two offsets, the tiles of rows
    0..299 overflow), the latter built both ways."""
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(kv)
    M, n_src = 3000, 4000
    t = rng.integers(0, n_src, size=(kv, M)).astype(np.int32)
    t[rng.random((kv, M)) > 0.3 / kv] = -1
    t[kv // 2] = rng.permutation(n_src)[:M]
    t[:, :300] = np.where(rng.random((kv, 300)) < 0.5, t[kv // 2, :300] % 700, -1)
    t[kv // 2, :300] = rng.integers(0, 700, 300)
    pf = torch.from_numpy(t).to(DEV)
    tiles = (M + TILE - 1) // TILE
    assert _check_plan(pf.clone(), n_src) >= 2  # (rows 0..299)
    order, words = gemm.mask_order(pf, with_words=True)
    perm = gemm.permute_table(pf, order)
    n_a = _check_plan(perm.clone(), n_src)
    n_b = _check_plan(perm.clone(), n_src, words)
    assert n_a == n_b and 1 <= n_a < tiles


def _planned_vs_direct(a, w, pairs, M, plan, dtype):
    """The direct kernel (no plan) and the planned kernels (staged, thin, thin
    with every heavy tile split over four workgroups) over a table in its own
    row order, through the C ABI: [direct, staged, thin, split]."""
    from spconv_triton.pytorch._impl import _lib, gemm

    L = _lib.lib()
    K, kv, C = w.shape[0], pairs.shape[0], w.shape[-1]
    packed = gemm.packed_weight(w, None, dtype, False)
    dt = _lib.dtype_code(dtype)
    s = _lib.stream_of(a.device)
    ident = torch.arange(M, dtype=torch.int32, device=DEV)
    outs = []
    for mode in ("direct", "staged", "thin", "split"):
        out = torch.full((M, K), float("nan"), dtype=dtype, device=DEV)
        if mode == "direct":
            rc = L.sp_conv_gemm_packed(_lib.ptr(a), dt, a.shape[0], _lib.ptr(packed), K, kv, C, 0,
                                       0, _lib.ptr(pairs), M, None, None, _lib.ptr(out), dt, s)
        else:
            rc = L.sp_conv_gemm_ordered(_lib.ptr(a), dt, a.shape[0], _lib.ptr(packed), K, kv, C,
                                        0, 0, _lib.ptr(pairs), M, _lib.ptr(ident),
                                        _lib.ptr(plan), plan.numel(),
                                        {"staged": 0, "thin": 1, "split": 2}[mode], None, 0,
                                        _lib.ptr(out), dt, s)
        _lib.check(rc, mode)
        outs.append(out)
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_planned_tiles_within_one_offset_group(dtype):
    """kv = 81: the direct kernel sums a row's offsets 64 at a time, each group
    over all reduction chunks, the planned kernels a tile's items chunk by
    chunk.  The plan therefore lists only tiles whose items lie in one group
    of 64 offsets; a tile with items in both ({13, 40, 67}, as the time
    neighbours of a 4-D submanifold table; {63, 64}; 22 items) or with more
    than 64 items is an overflow tile, gathered directly.  Tiles in group 0
    ({13, 40}; 32 items) and group 1 ({64}; {70, 80}; 11 items) are staged or
    thin, plus one item only and one tile with no pair; each tile's sources
    lie in a window of 250 rows.  C = 96 spans several chunks in every dtype.
    The staged and the thin kernel (12 workgroups: its quarter instance)
    equal the direct kernel bit for bit."""
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(5)
    kv, n_src, C, K = 81, 3000, 96, 64
    sets = [[13, 40, 67], [13, 40], [63, 64], [64], list(range(1, 12)) + list(range(65, 76)),
            list(range(0, 64, 2)), list(range(70)), [70, 80], [], list(range(65, 76)), [40],
            [13, 40, 67]]
    spans = {0, 2, 4, 6, 11}
    M = TILE * len(sets) - 77  # a partial last tile
    t = np.full((kv, TILE * len(sets)), -1, dtype=np.int32)
    for ti, ks in enumerate(sets):
        for k in ks:
            live = rng.random(TILE) < 0.7
            # sources in a window of 250 rows: the tile's rows fit the thin layout
            src = ti * 200 + rng.integers(0, 250, TILE)
            t[k, ti * TILE:(ti + 1) * TILE] = np.where(live, src, -1)
    t[:, M:] = -1
    pf = torch.from_numpy(np.ascontiguousarray(t[:, :M])).to(DEV)
    assert _check_plan(pf.clone(), n_src) == len(spans)
    P = _parse(gemm.gather_plan(pf, n_src), kv, M)
    for ti in range(len(sets)):
        assert (P["count"][ti] == LDS_ROWS) == (ti in spans), f"tile {ti}"
    torch.manual_seed(7)
    x, _ = _q(torch.randn(n_src, C), dtype)
    w, _ = _q(torch.randn(K, kv, C) / np.sqrt(kv * C), dtype)
    plan = gemm.gather_plan(pf, n_src)
    direct, staged, thin, split = _planned_vs_direct(x, w, pf, M, plan, dtype)
    assert not torch.isnan(direct).any()
    assert torch.equal(staged, direct), "staged kernel differs from the direct kernel"
    assert torch.equal(thin, direct), "thin kernel differs from the direct kernel"
    assert torch.equal(split, direct), "thin kernel (every tile split) differs"


def test_planned_metric_shape():
    """The benchmark layer's shape: 200k-voxel surface cloud, 64 -> 64, fp16."""
    from bench_data import surface_cloud

    idx = surface_cloud(200_000, 256, seed=0)
    res = _tables(idx, 1, [256] * 3, [3] * 3, [1] * 3, [1] * 3, True)
    pf = res[2]
    assert _check_plan(pf, idx.shape[0]) == 0
    torch.manual_seed(0)
    x = torch.randn(idx.shape[0], 64, device=DEV).half()
    w = (torch.randn(64, 3, 3, 3, 64, device=DEV) * 0.03).half()
    b = torch.randn(64, device=DEV).half()
    planned, direct = _both(x, w, b, False, pf, pf.shape[1])
    assert torch.equal(planned, direct)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("extra", [1, 14, 48, 49])
def test_planned_tail_tiles_split(extra, dtype):
    """A one-column-block planned GEMM whose tile count exceeds the device's CU
    count by 1..48 tiles runs those last tiles in quarters by the direct path
    (the staged kernel's SPLIT instances; 49 does not split).  The result is
    bit-identical to the unplanned GEMM, the last tile partial included."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    M = (cus + extra) * 256 - 17
    rng = np.random.default_rng(500 + extra)
    grid = 64
    idx = rand_indices(rng, 1, [grid] * 3, M)
    res = _tables(idx, 1, [grid] * 3, [3] * 3, [1] * 3, [1] * 3, True)
    pf = res[2]
    assert pf.shape[1] == M
    torch.manual_seed(extra)
    x, _ = _q(torch.randn(M, 48), dtype)
    w, _ = _q(torch.randn(64, 27, 48) / np.sqrt(27 * 48), dtype)
    b, _ = _q(torch.randn(64) * 0.1, dtype)
    planned, direct = _both(x, w, b, False, pf, M)
    assert torch.equal(planned, direct)


# ---------------------------------------------------------------------------
# row order: the GEMM over the rows in mask-argsort order
# ---------------------------------------------------------------------------

def test_table_stats_and_permute():
    """sp_table_stats counts pairs (sources in range only) and live (tile,
    offset) / (64-row block, offset) pairs; sp_permute_table gathers columns."""
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(31)
    for kv, M, n_src, p in [(27, 1000, 5000, 0.2), (125, 700, 300, 0.03), (8, 1, 10, 1.0),
                            (27, 512, 900, 0.0)]:
        t = _random_table(rng, kv, M, n_src, p)
        if M > 10:
            t[3, 5:9] = n_src + 2  # out of range: not a pair
        tn = t.cpu().numpy()
        ok = (tn >= 0) & (tn < n_src)
        got = gemm.table_stats(t, n_src)
        pad = lambda b: np.pad(ok, ((0, 0), (0, -M % b))).reshape(kv, -1, b).any(axis=2).sum()
        assert got == (int(ok.sum()), int(pad(256)), int(pad(64))), (kv, M, got)
        order_np = rng.permutation(M).astype(np.int32)
        perm = gemm.permute_table(t, torch.from_numpy(order_np).to(DEV))
        np.testing.assert_array_equal(perm.cpu().numpy(), tn[:, order_np])
        if kv <= 32:
            # with the rows' mask words the empty entries are not read
            bits = ((tn[:, order_np] >= 0).astype(np.uint64)
                    << np.arange(kv, dtype=np.uint64)[:, None]).sum(0).astype(np.uint32)
            words = torch.from_numpy(bits.view(np.int32).reshape(M, 1)).to(DEV)
            perm_w = gemm.permute_table(t, torch.from_numpy(order_np).to(DEV), words)
            np.testing.assert_array_equal(perm_w.cpu().numpy(), tn[:, order_np])


def _orders(a, w, bias, transpose, pairs, M):
    """The GEMM in natural and in mask row order, planned and unplanned."""
    from spconv_triton.pytorch._impl import gemm

    N = w.shape[-1] if transpose else w.shape[0]
    outs = {}
    prev = gemm.ROW_ORDER, gemm.USE_GATHER_PLAN, gemm.THIN_TILES
    for mode, use, thin in (("natural", True, "auto"), ("natural", False, "auto"),
                            ("mask", True, False), ("mask", False, "auto"),
                            ("mask", True, True), ("mask", True, 2)):
        gemm.ROW_ORDER, gemm.USE_GATHER_PLAN, gemm.THIN_TILES = mode, use, thin
        try:
            out = torch.empty((M, N), dtype=a.dtype, device=DEV)
            gemm._gemm(a, w, bias, transpose, pairs, M, None, None, out)
            key = {True: (mode, use, "thin"), 2: (mode, use, "split")}.get(thin, (mode, use))
            outs[key] = out
        finally:
            gemm.ROW_ORDER, gemm.USE_GATHER_PLAN, gemm.THIN_TILES = prev
    return outs


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("case", ["subm", "strided", "kv125", "kv125_chunks", "kv175", "kv245",
                                  "sparse_wide", "transposed", "subm_long"])
def test_mask_row_order_bit_identical(case, dtype):
    """Every row sums its offsets in ascending order whatever tile it falls in,
    so the mask-ordered GEMM (staged, overflow and direct tiles, and the thin
    kernel with the tiles it hands to the direct path, whole or in quarters)
    equals the natural-order one bit for bit, forward and input gradient.
    subm_long: a forward grid of 1 175 workgroups (5 column blocks), where the
    16-bit thin kernel gives its direct tiles to direct_tile, and a dgrad grid
    of 235, where it splits them into quarters.  kv125_chunks: 125 offsets
    (two of the direct kernel's groups of 64) over several reduction chunks,
    where only tiles whose items lie in one group are planned.  kv175 and
    kv245 (5 x 5 x 7 and 5 x 7 x 7 windows): three and four groups, on a
    sparse cloud (a few live offsets per wave) and a dense one."""
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(44)
    ks, C, K = 3, 32, 48
    transpose = False
    if case == "subm":
        grid, n, stride = 28, 6000, 1
    elif case == "strided":
        grid, n, stride = 28, 5000, 2
    elif case == "kv125":
        grid, n, stride, ks = 20, 2500, 1, 5
    elif case == "kv125_chunks":
        grid, n, stride, ks, C, K = 40, 2000, 1, 5, 96, 64
    elif case == "kv175":  # sparse
        grid, n, stride, ks, C, K = 30, 500, 1, (5, 5, 7), 40, 48
    elif case == "kv245":  # dense
        grid, n, stride, ks, C, K = 24, 2000, 1, (5, 7, 7), 72, 48
    elif case == "subm_long":
        grid, n, stride, C, K = 48, 60000, 1, 32, 320
    elif case == "transposed":  # about one pair per output: thin tiles; 2 column blocks
        grid, n, stride, C, K, transpose = 30, 800, 2, 48, 96, True
    else:  # wide layer; in mask order 18 of the 47 tiles overflow LDS
        grid, n, stride, C, K = 40, 6000, 1, 136, 128
    idx = rand_indices(rng, 2, [grid] * 3, n)
    subm = stride == 1
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops
    ksz = list(ks) if isinstance(ks, tuple) else [ks] * 3
    res = ops.get_indice_pairs_implicit_gemm(torch.from_numpy(idx).to(DEV), 2, [grid] * 3,
                                             ConvAlgo.MaskImplicitGemm, ksz, [stride] * 3,
                                             [0 if transpose else k // 2 for k in ksz], [1] * 3,
                                             [0] * 3, subm, transpose, is_train=True)
    pf, pb = res[2], res[3]
    kv = int(np.prod(ksz))
    torch.manual_seed(3)
    x, _ = _q(torch.randn(idx.shape[0], C), dtype)
    w, _ = _q(torch.randn(K, kv, C) / np.sqrt(kv * C), dtype)
    b, _ = _q(torch.randn(K) * 0.1, dtype)
    for what, a, bias, tr, table, M in (("forward", x, b, False, pf, pf.shape[1]),
                                        ("dgrad", None, None, True, pb, idx.shape[0])):
        if a is None:
            a, _ = _q(torch.randn(pf.shape[1], K), dtype)
        outs = _orders(a, w, bias, tr, table, M)
        ref = outs[("natural", True)]
        for key, o in outs.items():
            assert torch.equal(o, ref), f"{what} {key} differs from the natural planned GEMM"
    if case == "transposed":
        P = int((pf >= 0).sum())
        assert P <= 1.1 * pf.shape[1], "the case must have about one pair per row"
    if case == "kv125_chunks":
        plan = getattr(pf, "_spconv_triton_order")[1][2]
        # a mask-ordered kv > 64 plan is kept only while at most half its tiles
        # overflow (here most tiles hold offsets of both groups of 64)
        tiles = (pf.shape[1] + 255) // 256
        assert plan is None or gemm.plan_overflow_count(plan) <= \
            gemm.ORDERED_PLAN_MAX_OVERFLOW * tiles
    if case == "sparse_wide":
        variant = getattr(pf, "_spconv_triton_order")[1]
        plan = variant[2]
        assert gemm.plan_overflow_count(plan) > 0, "the case must exercise overflow tiles"
        np.testing.assert_array_equal(variant[1].cpu().numpy(),
                                      pf.cpu().numpy()[:, variant[0].cpu().numpy()])


def test_auto_row_order_decision():
    """auto: only wide layers on tables whose natural tiles are mostly empty
    are reordered.  Narrow layers never look at the table, and the first wide
    call on a table launches nothing; the second decides."""
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(8)
    # (voxels, grid, reordered): 30000 in 100^3 has 1.7 pairs per row, yet
    # nearly every offset has a pair in each natural tile (6.5 % of the MFMA
    # work is on pairs) and the mask order cuts the work to 23 %; in 40^3 the
    # mask order only cuts it to 66 %; 20^3 is dense (67 % on pairs); in
    # 200^3 rows are isolated and the table has 12 tiles: 37 % of the natural
    # work is on pairs, and the mask order would cut it only to 94 %
    for n, grid, sparse in ((30000, 100, True), (6000, 40, False), (6000, 20, False),
                            (3000, 200, False)):
        idx = rand_indices(rng, 1, [grid] * 3, n)
        pf = _tables(idx, 1, [grid] * 3, [3] * 3, [1] * 3, [1] * 3, True)[2]
        assert gemm.row_order_variant(pf, n, 64 * 64) is None
        assert getattr(pf, "_spconv_triton_order", None) is None, "narrow layers decide nothing"
        assert gemm.row_order_variant(pf, n, 128 * 128) is None
        assert pf._spconv_triton_order[1] == "seen", "a first wide call launches nothing"
        variant = gemm.row_order_variant(pf, n, 128 * 128)
        assert (variant is not None) == sparse
        if sparse:
            assert gemm.row_order_variant(pf, n, 64 * 64) is variant, "decision is memoised"
        else:
            assert pf._spconv_triton_order[1] == "natural"


def test_row_order_decision_for_fp32_operands(monkeypatch):
    """IEEE fp32 operands count the work per live (64-row block, offset) pair:
    on the LiDAR-like cloud (3.27 pairs per row) the mask order cuts that to
    about half, so an fp32 layer takes it, while a 16-bit one (256-row tile
    count: 50 %) takes it only through the band for sparse tables of 27 or
    more offsets.  The mask-ordered fp32 forward equals the natural one bit
    for bit and the fp64 oracle on sampled rows."""
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops
    from spconv_triton.pytorch._impl import gemm

    from bench_data import lidar_cloud

    shape = [41, 1600, 1408]
    idx = lidar_cloud(50000, batch=1, seed=0, shape=shape)
    t = torch.from_numpy(idx).to(DEV)

    def table():
        return ops.get_indice_pairs_implicit_gemm(t, 1, shape, ConvAlgo.MaskImplicitGemm, [3] * 3,
                                                  [1] * 3, [1] * 3, [1] * 3, [0] * 3, True, False,
                                                  is_train=False)[2]

    n = idx.shape[0]
    C = K = 128
    p16 = table()
    assert gemm.row_order_variant(p16, n, C * K, fp32=False) is None
    assert isinstance(gemm.row_order_variant(p16, n, C * K, fp32=False), tuple)
    monkeypatch.setattr(gemm, "ORDER_SPARSE_MIN_KV", 28)  # the band off for kv = 27
    p16 = table()
    for _ in range(2):
        assert gemm.row_order_variant(p16, n, C * K, fp32=False) is None
    assert p16._spconv_triton_order[1] == "natural"
    pf = table()
    assert gemm.row_order_variant(pf, n, C * K, fp32=True) is None  # the first call: "seen"
    variant = gemm.row_order_variant(pf, n, C * K, fp32=True)
    assert isinstance(variant, tuple), "the fp32 layer did not take the mask order"
    order = variant[0]
    assert torch.equal(torch.sort(order.long())[0], torch.arange(n, device=DEV))
    torch.manual_seed(5)
    x = torch.randn(n, C, device=DEV)
    w = torch.randn(K, 27, C, device=DEV) / np.sqrt(27 * C)
    out = gemm.conv_forward(x, w, pf, n)
    prev = gemm.ROW_ORDER
    gemm.ROW_ORDER = "natural"
    try:
        ref = gemm.conv_forward(x, w, table(), n)
    finally:
        gemm.ROW_ORDER = prev
    assert torch.equal(out, ref)
    rows = np.sort(np.random.default_rng(5).choice(n, 600, replace=False))
    want = orc.gemm_fwd(x.cpu().numpy(), w.cpu().numpy(), pf.cpu().numpy()[:, rows])
    got = out[torch.from_numpy(rows).to(DEV)].double().cpu().numpy()
    assert np.abs(got - want).max() <= 1e-5 * max(1.0, float(np.abs(want).max()))  # fp32 rtol


def test_row_order_decided_at_first_use_for_one_pair_per_row():
    """A transposed convolution of sparse voxels has about one pair per output
    row, and its rulebook is usually used once: the row order is decided at
    its first wide call from the pair count its generation returned (no
    "seen" step), the mask order is taken, and the forward equals the
    natural-order one bit for bit.  A narrow layer decides nothing."""
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(21)
    n, grid = 30000, 300
    t = torch.from_numpy(rand_indices(rng, 1, [grid] * 3, n)).to(DEV)

    def table():
        return ops.get_indice_pairs_implicit_gemm(t, 1, [grid] * 3, ConvAlgo.MaskImplicitGemm,
                                                  [3] * 3, [2] * 3, [0] * 3, [1] * 3, [0] * 3,
                                                  False, True, is_train=False)[2]

    pf = table()
    kv, M = pf.shape
    P = int((pf >= 0).sum())
    assert pf._spconv_triton_npairs == P
    C = K = 256
    assert P <= gemm.FIRST_USE_MAX_PAIRS_PER_ROW * M and M * kv * C * K >= gemm.FIRST_USE_MIN_MACS
    torch.manual_seed(3)
    x = torch.randn(n, C, device=DEV).half()
    w = (torch.randn(K, kv, C, device=DEV) / np.sqrt(kv * C)).half()
    assert gemm.row_order_variant(pf, n, 64 * 64) is None
    assert getattr(pf, "_spconv_triton_order", None) is None, "narrow layers decide nothing"
    out = gemm.conv_forward(x, w, pf, M)
    assert isinstance(pf._spconv_triton_order[1], tuple), "decided at the first wide call"
    order = pf._spconv_triton_order[1][0]
    assert torch.equal(torch.sort(order.long())[0], torch.arange(M, device=DEV))
    prev = gemm.ROW_ORDER
    gemm.ROW_ORDER = "natural"
    try:
        ref = gemm.conv_forward(x, w, table(), M)
    finally:
        gemm.ROW_ORDER = prev
    assert torch.equal(out, ref)


def test_row_order_decision_waits_out_graph_capture():
    """A wide sparse layer captured into a HIP graph at its second call (when
    the decision would read counters back) captures the natural-order GEMM;
    its replays equal the eager result, and the next eager call settles the
    mask order with the same result."""
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(8)
    n, grid, C, K = 30000, 100, 128, 128
    idx = rand_indices(rng, 1, [grid] * 3, n)
    pf = _tables(idx, 1, [grid] * 3, [3] * 3, [1] * 3, [1] * 3, True)[2]
    torch.manual_seed(2)
    x = torch.randn(n, C, device=DEV).half()
    w = (torch.randn(K, 27, C, device=DEV) / np.sqrt(27 * C)).half()
    eager = gemm.conv_forward(x, w, pf, n)  # first wide call: nothing launched
    assert pf._spconv_triton_order[1] == "seen"
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            out = gemm.conv_forward(x, w, pf, n)
    torch.cuda.current_stream().wait_stream(s)
    assert pf._spconv_triton_order[1] == "seen", "capture must not advance the decision"
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    settled = gemm.conv_forward(x, w, pf, n)
    assert isinstance(pf._spconv_triton_order[1], tuple), "the next eager call settles"
    assert torch.equal(settled, eager)


@pytest.mark.parametrize("case", ["wide_1024", "subm4d"])
def test_mask_row_order_full_size(case):
    """The stress configurations at their stated sizes: SubMConv3d 256 -> 256 on
    a 400k-voxel 1024^3 surface cloud (staged kernel, overflow tiles in mask
    order) and SubMConv4d 3^4 128 -> 128 at ~500k voxels (kv = 81: direct
    kernel).  The mask-ordered forward equals the natural one bit for bit, the
    rulebook and every 40th output row match the oracle, and the automatic
    rule picks the mask order for both."""
    from bench_data import surface_cloud
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops
    from spconv_triton.pytorch._impl import gemm

    if case == "wide_1024":
        idx = surface_cloud(400000, 1024, seed=0)
        shape, ks, C = [1024] * 3, [3] * 3, 256
    else:
        rng = np.random.default_rng(0)
        base = surface_cloud(8000, 512, seed=3)[:, 1:].astype(np.int64)
        rows = []
        for t in range(64):
            c = np.clip(base + (np.array([t // 8, t // 16, t // 4]) % 512), 0, 511)
            c = c[rng.random(c.shape[0]) < 0.98]
            rows.append(np.concatenate([np.zeros((c.shape[0], 1), np.int64),
                                        np.full((c.shape[0], 1), t), c], 1))
        idx = np.unique(np.concatenate(rows).astype(np.int32), axis=0)
        shape, ks, C = [64, 512, 512, 512], [3] * 4, 128
    nd = len(shape)
    res = ops.get_indice_pairs_implicit_gemm(torch.from_numpy(idx).to(DEV), 1, shape,
                                             ConvAlgo.MaskImplicitGemm, ks, [1] * nd, [1] * nd,
                                             [1] * nd, [0] * nd, True, False, is_train=False)
    pf = res[2]
    n = idx.shape[0]
    kv = pf.shape[0]
    torch.manual_seed(1)
    x = torch.randn(n, C, device=DEV).half()
    w = (torch.randn(C, kv, C, device=DEV) / np.sqrt(kv * C)).half()
    outs = {}
    for mode in ("natural", "mask"):
        gemm.ROW_ORDER = mode
        try:
            outs[mode] = gemm.conv_forward(x, w, pf, n)
        finally:
            gemm.ROW_ORDER = "auto"
    assert torch.equal(outs["natural"], outs["mask"])
    order = gemm.mask_order(pf)
    assert torch.equal(torch.sort(order.long())[0], torch.arange(n, device=DEV)), \
        "the mask order must be a permutation of the rows"
    # both configurations against the oracle at their stated sizes: the
    # rulebook (pair table, sorted masks and argsort) bit for bit -- int64
    # keys for the 4-D grid -- and every 40th output row of the GEMM
    from spconv_triton.pytorch._impl import pairs as P

    assert P.key_is_int64(1, shape, shape, True) == (case == "subm4d")
    exp = orc.igemm_pairs(idx, 1, shape, ks, [1] * nd, [1] * nd, [1] * nd, [0] * nd, True,
                          False, False)
    np.testing.assert_array_equal(pf.cpu().numpy(), exp[2])
    np.testing.assert_array_equal(res[4][0].cpu().numpy(), exp[4][0])
    np.testing.assert_array_equal(res[6][0].cpu().numpy(), exp[6][0])
    rows = torch.arange(0, n, 40, device=DEV)
    ref = orc.gemm_fwd(x.double().cpu().numpy(), w.double().cpu().numpy(),
                       pf[:, rows].cpu().numpy())
    for mode in ("natural", "mask"):
        out = outs[mode][rows].double().cpu().numpy()
        bad = np.abs(out - ref) > 1e-3 * np.abs(ref) + 1e-5
        assert not bad.any(), f"{mode}: {int(bad.sum())} of {bad.size} beyond the fp16 bound"
    pf2 = pf.clone()  # a fresh table: the automatic rule decides at its second wide call
    assert gemm.row_order_variant(pf2, n, C * C) is None
    assert gemm.row_order_variant(pf2, n, C * C) is not None


@pytest.mark.parametrize("M", [1, 63, 255, 257, 1000])
def test_mask_row_order_partial_tiles(M):
    """Ordered GEMM on tables whose last tile is partial (rows past M must not
    be written through the order) and on a single row, staged and direct."""
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(M)
    kv, n_src, C, K = 27, 700, 40, 72
    t = rng.integers(0, n_src, size=(kv, M)).astype(np.int32)
    t[rng.random((kv, M)) > 0.3] = -1
    pf = torch.from_numpy(t).to(DEV)
    torch.manual_seed(M)
    x, _ = _q(torch.randn(n_src, C), torch.float16)
    w, _ = _q(torch.randn(K, kv, C) * 0.05, torch.float16)
    outs = _orders(x, w, None, False, pf, M)
    ref = outs[("natural", True)]
    for key, o in outs.items():
        assert torch.equal(o, ref), f"{key} differs from the natural planned GEMM"


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_graph_replay_reads_updated_weights(dtype):
    """A forward + input gradient captured into a HIP graph after eager warm-up
    (packed weights cached) must read the weight's current values on every
    replay: after w.copy_(new) the replays equal an eager call with the new
    weight (the pack kernel is part of the graph)."""
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(12)
    n, grid, C, K = 6000, 40, 32, 48
    idx = rand_indices(rng, 1, [grid] * 3, n)
    res = _tables(idx, 1, [grid] * 3, [3] * 3, [1] * 3, [1] * 3, True)
    pf, pb = res[2], res[3]
    torch.manual_seed(5)
    x = torch.randn(n, C, device=DEV).to(dtype)
    gout = torch.randn(n, K, device=DEV).to(dtype)
    w = torch.nn.Parameter((torch.randn(K, 3, 3, 3, C, device=DEV) / np.sqrt(27 * C)).to(dtype))
    b = torch.nn.Parameter(torch.randn(K, device=DEV).to(dtype))
    for _ in range(2):  # warm-up: fills the packed-weight cache
        gemm.conv_forward(x, w, pf, n, bias=b)
        gemm.conv_backward_input(gout, w, pb, n)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            y = gemm.conv_forward(x, w, pf, n, bias=b)
            dx = gemm.conv_backward_input(gout, w, pb, n)
    torch.cuda.current_stream().wait_stream(s)
    for step in range(3):
        with torch.no_grad():
            w.copy_((torch.randn(K, 3, 3, 3, C, device=DEV) / np.sqrt(27 * C)).to(dtype))
            b.copy_(torch.randn(K, device=DEV).to(dtype))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ey = gemm.conv_forward(x, w, pf, n, bias=b)
        edx = gemm.conv_backward_input(gout, w, pb, n)
        torch.cuda.synchronize()
        assert torch.equal(y, ey), f"replay {step}: forward used stale weights"
        assert torch.equal(dx, edx), f"replay {step}: dgrad used stale weights"


def test_key_order_for_unordered_rows():
    """Rows in no spatial order (a random permutation of a surface cloud) make
    every natural tile overflow LDS; the table's second planned GEMM sorts its
    rows by linear key and reruns through the ordered kernel.  Results stay
    bit-identical: to the first (natural-order) call, to the unplanned kernel,
    and, row for row, to the same layer on the sorted cloud."""
    import bench_data
    from spconv_triton.pytorch._impl import gemm

    sorted_idx = bench_data.surface_cloud(120_000, 192, seed=4)
    perm = np.random.default_rng(4).permutation(sorted_idx.shape[0])
    idx = np.ascontiguousarray(sorted_idx[perm])
    n = idx.shape[0]
    pf = _tables(idx, 1, [192] * 3, [3] * 3, [1] * 3, [1] * 3, True)[2]
    pf_sorted = _tables(sorted_idx, 1, [192] * 3, [3] * 3, [1] * 3, [1] * 3, True)[2]
    torch.manual_seed(5)
    x_sorted = torch.randn(n, 64, device=DEV).half()
    x = x_sorted[torch.from_numpy(perm).to(DEV)].contiguous()
    w = (torch.randn(64, 27, 64, device=DEV) / np.sqrt(27 * 64)).half()
    b = torch.randn(64, device=DEV).half()
    first = gemm.conv_forward(x, w, pf, n, b)
    assert pf._spconv_triton_keyorder[1] == "seen"
    second = gemm.conv_forward(x, w, pf, n, b)
    variant = pf._spconv_triton_keyorder[1]
    assert isinstance(variant, tuple), "mostly overflowing tiles must settle the key order"
    order = variant[0].cpu().numpy()
    keys = np.ravel_multi_index(idx[:, 1:].T, [192] * 3)
    assert np.array_equal(keys[order], np.sort(keys))
    assert gemm.plan_overflow_count(variant[2]) == 0
    assert torch.equal(first, second)
    prev = gemm.USE_GATHER_PLAN
    gemm.USE_GATHER_PLAN = False
    try:
        direct = gemm.conv_forward(x, w, pf, n, b)
    finally:
        gemm.USE_GATHER_PLAN = prev
    assert torch.equal(second, direct)
    ref = gemm.conv_forward(x_sorted, w, pf_sorted, n, b)
    assert torch.equal(second, ref[torch.from_numpy(perm).to(DEV)])
    # the sorted cloud's own table keeps its natural order
    gemm.conv_forward(x_sorted, w, pf_sorted, n, b)
    assert pf_sorted._spconv_triton_keyorder[1] == "natural"
