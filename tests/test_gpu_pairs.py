"""GPU parity of rulebook generation: HIP hash pair generator vs the CPU oracle.

Everything here is integer work, so the bar is bit-exact: output coordinates
and their order, pair_fwd / pair_bwd tables, Native [2, kv, N] lists and npl,
sorted mask words and mask argsort (reference ``_impl/pairs.py``).
Covers subm / strided / dilated / transposed geometries in 1-4 D, kv up to 125
(multi-word masks), MaskSplit, num_out_act_bound, the int64 key path (with an
int32 translation-invariance check), batch independence and the error cases.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"

# (spatial shape, ksize, stride, padding, dilation, out_padding, subm, transpose)
GEOMS = [
    ([20, 18, 16], [3, 3, 3], [1] * 3, [1] * 3, [1] * 3, [0] * 3, True, False),
    ([20, 18, 16], [3, 1, 5], [1] * 3, [0] * 3, [2, 1, 1], [0] * 3, True, False),
    ([20, 18, 16], [3, 3, 3], [2] * 3, [1] * 3, [1] * 3, [0] * 3, False, False),
    ([20, 18, 16], [2, 3, 2], [2, 1, 3], [0, 1, 1], [1, 2, 1], [0] * 3, False, False),
    ([12, 10, 14], [3, 3, 3], [2] * 3, [1] * 3, [1] * 3, [1, 0, 1], False, True),
    ([12, 10, 14], [2, 2, 2], [2] * 3, [0] * 3, [1] * 3, [0] * 3, False, True),
    ([40, 36], [3, 3], [2, 2], [1, 1], [1, 1], [0, 0], False, False),
    ([40, 36], [5, 5], [1, 1], [2, 2], [1, 1], [0, 0], True, False),
    ([300], [3], [1], [1], [1], [0], True, False),
    ([300], [4], [3], [1], [1], [0], False, False),
    ([10, 8, 7, 6], [3, 3, 3, 3], [1] * 4, [1] * 4, [1] * 4, [0] * 4, True, False),
    ([16, 16, 16], [5, 5, 5], [1] * 3, [2] * 3, [1] * 3, [0] * 3, True, False),
    ([16, 16, 16], [5, 5, 5], [2] * 3, [2] * 3, [1] * 3, [0] * 3, False, False),
    ([16, 16, 16], [2, 2, 2], [2] * 3, [0] * 3, [1] * 3, [0] * 3, False, False),
    # 4-D subm whose leading dimension has kernel 5 and dilation 2 (the
    # brick index's 3x3x3 probe then runs 5 leading slices)
    ([9, 8, 7, 6], [5, 3, 3, 3], [1] * 4, [4, 1, 1, 1], [2, 1, 1, 1], [0] * 4, True, False),
]


def rand_indices(rng, batch, shape, n):
    vol = int(np.prod(shape))
    rows = []
    for b in range(batch):
        lin = rng.choice(vol, size=min(n, vol), replace=False)
        c = np.stack(np.unravel_index(lin, shape), 1)
        rows.append(np.concatenate([np.full((c.shape[0], 1), b), c], 1))
    idx = np.concatenate(rows, 0).astype(np.int32)
    return idx[rng.permutation(idx.shape[0])]


def _eq(a, b, what):
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape, f"{what}: shape {a.shape} != {b.shape}"
    bad = int((a != b).sum())
    assert bad == 0, f"{what}: {bad}/{a.size} entries differ"


def _igemm(idx, batch, g, is_train, split=False, bound=-1):
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    shape, ks, st, pad, dil, op, subm, tr = g
    algo = ConvAlgo.MaskSplitImplicitGemm if split else ConvAlgo.MaskImplicitGemm
    t = torch.from_numpy(idx).to(DEV)
    res = ops.get_indice_pairs_implicit_gemm(t, batch, shape, algo, ks, st, pad, dil, op, subm,
                                             tr, is_train=is_train, num_out_act_bound=bound)
    exp = orc.igemm_pairs(idx, batch, shape, ks, st, pad, dil, op, subm, tr, is_train,
                          is_mask_split=split, num_out_act_bound=bound)
    return res, exp, t


def _compare_igemm(res, exp, t, subm, is_train):
    if subm:
        assert res[0] is t, "subm must return the input indices object"
    else:
        _eq(res[0], exp[0], "out_indices")
    _eq(res[1], exp[1], "indice_num_per_loc")
    _eq(res[2], exp[2], "pair_fwd")
    if is_train:
        _eq(res[3], exp[3], "pair_bwd")
    else:
        assert res[3].numel() == 0
    for name, i in (("pair_mask_fwd", 4), ("pair_mask_bwd", 5), ("mask_argsort_fwd", 6),
                    ("mask_argsort_bwd", 7)):
        assert len(res[i]) == len(exp[i]), name
        for a, b in zip(res[i], exp[i]):
            _eq(a, b, name)
    assert [int(m[0]) for m in res[8]] == [int(m[0]) for m in exp[8]]


@pytest.mark.parametrize("is_train", [True, False])
@pytest.mark.parametrize("gi", range(len(GEOMS)))
def test_igemm_pairs_bit_exact(gi, is_train):
    g = GEOMS[gi]
    rng = np.random.default_rng(1000 + gi)
    idx = rand_indices(rng, 3, g[0], max(8, int(np.prod(g[0])) // 5))
    res, exp, t = _igemm(idx, 3, g, is_train)
    _compare_igemm(res, exp, t, g[6], is_train)


def _subm_uses_dense_grid(batch, shape, ks, n):
    """Whether sp_pairgen_subm takes its dense cell -> row grid (workspace of
    one int32 per cell) rather than the coordinate hash."""
    from spconv_triton.pytorch._impl import _lib

    g = _lib.make_geom(_lib.SP_PAIR_SUBM, batch, shape, shape, ks, [1] * len(shape),
                       [0] * len(shape), [1] * len(shape))
    return _lib.lib().sp_pairgen_workspace_size(g, n) == (batch * int(np.prod(shape)) + 8) * 4


SUBM_GEOMS = [i for i, g in enumerate(GEOMS) if g[6]]
CONV_GEOMS = [i for i, g in enumerate(GEOMS) if not g[6]]


def _align256(v):
    return (v + 255) // 256 * 256


def _conv_uses_bitmap(batch, g, n):
    """Whether sp_pairgen_conv_build takes its occupancy-bitmap path (int32
    keys, at most 4096 output cells per input row or 1024 per candidate): its
    workspace is then the bitmap, the word prefix, a counter and the scan's
    chunk sums."""
    from spconv_triton.pytorch._impl import _lib, pairs as P

    shape, ks, st, pad, dil, op, subm, tr = g
    out_shape = P._check_and_shape(torch.zeros(1, len(shape) + 1), shape, ks, st, pad, dil, op,
                                   False, tr)
    words = -(-batch * int(np.prod(out_shape)) // 32)
    w4 = words * 4
    size = _align256(_align256(_align256(w4) + w4) + 256) + _align256(-(-words // 4096) * 4)
    mode = _lib.SP_PAIR_TRANSPOSE if tr else _lib.SP_PAIR_REGULAR
    geom = _lib.make_geom(mode, batch, shape, out_shape, ks, st, pad, dil)
    return _lib.lib().sp_pairgen_workspace_size(geom, n) == size


@pytest.mark.parametrize("gi", CONV_GEOMS)
def test_conv_bitmap_and_hash_paths_bit_exact(gi):
    """Regular / transposed tables come from an occupancy bitmap of the
    output keys when the keys are int32 and the output volume is small next
    to the number of rows, else from the coordinate hash and a key sort; both
    must match the oracle bit for bit (output rows in ascending key order)."""
    shape, ks, st, pad, dil, op, subm, tr = GEOMS[gi]
    rng = np.random.default_rng(3000 + gi)
    n = max(8, int(np.prod(shape)) // 5)
    from spconv_triton.pytorch._impl import pairs as P

    def out_volume(sc):
        big = [x * sc for x in shape]
        return int(np.prod(P._check_and_shape(torch.zeros(1, len(shape) + 1), big, ks, st, pad,
                                              dil, op, False, tr)))

    scale = 8
    kv = int(np.prod(ks))
    while 3 * out_volume(scale) <= max(4096, 1024 * kv) * 3 * n:
        scale *= 2
    for s_ in (1, scale):
        big = [x * s_ for x in shape]
        g = (big, ks, st, pad, dil, op, subm, tr)
        idx = rand_indices(rng, 3, big, n)
        assert _conv_uses_bitmap(3, g, idx.shape[0]) == (s_ == 1)
        for is_train in (True, False):
            res, exp, t = _igemm(idx, 3, g, is_train)
            _compare_igemm(res, exp, t, False, is_train)
            # the pair count both paths return with the output count
            n_pairs = int((np.asarray(exp[2]) >= 0).sum())
            assert res[2]._spconv_triton_npairs == n_pairs
            if is_train:
                assert res[3]._spconv_triton_npairs == n_pairs
    assert _sort_drops() == 0, "a radix-sort scatter dropped positions"


@pytest.mark.parametrize("gi", SUBM_GEOMS)
def test_subm_dense_and_hash_paths_bit_exact(gi):
    """Subm tables come from a dense cell -> row grid when the key volume is
    small next to the number of rows, else from the coordinate hash; both
    must match the oracle bit for bit.  The same number of points is probed
    in the geometry's own grid (dense) and in a grid large enough per row for
    the hash (over 256 cells per row)."""
    shape, ks, st, pad, dil, op, subm, tr = GEOMS[gi]
    rng = np.random.default_rng(2000 + gi)
    n = max(8, int(np.prod(shape)) // 5)
    big_scale = 8
    while 3 * int(np.prod(shape)) * big_scale ** len(shape) <= 256 * 3 * n:
        big_scale *= 2
    for scale in (1, big_scale):
        big = [s * scale for s in shape]
        idx = rand_indices(rng, 3, big, n)
        assert _subm_uses_dense_grid(3, big, ks, idx.shape[0]) == (scale == 1)
        g = (big, ks, st, pad, dil, op, subm, tr)
        res, exp, t = _igemm(idx, 3, g, True)
        _compare_igemm(res, exp, t, True, True)


@pytest.mark.parametrize("gi", [0, 2, 3, 6, 7])
def test_mask_split_bit_exact(gi):
    g = GEOMS[gi]
    rng = np.random.default_rng(2000 + gi)
    idx = rand_indices(rng, 2, g[0], int(np.prod(g[0])) // 4)
    res, exp, t = _igemm(idx, 2, g, True, split=True)
    _compare_igemm(res, exp, t, g[6], True)


def test_mask_split_kv_over_32_raises():
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    idx = torch.from_numpy(rand_indices(np.random.default_rng(1), 1, [16] * 3, 300)).to(DEV)
    with pytest.raises(AssertionError, match="Not Implemented"):
        ops.get_indice_pairs_implicit_gemm(idx, 1, [16] * 3, ConvAlgo.MaskSplitImplicitGemm,
                                           [5] * 3, [1] * 3, [2] * 3, [1] * 3, [0] * 3, True)


@pytest.mark.parametrize("gi", [2, 4, 6, 12])
def test_num_out_act_bound(gi):
    g = GEOMS[gi]
    rng = np.random.default_rng(3000 + gi)
    idx = rand_indices(rng, 2, g[0], int(np.prod(g[0])) // 5)
    full = orc.igemm_pairs(idx, 2, *g[:8], True)
    bound = max(1, full[0].shape[0] // 3)
    res, exp, t = _igemm(idx, 2, g, True, bound=bound)
    assert res[0].shape[0] == bound
    _compare_igemm(res, exp, t, g[6], True)


@pytest.mark.parametrize("gi", range(len(GEOMS)))
def test_native_pairs_bit_exact(gi):
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    shape, ks, st, pad, dil, op, subm, tr = GEOMS[gi]
    rng = np.random.default_rng(4000 + gi)
    idx = rand_indices(rng, 2, shape, max(8, int(np.prod(shape)) // 5))
    t = torch.from_numpy(idx).to(DEV)
    out_inds, pair, npl = ops.get_indice_pairs(t, 2, shape, ConvAlgo.Native, ks, st, pad, dil,
                                               op, subm, tr)
    e_inds, e_pair, e_npl = orc.native_pairs(idx, 2, shape, ks, st, pad, dil, op, subm, tr)
    _eq(out_inds, e_inds, "out_indices")
    _eq(pair, e_pair, "pair")
    _eq(npl, e_npl, "indice_num_per_loc")
    # native -> gather tables, forward and inverse
    from spconv_triton.pytorch._impl import pairs as P

    n_out = out_inds.shape[0]
    pf, pb = P.native_pair_to_tables(pair, npl, idx.shape[0], n_out, False)
    e_pf, e_pb = orc.native_pair_to_tables(e_pair, idx.shape[0], n_out, False)
    _eq(pf, e_pf, "native pf")
    _eq(pb, e_pb, "native pb")
    ipf, ipb = P.native_pair_to_tables(pair, npl, n_out, idx.shape[0], True)
    _eq(ipf, e_pb, "inverse pf")
    _eq(ipb, e_pf, "inverse pb")
    # memoised
    pf2, _ = P.native_pair_to_tables(pair, npl, idx.shape[0], n_out, False)
    assert pf2 is pf


def _place(idx, offset):
    out = idx.copy()
    out[:, 1:] += np.asarray(offset, np.int32)
    return out


@pytest.mark.parametrize("subm", [True, False])
def test_int64_keys_match_oracle_and_int32_translation(subm):
    """Grid volume >= 2^31 selects 64-bit keys; tables equal the oracle's and
    the same cloud placed in a small (int32) grid (reference
    tests/test_int64_linearize.py:70-120)."""
    from spconv_triton.pytorch._impl import pairs as P

    rng = np.random.default_rng(7)
    small = [24, 24, 24]
    # keep the cloud off the small grid's upper faces, so that no strided
    # output is clipped there and both placements have the same outputs
    idx = rand_indices(rng, 2, [22, 22, 22], 2500)
    big_shape = [4096, 2048, 1024]
    off = [2048, 1024, 512]
    big = _place(idx, off)
    st = [1] * 3 if subm else [2] * 3
    g_small = (small, [3] * 3, st, [1] * 3, [1] * 3, [0] * 3, subm, False)
    g_big = (big_shape, [3] * 3, st, [1] * 3, [1] * 3, [0] * 3, subm, False)
    assert P.key_is_int64(2, big_shape, big_shape, subm)
    assert not P.key_is_int64(2, small, small, subm)
    res_b, exp_b, tb = _igemm(big, 2, g_big, True)
    _compare_igemm(res_b, exp_b, tb, subm, True)
    res_s, _, _ = _igemm(idx, 2, g_small, True)
    for i in (2, 3):
        _eq(res_b[i], res_s[i].cpu().numpy(), f"table {i} int64 vs int32")
    for i in (4, 5, 6, 7):
        for a, b in zip(res_b[i], res_s[i]):
            _eq(a, b.cpu().numpy(), f"mask {i} int64 vs int32")
    if not subm:
        shift = np.asarray([0] + [o // 2 for o in off], np.int32)
        _eq(res_b[0], res_s[0].cpu().numpy() + shift, "out_indices int64 vs int32")


def test_batches_are_independent():
    """Pairs of a multi-batch tensor equal the per-batch pairs (reference
    tests/test_large_batch.py:94-154)."""
    rng = np.random.default_rng(11)
    shape = [18, 18, 18]
    idx = rand_indices(rng, 4, shape, 900)
    g = (shape, [3] * 3, [2] * 3, [1] * 3, [1] * 3, [0] * 3, False, False)
    res, exp, t = _igemm(idx, 4, g, True)
    _compare_igemm(res, exp, t, False, True)
    out = res[0].cpu().numpy()
    assert (np.diff(out[:, 0]) >= 0).all(), "outputs grouped by batch"
    for b in range(4):
        sel = idx[:, 0] == b
        sub = idx[sel].copy()
        sub[:, 0] = 0
        r1, _, _ = _igemm(sub, 1, g, True)
        mine = out[out[:, 0] == b].copy()
        mine[:, 0] = 0
        _eq(r1[0], mine, f"batch {b} outputs")


def test_pairgen_deterministic():
    rng = np.random.default_rng(5)
    shape = [32, 32, 32]
    idx = rand_indices(rng, 2, shape, 5000)
    g = (shape, [3] * 3, [2] * 3, [1] * 3, [1] * 3, [0] * 3, False, False)
    a, _, _ = _igemm(idx, 2, g, True)
    b, _, _ = _igemm(idx, 2, g, True)
    for i in (0, 2, 3):
        assert torch.equal(a[i], b[i])


def test_errors():
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    empty = torch.zeros((0, 4), dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):
        ops.get_indice_pairs_implicit_gemm(empty, 1, [8] * 3, ConvAlgo.MaskImplicitGemm,
                                           [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3, True)
    one = torch.tensor([[0, 1, 1, 1]], dtype=torch.int32, device=DEV)
    with pytest.raises(NotImplementedError):
        ops.get_indice_pairs_implicit_gemm(one, 1, [8] * 3, ConvAlgo.MaskImplicitGemm, [2] * 3,
                                           [1] * 3, [0] * 3, [1] * 3, [0] * 3, True)
    # every candidate falls outside: "points vanished"
    with pytest.raises(ValueError, match="vanished"):
        # k=1, stride 2: the odd coordinate is never an exact multiple
        ops.get_indice_pairs_implicit_gemm(one, 1, [8] * 3, ConvAlgo.MaskImplicitGemm, [1] * 3,
                                           [2] * 3, [0] * 3, [1] * 3, [0] * 3, False)
    with pytest.raises(ValueError, match="reach zero"):
        ops.get_indice_pairs_implicit_gemm(one, 1, [2] * 3, ConvAlgo.MaskImplicitGemm, [5] * 3,
                                           [1] * 3, [0] * 3, [1] * 3, [0] * 3, False)


def test_large_subm_properties():
    """200k-voxel surface-like cloud: subm table invariants that hold at any size
    (centre offset is the identity; pair_bwd is pair_fwd with offsets reversed;
    masks sorted and argsort a permutation; bits equal the table)."""
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    from bench_data import surface_cloud

    idx = surface_cloud(200_000, 256, seed=0)
    t = torch.from_numpy(idx).to(DEV)
    res = ops.get_indice_pairs_implicit_gemm(t, 1, [256] * 3, ConvAlgo.MaskImplicitGemm,
                                             [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3, True,
                                             is_train=True)
    pf, pb = res[2], res[3]
    n = idx.shape[0]
    assert torch.equal(pf[13], torch.arange(n, dtype=torch.int32, device=DEV))
    assert torch.equal(pb, pf.flip(0))
    pm, ar = res[4][0][:, 0], res[6][0]
    words = pm.long() & 0xFFFFFFFF
    assert bool((words[1:] >= words[:-1]).all())
    assert torch.equal(torch.sort(ar.long())[0], torch.arange(n, device=DEV))
    bits = ((pf >= 0).long() << torch.arange(27, device=DEV)[:, None]).sum(0)
    assert torch.equal(bits[ar.long()], words)
    # spot-check against the oracle on a 20k subset of rows' neighbourhoods
    sub = idx[:20000]
    exp = orc.igemm_pairs(sub, 1, [256] * 3, [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3, True,
                          False, True)
    r2 = ops.get_indice_pairs_implicit_gemm(torch.from_numpy(sub).to(DEV), 1, [256] * 3,
                                            ConvAlgo.MaskImplicitGemm, [3] * 3, [1] * 3, [1] * 3,
                                            [1] * 3, [0] * 3, True, is_train=True)
    _eq(r2[2], exp[2], "pair_fwd 20k")
    _eq(r2[3], exp[3], "pair_bwd 20k")
    _eq(r2[4][0], exp[4][0], "pair_mask 20k")
    _eq(r2[6][0], exp[6][0], "mask_argsort 20k")


@pytest.mark.parametrize("n,grid", [(200_000, 256), (600_000, 512)])
def test_mask_sort_stable_large(n, grid):
    """The mask sort is a stable ascending sort of the mask words: at 200k rows
    (98 radix tiles) and 600k rows (293 tiles), mask_argsort equals numpy's
    stable argsort of the words that the table's bits define."""
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    from bench_data import surface_cloud

    idx = surface_cloud(n, grid, seed=3)
    t = torch.from_numpy(idx).to(DEV)
    res = ops.get_indice_pairs_implicit_gemm(t, 1, [grid] * 3, ConvAlgo.MaskImplicitGemm,
                                             [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3, True,
                                             is_train=False)
    pf = res[2].cpu().numpy()
    words = ((pf >= 0).astype(np.int64) << np.arange(27)[:, None]).sum(0)
    exp = np.argsort(words, kind="stable")
    np.testing.assert_array_equal(res[6][0].cpu().numpy(), exp)
    np.testing.assert_array_equal(res[4][0][:, 0].cpu().numpy().astype(np.int64) & 0xFFFFFFFF,
                                  words[exp])
    assert _sort_drops() == 0, "a radix-sort scatter dropped positions"


def _mask_sort(words, kv, split, ws, pm, ar):
    from spconv_triton.pytorch._impl import _lib

    n = words.shape[0]
    _lib.check(_lib.lib().sp_mask_sort(_lib.ptr(words), n, 1, kv, split, 1, _lib.ptr(pm),
                                       _lib.ptr(ar), _lib.ptr(ws), ws.numel(),
                                       _lib.stream_of(words.device)), "sp_mask_sort")


def _expect_sorted(w_np, split):
    keys = w_np.astype(np.uint64) & np.uint64(split)
    order = np.argsort(keys, kind="stable")
    return order.astype(np.int64), keys[order].astype(np.int64)


def test_mask_sort_single_word_cases():
    """Single-word mask sorts carry (key, row) pairs from pass to pass, with
    digit-major tile histograms and a per-digit prefix launch.  Against numpy's
    stable argsort: one to 160 radix tiles of 2048 rows (partial last tiles, a
    single row), 1 to 4 passes (kv 5, 9, 27, 32), a split mask, heavily
    repeated keys; every sort reuses one workspace that starts as random bytes
    (and holds the previous sort's histograms), so nothing may depend on its
    contents."""
    from spconv_triton.pytorch._impl import _lib

    rng = np.random.default_rng(5)
    L = _lib.lib()
    n_max = 160 * 2048
    ws = torch.from_numpy(rng.integers(0, 256, size=L.sp_mask_sort_workspace_size(n_max, 1),
                                       dtype=np.uint8)).to(DEV)
    cases = [(1, 27, 0xFFFFFFFF), (100, 9, 0xFFFFFFFF), (2048, 27, 0xFFFFFFFF),
             (2049, 5, 0xFFFFFFFF), (5000, 32, 0xFFFFFFFF), (70_001, 27, 0x3FFF),
             (131_072, 18, 0xFFFFFFFF), (128 * 2048 + 1, 27, 0xFFFFFFFF),
             (n_max - 3, 27, 0xFFFFFFFF), (n_max, 32, 0xFFFF0000)]
    for n, kv, split in cases:
        hi = (1 << kv) - 1
        w_np = rng.integers(0, hi + 1, size=n, dtype=np.int64)
        w_np[rng.random(n) < 0.5] &= 0x7  # many equal keys: stability matters
        words = torch.from_numpy(w_np.astype(np.uint32).view(np.int32)).to(DEV)
        pm = torch.empty(n, dtype=torch.int32, device=DEV)
        ar = torch.empty(n, dtype=torch.int32, device=DEV)
        _mask_sort(words, kv, split, ws, pm, ar)
        order, keys = _expect_sorted(w_np, split)
        np.testing.assert_array_equal(ar.cpu().numpy(), order, f"argsort n={n} kv={kv}")
        np.testing.assert_array_equal(pm.cpu().numpy().astype(np.int64) & 0xFFFFFFFF, keys,
                                      f"sorted words n={n} kv={kv}")
    assert _sort_drops() == 0, "a sort scatter dropped positions"


def test_mask_sort_graph_replays():
    """The single-word mask sort captured into a HIP graph: every replay (new
    words copied in between, eager sorts on the same workspace between replays)
    equals numpy's stable argsort."""
    from spconv_triton.pytorch._impl import _lib

    rng = np.random.default_rng(9)
    L = _lib.lib()
    n, kv = 150_000, 27
    ws = torch.empty(L.sp_mask_sort_workspace_size(n, 1), dtype=torch.uint8, device=DEV)
    words = torch.zeros(n, dtype=torch.int32, device=DEV)
    pm = torch.empty(n, dtype=torch.int32, device=DEV)
    ar = torch.empty(n, dtype=torch.int32, device=DEV)
    _mask_sort(words, kv, 0xFFFFFFFF, ws, pm, ar)  # warm-up
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            _mask_sort(words, kv, 0xFFFFFFFF, ws, pm, ar)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        w_np = rng.integers(0, 1 << kv, size=n, dtype=np.int64)
        w_np[rng.random(n) < 0.3] = 5
        words.copy_(torch.from_numpy(w_np.astype(np.int32)))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        order, keys = _expect_sorted(w_np, 0xFFFFFFFF)
        np.testing.assert_array_equal(ar.cpu().numpy(), order, f"replay {rep}")
        np.testing.assert_array_equal(pm.cpu().numpy().astype(np.int64) & 0xFFFFFFFF, keys)
        # an eager sort on the same workspace between replays
        pm2 = torch.empty_like(pm)
        ar2 = torch.empty_like(ar)
        _mask_sort(words, kv, 0xFFFFFFFF, ws, pm2, ar2)
        torch.cuda.synchronize()
        assert torch.equal(ar2, ar) and torch.equal(pm2, pm)
    assert _sort_drops() == 0


def _sort_drops() -> int:
    """Positions the radix-sort scatters dropped since the last call (0 for
    consistent histograms), then reset."""
    import ctypes

    from spconv_triton.pytorch._impl import _lib

    v = ctypes.c_uint64(0)
    _lib.check(_lib.lib().sp_sort_dropped_positions(ctypes.byref(v), 1),
               "sp_sort_dropped_positions")
    return int(v.value)


@pytest.mark.parametrize("training", [True, False])
def test_module_rulebooks_defer_mask_sorts(training):
    """Rulebooks built by the modules leave the mask sorts until a mask split is
    read (the gather-GEMM never reads them).  Forward and backward must not
    trigger them, and the values read afterwards, on the build stream or on
    another stream, equal the oracle's bit for bit."""
    import spconv_triton.pytorch as spconv

    rng = np.random.default_rng(21)
    shape = [24, 20, 18]
    idx = rand_indices(rng, 2, shape, 1500)
    t = torch.from_numpy(idx).to(DEV)
    torch.manual_seed(0)
    s1 = spconv.SubMConv3d(8, 8, 3, padding=1, indice_key="s1")
    c2 = spconv.SparseConv3d(8, 8, 3, stride=2, padding=1, indice_key="c2")
    s4 = spconv.SubMConv3d(8, 8, 3, padding=1, indice_key="s4")
    p3 = spconv.SparseMaxPool3d(2, stride=2, indice_key="p3")
    inv = spconv.SparseInverseConv3d(8, 8, 3, indice_key="c2")
    for m in (s1, c2, s4, p3, inv):
        m.to(DEV).train(training)
    feats = torch.randn(idx.shape[0], 8, device=DEV, requires_grad=training)
    h3 = s4(c2(s1(spconv.SparseConvTensor(feats, t, shape, 2))))
    pooled = p3(h3)
    y = inv(h3)
    if training:
        (y.features.square().sum() + pooled.features.sum()).backward()
    torch.cuda.synchronize()
    d = dict(y.indice_dict)
    d["p3"] = pooled.indice_dict["p3"]
    for key in ("s1", "c2", "s4", "p3"):
        assert d[key]._deferred_masks is not None, f"{key}: masks were sorted by the module"

    c2_out = d["c2"].out_indices.cpu().numpy()
    c2_shape = list(d["c2"].out_spatial_shape)
    cases = {  # key: (indices, geometry, is_train)
        "s1": (idx, (shape, [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3, True, False),
               training),
        "c2": (idx, (shape, [3] * 3, [2] * 3, [1] * 3, [1] * 3, [0] * 3, False, False), True),
        "s4": (c2_out, (c2_shape, [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3, True, False),
               training),
        "p3": (c2_out, (c2_shape, [2] * 3, [2] * 3, [0] * 3, [1] * 3, [0] * 3, False, False),
               True),
    }
    side = torch.cuda.Stream()
    for j, (key, (ind, g, is_train)) in enumerate(cases.items()):
        data = d[key]
        if j % 2:  # first read on another stream
            with torch.cuda.stream(side):
                splits = (data.pair_mask_fwd_splits, data.pair_mask_bwd_splits,
                          data.mask_argsort_fwd_splits, data.mask_argsort_bwd_splits)
            torch.cuda.current_stream().wait_stream(side)
        else:
            splits = (data.pair_mask_fwd_splits, data.pair_mask_bwd_splits,
                      data.mask_argsort_fwd_splits, data.mask_argsort_bwd_splits)
        assert data._deferred_masks is None
        shape_k, ks, st, pad, dil, op, subm, tr = g
        exp = orc.igemm_pairs(ind, 2, shape_k, ks, st, pad, dil, op, subm, tr, is_train)
        res = (data.out_indices, exp[1], data.pair_fwd, data.pair_bwd) + splits + (data.masks,)
        _compare_igemm(res, exp, data.indices if subm else None, subm, is_train)


def test_deferred_mask_splits_deepcopy():
    """A deep copy of a module-built rulebook (e.g. of a SparseConvTensor's
    indice_dict) carries the computed mask splits."""
    import copy

    import spconv_triton.pytorch as spconv

    rng = np.random.default_rng(5)
    shape = [20, 18, 16]
    idx = rand_indices(rng, 1, shape, 900)
    conv = spconv.SparseConv3d(4, 8, 3, stride=2, padding=1, indice_key="c").to(DEV)
    x = spconv.SparseConvTensor(torch.randn(idx.shape[0], 4, device=DEV),
                                torch.from_numpy(idx).to(DEV), shape, 1)
    y = conv(x)
    data = y.indice_dict["c"]
    dup = copy.deepcopy(data)
    for name in ("pair_mask_fwd_splits", "pair_mask_bwd_splits", "mask_argsort_fwd_splits",
                 "mask_argsort_bwd_splits"):
        a, b = getattr(data, name), getattr(dup, name)
        assert len(a) == len(b) > 0, name
        for u, v in zip(a, b):
            assert torch.equal(u, v) and u.data_ptr() != v.data_ptr(), name


def test_module_rulebook_pickles():
    """A SparseConvTensor whose indice_dict holds a module-built rulebook with
    deferred mask sorts pickles (the sorts run first; the copy holds their
    values), before and after the splits are read."""
    import pickle

    import spconv_triton.pytorch as spconv

    rng = np.random.default_rng(6)
    shape = [20, 18, 16]
    idx = rand_indices(rng, 1, shape, 900)
    conv = spconv.SparseConv3d(4, 8, 3, stride=2, padding=1, indice_key="c").to(DEV)
    subm = spconv.SubMConv3d(8, 8, 3, padding=1, indice_key="s").to(DEV)
    x = spconv.SparseConvTensor(torch.randn(idx.shape[0], 4, device=DEV),
                                torch.from_numpy(idx).to(DEV), shape, 1)
    y = subm(conv(x))
    for key in ("c", "s"):
        assert y.indice_dict[key]._deferred_masks is not None
    y2 = pickle.loads(pickle.dumps(y))
    assert torch.equal(y2.features, y.features) and torch.equal(y2.indices, y.indices)
    for key in ("c", "s"):
        a, b = y.indice_dict[key], y2.indice_dict[key]
        assert torch.equal(a.pair_fwd, b.pair_fwd)
        for name in ("pair_mask_fwd_splits", "mask_argsort_fwd_splits"):
            u, v = getattr(a, name), getattr(b, name)
            assert len(u) == len(v) > 0
            for s, t in zip(u, v):
                assert torch.equal(s, t), (key, name)


@pytest.mark.parametrize("subm,big_shape", [(True, [64, 512, 512, 512]),
                                            (False, [64, 1024, 1024, 1024])])
def test_int64_keys_4d_match_oracle_and_int32_translation(subm, big_shape):
    """4-D clouds in grids whose key volume exceeds 2^31 (config 5 case 1's
    [64, 512, 512, 512] for subm): 64-bit keys, tables equal to the oracle's
    and to those of the same cloud in a small int32 grid (reference
    tests/test_int64_linearize.py:70-120, pairs.py:166-171)."""
    from spconv_triton.pytorch._impl import pairs as P

    rng = np.random.default_rng(17)
    small = [16, 16, 16, 16]
    idx = rand_indices(rng, 2, [14, 14, 14, 14], 3000)
    off = [24, 200, 300, 100]  # even: strided outputs shift by off / 2
    big = _place(idx, off)
    st = [1] * 4 if subm else [2] * 4
    g_small = (small, [3] * 4, st, [1] * 4, [1] * 4, [0] * 4, subm, False)
    g_big = (big_shape, [3] * 4, st, [1] * 4, [1] * 4, [0] * 4, subm, False)
    out_big = big_shape if subm else [s // 2 for s in big_shape]
    assert P.key_is_int64(2, big_shape, out_big, subm)
    assert not P.key_is_int64(2, small, small, subm)
    for is_train in (True, False):
        res_b, exp_b, tb = _igemm(big, 2, g_big, is_train)
        _compare_igemm(res_b, exp_b, tb, subm, is_train)
    res_b, _, _ = _igemm(big, 2, g_big, True)
    res_s, _, _ = _igemm(idx, 2, g_small, True)
    for i in (2, 3):
        _eq(res_b[i], res_s[i].cpu().numpy(), f"table {i} int64 vs int32")
    for i in (4, 5, 6, 7):
        for a, b in zip(res_b[i], res_s[i]):
            _eq(a, b.cpu().numpy(), f"mask {i} int64 vs int32")
    if not subm:
        shift = np.asarray([0] + [o // 2 for o in off], np.int32)
        _eq(res_b[0], res_s[0].cpu().numpy() + shift, "out_indices int64 vs int32")


@pytest.mark.parametrize("gi", [0, 2, 4, 11])
def test_unsorted_masks_bit_exact(gi):
    """do_sort=False (reference pairs.py:386-388, SPCONV_DO_SORT=0): raw mask
    words in row order and an identity argsort, forward and backward splits,
    plain and MaskSplit, equal to the oracle."""
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    shape, ks, st, pad, dil, op, subm, tr = GEOMS[gi]
    rng = np.random.default_rng(5000 + gi)
    idx = rand_indices(rng, 2, shape, max(8, int(np.prod(shape)) // 5))
    t = torch.from_numpy(idx).to(DEV)
    kv = int(np.prod(ks))
    for split in ((False, True) if kv <= 32 else (False,)):
        algo = ConvAlgo.MaskSplitImplicitGemm if split else ConvAlgo.MaskImplicitGemm
        res = ops.get_indice_pairs_implicit_gemm(t, 2, shape, algo, ks, st, pad, dil, op, subm,
                                                 tr, is_train=True, do_sort=False)
        exp = orc.igemm_pairs(idx, 2, shape, ks, st, pad, dil, op, subm, tr, True,
                              is_mask_split=split, do_sort=False)
        _compare_igemm(res, exp, t, subm, True)
        for ar in res[6]:
            assert torch.equal(ar, torch.arange(ar.numel(), dtype=torch.int32, device=DEV))


def _subm_tables_direct(idx_t, batch, shape, ks, kept_grid):
    """pair_fwd / pair_bwd / mask words of a subm build through one of the
    two C-ABI entry points: the cleared-workspace build (sp_pairgen_subm) or
    the kept-grid build (sp_pairgen_subm_grid, through the package's grid)."""
    from spconv_triton.pytorch._impl import _lib, pairs as P

    L = _lib.lib()
    nd = len(shape)
    n = idx_t.shape[0]
    kv = int(np.prod(ks))
    g = _lib.make_geom(_lib.SP_PAIR_SUBM, batch, shape, shape, ks, [1] * nd,
                       [k // 2 for k in ks], [1] * nd)
    pf = torch.empty((kv, n), dtype=torch.int32, device=DEV)
    pb = torch.empty((kv, n), dtype=torch.int32, device=DEV)
    words = torch.empty((n, (kv + 31) // 32), dtype=torch.int32, device=DEV)
    stream = _lib.stream_of(torch.device(DEV))
    if kept_grid:
        cells = L.sp_pairgen_subm_grid_cells(g, n)
        assert cells > 0
        grid, epoch = P._subm_grid(torch.device(DEV), cells)
        npl = torch.full((kv,), 7, dtype=torch.int32, device=DEV)
        _lib.check(L.sp_pairgen_subm_grid(g, _lib.ptr(idx_t), n, _lib.ptr(pf), _lib.ptr(pb),
                                          _lib.ptr(words), _lib.ptr(npl), _lib.ptr(grid),
                                          grid.numel(), epoch, stream), "sp_pairgen_subm_grid")
        assert int(npl.abs().sum()) == 0, "npl must come back zeroed"
    else:
        ws = _lib.workspace(L.sp_pairgen_workspace_size(g, n), torch.device(DEV))
        _lib.check(L.sp_pairgen_subm(g, _lib.ptr(idx_t), n, _lib.ptr(pf), _lib.ptr(pb),
                                     _lib.ptr(words), _lib.ptr(ws), ws.numel(), stream),
                   "sp_pairgen_subm")
    return pf, pb, words


def test_subm_kept_grid_across_builds_and_epoch_wrap():
    """The kept grid is never cleared between builds: cells stamped by earlier
    builds -- of other geometries too -- must read as empty.  Builds of two
    clouds alternate across the epoch wrap (epoch 255, then a refill and
    epoch 1); every build matches the oracle and the cleared-workspace path."""
    from spconv_triton.pytorch._impl import pairs as P

    rng = np.random.default_rng(77)
    clouds = []
    for shape in ([30, 16, 26], [24, 20, 22]):  # the larger grid first: it is kept
        idx = rand_indices(rng, 2, shape, int(np.prod(shape)) // 4)
        clouds.append((shape, idx, torch.from_numpy(idx).to(DEV)))
    P.release_pairgen_grids()
    key = (torch.device(DEV).index, torch.cuda.current_stream(torch.device(DEV)).cuda_stream)
    seen = []
    for step in range(8):
        if step == 3:  # jump to the end of the epoch range
            grid, _ = P._GRIDS[key]
            P._GRIDS[key] = (grid, 253)
        shape, idx, t = clouds[step % 2]
        pf, pb, words = _subm_tables_direct(t, 2, shape, [3, 3, 3], True)
        seen.append(P._GRIDS[key][1])
        exp = orc.igemm_pairs(idx, 2, shape, [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3, True,
                              False, True)
        _eq(pf, exp[2], f"pair_fwd build {step}")
        _eq(pb, exp[3], f"pair_bwd build {step}")
        rf, rb, rw = _subm_tables_direct(t, 2, shape, [3, 3, 3], False)
        assert torch.equal(pf, rf) and torch.equal(pb, rb) and torch.equal(words, rw)
    assert seen == [1, 2, 3, 254, 255, 1, 2, 3], seen


def test_subm_duplicate_coordinates_keep_smallest_row_both_paths():
    """Duplicate coordinates are outside the reference's contract; both subm
    builds resolve a cell held by several rows to its smallest row."""
    rng = np.random.default_rng(5)
    shape = [16, 16, 16]
    idx = rand_indices(rng, 1, shape, 600)
    dup = idx[rng.choice(idx.shape[0], 80, replace=False)]
    idx = np.concatenate([idx, dup], 0)[rng.permutation(idx.shape[0] + 80)].astype(np.int32)
    t = torch.from_numpy(idx).to(DEV)
    kept = _subm_tables_direct(t, 1, shape, [3, 3, 3], True)
    cleared = _subm_tables_direct(t, 1, shape, [3, 3, 3], False)
    for a, b in zip(kept, cleared):
        assert torch.equal(a, b)
    # the centre offset of a duplicated cell names the cell's smallest row
    keys = np.ravel_multi_index(idx[:, 1:].T, shape)
    first = {}
    for r, k in enumerate(keys):
        first.setdefault(k, r)
    centre = kept[0][13].cpu().numpy()
    assert all(centre[r] == first[k] for r, k in enumerate(keys))


def test_subm_build_inside_graph_capture_replays():
    """A subm rulebook built while the stream is captured takes the clearing
    path (a replay reruns the capture's kernels with their arguments); replays
    equal the eager build."""
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    rng = np.random.default_rng(8)
    shape = [20, 20, 20]
    idx = torch.from_numpy(rand_indices(rng, 1, shape, 1500)).to(DEV)

    def build():
        return ops.get_indice_pairs_implicit_gemm(idx, 1, shape, ConvAlgo.MaskImplicitGemm,
                                                  [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3,
                                                  True, is_train=True)

    eager = build()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        build()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = build()
    for _ in range(3):
        cap[2].fill_(-5)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(cap[2], eager[2]) and torch.equal(cap[3], eager[3])
        build()  # eager work between replays
