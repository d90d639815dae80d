"""Pin the CPU oracle (CPU-only; no GPU).

The oracle is the checker for every GPU parity test, so it is itself checked:

* against the reference's golden vectors (spconv 2.3.8 outputs held by the
  reference's own test data, extracted to ``tests/golden``): UNet fwd+bwd,
  SubMConv2d+SparseConv2d pipeline, max/avg pooling incl. dilation and kv=125;
* against brute-force enumeration of the rulebook on tiny dense grids, for
  subm / strided / dilated / transposed geometries;
* against closed-form literals of the reference tests (output sizes,
  max-pool zero-init quirk) and structural invariants (mask sortedness and
  stability, Native compaction order, inverse restores the input rows).
"""

import itertools

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from oracle_pipeline import build_unet, canonical_order, OTensor, run_pipeline


def _close(actual, expected, atol, msg):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{msg}: shape {a.shape} != {e.shape}"
    if a.size:
        err = float(np.abs(a - e).max())
        assert err <= atol, f"{msg}: max abs err {err:.3e} > atol {atol:.3e}"


# ---------------------------------------------------------------------------
# golden vectors
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case_id", ["unet3d_float32", "unet3d_float16"])
def test_oracle_unet_golden(golden, case_id):
    case = golden("net.pt", case_id)
    expect = case["expect"]
    fwd, named = build_unet(case["state_dict"])
    inp = case["input"]
    feats = inp["features"].to(torch.float64).clone().requires_grad_(True)
    x = OTensor(feats, inp["indices"].numpy(), inp["spatial_shape"], inp["batch_size"])
    out = fwd(x)
    assert list(out.spatial_shape) == list(expect["out_spatial_shape"])
    order = canonical_order(out.indices, out.spatial_shape)
    np.testing.assert_array_equal(out.indices[order], expect["out_indices"].numpy())
    _close(out.features.detach().numpy()[order], expect["out_features"], expect["atol_out"], "out")
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    out.features.backward(expect["grad_out"].to(torch.float64)[torch.from_numpy(inv)])
    _close(feats.grad, expect["grad_input"], expect["atol_grad_input"], "grad_input")
    for k, ginfo in expect["grad_params"].items():
        _close(named[k].grad, ginfo["grad"], ginfo["atol"], k)


@pytest.mark.parametrize("name,case_id", [
    ("misc.pt", "seq2d_mixed"),
    ("ext_pool.pt", "avgp3d_subm"),
    ("ext_pool.pt", "maxp3d_subm"),
    ("ext_pool.pt", "maxp3d_d2"),
    ("ext_pool.pt", "maxp3d_k5_kv125"),
])
def test_oracle_pipeline_golden(golden, name, case_id):
    case = golden(name, case_id)
    expect = case["expect"]
    out, feats, layers = run_pipeline(case)
    assert list(out.spatial_shape) == list(expect["out_spatial_shape"])
    order = canonical_order(out.indices, out.spatial_shape)
    np.testing.assert_array_equal(out.indices[order], expect["out_indices"].numpy())
    _close(out.features.detach().numpy()[order], expect["out_features"], expect["atol_out"], "out")
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    out.features.backward(expect["grad_out"].to(torch.float64)[torch.from_numpy(inv)])
    _close(feats.grad, expect["grad_input"], expect["atol_grad_input"], "grad_input")
    named = {}
    for li, layer in enumerate(layers):
        for k, v in layer.params().items():
            named[f"{li}.{k}"] = v
    for k, ginfo in expect["grad_params"].items():
        _close(named[k].grad, ginfo["grad"], ginfo["atol"], k)


# ---------------------------------------------------------------------------
# brute force on tiny grids
# ---------------------------------------------------------------------------

def _rand_indices(rng, batch, shape, n):
    vol = int(np.prod(shape))
    pts = []
    for b in range(batch):
        lin = rng.choice(vol, size=min(n, vol), replace=False)
        coords = np.stack(np.unravel_index(lin, shape), 1)
        pts.append(np.concatenate([np.full((coords.shape[0], 1), b), coords], 1))
    idx = np.concatenate(pts, 0).astype(np.int32)
    return idx[rng.permutation(idx.shape[0])]


def _brute_pairs(idx, shape, ksize, stride, padding, dilation, out_padding, subm, transpose):
    """Enumerate (k, j, out_coord) directly from the geometric definition."""
    ndim = len(shape)
    inputs = {tuple(r): j for j, r in enumerate(idx.tolist())}
    offs = list(itertools.product(*[range(k) for k in ksize]))
    if subm:
        out_shape = list(shape)
    elif transpose:
        out_shape = orc.get_deconv_output_size(shape, ksize, stride, padding, dilation, out_padding)
    else:
        out_shape = orc.get_conv_output_size(shape, ksize, stride, padding, dilation)
    pairs = []
    for j, row in enumerate(idx.tolist()):
        b, x = row[0], row[1:]
        for k, off in enumerate(offs):
            o = []
            ok = True
            for d in range(ndim):
                if subm:
                    v = x[d] + (ksize[d] // 2) * dilation[d] - off[d] * dilation[d]
                elif transpose:
                    v = x[d] * stride[d] - padding[d] + off[d] * dilation[d]
                else:
                    num = x[d] + padding[d] - off[d] * dilation[d]
                    if num < 0 or num % stride[d]:
                        ok = False
                        break
                    v = num // stride[d]
                if not (0 <= v < out_shape[d]):
                    ok = False
                    break
                o.append(v)
            if not ok:
                continue
            if subm and (b, *o) not in inputs:
                continue
            pairs.append((k, j, (b, *o)))
    return pairs, out_shape


GEOMS = [
    # (shape, ksize, stride, padding, dilation, out_padding, subm, transpose)
    ([9, 8, 7], [3, 3, 3], [1, 1, 1], [1, 1, 1], [1, 1, 1], [0, 0, 0], True, False),
    ([9, 8, 7], [3, 1, 5], [1, 1, 1], [0, 0, 0], [2, 1, 1], [0, 0, 0], True, False),
    ([9, 8, 7], [3, 3, 3], [2, 2, 2], [1, 1, 1], [1, 1, 1], [0, 0, 0], False, False),
    ([9, 8, 7], [2, 3, 2], [2, 1, 3], [0, 1, 1], [1, 2, 1], [0, 0, 0], False, False),
    ([6, 5, 7], [3, 3, 3], [2, 2, 2], [1, 1, 1], [1, 1, 1], [1, 0, 1], False, True),
    ([12, 11], [3, 3], [2, 2], [1, 1], [1, 1], [0, 0], False, False),
    ([10, 6, 5, 4], [3, 3, 3, 3], [1, 1, 1, 1], [1, 1, 1, 1], [1, 1, 1, 1], [0] * 4, True, False),
]


@pytest.mark.parametrize("gi", range(len(GEOMS)))
def test_oracle_pairs_brute_force(gi):
    shape, ksize, stride, padding, dilation, out_padding, subm, transpose = GEOMS[gi]
    rng = np.random.default_rng(100 + gi)
    idx = _rand_indices(rng, 2, shape, max(4, int(np.prod(shape)) // 6))
    pairs, out_shape = _brute_pairs(idx, shape, ksize, stride, padding, dilation, out_padding,
                                    subm, transpose)
    kv = int(np.prod(ksize))
    res = orc.igemm_pairs(idx, 2, shape, ksize, stride, padding, dilation, out_padding, subm,
                          transpose, True)
    out_inds, npl, pf, pb = res[0], res[1], res[2], res[3]
    if subm:
        out_keys = [tuple(r) for r in idx.tolist()]
    else:
        expect_set = sorted({p[2] for p in pairs},
                            key=lambda c: np.ravel_multi_index(c, [2, *out_shape]))
        out_keys = [tuple(r) for r in out_inds.tolist()]
        assert out_keys == expect_set, "output rows must be sorted unique keys"
    row_of = {c: r for r, c in enumerate(out_keys)}
    exp_pf = np.full((kv, len(out_keys)), -1, np.int32)
    exp_pb = np.full((kv, idx.shape[0]), -1, np.int32)
    for k, j, o in pairs:
        exp_pf[k, row_of[o]] = j
        exp_pb[k, j] = row_of[o]
    np.testing.assert_array_equal(pf, exp_pf)
    np.testing.assert_array_equal(pb, exp_pb)
    assert not npl.any()
    # Native format: per-offset ascending input rows, npl subm quirk
    n_inds, pair, n_npl = orc.native_pairs(idx, 2, shape, ksize, stride, padding, dilation,
                                           out_padding, subm, transpose)
    for k in range(kv):
        js = [j for (kk, j, o) in pairs if kk == k]
        cnt = len(js)
        np.testing.assert_array_equal(pair[0, k, :cnt], np.array(js, np.int32))
        np.testing.assert_array_equal(pair[1, k, :cnt], exp_pb[k, js])
        assert (pair[:, k, cnt:] == -1).all()
        assert n_npl[k] == (cnt if (not subm or k < kv // 2) else 0)
    # native -> tables round trip equals the igemm tables
    t_pf, t_pb = orc.native_pair_to_tables(pair, idx.shape[0], len(out_keys), False)
    np.testing.assert_array_equal(t_pf, exp_pf)
    np.testing.assert_array_equal(t_pb, exp_pb)
    # inverse swap restores the input side
    i_pf, i_pb = orc.native_pair_to_tables(pair, len(out_keys), idx.shape[0], True)
    np.testing.assert_array_equal(i_pf, exp_pb)
    np.testing.assert_array_equal(i_pb, exp_pf)


def test_oracle_subm_center_is_identity():
    rng = np.random.default_rng(7)
    idx = _rand_indices(rng, 3, [16, 16, 16], 300)
    res = orc.igemm_pairs(idx, 3, [16, 16, 16], [3, 3, 3], [1] * 3, [1] * 3, [1] * 3, [0] * 3,
                          True, False, False)
    np.testing.assert_array_equal(res[2][13], np.arange(idx.shape[0], dtype=np.int32))
    assert res[3] is None  # eval subm: no pair_bwd


def test_oracle_masks_sorted_stable():
    rng = np.random.default_rng(3)
    kv, n = 27, 5000
    table = np.where(rng.random((kv, n)) < 0.3, rng.integers(0, n, (kv, n)), -1).astype(np.int32)
    table[:, :2000] = np.where(rng.random((kv, 1)) < 0.5, 1, -1)  # many ties
    pms, args = orc.mask_splits(table, orc.split_masks(kv, False))
    pm, ar = pms[0][:, 0].astype(np.int64) & 0xFFFFFFFF, args[0]
    bits = np.zeros(n, np.int64)
    for k in range(kv):
        bits |= (table[k] >= 0).astype(np.int64) << k
    expect_order = np.argsort(bits, kind="stable")
    np.testing.assert_array_equal(ar, expect_order)
    np.testing.assert_array_equal(pm, bits[expect_order])


def test_oracle_masks_multiword_and_split():
    rng = np.random.default_rng(4)
    kv, n = 125, 3000
    table = np.where(rng.random((kv, n)) < 0.1, 1, -1).astype(np.int32)
    pms, args = orc.mask_splits(table, orc.split_masks(kv, False))
    words = np.zeros((n, 4), np.int64)
    for k in range(kv):
        words[:, k // 32] |= (table[k] >= 0).astype(np.int64) << (k % 32)
    order = np.lexsort([words[:, w] for w in range(4)])  # last key (word 3) most significant
    np.testing.assert_array_equal(args[0], order)
    np.testing.assert_array_equal(pms[0].astype(np.int64) & 0xFFFFFFFF, words[order])
    m = orc.split_masks(27, True)
    assert [int(v[0]) for v in m] == [(1 << 14) - 1, ((1 << 13) - 1) << 14]
    # the unsigned order must survive the int32 wrap: bit 31 set sorts last
    t2 = np.full((32, 3), -1, np.int32)
    t2[31, 0] = 5
    t2[0, 1] = 5
    pms2, args2 = orc.mask_splits(t2, orc.split_masks(32, False))
    np.testing.assert_array_equal(args2[0], [2, 1, 0])
    assert pms2[0][2, 0] == np.int32(-2 ** 31)


def test_oracle_output_sizes():
    f = orc.get_conv_output_size
    assert f([32, 32, 32], [3, 3, 3], [2, 2, 2], [1, 1, 1], [1, 1, 1]) == [16, 16, 16]
    assert f([7, 8], [3, 3], [2, 2], [1, 1], [1, 1]) == [4, 4]
    assert f([24], [3], [1], [2], [2]) == [24]
    assert f([13, 7], [-1, 3], [1, 1], [0, 0], [1, 1]) == [1, 5]
    assert f([10], [2], [2], [0], [1]) == [5]
    g = orc.get_deconv_output_size
    assert g([16, 16, 16], [2, 2, 2], [2, 2, 2], [0, 0, 0], [1, 1, 1], [0, 0, 0]) == [32, 32, 32]
    assert g([16], [3], [2], [1], [1], [1]) == [32]
    with pytest.raises(ValueError):
        g([8], [-1], [1], [0], [1], [0])


def test_oracle_maxpool_zero_init_quirk():
    idx = np.array([[0, 0, 0, 0], [0, 0, 0, 1], [0, 4, 4, 4], [0, 4, 4, 5]], np.int32)
    feats = np.array([[-1.0], [-2.0], [3.0], [-0.5]], np.float32)
    res = orc.igemm_pairs(idx, 1, [8, 8, 8], [2] * 3, [2] * 3, [0] * 3, [1] * 3, [0] * 3, False, False, True)
    out = orc.maxpool_fwd(feats, res[2])
    order = np.argsort(res[0][:, 1], kind="stable")
    np.testing.assert_array_equal(out[order, 0], [0.0, 3.0])


def test_oracle_gemm_against_dense_conv():
    """fp64 gather-GEMM == dense torch conv3d on a tiny fully-occupied grid."""
    rng = np.random.default_rng(11)
    S, C, K = 5, 3, 4
    coords = np.stack(np.meshgrid(*[np.arange(S)] * 3, indexing="ij"), -1).reshape(-1, 3)
    idx = np.concatenate([np.zeros((coords.shape[0], 1)), coords], 1).astype(np.int32)
    X = rng.standard_normal((idx.shape[0], C))
    W = rng.standard_normal((K, 3, 3, 3, C))
    res = orc.igemm_pairs(idx, 1, [S] * 3, [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3, True, False, True)
    out = orc.gemm_fwd(X, W.reshape(K, 27, C), res[2])
    dense = torch.from_numpy(X.T.reshape(1, C, S, S, S))
    wt = torch.from_numpy(W).permute(0, 4, 1, 2, 3)  # [K, C, kz, ky, kx]
    ref = torch.nn.functional.conv3d(dense, wt, padding=1)[0].reshape(K, -1).T.numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)
    # wgrad / dgrad are the adjoints of fwd: <G, fwd(X, W)> == <dgrad(G), X> == <wgrad(X, G), W>
    G = rng.standard_normal(out.shape)
    lhs = float((G * out).sum())
    dX = orc.gemm_dgrad(G, W.reshape(K, 27, C), res[3])
    dW = orc.gemm_wgrad(X, G, res[2], K, C)
    assert abs(lhs - float((dX * X).sum())) < 1e-9 * max(1.0, abs(lhs))
    assert abs(lhs - float((dW * W.reshape(K, 27, C)).sum())) < 1e-9 * max(1.0, abs(lhs))


def test_oracle_gemm_fwd_f32_matches_fp64():
    """The fp32 gather-GEMM (timed as bench.py's CPU baseline) against the fp64
    one pinned above: same pairs, bias and layout, within fp32 accumulation
    error, |out32 - out64| <= 1e-5 * S + 1e-6 with S = sum |x||w| (the fp64
    GEMM of |X| and |W|).  A dropped offset, a transposed weight or a missing
    bias moves entries by O(S) and fails the bound; the random table has empty
    entries (-1) and rows without any pair."""
    rng = np.random.default_rng(12)
    n_in, n_out, C, K, kv = 700, 500, 24, 40, 27
    pf = rng.integers(0, n_in, size=(kv, n_out)).astype(np.int32)
    pf[rng.random((kv, n_out)) > 0.35] = -1
    pf[:, 17] = -1  # a row without any pair: bias only
    X = rng.standard_normal((n_in, C)).astype(np.float32)
    W = rng.standard_normal((K, kv, C)).astype(np.float32)
    b = rng.standard_normal(K).astype(np.float32)
    ref = orc.gemm_fwd(X, W, pf, b)
    out = orc.gemm_fwd_f32(X, W, pf, b)
    assert out.dtype == np.float32 and out.shape == (n_out, K)
    S = orc.gemm_fwd(np.abs(X), np.abs(W), pf)
    err = np.abs(out.astype(np.float64) - ref)
    assert (err <= 1e-5 * S + 1e-6).all(), f"max err/S {(err / np.maximum(S, 1e-30)).max():.2e}"
    np.testing.assert_array_equal(out[17], b)
    no_bias = orc.gemm_fwd_f32(X, W, pf)
    np.testing.assert_array_equal(no_bias[17], np.zeros(K, np.float32))


def _canon_voxels(idx, vox, npv):
    """Voxels sorted by coordinate, points inside a voxel sorted
    lexicographically (the reference's canonical form, tests/helpers.py:442-465)."""
    idx = np.asarray(idx, np.int64)
    vox = np.asarray(vox, np.float64)
    npv = np.asarray(npv, np.int64)
    if idx.shape[0] == 0:
        return idx, vox, npv
    maxc = int(idx.max()) + 2
    key = np.zeros(idx.shape[0], np.int64)
    for d in range(idx.shape[1]):
        key = key * maxc + idx[:, d]
    order = np.argsort(key, kind="stable")
    idx, vox, npv = idx[order], vox[order].copy(), npv[order]
    for i in range(vox.shape[0]):
        n = int(min(npv[i], vox.shape[1]))
        pts = vox[i, :n]
        pkey = pts[:, 0].copy()
        for d in range(1, pts.shape[1]):
            pkey = pkey * 131071.0 + pts[:, d]
        vox[i, :n] = pts[np.argsort(pkey, kind="stable")]
    return idx, vox, npv


@pytest.mark.parametrize("case_id", ["p2v_cpu_basic", "p2v_cpu_trunc", "p2v_cpu_cap",
                                     "p2v1d_basic", "p2v4d_basic"])
def test_oracle_point_to_voxel_golden(golden, case_id):
    """The oracle's voxelisation against spconv 2.3.8's (the reference's
    goldens): bitwise for the first-come-first-served CPU cases, in the
    reference's canonical form for the others."""
    case = golden("ext_p2v.pt", case_id)
    ctor = case["ctor"]
    vox, idx, npv, pcvid = orc.point_to_voxel(
        case["points"].numpy(), ctor["vsize_xyz"], ctor["coors_range_xyz"],
        ctor["num_point_features"], ctor["max_num_voxels"], ctor["max_num_points_per_voxel"])
    expect = case["expect"]
    if case["kind"] == "p2v_cpu":
        np.testing.assert_array_equal(idx, expect["indices"].numpy())
        np.testing.assert_array_equal(npv, expect["num_per_voxel"].numpy())
        np.testing.assert_array_equal(pcvid, expect["pc_voxel_id"].numpy())
        np.testing.assert_array_equal(vox, expect["voxels"].numpy())
    else:
        ic, vc, nc = _canon_voxels(idx, vox, npv)
        np.testing.assert_array_equal(ic, expect["indices_canon"].numpy())
        np.testing.assert_array_equal(nc, expect["num_per_voxel_canon"].numpy())
        if expect["check_contents"]:
            np.testing.assert_allclose(vc, expect["voxels_canon"].numpy(), atol=1e-5, rtol=0)


@pytest.mark.parametrize("case_id", ["sparse_add", "sparse_add_hash_based",
                                     "add_table_misaligned"])
def test_oracle_sparse_add_golden(golden, case_id):
    case = golden("misc.pt", case_id)
    a, b = case["inputs"]
    shape = [a["batch_size"], *a["spatial_shape"]]
    ind, feats = orc.hash_sparse_add([a["indices"].numpy(), b["indices"].numpy()],
                                     [a["features"].numpy(), b["features"].numpy()], shape)
    expect = case["expect"]
    order = canonical_order(ind, a["spatial_shape"])
    np.testing.assert_array_equal(order, np.arange(ind.shape[0]))  # already ascending
    np.testing.assert_array_equal(ind, expect["out_indices"].numpy())
    np.testing.assert_allclose(feats, expect["out_features"].numpy(), atol=expect["atol_out"],
                               rtol=0)


@pytest.mark.parametrize("gi", [2, 3, 4, 5])
def test_oracle_num_out_act_bound_subset(gi):
    """num_out_act_bound B (reference pairs.py:318-323, its own check is the
    subset property of tests/test_ext_conv.py:62-80): the bounded outputs
    are the first B unbounded ones, pair_fwd is the unbounded table's first B
    columns, pair_bwd the unbounded one with entries >= B set to -1, and the
    masks are those of the bounded tables.  Subm ignores the bound."""
    shape, ksize, stride, padding, dilation, out_padding, subm, transpose = GEOMS[gi]
    rng = np.random.default_rng(500 + gi)
    idx = _rand_indices(rng, 2, shape, max(4, int(np.prod(shape)) // 5))
    args = (idx, 2, shape, ksize, stride, padding, dilation, out_padding, subm, transpose, True)
    full = orc.igemm_pairs(*args)
    n_full = full[0].shape[0]
    for bound in (1, n_full // 3, n_full - 1, n_full, n_full + 5):
        res = orc.igemm_pairs(*args, num_out_act_bound=bound)
        b = min(bound, n_full)
        np.testing.assert_array_equal(res[0], full[0][:b])
        np.testing.assert_array_equal(res[2], full[2][:, :b])
        np.testing.assert_array_equal(res[3], np.where(full[3] < b, full[3], -1))
        bits = ((res[2] >= 0).astype(np.int64) << np.arange(res[2].shape[0])[:, None]).sum(0)
        order = np.argsort(bits, kind="stable")
        np.testing.assert_array_equal(res[6][0], order)
        bwd_bits = ((res[3] >= 0).astype(np.int64) << np.arange(res[3].shape[0])[:, None]).sum(0)
        np.testing.assert_array_equal(res[7][0], np.argsort(bwd_bits, kind="stable"))
    sub = GEOMS[0]
    s_args = (idx[:50], 2, sub[0], *sub[1:6], True, False, True)
    np.testing.assert_array_equal(orc.igemm_pairs(*s_args, num_out_act_bound=3)[2],
                                  orc.igemm_pairs(*s_args)[2])


@pytest.mark.parametrize("kv", [27, 125])
def test_oracle_masks_unsorted(kv):
    """do_sort=False (reference pairs.py:386-388): the raw mask words of every
    row in row order (word 0 ANDed with the split mask), the identity argsort."""
    rng = np.random.default_rng(kv)
    n = 2000
    table = np.where(rng.random((kv, n)) < 0.3, 1, -1).astype(np.int32)
    mic = (kv + 31) // 32
    words = np.zeros((n, mic), np.int64)
    for k in range(kv):
        words[:, k // 32] |= (table[k] >= 0).astype(np.int64) << (k % 32)
    splits = orc.split_masks(kv, kv <= 32)
    pms, args = orc.mask_splits(table, splits, do_sort=False)
    assert len(pms) == len(splits)
    for m, pm, ar in zip(splits, pms, args):
        exp = words.copy()
        exp[:, 0] &= int(m[0])
        np.testing.assert_array_equal(ar, np.arange(n, dtype=np.int32))
        np.testing.assert_array_equal(pm.astype(np.int64) & 0xFFFFFFFF, exp)
