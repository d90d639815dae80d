"""PointToVoxel, HashTable and sparse_add on the GPU.

PointToVoxel (csrc/sp_voxel.hip) is first-come-first-served, so its results
are deterministic: they must equal the reference's goldens bit for bit
(spconv 2.3.8 CPU outputs, tests/golden/ext_p2v.pt -- the reference itself
only checks its GPU path in canonical form) and the CPU oracle
(oracle.point_to_voxel, pinned by those goldens) on larger seeded clouds,
through the voxel cap, per-voxel truncation, points out of range or NaN, f64
points, 1-D and 4-D grids.  HashTable (csrc/sp_hashtable.hip) is checked
against a Python dict model of the reference's semantics (hash.py:38-110:
last write wins, ascending enumeration); sparse_add against the reference's
goldens and the oracle.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from test_oracle_golden import _canon_voxels

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _p2v(ctor, points, **kw):
    from spconv_triton.pytorch import utils as putils

    p2v = putils.PointToVoxel(device=torch.device(DEV), **ctor)
    return p2v, p2v.generate_voxel_with_id(points.to(DEV), **kw)


def _orc(ctor, points, **kw):
    return orc.point_to_voxel(points.cpu().numpy(), ctor["vsize_xyz"], ctor["coors_range_xyz"],
                              ctor["num_point_features"], ctor["max_num_voxels"],
                              ctor["max_num_points_per_voxel"], **kw)


def _eq(res, exp, what):
    vox, idx, npv, pcvid = [t.cpu().numpy() for t in res]
    evox, eidx, enpv, epcvid = exp
    np.testing.assert_array_equal(idx, eidx, err_msg=f"{what}: indices")
    np.testing.assert_array_equal(npv, enpv, err_msg=f"{what}: num_per_voxel")
    np.testing.assert_array_equal(pcvid, epcvid, err_msg=f"{what}: pc_voxel_id")
    np.testing.assert_array_equal(vox, evox, err_msg=f"{what}: voxels")


@pytest.mark.parametrize("case_id", ["p2v_cpu_basic", "p2v_cpu_trunc", "p2v_cpu_cap",
                                     "p2v1d_basic", "p2v4d_basic"])
def test_point_to_voxel_golden(golden, case_id):
    case = golden("ext_p2v.pt", case_id)
    p2v, res = _p2v(case["ctor"], case["points"])
    expect = case["expect"]
    if case["kind"] == "p2v_cpu":
        _eq(res, (expect["voxels"].numpy(), expect["indices"].numpy(),
                  expect["num_per_voxel"].numpy(), expect["pc_voxel_id"].numpy()), case_id)
    else:
        ic, vc, nc = _canon_voxels(res[1].cpu(), res[0].cpu(), res[2].cpu())
        np.testing.assert_array_equal(ic, expect["indices_canon"].numpy())
        np.testing.assert_array_equal(nc, expect["num_per_voxel_canon"].numpy())
        if expect["check_contents"]:
            np.testing.assert_allclose(vc, expect["voxels_canon"].numpy(), atol=1e-5, rtol=0)
    # the metadata the reference derives (ZYX order)
    ctor = case["ctor"]
    nd = len(ctor["vsize_xyz"])
    assert p2v.vsize == list(reversed(ctor["vsize_xyz"]))
    assert p2v.coors_range == (list(reversed(ctor["coors_range_xyz"][:nd]))
                               + list(reversed(ctor["coors_range_xyz"][nd:])))


def _cloud(n, ndim, seed, dtype=torch.float32, extra=1, spread=2.4):
    g = torch.Generator().manual_seed(seed)
    pts = (torch.rand(n, ndim + extra, generator=g, dtype=torch.float64) * 2 - 1) * spread
    # clustered points so voxels hold several points
    pts[: n // 2, :ndim] = torch.round(pts[: n // 2, :ndim] * 4) / 4 + 0.01 * pts[n // 2:n, :ndim]
    return pts.to(dtype)


CASES = [
    # (ndim, n, vsize, max_voxels, max_points, dtype)
    (3, 200_000, 0.05, 60_000, 5, torch.float32),    # cap reached, truncation
    (3, 200_000, 0.1, 200_000, 32, torch.float32),   # no cap
    (3, 50_000, 0.07, 10_000, 3, torch.float64),     # f64 points
    (1, 20_000, 0.01, 1_000, 8, torch.float32),
    (2, 30_000, 0.05, 5_000, 6, torch.float32),
    (4, 50_000, 0.2, 20_000, 4, torch.float32),
]


@pytest.mark.parametrize("ci", range(len(CASES)))
def test_point_to_voxel_matches_oracle(ci):
    ndim, n, vs, max_vox, max_pts, dtype = CASES[ci]
    pts = _cloud(n, ndim, 40 + ci, dtype)
    pts[::997, 0] = float("nan")  # NaN coordinates are out of range
    ctor = dict(vsize_xyz=[vs] * ndim, coors_range_xyz=[-2.0] * ndim + [2.0] * ndim,
                num_point_features=ndim + 1, max_num_voxels=max_vox,
                max_num_points_per_voxel=max_pts)
    _, res = _p2v(ctor, pts)
    _eq(res, _orc(ctor, pts), f"case {ci}")


def test_point_to_voxel_empty_mean():
    """empty_mean fills empty slots with the voxel's mean (the sum over all
    slots, in slot order, over the clamped count: one rounding order of the
    reference's, within 2 ulp of the oracle's numpy sum)."""
    pts = _cloud(20_000, 3, 7)
    ctor = dict(vsize_xyz=[0.1] * 3, coors_range_xyz=[-2.0] * 3 + [2.0] * 3,
                num_point_features=4, max_num_voxels=30_000, max_num_points_per_voxel=6)
    _, res = _p2v(ctor, pts, empty_mean=True)
    exp = _orc(ctor, pts, empty_mean=True)
    np.testing.assert_array_equal(res[1].cpu().numpy(), exp[1])
    np.testing.assert_allclose(res[0].cpu().numpy(), exp[0], rtol=3e-7, atol=1e-7)


def test_point_to_voxel_edge_cases():
    from spconv_triton.pytorch import utils as putils

    ctor = dict(vsize_xyz=[0.1] * 3, coors_range_xyz=[0, 0, 0, 1, 1, 1], num_point_features=3,
                max_num_voxels=10, max_num_points_per_voxel=2)
    p2v = putils.PointToVoxel(device=torch.device(DEV), **ctor)
    # no points at all, then none in range
    for pts in (torch.zeros(0, 3), torch.full((5, 3), 7.0)):
        vox, idx, npv, pcvid = p2v.generate_voxel_with_id(pts.to(DEV))
        assert vox.shape == (0, 2, 3) and idx.shape == (0, 3) and npv.shape == (0,)
        assert pcvid.shape == (pts.shape[0],) and bool((pcvid == -1).all())
    # clear_voxels=False keeps the previous call's contents in unused slots
    a = torch.tensor([[0.05, 0.05, 0.05], [0.06, 0.05, 0.05]], device=DEV)
    p2v.generate_voxel_with_id(a)
    b = torch.tensor([[0.05, 0.05, 0.05]], device=DEV)
    vox, _, npv, _ = p2v.generate_voxel_with_id(b, clear_voxels=False)
    assert int(npv[0]) == 1 and torch.equal(vox[0, 1].cpu(), a[1].cpu())
    with pytest.raises(AssertionError):
        p2v.generate_voxel_with_id(a.cpu())


def test_point_to_voxel_cap_and_truncation():
    """The reference's structural checks (tests/test_ext_p2v.py:47-85): with
    the voxel cap exactly cap voxels survive and dropped points get -1;
    points past max_points_per_voxel keep their voxel id."""
    from spconv_triton.pytorch import utils as putils

    g = torch.Generator().manual_seed(3)
    pc = torch.rand(500, 3, generator=g).to(DEV)
    p2v = putils.PointToVoxel([0.05] * 3, [0, 0, 0, 1, 1, 1], 3, 20, 4, torch.device(DEV))
    vox, idx, npv, pcvid = p2v.generate_voxel_with_id(pc)
    assert idx.shape[0] == 20 and int(pcvid.max()) == 19 and int((pcvid < 0).sum()) > 0
    valid = pcvid >= 0
    q = (pc[valid] / 0.05).floor().long().flip(1)
    assert torch.equal(idx.long()[pcvid[valid]], q)
    pc = torch.tensor([[0.05, 0.05, 0.05], [0.051, 0.05, 0.05], [0.052, 0.05, 0.05],
                       [0.3, 0.3, 0.3]], device=DEV)
    p2v = putils.PointToVoxel([0.1] * 3, [0, 0, 0, 1, 1, 1], 3, 10, 2, torch.device(DEV))
    vox, idx, npv, pcvid = p2v.generate_voxel_with_id(pc)
    counts = torch.bincount(pcvid[pcvid >= 0], minlength=idx.shape[0])
    by = {tuple(c.tolist()): int(n) for c, n in zip(idx.cpu(), counts.cpu())}
    assert by[(0, 0, 0)] == 3 and by[(3, 3, 3)] == 1
    npv_by = {tuple(c.tolist()): int(n) for c, n in zip(idx.cpu(), npv.cpu())}
    assert npv_by[(0, 0, 0)] == 2


def test_gather_features_by_pc_voxel_id():
    from spconv_triton.pytorch import utils as putils

    feats = torch.arange(12, dtype=torch.float32, device=DEV).reshape(4, 3)
    ids = torch.tensor([2, -1, 0, 3, -1], device=DEV)
    out = putils.gather_features_by_pc_voxel_id(feats, ids, invalid_value=-5)
    exp = torch.tensor([[6, 7, 8], [-5, -5, -5], [0, 1, 2], [9, 10, 11], [-5, -5, -5]],
                       dtype=torch.float32)
    assert torch.equal(out.cpu(), exp)


# ---- HashTable ---------------------------------------------------------------

class _Model:
    """The reference's semantics: a dict, last write wins, sorted enumeration."""

    def __init__(self):
        self.d = {}

    def insert(self, keys, values):
        for k, v in zip(keys, values):
            self.d[k] = v

    def query(self, keys):
        return [self.d.get(k, 0) for k in keys], [k not in self.d for k in keys]


@pytest.mark.parametrize("key_dtype,value_dtype", [(torch.int32, torch.int32),
                                                   (torch.int64, torch.int64),
                                                   (torch.int64, torch.float32),
                                                   (torch.int32, torch.float64)])
def test_hash_table_semantics(key_dtype, value_dtype):
    from spconv_triton.pytorch.hash import HashTable

    rng = np.random.default_rng(5)
    lo, hi = (-2 ** 31, 2 ** 31 - 1) if key_dtype == torch.int32 else (-2 ** 62, 2 ** 62)
    ht = HashTable(torch.device(DEV), key_dtype, value_dtype, max_size=30_000)
    model = _Model()
    pool = rng.integers(lo, hi, size=12_000)
    for rnd in range(3):
        keys = rng.choice(pool, size=9_000)  # duplicates inside and across calls
        vals = rng.integers(-1000, 1000, size=keys.size)
        ht.insert(torch.from_numpy(keys).to(key_dtype), torch.from_numpy(vals).to(value_dtype))
        model.insert(keys.tolist(), vals.tolist())
    q = np.concatenate([pool[:5000], rng.integers(lo, hi, size=2000)])
    out, empty = ht.query(torch.from_numpy(q).to(key_dtype).to(DEV))
    ev, ee = model.query(q.tolist())
    np.testing.assert_array_equal(out.cpu().double().numpy(), np.asarray(ev, np.float64))
    np.testing.assert_array_equal(empty.cpu().numpy(), np.asarray(ee))
    # insert_exist_keys updates stored keys only (last occurrence wins)
    upd = np.concatenate([pool[:100], pool[:100], rng.integers(lo, hi, size=50)])
    uv = rng.integers(2000, 3000, size=upd.size)
    found = ht.insert_exist_keys(torch.from_numpy(upd).to(key_dtype),
                                 torch.from_numpy(uv).to(value_dtype))
    np.testing.assert_array_equal(found.cpu().numpy(), [k in model.d for k in upd.tolist()])
    model.insert([k for k in upd.tolist() if k in model.d],
                 [v for k, v in zip(upd.tolist(), uv.tolist()) if k in model.d])
    # items: ascending keys, then assign_arange_ numbers them
    k, v, cnt = ht.items()
    n = int(cnt.item())
    assert n == len(model.d) and cnt.dtype == (torch.int32 if key_dtype == torch.int32
                                               else torch.int64)
    sk = sorted(model.d)
    np.testing.assert_array_equal(k[:n].cpu().numpy(), sk)
    np.testing.assert_array_equal(v[:n].cpu().double().numpy(),
                                  np.asarray([model.d[x] for x in sk], np.float64))
    assert int(ht.assign_arange_().item()) == n
    out, _ = ht.query(torch.tensor(sk, dtype=key_dtype, device=DEV))
    np.testing.assert_array_equal(out.cpu().double().numpy(), np.arange(n, dtype=np.float64))


def test_hash_table_reference_cases():
    """tests/test_ext_misc.py:14-48 of the reference, and its error paths."""
    from spconv_triton.pytorch.hash import HashTable

    dev = torch.device(DEV)
    ht = HashTable(dev, torch.int32, torch.int32, max_size=64)
    ht.insert(torch.tensor([3, 7, 11], dtype=torch.int32, device=DEV),
              torch.tensor([30, 70, 110], dtype=torch.int32, device=DEV))
    ht.insert_exist_keys(torch.tensor([7, 99], dtype=torch.int32, device=DEV),
                         torch.tensor([777, 999], dtype=torch.int32, device=DEV))
    out, empty = ht.query(torch.tensor([3, 7, 11, 99], dtype=torch.int32, device=DEV))
    assert out.cpu().tolist() == [30, 777, 110, 0] and empty.cpu().tolist() == [0, 0, 0, 1]
    ht = HashTable(dev, torch.int32, torch.int32, max_size=64)
    ht.insert(torch.tensor([5, 1, 9], dtype=torch.int32, device=DEV),
              torch.tensor([50, 10, 90], dtype=torch.int32, device=DEV))
    k, v, cnt = ht.items()
    assert int(cnt.item()) == 3 and k[:3].cpu().tolist() == [1, 5, 9]
    assert v[:3].cpu().tolist() == [10, 50, 90] and k.shape == (64,)
    k, v, cnt = ht.items(2)
    assert int(cnt.item()) == 2 and k.cpu().tolist() == [1, 5]
    with pytest.raises(AssertionError):
        HashTable(dev, torch.float32, torch.int32, max_size=8)
    with pytest.raises(AssertionError):
        HashTable(dev, torch.int32, torch.int32)
    small = HashTable(dev, torch.int32, torch.int32, max_size=4)
    with pytest.raises(AssertionError, match="full"):
        small.insert(torch.arange(5, dtype=torch.int32, device=DEV))
    big = HashTable(dev, torch.int64, torch.int32, max_size=4)
    with pytest.raises(ValueError, match="reserved"):
        big.insert(torch.tensor([2 ** 63 - 1], dtype=torch.int64, device=DEV))


# ---- sparse_add ----------------------------------------------------------------

def _sp(inp, dev=DEV):
    import spconv_triton.pytorch as spconv

    return spconv.SparseConvTensor(inp["features"].to(dev), inp["indices"].to(dev),
                                   list(inp["spatial_shape"]), int(inp["batch_size"]))


@pytest.mark.parametrize("case_id", ["sparse_add", "sparse_add_hash_based",
                                     "add_table_misaligned"])
def test_sparse_add_golden(golden, case_id):
    from spconv_triton.pytorch import functional as F
    from spconv_triton.pytorch import tables

    case = golden("misc.pt", case_id)
    xa, xb = _sp(case["inputs"][0]), _sp(case["inputs"][1])
    if case["fn"] == "sparse_add":
        out = F.sparse_add(xa, xb)
    elif case["fn"] == "sparse_add_hash_based":
        out = F.sparse_add_hash_based(xa, xb)
    else:
        out = tables.AddTableMisaligned()([xa, xb])
    expect = case["expect"]
    # rows come out in ascending key order: the canonical order itself
    assert torch.equal(out.indices.cpu(), expect["out_indices"])
    err = (out.features.cpu() - expect["out_features"]).abs().max().item()
    assert err <= expect["atol_out"]
    assert list(out.spatial_shape) == expect["out_spatial_shape"]


def test_sparse_add_three_inputs_and_grad():
    """Three operands against the oracle (features of equal coordinates added
    in input order: bit-exact), gradients route to every operand, and the
    largest operand's indice_dict is kept when no coordinate is new."""
    import spconv_triton.pytorch as spconv
    from spconv_triton.pytorch import functional as F

    from bench_data import uniform_cloud

    shape = [24, 24, 24]
    ins = []
    for s in range(3):
        idx = uniform_cloud(3000, shape, seed=20 + s, batch=2)
        f = torch.randn(idx.shape[0], 16, generator=torch.Generator().manual_seed(s))
        ins.append((idx, f))
    xs = [spconv.SparseConvTensor(f.to(DEV).requires_grad_(True), torch.from_numpy(i).to(DEV),
                                  shape, 2) for i, f in ins]
    out = F.sparse_add(*xs)
    ind, feats = orc.hash_sparse_add([i for i, _ in ins], [f.numpy() for _, f in ins],
                                     [2, *shape])
    np.testing.assert_array_equal(out.indices.cpu().numpy(), ind)
    np.testing.assert_array_equal(out.features.detach().cpu().numpy(), feats)
    out.features.sum().backward()
    for x in xs:
        assert torch.equal(x.features.grad.cpu(), torch.ones_like(x.features.grad.cpu()))
    conv = spconv.SubMConv3d(16, 16, 3, indice_key="keep").to(DEV)
    with torch.no_grad():
        y = conv(spconv.SparseConvTensor(ins[0][1].to(DEV), torch.from_numpy(ins[0][0]).to(DEV),
                                         shape, 2))
    z = F.sparse_add(y, y.replace_feature(y.features * 0.5))
    assert z.find_indice_pair("keep") is not None
