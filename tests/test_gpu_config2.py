"""Config 2 at its stated size: the reference's quickstart chain (reference
README.md:56-58) on the 200k-voxel 256^3 surface cloud, fp16 inference,
batch 1, one shared indice_key for the strided layer and its inverse:

    SubMConv3d(3 -> 32, k3, indice_key="subm0")
    SparseConv3d(32 -> 64, k3, s2, p1, indice_key="down0")
    SparseInverseConv3d(64 -> 32, k3, indice_key="down0")

Integer work bit for bit against the CPU oracle: the subm table, the strided
layer's output coordinates, pair_fwd and pair_bwd (bitmap path at this size),
and the inverse layer's output rows, which must be the input rows
(reference tests/test_conv.py:75-87).  Features layer by layer against the
oracle's fp64 gather-GEMM fed with the GPU's own fp16 input to that layer, on
every 7th output row: |out - ref| <= 1e-3 * |ref| + 1e-5 (north-star fp16
rtol; fp16 output rounding alone is 4.9e-4 relative).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
N = 200_000
GRID = 256


def _eq(a, b, what):
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)
    assert a.shape == b.shape, f"{what}: shape {a.shape} != {b.shape}"
    bad = int((a != b).sum())
    assert bad == 0, f"{what}: {bad}/{a.size} entries differ"


def _check_layer(layer, x_in, table, y, what):
    K, C = layer.weight.shape[0], layer.weight.shape[-1]
    rows = torch.arange(0, y.shape[0], 7, device=DEV)
    w = layer.weight.detach().double().cpu().numpy().reshape(K, -1, C)
    b = None if layer.bias is None else layer.bias.detach().double().cpu().numpy()
    ref = orc.gemm_fwd(x_in.detach().double().cpu().numpy(), w, table[:, rows].cpu().numpy(), b)
    out = y[rows].detach().double().cpu().numpy()
    err = np.abs(out - ref)
    bad = err > 1e-3 * np.abs(ref) + 1e-5
    assert not bad.any(), f"{what}: {int(bad.sum())}/{bad.size} beyond tolerance, max {err.max():.3e}"


def test_quickstart_chain_200k_fp16():
    import spconv_triton.pytorch as spconv

    from bench_data import surface_cloud

    idx = surface_cloud(N, GRID, seed=0)
    t = torch.from_numpy(idx).to(DEV)
    torch.manual_seed(0)
    net = spconv.SparseSequential(
        spconv.SubMConv3d(3, 32, 3, padding=1, indice_key="subm0"),
        spconv.SparseConv3d(32, 64, 3, stride=2, padding=1, indice_key="down0"),
        spconv.SparseInverseConv3d(64, 32, 3, indice_key="down0"),
    ).to(DEV).half().eval()
    feats = torch.randn(N, 3, device=DEV).half()
    with torch.no_grad():
        x = spconv.SparseConvTensor(feats, t, [GRID] * 3, 1)
        h1 = net[0](x)
        h2 = net[1](h1)
        out = net[2](h2)
        out_seq = net(spconv.SparseConvTensor(feats, t, [GRID] * 3, 1))
    for h in (h1, h2, out):
        assert h.features.dtype == torch.float16
    assert torch.equal(out_seq.features, out.features), "sequential == layer by layer"
    assert torch.equal(out_seq.indices, out.indices)

    # subm rulebook
    exp_s = orc.igemm_pairs(idx, 1, [GRID] * 3, [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3,
                            True, False, False)
    pf_s = h1.indice_dict["subm0"].pair_fwd
    _eq(pf_s, exp_s[2], "subm pair_fwd")
    # strided rulebook (output coordinates in ascending key order, both tables)
    exp_d = orc.igemm_pairs(idx, 1, [GRID] * 3, [3] * 3, [2] * 3, [1] * 3, [1] * 3, [0] * 3,
                            False, False, True)
    down = h2.indice_dict["down0"]
    _eq(h2.indices, exp_d[0], "strided out_indices")
    _eq(down.out_indices, exp_d[0], "rulebook out_indices")
    _eq(down.pair_fwd, exp_d[2], "strided pair_fwd")
    _eq(down.pair_bwd, exp_d[3], "strided pair_bwd")
    assert list(h2.spatial_shape) == [GRID // 2] * 3
    # the inverse restores the input rows, in their order
    assert torch.equal(out.indices, t)
    assert list(out.spatial_shape) == [GRID] * 3

    _check_layer(net[0], feats, pf_s, h1.features, "subm 3 -> 32")
    _check_layer(net[1], h1.features, down.pair_fwd, h2.features, "strided 32 -> 64")
    # the inverse layer's forward table is the strided layer's pair_bwd
    _check_layer(net[2], h2.features, down.pair_bwd, out.features, "inverse 64 -> 32")
