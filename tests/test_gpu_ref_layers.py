"""The layer class of the reference's published benchmark plots, at its size,
against the fp64 oracle.

Reference plots (README.md:112-130 of the reference): K = 3, C = 256 in and
out, batch 1, ~50 000 voxels in a 41 x 1600 x 1408 grid; submanifold, strided
(k3 s2 p1) and transposed (k3 s2) convolutions, in fp16, fp32 and TF32.  The
voxels here are uniform in that grid (the reference's cloud is unpublished),
which gives about one pair per output row: with the automatic row order these
tables are taken in mask order and run the thin kernel (``gather_gemm_thin``),
in its quarter instances (fp32 operands, or 16-bit grids of at most 1 024
workgroups) and its whole-tile instances (larger 16-bit grids).  TF32 runs as
split-bf16 products (16-bit operands, a tripled reduction).

Each case asserts that the thin kernel was chosen, compares every 7th output
row of the forward and of the input gradient with ``orc.gemm_fwd`` /
``orc.gemm_dgrad`` (restating reference ``_impl/gemm.py:254-321``) and checks
that the natural row order gives the same result bit for bit.  Bounds, as in
the GEMM tests: fp16 |d| <= 1e-3 |ref| + 1e-5; fp32 |d| <= 1e-5 max(1, max
|ref|); TF32 |d| <= 1e-4 S + 1e-6 with S the oracle GEMM of |A| and |W|.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
SHAPE = [41, 1600, 1408]
C = K = 256
EVERY = 7


@pytest.fixture(scope="module")
def cloud():
    from bench_data import uniform_cloud

    return uniform_cloud(50000, SHAPE, seed=0)


def _pairs(idx, kind):
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    subm, transpose = kind == "subm", kind == "transposed"
    stride = 1 if subm else 2
    pad = 0 if transpose else 1
    res = ops.get_indice_pairs_implicit_gemm(torch.from_numpy(idx).to(DEV), 1, SHAPE,
                                             ConvAlgo.MaskImplicitGemm, [3] * 3, [stride] * 3,
                                             [pad] * 3, [1] * 3, [0] * 3, subm, transpose,
                                             is_train=True)
    return res[2], res[3]


def _operand(shape, dtype, scale=1.0):
    t = torch.randn(*shape) * scale
    if dtype == "fp16":
        t = t.half()
    return t.to(DEV)


def _check(out, ref, dtype, what, scale=None):
    out = out.detach().double().cpu().numpy()
    err = np.abs(out - ref)
    if dtype == "fp16":
        tol = 1e-3 * np.abs(ref) + 1e-5
    elif dtype == "fp32":
        tol = 1e-5 * max(1.0, float(np.abs(ref).max()))
    else:
        tol = 1e-4 * scale + 1e-6
    bad = err > tol
    assert not bad.any(), (f"{what}: {int(bad.sum())}/{bad.size} beyond the {dtype} bound, "
                           f"max err {err.max():.3e}")


def _run(fn, table, expect_thin, what):
    """The call settles the row order (a subm table at its second wide call,
    a table with about one pair per row at its first); returns the result of
    the call after that and checks which variant ran."""
    fn()
    out = fn()
    variant = getattr(table, "_spconv_triton_order", (None, None))[1]
    if expect_thin:
        assert isinstance(variant, tuple), f"{what}: the mask order was not taken"
        assert getattr(variant[1], "_spconv_triton_thin", False), \
            f"{what}: the thin kernel was not chosen"
    return out


def _natural(fn):
    from spconv_triton.pytorch._impl import gemm

    prev = gemm.ROW_ORDER
    gemm.ROW_ORDER = "natural"
    try:
        return fn()
    finally:
        gemm.ROW_ORDER = prev


@pytest.mark.parametrize("dtype", ["fp16", "fp32", "tf32"])
@pytest.mark.parametrize("kind", ["subm", "strided", "transposed"])
def test_reference_class_layer_matches_oracle(cloud, kind, dtype):
    from spconv_triton import constants
    from spconv_triton.pytorch._impl import gemm

    print(f"[ref_c256] {kind} {dtype}", flush=True)
    pf, pb = _pairs(cloud, kind)
    n_in = cloud.shape[0]
    kv, n_out = pf.shape
    assert int((pf >= 0).sum()) <= 1.1 * n_out, "the case must have about one pair per row"
    torch.manual_seed(3)
    x = _operand((n_in, C), dtype)
    w = _operand((K, kv, C), dtype, 1.0 / np.sqrt(kv * C))
    g = _operand((n_out, K), dtype)
    xn, wn, gn = (t.double().cpu().numpy() for t in (x, w, g))
    prev = constants.SPCONV_ALLOW_TF32
    constants.SPCONV_ALLOW_TF32 = dtype == "tf32"
    try:
        fwd = _run(lambda: gemm.conv_forward(x, w, pf, n_out), pf, True, f"{kind} forward")
        nat = _natural(lambda: gemm.conv_forward(x, w, pf.clone(), n_out))
        assert torch.equal(fwd, nat), "forward: mask order (thin kernel) != natural order"
        # the submanifold input gradient's table is the forward's, transposed:
        # one pair per row as well
        dx = _run(lambda: gemm.conv_backward_input(g, w, pb, n_in), pb, kind == "subm",
                  f"{kind} dgrad")
        nat = _natural(lambda: gemm.conv_backward_input(g, w, pb.clone(), n_in))
        assert torch.equal(dx, nat), "dgrad: mask order != natural order"
    finally:
        constants.SPCONV_ALLOW_TF32 = prev
    rows = np.arange(0, n_out, EVERY)
    pfn = pf.cpu().numpy()[:, rows]
    ref = orc.gemm_fwd(xn, wn, pfn)
    s = orc.gemm_fwd(np.abs(xn), np.abs(wn), pfn) if dtype == "tf32" else None
    _check(fwd[torch.from_numpy(rows).to(DEV)], ref, dtype, f"{kind} forward", s)
    rows = np.arange(0, n_in, EVERY)
    pbn = pb.cpu().numpy()[:, rows]
    ref = orc.gemm_dgrad(gn, wn, pbn)
    s = orc.gemm_dgrad(np.abs(gn), np.abs(wn), pbn) if dtype == "tf32" else None
    _check(dx[torch.from_numpy(rows).to(DEV)], ref, dtype, f"{kind} dgrad", s)


@pytest.mark.parametrize("dtype", ["fp16", "fp32", "tf32"])
def test_lidar_cloud_layer_matches_oracle(dtype):
    """The same layer (SubMConv3d 256 -> 256, 50k voxels in 41 x 1600 x 1408)
    on the LiDAR-like cloud of ``bench_data.lidar_cloud`` (3.27 pairs per
    row).  Its table takes the mask order at the second call: 16-bit operands
    (fp16, and TF32's split bf16) through the band for sparse tables of 27 or
    more offsets, run by the staged kernel, whose tiles mostly overflow LDS
    and take its direct path; fp32 through the per-64-row-block work count,
    run by the thin kernel with every heavy tile split over four workgroups.
    Every 7th output row of the forward is compared with the fp64 oracle and
    the whole output with the natural order's, bit for bit."""
    from spconv_triton import constants
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops
    from spconv_triton.pytorch._impl import gemm

    from bench_data import lidar_cloud

    print(f"[lidar_c256] {dtype}", flush=True)
    idx = lidar_cloud(50000, batch=1, seed=0, shape=SHAPE)
    pf = ops.get_indice_pairs_implicit_gemm(torch.from_numpy(idx).to(DEV), 1, SHAPE,
                                            ConvAlgo.MaskImplicitGemm, [3] * 3, [1] * 3, [1] * 3,
                                            [1] * 3, [0] * 3, True, False, is_train=False)[2]
    kv, n = pf.shape
    torch.manual_seed(4)
    x = _operand((n, C), dtype)
    w = _operand((K, kv, C), dtype, 1.0 / np.sqrt(kv * C))
    prev = constants.SPCONV_ALLOW_TF32
    constants.SPCONV_ALLOW_TF32 = dtype == "tf32"
    try:
        out = _run(lambda: gemm.conv_forward(x, w, pf, n), pf, False, "forward")
        variant = pf._spconv_triton_order[1]
        assert isinstance(variant, tuple) and variant[2] is not None, \
            "the planned mask order was not taken"
        assert not getattr(variant[1], "_spconv_triton_thin", False)
        nat = _natural(lambda: gemm.conv_forward(x, w, pf.clone(), n))
    finally:
        constants.SPCONV_ALLOW_TF32 = prev
    assert torch.equal(out, nat), "forward: mask order != natural order"
    rows = np.arange(0, n, EVERY)
    xn, wn = (t.double().cpu().numpy() for t in (x, w))
    pfn = pf.cpu().numpy()[:, rows]
    ref = orc.gemm_fwd(xn, wn, pfn)
    s = orc.gemm_fwd(np.abs(xn), np.abs(wn), pfn) if dtype == "tf32" else None
    _check(out[torch.from_numpy(rows).to(DEV)], ref, dtype, "forward", s)
