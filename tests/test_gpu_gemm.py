"""GPU parity of the MFMA gather-GEMM (forward, input gradient, weight gradient)
against the CPU oracle's fp64 restatement of reference ``_impl/gemm.py``.

Tolerances (written per test):
* fp32 inputs: |out - ref| <= 1e-5 * max(1, max|ref|)  (north-star rtol 1e-5);
* fp16 inputs: |out - ref| <= 1e-3 * |ref| + 1e-5       (north-star rtol 1e-3;
  fp16 output rounding alone is 4.9e-4 relative);
* bf16 inputs: |out - ref| <= 8e-3 * |ref| + 1e-4       (bf16 output rounding
  is 3.9e-3 relative).
The oracle receives the exact values the GPU sees (inputs rounded to the
storage dtype first), so the bound covers accumulation + output rounding only.
The masked path must be bit-identical to the dense path.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL = {
    torch.float32: lambda ref: 1e-5 * max(1.0, float(np.abs(ref).max())),
    torch.float16: lambda ref: 1e-3 * np.abs(ref) + 1e-5,
    torch.bfloat16: lambda ref: 8e-3 * np.abs(ref) + 1e-4,
}


def rand_indices(rng, batch, shape, n):
    vol = int(np.prod(shape))
    rows = []
    for b in range(batch):
        lin = rng.choice(vol, size=min(n, vol), replace=False)
        c = np.stack(np.unravel_index(lin, shape), 1)
        rows.append(np.concatenate([np.full((c.shape[0], 1), b), c], 1))
    idx = np.concatenate(rows, 0).astype(np.int32)
    return idx[rng.permutation(idx.shape[0])]


def _tables(idx, batch, shape, ks, st, pad, subm):
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    res = ops.get_indice_pairs_implicit_gemm(torch.from_numpy(idx).to(DEV), batch, shape,
                                             ConvAlgo.MaskImplicitGemm, ks, st, pad, [1] * 3,
                                             [0] * 3, subm, False, is_train=True)
    return res


def _check(out, ref, dtype, what):
    out = out.detach().float().cpu().double().numpy()
    tol = TOL[dtype](ref)
    err = np.abs(out - ref)
    bad = err > tol
    assert not bad.any(), (f"{what}: {int(bad.sum())}/{bad.size} beyond tolerance, "
                           f"max err {err.max():.3e}")


def _q(t, dtype):
    """Round to the storage dtype and return (gpu tensor, fp64 numpy of the same values)."""
    g = t.to(DEV, dtype)
    return g, g.detach().double().cpu().numpy()


CASES = [
    # (C, K, n, subm, stride)
    (64, 64, 6000, True, 1),
    (16, 16, 3000, True, 1),
    (3, 32, 2000, True, 1),
    (32, 64, 5000, False, 2),
    (64, 128, 4000, True, 1),
    (6, 16, 2500, False, 2),
    (128, 96, 3000, True, 1),
    (40, 24, 2500, True, 1),
    # wide layers: the weight gradient takes 128 x 128 (c, n) blocks
    (128, 256, 2500, True, 1),
    (256, 136, 3000, False, 2),
    (130, 128, 2000, True, 1),  # rows not a whole number of 16-byte vectors
    (32, 20, 2500, True, 1),  # input rows vectors, gradient rows not
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("ci", range(len(CASES)))
def test_forward_matches_oracle(ci, dtype):
    from spconv_triton.pytorch._impl import gemm

    C, K, n, subm, stride = CASES[ci]
    rng = np.random.default_rng(50 + ci)
    shape = [28, 28, 28]
    idx = rand_indices(rng, 2, shape, n)
    res = _tables(idx, 2, shape, [3] * 3, [stride] * 3, [1] * 3, subm)
    pf = res[2]
    n_out = pf.shape[1]
    torch.manual_seed(ci)
    x, xn = _q(torch.randn(idx.shape[0], C), dtype)
    w, wn = _q(torch.randn(K, 3, 3, 3, C) / np.sqrt(27 * C), dtype)
    b, bn = _q(torch.randn(K) * 0.1, dtype)
    ref = orc.gemm_fwd(xn, wn.reshape(K, 27, C), pf.cpu().numpy(), bn)
    out = gemm.conv_forward(x, w, pf, n_out, bias=b)
    assert out.dtype == dtype and out.shape == (n_out, K)
    _check(out, ref, dtype, "dense forward")
    pm, ar = res[4][0][:, 0], res[6][0]
    outm = gemm.conv_forward(x, w, pf, n_out, bias=b, pair_mask=pm, mask_argsort=ar)
    assert torch.equal(outm, out), "masked path must equal the dense path bit for bit"


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_forward_output_dtype(out_dtype):
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(3)
    idx = rand_indices(rng, 1, [20] * 3, 2000)
    pf = _tables(idx, 1, [20] * 3, [3] * 3, [1] * 3, [1] * 3, True)[2]
    x, xn = _q(torch.randn(idx.shape[0], 16), torch.float16)
    w, wn = _q(torch.randn(32, 3, 3, 3, 16) * 0.05, torch.float16)
    ref = orc.gemm_fwd(xn, wn.reshape(32, 27, 16), pf.cpu().numpy())
    out = gemm.conv_forward(x, w, pf, pf.shape[1], out_dtype=out_dtype)
    assert out.dtype == out_dtype
    _check(out, ref, torch.float16, "forward out dtype")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("ci", [0, 1, 3, 5, 6, 8, 9, 10, 11])
def test_dgrad_and_wgrad_match_oracle(ci, dtype):
    from spconv_triton.pytorch._impl import gemm

    C, K, n, subm, stride = CASES[ci]
    rng = np.random.default_rng(70 + ci)
    shape = [28, 28, 28]
    idx = rand_indices(rng, 2, shape, n)
    res = _tables(idx, 2, shape, [3] * 3, [stride] * 3, [1] * 3, subm)
    pf, pb = res[2], res[3]
    n_out = pf.shape[1]
    torch.manual_seed(100 + ci)
    x, xn = _q(torch.randn(idx.shape[0], C), dtype)
    g, gn = _q(torch.randn(n_out, K), dtype)
    w, wn = _q(torch.randn(K, 3, 3, 3, C) / np.sqrt(27 * C), dtype)
    ref_dx = orc.gemm_dgrad(gn, wn.reshape(K, 27, C), pb.cpu().numpy())
    dx = gemm.conv_backward_input(g, w, pb, idx.shape[0])
    _check(dx, ref_dx, dtype, "dgrad dense")
    if not subm:
        pm, ar = res[5][0][:, 0], res[7][0]
        dxm = gemm.conv_backward_input(g, w, pb, idx.shape[0], pair_mask=pm, mask_argsort=ar)
        assert torch.equal(dxm, dx), "masked dgrad must equal dense dgrad"
    ref_dw = orc.gemm_wgrad(xn, gn, pf.cpu().numpy(), K, C)
    dw = gemm.conv_backward_weight(x, g, pf, (K, 27, C))
    # the weight gradient sums ~n_out/4 products per entry: scale the bound by
    # the reduction length (fp16/bf16 outputs still round once at the end)
    scale = np.sqrt(np.maximum(1.0, orc.gemm_wgrad(np.abs(xn), np.abs(gn), pf.cpu().numpy(),
                                                    K, C)))
    out = dw.float().cpu().double().numpy()
    tol = TOL[dtype](ref_dw) + 1e-6 * scale
    assert (np.abs(out - ref_dw) <= tol).all(), \
        f"wgrad max err {np.abs(out - ref_dw).max():.3e}"
    dw2 = gemm.conv_backward_weight(x, g, pf, (K, 27, C))
    assert torch.equal(dw, dw2), "weight gradient must be deterministic"


def test_adjoint_identity_fp32():
    """<G, fwd(X)> == <dgrad(G), X> == <wgrad(X, G), W> on the GPU (fp32)."""
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(9)
    idx = rand_indices(rng, 1, [24] * 3, 4000)
    res = _tables(idx, 1, [24] * 3, [3] * 3, [2] * 3, [1] * 3, False)
    pf, pb = res[2], res[3]
    torch.manual_seed(0)
    x = torch.randn(idx.shape[0], 32, device=DEV)
    w = torch.randn(48, 3, 3, 3, 32, device=DEV) * 0.05
    g = torch.randn(pf.shape[1], 48, device=DEV)
    y = gemm.conv_forward(x, w, pf, pf.shape[1])
    dx = gemm.conv_backward_input(g, w, pb, x.shape[0])
    dw = gemm.conv_backward_weight(x, g, pf, (48, 27, 32))
    a = float((g.double() * y.double()).sum())
    b = float((dx.double() * x.double()).sum())
    c = float((dw.double() * w.reshape(48, 27, 32).double()).sum())
    assert abs(a - b) <= 1e-4 * max(1.0, abs(a))
    assert abs(a - c) <= 1e-4 * max(1.0, abs(a))


def test_packed_weight_cache_invalidates_on_update():
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(2)
    idx = rand_indices(rng, 1, [16] * 3, 1500)
    pf = _tables(idx, 1, [16] * 3, [3] * 3, [1] * 3, [1] * 3, True)[2]
    x = torch.randn(idx.shape[0], 16, device=DEV)
    w = torch.nn.Parameter(torch.randn(16, 3, 3, 3, 16, device=DEV) * 0.1)
    y1 = gemm.conv_forward(x, w, pf, pf.shape[1])
    with torch.no_grad():
        w.mul_(2.0)
    y2 = gemm.conv_forward(x, w, pf, pf.shape[1])
    torch.testing.assert_close(y2, 2 * y1, rtol=1e-5, atol=1e-5)


def test_large_metric_shape_properties():
    """Metric shape (200k voxels, 64->64 fp16): linearity in the features and
    masked == dense, checks that hold at full size without the oracle."""
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops
    from spconv_triton.pytorch._impl import gemm

    from bench_data import surface_cloud

    idx = surface_cloud(200_000, 256, seed=1)
    res = ops.get_indice_pairs_implicit_gemm(torch.from_numpy(idx).to(DEV), 1, [256] * 3,
                                             ConvAlgo.MaskImplicitGemm, [3] * 3, [1] * 3,
                                             [1] * 3, [1] * 3, [0] * 3, True, is_train=False)
    pf, pm, ar = res[2], res[4][0][:, 0], res[6][0]
    torch.manual_seed(0)
    x1 = torch.randn(idx.shape[0], 64, device=DEV).half()
    x2 = torch.randn(idx.shape[0], 64, device=DEV).half()
    w = (torch.rand(64, 3, 3, 3, 64, device=DEV) * 2 - 1).mul(1 / np.sqrt(1728)).half()
    n = idx.shape[0]
    y = gemm.conv_forward(x1, w, pf, n, pair_mask=pm, mask_argsort=ar, out_dtype=torch.float32)
    yd = gemm.conv_forward(x1, w, pf, n, out_dtype=torch.float32)
    assert torch.equal(y, yd)
    y2 = gemm.conv_forward(x2, w, pf, n, pair_mask=pm, mask_argsort=ar, out_dtype=torch.float32)
    y12 = gemm.conv_forward((x1.float() + x2.float()).half(), w, pf, n, pair_mask=pm,
                            mask_argsort=ar, out_dtype=torch.float32)
    # x1 + x2 rounds to fp16 once: compare against the fp32 sum within that rounding
    err = (y12 - (y + y2)).abs().max().item()
    assert err <= 2e-2, err
    # a 5k-row slice against the oracle (rows keep all their neighbours)
    rows = torch.arange(0, n, 40, device=DEV)
    xn = x1.double().cpu().numpy()
    wn = w.double().cpu().numpy().reshape(64, 27, 64)
    ref = orc.gemm_fwd(xn, wn, pf[:, rows].cpu().numpy())
    out = y[rows].cpu().double().numpy()
    assert (np.abs(out - ref) <= 1e-5 * np.abs(ref) + 1e-5).all()


# kernel volumes above one 64-offset group of the direct kernel: (shape,
# ksize, C, K, voxels per sample, subm, stride)
WIDE_KV = [
    ([12, 12, 10, 10], [3, 3, 3, 3], 32, 48, 2500, True, 1),  # kv = 81, 4-D
    ([20, 20, 20], [5, 5, 5], 24, 40, 2500, True, 1),  # kv = 125
    ([24, 24, 24], [5, 5, 5], 16, 32, 3000, False, 2),  # kv = 125, strided
    ([10, 10, 8, 8], [3, 3, 3, 3], 128, 128, 1200, True, 1),  # kv = 81, config 5 case 1 widths
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("ci", range(len(WIDE_KV)))
def test_wide_kernel_volume_matches_oracle(ci, dtype):
    """Forward, input gradient and weight gradient with kv = 81 / 125 against
    the fp64 oracle, in natural and in mask row order (reference
    gemm.py:254-321: every offset group, including the ones past offset 63)."""
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops
    from spconv_triton.pytorch._impl import gemm

    shape, ks, C, K, n, subm, stride = WIDE_KV[ci]
    nd = len(shape)
    rng = np.random.default_rng(300 + ci)
    idx = rand_indices(rng, 2, shape, n)
    pad = [k // 2 for k in ks]
    res = ops.get_indice_pairs_implicit_gemm(torch.from_numpy(idx).to(DEV), 2, shape,
                                             ConvAlgo.MaskImplicitGemm, ks, [stride] * nd, pad,
                                             [1] * nd, [0] * nd, subm, False, is_train=True)
    pf, pb = res[2], res[3]
    kv, n_out = pf.shape
    assert kv == int(np.prod(ks)) > 64
    exp = orc.igemm_pairs(idx, 2, shape, ks, [stride] * nd, pad, [1] * nd, [0] * nd, subm,
                          False, True)
    np.testing.assert_array_equal(pf.cpu().numpy(), exp[2])
    torch.manual_seed(400 + ci)
    x, xn = _q(torch.randn(idx.shape[0], C), dtype)
    g, gn = _q(torch.randn(n_out, K), dtype)
    w, wn = _q(torch.randn(K, kv, C) / np.sqrt(kv * C), dtype)
    b, bn = _q(torch.randn(K) * 0.1, dtype)
    ref = orc.gemm_fwd(xn, wn, pf.cpu().numpy(), bn)
    ref_dx = orc.gemm_dgrad(gn, wn, pb.cpu().numpy())
    prev = gemm.ROW_ORDER
    try:
        for mode in ("natural", "mask"):
            gemm.ROW_ORDER = mode
            out = gemm.conv_forward(x, w, pf, n_out, bias=b)
            _check(out, ref, dtype, f"forward kv={kv} ({mode} order)")
            dx = gemm.conv_backward_input(g, w, pb, idx.shape[0])
            _check(dx, ref_dx, dtype, f"dgrad kv={kv} ({mode} order)")
    finally:
        gemm.ROW_ORDER = prev
    ref_dw = orc.gemm_wgrad(xn, gn, pf.cpu().numpy(), K, C)
    dw = gemm.conv_backward_weight(x, g, pf, (K, kv, C))
    scale = np.sqrt(np.maximum(1.0, orc.gemm_wgrad(np.abs(xn), np.abs(gn), pf.cpu().numpy(),
                                                    K, C)))
    tol = TOL[dtype](ref_dw) + 1e-6 * scale
    err = np.abs(dw.float().cpu().double().numpy() - ref_dw)
    assert (err <= tol).all(), f"wgrad kv={kv} max err {err.max():.3e}"
