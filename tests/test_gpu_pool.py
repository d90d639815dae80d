"""GPU parity of sparse max/avg pooling against the CPU oracle (reference
``_impl/pool.py``).  Pooling reductions are tile-independent, so the bar is
bit-exact for every dtype (fp32 accumulator, fp64 for double inputs), including
the zero-init and equality-routing quirks of max-pool and the count-multiplying
avg-pool backward."""

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def rand_indices(rng, batch, shape, n):
    vol = int(np.prod(shape))
    rows = []
    for b in range(batch):
        lin = rng.choice(vol, size=min(n, vol), replace=False)
        c = np.stack(np.unravel_index(lin, shape), 1)
        rows.append(np.concatenate([np.full((c.shape[0], 1), b), c], 1))
    idx = np.concatenate(rows, 0).astype(np.int32)
    return idx[rng.permutation(idx.shape[0])]


def _tables(idx, batch, shape, ks, st, pad, dil, subm):
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    return ops.get_indice_pairs_implicit_gemm(torch.from_numpy(idx).to(DEV), batch, shape,
                                              ConvAlgo.MaskImplicitGemm, ks, st, pad, dil,
                                              [0] * 3, subm, False, is_train=True)


GEOMS = [
    ([2] * 3, [2] * 3, [0] * 3, [1] * 3, False),
    ([3] * 3, [2] * 3, [1] * 3, [1] * 3, False),
    ([3] * 3, [1] * 3, [1] * 3, [1] * 3, True),
    ([3] * 3, [1] * 3, [2] * 3, [2] * 3, True),
    ([5] * 3, [2] * 3, [2] * 3, [1] * 3, False),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("gi", range(len(GEOMS)))
@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("C", [24, 5])  # whole 16-byte pieces (vector kernels) or not
def test_maxpool_bit_exact(gi, dtype, ties, C):
    from spconv_triton.pytorch._impl import pool

    ks, st, pad, dil, subm = GEOMS[gi]
    rng = np.random.default_rng(gi * 7 + int(ties))
    idx = rand_indices(rng, 2, [22] * 3, 2500)
    res = _tables(idx, 2, [22] * 3, ks, st, pad, dil, subm)
    pf, pb = res[2], res[3]
    x = torch.randn(idx.shape[0], C)
    if ties:
        x = torch.round(x * 2) / 2  # many equal values: equality routing matters
    x = x.to(DEV, dtype)
    n_out = pf.shape[1]
    out = pool.maxpool_forward(x, pf, n_out)
    xn = x.cpu().numpy() if dtype != torch.bfloat16 else x.float().cpu().numpy()
    ref = orc.maxpool_fwd(xn, pf.cpu().numpy())
    np.testing.assert_array_equal(out.float().cpu().numpy() if dtype == torch.bfloat16
                                  else out.cpu().numpy(), ref.astype(xn.dtype))
    g = torch.randn(n_out, C).to(DEV, dtype)
    dx = pool.maxpool_backward(x, out, g, pb)
    gn = g.float().cpu().numpy() if dtype == torch.bfloat16 else g.cpu().numpy()
    on = out.float().cpu().numpy() if dtype == torch.bfloat16 else out.cpu().numpy()
    ref_dx = orc.maxpool_bwd(xn, on, gn, pb.cpu().numpy())
    if dtype in (torch.float16, torch.bfloat16):
        # oracle accumulates in fp32 and returns fp32; the GPU stores the same
        # fp32 sum rounded to the storage dtype
        ref_dx = torch.from_numpy(ref_dx).to(dtype).float().numpy()
        np.testing.assert_array_equal(dx.float().cpu().numpy(), ref_dx)
    else:
        np.testing.assert_array_equal(dx.cpu().numpy(), ref_dx)


def test_maxpool_zero_init_all_negative():
    from spconv_triton.pytorch._impl import pool

    idx = np.array([[0, 0, 0, 0], [0, 0, 0, 1], [0, 4, 4, 4], [0, 4, 4, 5]], np.int32)
    res = _tables(idx, 1, [8] * 3, [2] * 3, [2] * 3, [0] * 3, [1] * 3, False)
    x = torch.tensor([[-1.0], [-2.0], [3.0], [-0.5]], device=DEV)
    out = pool.maxpool_forward(x, res[2], res[2].shape[1])
    order = torch.argsort(res[0][:, 1].long())
    assert out[order, 0].tolist() == [0.0, 3.0]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16])
@pytest.mark.parametrize("gi", [0, 1, 2])
@pytest.mark.parametrize("C", [16, 3])
def test_avgpool_bit_exact(gi, dtype, C):
    from spconv_triton.pytorch._impl import pool

    ks, st, pad, dil, subm = GEOMS[gi]
    rng = np.random.default_rng(40 + gi)
    idx = rand_indices(rng, 2, [22] * 3, 2500)
    res = _tables(idx, 2, [22] * 3, ks, st, pad, dil, subm)
    pf, pb = res[2], res[3]
    x = torch.randn(idx.shape[0], C).to(DEV, dtype)
    n_out = pf.shape[1]
    out, count = pool.avgpool_forward(x, pf, n_out)
    ref, ref_count = orc.avgpool_fwd(x.cpu().numpy(), pf.cpu().numpy())
    np.testing.assert_array_equal(count.cpu().numpy(), ref_count)
    np.testing.assert_array_equal(out.cpu().numpy(), ref)
    g = torch.randn(n_out, C).to(DEV, dtype)
    dx = pool.avgpool_backward(g, pb, count)
    ref_dx = orc.avgpool_bwd(g.cpu().numpy(), ref_count, pb.cpu().numpy())
    np.testing.assert_array_equal(dx.cpu().numpy(), ref_dx)


def _unaligned(t: torch.Tensor) -> torch.Tensor:
    """A contiguous copy of ``t`` whose data starts one element past a 16-byte
    boundary (the pool entry points then take their element-wise kernels)."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    u = buf[1:].view(t.shape)
    u.copy_(t)
    assert u.data_ptr() % 16 != 0
    return u


@pytest.mark.parametrize("dtype,C,unaligned", [
    (torch.float16, 2048, False),  # 256 pieces per row: one row per vector workgroup
    (torch.float32, 1100, False),  # 275 pieces: element-wise kernels
    (torch.float16, 24, True),     # whole pieces, unaligned data: element-wise kernels
])
def test_pool_wide_and_unaligned_rows(dtype, C, unaligned):
    from spconv_triton.pytorch._impl import pool

    ks, st, pad, dil, subm = GEOMS[1]
    rng = np.random.default_rng(77)
    idx = rand_indices(rng, 2, [22] * 3, 1200)
    res = _tables(idx, 2, [22] * 3, ks, st, pad, dil, subm)
    pf, pb = res[2], res[3]
    n_out = pf.shape[1]
    x = (torch.round(torch.randn(idx.shape[0], C) * 2) / 2).to(DEV, dtype)
    g = torch.randn(n_out, C).to(DEV, dtype)
    if unaligned:
        x, g = _unaligned(x), _unaligned(g)
    xn, gn = x.cpu().numpy(), g.cpu().numpy()
    out = pool.maxpool_forward(x, pf, n_out)
    ref = orc.maxpool_fwd(xn, pf.cpu().numpy())
    np.testing.assert_array_equal(out.cpu().numpy(), ref.astype(xn.dtype))
    outa = _unaligned(out) if unaligned else out
    dx = pool.maxpool_backward(x, outa, g, pb)
    ref_dx = orc.maxpool_bwd(xn, out.cpu().numpy(), gn, pb.cpu().numpy())
    np.testing.assert_array_equal(dx.cpu().numpy(), ref_dx.astype(xn.dtype))
    avg, count = pool.avgpool_forward(x, pf, n_out)
    ref_avg, ref_count = orc.avgpool_fwd(xn, pf.cpu().numpy())
    np.testing.assert_array_equal(count.cpu().numpy(), ref_count)
    np.testing.assert_array_equal(avg.cpu().numpy(), ref_avg)
    dxa = pool.avgpool_backward(g, pb, count)
    ref_dxa = orc.avgpool_bwd(gn, ref_count, pb.cpu().numpy())
    np.testing.assert_array_equal(dxa.cpu().numpy(), ref_dxa)
