"""SPCONV_ALLOW_TF32: fp32 GEMMs as split-bf16 products on the bf16 matrix cores.

The reference switches its fp32 ``tl.dot`` to TF32 when the flag is set
(reference ``_impl/gemm.py:456-463``, used by the forward :564, the input
gradient :627 and the weight gradient :708).  gfx950 has no xf32 MFMA, so the
flag is served by hi*hi + hi*lo + lo*hi with hi = bf16(x), lo = bf16(x - hi)
(Henry, Tang & Heinecke, ARITH 2019).

Bounds, written per check:
* each product a*b is recovered to within 3 * 2^-16 * |a||b| (the dropped
  lo*lo term and the rounding of lo), and the fp32 accumulation adds about
  2^-24 per term, so |out - ref| <= 1e-4 * S + 1e-6 with S = sum |a||b| (the
  oracle's GEMM of |X| and |W|);
* the reference's own TF32 contract is looser (3 x its TF32-vs-IEEE deviation
  + 1e-3, reference tests/test_tf32.py:1-20): TF32 rounds inputs to 2^-11.
Engagement (reference tests/test_tf32.py:150-190): with the flag on the
result must differ from the flag-off (IEEE) result, and the IEEE result must
be the closer one to the fp64 oracle.
"""

import contextlib

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from test_gpu_gemm import CASES, _tables, rand_indices

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@contextlib.contextmanager
def tf32(on):
    from spconv_triton import constants

    prev = constants.SPCONV_ALLOW_TF32
    constants.SPCONV_ALLOW_TF32 = on
    try:
        yield
    finally:
        constants.SPCONV_ALLOW_TF32 = prev


def _bound_check(out, ref, scale, what):
    out = out.detach().double().cpu().numpy()
    err = np.abs(out - ref)
    tol = 1e-4 * scale + 1e-6
    bad = err > tol
    assert not bad.any(), (f"{what}: {int(bad.sum())}/{bad.size} beyond 1e-4*S, "
                           f"max err/S {(err / np.maximum(scale, 1e-30)).max():.2e}")
    return float(err.max())


@pytest.mark.parametrize("ci", [0, 1, 3, 4, 8, 9, 10, 11])
def test_split_bf16_gemms_match_oracle(ci):
    from spconv_triton.pytorch._impl import gemm

    C, K, n, subm, stride = CASES[ci]
    rng = np.random.default_rng(600 + ci)
    idx = rand_indices(rng, 2, [28] * 3, n)
    res = _tables(idx, 2, [28] * 3, [3] * 3, [stride] * 3, [1] * 3, subm)
    pf, pb = res[2], res[3]
    n_out = pf.shape[1]
    torch.manual_seed(700 + ci)
    x = torch.randn(idx.shape[0], C, device=DEV)
    g = torch.randn(n_out, K, device=DEV)
    w = torch.randn(K, 3, 3, 3, C, device=DEV) / np.sqrt(27 * C)
    b = torch.randn(K, device=DEV) * 0.1
    xn, gn, wn, bn = (t.double().cpu().numpy() for t in (x, g, w, b))
    wn = wn.reshape(K, 27, C)
    pfn, pbn = pf.cpu().numpy(), pb.cpu().numpy()
    ref = orc.gemm_fwd(xn, wn, pfn, bn)
    ref_dx = orc.gemm_dgrad(gn, wn, pbn)
    ref_dw = orc.gemm_wgrad(xn, gn, pfn, K, C)
    s_fwd = orc.gemm_fwd(np.abs(xn), np.abs(wn), pfn)
    s_dx = orc.gemm_dgrad(np.abs(gn), np.abs(wn), pbn)
    s_dw = orc.gemm_wgrad(np.abs(xn), np.abs(gn), pfn, K, C)
    outs = {}
    for on in (True, False):
        with tf32(on):
            outs[on] = (gemm.conv_forward(x, w, pf, n_out, bias=b),
                        gemm.conv_backward_input(g, w, pb, idx.shape[0]),
                        gemm.conv_backward_weight(x, g, pf, (K, 27, C)))
    for t in outs[True]:
        assert t.dtype == torch.float32
    checks = (("forward", ref, s_fwd), ("dgrad", ref_dx, s_dx), ("wgrad", ref_dw, s_dw))
    for i, (name, r, sc) in enumerate(checks):
        on, off = outs[True][i], outs[False][i]
        e_on = _bound_check(on, r, sc, f"{name} (split-bf16)")
        e_off = float(np.abs(off.double().cpu().numpy() - r).max())
        # engagement: the flag changes the result, and IEEE fp32 is the closer one
        assert not torch.equal(on, off), f"{name}: SPCONV_ALLOW_TF32 changed nothing"
        assert e_off < e_on, f"{name}: IEEE error {e_off:.2e} not below split {e_on:.2e}"
    # deterministic, like the IEEE path
    with tf32(True):
        again = gemm.conv_backward_weight(x, g, pf, (K, 27, C))
    assert torch.equal(again, outs[True][2])


def test_split_bf16_parts():
    """sp_split_bf16x3 patterns: hi = bf16(x), lo = bf16(x - hi), in the three
    layouts, on rows whose width is (not) a multiple of 4."""
    from spconv_triton.pytorch._impl import gemm

    torch.manual_seed(0)
    for cols in (64, 37):
        x = torch.randn(513, cols, device=DEV) * 3
        hi = x.to(torch.bfloat16)
        lo = (x - hi.float()).to(torch.bfloat16)
        exp = {0: (hi, hi, lo), 1: (hi, lo, hi), 2: (hi, lo)}
        for pattern, parts in exp.items():
            out = gemm.split_bf16(x, pattern)
            assert torch.equal(out, torch.cat(parts, 1)), (cols, pattern)
        # the parts recover x to about 2^-16 relative
        rec = hi.double() + lo.double()
        assert float(((rec - x.double()).abs() / x.double().abs().clamp_min(1e-30)).max()) \
            <= 2.0 ** -16


def test_tf32_module_training_step():
    """A SubMConv3d + SparseConv3d training step in fp32 with the flag on:
    outputs and every gradient within 1e-3 of the largest IEEE value (the
    elementwise 1e-4 * S bound, with S / max|out| up to about sqrt(terms)),
    and different from the IEEE step."""
    import spconv_triton.pytorch as spconv

    rng = np.random.default_rng(3)
    idx = rand_indices(rng, 2, [24] * 3, 3000)
    t = torch.from_numpy(idx).to(DEV)
    torch.manual_seed(1)
    net = spconv.SparseSequential(
        spconv.SubMConv3d(32, 64, 3, padding=1, indice_key="s"),
        spconv.SparseConv3d(64, 32, 3, stride=2, padding=1),
    ).to(DEV).train()
    feats = torch.randn(idx.shape[0], 32, device=DEV)
    res = {}
    for on in (False, True):
        net.zero_grad()
        f = feats.clone().requires_grad_(True)
        with tf32(on):
            y = net(spconv.SparseConvTensor(f, t, [24] * 3, 2))
            (y.features * torch.linspace(-1, 1, y.features.numel(), device=DEV)
             .reshape(y.features.shape)).sum().backward()
        res[on] = [y.features.detach().clone(), f.grad.clone()] + \
                  [p.grad.clone() for p in net.parameters()]
    for a, b in zip(res[True], res[False]):
        scale = float(b.abs().max())
        assert float((a - b).abs().max()) <= 1e-3 * max(scale, 1e-6)
    assert not torch.equal(res[True][0], res[False][0])


def test_fp16_accumulation_flags_served_at_fp32():
    """SPCONV_ALLOW_FP16_ACCUM / fp32_accum=False (reference _impl/gemm.py:456-498)
    ask for fp16 accumulation, which gfx950's MFMAs do not offer: the flags are
    accepted and the GEMMs accumulate in fp32, so the results equal the
    default ones bit for bit (forward, input gradient and weight gradient in
    fp16, through the GEMM wrappers and through a module training step)."""
    import spconv_triton.pytorch as spconv
    from spconv_triton import constants
    from spconv_triton.pytorch._impl import gemm

    rng = np.random.default_rng(8)
    idx = rand_indices(rng, 2, [24] * 3, 3000)
    res = _tables(idx, 2, [24] * 3, [3] * 3, [1] * 3, [1] * 3, True)
    pf, pb = res[2], res[3]
    torch.manual_seed(5)
    x = torch.randn(idx.shape[0], 32, device=DEV).half()
    g = torch.randn(pf.shape[1], 48, device=DEV).half()
    w = (torch.randn(48, 3, 3, 3, 32, device=DEV) / 30).half()
    n = idx.shape[0]
    for acc in (None, True):
        assert torch.equal(gemm.conv_forward(x, w, pf, n, fp32_accum=False),
                           gemm.conv_forward(x, w, pf, n, fp32_accum=acc))
        assert torch.equal(gemm.conv_backward_input(g, w, pb, n, fp32_accum=False),
                           gemm.conv_backward_input(g, w, pb, n, fp32_accum=acc))
        assert torch.equal(gemm.conv_backward_weight(x, g, pf, w.shape, fp32_accum=False),
                           gemm.conv_backward_weight(x, g, pf, w.shape, fp32_accum=acc))

    t = torch.from_numpy(idx).to(DEV)
    torch.manual_seed(6)
    net = spconv.SparseSequential(spconv.SubMConv3d(32, 48, 3, padding=1, indice_key="s"),
                                  spconv.SparseConv3d(48, 16, 3, stride=2, padding=1))
    net = net.to(DEV).half().train()
    out = {}
    prev = constants.SPCONV_ALLOW_FP16_ACCUM
    try:
        for flag in (False, True):
            constants.SPCONV_ALLOW_FP16_ACCUM = flag
            net.zero_grad()
            f = x.clone().requires_grad_(True)
            y = net(spconv.SparseConvTensor(f, t, [24] * 3, 2))
            y.features.float().square().sum().backward()
            out[flag] = [y.features.clone(), f.grad.clone()] + [p.grad.clone()
                                                                 for p in net.parameters()]
    finally:
        constants.SPCONV_ALLOW_FP16_ACCUM = prev
    for a, b in zip(out[True], out[False]):
        assert torch.equal(a, b)
