"""Benchmark configurations 1, 3 and 4 at their stated sizes, checked against
the CPU oracle inside the real networks.

* config 1: SubMConv3d 16 -> 16 fp32, 2 000 uniform voxels in 64^3, batch 1
  (the reference's CPU-runnable case): the rulebook bit for bit, the forward
  on every row, the input and weight gradients on every entry;
* config 3: VoxelBackBone8x-style encoder (the layer list of
  ``bench_configs.ENCODER``), fp16 eval, 4 x 20k LiDAR voxels in
  [41, 1600, 1408];
* config 4: sparse ResUNet training step (``bench_configs.RESUNET``), fp16
  autocast, 2 x 120k urban voxels in [128, 2048, 2048].

For configs 3 and 4 every rulebook a layer builds (subm, strided, pooling) is
compared bit for bit with the oracle's ``igemm_pairs`` on the layer's own input
coordinates (reference ``_impl/pairs.py:281-426``), and every gather-GEMM call
of the pass is recorded and checked against the oracle's fp64 GEMM fed with
the exact values the GPU received (reference ``_impl/gemm.py:501-713``):
forward on every 11th output row, input gradient on every 11th input row,
weight gradient on 5 output channels.  Bound for 16-bit outputs, per entry:
|out - ref| <= 1e-3 |ref| + e |ref_abs| + 6e-8, where ref_abs is the same
product of the absolute values (the size of the sum's terms, which bounds the
fp32 accumulation error), e = 3e-5 for the forward and input gradient and 1e-4
for the weight gradient (up to ~60k products per entry), and 6e-8 covers fp16
subnormal rounding (gradients of a 240k-row mean loss reach that range).  A
wrong offset, row or channel moves an entry by about the size of one offset's
contribution, orders of magnitude above e |ref_abs|.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _np(t):
    return t.detach().double().cpu().numpy()


def _within(out, ref, ref_abs, rel, e, what):
    err = np.abs(out - ref)
    bad = err > rel * np.abs(ref) + e * ref_abs + 6e-8
    assert not bad.any(), (f"{what}: {int(bad.sum())}/{bad.size} beyond tolerance, "
                           f"max err {err.max():.3e}")


class _Recorder:
    """Wraps the gather-GEMM entry points of ``_impl.gemm`` and keeps a copy of
    every call's operands and result."""

    def __init__(self, monkeypatch):
        from spconv_triton.pytorch._impl import gemm

        self.fwd, self.dgrad, self.wgrad = [], [], []
        f0, d0, w0 = gemm.conv_forward, gemm.conv_backward_input, gemm.conv_backward_weight

        def fwd(features, filters, pair_fwd, n_out, bias=None, **kw):
            out = f0(features, filters, pair_fwd, n_out, bias=bias, **kw)
            self.fwd.append((features.detach().clone(), filters.detach().clone(),
                             pair_fwd.clone(), None if bias is None else bias.detach().clone(),
                             out.detach().clone()))
            return out

        def dgrad(grad_out, filters, pair_bwd, n_in, **kw):
            out = d0(grad_out, filters, pair_bwd, n_in, **kw)
            self.dgrad.append((grad_out.detach().clone(), filters.detach().clone(),
                               pair_bwd.clone(), out.detach().clone()))
            return out

        def wgrad(features, grad_out, pair_fwd, weight_shape, **kw):
            out = w0(features, grad_out, pair_fwd, weight_shape, **kw)
            self.wgrad.append((features.detach().clone(), grad_out.detach().clone(),
                               pair_fwd.clone(), out.detach().clone()))
            return out

        monkeypatch.setattr(gemm, "conv_forward", fwd)
        monkeypatch.setattr(gemm, "conv_backward_input", dgrad)
        monkeypatch.setattr(gemm, "conv_backward_weight", wgrad)

    def check(self, step=11, n_cols=5):
        for i, (x, w, pf, b, out) in enumerate(self.fwd):
            K, C = w.shape[0], w.shape[-1]
            wn = _np(w).reshape(K, -1, C)
            rows = np.arange(0, out.shape[0], step)
            pfr = pf.cpu().numpy()[:, rows]
            xn = _np(x)
            ref = orc.gemm_fwd(xn, wn, pfr, None if b is None else _np(b))
            ref_abs = orc.gemm_fwd(np.abs(xn), np.abs(wn), pfr,
                                   None if b is None else np.abs(_np(b)))
            _within(_np(out)[rows], ref, ref_abs, 1e-3, 3e-5, f"forward call {i} ({C}->{K})")
        for i, (g, w, pb, out) in enumerate(self.dgrad):
            K, C = w.shape[0], w.shape[-1]
            wn = _np(w).reshape(K, -1, C)
            rows = np.arange(0, out.shape[0], step)
            pbr = pb.cpu().numpy()[:, rows]
            gn = _np(g)
            ref = orc.gemm_dgrad(gn, wn, pbr)
            ref_abs = orc.gemm_dgrad(np.abs(gn), np.abs(wn), pbr)
            _within(_np(out)[rows], ref, ref_abs, 1e-3, 3e-5, f"dgrad call {i} ({K}->{C})")
        for i, (x, g, pf, out) in enumerate(self.wgrad):
            K, C = out.shape[0], out.shape[-1]
            cols = np.unique(np.linspace(0, K - 1, n_cols).round().astype(np.int64))
            xn, gn = _np(x), _np(g)[:, cols]
            pfn = pf.cpu().numpy()
            ref = orc.gemm_wgrad(xn, gn, pfn, len(cols), C)
            ref_abs = orc.gemm_wgrad(np.abs(xn), np.abs(gn), pfn, len(cols), C)
            got = _np(out).reshape(K, -1, C)[cols]
            _within(got, ref, ref_abs, 1e-3, 1e-4, f"wgrad call {i} ({C}->{K})")


def _hook_rulebooks(modules):
    """Forward hooks on the layers that build a rulebook (not the inverse
    convolutions, which reuse one): each records the layer's input
    coordinates and the rulebook it stored under its indice_key."""
    from spconv_triton.pytorch.conv import SparseConvolution

    seen = []

    def hook(mod, inputs, output):
        x = inputs[0]
        seen.append((mod, x.indices.clone(), list(x.spatial_shape), x.batch_size,
                     output.indice_dict[mod.indice_key]))

    handles = []
    for m in modules:
        if getattr(m, "indice_key", None) is None:
            continue
        if isinstance(m, SparseConvolution) and m.inverse:
            continue
        handles.append(m.register_forward_hook(hook))
    return seen, handles


def _check_rulebooks(seen, is_train):
    checked = set()
    for mod, idx, shape, bs, data in seen:
        if mod.indice_key in checked:
            continue
        checked.add(mod.indice_key)
        subm = bool(getattr(mod, "subm", False))
        out_pad = list(getattr(mod, "output_padding", [0] * 3))
        exp = orc.igemm_pairs(idx.cpu().numpy(), bs, shape, list(mod.kernel_size),
                              list(mod.stride), list(mod.padding), list(mod.dilation), out_pad,
                              subm, False, is_train)
        what = f"rulebook {mod.indice_key}"
        np.testing.assert_array_equal(data.pair_fwd.cpu().numpy(), exp[2], f"{what} pair_fwd")
        if not subm:
            np.testing.assert_array_equal(data.out_indices.cpu().numpy(), exp[0],
                                          f"{what} out_indices")
            if is_train and data.pair_bwd is not None:
                np.testing.assert_array_equal(data.pair_bwd.cpu().numpy(), exp[3],
                                              f"{what} pair_bwd")
    return checked


def test_config1_subm_16_fp32():
    """Config 1 exactly: rulebook, forward, input and weight gradient against
    the oracle (fp32 bound 1e-5 * max(1, max|ref|), as for the fp32 GEMM cases)."""
    import spconv_triton.pytorch as spconv

    from bench_data import uniform_cloud

    idx = uniform_cloud(2000, [64] * 3, seed=1)
    t = torch.from_numpy(idx).to(DEV)
    torch.manual_seed(11)
    conv = spconv.SubMConv3d(16, 16, 3, padding=1, bias=True, indice_key="c1").to(DEV)
    feats = torch.randn(idx.shape[0], 16, device=DEV, requires_grad=True)
    y = conv(spconv.SparseConvTensor(feats, t, [64] * 3, 1))
    g = torch.randn_like(y.features)
    (y.features * g).sum().backward()

    exp = orc.igemm_pairs(idx, 1, [64] * 3, [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3,
                          True, False, True)
    pf = exp[2]
    np.testing.assert_array_equal(y.indice_dict["c1"].pair_fwd.cpu().numpy(), pf)
    assert torch.equal(y.indices, t)
    w = _np(conv.weight).reshape(16, 27, 16)

    def close(out, ref, what):
        err = np.abs(_np(out) - ref).max()
        assert err <= 1e-5 * max(1.0, float(np.abs(ref).max())), f"{what}: max err {err:.3e}"

    close(y.features, orc.gemm_fwd(_np(feats), w, pf, _np(conv.bias)), "forward")
    np.testing.assert_array_equal(y.indice_dict["c1"].pair_bwd.cpu().numpy(), exp[3])
    close(feats.grad, orc.gemm_dgrad(_np(g), w, exp[3]), "input gradient")
    dw = orc.gemm_wgrad(_np(feats), _np(g), pf, 16, 16)
    close(conv.weight.grad.reshape(16, 27, 16), dw, "weight gradient")
    close(conv.bias.grad, _np(g).sum(0), "bias gradient")


def test_config3_encoder_full_size(monkeypatch):
    """Config 3 at 4 x 20k voxels, fp16 eval: every rulebook bit for bit, every
    GEMM call on row slices."""
    import bench_configs
    import spconv_triton.pytorch as spconv

    from bench_data import lidar_cloud

    shape = [41, 1600, 1408]
    idx = lidar_cloud(20000, batch=4, seed=0, shape=shape)
    it = torch.from_numpy(idx).to(DEV)
    torch.manual_seed(3)
    feats = torch.rand(idx.shape[0], 4, device=DEV).half()
    net = bench_configs.build(bench_configs.ENCODER).half().eval()
    rec = _Recorder(monkeypatch)
    seen, handles = _hook_rulebooks(net)
    try:
        with torch.no_grad():
            out = net(spconv.SparseConvTensor(feats, it, shape, 4))
    finally:
        for h in handles:
            h.remove()
    assert out.features.shape[0] > 0
    keys = _check_rulebooks(seen, is_train=False)
    assert keys == {"subm1", "spconv2", "subm2", "spconv3", "subm3", "spconv4", "subm4",
                    "spconv_down2"}
    assert len(rec.fwd) == 11
    rec.check()


def test_config4_resunet_step_full_size(monkeypatch):
    """Config 4 at 2 x 120k voxels, fp16 autocast training step: every rulebook
    (subm, k2 s2 convolutions, max-pool) bit for bit, every forward, input- and
    weight-gradient GEMM of the step on slices."""
    import bench_configs
    import spconv_triton.pytorch as spconv

    from bench_data import urban_cloud

    shape = [128, 2048, 2048]
    idx = urban_cloud(120000, batch=2, seed=9, shape=shape)
    it = torch.from_numpy(idx).to(DEV)
    n = idx.shape[0]
    torch.manual_seed(4)
    feats = torch.rand(n, 4, device=DEV)
    labels = torch.randint(0, 20, (n,), device=DEV)
    parts = {k: bench_configs.build(v).train() for k, v in bench_configs.RESUNET.items()}
    head = spconv.SubMConv3d(32, 20, 1, bias=True).to(DEV)
    join = spconv.JoinTable()
    rec = _Recorder(monkeypatch)
    seen, handles = _hook_rulebooks([m for p in parts.values() for m in p])
    try:
        x = spconv.SparseConvTensor(feats.clone().requires_grad_(True), it, shape, 2)
        with torch.autocast("cuda", dtype=torch.float16):
            s0 = parts["stem"](x)
            s1 = parts["e1"](s0)
            s2 = parts["e2"](s1)
            s3 = parts["e3"](s2)
            u = parts["m2"](join([parts["u3"](s3), s2]))
            u = parts["m1"](join([parts["u2"](u), s1]))
            u = parts["m0"](join([parts["u1"](u), s0]))
            logits = head(u)
            loss = torch.nn.functional.cross_entropy(logits.features.float(), labels)
        loss.backward()
    finally:
        for h in handles:
            h.remove()
    assert torch.isfinite(loss).item()
    keys = _check_rulebooks(seen, is_train=True)
    assert keys == {"s0", "d1", "s1", "p2", "s2", "d3", "s3"}
    # 12 convolutions (the 1x1 head is a dense product, no gather-GEMM)
    assert len(rec.fwd) == 12 and len(rec.wgrad) == 12, (len(rec.fwd), len(rec.wgrad))
    assert len(rec.dgrad) >= 11, len(rec.dgrad)
    rec.check()
