"""Whole networks on this package against the CPU oracle pipeline.

Two networks of the benchmark configurations, at sizes the fp64 oracle runs in
seconds, with the same seeded weights and BatchNorm statistics on both sides
(oracle_pipeline.py: fp64 sparse ops from oracle/, dense glue in torch fp64):

* the VoxelBackBone8x-style LiDAR encoder, inference: SubM(4->16), then
  [SparseConv s2 + 2 x SubM] at 32, 64 and 64 channels, then
  SparseConv(64->128, k(3,1,1), s(2,1,1)), each followed by BatchNorm + ReLU,
  on two samples of a ground-plane-and-boxes scene (bench_data.lidar_cloud);
* a sparse ResUNet training step: encoder 32->64->128->256 with a strided
  SparseConv3d, a SparseMaxPool3d(k2, s2) and another strided SparseConv3d;
  decoder of SparseInverseConv3d layers (the last one inverting the pool's
  rulebook) with skip concatenation (JoinTable), a 1x1 SubM head over 20
  classes and a cross-entropy loss, on two samples of a road/wall/object scene
  (bench_data.urban_cloud).  Loss, logits, the input gradient and every
  parameter gradient are compared.

Layer semantics followed on the oracle side are the reference's module layer
(conv.py:119-513, pool.py:84-235, tables.py:15-42).  Output coordinates must
match exactly, in the same order; features and gradients must agree within a
tolerance relative to the largest reference value, stated in each test
(several layers of fp32 or fp16 arithmetic with BatchNorm between them).
"""

import math

import numpy as np
import pytest
import torch

import oracle_pipeline as op

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _rel_check(name, actual, expected, rtol):
    a = actual.detach().cpu().double()
    e = expected.detach().cpu().double()
    assert a.shape == e.shape, f"{name}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    scale = e.abs().max().item()
    err = (a - e).abs().max().item()
    print(f"{name}: max err / max|ref| = {err / max(scale, 1e-30):.2e}")
    assert err <= rtol * max(scale, 1e-30), (
        f"{name}: max abs err {err:.3e} > {rtol:g} x max|ref| {scale:.3e}")
    return err / max(scale, 1e-30)


class _Params:
    """Seeded weights in the reference's KRSC layout, and BatchNorm state."""

    def __init__(self, seed):
        self.g = torch.Generator().manual_seed(seed)

    def conv(self, cout, ksize, cin):
        fan_in = cin * int(np.prod(ksize))
        bound = 1.0 / math.sqrt(fan_in) * math.sqrt(3.0)
        return (torch.rand(cout, *ksize, cin, generator=self.g, dtype=torch.float64) * 2 - 1) * bound

    def bias(self, cout):
        return torch.randn(cout, generator=self.g, dtype=torch.float64) * 0.1

    def bn(self, c):
        return {
            "weight": torch.rand(c, generator=self.g, dtype=torch.float64) + 0.5,
            "bias": torch.randn(c, generator=self.g, dtype=torch.float64) * 0.1,
            "running_mean": torch.randn(c, generator=self.g, dtype=torch.float64) * 0.1,
            "running_var": torch.rand(c, generator=self.g, dtype=torch.float64) + 0.5,
        }


def _k3(k):
    return [k] * 3 if isinstance(k, int) else list(k)


class _Net:
    """The same network as spconv_triton modules (GPU) and oracle layers (CPU).

    Blocks: ("subm", cin, cout, k, key), ("conv", cin, cout, k, stride, pad, key),
    ("inv", cin, cout, k, key), ("pool", k, stride, key); every conv block is
    followed by BatchNorm + ReLU.  `pairs` keeps (gpu module, oracle layer)
    for the parameter comparison.
    """

    def __init__(self, blocks, params, dtype):
        import spconv_triton.pytorch as spconv

        self.gpu, self.orc, self.pairs = [], [], []
        for blk in blocks:
            kind = blk[0]
            if kind == "pool":
                _, k, stride, key = blk
                self.gpu.append(spconv.SparseMaxPool3d(k, stride, indice_key=key).to(DEV))
                self.orc.append(op.OPool(3, kernel_size=k, stride=stride, indice_key=key))
                continue
            if kind == "subm":
                _, cin, cout, k, key = blk
                g = spconv.SubMConv3d(cin, cout, k, padding=1, bias=False, indice_key=key)
                o = op.OConv(3, cin, cout, k, padding=1, bias=False, subm=True, indice_key=key)
            elif kind == "conv":
                _, cin, cout, k, stride, pad, key = blk
                g = spconv.SparseConv3d(cin, cout, k, stride=stride, padding=pad, bias=False,
                                        indice_key=key)
                o = op.OConv(3, cin, cout, k, stride=stride, padding=pad, bias=False,
                             indice_key=key)
            else:
                _, cin, cout, k, key = blk
                g = spconv.SparseInverseConv3d(cin, cout, k, bias=False, indice_key=key)
                o = op.OConv(3, cin, cout, k, bias=False, inverse=True, indice_key=key)
            # both sides get the weights rounded to the GPU's dtype
            w = params.conv(cout, _k3(k), cin).to(dtype).to(torch.float64)
            with torch.no_grad():
                g.weight.copy_(w.to(g.weight.dtype))
                o.weight.copy_(w)
            bn_g = torch.nn.BatchNorm1d(cout)
            bn_o = torch.nn.BatchNorm1d(cout)
            state = params.bn(cout)
            with torch.no_grad():
                for name, v in state.items():
                    getattr(bn_g, name).copy_(v.to(dtype).float())
                    getattr(bn_o, name).copy_(v.to(dtype).float())
            seq = spconv.SparseSequential(g, bn_g, torch.nn.ReLU()).to(DEV)
            if dtype == torch.float16:
                seq = seq.half()
            self.gpu.append(seq)
            oseq = op.OSeq([o, op.ODense(bn_o), op.ODense(torch.nn.ReLU())])
            self.orc.append(oseq)
            self.pairs.append((seq, oseq))

    def train(self, mode):
        for m in self.gpu:
            m.train(mode)
        self.training = mode

    def gpu_params(self):
        return [p for m in self.gpu for p in m.parameters()]

    def orc_params(self):
        out = []
        for o in self.orc:
            if isinstance(o, op.OSeq):
                p = o.params()
                out.extend([p["0.weight"], p["1.weight"], p["1.bias"]])
        return out


def _orc_input(idx, feats, shape, batch, requires_grad=False, dtype=torch.float64):
    f = feats.to(dtype).to(torch.float64).clone()  # the GPU input, rounded alike
    if requires_grad:
        f.requires_grad_(True)
    return op.OTensor(f, idx, shape, batch), f


def _gpu_input(idx, feats, shape, batch, dtype, requires_grad=False):
    import spconv_triton.pytorch as spconv

    f = feats.to(DEV, dtype).clone()
    if requires_grad:
        f.requires_grad_(True)
    return spconv.SparseConvTensor(f, torch.from_numpy(idx).to(DEV), shape, batch), f


VBB_BLOCKS = [
    ("subm", 4, 16, 3, "subm1"),
    ("conv", 16, 32, 3, 2, 1, "spconv2"),
    ("subm", 32, 32, 3, "subm2"),
    ("subm", 32, 32, 3, "subm2"),
    ("conv", 32, 64, 3, 2, 1, "spconv3"),
    ("subm", 64, 64, 3, "subm3"),
    ("subm", 64, 64, 3, "subm3"),
    ("conv", 64, 64, 3, 2, (0, 1, 1), "spconv4"),
    ("subm", 64, 64, 3, "subm4"),
    ("subm", 64, 64, 3, "subm4"),
    ("conv", 64, 128, (3, 1, 1), (2, 1, 1), 0, "spconv_down2"),
]


# fp32: every GEMM accumulates in IEEE fp32; 11 layers with BatchNorm between
# them stay within 1e-5 of the largest output (measured: 4e-7).  fp16:
# activations are rounded to fp16 after every layer (unit roundoff 4.9e-4);
# measured 4.5e-4 of the largest output, bound 5e-3.
@pytest.mark.parametrize("dtype,rtol", [(torch.float32, 1e-5), (torch.float16, 5e-3)])
def test_voxel_backbone_encoder(dtype, rtol):
    from bench_data import lidar_cloud

    shape = [41, 200, 176]
    idx = lidar_cloud(3000, batch=2, seed=5, shape=shape)
    feats = torch.rand(idx.shape[0], 4, generator=torch.Generator().manual_seed(6),
                       dtype=torch.float64)
    net = _Net(VBB_BLOCKS, _Params(7), dtype)
    net.train(False)
    x, _ = _gpu_input(idx, feats, shape, 2, dtype)
    xo, _ = _orc_input(idx, feats, shape, 2, dtype=dtype)
    with torch.no_grad():
        for g, o in zip(net.gpu, net.orc):
            x = g(x)
            xo = o(xo, False)
    assert list(x.spatial_shape) == list(xo.spatial_shape) == [2, 25, 22]
    assert x.indices.shape[0] > 0
    np.testing.assert_array_equal(x.indices.cpu().numpy(), xo.indices)
    assert x.features.dtype == dtype
    _rel_check("encoder output", x.features, xo.features, rtol)


def _resunet(dtype):
    blocks = {
        "stem": [("subm", 4, 32, 3, "s0")],
        "e1": [("conv", 32, 64, 2, 2, 0, "d1"), ("subm", 64, 64, 3, "s1")],
        "e2": [("pool", 2, 2, "p2"), ("subm", 64, 128, 3, "s2")],
        "e3": [("conv", 128, 256, 2, 2, 0, "d3"), ("subm", 256, 256, 3, "s3")],
        "u3": [("inv", 256, 128, 2, "d3")],
        "m2": [("subm", 256, 128, 3, "s2")],
        "u2": [("inv", 128, 64, 2, "p2")],
        "m1": [("subm", 128, 64, 3, "s1")],
        "u1": [("inv", 64, 32, 2, "d1")],
        "m0": [("subm", 64, 32, 3, "s0")],
    }
    params = _Params(11)
    return {k: _Net(v, params, dtype) for k, v in blocks.items()}, params


def _run(parts, x, head, join, cat):
    def seq(name, t):
        net = parts[name]
        for m in net.gpu if not isinstance(t, op.OTensor) else net.orc:
            t = m(t) if not isinstance(t, op.OTensor) else m(t, net.training)
        return t

    s0 = seq("stem", x)
    s1 = seq("e1", s0)
    s2 = seq("e2", s1)
    s3 = seq("e3", s2)
    u = seq("m2", join([seq("u3", s3), s2]))
    u = seq("m1", join([seq("u2", u), s1]))
    u = seq("m0", join([seq("u1", u), s0]))
    return head(u)


def _resunet_step(autocast, loss_scale=1.0):
    import spconv_triton.pytorch as spconv
    from bench_data import urban_cloud

    shape = [64, 256, 256]
    idx = urban_cloud(4000, batch=2, seed=9, shape=shape)
    n = idx.shape[0]
    gen = torch.Generator().manual_seed(10)
    feats = torch.rand(n, 4, generator=gen, dtype=torch.float64)
    labels = torch.randint(0, 20, (n,), generator=gen)
    parts, params = _resunet(torch.float32)
    for p in parts.values():
        p.train(True)
    hw = params.conv(20, [1, 1, 1], 32).float().double()
    hb = params.bias(20).float().double()
    head_g = spconv.SubMConv3d(32, 20, 1, bias=True).to(DEV)
    head_o = op.OConv(3, 32, 20, 1, bias=True, subm=True)
    with torch.no_grad():
        head_g.weight.copy_(hw.float())
        head_g.bias.copy_(hb.float())
        head_o.weight.copy_(hw)
        head_o.bias.copy_(hb)
    for t in (head_o.weight, head_o.bias):
        t.requires_grad_(True)
    for p in parts.values():
        for t in p.orc_params():
            t.requires_grad_(True)

    x, fg = _gpu_input(idx, feats, shape, 2, torch.float32, requires_grad=True)
    join = spconv.JoinTable()
    with torch.autocast("cuda", dtype=torch.float16, enabled=autocast):
        logits = _run(parts, x, head_g, join, None)
        loss = torch.nn.functional.cross_entropy(logits.features.float(), labels.to(DEV))
    (loss * loss_scale).backward()

    xo, fo = _orc_input(idx, feats, shape, 2, requires_grad=True, dtype=torch.float32)
    ojoin = lambda ts: ts[0].replace(torch.cat([t.features for t in ts], 1))
    op.ROUND = torch.float16 if autocast else None
    try:
        logits_o = _run(parts, xo, lambda t: head_o(t, True), ojoin, None)
        loss_o = torch.nn.functional.cross_entropy(logits_o.features, labels)
        # the same loss scale, so that the oracle rounds gradients to fp16 at
        # the magnitudes the GPU sees (a power of two: exact in fp64)
        (loss_o * loss_scale).backward()
    finally:
        op.ROUND = None

    np.testing.assert_array_equal(logits.indices.cpu().numpy(), logits_o.indices)
    s = 1.0 / loss_scale
    grads = [("grad input", fg.grad * s, fo.grad * s),
             ("head weight grad", head_g.weight.grad * s, head_o.weight.grad * s),
             ("head bias grad", head_g.bias.grad * s, head_o.bias.grad * s)]
    for name, p in parts.items():
        gp, opp = p.gpu_params(), p.orc_params()
        assert len(gp) == len(opp)
        grads += [(f"{name}.{i} grad", a.grad * s, e.grad * s)
                  for i, (a, e) in enumerate(zip(gp, opp))]
    return (loss, loss_o), (logits.features, logits_o.features), grads


def test_resunet_training_step():
    """fp32 forward + backward (IEEE fp32 GEMMs).  Measured against the fp64
    oracle: loss 7e-8, logits 1.1e-6, gradients <= 2.1e-6 of the largest
    reference value; bounds 1e-6, 1e-5 and 2e-5."""
    (loss, loss_o), (lg, lo), grads = _resunet_step(False)
    _rel_check("loss", loss, loss_o, 1e-6)
    _rel_check("logits", lg, lo, 1e-5)
    for name, a, e in grads:
        _rel_check(name, a, e, 2e-5)


def _l2_check(name, actual, expected, max_rel_l2, min_cos):
    a = actual.detach().cpu().double().flatten()
    e = expected.detach().cpu().double().flatten()
    rel = ((a - e).norm() / e.norm()).item()
    cos = (a @ e / (a.norm() * e.norm())).item()
    print(f"{name}: relative L2 {rel:.2e}, cosine {cos:.6f}")
    assert rel <= max_rel_l2 and cos >= min_cos, (
        f"{name}: relative L2 error {rel:.3e} (bound {max_rel_l2}), cosine {cos:.6f} "
        f"(bound {min_cos})")


# Measured (relative L2, cosine) of every fp16-autocast ResUNet gradient
# against the fp64 oracle on MI355X (the kernels are deterministic, so these
# repeat); the test bounds each at 1.5x its own error.
FP16_GRAD_ERRORS = {
    "grad input": (0.0403, 0.999186),
    "head weight grad": (0.000308, 1.000000),
    "head bias grad": (0.000211, 1.000000),
    "stem.0 grad": (0.0347, 0.999397),
    "stem.1 grad": (0.0274, 0.999632),
    "stem.2 grad": (0.0366, 0.999328),
    "e1.0 grad": (0.0483, 0.998834),
    "e1.1 grad": (0.0474, 0.998884),
    "e1.2 grad": (0.0495, 0.998868),
    "e1.3 grad": (0.0496, 0.998768),
    "e1.4 grad": (0.0525, 0.998623),
    "e1.5 grad": (0.0452, 0.998987),
    "e2.0 grad": (0.0547, 0.998507),
    "e2.1 grad": (0.0571, 0.998383),
    "e2.2 grad": (0.0494, 0.998787),
    "e3.0 grad": (0.0558, 0.998443),
    "e3.1 grad": (0.059, 0.998269),
    "e3.2 grad": (0.0575, 0.998393),
    "e3.3 grad": (0.0553, 0.998468),
    "e3.4 grad": (0.062, 0.998089),
    "e3.5 grad": (0.0517, 0.998675),
    "u3.0 grad": (0.0544, 0.998519),
    "u3.1 grad": (0.0509, 0.998724),
    "u3.2 grad": (0.0477, 0.998866),
    "m2.0 grad": (0.0505, 0.998725),
    "m2.1 grad": (0.047, 0.998899),
    "m2.2 grad": (0.0406, 0.999176),
    "u2.0 grad": (0.049, 0.998800),
    "u2.1 grad": (0.0477, 0.998864),
    "u2.2 grad": (0.0493, 0.998860),
    "m1.0 grad": (0.0428, 0.999084),
    "m1.1 grad": (0.0296, 0.999573),
    "m1.2 grad": (0.0272, 0.999630),
    "u1.0 grad": (0.0313, 0.999510),
    "u1.1 grad": (0.0121, 0.999933),
    "u1.2 grad": (0.0246, 0.999701),
    "m0.0 grad": (0.0142, 0.999900),
    "m0.1 grad": (0.000244, 1.000000),
    "m0.2 grad": (0.00224, 0.999998),
}


def test_resunet_training_step_autocast_fp16():
    """The same step under torch.autocast(float16): sparse convolutions take
    fp16 inputs and return fp16 (fp32 accumulation), as the reference's
    custom_fwd(cast_inputs=float16) does; the loss is scaled by 2^12 before
    the backward pass, as GradScaler does, and the gradients unscaled.  The
    oracle rounds to fp16 at the same tensors, forward and backward
    (oracle_pipeline.ROUND).

    Bounds: loss 1e-4 and logits 5e-3 of the largest reference value.  The
    gradients are compared by relative L2 error and cosine similarity, each
    bounded at 1.5x its measured error (FP16_GRAD_ERRORS: relative L2 2e-4 to
    6.2e-2): fp16 storage alone moves this network's gradients by 1.5-6.7 % in
    L2 (cosine >= 0.9977) from the fp64 ones -- measured on the oracle with and
    without the rounding -- and by up to 16 % of the largest value
    element-wise, so element-wise bounds do not apply.  One wrong offset in one
    layer's input gradient moves that layer's and every earlier layer's
    gradients by far more than half their error again."""
    (loss, loss_o), (lg, lo), grads = _resunet_step(True, loss_scale=4096.0)
    _rel_check("loss", loss, loss_o, 1e-4)
    _rel_check("logits", lg, lo, 5e-3)
    bad = []
    assert {name for name, _, _ in grads} == set(FP16_GRAD_ERRORS)
    for name, a, e in grads:
        rel, cos = FP16_GRAD_ERRORS[name]
        try:
            # (cosines are recorded to 6 decimals: 1e-6 of slack for the rounding)
            _l2_check(name, a, e, 1.5 * rel, 1.0 - (1.5 * (1.0 - cos) + 1e-6))
        except AssertionError as exc:
            bad.append(str(exc))
    assert not bad, "\n".join(bad)
