"""The reference's golden cases (spconv 2.3.8 outputs held in the reference's
tests/data, extracted to tests/golden) run through this package's modules on
the GPU, with the reference's own tolerances (``atol_*`` stored in each case)
and its canonical output ordering (reference tests/helpers.py:94-177, :245-325,
tests/test_network.py:14-81).
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def canonical_order(indices, spatial_shape):
    lin = indices[:, 0].long()
    for i, s in enumerate(spatial_shape):
        lin = lin * int(s) + indices[:, i + 1].long()
    return torch.argsort(lin)


def inverse_permutation(order):
    inv = torch.empty_like(order)
    inv[order] = torch.arange(order.numel(), device=order.device)
    return inv


def assert_close(actual, expected, atol, msg):
    a = actual.detach().cpu().double()
    e = expected.detach().cpu().double()
    assert a.shape == e.shape, f"{msg}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    if a.numel():
        err = (a - e).abs().max().item()
        assert err <= atol, f"{msg}: max abs err {err:.3e} > atol {atol:.3e}"


def _resolve(ctor):
    import spconv_triton.pytorch as spconv
    from spconv_triton.compat import tv

    ctor = dict(ctor or {})
    if isinstance(ctor.get("algo"), str):
        ctor["algo"] = getattr(spconv.ConvAlgo, ctor["algo"].split(".")[-1])
    if isinstance(ctor.get("act_type"), str):
        ctor["act_type"] = getattr(tv.gemm.Activation, ctor["act_type"].split(".")[-1])
    return ctor


def build_layer(spec, dtype):
    import spconv_triton.pytorch as spconv
    from spconv_triton.pytorch import conv as spconv_conv
    from spconv_triton.pytorch import pool as spconv_pool

    cls_name = spec["cls"]
    if cls_name == "SparseSequential":
        return spconv.SparseSequential(*[build_layer(c, dtype) for c in spec["children"]])
    if cls_name.startswith("nn."):
        cls = getattr(torch.nn, cls_name[3:])
    else:
        cls = (getattr(spconv, cls_name, None) or getattr(spconv_conv, cls_name, None)
               or getattr(spconv_pool, cls_name))
    layer = cls(**_resolve(spec.get("ctor"))).to(DEV)
    if dtype == torch.float16:
        layer = layer.half()
    with torch.no_grad():
        for name, value in (spec.get("params") or {}).items():
            if value is not None:
                getattr(layer, name).copy_(value.to(DEV))
    return layer


def build_unet3d(in_channels=6, base=16):
    import spconv_triton.pytorch as sp

    nn = torch.nn

    class UNet3d(nn.Module):
        def __init__(self):
            super().__init__()
            self.stem = sp.SparseSequential(
                sp.SubMConv3d(in_channels, base, 3, padding=1, indice_key="s0", bias=False),
                nn.BatchNorm1d(base), nn.ReLU(),
                sp.SubMConv3d(base, base, 3, padding=1, indice_key="s0", bias=False))
            self.down = sp.SparseConv3d(base, base * 2, 3, stride=2, padding=1,
                                        indice_key="d0", bias=False)
            self.mid = sp.SparseSequential(
                sp.SubMConv3d(base * 2, base * 2, 3, padding=1, indice_key="s1", bias=False),
                nn.BatchNorm1d(base * 2), nn.ReLU())
            self.up = sp.SparseInverseConv3d(base * 2, base, 3, indice_key="d0", bias=False)
            self.join = sp.JoinTable()
            self.head = sp.SubMConv3d(base * 2, 8, 1, bias=True)

        def forward(self, x):
            a = self.stem(x)
            b = self.down(a)
            c = self.mid(b)
            d = self.up(c)
            return self.head(self.join([d, a]))

    return UNet3d()


def _sparse_input(inp, requires_grad):
    import spconv_triton.pytorch as spconv

    feats = inp["features"].to(DEV).clone()
    if requires_grad:
        feats.requires_grad_(True)
    x = spconv.SparseConvTensor(feats, inp["indices"].to(DEV), list(inp["spatial_shape"]),
                                int(inp["batch_size"]))
    return x, feats


@pytest.mark.parametrize("case_id", ["unet3d_float32", "unet3d_float16"])
def test_unet_golden(golden, case_id):
    case = golden("net.pt", case_id)
    expect = case["expect"]
    dtype = getattr(torch, case["dtype"])
    net = build_unet3d().to(DEV)
    if dtype == torch.float16:
        net = net.half()
    missing, unexpected = net.load_state_dict({k: v.to(DEV) for k, v in
                                               case["state_dict"].items()})
    assert not missing and not unexpected
    assert sorted(net.state_dict().keys()) == sorted(case["state_dict"].keys())
    net.train()
    x, feats = _sparse_input(case["input"], True)
    out = net(x)
    assert list(out.spatial_shape) == list(expect["out_spatial_shape"])
    order = canonical_order(out.indices.cpu(), out.spatial_shape)
    assert torch.equal(out.indices.cpu()[order], expect["out_indices"])
    assert out.features.dtype == dtype
    assert_close(out.features.cpu()[order], expect["out_features"], expect["atol_out"], "out")
    inv = inverse_permutation(order.to(DEV))
    out.features.backward(expect["grad_out"].to(DEV)[inv].to(out.features.dtype))
    assert_close(feats.grad, expect["grad_input"], expect["atol_grad_input"], "grad_input")
    named = dict(net.named_parameters())
    assert set(expect["grad_params"]) == {k for k, p in named.items() if p.requires_grad}
    for k, ginfo in expect["grad_params"].items():
        assert_close(named[k].grad, ginfo["grad"], ginfo["atol"], f"{k}.grad")


@pytest.mark.parametrize("name,case_id", [
    ("misc.pt", "seq2d_mixed"),
    ("ext_pool.pt", "avgp3d_subm"),
    ("ext_pool.pt", "maxp3d_subm"),
    ("ext_pool.pt", "maxp3d_d2"),
    ("ext_pool.pt", "maxp3d_k5_kv125"),
])
def test_pipeline_golden(golden, name, case_id):
    case = golden(name, case_id)
    expect = case["expect"]
    dtype = getattr(torch, case["dtype"])
    training = bool(case["training"])
    layers = [build_layer(s, dtype) for s in case["layers"]]
    for layer in layers:
        layer.train(training)
    x, feats = _sparse_input(case["input"], training)
    out = x
    with torch.set_grad_enabled(training):
        for layer in layers:
            out = layer(out)
    assert list(out.spatial_shape) == list(expect["out_spatial_shape"])
    order = canonical_order(out.indices.cpu(), out.spatial_shape)
    assert torch.equal(out.indices.cpu()[order], expect["out_indices"])
    assert out.features.dtype == dtype
    assert_close(out.features.cpu()[order], expect["out_features"], expect["atol_out"], "out")
    if not training:
        return
    inv = inverse_permutation(order.to(DEV))
    out.features.backward(expect["grad_out"].to(DEV)[inv].to(out.features.dtype))
    assert_close(feats.grad, expect["grad_input"], expect["atol_grad_input"], "grad_input")
    named = {}
    for li, layer in enumerate(layers):
        for pname, p in layer.named_parameters():
            named[f"{li}.{pname}"] = p
    assert set(named) == set(expect["grad_params"])
    for k, ginfo in expect["grad_params"].items():
        assert_close(named[k].grad, ginfo["grad"], ginfo["atol"], f"{k}.grad")


def test_autocast_eval_dtype(golden):
    """Eval convs bypass autocast and return the weight dtype (reference
    conv.py:453-478, tests/test_module_protocol.py:88-105)."""
    case = golden("proto.pt", "autocast_subm3d")
    expect = case["expect"]
    layer = build_layer(case["layers"][0], torch.float32).eval()
    x, _ = _sparse_input(case["input"], False)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
        out = layer(x)
    assert str(out.features.dtype) == expect["out_dtype"]
    order = canonical_order(out.indices.cpu(), out.spatial_shape)
    assert torch.equal(out.indices.cpu()[order], expect["out_indices"])
    assert_close(out.features.float().cpu()[order], expect["out_features"], expect["atol_out"],
                 "out")


def test_inverse_restores_input_rows():
    """SparseInverseConv3d reproduces the exact input indices of the strided conv
    that shares its key (reference tests/test_conv.py:75-87)."""
    import spconv_triton.pytorch as spconv

    from bench_data import uniform_cloud

    idx = torch.from_numpy(uniform_cloud(3000, [32, 32, 32], seed=4, batch=2)).to(DEV)
    perm = torch.randperm(idx.shape[0], device=DEV)
    idx = idx[perm].contiguous()
    x = spconv.SparseConvTensor(torch.randn(idx.shape[0], 8, device=DEV), idx, [32] * 3, 2)
    down = spconv.SparseConv3d(8, 16, 3, stride=2, padding=1, indice_key="k").to(DEV)
    up = spconv.SparseInverseConv3d(16, 8, 3, indice_key="k").to(DEV)
    y = up(down(x))
    assert torch.equal(y.indices, idx)
    assert y.spatial_shape == [32] * 3


@pytest.mark.parametrize("algo", ["Native", "MaskImplicitGemm"])
def test_native_and_igemm_modules_agree(algo):
    """The same network under both algorithms gives the same outputs."""
    import spconv_triton.pytorch as spconv

    from bench_data import surface_cloud

    idx = torch.from_numpy(surface_cloud(20000, 64, seed=2)).to(DEV)
    torch.manual_seed(0)
    feats = torch.randn(idx.shape[0], 16, device=DEV)

    def run(a):
        torch.manual_seed(1)
        a = getattr(spconv.ConvAlgo, a)
        net = spconv.SparseSequential(
            spconv.SubMConv3d(16, 32, 3, indice_key="a", algo=a),
            spconv.SparseConv3d(32, 32, 3, stride=2, padding=1, algo=a),
            spconv.SubMConv3d(32, 16, 3, algo=a)).to(DEV).eval()
        with torch.no_grad():
            return net(spconv.SparseConvTensor(feats, idx, [64] * 3, 1))

    a = run("Native")
    b = run(algo)
    assert torch.equal(a.indices, b.indices)
    torch.testing.assert_close(a.features, b.features, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("case_id", ["tables_jointable", "tables_addtable"])
def test_tables_golden(golden, case_id):
    """JoinTable / AddTable over two SubMConv2d branches of one input, against
    spconv's outputs (reference tests/test_misc_modules.py:15-33)."""
    import spconv_triton.pytorch as spconv

    case = golden("misc.pt", case_id)
    x, _ = _sparse_input(case["input"], False)
    branches = [build_layer(s, torch.float32) for s in case["branch_specs"]]
    with torch.no_grad():
        outs = [b(x) for b in branches]
        out = getattr(spconv, case["table"])()(outs)
    expect = case["expect"]
    order = canonical_order(out.indices.cpu(), out.spatial_shape)
    assert torch.equal(out.indices.cpu()[order], expect["out_indices"])
    assert_close(out.features.cpu()[order], expect["out_features"], expect["atol_out"], case_id)
    assert list(out.spatial_shape) == list(expect["out_spatial_shape"])


def _keyed_input(n=600, shape=(16, 16, 16), C=8, seed=0):
    import spconv_triton.pytorch as spconv

    rng = np.random.default_rng(seed)
    lin = rng.choice(int(np.prod(shape)), size=n, replace=False)
    c = np.stack(np.unravel_index(lin, shape), 1)
    idx = np.concatenate([np.zeros((n, 1)), c], 1).astype(np.int32)
    return spconv.SparseConvTensor(torch.randn(n, C, device=DEV),
                                   torch.from_numpy(idx).to(DEV), list(shape), 1)


def test_indice_key_validation_errors():
    """indice_key reuse rules (reference conv.py:211-219, :282-289, :515-567,
    tests/test_conv_edge.py:29-45): a non-subm layer on a key that already
    exists, a different algo on a shared key, and subm layers sharing a key
    with a different kernel size, dilation, spatial shape or row count."""
    import spconv_triton.pytorch as spconv

    x = _keyed_input()
    with torch.no_grad():
        a = spconv.SubMConv3d(8, 8, 3, padding=1, indice_key="k").to(DEV)(x)
        # a strided layer may not register a key that exists
        with pytest.raises(AssertionError):
            spconv.SparseConv3d(8, 8, 3, stride=2, padding=1, indice_key="k").to(DEV)(a)
        # the layers of one key must share the algorithm
        with pytest.raises(AssertionError, match="same algo"):
            spconv.SubMConv3d(8, 8, 3, padding=1, indice_key="k",
                              algo=spconv.ConvAlgo.Native).to(DEV)(a)
        with pytest.raises(ValueError, match="same kernel"):
            spconv.SubMConv3d(8, 8, 5, padding=2, indice_key="k",
                              large_kernel_fast_algo=True).to(DEV)(a)
        with pytest.raises(ValueError, match="same dilation"):
            spconv.SubMConv3d(8, 8, 3, padding=2, dilation=2, indice_key="k").to(DEV)(a)
        other = spconv.SparseConvTensor(a.features, a.indices, [20, 16, 16], 1,
                                        indice_dict=a.indice_dict)
        with pytest.raises(ValueError, match="same spatial structure"):
            spconv.SubMConv3d(8, 8, 3, padding=1, indice_key="k").to(DEV)(other)
        fewer = spconv.SparseConvTensor(a.features[:500], a.indices[:500], [16, 16, 16], 1,
                                        indice_dict=a.indice_dict)
        with pytest.raises(ValueError, match="same num of indices"):
            spconv.SubMConv3d(8, 8, 3, padding=1, indice_key="k").to(DEV)(fewer)
        # reuse by a matching subm layer is fine and returns the same rows
        b = spconv.SubMConv3d(8, 8, 3, padding=1, indice_key="k").to(DEV)(a)
        assert b.indices is a.indices
        # an inverse layer on a key its strided layer registered must match it
        d = spconv.SparseConv3d(8, 8, 3, stride=2, padding=1, indice_key="d").to(DEV)(b)
        with pytest.raises(ValueError, match="same kernel"):
            spconv.SparseInverseConv3d(8, 8, 2, indice_key="d").to(DEV)(d)
        up = spconv.SparseInverseConv3d(8, 8, 3, indice_key="d").to(DEV)(d)
        assert torch.equal(up.indices, b.indices)
