"""Run golden pipeline cases through the CPU oracle (test infrastructure).

Sparse ops go through ``oracle/oracle.py`` (fp64 GEMM, sort-based pair
generation); dense glue (BatchNorm, ReLU, concatenation) runs in torch on the
CPU in float64, with autograd wiring the oracle's dgrad/wgrad.  The layer
semantics restated here are those of the reference's module layer:

* algo choice, conv1x1 quirk, train/eval bias placement, indice_key reuse and
  the inverse-conv table swap: ``spconv_triton/pytorch/conv.py:95-103, :119-513``
* max-pool algo choice: ``spconv_triton/pytorch/pool.py:58-66, :84-235``
* avg-pool: ``spconv_triton/pytorch/pool.py:276-403``
* JoinTable: ``spconv_triton/pytorch/tables.py:15-42``
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import oracle as orc  # noqa: E402


def expand_nd(ndim, val):
    if isinstance(val, int):
        return [val] * ndim
    res = list(val)
    assert len(res) == ndim
    return [int(v) for v in res]


class OTensor:
    """Minimal stand-in for SparseConvTensor on the CPU oracle."""

    def __init__(self, features, indices, spatial_shape, batch_size, indice_dict=None):
        self.features = features
        self.indices = np.ascontiguousarray(np.asarray(indices, dtype=np.int32))
        self.spatial_shape = [int(s) for s in spatial_shape]
        self.batch_size = int(batch_size)
        self.indice_dict = indice_dict if indice_dict is not None else {}

    def replace(self, feats):
        return OTensor(feats, self.indices, self.spatial_shape, self.batch_size, self.indice_dict)


# Storage precision to emulate (None: plain fp64).  With torch.float16 the
# oracle rounds every tensor that the GPU path stores in fp16 under
# torch.autocast -- sparse-op inputs, weights and outputs, dense-glue outputs,
# and the gradients flowing back through each of them -- while all arithmetic
# stays fp64, so only accumulation order separates it from the GPU.
ROUND = None


class _RoundFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, dtype):
        ctx.dtype = dtype
        return x.to(dtype).to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        return g.to(ctx.dtype).to(g.dtype), None


def _r(x):
    return x if ROUND is None else _RoundFn.apply(x, ROUND)


class _GemmFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, feats, weight, pf, pb):
        K = weight.shape[0]
        C = weight.shape[-1]
        w = weight.detach().reshape(K, -1, C).numpy()
        out = orc.gemm_fwd(feats.detach().numpy(), w, pf)
        ctx.save_for_backward(feats, weight)
        ctx.pf, ctx.pb = pf, pb
        return torch.from_numpy(out)

    @staticmethod
    def backward(ctx, g):
        feats, weight = ctx.saved_tensors
        K = weight.shape[0]
        C = weight.shape[-1]
        w = weight.detach().reshape(K, -1, C).numpy()
        gn = g.detach().contiguous().numpy()
        dx = orc.gemm_dgrad(gn, w, ctx.pb)
        dw = orc.gemm_wgrad(feats.detach().numpy(), gn, ctx.pf, K, C)
        return torch.from_numpy(dx), torch.from_numpy(dw).reshape(weight.shape), None, None


class _MaxPoolFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, feats, pf, pb):
        out = orc.maxpool_fwd(feats.detach().numpy(), pf)
        ctx.save_for_backward(feats)
        ctx.out = out
        ctx.pb = pb
        return torch.from_numpy(out)

    @staticmethod
    def backward(ctx, g):
        (feats,) = ctx.saved_tensors
        dx = orc.maxpool_bwd(feats.detach().numpy(), ctx.out, g.detach().contiguous().numpy(), ctx.pb)
        return torch.from_numpy(dx), None, None


class _AvgPoolFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, feats, pf, pb):
        out, count = orc.avgpool_fwd(feats.detach().numpy(), pf)
        ctx.count = count
        ctx.pb = pb
        return torch.from_numpy(out)

    @staticmethod
    def backward(ctx, g):
        dx = orc.avgpool_bwd(g.detach().contiguous().numpy(), ctx.count, ctx.pb)
        return torch.from_numpy(dx), None, None


class OConv:
    def __init__(self, ndim, in_channels, out_channels, kernel_size=3, stride=1, padding=0,
                 dilation=1, bias=True, subm=False, transposed=False, inverse=False,
                 indice_key=None, output_padding=0, algo=None, **_):
        self.ndim = ndim
        self.cin, self.cout = in_channels, out_channels
        self.ksize = expand_nd(ndim, kernel_size)
        self.stride = expand_nd(ndim, stride)
        self.padding = expand_nd(ndim, padding)
        self.dilation = expand_nd(ndim, dilation)
        self.output_padding = expand_nd(ndim, output_padding)
        self.subm, self.transposed, self.inverse = subm, transposed, inverse
        self.indice_key = indice_key
        kv = int(np.prod(self.ksize))
        self.conv1x1 = kv == 1 and (subm or int(np.prod(self.stride)) == 1)
        self.weight = torch.zeros(out_channels, *self.ksize, in_channels, dtype=torch.float64)
        self.bias = torch.zeros(out_channels, dtype=torch.float64) if bias else None

    def params(self):
        out = {"weight": self.weight}
        if self.bias is not None:
            out["bias"] = self.bias
        return out

    def __call__(self, x: OTensor, training=True):
        feats = x.features
        if self.conv1x1:
            # raw reinterpretation (conv.py:198-201)
            out = _r(_r(feats) @ _r(self.weight).view(self.cin, self.cout))
            if self.bias is not None:
                out = _r(out + self.bias)
            return x.replace(out)
        indice_dict = dict(x.indice_dict)
        if self.inverse:
            d = x.indice_dict[self.indice_key]
            pf, pb = d["pair_bwd"], d["pair_fwd"]
            outids = d["indices"]
            out_shape = d["spatial_shape"]
        elif self.indice_key is not None and self.indice_key in x.indice_dict:
            d = x.indice_dict[self.indice_key]
            pf, pb, outids, out_shape = d["pair_fwd"], d["pair_bwd"], d["out_indices"], d["out_spatial_shape"]
        else:
            res = orc.igemm_pairs(x.indices, x.batch_size, x.spatial_shape, self.ksize, self.stride,
                                  self.padding, self.dilation, self.output_padding, self.subm,
                                  self.transposed, True)
            outids, pf, pb = res[0], res[2], res[3]
            if self.subm:
                out_shape = list(x.spatial_shape)
            elif self.transposed:
                out_shape = orc.get_deconv_output_size(x.spatial_shape, self.ksize, self.stride,
                                                       self.padding, self.dilation, self.output_padding)
            else:
                out_shape = orc.get_conv_output_size(x.spatial_shape, self.ksize, self.stride,
                                                     self.padding, self.dilation)
            if self.indice_key is not None:
                indice_dict[self.indice_key] = {"pair_fwd": pf, "pair_bwd": pb, "out_indices": outids,
                                                "indices": x.indices, "spatial_shape": list(x.spatial_shape),
                                                "out_spatial_shape": out_shape}
        out = _r(_GemmFn.apply(_r(feats), _r(self.weight), pf, pb))
        if self.bias is not None:
            out = out + self.bias
        return OTensor(out, outids, out_shape, x.batch_size, indice_dict)


class OPool:
    def __init__(self, ndim, kernel_size=3, stride=1, padding=0, dilation=1, subm=False,
                 indice_key=None, is_max=True, algo=None, **_):
        self.ndim = ndim
        self.ksize = expand_nd(ndim, kernel_size)
        self.stride = self.ksize.copy() if stride is None else expand_nd(ndim, stride)
        self.padding = expand_nd(ndim, padding)
        self.dilation = expand_nd(ndim, dilation)
        self.subm = subm
        self.is_max = is_max
        self.indice_key = indice_key  # registered like a conv's (reference pool.py:152-201)

    def params(self):
        return {}

    def __call__(self, x: OTensor, training=True):
        res = orc.igemm_pairs(x.indices, x.batch_size, x.spatial_shape, self.ksize, self.stride,
                              self.padding, self.dilation, [0] * self.ndim, self.subm, False, True)
        outids, pf, pb = res[0], res[2], res[3]
        out_shape = list(x.spatial_shape) if self.subm else orc.get_conv_output_size(
            x.spatial_shape, self.ksize, self.stride, self.padding, self.dilation)
        fn = _MaxPoolFn if self.is_max else _AvgPoolFn
        out = _r(fn.apply(_r(x.features), pf, pb))
        indice_dict = dict(x.indice_dict)
        if self.indice_key is not None:
            indice_dict[self.indice_key] = {"pair_fwd": pf, "pair_bwd": pb, "out_indices": outids,
                                            "indices": x.indices,
                                            "spatial_shape": list(x.spatial_shape),
                                            "out_spatial_shape": out_shape}
        return OTensor(out, outids, out_shape, x.batch_size, indice_dict)


class ODense:
    """BatchNorm1d / ReLU applied to features."""

    def __init__(self, mod):
        self.mod = mod.double()

    def params(self):
        return dict(self.mod.named_parameters())

    def __call__(self, x: OTensor, training=True):
        self.mod.train(training)
        return x.replace(_r(self.mod(x.features)))


class OSeq:
    def __init__(self, children):
        self.children = children

    def params(self):
        out = {}
        for i, c in enumerate(self.children):
            for k, v in c.params().items():
                out[f"{i}.{k}"] = v
        return out

    def __call__(self, x, training=True):
        for c in self.children:
            x = c(x, training)
        return x


_CONV = {
    "SubMConv": dict(subm=True), "SparseConv": dict(), "SparseInverseConv": dict(inverse=True),
    "SparseConvTranspose": dict(transposed=True),
}


def build_layer(spec):
    cls = spec["cls"]
    ctor = dict(spec.get("ctor") or {})
    if cls == "SparseSequential":
        layer = OSeq([build_layer(c) for c in spec["children"]])
    elif cls.startswith("nn."):
        layer = ODense(getattr(torch.nn, cls[3:])(**ctor))
    elif cls in ("SparseMaxPool", "SparseAvgPool"):
        layer = OPool(is_max=cls == "SparseMaxPool", **ctor)
    elif cls[:-2] in ("SparseMaxPool", "SparseAvgPool"):
        layer = OPool(int(cls[-2]), is_max=cls.startswith("SparseMaxPool"), **ctor)
    else:
        base, nd = cls[:-2], int(cls[-2])
        layer = OConv(nd, **_CONV[base], **ctor)
    params = spec.get("params") or {}
    own = layer.params() if not isinstance(layer, OSeq) else {}
    with torch.no_grad():
        for name, value in params.items():
            if value is None:
                continue
            own[name].copy_(value.to(torch.float64))
    return layer


def run_pipeline(case):
    """Returns (out OTensor, feats leaf, layers)."""
    layers = [build_layer(s) for s in case["layers"]]
    for layer in layers:
        for p in layer.params().values():
            p.requires_grad_(True)
    inp = case["input"]
    feats = inp["features"].to(torch.float64).clone().requires_grad_(True)
    x = OTensor(feats, inp["indices"].numpy(), inp["spatial_shape"], inp["batch_size"])
    training = bool(case.get("training", True))
    for layer in layers:
        x = layer(x, training)
    return x, feats, layers


def build_unet(state_dict, in_channels=6, base=16):
    """The reference test network (tests/helpers.py:332-371 of the reference)."""
    stem = OSeq([OConv(3, in_channels, base, 3, padding=1, indice_key="s0", bias=False, subm=True),
                 ODense(torch.nn.BatchNorm1d(base)), ODense(torch.nn.ReLU()),
                 OConv(3, base, base, 3, padding=1, indice_key="s0", bias=False, subm=True)])
    down = OConv(3, base, base * 2, 3, stride=2, padding=1, indice_key="d0", bias=False)
    mid = OSeq([OConv(3, base * 2, base * 2, 3, padding=1, indice_key="s1", bias=False, subm=True),
                ODense(torch.nn.BatchNorm1d(base * 2)), ODense(torch.nn.ReLU())])
    up = OConv(3, base * 2, base, 3, indice_key="d0", bias=False, inverse=True)
    head = OConv(3, base * 2, 8, 1, bias=True, subm=True)
    mods = {"stem": stem, "down": down, "mid": mid, "up": up, "head": head}
    named = {}
    for mname, m in mods.items():
        for k, v in m.params().items():
            named[f"{mname}.{k}"] = v
    bn_bufs = {"stem.1": stem.children[1].mod, "mid.1": mid.children[1].mod}
    with torch.no_grad():
        for k, v in state_dict.items():
            if k in named:
                named[k].copy_(v.to(torch.float64))
            else:
                mod_name, buf = k.rsplit(".", 1)
                getattr(bn_bufs[mod_name], buf).copy_(v)
    for p in named.values():
        p.requires_grad_(True)

    def forward(x):
        a = stem(x)
        b = down(a)
        c = mid(b)
        d = up(c)
        e = d.replace(torch.cat([d.features, a.features], 1))
        return head(e)

    return forward, named


def canonical_order(indices: np.ndarray, spatial_shape) -> np.ndarray:
    lin = indices[:, 0].astype(np.int64)
    for i, s in enumerate(spatial_shape):
        lin = lin * int(s) + indices[:, i + 1].astype(np.int64)
    return np.argsort(lin, kind="stable")


def kaiming_bound(fan_in: int, a: float = math.sqrt(5)) -> float:
    gain = math.sqrt(2.0 / (1 + a * a))
    return math.sqrt(3.0) * gain / math.sqrt(fan_in)
