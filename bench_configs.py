"""Timings of the benchmark configurations other than the headline one.

``bench.py`` measures the headline layer (one JSON line, the driver's
contract).  This script times the other configurations of the baseline at
their stated sizes, on synthetic clouds from ``bench_data`` and random
weights, and prints one JSON object per configuration:

* ``encoder``: VoxelBackBone8x-style encoder, fp16 eval, batch 4 x ~20k
  LiDAR voxels in [41, 1600, 1408]; rulebooks rebuilt every pass;
* ``resunet``: sparse ResUNet training step (forward + backward), fp16
  autocast, batch 2 x ~120k voxels in [128, 2048, 2048]; rulebooks rebuilt
  every step;
* ``subm4d``: SubMConv4d 3^4, 128 -> 128 fp16, ~500k voxels in
  [64, 512, 512, 512], rulebook cached, with its pairs per row and the
  matrix-core utilisation (useful flop 2 * pairs * C * K);
* ``wide``: SubMConv3d 256 -> 256 fp16, 400k voxels of a 1024^3 surface
  cloud, rulebook cached, with the same two figures;
* ``config1``: SubMConv3d 16 -> 16 fp32, 2,000 uniform voxels in 64^3,
  rulebook rebuilt every pass (the reference's CPU-runnable case);
* ``quickstart``: the reference README chain SubMConv3d(3 -> 32) ->
  SparseConv3d(32 -> 64, s2) -> SparseInverseConv3d(64 -> 32), fp16 eval, 200k
  surface voxels in 256^3, rulebooks rebuilt every pass (config 2);
* ``lidar_c256``: SubMConv3d 256 -> 256 on a 50k-voxel LiDAR cloud, rulebook
  cached, in fp16, IEEE fp32 and fp32 with SPCONV_ALLOW_TF32 (split-bf16
  products), with the pairs per row and the matrix-core utilisation;
* ``ref_c256``: the layer class of the reference's published plots (K3, C256,
  50k voxels in [41, 1600, 1408], batch 1) on uniform voxels: submanifold with
  the rulebook cached, strided and transposed with pair generation, in fp16,
  fp32 and TF32-equivalent;
* ``wgrad``: the weight gradient of each convolution of the ``resunet``
  network, one call per layer, with its achieved algorithmic GB/s.

Usage: ``python bench_configs.py [--config NAME ...] [--reps R]``.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "spconv-triton_amd"))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402
import torch  # noqa: E402

from bench_data import lidar_cloud, surface_cloud, urban_cloud  # noqa: E402

DEV = torch.device("cuda:0")

# (kind, cin, cout, kernel, [stride, padding,] indice_key); every conv is
# followed by BatchNorm + ReLU
ENCODER = [
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

RESUNET = {
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


def build(blocks):
    import spconv_triton.pytorch as spconv

    mods = []
    for blk in blocks:
        kind = blk[0]
        if kind == "pool":
            _, k, stride, key = blk
            mods.append(spconv.SparseMaxPool3d(k, stride, indice_key=key))
            continue
        if kind == "subm":
            _, cin, cout, k, key = blk
            conv = spconv.SubMConv3d(cin, cout, k, padding=1, bias=False, indice_key=key)
        elif kind == "conv":
            _, cin, cout, k, stride, pad, key = blk
            conv = spconv.SparseConv3d(cin, cout, k, stride=stride, padding=pad, bias=False,
                                       indice_key=key)
        else:
            _, cin, cout, k, key = blk
            conv = spconv.SparseInverseConv3d(cin, cout, k, bias=False, indice_key=key)
        mods += [conv, torch.nn.BatchNorm1d(cout), torch.nn.ReLU()]
    return spconv.SparseSequential(*mods).to(DEV)


def median_ms(fn, reps):
    ts = []
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(ts)


def cfg_encoder(reps):
    import spconv_triton.pytorch as spconv

    shape = [41, 1600, 1408]
    idx = lidar_cloud(20000, batch=4, seed=0, shape=shape)
    it = torch.from_numpy(idx).to(DEV)
    feats = torch.rand(idx.shape[0], 4, device=DEV).half()
    net = build(ENCODER).half().eval()

    def step():
        with torch.no_grad():
            return net(spconv.SparseConvTensor(feats, it, shape, 4))

    for _ in range(3):
        step()
    return {"voxels": int(idx.shape[0]), "median_ms": median_ms(step, reps),
            "what": "encoder forward, fp16 eval, rulebooks rebuilt every pass"}


def cfg_resunet(reps):
    import spconv_triton.pytorch as spconv

    shape = [128, 2048, 2048]
    idx = urban_cloud(120000, batch=2, seed=9, shape=shape)
    it = torch.from_numpy(idx).to(DEV)
    n = idx.shape[0]
    feats = torch.rand(n, 4, device=DEV)
    labels = torch.randint(0, 20, (n,), device=DEV)
    parts = {k: build(v).train() for k, v in RESUNET.items()}
    head = spconv.SubMConv3d(32, 20, 1, bias=True).to(DEV)
    join = spconv.JoinTable()
    params = [p for m in parts.values() for p in m.parameters()] + list(head.parameters())

    def step():
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
        for p in params:
            p.grad = None

    for _ in range(3):
        step()
    return {"voxels": int(n), "median_ms": median_ms(step, reps),
            "what": "training step (forward + backward), fp16 autocast, rulebooks rebuilt"}


def _cached_layer(conv, idx, shape, C, reps):
    import spconv_triton.pytorch as spconv

    it = torch.from_numpy(idx).to(DEV)
    feats = torch.randn(idx.shape[0], C, device=DEV).half()
    bs = int(idx[:, 0].max()) + 1
    with torch.no_grad():
        y = conv(spconv.SparseConvTensor(feats, it, shape, bs))
        rb = y.indice_dict[conv.indice_key]
        if getattr(rb, "pair_fwd", None) is not None:  # implicit-GEMM rulebook
            pairs = int((rb.pair_fwd >= 0).sum().item())
        else:  # Native rulebook: per-offset pair counts
            pairs = int(rb.indice_pair_num.sum().item())
            if rb.is_subm:  # it lists the offsets before the centre only (symmetry)
                pairs = 2 * pairs + int(rb.out_indices.shape[0])
        xc = spconv.SparseConvTensor(feats, it, shape, bs, indice_dict=y.indice_dict)
        for _ in range(5):
            conv(xc)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 10 * reps
        e0.record()
        for _ in range(n):
            conv(xc)
        e1.record()
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n, pairs


def _mfma_report(ms, pairs, n, C, K):
    """Useful matrix-core work of a layer: 2 * pairs * C * K flop over its time,
    as a fraction of the fp16 dense peak (2.5 PFLOP/s)."""
    tflops = 2.0 * pairs * C * K / (ms * 1e-3) / 1e12
    return {"pairs_per_row": round(pairs / n, 3), "useful_tflops": round(tflops, 1),
            "matrix_core_frac": round(tflops / 2500.0, 4), "peak_used": "fp16 2.5 PFLOP/s"}


def cfg_subm4d(reps):
    import spconv_triton.pytorch as spconv

    # 64 time steps of a slowly drifting surface cloud in 512^3
    rng = np.random.default_rng(0)
    base = surface_cloud(8000, 512, seed=3)[:, 1:].astype(np.int64)
    rows = []
    for t in range(64):
        c = np.clip(base + (np.array([t // 8, t // 16, t // 4]) % 512), 0, 511)
        c = c[rng.random(c.shape[0]) < 0.98]
        rows.append(np.concatenate([np.zeros((c.shape[0], 1), np.int64),
                                    np.full((c.shape[0], 1), t), c], 1))
    idx = np.unique(np.concatenate(rows).astype(np.int32), axis=0)
    torch.manual_seed(0)
    conv = spconv.SubMConv4d(128, 128, 3, padding=1, bias=False, indice_key="k").to(DEV)
    ms, pairs = _cached_layer(conv.half().eval(), idx, [64, 512, 512, 512], 128, reps)
    return {"voxels": int(idx.shape[0]), "median_ms": ms,
            **_mfma_report(ms, pairs, int(idx.shape[0]), 128, 128),
            "what": "SubMConv4d 3^4 128->128 fp16 forward, rulebook cached (mean)"}


def cfg_wide(reps):
    import spconv_triton.pytorch as spconv

    idx = surface_cloud(400000, 1024, seed=0)
    torch.manual_seed(0)
    conv = spconv.SubMConv3d(256, 256, 3, padding=1, bias=False, indice_key="k").to(DEV)
    ms, pairs = _cached_layer(conv.half().eval(), idx, [1024] * 3, 256, reps)
    return {"voxels": int(idx.shape[0]), "median_ms": ms,
            **_mfma_report(ms, pairs, int(idx.shape[0]), 256, 256),
            "what": "SubMConv3d 256->256 fp16 forward, 1024^3 surface cloud, rulebook cached (mean)"}


def cfg_config1(reps):
    import spconv_triton.pytorch as spconv

    from bench_data import uniform_cloud

    idx = uniform_cloud(2000, [64] * 3, seed=0)
    it = torch.from_numpy(idx).to(DEV)
    torch.manual_seed(0)
    feats = torch.randn(idx.shape[0], 16, device=DEV)
    conv = spconv.SubMConv3d(16, 16, 3, padding=1, indice_key="k").to(DEV).eval()

    def step():
        with torch.no_grad():
            return conv(spconv.SparseConvTensor(feats, it, [64] * 3, 1))

    for _ in range(5):
        step()
    return {"voxels": int(idx.shape[0]), "median_ms": median_ms(step, 10 * reps),
            "what": "SubMConv3d 16->16 fp32 eval, rulebook rebuilt every pass (Python host in "
                    "the loop)"}


def cfg_quickstart(reps):
    import spconv_triton.pytorch as spconv

    idx = surface_cloud(200_000, 256, seed=0)
    it = torch.from_numpy(idx).to(DEV)
    torch.manual_seed(0)
    feats = torch.randn(idx.shape[0], 3, device=DEV).half()
    net = spconv.SparseSequential(
        spconv.SubMConv3d(3, 32, 3, padding=1, indice_key="subm0"),
        spconv.SparseConv3d(32, 64, 3, stride=2, padding=1, indice_key="down0"),
        spconv.SparseInverseConv3d(64, 32, 3, indice_key="down0"),
    ).to(DEV).half().eval()

    def step():
        with torch.no_grad():
            return net(spconv.SparseConvTensor(feats, it, [256] * 3, 1))

    for _ in range(3):
        step()
    return {"voxels": int(idx.shape[0]), "median_ms": median_ms(step, reps),
            "what": "quickstart chain fp16 eval, rulebooks rebuilt every pass"}


def cfg_lidar_c256(reps):
    import spconv_triton.pytorch as spconv
    from spconv_triton import constants

    shape = [41, 1600, 1408]
    idx = lidar_cloud(50000, batch=1, seed=0, shape=shape)
    it = torch.from_numpy(idx).to(DEV)
    n = int(idx.shape[0])
    out = {"voxels": n}
    for name, dtype, tf32, peak in (("fp16", torch.float16, False, 2500.0),
                                    ("fp32", torch.float32, False, 157.3),
                                    ("tf32", torch.float32, True, 2500.0 / 3)):
        torch.manual_seed(0)
        conv = spconv.SubMConv3d(256, 256, 3, padding=1, bias=False, indice_key="k").to(DEV)
        conv = conv.to(dtype).eval()
        feats = torch.randn(n, 256, device=DEV).to(dtype)
        prev = constants.SPCONV_ALLOW_TF32
        constants.SPCONV_ALLOW_TF32 = tf32
        try:
            with torch.no_grad():
                y = conv(spconv.SparseConvTensor(feats, it, shape, 1))
                pairs = int((y.indice_dict["k"].pair_fwd >= 0).sum().item())
                xc = spconv.SparseConvTensor(feats, it, shape, 1, indice_dict=y.indice_dict)
                for _ in range(5):
                    conv(xc)
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                k = 10 * reps
                e0.record()
                for _ in range(k):
                    conv(xc)
                e1.record()
                torch.cuda.synchronize()
                ms = e0.elapsed_time(e1) / k
        finally:
            constants.SPCONV_ALLOW_TF32 = prev
        tflops = 2.0 * pairs * 256 * 256 / (ms * 1e-3) / 1e12
        out[name] = {"ms": round(ms, 4), "pairs_per_row": round(pairs / n, 3),
                     "useful_tflops": round(tflops, 1),
                     "matrix_core_frac": round(tflops / peak, 4),
                     "peak_used": {"fp16": "fp16 2.5 PFLOP/s",
                                   "fp32": "fp32 matrix 157.3 TFLOP/s",
                                   "tf32": "bf16 2.5 PFLOP/s / 3 products"}[name]}
    out["what"] = "SubMConv3d 256->256 forward, rulebook cached (mean of events)"
    return out


def _event_ms(fn, n):
    """Mean ms per call of ``fn`` over ``n`` back-to-back calls, between two
    events (the calls that sync the host, such as pair generation with an
    output-size readback, are included as the reference's timings include
    them)."""
    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n


def cfg_ref_c256(reps):
    """The layer class of the reference's published plots (K3, C256, batch 1,
    ~50k voxels in 41 x 1600 x 1408): submanifold with the rulebook cached,
    strided (k3 s2 p1) and transposed (k3 s2) with the rulebook rebuilt every
    pass.  The reference's harness and cloud are not published; the voxels here
    are uniform in the grid."""
    import spconv_triton.pytorch as spconv
    from bench_data import uniform_cloud
    from spconv_triton import constants

    shape = [41, 1600, 1408]
    idx = uniform_cloud(50000, shape, seed=0)
    it = torch.from_numpy(idx).to(DEV)
    n = int(idx.shape[0])
    out = {"voxels": n}
    for name, dtype, tf32 in (("fp16", torch.float16, False), ("fp32", torch.float32, False),
                              ("tf32", torch.float32, True)):
        torch.manual_seed(0)
        feats = torch.randn(n, 256, device=DEV).to(dtype)
        subm = spconv.SubMConv3d(256, 256, 3, padding=1, bias=False, indice_key="k")
        down = spconv.SparseConv3d(256, 256, 3, stride=2, padding=1, bias=False)
        up = spconv.SparseConvTranspose3d(256, 256, 3, stride=2, bias=False)
        subm, down, up = (m.to(DEV).to(dtype).eval() for m in (subm, down, up))
        prev = constants.SPCONV_ALLOW_TF32
        constants.SPCONV_ALLOW_TF32 = tf32
        try:
            with torch.no_grad():
                y = subm(spconv.SparseConvTensor(feats, it, shape, 1))
                pairs = int((y.indice_dict["k"].pair_fwd >= 0).sum().item())
                xc = spconv.SparseConvTensor(feats, it, shape, 1, indice_dict=y.indice_dict)
                k = 10 * reps
                res = {"subm_ms": _event_ms(lambda: subm(xc), k),
                       "sparse_s2_ms": _event_ms(
                           lambda: down(spconv.SparseConvTensor(feats, it, shape, 1)), k),
                       "transpose_s2_ms": _event_ms(
                           lambda: up(spconv.SparseConvTensor(feats, it, shape, 1)), k)}
                n_up = int(up(spconv.SparseConvTensor(feats, it, shape, 1)).features.shape[0])
        finally:
            constants.SPCONV_ALLOW_TF32 = prev
        out[name] = {key: round(v, 4) for key, v in res.items()}
    out["subm_pairs_per_row"] = round(pairs / n, 3)
    out["transpose_out_voxels"] = n_up
    out["what"] = ("K3 C256 batch 1, 50k uniform voxels in 41x1600x1408: subm forward with the "
                   "rulebook cached; strided and transposed forwards with pair generation, "
                   "mean of events")
    return out


def cfg_wgrad(reps):
    """The weight gradient of every convolution of the sparse ResUNet training
    step (config 4, fp16 autocast, 2 x 120k urban voxels): the step runs once
    with the weight-gradient calls recorded, then each call is timed on its
    own.  Algorithmic bytes of a call: its pairs' gathered rows,
    2 * P * (C + K), plus the 8-byte (input row, output row) signal of each
    pair."""
    import spconv_triton.pytorch as spconv
    from spconv_triton.pytorch._impl import gemm as G

    shape = [128, 2048, 2048]
    idx = urban_cloud(120000, batch=2, seed=9, shape=shape)
    it = torch.from_numpy(idx).to(DEV)
    n = idx.shape[0]
    feats = torch.rand(n, 4, device=DEV)
    labels = torch.randint(0, 20, (n,), device=DEV)
    parts = {k: build(v).train() for k, v in RESUNET.items()}
    head = spconv.SubMConv3d(32, 20, 1, bias=True).to(DEV)
    join = spconv.JoinTable()
    calls = []
    orig = G.conv_backward_weight

    def record(features, grad_out, pair_fwd, weight_shape_krsc, fp32_accum=None):
        calls.append((features, grad_out, pair_fwd, tuple(weight_shape_krsc)))
        return orig(features, grad_out, pair_fwd, weight_shape_krsc, fp32_accum)

    G.conv_backward_weight = record
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
            loss = torch.nn.functional.cross_entropy(head(u).features.float(), labels)
        loss.backward()
    finally:
        G.conv_backward_weight = orig
    layers = []
    tot_ms = tot_bytes = 0.0
    for xf, gf, pf, wshape in calls:
        K, C, kv = wshape[0], wshape[-1], int(pf.shape[0])
        P = int((pf >= 0).sum().item())
        ms = _event_ms(lambda: orig(xf, gf, pf, wshape), 5 * reps)
        nbytes = float(xf.element_size()) * P * (C + K) + 8.0 * P
        tot_ms += ms
        tot_bytes += nbytes
        layers.append({"C": C, "K": K, "kv": kv, "pairs": P, "dtype": str(xf.dtype)[6:],
                       "ms": round(ms, 4), "GBps": round(nbytes / ms / 1e6, 1)})
    return {"layers": layers, "total_ms": tot_ms, "total_GBps": round(tot_bytes / tot_ms / 1e6, 1),
            "frac_of_8TBps": round(tot_bytes / tot_ms / 1e6 / 8000.0, 3)}


CONFIGS = {"encoder": cfg_encoder, "resunet": cfg_resunet, "subm4d": cfg_subm4d,
           "wide": cfg_wide, "config1": cfg_config1, "quickstart": cfg_quickstart,
           "lidar_c256": cfg_lidar_c256, "ref_c256": cfg_ref_c256, "wgrad": cfg_wgrad}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--config", nargs="*", choices=sorted(CONFIGS), default=list(CONFIGS))
    ap.add_argument("--reps", type=int, default=10)
    args = ap.parse_args()
    if not torch.cuda.is_available():
        print("bench_configs.py needs a GPU", file=sys.stderr)
        return 2
    for name in args.config:
        res = CONFIGS[name](args.reps)
        print(json.dumps({"config": name, **{k: (round(v, 4) if isinstance(v, float) else v)
                                            for k, v in res.items()}}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
