"""Benchmark of the sparse-convolution hot path on one MI355X.

Workload (BASELINE.json metric): SubMConv3d 3x3x3, 64 -> 64 channels, fp16,
eval, bias on, Kaiming-uniform weights; input 200k unique voxels of a seeded
surface-like cloud (sphere shells + plane patches) in a 256^3 grid, batch 1,
features N(0, 1).  A step is one forward of the layer with its rulebook
cached under its indice_key (the reference times subm "with the neighborhood
map cached & reused"); steps are replayed from a HIP graph so the GPU, not the
Python host, is measured.  Also reported:

* pairgen_ms: cold build of the subm rulebook (hash build + probe + mask sort)
  plus the gather plan the GEMM stages its rows with (both are built once per
  rulebook and reused by every layer sharing the indice_key);
* eager_ms: the same forward called from Python without a graph;
* roofline: the gather-GEMM kernel's algorithmic bytes per launch over its
  average launch time (HIP events on the stream it runs on);
* cpu_baseline: the CPU oracle (C/OpenMP restatement of the reference
  algorithm, fp32) on the same layer, on a bounded sample of rows.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "spconv-triton_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "fwd ms + Mvoxels/s, SubMConv3d 64→64 fp16 @200k voxels; pairgen ms; %roofline"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
N_VOXELS = 200_000
GRID = 256
C_IN = C_OUT = 64
KV = 27


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_layer(torch, spconv, dev):
    torch.manual_seed(0)
    conv = spconv.SubMConv3d(C_IN, C_OUT, 3, padding=1, bias=True, indice_key="subm0")
    return conv.to(dev).half().eval()


def gemm_bytes(n_in: int, n_out: int, plan_bytes: int) -> int:
    """Algorithmic HBM bytes of one forward launch: features read once, output
    written once, weights once, and the gather-plan entries the kernel needs
    (see plan_read_bytes)."""
    e = 2
    return e * (n_in * C_IN + n_out * C_OUT + KV * C_IN * C_OUT) + plan_bytes


def plan_read_bytes(plan, kv: int, n_out: int) -> int:
    """Bytes of the gather plan the staged kernel needs: per tile its
    distinct-row list (4 B per row) and, per item of its groups of 4 items, one
    uint16 LDS address per output row (csrc/sp_plan.h layout: 256-row tiles,
    896 staged rows)."""
    import numpy as np

    tile, lds_rows = 256, 896
    nt = (n_out + tile - 1) // tile
    buf = plan.cpu().numpy()
    count = buf[256:256 + nt * 4].view(np.int32).astype(np.int64)
    align = lambda v: (v + 255) // 256 * 256
    ovf_off = align(256 + nt * 4)
    rows_off = align(ovf_off + nt * 4)
    nact_off = align(rows_off + nt * lds_rows * 4)
    nact = buf[nact_off:nact_off + nt * 4].view(np.int32).astype(np.int64)
    staged = count < lds_rows
    items = (nact + 3) // 4 * 4
    return int((count[staged] * 4).sum() + (items[staged] * tile * 2).sum())


def cpu_baseline(idx, feats_np, w_np, b_np, pf_np):
    """Oracle forward (fp32) on a bounded row sample; returns the dict for the JSON line."""
    import numpy as np

    from oracle import oracle as orc

    threads = len(os.sched_getaffinity(0))
    threads = min(threads, int(os.environ.get("OMP_NUM_THREADS", threads)))
    orc.set_num_threads(threads)
    rows = 50_000
    pf_s = np.ascontiguousarray(pf_np[:, :rows])
    w = w_np.reshape(C_OUT, KV, C_IN).astype(np.float32)
    x = feats_np.astype(np.float32)
    reps = 0
    t0 = time.perf_counter()
    while True:
        orc.gemm_fwd_f32(x, w, pf_s, b_np.astype(np.float32))
        reps += 1
        el = time.perf_counter() - t0
        if el > 10.0 or reps >= 50:
            break
    per_row = el / (reps * rows)
    # the reference's pair generation on the CPU (sort + binary search) for the full cloud
    t1 = time.perf_counter()
    orc.igemm_pairs(idx, 1, [GRID] * 3, [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3, True, False,
                    False)
    pairgen_s = time.perf_counter() - t1
    return {
        "value": round(1.0 / per_row / 1e6, 4),
        "unit": "Mvoxels/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle/spconv_oracle.c gemm_fwd_f32 (fp32; the host has no fp16 GEMM) on "
                   f"{rows} of the {N_VOXELS} output rows x {reps} passes, {threads} OpenMP "
                   f"threads; oracle sort-based pair generation of the full cloud "
                   f"{pairgen_s * 1e3:.1f} ms"),
        "pairgen_ms": round(pairgen_s * 1e3, 2),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device copy (reference point for the "
                         "FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch

        src = torch.ones(64 * 2 ** 20, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel() * 4}))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the sparse-conv hot path would shard by batch sample)",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import spconv_triton.pytorch as spconv
    from bench_data import surface_cloud
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops
    from spconv_triton.pytorch._impl import gemm as gemm_impl

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    log("generating the 200k-voxel surface cloud")
    idx_np = surface_cloud(N_VOXELS, GRID, seed=0)
    idx = torch.from_numpy(idx_np).to(dev)
    torch.manual_seed(1)
    feats = torch.randn(N_VOXELS, C_IN, device=dev).half()
    conv = build_layer(torch, spconv, dev)

    # ---- cold pair generation (rulebook + gather plan) ---------------------
    def pairgen():
        return ops.get_indice_pairs_implicit_gemm(idx, 1, [GRID] * 3, ConvAlgo.MaskImplicitGemm,
                                                  [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3,
                                                  True, is_train=False)

    log("pair generation")
    for _ in range(5):
        res = pairgen()
        gemm_impl.gather_plan(res[2], N_VOXELS)
    torch.cuda.synchronize()
    pg, pg_rules = [], []
    for _ in range(30):
        s, m, e = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        s.record()
        res = pairgen()
        m.record()
        gemm_impl.gather_plan(res[2], N_VOXELS)
        e.record()
        torch.cuda.synchronize()
        pg.append(s.elapsed_time(e))
        pg_rules.append(s.elapsed_time(m))
    pairgen_ms = statistics.median(pg)
    rules_ms = statistics.median(pg_rules)
    pf = res[2]
    n_pairs = int((pf >= 0).sum().item())

    # ---- forward with the rulebook cached --------------------------------
    with torch.no_grad():
        x0 = spconv.SparseConvTensor(feats, idx, [GRID] * 3, 1)
        y0 = conv(x0)  # builds and caches the rulebook under "subm0"
        xc = spconv.SparseConvTensor(feats, idx, [GRID] * 3, 1, indice_dict=y0.indice_dict)
        for _ in range(3):
            y = conv(xc)
        torch.cuda.synchronize()
        # eager timing (Python host in the loop)
        t0 = time.perf_counter()
        for _ in range(200):
            y = conv(xc)
        torch.cuda.synchronize()
        eager_ms = (time.perf_counter() - t0) / 200 * 1e3

        log("capturing the forward in a HIP graph")
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                conv(xc)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            yg = conv(xc)
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(yg.features, y.features):
            raise RuntimeError("graph replay differs from the eager forward")

        log(f"warmup {args.warmup}, timed {args.steps} steps")
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        wall_s = time.perf_counter() - t0
        ms_per_step = wall_s / args.steps * 1e3

        # kernel-level timing for the roofline: events on the stream the GEMM
        # kernel runs on (torch's current stream, which the library uses)
        stream = torch.cuda.current_stream()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 500
        s.record(stream)
        for _ in range(reps):
            graph.replay()
        e.record(stream)
        torch.cuda.synchronize()
        kernel_ms = s.elapsed_time(e) / reps

    # HBM bytes per launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE runs,
    # scaled by a 256 MiB copy (profiles/gather_gemm_traffic.json)
    traffic = None
    tfile = ROOT / "profiles" / "gather_gemm_traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("bytes_per_launch")
    plan = gemm_impl.gather_plan(y0.indice_dict["subm0"].pair_fwd, N_VOXELS)
    n_overflow = gemm_impl.plan_overflow_count(plan)
    nbytes = gemm_bytes(N_VOXELS, N_VOXELS, plan_read_bytes(plan, KV, N_VOXELS))
    flops = 2.0 * n_pairs * C_IN * C_OUT
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    mvox = N_VOXELS / (ms_per_step * 1e-3) / 1e6

    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline (oracle)")
        w_np = conv.weight.detach().float().cpu().numpy()
        b_np = conv.bias.detach().float().cpu().numpy()
        cpu = cpu_baseline(idx_np, feats.float().cpu().numpy(), w_np, b_np, pf.cpu().numpy())

    line = {
        "metric": METRIC,
        "value": round(mvox, 2),
        "unit": "Mvoxels/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "SubMConv3d k3 64->64 fp16 eval, 200k-voxel surface cloud in 256^3, "
                        "batch 1, rulebook cached, HIP-graph replay",
            "n_voxels": N_VOXELS,
            "pairs": n_pairs,
            "parallelism": "single_gpu",
        },
        "fwd_ms": round(ms_per_step, 5),
        "eager_ms": round(eager_ms, 5),
        "pairgen_ms": round(pairgen_ms, 4),
        "pairgen_parts_ms": {"rulebook": round(rules_ms, 4),
                             "gather_plan": round(pairgen_ms - rules_ms, 4)},
        "overflow_tiles": int(n_overflow),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "gather_gemm_staged<f16,f16,VEC>",
            "kernel_ms": round(kernel_ms, 5),
            "algorithmic_bytes": nbytes,
            "mfma_tflops": round(flops / (kernel_ms * 1e-3) / 1e12, 2),
            "mfma_frac": round(flops / (kernel_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
