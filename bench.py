"""Benchmark of the sparse-convolution hot path on one MI355X.

Workload (BASELINE.json metric): SubMConv3d 3x3x3, 64 -> 64 channels, fp16,
eval, bias on, Kaiming-uniform weights; input 200k unique voxels of a seeded
surface-like cloud (sphere shells + plane patches) in a 256^3 grid, batch 1,
features N(0, 1).  A step is one forward of the layer called from Python
with its rulebook cached under its indice_key (the reference times subm "with
the neighborhood map cached & reused", also from Python); the relaid weights
are cached too, until the weight changes.  Also reported:

* pairgen_ms: cold build of the subm rulebook (lookup grid + probe + mask
  sort) plus the gather plan the GEMM stages its rows with (both are built once
  per rulebook and reused by every layer sharing the indice_key), with events
  around a build issued from an idle host; pairgen_gpu_ms: the same build
  queued behind GPU work, so its kernels run back to back;
* graph_ms: the forward replayed from a HIP graph (the graph also holds the
  weight relayout, so that replays see in-place weight updates);
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


def _time_reps(fn, budget_s, max_reps):
    reps = 0
    t0 = time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el > budget_s or reps >= max_reps:
            return el / reps, reps


def cpu_baseline(idx, feats_np, w_np, b_np, pf_np):
    """Oracle forward (fp32) on bounded row samples; returns the dict for the JSON line.

    * value: all allowed host threads, 50k of the 200k output rows;
    * single_thread: one thread, 5k rows;
    * config1: BASELINE config 1 in full (2,000 uniform voxels in 64^3,
      SubMConv3d 16 -> 16 fp32): the oracle's sort-based rulebook plus its
      forward, at all threads and at one thread."""
    import numpy as np

    from bench_data import uniform_cloud
    from oracle import oracle as orc

    threads = len(os.sched_getaffinity(0))
    threads = min(threads, int(os.environ.get("OMP_NUM_THREADS", threads)))
    w = w_np.reshape(C_OUT, KV, C_IN).astype(np.float32)
    x = feats_np.astype(np.float32)
    b = b_np.astype(np.float32)

    orc.set_num_threads(threads)
    rows = 50_000
    pf_s = np.ascontiguousarray(pf_np[:, :rows])
    per_pass, reps = _time_reps(lambda: orc.gemm_fwd_f32(x, w, pf_s, b), 10.0, 50)
    per_row = per_pass / rows
    # the reference's pair generation on the CPU (sort + binary search) for the full cloud
    t1 = time.perf_counter()
    orc.igemm_pairs(idx, 1, [GRID] * 3, [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3, True, False,
                    False)
    pairgen_s = time.perf_counter() - t1

    orc.set_num_threads(1)
    rows1 = 5_000
    pf_1 = np.ascontiguousarray(pf_np[:, :rows1])
    per_pass1, reps1 = _time_reps(lambda: orc.gemm_fwd_f32(x, w, pf_1, b), 4.0, 50)
    per_row1 = per_pass1 / rows1

    # 2,000 uniform voxels in 64^3, SubMConv3d 16 -> 16 fp32, batch 1
    idx1 = uniform_cloud(2000, [64] * 3, seed=0)
    rng = np.random.default_rng(0)
    x1 = rng.standard_normal((idx1.shape[0], 16)).astype(np.float32)
    bound = 1.0 / np.sqrt(16 * 27)
    w1 = rng.uniform(-bound, bound, (16, 27, 16)).astype(np.float32)
    b1 = rng.uniform(-bound, bound, 16).astype(np.float32)

    def config1():
        res = orc.igemm_pairs(idx1, 1, [64] * 3, [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3,
                              True, False, False)
        orc.gemm_fwd_f32(x1, w1, res[2], b1)

    c1 = {}
    for nt in (threads, 1):
        orc.set_num_threads(nt)
        c1[nt] = _time_reps(config1, 2.0, 200)[0]
    orc.set_num_threads(threads)
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
        "single_thread": {"value": round(1.0 / per_row1 / 1e6, 4), "unit": "Mvoxels/s",
                          "cores": 1, "sample": f"{rows1} output rows x {reps1} passes"},
        "config1": {"workload": "SubMConv3d k3 16->16 fp32, 2000 uniform voxels in 64^3, "
                                "batch 1: oracle rulebook + forward",
                    "ms": round(c1[threads] * 1e3, 3), "cores": threads,
                    "ms_1thread": round(c1[1] * 1e3, 3)},
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
    from spconv_triton.pytorch._impl import _lib
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
        log(f"warmup {args.warmup}, timed {args.steps} steps")
        for _ in range(args.warmup):
            y = conv(xc)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            y = conv(xc)
        torch.cuda.synchronize()
        wall_s = time.perf_counter() - t0
        ms_per_step = wall_s / args.steps * 1e3

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

        for _ in range(50):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(500):
            graph.replay()
        torch.cuda.synchronize()
        graph_ms = (time.perf_counter() - t0) / 500 * 1e3

    # ---- the GEMM kernel alone, for the roofline: one graph holding
    # GEMM_LAUNCHES back-to-back launches of the planned gather-GEMM (the
    # module's graph above also holds the weight pack), replayed between HIP
    # events on the stream the launches are captured on
    pf_c = y0.indice_dict["subm0"].pair_fwd
    plan = gemm_impl.gather_plan(pf_c, N_VOXELS)
    packed = gemm_impl.packed_weight(conv.weight, conv.bias, torch.float16, False)
    out_k = torch.empty((N_VOXELS, C_OUT), dtype=torch.float16, device=dev)
    L = _lib.lib()
    f16 = _lib.dtype_code(torch.float16)
    kstream = torch.cuda.Stream()
    kstream.wait_stream(torch.cuda.current_stream())

    def launch():
        _lib.check(L.sp_conv_gemm_planned(_lib.ptr(feats), f16, N_VOXELS, _lib.ptr(packed), C_OUT,
                                          KV, C_IN, 0, 1, _lib.ptr(pf_c), N_VOXELS,
                                          _lib.ptr(plan), plan.numel(), _lib.ptr(out_k), f16,
                                          _lib.stream_of(dev)), "sp_conv_gemm_planned")

    GEMM_LAUNCHES = 20
    with torch.cuda.stream(kstream):
        launch()
        kgraph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(kgraph, stream=kstream):
            for _ in range(GEMM_LAUNCHES):
                launch()
        kgraph.replay()
        kstream.synchronize()
        if not torch.equal(out_k, y.features):
            raise RuntimeError("the kernel graph differs from the module forward")
        ks, ke = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        replays = 25
        ks.record(kstream)
        for _ in range(replays):
            kgraph.replay()
        ke.record(kstream)
        kstream.synchronize()
    kernel_ms = ks.elapsed_time(ke) / (replays * GEMM_LAUNCHES)

    # ---- the cold rulebook's GPU time with the host ahead: three forward
    # replays (~0.18 ms of GPU work) are queued first, so the build's kernels
    # are all enqueued before the GPU reaches them and run back to back (the
    # events above also hold the gaps where the GPU waited for the host)
    pg_gpu, pg_gpu_rules, pg_host = [], [], []
    for _ in range(20):
        for _ in range(3):
            graph.replay()
        s, m, e = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        s.record()
        t0 = time.perf_counter()
        res = pairgen()
        m.record()
        gemm_impl.gather_plan(res[2], N_VOXELS)
        pg_host.append((time.perf_counter() - t0) * 1e3)
        e.record()
        torch.cuda.synchronize()
        pg_gpu.append(s.elapsed_time(e))
        pg_gpu_rules.append(s.elapsed_time(m))
    pairgen_gpu_ms = statistics.median(pg_gpu)
    rules_gpu_ms = statistics.median(pg_gpu_rules)

    # HBM bytes per launch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE runs,
    # scaled by a 256 MiB copy: a stored profile, not measured in this run
    traffic = None
    tfile = ROOT / "profiles" / "gather_gemm_traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("bytes_per_launch")
    n_overflow = gemm_impl.plan_overflow_count(plan)
    nbytes = gemm_bytes(N_VOXELS, N_VOXELS, plan_read_bytes(plan, KV, N_VOXELS))
    flops = 2.0 * n_pairs * C_IN * C_OUT
    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    mvox = N_VOXELS / (ms_per_step * 1e-3) / 1e6
    # pair generation (subm, eval): coordinates read, pair_fwd written, sorted
    # mask words + argsort written
    pg_bytes = 4 * N_VOXELS * 4 + 4 * KV * N_VOXELS + 8 * N_VOXELS
    pg_achieved = pg_bytes / (rules_gpu_ms * 1e-3) / 1e9

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
                        "batch 1, rulebook cached, forward called from Python",
            "n_voxels": N_VOXELS,
            "pairs": n_pairs,
            "parallelism": "single_gpu",
        },
        "fwd_ms": round(ms_per_step, 5),
        "graph_ms": round(graph_ms, 5),
        "pairgen_ms": round(pairgen_ms, 4),
        "pairgen_parts_ms": {"rulebook": round(rules_ms, 4),
                             "gather_plan": round(pairgen_ms - rules_ms, 4)},
        "pairgen_gpu_ms": round(pairgen_gpu_ms, 4),
        "pairgen_gpu_parts_ms": {"rulebook": round(rules_gpu_ms, 4),
                                 "gather_plan": round(pairgen_gpu_ms - rules_gpu_ms, 4)},
        "pairgen_host_ms": round(statistics.median(pg_host), 4),
        "pairgen_note": "pairgen_ms: events around the cold build issued from an idle host "
                        "(includes GPU waits on the Python host); pairgen_gpu_ms: the same "
                        "build queued behind GPU work, its kernels back to back; "
                        "pairgen_host_ms: the host's time to issue the build",
        "overflow_tiles": int(n_overflow),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": "stored rocprofv3 FETCH_SIZE/WRITE_SIZE profile "
                              "(profiles/gather_gemm_traffic.json), not this run",
            "kernel": "gather_gemm_staged<f16,f16,VEC,natural,SPLIT>",
            "kernel_ms": round(kernel_ms, 5),
            "kernel_ms_source": f"HIP events around {GEMM_LAUNCHES}-launch graphs of the GEMM "
                                "alone, per launch",
            "algorithmic_bytes": nbytes,
            "mfma_tflops": round(flops / (kernel_ms * 1e-3) / 1e12, 2),
            "mfma_frac": round(flops / (kernel_ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
        },
        "pairgen_roofline": {
            "bound": "hbm",
            "achieved": round(pg_achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(pg_achieved / HBM_PEAK_GBS, 4),
            "algorithmic_bytes": pg_bytes,
            "ms": round(rules_gpu_ms, 5),
            "what": "cold subm rulebook (eval): 4*N*(D+1) coordinates + 4*kv*N pair_fwd + "
                    "8*N sorted mask words and argsort, over the rulebook's GPU time "
                    "(pairgen_gpu_parts_ms.rulebook)",
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
