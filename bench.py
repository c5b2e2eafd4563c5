"""Benchmark of the tagged-op hot path on one MI355X.

Workload "conv_suite": one step is one hipGraph replay of the BASELINE op
configs at their real shapes, all through the C-ABI:
  1x1 512->256 @100^2 + ReLU; the F(4,3) sweep (256 @100/50/25, 48 @200,
  96 @100, SiLU); the im2col convs (k2 48->24 @401, k3s2 256 @100 and @50,
  k3s2 3->32 @800); MSDeformAttn at 300 queries.
The headline metric's first half (ms/image of the full network) needs the
whole PP-DocLayoutV3 graph; this workload reports its second half: conv GEMM
TFLOPS as a percentage of the FP32 matrix peak, summed over the suite's conv
GEMM kernels (Winograd counted at its 36-plane GEMM FLOPs).

Timing: W untimed warm-up replays, then K replays between
torch.cuda.synchronize() (and HIP events on the replay stream).  Per-kernel
times come from HIP events around repeated launches of each node on the
stream it is launched on.  The CPU baseline is the oracle's restatement of
the reference CPU path (im2col + FP32 GEMM convs, the msdeform loop) on the
host cores, over a bounded number of suite passes.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "ppdoclayout-ggml_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBPS = 8000.0
METRIC = "ms/image @800×800 FP32 (hipGraph); conv GEMM TFLOPS as % of FP32 MFMA peak"


def time_nodes(suite, stream, reps):
    """Average device time (us) of each node: `reps` back-to-back launches
    between two HIP events recorded on the launch stream."""
    import torch

    out = {}
    for n in suite.nodes:
        for _ in range(3):
            n.launch(stream.cuda_stream)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            n.launch(stream.cuda_stream)
        e1.record(stream)
        e1.synchronize()
        out[n.name] = e0.elapsed_time(e1) * 1000.0 / reps
    return out


def measured_traffic(node):
    """HBM bytes per launch of `node` (FETCH_SIZE + WRITE_SIZE, copy-calibrated)
    from the committed rocprofv3 summary, or (None, None) if not profiled."""
    path = os.path.join(ROOT, "profiles", "conv_suite_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)["nodes"].get(node)
    except (OSError, ValueError, KeyError):
        return None, None
    if not rec:
        return None, None
    return rec["bytes"], "profiles/conv_suite_traffic.json (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)"


def cpu_baseline(budget_s):
    """Suite passes through the oracle's reference CPU path until budget_s."""
    import numpy as np

    import oracle
    import workloads

    rng = np.random.default_rng(workloads.SEED)
    cases = []
    x = rng.random((512, 100, 100)).astype(np.float32)
    w, b = workloads._conv_weights(rng, 512, 256, 1)
    cases.append(("conv", x, w, b, 1, 0, 1))
    for (C, Hh, W) in workloads.WINOGRAD_SWEEP:
        x = rng.random((C, Hh, W)).astype(np.float32)
        w, b = workloads._conv_weights(rng, C, C, 3)
        cases.append(("conv", x, w, b, 1, 1, 2))
    for (IC, IH, IW, OC, K, S, P) in workloads.IM2COL_CONVS:
        x = rng.random((IC, IH, IW)).astype(np.float32)
        w, b = workloads._conv_weights(rng, IC, OC, K)
        cases.append(("conv", x, w, b, S, P, 0))
    ms_in = workloads.msdef_inputs(rng)
    nthreads = os.cpu_count() or 1
    passes, t0 = 0, time.perf_counter()
    while True:
        for c in cases:
            _, x, w, b, S, P, act = c
            oracle.conv2d_ref(x, w, b, S, P, act, nthreads)
        oracle.msdeform(*ms_in, nthreads)
        passes += 1
        el = time.perf_counter() - t0
        if el >= budget_s or passes >= 50:
            break
    return el * 1000.0 / passes, passes, nthreads


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run a plain copy of this many MiB (PMC byte-counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (images are independent; "
              "scale by running one process per GPU). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import ppdl_hip
    import workloads

    torch.cuda.set_device(0)
    ppdl_hip.lib()
    suite = workloads.ConvSuite()
    stream = torch.cuda.Stream()

    # capture one pass into a hipGraph
    with torch.cuda.stream(stream):
        suite.run(stream.cuda_stream)  # eager warm pass (also first-touch)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        suite.run(stream.cuda_stream)
    torch.cuda.synchronize()

    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            graph.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(args.steps):
            graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1000.0
    ms_per_step = e0.elapsed_time(e1) / args.steps

    # per-kernel device times (HIP events on the launch stream)
    with torch.cuda.stream(stream):
        kt = time_nodes(suite, stream, args.kernel_reps)
    torch.cuda.synchronize()

    if args.calib_copy_mib > 0:
        # a plain elementwise copy of known size: reads and writes exactly
        # calib_copy_mib MiB, the scale for HBM byte counters
        n = args.calib_copy_mib * (1 << 20) // 4
        a = torch.ones(n, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            torch.mul(a, 1.0, out=b)
        torch.cuda.synchronize()
        del a, b

    kernels = {}
    gemm_flops = gemm_us = 0.0
    dominant = None
    for n in suite.nodes:
        us = kt[n.name]
        rec = {"us": round(us, 2)}
        if n.kind == "gemm":
            tf = n.flops / (us * 1e-6) / 1e12
            rec.update(tflops=round(tf, 2), frac=round(tf / PEAK_FP32_MFMA_TFLOPS, 4))
            gemm_flops += n.flops
            gemm_us += us
            if dominant is None or us > kt[dominant.name]:
                dominant = n
        else:
            gbps = n.bytes / (us * 1e-6) / 1e9
            rec.update(gbps=round(gbps, 1), frac=round(gbps / PEAK_HBM_GBPS, 4))
        kernels[n.name] = rec
    agg_tflops = gemm_flops / (gemm_us * 1e-6) / 1e12
    value = 100.0 * agg_tflops / PEAK_FP32_MFMA_TFLOPS

    dom_us = kt[dominant.name]
    dom_tf = dominant.flops / (dom_us * 1e-6) / 1e12
    traffic, traffic_src = measured_traffic(dominant.name)
    roofline = {
        "bound": "mfma",
        "kernel": dominant.name,
        "achieved": round(dom_tf, 2),
        "peak": PEAK_FP32_MFMA_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(dom_tf / PEAK_FP32_MFMA_TFLOPS, 4),
        "traffic": traffic,
        "traffic_source": traffic_src,
        "algorithmic_bytes": dominant.bytes,
        "flops_per_launch": dominant.flops,
        "us_per_launch": round(dom_us, 2),
    }

    cpu = None
    if not args.no_cpu:
        cpu_ms, passes, cores = cpu_baseline(args.cpu_budget)
        cpu = {
            "value": round(cpu_ms, 2),
            "unit": "ms/step",
            "cores": cores,
            "kind": "port",
            "sample": f"{passes} full passes of the same suite through the oracle's restatement of the "
                      f"reference CPU path (im2col + FP32 GEMM convs with bias/act, msdeform loop), "
                      f"{cores} OpenMP threads",
            "gpu_ms_per_step": round(ms_per_step, 4),
        }

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "% of FP32 MFMA peak (conv GEMMs, 157.3 TFLOP/s)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "wall_ms_per_step": round(wall_ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded U(0,1) activations, N(0,1/sqrt(fan_in)) weights)",
        "config": {
            "workload": "conv_suite: BASELINE configs 1-4 (1x1 512->256@100^2; F(4,3) 256@100/50/25, "
                        "48@200, 96@100; im2col k2 48->24@401, k3s2 256@100/@50, 3->32@800; "
                        "MSDeformAttn 300q) as one hipGraph, 21 tagged-op launches per step",
            "conv_gemm_tflops": round(agg_tflops, 2),
            "conv_gemm_gflop_per_step": round(gemm_flops / 1e9, 3),
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
