"""Benchmark of PP-DocLayoutV3 inference on one MI355X.

Default workload "network": the full PP-DocLayoutV3 graph at 800x800 (HGNetV2
backbone, hybrid encoder, 6-layer deformable decoder, heads) with seeded
random-init FP32 weights of that architecture written as a GGUF, on a seeded
U(0,1) 3x800x800 input.  One step is one hipGraph replay of the whole graph
(the span the reference reports as infer_ms: no host copies).  `value` is the
device time per image from HIP events on the replay stream.

The metric's second half, conv GEMM TFLOPS as a fraction of the FP32 matrix
peak, comes from the per-node profile (ppdl_profile_nodes: every node
captured `kernel_reps` times into a graph of its own and replayed between HIP
events on the graph's stream, so no host launch cost is counted): algorithmic
conv GEMM FLOP (Winograd counted at its 36-plane GEMM) over the conv GEMM
nodes' time.

roofline: the GEMM kernel with the largest total time in one image, its
algorithmic FLOP per launch over its mean launch time; traffic is its HBM
bytes per launch from the committed rocprofv3 --pmc summary.

cpu_baseline: the oracle's restatement of the reference CPU path (im2col +
FP32 GEMM convs, the stock ops in numpy) on the same weights and image, timed
per image on the host over a bounded number of images (median, p10, p90),
plus one image on a single thread.

Workload "conv_suite": the single-op configurations (1x1 512->256 @100^2,
the F(4,3) sweep, the im2col convs, MSDeformAttn) as one hipGraph.
"""
import argparse
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "ppdoclayout-ggml_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBPS = 8000.0
METRIC = "ms/image @800×800 FP32 (hipGraph); conv GEMM TFLOPS as % of FP32 MFMA peak"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "network_traffic.json")
SUITE_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "conv_suite_traffic.json")


_HIP = None


def hip_rt():
    """libamdhip64 through ctypes: the network path needs device sync and one
    plain copy, and touches no torch (the library owns the HIP context)."""
    global _HIP
    if _HIP is None:
        import ctypes

        for name in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
            try:
                _HIP = ctypes.CDLL(name)
                break
            except OSError:
                continue
        if _HIP is None:
            raise RuntimeError("libamdhip64.so not found")
        _HIP.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        _HIP.hipFree.argtypes = [ctypes.c_void_p]
        _HIP.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
        _HIP.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return _HIP


def sync():
    if hip_rt().hipDeviceSynchronize() != 0:
        raise RuntimeError("hipDeviceSynchronize failed")


def calib_copy_hip(mib):
    """A plain device-to-device copy of `mib` MiB (the runtime's blit kernel
    reads and writes exactly that many bytes): the scale for the HBM byte
    counters of a --pmc run."""
    import ctypes

    h = hip_rt()
    n = mib * (1 << 20)
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    if h.hipMalloc(ctypes.byref(a), n) or h.hipMalloc(ctypes.byref(b), n):
        raise RuntimeError("hipMalloc failed")
    h.hipMemset(a, 0, n)
    for _ in range(3):
        h.hipMemcpy(b, a, n, 3)  # hipMemcpyDeviceToDevice
    sync()
    h.hipFree(a)
    h.hipFree(b)


def measured_traffic(path, key):
    """HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, copy-calibrated) of
    `key` from a committed rocprofv3 summary, or (None, None)."""
    try:
        with open(path) as f:
            rec = json.load(f)["kernels"].get(key)
    except (OSError, ValueError, KeyError):
        return None, None
    if not rec:
        return None, None
    return rec["bytes"], os.path.relpath(path, ROOT) + " (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)"


def calib_copy(mib):
    """A plain elementwise copy of known size: reads and writes exactly `mib`
    MiB, the scale for the HBM byte counters of a --pmc run."""
    import torch

    n = mib * (1 << 20) // 4
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        torch.mul(a, 1.0, out=b)
    torch.cuda.synchronize()


# ---------------------------------------------------------------- network
def _spread(ms):
    """median / p10 / p90 of a list of per-image times (nearest rank)."""
    v = sorted(ms)
    q = lambda f: v[min(len(v) - 1, int(round(f * (len(v) - 1))))]  # noqa: E731
    return q(0.5), q(0.1), q(0.9)


def network_cpu_baseline(weights, image, budget_s):
    """The oracle's restatement of the reference CPU path on the host cores:
    images timed one by one at all threads until budget_s (at most 20), then
    one image on a single thread (OpenMP convs and numpy's BLAS both
    pinned to one)."""
    from threadpoolctl import threadpool_limits

    from oracle import ppdl_net

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    net = ppdl_net.Net(weights, threads=threads)
    per, t0 = [], time.perf_counter()
    while len(per) < 20 and (time.perf_counter() - t0) < budget_s:
        t = time.perf_counter()
        net.forward(image)
        per.append((time.perf_counter() - t) * 1000.0)
    one = ppdl_net.Net(weights, threads=1)
    with threadpool_limits(limits=1):
        t = time.perf_counter()
        one.forward(image)
        single = (time.perf_counter() - t) * 1000.0
    return per, threads, single


def run_network(args):
    import pages
    import ppdoclayout as P
    import synth_gguf

    tmp = tempfile.mkdtemp(prefix="ppdl_bench_")
    path = os.path.join(tmp, "ppdlv3-random-seed0.gguf")
    weights = synth_gguf.write_random_model(path, seed=0)
    image = pages.uniform_page(0)
    ctx = P.PPDocLayout(path, P.BACKEND_HIP)
    launches = ctx.graph_nodes()
    ctx.compute(image)  # uploads the page (resident from here on) and replays once

    if args.warmup > 0:
        ctx.time_graph(args.warmup)
    sync()
    t0 = time.perf_counter()
    ms = ctx.time_graph(args.steps)  # HIP events around `steps` replays on the graph's stream
    sync()
    wall_ms = (time.perf_counter() - t0) * 1000.0 / args.steps

    # per-replay distribution (one replay between HIP events, synchronised)
    per = sorted(ctx.time_graph(1) for _ in range(max(args.steps, 20)))
    pct = lambda q: per[min(len(per) - 1, int(round(q * (len(per) - 1))))]  # noqa: E731
    # end to end through ppdl_infer: page upload, replay, result downloads and
    # the host postprocess (the reference's infer_ms span excludes the copies)
    n_e2e = max(5, min(20, args.steps))
    ctx.infer(image)
    t1 = time.perf_counter()
    for _ in range(n_e2e):
        ctx.infer(image)
    e2e_ms = (time.perf_counter() - t1) * 1000.0 / n_e2e

    nodes = ctx.profile_nodes(args.kernel_reps)
    if args.calib_copy_mib > 0:
        calib_copy_hip(args.calib_copy_mib)
    ctx.close()

    conv = [n for n in nodes if n["cls"] == P.NODE_CONV_GEMM]
    lin = [n for n in nodes if n["cls"] == P.NODE_LINEAR_GEMM]
    conv_fl, conv_us = sum(n["flops"] for n in conv), sum(n["us"] for n in conv)
    lin_fl, lin_us = sum(n["flops"] for n in lin), sum(n["us"] for n in lin)
    conv_tf = conv_fl / (conv_us * 1e-6) / 1e12
    lin_tf = lin_fl / (lin_us * 1e-6) / 1e12

    # dominant GEMM kernel: largest total time over the single-kernel GEMM nodes
    groups = {}
    for n in conv + lin:
        if n["kernels"] != 1:
            continue
        g = groups.setdefault(n["kernel"], {"us": 0.0, "flops": 0.0, "bytes": 0.0, "launches": 0})
        g["us"] += n["us"]
        g["flops"] += n["flops"]
        g["bytes"] += n["bytes"]
        g["launches"] += 1
    dom_name, dom = max(groups.items(), key=lambda kv: kv[1]["us"])
    if args.roofline_kernel:  # a profiler's per-dispatch cost can reorder the groups: pin the kernel by name
        if args.roofline_kernel not in groups:
            raise SystemExit("no single-kernel GEMM group named %r" % args.roofline_kernel)
        dom_name, dom = args.roofline_kernel, groups[args.roofline_kernel]
    # every single-kernel GEMM group, largest per-image time first
    gemm_kernels = [{"kernel": k, "launches": v["launches"], "us_per_image": round(v["us"], 1),
                     "us_per_launch": round(v["us"] / v["launches"], 2),
                     "tflops": round(v["flops"] / (v["us"] * 1e-6) / 1e12, 2),
                     "frac": round(v["flops"] / (v["us"] * 1e-6) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4)}
                    for k, v in sorted(groups.items(), key=lambda kv: -kv[1]["us"])]
    dom_us = dom["us"] / dom["launches"]
    dom_fl = dom["flops"] / dom["launches"]
    dom_tf = dom_fl / (dom_us * 1e-6) / 1e12
    traffic, traffic_src = measured_traffic(TRAFFIC_FILE, dom_name)
    roofline = {
        "bound": "mfma",
        "kernel": dom_name,
        "achieved": round(dom_tf, 2),
        "peak": PEAK_FP32_MFMA_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(dom_tf / PEAK_FP32_MFMA_TFLOPS, 4),
        "traffic": traffic,
        "traffic_source": traffic_src,
        "flops_per_launch": round(dom_fl),
        "algorithmic_bytes_per_launch": round(dom["bytes"] / dom["launches"]),
        "us_per_launch": round(dom_us, 2),
        "launches_per_image": dom["launches"],
    }

    cpu = None
    if not args.no_cpu:
        per_img, cores, single = network_cpu_baseline(weights, image, args.cpu_budget)
        med, p10, p90 = _spread(per_img)
        cpu = {
            "value": round(med, 1),
            "unit": "ms/image",
            "cores": cores,
            "kind": "port",
            "sample": f"{len(per_img)} full 800x800 U(0,1) images, each timed, through the oracle's restatement "
                      f"of the reference CPU path (im2col + FP32 GEMM convs in C, stock ops and linears in numpy) "
                      f"at {cores} threads (value = median), then one image on 1 thread",
            "p10": round(p10, 1),
            "p90": round(p90, 1),
            "mean": round(sum(per_img) / len(per_img), 1),
            "single_thread_ms_per_image": round(single, 1),
        }

    top = sorted(nodes, key=lambda n: -n["us"])[:12]
    line = {
        "metric": METRIC,
        "value": round(ms, 4),
        "unit": "ms/image",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "wall_ms_per_step": round(wall_ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded random-init FP32 weights of the PP-DocLayoutV3 architecture (GGUF), "
                "seeded U(0,1) 3x800x800 input; inputs resident in HBM",
        "config": {
            "workload": "network: full PP-DocLayoutV3 @800x800 (HGNetV2-L backbone, hybrid encoder, 6-layer "
                        "deformable decoder, class/box/mask/order heads) as one hipGraph replay",
            "kernel_launches_per_image": launches,
            "conv_gemm_tflops": round(conv_tf, 2),
            "conv_gemm_pct_of_fp32_mfma_peak": round(100.0 * conv_tf / PEAK_FP32_MFMA_TFLOPS, 2),
            "conv_gemm_gflop_per_image": round(conv_fl / 1e9, 3),
            "conv_gemm_us_per_image": round(conv_us, 1),
            "linear_gemm_tflops": round(lin_tf, 2),
            "linear_gemm_gflop_per_image": round(lin_fl / 1e9, 3),
            "node_us_sum": round(sum(n["us"] for n in nodes), 1),
        },
        "roofline": roofline,
        "gemm_kernels": gemm_kernels,
        "cpu_baseline": cpu,
        "replay_ms": {"median": round(pct(0.5), 4), "p10": round(pct(0.1), 4), "p90": round(pct(0.9), 4),
                      "replays": len(per)},
        "e2e_ms_per_image": {"value": round(e2e_ms, 3), "images": n_e2e,
                             "span": "ppdl_infer: 7.7 MB page upload, graph replay, result downloads, host postprocess"},
        "top_nodes": [{"name": n["name"], "us": round(n["us"], 2), "kernel": n["kernel"]} for n in top],
    }
    return line


# ---------------------------------------------------------------- op suite
def time_nodes(suite, stream, reps):
    """Average device time (us) of each suite node: the node captured `reps`
    times into a graph of its own, one replay between two HIP events on the
    launch stream (no host launch cost per kernel)."""
    import torch

    out = {}
    for n in suite.nodes:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for _ in range(reps):
                n.launch(stream.cuda_stream)
        g.replay()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
        e1.synchronize()
        out[n.name] = e0.elapsed_time(e1) * 1000.0 / reps
    return out


def suite_cpu_baseline(budget_s):
    """Suite passes through the oracle's reference CPU path until budget_s."""
    import numpy as np

    import oracle
    import workloads

    rng = np.random.default_rng(workloads.SEED)
    cases = []
    x = rng.random((512, 100, 100)).astype(np.float32)
    w, b = workloads._conv_weights(rng, 512, 256, 1)
    cases.append((x, w, b, 1, 0, 1))
    for (C, Hh, W) in workloads.WINOGRAD_SWEEP:
        x = rng.random((C, Hh, W)).astype(np.float32)
        w, b = workloads._conv_weights(rng, C, C, 3)
        cases.append((x, w, b, 1, 1, 2))
    for (IC, IH, IW, OC, K, S, P) in workloads.IM2COL_CONVS:
        x = rng.random((IC, IH, IW)).astype(np.float32)
        w, b = workloads._conv_weights(rng, IC, OC, K)
        cases.append((x, w, b, S, P, 0))
    ms_in = workloads.msdef_inputs(rng)
    nthreads = os.cpu_count() or 1
    passes, t0 = 0, time.perf_counter()
    while True:
        for (x, w, b, S, P, act) in cases:
            oracle.conv2d_ref(x, w, b, S, P, act, nthreads)
        oracle.msdeform(*ms_in, nthreads)
        passes += 1
        el = time.perf_counter() - t0
        if el >= budget_s or passes >= 50:
            break
    return el * 1000.0 / passes, passes, nthreads


def run_suite(args):
    import torch

    import ppdl_hip
    import workloads

    ppdl_hip.lib()
    suite = workloads.ConvSuite()
    stream = torch.cuda.Stream()
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
    with torch.cuda.stream(stream):
        kt = time_nodes(suite, stream, args.kernel_reps)
    torch.cuda.synchronize()
    if args.calib_copy_mib > 0:
        calib_copy(args.calib_copy_mib)

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
    dom_us = kt[dominant.name]
    dom_tf = dominant.flops / (dom_us * 1e-6) / 1e12
    try:
        with open(SUITE_TRAFFIC_FILE) as f:
            rec = json.load(f)["nodes"].get(dominant.name)
        traffic = rec["bytes"] if rec else None
    except (OSError, ValueError, KeyError):
        traffic = None
    cpu = None
    if not args.no_cpu:
        cpu_ms, passes, cores = suite_cpu_baseline(args.cpu_budget)
        cpu = {
            "value": round(cpu_ms, 2),
            "unit": "ms/step",
            "cores": cores,
            "kind": "port",
            "sample": f"{passes} full passes of the same suite through the oracle's restatement of the "
                      f"reference CPU path (im2col + FP32 GEMM convs with bias/act, msdeform loop), "
                      f"{cores} OpenMP threads",
        }
    return {
        "metric": METRIC,
        "value": round(100.0 * agg_tflops / PEAK_FP32_MFMA_TFLOPS, 3),
        "unit": "% of FP32 MFMA peak (conv GEMMs of the op suite, 157.3 TFLOP/s)",
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
            "workload": "conv_suite: 1x1 512->256@100^2; F(4,3) 256@100/50/25, 48@200, 96@100; im2col k2 "
                        "48->24@401, k3s2 256@100/@50, 3->32@800; MSDeformAttn 300q; one hipGraph, 21 launches",
            "conv_gemm_tflops": round(agg_tflops, 2),
            "conv_gemm_gflop_per_step": round(gemm_flops / 1e9, 3),
        },
        "roofline": {
            "bound": "mfma", "kernel": dominant.name, "achieved": round(dom_tf, 2),
            "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s", "frac": round(dom_tf / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": traffic, "flops_per_launch": dominant.flops, "us_per_launch": round(dom_us, 2),
        },
        "cpu_baseline": cpu,
        "kernels": kernels,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", choices=["network", "conv_suite"], default="network")
    ap.add_argument("--kernel-reps", type=int, default=10, help="runs per node in the per-node profile (captured into one graph)")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--roofline-kernel", default="",
                    help="report the roofline for this GEMM kernel instead of the one with the largest per-image time")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run a plain copy of this many MiB (PMC byte-counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (images are independent; "
              "scale by running one process per GPU). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    line = run_network(args) if args.workload == "network" else run_suite(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
