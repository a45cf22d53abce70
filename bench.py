"""Benchmark: DSINE AngMF propagate on one MI355X.

A step is one pass of the hot path over one batch: one angmf_propagate call
(workload 2: B=1, 256x256, k=5, fp32) through the C ABI, inputs resident in
HBM.  To keep the 256 MB Infinity Cache from serving the inputs, each step
reads a different one of `--sets` input copies (together > 512 MB); the warm
number (same inputs every step) is reported beside it.

The K timed steps are the K kernel launches of one captured HIP graph,
replayed once between two HIP events on the replay stream: the kernels run
back to back, so the region measures the GPU, not Python's launch overhead
(the same K steps launched eagerly from Python are reported as "eager").

Prints one JSON line (rank 0):
  value       Mpixel/s over the timed region (K steps / event time)
  roofline    HBM roofline of the kernel: algorithmic bytes per launch /
              average launch duration (event time of the region / K)
  cpu_baseline  the CPU oracle (double-precision restatement of the
              reference's CPU twin), one thread, on a bounded sample
  cpu_baseline_all_cores  the same oracle with its rows over the host's
              CPU share (OpenMP), labelled separately
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def host_share() -> int:
    """Host threads this process may use: OMP_NUM_THREADS when the job
    scheduler sets it, else the CPUs in this process's affinity mask."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


PROFILE = os.path.join(ROOT, "profiles", "angmf_f32_k5_256x256_traffic.json")


def traffic_from_profile(w):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the same counters on a
    plain copy of known size), if it covers this workload."""
    try:
        with open(PROFILE) as f:
            p = json.load(f)
    except (OSError, ValueError):
        return None
    if p.get("workload") != w.name:
        return None
    return p.get("traffic_bytes_per_launch")


def cpu_baseline(w, inp, seconds: float, nthreads: int = 1):
    """Time the oracle on whole images of the workload until `seconds` of
    CPU work; returns (Mpixel/s, passes)."""
    import oracle
    passes = 0
    t0 = time.perf_counter()
    while True:
        oracle.angmf_propagate(inp["pred_norm"], inp["prob"], inp["xy"], inp["angle"],
                               inp["ray"], inp["intrinsics"], w.H, w.W, w.k,
                               nthreads=nthreads)
        passes += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return passes * w.B * w.HW * w.calls / el / 1e6, passes, el


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", type=int, default=2)
    ap.add_argument("--sets", type=int, default=0, help="rotating input sets (0 = auto, > 512 MB)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--ray-from-intrinsics", action="store_true",
                    help="form each pixel's ray from fu, cu, fv, cv in the kernel "
                         "(BVML_DSINE_RAY_FROM_INTRINSICS) instead of reading the ray planes")
    ap.add_argument("--calib", action="store_true",
                    help="also run 10 plain device copies of one launch's byte count "
                         "(the reference kernel for the FETCH_SIZE / WRITE_SIZE scale)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the op shards by frames or row bands with no collective on the path, "
              "so run --gpus 1", file=sys.stderr)
        return 2

    import torch
    from brovisionml_amd import _lib, workloads as wl

    if not torch.cuda.is_available():
        print("bench.py: no HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    _lib.load()

    w = wl.WORKLOADS[args.workload]
    inp = wl.make_inputs(w)
    fu, cu, fv, cv = inp["intrinsics"]
    B, H, W, k = w.B, w.H, w.W, w.k
    bytes_per_call = w.algorithmic_bytes(shared_ray=True) // w.calls
    flags = _lib.DEFAULT
    if args.ray_from_intrinsics:
        flags |= _lib.RAY_FROM_INTRINSICS
        bytes_per_call -= 3 * w.HW * 4  # the shared ray's 3 planes are not read
    set_bytes = bytes_per_call
    nsets = args.sets or max(2, int(np.ceil(512e6 / set_bytes)))

    def dev_set():
        return {key: torch.from_numpy(np.ascontiguousarray(inp[key])).to(dev)
                for key in ("pred_norm", "prob", "xy", "angle", "ray")}

    base = dev_set()
    sets = [base] + [{key: t.clone() for key, t in base.items()} for _ in range(nsets - 1)]
    outs = [torch.empty_like(s["pred_norm"]) for s in sets]

    def launch(i: int) -> None:
        s = sets[i]
        sptr = torch.cuda.current_stream(dev).cuda_stream
        pn = s["pred_norm"]
        for c in range(w.calls):
            dst = outs[i]
            st = _lib.angmf_propagate_f32(
                pn.data_ptr(), s["prob"].data_ptr(), s["xy"].data_ptr(), s["angle"].data_ptr(),
                0 if args.ray_from_intrinsics else s["ray"].data_ptr(), fu, cu, fv, cv, B, H, W,
                k, 0, dst.data_ptr(), flags, sptr)
            if st != 0:
                raise RuntimeError(f"angmf_propagate_f32 failed: {st} {_lib.last_error()}")
            pn = dst

    def capture(rotate: bool):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(args.steps):
                launch(i % nsets if rotate else 0)
        return g

    def timed_graph(g):
        stream = torch.cuda.current_stream(dev)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3  # seconds for args.steps steps

    def timed_eager(steps: int) -> float:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            launch(i % nsets)
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    for i in range(args.warmup):
        launch(i % nsets)
    torch.cuda.synchronize()
    g_cold = capture(True)
    g_warm = capture(False)
    for _ in range(2):
        g_cold.replay()
        g_warm.replay()
    torch.cuda.synchronize()
    t_cold = timed_graph(g_cold)
    t_warm = timed_graph(g_warm)
    t_eager = timed_eager(args.steps)

    # same-box copy ceiling: device copies that each move one launch's
    # algorithmic bytes (half read, half written), rotating over the same
    # footprint as the kernel's input sets so they miss the Infinity Cache alike
    # (captured in one graph like the kernel's launches, so host launch cost
    # stays out of the figure)
    n_copy = bytes_per_call // 8
    src = torch.ones(nsets, n_copy, dtype=torch.float32, device=dev)
    dst_c = torch.empty_like(src)
    pairs = [(dst_c[i], src[i]) for i in range(nsets)]
    n_rep = 4 * nsets
    g_copy = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_copy):
        for i in range(n_rep):
            d, s_ = pairs[i % nsets]
            d.copy_(s_)
    g_copy.replay()
    copy_s = timed_graph(g_copy)
    copy_gbps = 2 * n_copy * 4 * n_rep / copy_s / 1e9
    del g_copy, pairs, src, dst_c

    if args.calib:
        n = bytes_per_call // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()

    launch_s = t_cold / (args.steps * w.calls)
    ms_per_step = t_cold * 1e3 / args.steps
    mpix = B * H * W * w.calls * args.steps / t_cold / 1e6
    achieved = bytes_per_call / launch_s / 1e9
    achieved_w = bytes_per_call / (t_warm / (args.steps * w.calls)) / 1e9

    line = {
        "metric": "Mpixel/s (+ achieved HBM GB/s, % of peak), DSINE propagation 256x256 k=5 fp32",
        "value": round(mpix, 2),
        "unit": "Mpixel/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": w.name, "B": B, "H": H, "W": W, "k": k, "calls_per_step": w.calls,
            "ray": "from-intrinsics" if args.ray_from_intrinsics else "shared",
            "inputs": f"{nsets} rotating HBM-resident copies "
            f"({nsets * set_bytes / 1e6:.0f} MB > 256 MB Infinity Cache)",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": None if args.ray_from_intrinsics else traffic_from_profile(w),
            "kernel": f"angmf_f32_kernel<{k}>",
            "bytes_per_launch": bytes_per_call,
            "launch_us_mean": round(launch_s * 1e6, 3),
            "copy_ceiling_gbps": round(copy_gbps, 1),
        },
        "warm": {
            "value": round(B * H * W * w.calls * args.steps / t_warm / 1e6, 2),
            "launch_us_mean": round(t_warm / (args.steps * w.calls) * 1e6, 3),
            "achieved_gbps": round(achieved_w, 1),
        },
        "eager": {
            "value": round(B * H * W * w.calls * args.steps / t_eager / 1e6, 2),
            "us_per_step": round(t_eager / args.steps * 1e6, 3),
            "note": "the same steps launched one by one from Python (host-bound)",
        },
        "gpu": torch.cuda.get_device_name(dev),
    }

    if not args.no_cpu:
        v1, passes, el = cpu_baseline(w, inp, args.cpu_seconds, 1)
        line["cpu_baseline"] = {
            "value": round(v1, 4), "unit": "Mpixel/s", "cores": 1, "kind": "port",
            "sample": f"{passes} passes over the {w.name} input ({H}x{W}, k={k}), "
                      f"{el:.1f} s, oracle restatement of src/dsine_ops.cpp in double",
            "cpu": cpu_model(),
            "host_threads": os.cpu_count(),
        }
        # the same oracle with its rows split over the host's CPU share
        # (OpenMP); the reference itself is single-threaded
        nt = host_share()
        if nt > 1:
            vn, passes_n, el_n = cpu_baseline(w, inp, args.cpu_seconds / 2, nt)
            line["cpu_baseline_all_cores"] = {
                "value": round(vn, 4), "unit": "Mpixel/s", "cores": nt, "kind": "port",
                "sample": f"{passes_n} passes, {el_n:.1f} s, rows over {nt} OpenMP threads",
            }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
