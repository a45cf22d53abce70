"""Benchmark: DSINE AngMF propagate on one MI355X (and, with --op upsample,
the refiner's fused convex upsample + L2-normalise).

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

--op upsample measures bvml_dsine_convex_upsample_f32 on the refiner's
shape (C=3, s=8) at the 256x256 grid (a 2048x2048 output) the same way; its
value is output Mpixel/s.
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


PROFILES = {
    "angmf": os.path.join(ROOT, "profiles", "angmf_f32_k5_256x256_traffic.json"),
    "upsample": os.path.join(ROOT, "profiles", "upsample8_c3_256x256_traffic.json"),
}


def traffic_from_profile(op: str, name: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the same counters on a
    plain copy of known size), if it covers this workload."""
    try:
        with open(PROFILES[op]) as f:
            p = json.load(f)
    except (OSError, ValueError):
        return None
    if p.get("workload") != name:
        return None
    return p.get("traffic_bytes_per_launch")


def timed_cpu(fn, seconds: float):
    """Run fn() until `seconds` of wall time; returns (passes, elapsed)."""
    passes = 0
    t0 = time.perf_counter()
    while True:
        fn()
        passes += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return passes, el


class Timer:
    """Graph-captured timing of K launches of `launch(i)` (i selects the
    input set), plus the eager and warm variants and the same-box copy
    ceiling over the same footprint."""

    def __init__(self, dev, launch, nsets: int, steps: int, warmup: int, bytes_per_call: int):
        import torch
        self.torch, self.dev = torch, dev
        self.launch, self.nsets, self.steps = launch, nsets, steps
        self.bytes_per_call = bytes_per_call
        for i in range(warmup):
            launch(i % nsets)
        torch.cuda.synchronize()

    def capture(self, rotate: bool):
        g = self.torch.cuda.CUDAGraph()
        with self.torch.cuda.graph(g):
            for i in range(self.steps):
                self.launch(i % self.nsets if rotate else 0)
        return g

    def timed_graph(self, g):
        torch = self.torch
        stream = torch.cuda.current_stream(self.dev)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3

    def timed_eager(self) -> float:
        torch = self.torch
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(self.steps):
            self.launch(i % self.nsets)
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    def run(self):
        """(cold s, warm s, eager s) for self.steps steps."""
        g_cold = self.capture(True)
        g_warm = self.capture(False)
        for _ in range(2):
            g_cold.replay()
            g_warm.replay()
        self.torch.cuda.synchronize()
        return self.timed_graph(g_cold), self.timed_graph(g_warm), self.timed_eager()

    def copy_ceiling_gbps(self) -> float:
        """Device copies that each move one launch's algorithmic bytes (half
        read, half written), rotating over the same footprint as the kernel's
        input sets so they miss the Infinity Cache alike, captured in one
        graph like the kernel's launches."""
        torch = self.torch
        n_copy = self.bytes_per_call // 8
        src = torch.ones(self.nsets, n_copy, dtype=torch.float32, device=self.dev)
        dst = torch.empty_like(src)
        pairs = [(dst[i], src[i]) for i in range(self.nsets)]
        n_rep = 4 * self.nsets
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n_rep):
                d, s_ = pairs[i % self.nsets]
                d.copy_(s_)
        g.replay()
        t = self.timed_graph(g)
        return 2 * n_copy * 4 * n_rep / t / 1e9

    def calib(self) -> None:
        """10 plain device copies of one launch's byte count (the reference
        kernel for the FETCH_SIZE / WRITE_SIZE scale)."""
        torch = self.torch
        src = torch.ones(self.bytes_per_call // 4, dtype=torch.float32, device=self.dev)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()


def base_line(args, metric, value, unit, ms_per_step, config):
    return {
        "metric": metric,
        "value": round(value, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": config,
    }


def roofline(bytes_per_call, launch_s, traffic, kernel, copy_gbps):
    achieved = bytes_per_call / launch_s / 1e9
    return {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBPS, 4),
        "traffic": traffic,
        "kernel": kernel,
        "bytes_per_launch": bytes_per_call,
        "launch_us_mean": round(launch_s * 1e6, 3),
        "copy_ceiling_gbps": round(copy_gbps, 1),
    }


def bench_angmf(args, dev) -> dict:
    import torch
    import oracle
    from brovisionml_amd import _lib, workloads as wl

    w = wl.WORKLOADS[args.workload]
    inp = wl.make_inputs(w)
    fu, cu, fv, cv = inp["intrinsics"]
    B, H, W, k = w.B, w.H, w.W, w.k
    bytes_per_call = w.algorithmic_bytes(shared_ray=True) // w.calls
    flags = _lib.DEFAULT
    if args.ray_from_intrinsics:
        flags |= _lib.RAY_FROM_INTRINSICS
        bytes_per_call -= 3 * w.HW * 4  # the shared ray's 3 planes are not read
    cpu_inp = inp  # the CPU leg always runs the op on activated planes
    if args.logits:
        # the heads' raw logits: the prob planes' logits and the angle
        # planes' logits of angle / pi, so the activations give back the
        # workload's own planes
        flags |= _lib.LOGITS
        inp = dict(inp)
        for key, scale in (("prob", 1.0), ("angle", np.pi)):
            q = np.clip(inp[key].astype(np.float64) / scale, 1e-6, 1 - 1e-6)
            inp[key] = np.log(q / (1.0 - q)).astype(np.float32)
    nsets = args.sets or max(2, int(np.ceil(512e6 / bytes_per_call)))

    base = {key: torch.from_numpy(np.ascontiguousarray(inp[key])).to(dev)
            for key in ("pred_norm", "prob", "xy", "angle", "ray")}
    sets = [base] + [{key: t.clone() for key, t in base.items()} for _ in range(nsets - 1)]
    outs = [torch.empty_like(s["pred_norm"]) for s in sets]

    def launch(i: int) -> None:
        s = sets[i]
        sptr = torch.cuda.current_stream(dev).cuda_stream
        pn = s["pred_norm"]
        for _ in range(w.calls):
            dst = outs[i]
            st = _lib.angmf_propagate_f32(
                pn.data_ptr(), s["prob"].data_ptr(), s["xy"].data_ptr(), s["angle"].data_ptr(),
                0 if args.ray_from_intrinsics else s["ray"].data_ptr(), fu, cu, fv, cv, B, H, W,
                k, 0, dst.data_ptr(), flags, sptr)
            if st != 0:
                raise RuntimeError(f"angmf_propagate_f32 failed: {st} {_lib.last_error()}")
            pn = dst

    tm = Timer(dev, launch, nsets, args.steps, args.warmup, bytes_per_call)
    t_cold, t_warm, t_eager = tm.run()
    copy_gbps = tm.copy_ceiling_gbps()
    if args.calib:
        tm.calib()

    launch_s = t_cold / (args.steps * w.calls)
    px = B * H * W * w.calls * args.steps
    line = base_line(
        args, "Mpixel/s (+ achieved HBM GB/s, % of peak), DSINE propagation 256x256 k=5 fp32",
        px / t_cold / 1e6, "Mpixel/s", t_cold * 1e3 / args.steps,
        {
            "workload": w.name, "B": B, "H": H, "W": W, "k": k, "calls_per_step": w.calls,
            "ray": "from-intrinsics" if args.ray_from_intrinsics else "shared",
            "prob_angle": "logits, activated in the kernel" if args.logits else "activated",
            "inputs": f"{nsets} rotating HBM-resident copies "
                      f"({nsets * bytes_per_call / 1e6:.0f} MB > 256 MB Infinity Cache)",
        })
    line["roofline"] = roofline(
        bytes_per_call, launch_s,
        None if args.ray_from_intrinsics else traffic_from_profile("angmf", w.name),
        f"angmf_f32_kernel<{k}>", copy_gbps)
    line["warm"] = {
        "value": round(px / t_warm / 1e6, 2),
        "launch_us_mean": round(t_warm / (args.steps * w.calls) * 1e6, 3),
        "achieved_gbps": round(bytes_per_call / (t_warm / (args.steps * w.calls)) / 1e9, 1),
    }
    line["eager"] = {
        "value": round(px / t_eager / 1e6, 2),
        "us_per_step": round(t_eager / args.steps * 1e6, 3),
        "note": "the same steps launched one by one from Python (host-bound)",
    }
    line["gpu"] = torch.cuda.get_device_name(dev)

    if args.logits:
        # the unfused step for comparison: the refiner's two activation
        # passes (here torch's sigmoid kernels) over the same rotating
        # logits, then the op on the activated planes
        acts = [(torch.empty_like(s_["prob"]), torch.empty_like(s_["angle"])) for s_ in sets]
        kpi = float(np.float32(np.pi))

        def launch_unfused(i: int) -> None:
            s_ = sets[i]
            ap_, aa_ = acts[i]
            torch.sigmoid(s_["prob"], out=ap_)
            torch.sigmoid(s_["angle"], out=aa_)
            aa_.mul_(kpi)
            sptr = torch.cuda.current_stream(dev).cuda_stream
            st = _lib.angmf_propagate_f32(
                s_["pred_norm"].data_ptr(), ap_.data_ptr(), s_["xy"].data_ptr(), aa_.data_ptr(),
                0 if args.ray_from_intrinsics else s_["ray"].data_ptr(), fu, cu, fv, cv, B, H,
                W, k, 0, outs[i].data_ptr(), flags & ~_lib.LOGITS, sptr)
            if st != 0:
                raise RuntimeError(f"angmf_propagate_f32 failed: {st} {_lib.last_error()}")

        tu = Timer(dev, launch_unfused, nsets, args.steps, args.warmup, bytes_per_call)
        g_u = tu.capture(True)
        g_u.replay()
        t_unfused = tu.timed_graph(g_u)
        line["unfused"] = {
            "us_per_step": round(t_unfused / args.steps * 1e6, 3),
            "note": "torch sigmoid on the prob logits, sigmoid and * pi on the angle logits, "
                    "then the op on the activated planes; same rotating inputs, one graph",
        }

    if not args.no_cpu:
        def cpu_pass(nt):
            return lambda: oracle.angmf_propagate(
                cpu_inp["pred_norm"], cpu_inp["prob"], cpu_inp["xy"], cpu_inp["angle"],
                cpu_inp["ray"], cpu_inp["intrinsics"], H, W, k, nthreads=nt)

        passes, el = timed_cpu(cpu_pass(1), args.cpu_seconds)
        line["cpu_baseline"] = {
            "value": round(passes * B * w.HW * w.calls / el / 1e6, 4), "unit": "Mpixel/s",
            "cores": 1, "kind": "port",
            "sample": f"{passes} passes over the {w.name} input ({H}x{W}, k={k}), "
                      f"{el:.1f} s, oracle restatement of src/dsine_ops.cpp in double",
            "cpu": cpu_model(),
            "host_threads": os.cpu_count(),
        }
        # the same oracle with its rows split over the host's CPU share
        # (OpenMP); the reference itself is single-threaded
        nt = host_share()
        if nt > 1:
            passes_n, el_n = timed_cpu(cpu_pass(nt), args.cpu_seconds / 2)
            line["cpu_baseline_all_cores"] = {
                "value": round(passes_n * B * w.HW * w.calls / el_n / 1e6, 4),
                "unit": "Mpixel/s", "cores": nt, "kind": "port",
                "sample": f"{passes_n} passes, {el_n:.1f} s, rows over {nt} OpenMP threads",
            }
    return line


def bench_upsample(args, dev) -> dict:
    import torch
    import oracle
    from brovisionml_amd import _lib, workloads as wl

    w = wl.UPSAMPLE_WORKLOADS[args.workload]
    x, mask = wl.make_upsample_inputs(w)
    B, C, H, W, s = w.B, w.C, w.H, w.W, w.s
    bytes_per_call = w.algorithmic_bytes()
    nsets = args.sets or max(2, int(np.ceil(512e6 / bytes_per_call)))
    flags = _lib.FP64 if args.precise else _lib.DEFAULT
    eps = float(np.float32(1e-12))

    xs = [torch.from_numpy(x).to(dev)]
    ms = [torch.from_numpy(mask).to(dev)]
    for _ in range(nsets - 1):
        xs.append(xs[0].clone())
        ms.append(ms[0].clone())
    outs = [torch.empty((B, C, s * H, s * W), dtype=torch.float32, device=dev)
            for _ in range(nsets)]

    def launch(i: int) -> None:
        sptr = torch.cuda.current_stream(dev).cuda_stream
        st = _lib.convex_upsample_f32(xs[i].data_ptr(), ms[i].data_ptr(), B, C, H, W, s, True,
                                      eps, outs[i].data_ptr(), flags, sptr)
        if st != 0:
            raise RuntimeError(f"convex_upsample_f32 failed: {st} {_lib.last_error()}")

    tm = Timer(dev, launch, nsets, args.steps, args.warmup, bytes_per_call)
    t_cold, t_warm, t_eager = tm.run()
    copy_gbps = tm.copy_ceiling_gbps()
    if args.calib:
        tm.calib()

    launch_s = t_cold / args.steps
    opx = B * s * s * H * W * args.steps  # output pixels
    line = base_line(
        args, "output Mpixel/s (+ achieved HBM GB/s, % of peak), DSINE convex upsample x8 + "
              "L2 normalise, 256x256 -> 2048x2048 fp32",
        opx / t_cold / 1e6, "Mpixel/s", t_cold * 1e3 / args.steps,
        {
            "workload": w.name, "B": B, "C": C, "H": H, "W": W, "scale": s,
            "mask": f"logits ~ N(0, {w.mask_sigma}^2)", "x": "unit normals, independent per pixel",
            "kernel_mode": "fp64" if args.precise else "fast",
            "inputs": f"{nsets} rotating HBM-resident copies "
                      f"({nsets * bytes_per_call / 1e6:.0f} MB > 256 MB Infinity Cache)",
        })
    line["roofline"] = roofline(
        bytes_per_call, launch_s,
        None if args.precise else traffic_from_profile("upsample", w.name),
        f"upsample8_kernel<{C}>" if s == 8 else f"upsample_kernel<{C}>", copy_gbps)
    line["warm"] = {
        "value": round(opx / t_warm / 1e6, 2),
        "launch_us_mean": round(t_warm / args.steps * 1e6, 3),
        "achieved_gbps": round(bytes_per_call / (t_warm / args.steps) / 1e9, 1),
    }
    line["eager"] = {
        "value": round(opx / t_eager / 1e6, 2),
        "us_per_step": round(t_eager / args.steps * 1e6, 3),
        "note": "the same steps launched one by one from Python (host-bound)",
    }
    line["gpu"] = torch.cuda.get_device_name(dev)

    if not args.no_cpu:
        def cpu_pass(nt):
            return lambda: oracle.convex_upsample(x, mask, H, W, s, normalize=True, eps=eps,
                                                  nthreads=nt)

        passes, el = timed_cpu(cpu_pass(1), args.cpu_seconds)
        line["cpu_baseline"] = {
            "value": round(passes * B * s * s * w.HW / el / 1e6, 4), "unit": "Mpixel/s",
            "cores": 1, "kind": "port",
            "sample": f"{passes} passes over the {w.name} input ({H}x{W} -> {s * H}x{s * W}), "
                      f"{el:.1f} s, oracle restatement of the upsample + normalise in double",
            "cpu": cpu_model(),
            "host_threads": os.cpu_count(),
        }
        nt = host_share()
        if nt > 1:
            passes_n, el_n = timed_cpu(cpu_pass(nt), args.cpu_seconds / 2)
            line["cpu_baseline_all_cores"] = {
                "value": round(passes_n * B * s * s * w.HW / el_n / 1e6, 4),
                "unit": "Mpixel/s", "cores": nt, "kind": "port",
                "sample": f"{passes_n} passes, {el_n:.1f} s, rows over {nt} OpenMP threads",
            }
    return line


def bench_refiner(args, dev) -> dict:
    """The whole NRN refiner forward (brovisionml_amd/refiner.py: 5 iterations
    of ConvGRU + heads on MIOpen, the package's propagate with fused
    activations and its upsample + normalise) at a 256x256 grid (a 2048x2048
    image), synthetic weights and decoder outputs, one forward per step,
    captured in one graph.  The CPU leg is its restatement in oracle/refiner.py
    (float64 convolutions, the C oracle's ops) on a 24x32 grid."""
    import torch
    from brovisionml_amd import refiner as rf, workloads as wl

    H = W = 256 if args.workload is None or args.workload == 0 else 64
    rng = np.random.default_rng(0)
    normal = rng.standard_normal((1, 3, H, W))
    normal[:, 2] = np.abs(normal[:, 2]) + 0.5
    normal = (normal / np.linalg.norm(normal, axis=1, keepdims=True)).astype(np.float32)
    feature = rng.standard_normal((1, 64, H, W)).astype(np.float32)
    hidden = rng.uniform(-1, 1, (1, 64, H, W)).astype(np.float32)
    model = rf.Refiner(rf.random_weights(0), dev)
    dec = rf.DecoderOutput(*(torch.from_numpy(a).to(dev) for a in (normal, feature, hidden)))
    intr = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    cond = model.conditioning(intr, H, W, 8 * H, 8 * W)
    for _ in range(3):
        model.forward(dec, intr, 8 * H, 8 * W, cond=cond)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(args.steps):
            model.forward(dec, intr, 8 * H, 8 * W, cond=cond)
    g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3
    opx = 64 * H * W * args.steps
    line = base_line(args, f"output Mpixel/s, DSINE NRN refiner forward (5 iterations), {H}x{W} "
                           f"grid -> {8 * H}x{8 * W} fp32", opx / t / 1e6, "Mpixel/s",
                     t * 1e3 / args.steps,
                     {"workload": f"dsine-refiner-{H}x{W}", "H": H, "W": W, "iterations": 5,
                      "weights": "synthetic (uniform +-1/sqrt(fan_in))",
                      "convolutions": "torch F.conv2d (MIOpen), fp32"})
    line["gpu"] = torch.cuda.get_device_name(dev)
    if not args.no_cpu:
        import oracle.refiner as oref
        h2, w2 = 24, 32
        intr2 = wl.intrins_from_fov(8 * h2, 8 * w2, 60.0)
        fuv2 = wl.scaled_intrinsics(intr2, h2, w2, 8 * h2, 8 * w2)
        ray2 = wl.build_ray8(intr2, h2, w2, 8 * h2, 8 * w2).reshape(3, h2, w2)
        uv2 = rf.uv_map(intr2, h2, w2, 8 * h2, 8 * w2)
        w0 = rf.random_weights(0)
        n2, f2, hd2 = normal[0, :, :h2, :w2], feature[0, :, :h2, :w2], hidden[0, :, :h2, :w2]
        n2 = (n2 / np.linalg.norm(n2, axis=0)).astype(np.float32)
        nthr = torch.get_num_threads()
        torch.set_num_threads(1)
        passes, el = timed_cpu(lambda: oref.refine_forward(w0, n2, f2, hd2, intr2, fuv2, ray2,
                                                           uv2), args.cpu_seconds)
        torch.set_num_threads(nthr)
        line["cpu_baseline"] = {
            "value": round(passes * 64 * h2 * w2 / el / 1e6, 4), "unit": "Mpixel/s", "cores": 1,
            "kind": "port",
            "sample": f"{passes} forwards of a {h2}x{w2} grid, {el:.1f} s: float64 torch "
                      "convolutions and the C oracle's ops, one thread",
            "cpu": cpu_model(),
        }
    return line


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--op", choices=("angmf", "upsample", "refiner"), default="angmf")
    ap.add_argument("--workload", type=int, default=None,
                    help="index into the op's workloads (default: angmf 2, upsample 0)")
    ap.add_argument("--sets", type=int, default=0, help="rotating input sets (0 = auto, > 512 MB)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--ray-from-intrinsics", action="store_true",
                    help="angmf: form each pixel's ray from fu, cu, fv, cv in the kernel "
                         "(BVML_DSINE_RAY_FROM_INTRINSICS) instead of reading the ray planes")
    ap.add_argument("--logits", action="store_true",
                    help="angmf: prob and angle hold the heads' raw logits and the kernel applies "
                         "the activations (BVML_DSINE_LOGITS); also times the unfused step")
    ap.add_argument("--precise", action="store_true",
                    help="upsample: the double-precision kernel (BVML_DSINE_FP64)")
    ap.add_argument("--calib", action="store_true",
                    help="also run 10 plain device copies of one launch's byte count "
                         "(the reference kernel for the FETCH_SIZE / WRITE_SIZE scale)")
    args = ap.parse_args()
    if args.workload is None and args.op != "refiner":
        args.workload = 2 if args.op == "angmf" else 0

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the op shards by frames or row bands with no collective on the path, "
              "so run --gpus 1", file=sys.stderr)
        return 2

    import torch
    from brovisionml_amd import _lib

    if not torch.cuda.is_available():
        print("bench.py: no HIP device", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    _lib.load()
    line = {"angmf": bench_angmf, "upsample": bench_upsample,
            "refiner": bench_refiner}[args.op](args, dev)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
