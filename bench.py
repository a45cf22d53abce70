"""Benchmark: DSINE AngMF propagate on one MI355X (and, with --op upsample,
the refiner's fused convex upsample + L2-normalise; --op refiner, the whole
refiner forward).

A step is one pass of the hot path over one batch: one angmf_propagate call
(workload 2: B=1, 256x256, k=5, fp32) through the C ABI, inputs resident in
HBM.  Each step reads a different one of `--sets` input sets, each an
independent seeded draw of the workload (draw 0 is its stated seed), which
together exceed 512 MB, so the 256 MB Infinity Cache cannot serve them; the
timed replay starts after a 512 MB flush.  The warm figure (one set, read by
every step) is measured after the cold ones, on a set of its own.

The K timed steps of the propagate are K calls of its C ABI enqueued back to
back from C++ (tests/hw/probe.hip, bvml_probe_angmf_loop), as a C++ caller
such as the refiner issues them: a short bounded spin kernel holds the stream
while the host enqueues the K calls, and two HIP events on that stream, one
right after the spin and one after the last call, bracket exactly the K
launches on the GPU.  The same K launches captured in one HIP graph and
replayed between two events are reported beside it ("graph"): a replay
carries a fixed cost of its own (about 9 us on the GPU at 256 x 256, so
0.45 us per launch at K = 20), and the first replay timed in a process read
about 20% slow, with a host-side gap inside its events.  The upsample and
the refiner forward are timed as graph replays.  Per-launch durations come
from an eager pass over the same rotation with an event pair around every
launch (median and max reported).

Prints one JSON line (rank 0):
  value         Mpixel/s over the timed region (K steps / event time)
  roofline      algorithmic bytes per launch / mean launch time, against the
                8 TB/s HBM peak, with the same-box read ceiling (a streaming
                read of each set's inputs) and copy ceiling over the same
                rotating footprint
  cpu_baseline  the CPU oracle (double-precision restatement of the
                reference's CPU twin), one thread, on a bounded sample
  configs       the other workloads (0, 1, 3, 4): cold and warm time per call,
                Mpixel/s, roofline fraction and their own CPU baseline
  fp64          the double-precision reference-order kernel on the headline
                workload (BVML_DSINE_FP64)
  recompute     per set, the pixels below the fast path's cancellation
                threshold (recomputed in double), from the oracle's sums
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix peak
HBM_PEAK_GBPS = 8000.0
FLUSH_BYTES = 512 << 20
# Back-to-back work before each timed region, to bring the clocks up (Timer.ramp).
RAMP_SECONDS = 0.3
# The ramp before the process's first timed region (Timer.timed_graph): on a
# box that has just been idle, the first timed regions ran about 20% slower
# than every later one after a 0.3 s ramp (a 256 x 256 call: 10.5 and 10.1 us
# per launch in the first two regions of a process, 8.7-8.9 in the next
# sixteen, each after its own ramp of graph replays), and 2 s of Python-launched
# work before the first ramp did not change that (10.4 us): the GPU needs
# longer at full load the first time.
SETTLE_SECONDS = 2.0


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


PROFILES = os.path.join(ROOT, "profiles")


def traffic_from_profile(op: str, name: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (profiles/<op>_*_traffic.json: FETCH_SIZE + WRITE_SIZE per dispatch,
    scaled by the same counters on a plain copy of known size) that covers
    this workload, if any."""
    import glob
    for path in sorted(glob.glob(os.path.join(PROFILES, f"{op}*_traffic.json"))):
        try:
            with open(path) as f:
                p = json.load(f)
        except (OSError, ValueError):
            continue
        if p.get("workload") == name:
            return p.get("traffic_bytes_per_launch")
    return None


def angmf_kernel_name(w, flags) -> str:
    """The fp32 kernel instantiation a launch of workload w runs, spelled as
    rocprofv3 prints it: angmf_f32_kernel<k, waves per group, rays from the
    intrinsics, logits, non-temporal plane loads>."""
    from brovisionml_amd import _lib
    _, intr = w.intrinsics()
    fp32, g, _, _, nt = _lib.angmf_plan_full(w.B, w.H, w.W, w.k, *intr, flags=flags)
    if not fp32:
        return f"angmf_f64_kernel<{w.k}>"
    tf = lambda b: "true" if b else "false"
    return (f"angmf_f32_kernel<{w.k}, {g}, {tf(flags & _lib.RAY_FROM_INTRINSICS)}, "
            f"{tf(flags & _lib.LOGITS)}, {tf(nt)}>")


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
    """Timing of `launch(i)` (i selects the input set) over a rotation of
    nsets sets: graph-captured cold and warm replays, an eager pass with
    per-launch events, and the same-box read and copy ceilings over the same
    footprint."""

    ramp_seconds = RAMP_SECONDS
    settled = False  # whether this process has run its SETTLE_SECONDS ramp

    def __init__(self, dev, launch, nsets: int, steps: int, warmup: int, bytes_per_call: int,
                 warm_index: int | None = None, loop=None):
        import torch
        self.torch, self.dev = torch, dev
        self.launch, self.nsets, self.steps = launch, nsets, steps
        # loop(indices) -> seconds: the launches of those sets enqueued back
        # to back from C++ and timed on the GPU (angmf_loop); None: time
        # graph replays
        self.loop = loop
        self.bytes_per_call = bytes_per_call
        self.warm_index = warm_index
        self._flush_buf = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)
        self._mark_buf = torch.zeros(1, dtype=torch.int32, device=dev)
        for i in range(warmup):
            launch(i % nsets)
        torch.cuda.synchronize()

    def flush(self):
        """Read 512 MB, so nothing read before stays in the Infinity Cache.  A
        read, not a write: 512 MB of dirty lines would be written back while
        the timed kernels run and take HBM bandwidth from them."""
        self._flush_sum = self._flush_buf.sum()

    def mark(self):
        """One tiny kernel (a 1-element bitwise not, which nothing else here
        launches) right before each timed region, so a kernel trace of the run
        can find the timed launches among the clock ramp's."""
        self._mark_buf.bitwise_not_()

    def capture(self, sets):
        g = self.torch.cuda.CUDAGraph()
        with self.torch.cuda.graph(g):
            for i in sets:
                self.launch(i)
        return g

    def ramp(self, work, seconds: float | None = None) -> None:
        """Run `work` back to back for ramp_seconds (or `seconds`): the GPU lowers its clocks
        when idle (input generation on the host leaves it idle for seconds)
        and takes tens of milliseconds of load to raise them again, so a
        timed replay straight after idle time measures the clock ramp, not
        the kernel (4 x 512 x 512, k = 7: 184 us per launch right after 5 s of
        idle, 152 us at steady clocks)."""
        torch = self.torch
        limit = self.ramp_seconds if seconds is None else seconds
        t0 = time.perf_counter()
        while True:
            work()
            torch.cuda.synchronize()
            if time.perf_counter() - t0 >= limit:
                return

    def timed_graph(self, g, flush: bool):
        torch = self.torch
        stream = torch.cuda.current_stream(self.dev)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        self.ramp(g.replay, None if Timer.settled else SETTLE_SECONDS)
        Timer.settled = True
        if flush:
            self.flush()
        self.mark()
        torch.cuda.synchronize()
        e0.record(stream)
        g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3

    def timed_loop(self, idx, flush: bool) -> float:
        """Seconds for the launches of sets idx enqueued from C++ (self.loop),
        after the ramp (the same loop back to back) and, if asked, a flush."""
        torch = self.torch
        self.ramp(lambda: self.loop(idx), None if Timer.settled else SETTLE_SECONDS)
        Timer.settled = True
        if flush:
            self.flush()
        self.mark()
        torch.cuda.synchronize()
        t = self.loop(idx)
        torch.cuda.synchronize()
        return t

    def cold(self) -> float:
        """Seconds for self.steps launches rotating over the sets, starting
        after a flush: the C++ loop where the Timer has one, else one graph
        replay."""
        idx = [i % self.nsets for i in range(self.steps)]
        if self.loop is not None:
            return self.timed_loop(idx, flush=True)
        return self.cold_graph()

    def cold_graph(self) -> float:
        """cold() as one replay of a graph of the launches."""
        g = self.capture([i % self.nsets for i in range(self.steps)])
        g.replay()
        return self.timed_graph(g, flush=True)

    def warm(self) -> float:
        """Seconds for self.steps launches of one set (Infinity Cache warm)."""
        w = self.warm_index if self.warm_index is not None else 0
        if self.loop is not None:
            return self.timed_loop([w] * self.steps, flush=False)
        g = self.capture([w] * self.steps)
        g.replay()
        return self.timed_graph(g, flush=False)

    def eager(self):
        """(total s, per-launch us list): the rotation launched one by one
        from Python with an event pair around each launch (after a flush)."""
        torch = self.torch
        stream = torch.cuda.current_stream(self.dev)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(self.steps)]

        def rotation():
            for i in range(self.steps):
                self.launch(i % self.nsets)
        self.ramp(rotation)
        self.flush()
        self.mark()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(self.steps):
            ev[i][0].record(stream)
            self.launch(i % self.nsets)
            ev[i][1].record(stream)
        torch.cuda.synchronize()
        total = time.perf_counter() - t0
        return total, [a.elapsed_time(b) * 1e3 for a, b in ev]

    def read_ceiling_gbps(self, bufs) -> float:
        """A streaming read of one set's inputs (one flat buffer per set;
        each lane issues 2, 4 or 8 float4 non-temporal loads before using
        them, tests/hw/probe.hip) per launch, over the same rotation,
        captured in one graph: the same-box read rate of this footprint, the
        best of the three unrolls."""
        torch = self.torch
        from tests.hw import probe
        best = 0.0
        for unroll in (2, 4, 8):
            n_part = max(probe.read_partials(b.numel(), unroll) for b in bufs)
            part = torch.empty(n_part, dtype=torch.float32, device=self.dev)
            n_rep = max(self.steps, 2 * len(bufs))
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                sptr = torch.cuda.current_stream(self.dev).cuda_stream
                for i in range(n_rep):
                    b = bufs[i % len(bufs)]
                    probe.stream_read(b.data_ptr(), b.numel(), unroll, part.data_ptr(), n_part,
                                      sptr)
            g.replay()
            t = self.timed_graph(g, flush=True)
            best = max(best, sum(bufs[i % len(bufs)].numel() * 4 for i in range(n_rep)) / t / 1e9)
        return best

    def copy_ceiling_gbps(self) -> float:
        """Device copies that each move one launch's algorithmic bytes (half
        read, half written), rotating over a footprint of the kernel's
        size, captured in one graph like the kernel's launches."""
        torch = self.torch
        n_copy = self.bytes_per_call // 8
        nsets = max(2, int(np.ceil(FLUSH_BYTES / (2 * n_copy * 4))))
        src = torch.ones(nsets, n_copy, dtype=torch.float32, device=self.dev)
        dst = torch.empty_like(src)
        n_rep = max(self.steps, 2 * nsets)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n_rep):
                dst[i % nsets].copy_(src[i % nsets])
        g.replay()
        t = self.timed_graph(g, flush=True)
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


def roofline(bytes_per_call, launch_s, traffic, kernel, copy_gbps, read_gbps=None):
    achieved = bytes_per_call / launch_s / 1e9
    r = {
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
    if read_gbps is not None:
        r["read_ceiling_gbps"] = round(read_gbps, 1)
        r["frac_of_read_ceiling"] = round(achieved / read_gbps, 4)
    return r


# ---------------------------------------------------------------------------
# angmf_propagate
# ---------------------------------------------------------------------------

PLANES = ("pred_norm", "prob", "xy", "angle")


def _activate_logits(inp):
    """The heads' raw logits of a draw's planes: the prob planes' logits and
    the angle planes' logits of angle / pi, so the activations give them back."""
    inp = dict(inp)
    for key, scale in (("prob", 1.0), ("angle", np.pi)):
        q = np.clip(inp[key].astype(np.float64) / scale, 1e-6, 1 - 1e-6)
        inp[key] = np.log(q / (1.0 - q)).astype(np.float32)
    return inp


class AngmfSets:
    """nsets independent draws of a workload on the device, each one flat
    buffer (so a single reduction reads a whole set) with views per tensor,
    and an output per set."""

    def __init__(self, w, nsets, dev, logits=False, extra_warm=True):
        import torch
        self.w, self.nsets = w, nsets
        self.sets, self.bufs, self.outs, self.host = [], [], [], []
        total = nsets + (1 if extra_warm else 0)
        for d in range(total):
            inp = w_inputs(w, d if d < nsets else 0)
            self.host.append(inp if d < nsets else None)
            dev_inp = _activate_logits(inp) if logits else inp
            arrs = [np.ascontiguousarray(dev_inp[k], np.float32).ravel() for k in PLANES]
            arrs.append(np.ascontiguousarray(inp["ray"], np.float32).ravel())
            flat = torch.from_numpy(np.concatenate(arrs)).to(dev)
            views, off = {}, 0
            for key, a in zip(PLANES + ("ray",), arrs):
                views[key] = flat[off:off + a.size]
                off += a.size
            self.sets.append(views)
            self.bufs.append(flat)
            self.outs.append(torch.empty_like(views["pred_norm"]))
        self.intr = self.host[0]["intrinsics"]
        self.warm_index = nsets if extra_warm else 0


def w_inputs(w, draw):
    return wl_mod().make_inputs(w, draw)


def wl_mod():
    from brovisionml_amd import workloads
    return workloads


def nsets_for(bytes_per_call: int, cap: int = 256) -> int:
    return int(min(cap, max(2, np.ceil(FLUSH_BYTES / bytes_per_call))))


def angmf_launcher(sets: AngmfSets, dev, flags: int, ray_from_intrinsics: bool, calls: int):
    import torch
    from brovisionml_amd import _lib
    w = sets.w
    fu, cu, fv, cv = sets.intr

    def launch(i: int) -> None:
        s = sets.sets[i]
        sptr = torch.cuda.current_stream(dev).cuda_stream
        pn = s["pred_norm"]
        for c in range(calls):
            # a chain: each call's output feeds the next call's pred_norm; the
            # set's output buffer alternates with a second one
            dst = sets.outs[i] if c % 2 == 0 else sets.outs2[i]
            st = _lib.angmf_propagate_f32(
                pn.data_ptr(), s["prob"].data_ptr(), s["xy"].data_ptr(), s["angle"].data_ptr(),
                0 if ray_from_intrinsics else s["ray"].data_ptr(), fu, cu, fv, cv, w.B, w.H,
                w.W, w.k, 0, dst.data_ptr(), flags, sptr)
            if st != 0:
                raise RuntimeError(f"angmf_propagate_f32 failed: {st} {_lib.last_error()}")
            pn = dst

    if calls > 1:
        sets.outs2 = [torch.empty_like(o) for o in sets.outs]
    return launch


def angmf_loop_timer(sets: AngmfSets, dev, flags: int, ray_from_intrinsics: bool, calls: int):
    """loop(indices) -> seconds: the calls of those sets (a chain of `calls`
    per set, each output feeding the next) enqueued back to back from C++
    through the C ABI's function pointer (tests/hw/probe.hip), timed by HIP
    events on the current stream right after a bounded spin that holds the
    stream while they are enqueued."""
    import ctypes
    import torch
    from brovisionml_amd import _lib
    from tests.hw import probe
    w = sets.w
    fn = ctypes.cast(_lib.load().bvml_dsine_angmf_propagate_f32, ctypes.c_void_p).value
    if calls > 1 and not hasattr(sets, "outs2"):
        sets.outs2 = [torch.empty_like(o) for o in sets.outs]

    def rows(i):
        s = sets.sets[i]
        pn, out = s["pred_norm"].data_ptr(), []
        for c in range(calls):
            dst = (sets.outs[i] if c % 2 == 0 else sets.outs2[i]).data_ptr()
            out.append([pn, s["prob"].data_ptr(), s["xy"].data_ptr(), s["angle"].data_ptr(),
                        0 if ray_from_intrinsics else s["ray"].data_ptr(), dst])
            pn = dst
        return out

    def loop(idx) -> float:
        ptrs = [r for i in idx for r in rows(i)]
        # the spin covers the host's enqueueing: about 5 us per call, doubled
        spin_us = min(1e5, 10.0 * len(ptrs) + 100.0)
        return probe.angmf_loop(fn, ptrs, sets.intr, w.B, w.H, w.W, w.k, flags, spin_us,
                                torch.cuda.current_stream(dev).cuda_stream)
    return loop


def recompute_counts(sets: AngmfSets, flags: int, nthreads: int):
    """Per set: pixels below the fast path's cancellation threshold, from
    the oracle's double sums (|acc|^2 / sum (prob/|p|)^2)."""
    import oracle
    from brovisionml_amd import _lib
    w = sets.w
    t = _lib.angmf_recompute_ratio(w.k, flags)
    counts = []
    for inp in sets.host:
        if inp is None:
            continue
        _, acc, qs = oracle.angmf_propagate(inp["pred_norm"], inp["prob"], inp["xy"],
                                            inp["angle"], inp["ray"], inp["intrinsics"], w.H,
                                            w.W, w.k, nthreads=nthreads, return_acc=True,
                                            return_qs=True)
        a2 = (acc.reshape(w.B, 3, -1) ** 2).sum(axis=1)
        counts.append(int((a2 < t * qs).sum()))
    return t, counts


def cpu_baseline_angmf(w, inp, seconds: float, nthreads: int = 1):
    """The oracle on whole images (or row bands of a large one) of the
    workload for about `seconds`: (Mpixel/s, sample text)."""
    import oracle
    H, W, k, B = w.H, w.W, w.k, w.B
    band = H if (B * w.HW <= 1 << 17 or w.calls > 1) else max(1, (1 << 17) // (B * W))
    px_done, passes, y0 = 0, 0, 0
    t0 = time.perf_counter()
    while True:
        y1 = min(H, y0 + band)
        pn = inp["pred_norm"]
        for _ in range(w.calls):
            # (a chain runs whole images: band == H whenever calls > 1)
            pn = oracle.angmf_propagate(pn, inp["prob"], inp["xy"], inp["angle"], inp["ray"],
                                        inp["intrinsics"], H, W, k, rows=(y0, y1),
                                        nthreads=nthreads)
        px_done += B * (y1 - y0) * W * w.calls
        passes += 1
        y0 = 0 if y1 >= H else y1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    what = (f"{passes} passes of {band} of {H} rows" if band < H else f"{passes} passes")
    return px_done / el / 1e6, f"{what} over the {w.name} input (B={B}, {H}x{W}, k={k}), {el:.1f} s"


def measure_angmf(args, dev, w, steps, warmup, flags=0, ray_from_intrinsics=False,
                  logits=False, with_ceilings=True, with_eager=True):
    """Cold/warm timing of one workload; returns a dict of figures."""
    import torch
    bytes_per_call = w.algorithmic_bytes(shared_ray=True) // w.calls
    if ray_from_intrinsics:
        bytes_per_call -= 3 * w.HW * 4
    nsets = args.sets or nsets_for(bytes_per_call * w.calls)
    sets = AngmfSets(w, nsets, dev, logits=logits)
    launch = angmf_launcher(sets, dev, flags, ray_from_intrinsics, w.calls)
    loop = angmf_loop_timer(sets, dev, flags, ray_from_intrinsics, w.calls)
    tm = Timer(dev, launch, nsets, steps, warmup, bytes_per_call, warm_index=sets.warm_index,
               loop=loop)
    t_cold = tm.cold()
    res = {"sets": sets, "timer": tm, "bytes_per_call": bytes_per_call, "nsets": nsets,
           "launch_s": t_cold / (steps * w.calls), "t_cold": t_cold}
    if with_eager:
        res["t_cold_graph"] = tm.cold_graph()
    if with_eager:
        t_eager, per = tm.eager()
        res["t_eager"], res["per_launch_us"] = t_eager, per
    res["t_warm"] = tm.warm()
    if with_ceilings:
        res["copy_gbps"] = tm.copy_ceiling_gbps()
        res["read_gbps"] = tm.read_ceiling_gbps(sets.bufs[:nsets])
    torch.cuda.synchronize()
    return res


def bench_angmf(args, dev) -> dict:
    import torch
    from brovisionml_amd import _lib
    W_ = wl_mod()

    w = W_.WORKLOADS[args.workload]
    flags = _lib.DEFAULT
    if args.ray_from_intrinsics:
        flags |= _lib.RAY_FROM_INTRINSICS
    if args.logits:
        flags |= _lib.LOGITS
    m = measure_angmf(args, dev, w, args.steps, args.warmup, flags, args.ray_from_intrinsics,
                      args.logits)
    sets, tm, bytes_per_call, nsets = m["sets"], m["timer"], m["bytes_per_call"], m["nsets"]
    if args.calib:
        tm.calib()
    B, H, W, k = w.B, w.H, w.W, w.k
    px = B * H * W * w.calls * args.steps
    per = np.array(m["per_launch_us"])
    line = base_line(
        args, "Mpixel/s (+ achieved HBM GB/s, % of peak), DSINE propagation 256x256 k=5 fp32",
        px / m["t_cold"] / 1e6, "Mpixel/s", m["t_cold"] * 1e3 / args.steps,
        {
            "workload": w.name, "B": B, "H": H, "W": W, "k": k, "calls_per_step": w.calls,
            "ray": "from-intrinsics" if args.ray_from_intrinsics else "shared",
            "prob_angle": "logits, activated in the kernel" if args.logits else "activated",
            "inputs": f"{nsets} independent seeded draws, rotating "
                      f"({nsets * bytes_per_call * w.calls / 1e6:.0f} MB > 256 MB Infinity "
                      "Cache); timed after a 512 MB flush",
            "timing": "K calls enqueued back to back from C++ behind a spin that holds the "
                      "stream; HIP events around the K launches on the GPU",
        })
    line["roofline"] = roofline(
        bytes_per_call, m["launch_s"],
        None if (args.ray_from_intrinsics or args.logits) else traffic_from_profile("angmf", w.name),
        angmf_kernel_name(w, flags), m["copy_gbps"], m["read_gbps"])
    line["per_launch"] = {
        "us_median": round(float(np.median(per)), 3),
        "us_max": round(float(per.max()), 3),
        "us_min": round(float(per.min()), 3),
        "note": "eager pass over the same rotation, an event pair around each launch "
                "(includes the events' own overhead)",
    }
    line["warm"] = {
        "value": round(px / m["t_warm"] / 1e6, 2),
        "launch_us_mean": round(m["t_warm"] / (args.steps * w.calls) * 1e6, 3),
        "achieved_gbps": round(bytes_per_call / (m["t_warm"] / (args.steps * w.calls)) / 1e9, 1),
        "note": "one set, not part of the rotation, read by every launch",
    }
    line["eager"] = {
        "value": round(px / m["t_eager"] / 1e6, 2),
        "us_per_step": round(m["t_eager"] / args.steps * 1e6, 3),
        "note": "the same steps launched one by one from Python with per-launch events",
    }
    line["graph"] = {
        "value": round(px / m["t_cold_graph"] / 1e6, 2),
        "us_per_step": round(m["t_cold_graph"] / args.steps * 1e6, 3),
        "note": "the same K launches captured in one HIP graph, one replay between two events "
                "after a flush (a replay carries a fixed cost of its own)",
    }
    line["gpu"] = torch.cuda.get_device_name(dev)
    nt = host_share()
    t_ratio, counts = recompute_counts(sets, flags, nt)
    line["recompute"] = {
        "threshold": t_ratio,
        "pixels_per_call_mean": round(float(np.mean(counts)), 3),
        "pixels_per_call_max": int(max(counts)),
        "calls_with_any": int(sum(c > 0 for c in counts)),
        "calls": len(counts),
        "note": "pixels with |acc|^2 < threshold * sum (prob/|p|)^2 (oracle sums), which the "
                "fast path recomputes in double",
    }

    if not args.logits and not args.ray_from_intrinsics:
        # the double-precision reference-order kernel on the same rotation
        fl = flags | _lib.FP64
        launch64 = angmf_launcher(sets, dev, fl, False, w.calls)
        k64 = max(4, args.steps // 4)
        t64 = Timer(dev, launch64, nsets, k64, 1, bytes_per_call, warm_index=sets.warm_index,
                    loop=angmf_loop_timer(sets, dev, fl, False, w.calls))
        t = t64.cold()
        line["fp64"] = {
            "kernel": f"angmf_f64_kernel<{k}>",
            "launch_us_mean": round(t / k64 * 1e6, 3),
            "achieved_gbps": round(bytes_per_call / (t / k64) / 1e9, 1),
            "note": "BVML_DSINE_FP64: every neighbour in double in the reference's operation "
                    "order, one pixel per lane",
        }

    if args.logits:
        # the unfused step for comparison: the refiner's two activation
        # passes (here torch's sigmoid kernels) over the same rotating
        # logits, then the op on the activated planes
        acts = [(torch.empty_like(s_["prob"]), torch.empty_like(s_["angle"]))
                for s_ in sets.sets]
        kpi = float(np.float32(np.pi))
        fu, cu, fv, cv = sets.intr

        def launch_unfused(i: int) -> None:
            s_ = sets.sets[i]
            ap_, aa_ = acts[i]
            torch.sigmoid(s_["prob"], out=ap_)
            torch.sigmoid(s_["angle"], out=aa_)
            aa_.mul_(kpi)
            sptr = torch.cuda.current_stream(dev).cuda_stream
            st = _lib.angmf_propagate_f32(
                s_["pred_norm"].data_ptr(), ap_.data_ptr(), s_["xy"].data_ptr(), aa_.data_ptr(),
                0 if args.ray_from_intrinsics else s_["ray"].data_ptr(), fu, cu, fv, cv, B, H,
                W, k, 0, sets.outs[i].data_ptr(), flags & ~_lib.LOGITS, sptr)
            if st != 0:
                raise RuntimeError(f"angmf_propagate_f32 failed: {st} {_lib.last_error()}")

        tu = Timer(dev, launch_unfused, nsets, args.steps, args.warmup, bytes_per_call)
        line["unfused"] = {
            "us_per_step": round(tu.cold() / args.steps * 1e6, 3),
            "note": "torch sigmoid on the prob logits, sigmoid and * pi on the angle logits, "
                    "then the op on the activated planes; same rotating inputs, one graph",
        }

    inp0 = sets.host[0]
    del sets, tm, m
    torch.cuda.empty_cache()

    if not args.no_cpu:
        v, sample = cpu_baseline_angmf(w, inp0, args.cpu_seconds)
        line["cpu_baseline"] = {
            "value": round(v, 4), "unit": "Mpixel/s", "cores": 1, "kind": "port",
            "sample": sample + ", oracle restatement of src/dsine_ops.cpp in double",
            "cpu": cpu_model(), "host_threads": os.cpu_count(),
        }
        # the same oracle with its rows split over the host's CPU share
        # (OpenMP); the reference itself is single-threaded
        if nt > 1:
            vn, sample_n = cpu_baseline_angmf(w, inp0, args.cpu_seconds / 2, nthreads=nt)
            line["cpu_baseline_all_cores"] = {
                "value": round(vn, 4), "unit": "Mpixel/s", "cores": nt, "kind": "port",
                "sample": sample_n + f", rows over {nt} OpenMP threads",
            }

    if args.configs and not (args.logits or args.ray_from_intrinsics):
        line["configs"] = bench_configs(args, dev, [i for i in (0, 1, 2, 3, 4)
                                                    if i != args.workload])
        # the propagate as the refiner runs it: on the heads' raw logits
        # (BVML_DSINE_LOGITS), whose planes the heads pass has just written
        # (warm), and cold for comparison
        ml = measure_angmf(args, dev, w, args.steps, args.warmup, flags | _lib.LOGITS,
                           logits=True, with_ceilings=False, with_eager=False)
        line["logits"] = {
            "kernel": angmf_kernel_name(w, flags | _lib.LOGITS),
            "warm_us_per_call": round(ml["t_warm"] / (args.steps * w.calls) * 1e6, 3),
            "cold_us_per_call": round(ml["launch_s"] * 1e6, 3),
            "bytes_per_call": ml["bytes_per_call"],
            "note": "prob and angle as the heads' raw logits, the activations applied in the "
                    "kernel; warm: one set read by every launch, as the refiner's propagate "
                    "reads what its heads pass has just written",
        }
        del ml
        torch.cuda.empty_cache()
        # the refiner's next steps on the same line: the fused convex
        # upsample x8 + normalise, and the whole native refiner forward
        sub = argparse.Namespace(**vars(args))
        sub.workload, sub.sets, sub.precise, sub.calib = 0, 0, False, False
        sub.cpu_seconds = args.cpu_seconds / 2
        line["upsample"] = sub_line(bench_upsample(sub, dev))
        sub.workload, sub.driver = None, "native"
        line["refiner"] = sub_line(bench_refiner(sub, dev))
    return line


def sub_line(line: dict) -> dict:
    """Another op's bench line as a sub-object of the default line: the
    run-wide keys dropped."""
    run_keys = ("n_gpus", "steps", "warmup", "higher_is_better", "scaling", "vs_baseline",
                "dtype", "data")
    return {k: v for k, v in line.items() if k not in run_keys}


def bench_configs(args, dev, indices) -> dict:
    """The other workloads: cold/warm time per call, Mpixel/s, roofline
    fraction and a CPU baseline of each."""
    import torch
    W_ = wl_mod()
    out = {}
    for idx in indices:
        w = W_.WORKLOADS[idx]
        steps = max(4, min(args.steps, 20 if w.B * w.HW * w.K2 > 1 << 24 else args.steps))
        m = measure_angmf(args, dev, w, steps, 2, with_ceilings=False, with_eager=False)
        bpc, nsets = m["bytes_per_call"], m["nsets"]
        px_call = w.B * w.HW
        entry = {
            "B": w.B, "H": w.H, "W": w.W, "k": w.k, "calls_per_step": w.calls,
            "kernel": angmf_kernel_name(w, 0),
            "cold_us_per_call": round(m["launch_s"] * 1e6, 3),
            "warm_us_per_call": round(m["t_warm"] / (steps * w.calls) * 1e6, 3),
            "mpixel_s": round(px_call / m["launch_s"] / 1e6, 1),
            "achieved_gbps": round(bpc / m["launch_s"] / 1e9, 1),
            "frac": round(bpc / m["launch_s"] / 1e9 / HBM_PEAK_GBPS, 4),
            "bytes_per_call": bpc,
            "traffic": traffic_from_profile("angmf", w.name),
            "inputs": f"{nsets} independent draws ({nsets * bpc * w.calls / 1e6:.0f} MB), "
                      "timed after a 512 MB flush; K calls enqueued from C++",
        }
        if w.calls > 1:
            entry["note"] = f"{w.calls} chained calls per step (each output feeds the next call)"
        inp0 = m["sets"].host[0]
        del m
        torch.cuda.empty_cache()
        if not args.no_cpu:
            v, sample = cpu_baseline_angmf(w, inp0, args.cpu_seconds / 3)
            entry["cpu_baseline"] = {"value": round(v, 4), "unit": "Mpixel/s", "cores": 1,
                                     "kind": "port", "sample": sample}
        out[w.name] = entry
    return out


# ---------------------------------------------------------------------------
# RayReLU
# ---------------------------------------------------------------------------

def bench_ray_relu(args, dev) -> dict:
    """RayReLU in place on the normal map of a propagate workload's shape
    (src/dsine_ops.cu:58-74; the refiner runs it once per forward on the
    decoder's normals, src/dsine_refine.cpp:241-243): cold graph replays
    over independent draws, like the propagate's."""
    import torch
    from brovisionml_amd import _lib
    W_ = wl_mod()
    w = W_.WORKLOADS[args.workload]
    B, H, W, HW = w.B, w.H, w.W, w.HW
    # normal read + written per sample, the shared ray read once
    bytes_per_call = (B * 6 + 3) * HW * 4
    nsets = args.sets or nsets_for(bytes_per_call)
    bufs, normals, rays = [], [], []
    for d in range(nsets + 1):
        inp = W_.make_inputs(w, d if d < nsets else 0)
        flat = torch.from_numpy(np.concatenate([inp["pred_norm"].ravel(),
                                                inp["ray"].ravel()])).to(dev)
        normals.append(flat[:B * 3 * HW])
        rays.append(flat[B * 3 * HW:])
        bufs.append(flat)

    def launch(i: int) -> None:
        sptr = torch.cuda.current_stream(dev).cuda_stream
        st = _lib.ray_relu_f32(normals[i].data_ptr(), rays[i].data_ptr(), B, H, W, 0, sptr)
        if st != 0:
            raise RuntimeError(f"ray_relu_f32 failed: {st} {_lib.last_error()}")

    tm = Timer(dev, launch, nsets, args.steps, args.warmup, bytes_per_call, warm_index=nsets)
    t_cold = tm.cold()
    t_warm = tm.warm()
    copy_gbps = tm.copy_ceiling_gbps()
    read_gbps = tm.read_ceiling_gbps(bufs[:nsets])
    launch_s = t_cold / args.steps
    vec4 = HW % 4 == 0
    line = base_line(
        args, f"Mpixel/s (+ achieved HBM GB/s, % of peak), DSINE RayReLU {w.name}",
        B * HW * args.steps / t_cold / 1e6, "Mpixel/s", t_cold * 1e3 / args.steps,
        {"workload": w.name, "B": B, "H": H, "W": W,
         "kernel_mode": "4 pixels per lane" if vec4 else "1 pixel per lane",
         "inputs": f"{nsets} independent seeded draws, rotating; timed replay after a 512 MB "
                   "flush"})
    line["roofline"] = roofline(bytes_per_call, launch_s, None,
                                "ray_relu4_kernel" if vec4 else "ray_relu_kernel", copy_gbps,
                                read_gbps)
    line["warm"] = {"launch_us_mean": round(t_warm / args.steps * 1e6, 3)}
    line["gpu"] = torch.cuda.get_device_name(dev)
    return line


# ---------------------------------------------------------------------------
# convex upsample
# ---------------------------------------------------------------------------

def upsample_kernel_name(C: int, H: int, W: int, s: int, mask_ptr: int) -> str:
    """The kernel bvml_dsine_convex_upsample_f32 runs: at s = 8 the LDS-staged
    one when H*W is a multiple of 4 and the mask 16-byte aligned (the outputs
    here are fresh allocations, 16-byte aligned), else the register one."""
    if s != 8:
        return f"upsample_kernel<{C}>"
    if (H * W) % 4 == 0 and mask_ptr % 16 == 0:
        return f"upsample8_lds_kernel<{C}>"
    return f"upsample8_kernel<{C}>"


def bench_upsample(args, dev) -> dict:
    import torch
    import oracle
    from brovisionml_amd import _lib, workloads as wl

    w = wl.UPSAMPLE_WORKLOADS[args.workload]
    B, C, H, W, s = w.B, w.C, w.H, w.W, w.s
    bytes_per_call = w.algorithmic_bytes()
    nsets = args.sets or nsets_for(bytes_per_call)
    flags = _lib.FP64 if args.precise else _lib.DEFAULT
    eps = float(np.float32(1e-12))

    xs, ms, bufs = [], [], []
    x0 = mask0 = None
    for d in range(nsets + 1):
        x, mask = wl.make_upsample_inputs(w, d if d < nsets else 0)
        if d == 0:
            x0, mask0 = x, mask
        flat = torch.from_numpy(np.concatenate([x.ravel(), mask.ravel()])).to(dev)
        xs.append(flat[:x.size])
        ms.append(flat[x.size:])
        bufs.append(flat)
    outs = [torch.empty((B, C, s * H, s * W), dtype=torch.float32, device=dev)
            for _ in range(nsets + 1)]

    def launch(i: int) -> None:
        sptr = torch.cuda.current_stream(dev).cuda_stream
        st = _lib.convex_upsample_f32(xs[i].data_ptr(), ms[i].data_ptr(), B, C, H, W, s, True,
                                      eps, outs[i].data_ptr(), flags, sptr)
        if st != 0:
            raise RuntimeError(f"convex_upsample_f32 failed: {st} {_lib.last_error()}")

    tm = Timer(dev, launch, nsets, args.steps, args.warmup, bytes_per_call, warm_index=nsets)
    t_cold = tm.cold()
    t_eager, per = tm.eager()
    t_warm = tm.warm()
    copy_gbps = tm.copy_ceiling_gbps()
    read_gbps = tm.read_ceiling_gbps(bufs[:nsets])
    if args.calib:
        tm.calib()

    launch_s = t_cold / args.steps
    opx = B * s * s * H * W * args.steps  # output pixels
    per = np.array(per)
    line = base_line(
        args, "output Mpixel/s (+ achieved HBM GB/s, % of peak), DSINE convex upsample x8 + "
              "L2 normalise, 256x256 -> 2048x2048 fp32",
        opx / t_cold / 1e6, "Mpixel/s", t_cold * 1e3 / args.steps,
        {
            "workload": w.name, "B": B, "C": C, "H": H, "W": W, "scale": s,
            "mask": f"logits ~ N(0, {w.mask_sigma}^2)", "x": "unit normals, independent per pixel",
            "kernel_mode": "fp64" if args.precise else "fast",
            "inputs": f"{nsets} independent seeded draws, rotating "
                      f"({nsets * bytes_per_call / 1e6:.0f} MB > 256 MB Infinity Cache); "
                      "timed replay after a 512 MB flush",
        })
    line["roofline"] = roofline(
        bytes_per_call, launch_s,
        None if args.precise else traffic_from_profile("upsample", w.name),
        upsample_kernel_name(C, H, W, s, ms[0].data_ptr()), copy_gbps, read_gbps)
    line["per_launch"] = {"us_median": round(float(np.median(per)), 3),
                          "us_max": round(float(per.max()), 3)}
    line["warm"] = {
        "value": round(opx / t_warm / 1e6, 2),
        "launch_us_mean": round(t_warm / args.steps * 1e6, 3),
        "achieved_gbps": round(bytes_per_call / (t_warm / args.steps) / 1e9, 1),
    }
    line["eager"] = {
        "value": round(opx / t_eager / 1e6, 2),
        "us_per_step": round(t_eager / args.steps * 1e6, 3),
        "note": "the same steps launched one by one from Python with per-launch events",
    }
    line["gpu"] = torch.cuda.get_device_name(dev)
    del xs, ms, bufs, outs, tm
    torch.cuda.empty_cache()

    if not args.no_cpu:
        def cpu_pass(nt):
            return lambda: oracle.convex_upsample(x0, mask0, H, W, s, normalize=True, eps=eps,
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


# ---------------------------------------------------------------------------
# refiner forward
# ---------------------------------------------------------------------------

def refiner_kernel_rooflines(dev, H: int, W: int, reps: int):
    """The refiner's 5x5 ConvGRU convolutions (the implicit-GEMM kernels of
    brovisionml_amd/csrc/conv.hip) as its forward runs them, each timed alone
    on the refiner's map size with HIP events on their stream, against the
    fp32 matrix peak: every iteration convz + convr and convq over the hidden
    state's 64 channels (cin 64; the gates and the update in their
    epilogues, with the part over the other 66 channels added), and once per
    forward those parts over [feature | uv] (cin 66, plain convolutions).
    Algorithmic flops per launch = 2 * cout * cin * 25 * H * W.  Returns (the
    per-iteration convz + convr kernel's roofline, every kernel's figures)."""
    import torch
    from brovisionml_amd import _lib
    lib = _lib.load()
    C, ch, cx = 64, 64, 66
    g = torch.Generator().manual_seed(0)
    x = torch.randn(ch + cx, H, W, generator=g).to(dev)
    h = x[:C]
    xf = x[ch:]
    w = (torch.rand(3 * C, ch + cx, 5, 5, generator=g) - 0.5) / math.sqrt((ch + cx) * 25)
    wzr_h = torch.from_numpy(_lib.conv_pack_f32(w[:2 * C, :ch].numpy(), interleave=True)).to(dev)
    wzr_f = torch.from_numpy(_lib.conv_pack_f32(w[:2 * C, ch:].numpy(), interleave=True)).to(dev)
    wq_h = torch.from_numpy(_lib.conv_pack_f32(w[2 * C:, :ch].numpy())).to(dev)
    wq_f = torch.from_numpy(_lib.conv_pack_f32(w[2 * C:, ch:].numpy())).to(dev)
    b = torch.zeros(C, device=dev)
    z, rh, hn, hc = (torch.empty(C, H, W, device=dev) for _ in range(4))
    s_zr = torch.empty(2 * C, H, W, device=dev)
    s_q = torch.empty(C, H, W, device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    calls = {
        "conv_gru_gates (convz + convr over h, 5x5, 64 -> 128, + the [feature, uv] part)": (
            2 * 2 * C * ch * 25 * H * W,
            lambda: lib.bvml_dsine_conv_gru_gates_sum_f32(
                x.data_ptr(), ch, H, W, wzr_h.data_ptr(), C, s_zr.data_ptr(), b.data_ptr(),
                b.data_ptr(), h.data_ptr(), z.data_ptr(), rh.data_ptr(), sp)),
        "conv_gru_update (convq over r*h, 5x5, 64 -> 64, + the [feature, uv] part)": (
            2 * C * ch * 25 * H * W,
            lambda: lib.bvml_dsine_conv_gru_update_sum_f32(
                rh.data_ptr(), ch, H, W, wq_h.data_ptr(), C, s_q.data_ptr(), b.data_ptr(),
                z.data_ptr(), h.data_ptr(), hn.data_ptr(), hc.data_ptr(), sp)),
        "conv (convz + convr over [feature, uv], 5x5, 66 -> 128, once per forward)": (
            2 * 2 * C * cx * 25 * H * W,
            lambda: lib.bvml_dsine_conv_f32(xf.data_ptr(), cx, H, W, wzr_f.data_ptr(), 2 * C, 5,
                                            s_zr.data_ptr(), sp)),
        "conv (convq over [feature, uv], 5x5, 66 -> 64, once per forward)": (
            2 * C * cx * 25 * H * W,
            lambda: lib.bvml_dsine_conv_f32(xf.data_ptr(), cx, H, W, wq_f.data_ptr(), C, 5,
                                            s_q.data_ptr(), sp)),
    }
    # the [feature, uv] parts first, so that the fused kernels start from the
    # sums a forward gives them (an unwritten map's contents would reach their
    # activations instead)
    parts = [c for n, (_, c) in calls.items() if n.startswith("conv (")]
    for call in parts:
        call()
    out = {}
    for name, (flops, call) in calls.items():
        # each kernel back to back for RAMP_SECONDS first: the clocks drop
        # while the host packs the weights, and the first kernel timed would
        # otherwise run on the ramp (convz + convr 248 against 233 us)
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < RAMP_SECONDS:
            for _ in range(10):
                call()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / reps
        tf = flops / t / 1e12
        out[name] = {"us": round(t * 1e6, 1), "tflops": round(tf, 1),
                     "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4), "flops": flops}
    first = next(iter(out))
    r = out[first]
    roof = {"bound": "mfma", "achieved": r["tflops"], "peak": FP32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": r["frac"], "traffic": None, "kernel": first,
            "flops_per_launch": r["flops"], "launch_us_mean": r["us"]}
    return roof, out


def bench_refiner(args, dev) -> dict:
    """The whole NRN refiner forward at a 256x256 grid (a 2048x2048 image),
    synthetic weights and decoder outputs, one forward per step, `steps`
    forwards captured in one graph: the native refiner
    (libbvml_dsine_refine.so: the loop in C++, every convolution on the
    package's fp32 matrix-core kernels, the propagate with fused activations
    and the upsample + normalise; the line's value) and the Python driver
    (brovisionml_amd/refiner.py: torch's im2col + GEMM convolutions, the
    package's other kernels, with the up-mask head and upsample in every
    iteration) beside it.  The CPU leg is
    the restatement in oracle/refiner.py (float64 convolutions, the C
    oracle's ops) on a 24x32 grid."""
    import torch
    from brovisionml_amd import refiner as rf, workloads as wl

    H = W = 256 if args.workload is None or args.workload == 0 else 64
    rng = np.random.default_rng(0)
    normal = rng.standard_normal((1, 3, H, W))
    normal[:, 2] = np.abs(normal[:, 2]) + 0.5
    normal = (normal / np.linalg.norm(normal, axis=1, keepdims=True)).astype(np.float32)
    feature = rng.standard_normal((1, 64, H, W)).astype(np.float32)
    hidden = rng.uniform(-1, 1, (1, 64, H, W)).astype(np.float32)
    weights = rf.random_weights(0)
    dec = rf.DecoderOutput(*(torch.from_numpy(a).to(dev) for a in (normal, feature, hidden)))
    intr = wl.intrins_from_fov(8 * H, 8 * W, 60.0)
    stream = torch.cuda.current_stream(dev)

    def graph_time(step) -> float:
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(args.steps):
                step()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3

    t = t_py = None
    if args.driver in ("native", "both"):
        native = rf.NativeRefiner(weights)
        out = torch.empty((1, 3, 8 * H, 8 * W), dtype=torch.float32, device=dev)
        t = graph_time(lambda: native.forward(dec, intr, 8 * H, 8 * W, out=out))
    if args.driver in ("python", "both"):
        model = rf.Refiner(weights, dev)
        cond = model.conditioning(intr, H, W, 8 * H, 8 * W)
        t_py = graph_time(lambda: model.forward(dec, intr, 8 * H, 8 * W, cond=cond))
    opx = 64 * H * W * args.steps
    driver = "native refiner (C++, libbvml_dsine_refine.so)"
    if t is None:
        t, t_py, driver = t_py, None, "Python driver (brovisionml_amd/refiner.py)"
    line = base_line(args, f"output Mpixel/s, DSINE NRN refiner forward (5 iterations), {H}x{W} "
                           f"grid -> {8 * H}x{8 * W} fp32", opx / t / 1e6, "Mpixel/s",
                     t * 1e3 / args.steps,
                     {"workload": f"dsine-refiner-{H}x{W}", "H": H, "W": W, "iterations": 5,
                      "weights": "synthetic (uniform +-1/sqrt(fan_in))",
                      "driver": driver,
                      "convolutions": "5x5 and 3x3: implicit-GEMM fp32 MFMA kernels; the "
                                      "ConvGRU's parts over [feature, uv] once per forward"})
    if t_py is not None:
        line["python_driver"] = {"ms_per_step": round(t_py * 1e3 / args.steps, 4),
                                 "value": round(opx / t_py / 1e6, 2)}
    line["roofline"], line["kernels"] = refiner_kernel_rooflines(dev, H, W, args.steps)
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
    ap.add_argument("--op", choices=("angmf", "upsample", "refiner", "ray_relu"), default="angmf")
    ap.add_argument("--driver", choices=("native", "python", "both"), default="both",
                    help="--op refiner: the native refiner, the Python driver, or both (the "
                         "native one is the line's value)")
    ap.add_argument("--workload", type=int, default=None,
                    help="index into the op's workloads (default: angmf and ray_relu 2, "
                         "upsample 0)")
    ap.add_argument("--sets", type=int, default=0,
                    help="rotating input sets (0 = auto: > 512 MB, at most 256)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--ramp-seconds", type=float, default=RAMP_SECONDS,
                    help="back-to-back work before each timed region to bring the clocks up "
                         "(a counter pass may shorten it: the counters serialise the launches)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", dest="configs", action="store_false",
                    help="angmf: skip the other workloads' sub-object")
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
    Timer.ramp_seconds = args.ramp_seconds
    if args.workload is None and args.op != "refiner":
        args.workload = 2 if args.op in ("angmf", "ray_relu") else 0

    if args.gpus != 1:
        print(f"bench.py: measures one GPU only (--gpus {args.gpus} requested); "
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
    line = {"angmf": bench_angmf, "upsample": bench_upsample, "refiner": bench_refiner,
            "ray_relu": bench_ray_relu}[args.op](args, dev)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
