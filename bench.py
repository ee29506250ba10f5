#!/usr/bin/env python3
"""Benchmark: bf16 GEMV achieved HBM GB/s (% of peak) + us/call at 4096x14336, 1 GPU.

Workload (one "step"): the two Llama-3-8B FFN decode GEMVs of config C2 in the
row-dot layout -- up/gate W [14336,4096] @ x[4096] and down W [4096,14336] @
x[14336] -- bf16 weights ~N(0,0.02), f32 activations ~N(0,1), seed 0, weights
and activations resident in HBM before the timed region starts.  Cold cache:
each weight has COPIES (6) distinct device copies and consecutive steps
rotate through them, so 11 other weights (1.29 GB, 1.2 GiB) stream between
two reads of the same bytes (MI355X's Infinity Cache is 256 MB).

value         whole-job throughput: algorithmic bytes (2NK + 4K + 4N per GEMV)
              of the K timed steps over their host wall time, synchronized on
              both sides.  The K steps (2K launches on resident inputs) are
              captured once into a HIP graph on the library stream and the
              timed region is one replay of it, timed --repeats times (3),
              each bracketed by a synchronize: `value` takes the median
              (`timing` lists every repeat).  The per-shape batches below
              run first, so the timed region starts on a device that has been
              streaming, as a decode loop's steps do.  `eager` times the same
              K steps launched one Python call at a time.
roofline      algorithmic bytes per launch / average launch duration of the
              row-dot streaming kernels: HIP events on the library stream
              around a replay of the same K steps, queued behind an untimed
              replay so the events hold device time only (kernel durations
              and the gaps between them, as rocprof's kernel trace sees them).
              Each duration includes the fixed cost of a dispatch, which
              `dispatch_floor_us` measures alone with empty launches.  Peak:
              MI355X's 8 TB/s HBM3E.  `us_per_launch` times each shape in its
              own back-to-back batch, the same way.
read_ceiling  the same weights streamed by a read-only probe with the same
              128-bit nontemporal loads, timed the same way.
dropin        the reference's own operator surface, dmc_matmul_bf16_gpu(_t),
              with host x and y (PCIe and the synchronous round trip
              included): microseconds per call on C2 up/gate.  Never `value`.
cpu_baseline  the oracle's restatement of the reference CPU kernel
              dmc_matmul_bf16 (same fmaf chain and threading policy) on this
              host, on a bounded sample of the same workload.

    python bench.py [--gpus 1] [--steps 200] [--warmup 10] [--extended]
"""
from __future__ import annotations

import argparse
import ctypes
import gc
import json
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_GBS = 8000.0
METRIC = "bf16 GEMV achieved HBM GB/s (% of peak) + µs/call at 4096×14336, 1 GPU"
TRAFFIC_PROFILE = ROOT / "profiles" / "gemv_rd_stream_c2_traffic.md"


def b_alg(n: int, k: int, m: int = 1) -> int:
    """Algorithmic bytes per call: bf16 W + f32 x + f32 y."""
    return 2 * n * k + 4 * k * m + 4 * n * m


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def traffic_from_profile():
    """HBM bytes per launch of the C2 row-dot GEMVs measured by rocprofv3 --pmc
    (FETCH_SIZE + WRITE_SIZE, calibrated on a copy kernel of known size),
    averaged over the two shapes like `achieved`; read from the committed
    summary (a line `traffic_bytes_per_launch: N`), None when absent."""
    if not TRAFFIC_PROFILE.exists():
        return None
    for line in TRAFFIC_PROFILE.read_text().splitlines():
        if line.strip().startswith("traffic_bytes_per_launch:"):
            try:
                return int(float(line.split(":", 1)[1].strip()))
            except ValueError:
                return None
    return None


def cpu_baseline(seconds: float) -> dict:
    """The reference CPU path restated (oracle, 'port' build: scalar fmaf like
    the reference's x86 build) on C2's up/gate GEMV in the reference kernel's
    own layout, x @ W with W [4096,14336] (pre-transposed so no transpose is
    timed)."""
    import oracle
    from demonic_amd import workloads as W

    w, x = W.dense(14336, 4096, seed=0)
    wt = np.ascontiguousarray(w.T)
    k, n = wt.shape
    threads = oracle.gemv_ways(k, n)
    oracle.matmul_bf16(x, wt)  # warm caches and pages
    calls, t0 = 0, time.perf_counter()
    while True:
        oracle.matmul_bf16(x, wt)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds or calls >= 5000:
            break
    per = el / calls
    gbs = b_alg(n, k) / per / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"C2 up/gate x@W, W[{k},{n}] bf16, m=1: {calls} calls in {el:.1f}s "
                      f"({per * 1e6:.0f} us/call); oracle restatement of dmc_matmul_bf16 "
                      f"(jit.rs:29488): scalar libm fmaf chain, {threads} threads by the reference's "
                      f"column-split policy (jit.rs:29527-29529); host nproc={os.cpu_count()}"}


class Rotating:
    """COPIES device copies of one weight, plus its x and y regions."""

    def __init__(self, d, w: np.ndarray, x: np.ndarray, copies: int, n_out: int | None = None):
        self.d = d
        self.shape = w.shape
        first = d.DeviceBuffer.from_numpy(w)
        self.w = [first]
        for _ in range(copies - 1):
            c = d.DeviceBuffer(w.nbytes)
            c.copy_from(first)
            self.w.append(c)
        self.x = d.DeviceBuffer.from_numpy(x)
        rows = x.shape[0] if x.ndim == 2 else 1
        self.y = d.DeviceBuffer(4 * rows * (w.shape[0] if n_out is None else n_out))
        self.m = rows

    def free(self):
        for b in self.w + [self.x, self.y]:
            b.free()


# --no-graph: every batch launched one host call at a time (profiled runs:
# under rocprofv3 the replay of a captured graph has aborted or crashed the
# process on these boxes, while the same replays run cleanly without it)
GRAPHS = True


def batch_us(d, fn, reps: int, graph: bool = True) -> float:
    """Average device time of `reps` back-to-back launches of fn(0), fn(1), ...:
    HIP events on the library stream around the batch, kernel durations plus
    the gaps between them.  graph=True: the batch is captured once into a HIP
    graph (after one untimed call that lets the library size its buffers),
    and the timed replay is queued behind an untimed one, so the device goes
    from one to the other without waiting for the host to submit (the events
    then hold device time only, like rocprof's kernel trace); graph=False: one
    host call per launch, submission included."""
    fn(0)
    d.synchronize()
    g = None
    if graph and GRAPHS:
        with d.Graph() as g:
            for i in range(reps):
                fn(i)
        g.launch()
    e0, e1 = d.Event(), d.Event()
    d.synchronize()
    if g is not None:
        g.launch()  # untimed: keeps the device busy while the timed replay is submitted
        e0.record()
        g.launch()
    else:
        e0.record()
        for i in range(reps):
            fn(i)
    e1.record()
    e1.synchronize()
    if g is not None:
        g.destroy()
    return e0.elapsed_ms(e1) * 1e3 / reps


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--repeats", type=int, default=3,
                    help="time the K steps this many times (each bracketed by a synchronize) and report "
                         "the median")
    ap.add_argument("--copies", type=int, default=6, help="distinct device copies per weight")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--extended", action="store_true",
                    help="also time C1, C3, C4, C5 and the column-stream layout (stderr + 'extended')")
    ap.add_argument("--c3", action="store_true", help="also time C3, the 32-layer decode sweep")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch every batch one host call at a time, HIP graphs left out entirely "
                         "(for profiled runs; the timed C2 steps then run eagerly too)")
    ap.add_argument("--steps-only", action="store_true",
                    help="run the warm-up and the timed steps alone: no per-shape batches, read probe, "
                         "dispatch floor or drop-in calls (for the kernel-trace profile, whose per-kernel "
                         "averages are then the timed steps' own)")
    ap.add_argument("--no-c3", action="store_true",
                    help="leave C3 out of --extended (its HIP-graph replays are not traced: under rocprofv3 "
                         "one aborted the queue with a malformed-packet error)")
    ap.add_argument("--crossover", action="store_true",
                    help="only time the drop-in against the CPU kernel for k*n = 2^10 .. 2^24 (m = 1), "
                         "the measurement behind DMC_HIP_MIN_MACS")
    ap.add_argument("--skinny", action="store_true",
                    help="only C2's shapes at skinny and prefill M, each launch one host call (no HIP "
                         "graph): the workload of the counter profiles of the MFMA kernels")
    ap.add_argument("--f32", action="store_true",
                    help="only the f32-weight `W @ x` lines (row-dot f32 kernel and drop-in) at C2's shapes")
    a = ap.parse_args(argv)
    global GRAPHS
    GRAPHS = not a.no_graph

    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the GEMV shards by weight rows "
              "with no reduction, so N GPUs would each run this kernel on N-th of the rows); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import demonic_amd as d
    from demonic_amd import workloads as W

    if not d.available():
        print("bench.py: no usable gfx950 device: " + d._lib.load().dmc_hip_last_error().decode(),
              file=sys.stderr)
        return 1
    log(f"device {d.device_info()}")
    if a.crossover:
        print(json.dumps(crossover(d)), flush=True)
        return 0
    if a.skinny:
        print(json.dumps(skinny(d, W, a.steps)), flush=True)
        return 0
    if a.f32:
        print(json.dumps(f32_weights(d, a.steps)), flush=True)
        return 0

    t = time.perf_counter()
    c2 = W.c2()
    shapes = {name: Rotating(d, w, x, a.copies) for name, (w, x) in c2.items()}
    d.synchronize()
    log(f"C2 inputs resident in {time.perf_counter() - t:.1f}s")
    order = ["up", "down"]

    def launch(name, i):
        s = shapes[name]
        n, k = s.shape
        d.gemv_rd(s.x, s.w[i % len(s.w)], s.y, 1, k, n)

    for i in range(a.warmup):
        for name in order:
            launch(name, i)
    d.synchronize()

    def steps():
        for i in range(a.steps):
            for name in order:
                launch(name, i)

    def timed(run):
        """Host wall time of run(), bracketed by a synchronize on both sides."""
        d.synchronize()
        t0 = time.perf_counter()
        run()
        d.synchronize()
        return time.perf_counter() - t0

    repeats = max(1, a.repeats)

    def timed_median(run):
        """The median of `repeats` timings of run() (each bracketed by a
        synchronize), and all of them: a single timing of a short region
        varies by a few per cent from one to the next."""
        walls = [timed(run) for _ in range(repeats)]
        return sorted(walls)[len(walls) // 2], walls

    # per-shape launch durations, the read ceiling and the dispatch floor
    # (measured first: the timed region below then starts on a device that
    # has been streaming for a while, as a decode loop's steps do; each
    # shape's batch runs twice and the second is kept, so the first shape is
    # not the one that meets an idle device)
    # (at least 200 launches per batch: a graph replay has a fixed cost of
    # its own, ~7-30 us on these boxes, that a short batch would charge to
    # its kernels)
    reps = max(a.steps, 200)
    us, read_us, floor_us = {}, None, None
    if not a.steps_only:
        for nm in order:
            batch_us(d, lambda i, nm=nm: launch(nm, i), reps)
            us[nm] = batch_us(d, lambda i, nm=nm: launch(nm, i), reps)
        read_us = {nm: batch_us(d, lambda i, nm=nm: d.probe_read(shapes[nm].w[i % a.copies]), reps)
                   for nm in order}
        floor_us = batch_us(d, lambda i: d.probe_read(None, 0), reps)

    # timed region: K steps, each the two GEMVs, inputs resident, replayed
    # from a HIP graph captured once (after one untimed replay); with
    # --no-graph launched one call at a time
    replays = max(1, -(-400 // (2 * a.steps)))
    bytes_step = sum(b_alg(*shapes[nm].shape) for nm in order)
    e0, e1 = d.Event(), d.Event()
    if GRAPHS:
        with d.Graph() as graph:
            steps()
        graph.launch()
        d.synchronize()
        wall, walls = timed_median(graph.launch)
        # device time of the same K steps (HIP events; see batch_us), repeated
        # in one graph until it holds >= 400 launches: each graph replay
        # carries a fixed cost of its own (~20-30 us on these boxes), which
        # 40 launches (--steps 20) would otherwise charge to their kernels
        if replays > 1:
            graph.destroy()
            with d.Graph() as graph:
                for _ in range(replays):
                    steps()
            graph.launch()
        graph.launch()
        e0.record()
        graph.launch()
        e1.record()
        e1.synchronize()
        graph.destroy()
    else:
        steps()
        d.synchronize()
        wall, walls = timed_median(steps)
        e0.record()
        for _ in range(replays):
            steps()
        e1.record()
        e1.synchronize()
    value = bytes_step * a.steps / wall / 1e9
    ev_ms = e0.elapsed_ms(e1) / replays
    # the same K steps launched one call at a time (garbage collector paused)
    gc.disable()
    try:
        eager_wall, _ = timed_median(steps)
    finally:
        gc.enable()
    for nm in order:
        y = shapes[nm].y.download(np.float32, (shapes[nm].shape[0],))
        assert np.all(np.isfinite(y)), nm  # full parity lives in tests/

    b_up, b_down = (b_alg(*shapes[nm].shape) for nm in order)
    launch_us = ev_ms * 1e3 / (a.steps * len(order))
    achieved = (b_up + b_down) / 2 / (launch_us * 1e-6) / 1e9
    w_bytes = {nm: 2 * shapes[nm].shape[0] * shapes[nm].shape[1] for nm in order}
    read_gbs = sum(w_bytes.values()) / (sum(read_us.values()) * 1e-6) / 1e9 if read_us else None
    plans = {nm: d.plan("rd", 1, shapes[nm].shape[1], shapes[nm].shape[0],
                        x_addr=shapes[nm].x.addr, w_addr=shapes[nm].w[0].addr) for nm in order}
    roofline = {
        "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic_from_profile(),
        "kernel": "row-dot streaming GEMVs: gemv_rd_stream_kernel (up/gate), "
                  "gemv_rd_stream_x14_kernel (down, 14 waves splitting k, one workgroup per CU)",
        "bytes_per_launch": {"up": b_up, "down": b_down},
        "avg_launch_us": round(launch_us, 3),
        "us_per_launch": {nm: round(u, 3) for nm, u in us.items()},
        "frac_of_read_ceiling": round(achieved / read_gbs, 4) if read_gbs else None,
    }
    for b in shapes.values():
        b.free()

    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(wall / a.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16w-f32acc",
        "submission": ("one HIP graph replay of the K timed steps (2K kernel launches)" if GRAPHS
                       else "the K timed steps launched one call at a time (--no-graph)"),
        "timing": {"repeats": repeats, "statistic": "median of the repeats, each bracketed by a synchronize",
                   "ms_per_repeat": [round(w * 1e3, 4) for w in walls]},
        "eager": {"value": round(bytes_step * a.steps / eager_wall / 1e9, 1),
                  "note": "the same K steps launched one Python call at a time, host wall time"},
        "data": "synthetic: seeded N(0,0.02) bf16 weights, N(0,1) f32 activations (PCG64 seed 0)",
        "config": {"workload": "C2 Llama-3-8B FFN decode GEMVs, row-dot layout: up/gate W[14336,4096] "
                               "and down W[4096,14336], m=1, weights resident, cold cache "
                               f"({a.copies} rotating copies each)",
                   "us_per_call": {nm: round(u, 3) for nm, u in us.items()},
                   "frac_of_peak_value": round(value / PEAK_GBS, 4),
                   "event_ms_per_step": round(ev_ms / a.steps, 4),
                   "event_replays": replays,
                   "plans": {nm: {"waves": p.waves, "kvec": p.slices, "rows_per_group": p.rows_per_group,
                                  "rows_per_step": p.rows_or_rw, "groups": p.grid_x}
                             for nm, p in plans.items()}},
        "roofline": roofline,
        "read_ceiling": None if read_us is None else {
            "GB/s": round(read_gbs, 1), "us": {nm: round(u, 3) for nm, u in read_us.items()},
            "frac_of_peak": round(read_gbs / PEAK_GBS, 4)},
        "dispatch_floor_us": None if floor_us is None else round(floor_us, 3),
        "dropin": None if a.steps_only else dropin(d, W, 300),
        "cpu_baseline": None if a.no_cpu else cpu_baseline(a.cpu_seconds),
    }
    if a.extended:
        result["extended"] = extended(d, W, a.steps)
    if ((a.extended and not a.no_c3) or a.c3) and not GRAPHS:
        log("C3 left out: its decode step is a captured graph (--no-graph)")
    elif (a.extended and not a.no_c3) or a.c3:
        result["c3"] = c3(d, W)
    print(json.dumps(result), flush=True)
    return 0


def extended(d, W, reps: int) -> dict:
    """Secondary configurations (stderr + the JSON 'extended' field)."""
    out = {}

    def record(label, us, n, k, m=1):
        gbs = b_alg(n, k, m) / (us * 1e-6) / 1e9
        out[label] = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
        log(f"{label}: {us:.2f} us  {gbs:.0f} GB/s  {gbs / PEAK_GBS:.1%}")

    c2 = W.c2()
    cases = [("C1 rd [4096,4096]", W.c1(), "rd"),
             ("C2 cs up x@W W[4096,14336]", c2["up"], "cs"),
             ("C2 cs down x@W W[14336,4096]", c2["down"], "cs")]
    for label, (w, x), layout in cases:
        n, k = w.shape
        wl = w if layout == "rd" else np.ascontiguousarray(w.T)
        copies = max(2, min(12, int(1.2e9 // wl.nbytes) + 1))
        s = Rotating(d, wl, x, copies, n_out=n)
        if layout == "rd":
            f = lambda i: d.gemv_rd(s.x, s.w[i % copies], s.y, 1, k, n)  # noqa: E731
        else:
            f = lambda i: d.gemv_cs(s.x, s.w[i % copies], s.y, 1, k, n)  # noqa: E731
        for i in range(3):
            f(i)
        record(label, batch_us(d, f, reps), n, k)
        s.free()
    out.update(f32_weights(d, reps))
    # C4 LM head, skinny M: one resident copy (1.05 GB exceeds the 256 MB cache)
    t = time.perf_counter()
    w, _ = W.dense(W.LM_HEAD[0], W.LM_HEAD[1], seed=0, m=1)
    log(f"C4 weight generated in {time.perf_counter() - t:.1f}s")
    n, k = w.shape
    dw = d.DeviceBuffer.from_numpy(w)
    for m in (1, 2, 4, 8, 16):
        x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
        dx = d.DeviceBuffer.from_numpy(x)
        dy = d.DeviceBuffer(4 * n * m)
        f = lambda i: d.gemv_rd(dx, dw, dy, m, k, n)  # noqa: E731
        f(0)
        record(f"C4 rd m={m}", batch_us(d, f, 60), n, k, m)
        dx.free()
        dy.free()
    dw.free()
    # C5 edge shapes, both layouts (timed, not gated)
    for (n, k) in W.C5_SHAPES:
        w, x, _ = W.c5(n, k)
        for layout in ("rd", "cs"):
            wl = w if layout == "rd" else np.ascontiguousarray(w.T)
            s = Rotating(d, wl, x, 3, n_out=n)
            if layout == "rd":
                f = lambda i: d.gemv_rd(s.x, s.w[i % 3], s.y, 1, k, n)  # noqa: E731
            else:
                f = lambda i: d.gemv_cs(s.x, s.w[i % 3], s.y, 1, k, n)  # noqa: E731
            f(0)
            record(f"C5 {layout} W[{n},{k}]", batch_us(d, f, reps), n, k)
            s.free()
    # Batched per-head projections, one launch over every head: the
    # reference's [B,1,S,K] @ [H,K,N] collapse (jit.rs:19914-19933) on device
    # regions, W [H,K,N] bf16.  q heads with one broadcast x (ls = 0), k/v
    # heads, and per-head inputs (ls = K); enough rotating copies that the
    # weights exceed the 256 MB cache.
    rng = np.random.default_rng(7)
    for label, heads, k, n, ls in (("batched q heads [32,4096,128]", 32, 4096, 128, 0),
                                   ("batched kv heads [8,4096,128]", 8, 4096, 128, 0),
                                   ("batched per-head x [32,128,4096]", 32, 128, 4096, 128)):
        wb = W_bf16(rng, heads * k, n)
        xb = rng.standard_normal(heads * k if ls else k).astype(np.float32)
        copies = max(3, -(-300_000_000 // wb.nbytes))
        s = Rotating(d, wb, xb, copies, n_out=heads * n)
        f = lambda i: d.gemv_cs(s.x, s.w[i % copies], s.y, 1, k, n, heads, ls, k * n)  # noqa: E731
        f(0)
        us = batch_us(d, f, reps)
        gbs = (wb.nbytes + xb.nbytes + 4 * heads * n) / (us * 1e-6) / 1e9
        out[label] = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
        log(f"{label}: {us:.2f} us  {gbs:.0f} GB/s  {gbs / PEAK_GBS:.1%}")
        s.free()
        if ls == 0:
            # The same projections through the drop-in's batched entry with
            # host x and y, in the deferred protocol (eight calls, one
            # flush): one broadcast x over consecutive heads runs as one
            # row-dot GEMV over the heads' stacked resident transposes.
            # Distinct weights rotate so that every call reads cold bytes.
            lib = d._lib.load()
            nw = copies
            hw = [W_bf16(rng, heads * k, n) for _ in range(nw)]
            ys = [np.empty(heads * n, np.float32) for _ in range(8)]
            dfr, flush = lib.dmc_matmul_bf16_gpu_batched_deferred, lib.dmc_matmul_bf16_gpu_flush
            groups = max(1, reps // 8)
            for g in range(-(-nw // 8) + groups):  # every weight's upload untimed
                if g == -(-nw // 8):
                    t0 = time.perf_counter()
                for j in range(8):
                    dfr(xb.ctypes.data, hw[(8 * g + j) % nw].ctypes.data, ys[j].ctypes.data, 1, k, n, heads, 0,
                        k * n)
                flush()
            us = (time.perf_counter() - t0) / (8 * groups) * 1e6
            gbs = (wb.nbytes + xb.nbytes + 4 * heads * n) / (us * 1e-6) / 1e9
            dl = f"drop-in {label} deferred x8 + flush"
            out[dl] = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
            log(f"{dl}: {us:.2f} us/call  {gbs:.0f} GB/s  {gbs / PEAK_GBS:.1%} (PCIe-inclusive)")
            del hw
    # One GPU's share of C2 under 8-way tensor parallelism (rows of gate/up,
    # k of down split eight ways): W[1792,4096] and W[4096,1792], 14.7 MB
    # each, 20 rotating copies (294 MB between reuses, above the 256 MB
    # cache).  Against the time 8 TB/s would take (`ideal_us`) and an empty
    # launch (`floor_us`): at this size a launch is mostly dispatch.
    floor_us = batch_us(d, lambda i: d.probe_read(None, 0), 200)
    rng = np.random.default_rng(8)
    for label, n, k in (("TP8 gate/up rd W[1792,4096]", 1792, 4096), ("TP8 down rd W[4096,1792]", 4096, 1792)):
        w = W_bf16(rng, n, k)
        x = rng.standard_normal(k).astype(np.float32)
        s = Rotating(d, w, x, 20, n_out=n)
        f = lambda i: d.gemv_rd(s.x, s.w[i % 20], s.y, 1, k, n)  # noqa: E731
        f(0)
        us = batch_us(d, f, 200)
        read_us = batch_us(d, lambda i: d.probe_read(s.w[i % 20]), 200)
        gbs = b_alg(n, k) / (us * 1e-6) / 1e9
        out[label] = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4),
                      "ideal_us": round(b_alg(n, k) / PEAK_GBS / 1e3, 3), "floor_us": round(floor_us, 3),
                      "read_probe_us": round(read_us, 3)}
        log(f"{label}: {us:.2f} us  {gbs:.0f} GB/s  {gbs / PEAK_GBS:.1%}  (ideal {out[label]['ideal_us']:.2f}, "
            f"empty launch {floor_us:.2f}, read probe {read_us:.2f})")
        s.free()
    # C2's shapes at a few activation rows (MFMA kernels)
    for name, (w, _) in (("up", c2["up"]), ("down", c2["down"])):
        n, k = w.shape
        for m in (2, 4, 8, 16):
            x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
            s = Rotating(d, w, x, 5, n_out=n)
            f = lambda i: d.gemv_rd(s.x, s.w[i % 5], s.y, m, k, n)  # noqa: E731
            f(0)
            record(f"C2 rd {name} m={m}", batch_us(d, f, reps), n, k, m)
            s.free()
    # prefill-sized M on C2's shapes (the gemm layout): TFLOP/s of x.W products
    for name, (w, _) in (("up", c2["up"]), ("down", c2["down"])):
        n, k = w.shape
        for m in (64, 512):
            x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
            s = Rotating(d, w, x, 3, n_out=n)
            f = lambda i: d.gemv_rd(s.x, s.w[i % 3], s.y, m, k, n)  # noqa: E731
            # 40 launches after as many untimed ones: the matrix cores reach
            # their steady rate only after a few milliseconds of this load
            us = batch_us(d, f, 40)
            tfs = 2.0 * m * n * k / (us * 1e-6) / 1e12
            out[f"C2 rd {name} prefill m={m}"] = {"us": round(us, 3), "TFLOP/s": round(tfs, 1),
                                                  "GB/s": round(b_alg(n, k, m) / (us * 1e-6) / 1e9, 1)}
            log(f"C2 rd {name} prefill m={m}: {us:.1f} us  {tfs:.1f} TFLOP/s")
            s.free()
    out.update(helpers(d, c2["up"][0]))
    out.update(ingress(d, c2["down"][0]))
    return out


def f32_weights(d, reps: int) -> dict:
    """The f32 path of `W @ x` (jit.rs:20806-20831) at C2's shapes with f32
    weights (235 MB each): the row-dot f32 kernel on device pointers (bytes
    4NK + 4K + 4N), and the drop-in dmc_matmul_f32_gpu with host x and y."""
    out = {}
    rng = np.random.default_rng(32)
    for n, k in ((14336, 4096), (4096, 14336)):
        w = np.float32(0.02) * rng.standard_normal((n, k), dtype=np.float32)
        x = rng.standard_normal(k, dtype=np.float32)
        copies = 6
        s = Rotating(d, w, x, copies, n_out=n)
        f = lambda i: d.gemv_f32_rd(s.x, s.w[i % copies], s.y, 1, k, n)  # noqa: E731
        for i in range(3):
            f(i)
        us = batch_us(d, f, reps)
        gbs = (4 * n * k + 4 * k + 4 * n) / (us * 1e-6) / 1e9
        label = f"f32 rd W@x W[{n},{k}]"
        out[label] = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
        log(f"{label}: {us:.2f} us  {gbs:.0f} GB/s  {gbs / PEAK_GBS:.1%}")
        s.free()
        d.matmul_f32_gpu(w, x)  # first touch: the weight becomes resident
        calls = 100
        t = time.perf_counter()
        for _ in range(calls):
            d.matmul_f32_gpu(w, x)
        us = (time.perf_counter() - t) / calls * 1e6
        label = f"f32 drop-in W@x W[{n},{k}] host x/y"
        out[label] = {"us": round(us, 3)}
        log(f"{label}: {us:.2f} us/call (PCIe-inclusive)")
    d.release_weights()
    out["f32 cpu W@x"] = f32_cpu_baseline(w, x)
    log(f"f32 cpu W@x: {out['f32 cpu W@x']['value']} GB/s ({out['f32 cpu W@x']['sample']})")
    return out


def f32_cpu_baseline(w: np.ndarray, x: np.ndarray, seconds: float = 2.0) -> dict:
    """The reference's f32 `W @ x` restated (oracle matmul_f32: the scalar_matmul
    chain, one thread as the reference runs it, jit.rs:20715-20802) on the
    first 512 rows of w, timed on this host."""
    import oracle

    ws = np.ascontiguousarray(w[:512])
    k = ws.shape[1]
    oracle.matmul_f32(ws, x)
    calls, t0 = 0, time.perf_counter()
    while True:
        oracle.matmul_f32(ws, x)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = el / calls
    return {"value": round((4 * 512 * k + 4 * k + 4 * 512) / per / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": "port", "sample": f"W[512,{k}] f32 @ x: {calls} calls in {el:.1f}s"}


def ingress(d, w) -> dict:
    """Weight ingress: dmc_hip_vault_load_npz reading a C2 weight from an .npz
    in the page cache into HBM (stored: parallel positioned reads; deflated:
    one zlib stream), against the reference's CPU loader restated (the oracle's
    dmc_vault_load_npz: the whole entry read into host memory, CRC checked,
    data copied out).  GB/s = array bytes / wall time of one call."""
    import tempfile

    from oracle import npz as onpz

    out = {}
    with tempfile.TemporaryDirectory(prefix="dmc_ingress_") as td:
        for label, save in (("stored", np.savez), ("deflated", np.savez_compressed)):
            path = pathlib.Path(td) / f"{label}.npz"
            save(path, w=w)
            path.read_bytes()  # page cache
            times = []
            for _ in range(3):
                t0 = time.perf_counter()
                buf = d.vault_load_npz(path, "w", w.size, 2, 0)
                times.append(time.perf_counter() - t0)
                buf.free()
            t0 = time.perf_counter()
            host = onpz.vault_load_npz(path, "w", w.size, 2, 0)
            cpu = time.perf_counter() - t0
            assert host is not None and len(host) == w.nbytes
            dev = min(times)
            rec = {"bytes": w.nbytes, "file_bytes": path.stat().st_size, "us": round(dev * 1e6, 1),
                   "GB/s": round(w.nbytes / dev / 1e9, 2), "cpu_loader_us": round(cpu * 1e6, 1),
                   "cpu_loader_GB/s": round(w.nbytes / cpu / 1e9, 2)}
            out[f"ingress npz {label} W{list(w.shape)}"] = rec
            log(f"ingress npz {label}: {rec['GB/s']} GB/s into HBM ({rec['us']:.0f} us), "
                f"CPU loader {rec['cpu_loader_GB/s']} GB/s")
    return out


def helpers(d, w) -> dict:
    """The device bf16 helpers on C2's up/gate weight (bytes = read + write,
    two source and two destination regions rotated)."""
    out = {}
    rows, cols = w.shape
    srcs = [d.DeviceBuffer.from_numpy(w) for _ in range(2)]
    dsts = [d.DeviceBuffer(w.nbytes) for _ in range(2)]
    wides = [d.DeviceBuffer(2 * w.nbytes) for _ in range(2)]
    cases = [("transpose_2d bf16 [14336,4096]", 2 * w.nbytes,
              lambda i: d.bf16_transpose_2d(srcs[i % 2], dsts[i % 2], rows, cols)),
             ("bf16_upconvert 58.7M", 6 * w.size, lambda i: d.bf16_upconvert(srcs[i % 2], wides[i % 2], w.size)),
             ("f32_to_bf16 58.7M", 6 * w.size, lambda i: d.f32_to_bf16(wides[i % 2], dsts[i % 2], w.size))]
    for label, nbytes, f in cases:
        for i in range(3):
            f(i)
        us = batch_us(d, f, 60)
        gbs = nbytes / (us * 1e-6) / 1e9
        out[label] = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
        log(f"{label}: {us:.2f} us  {gbs:.0f} GB/s  {gbs / PEAK_GBS:.1%}")
    for b in srcs + dsts + wides:
        b.free()
    return out


def dropin(d, W, reps: int) -> dict:
    """The drop-in entries with HOST x and y -- the PCIe-inclusive rate, never
    `value`.  C2 up/gate through dmc_matmul_bf16_gpu_t (x @ W', W [N,K]) and
    dmc_matmul_bf16_gpu (x @ W, W [K,N], the reference's layout).  Each call
    copies x in, launches, copies y out and synchronizes; weights are made
    resident by their first call (content key), and three distinct weights
    rotate so every call reads cold bytes.  Host wall time per call."""
    lib = d._lib.load()
    n, k = 14336, 4096
    out = {}
    mats = [W.dense(n, k, seed=100 + s, m=1)[0] for s in range(3)]
    x = np.random.default_rng(0).standard_normal(k).astype(np.float32)
    y = np.empty(n, np.float32)
    for label, entry, ws in (("drop-in rd x@W' host x/y", lib.dmc_matmul_bf16_gpu_t, mats),
                             ("drop-in cs x@W host x/y", lib.dmc_matmul_bf16_gpu,
                              [np.ascontiguousarray(w.T) for w in mats])):
        ptrs = [w.ctypes.data for w in ws]
        for p in ptrs:
            entry(x.ctypes.data, p, y.ctypes.data, 1, k, n)
        t0 = time.perf_counter()
        for i in range(reps):
            entry(x.ctypes.data, ptrs[i % 3], y.ctypes.data, 1, k, n)
        us = (time.perf_counter() - t0) / reps * 1e6
        gbs = b_alg(n, k) / (us * 1e-6) / 1e9
        out[label] = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
        log(f"{label}: {us:.2f} us/call  {gbs:.0f} GB/s  {gbs / PEAK_GBS:.1%} (PCIe-inclusive)")
        assert np.all(np.isfinite(y)), label
    # The reference's deferred protocol (gpu.rs:439-474), as its JIT issues
    # consecutive GEMVs: eight deferred x @ W calls, then one flush that waits
    # once and copies the eight y's out.  Host wall time per call.
    dfr, flush = lib.dmc_matmul_bf16_gpu_batched_deferred, lib.dmc_matmul_bf16_gpu_flush
    wts = [np.ascontiguousarray(w.T) for w in mats]
    ptrs = [w.ctypes.data for w in wts]
    ys = [np.empty(n, np.float32) for _ in range(8)]
    groups = max(1, reps // 8)
    for g in range(groups + 1):  # the first group untimed
        if g == 1:
            t0 = time.perf_counter()
        for j in range(8):
            dfr(x.ctypes.data, ptrs[(8 * g + j) % 3], ys[j].ctypes.data, 1, k, n, 1, 0, 0)
        flush()
    us = (time.perf_counter() - t0) / (8 * groups) * 1e6
    gbs = b_alg(n, k) / (us * 1e-6) / 1e9
    label = "drop-in cs x@W deferred x8 + flush"
    out[label] = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
    log(f"{label}: {us:.2f} us/call  {gbs:.0f} GB/s  {gbs / PEAK_GBS:.1%} (PCIe-inclusive)")
    assert all(np.all(np.isfinite(v)) for v in ys), label
    d.release_weights()
    return out


def skinny(d, W, reps: int) -> dict:
    """C2's shapes at m = 2 .. 16 (the streaming, 14-wave and skinny-M MFMA
    kernels) and 64 / 512 (prefill, the gemm layout), `reps` launches each,
    one host call per launch: no HIP graph, so counter collection sees
    ordinary dispatches."""
    out = {}
    c2 = W.c2()
    for name, (w, _) in (("up", c2["up"]), ("down", c2["down"])):
        n, k = w.shape
        for m in (2, 3, 4, 8, 12, 16, 64, 512):
            x = np.random.default_rng(m).standard_normal((m, k)).astype(np.float32)
            s = Rotating(d, w, x, 3, n_out=n)
            f = lambda i: d.gemv_rd(s.x, s.w[i % 3], s.y, m, k, n)  # noqa: E731
            f(0)
            us = batch_us(d, f, reps, graph=False)
            p = d.plan("rd", m, k, n, x_addr=s.x.addr, w_addr=s.w[0].addr)
            out[f"C2 rd {name} m={m}"] = {"us": round(us, 3), "GB/s": round(b_alg(n, k, m) / (us * 1e-6) / 1e9, 1),
                                          "TFLOP/s": round(2.0 * m * n * k / (us * 1e-6) / 1e12, 1),
                                          "layout": {-6: "wide", -7: "rows16", -8: "gemm"}.get(
                                              p.slices, "x14" if p.waves == 14 else
                                              "x8" if (p.waves, p.rows_or_rw, p.rows_per_group) == (8, 4, 16) else "stream")}
            log(f"C2 rd {name} m={m}: {us:.2f} us ({out[f'C2 rd {name} m={m}']['layout']})")
            s.free()
    return out


def crossover(d) -> dict:
    """Per-call time of the synchronous drop-in x @ W (dmc_matmul_bf16_gpu:
    host x and y, resident weight, content key, launch, wait) against the
    reference's CPU kernel restated (the oracle's dmc_matmul_bf16, its own
    thread policy) on this host, for m = 1 and k*n = 2^10 .. 2^24 (k = 2^ceil(e/2),
    n = 2^floor(e/2)).  The route threshold DMC_HIP_MIN_MACS is the smallest
    k*n from which the device wins at every larger size measured."""
    import oracle

    lib = d._lib.load()
    rows = []
    rng = np.random.default_rng(0)
    for e in range(10, 25):
        k, n = 1 << ((e + 1) // 2), 1 << (e // 2)
        w = W_bf16(rng, k, n)
        x = rng.standard_normal(k).astype(np.float32)
        y = np.empty(n, np.float32)
        lib.dmc_matmul_bf16_gpu(x.ctypes.data, w.ctypes.data, y.ctypes.data, 1, k, n)  # resident now

        def gpu():
            lib.dmc_matmul_bf16_gpu(x.ctypes.data, w.ctypes.data, y.ctypes.data, 1, k, n)

        def cpu():
            oracle.matmul_bf16(x, w)

        times = {}
        for name, fn in (("gpu_us", gpu), ("cpu_us", cpu)):
            fn()
            calls, t0 = 0, time.perf_counter()
            while True:
                fn()
                calls += 1
                el = time.perf_counter() - t0
                if (el >= 0.05 and calls >= 5) or calls >= 2000:
                    break
            times[name] = round(el / calls * 1e6, 2)
        rows.append({"k": k, "n": n, "kn": k * n, "cpu_threads": oracle.gemv_ways(k, n), **times})
        log(f"crossover k*n=2^{e} (k={k} n={n}): gpu {times['gpu_us']:.1f} us  cpu {times['cpu_us']:.1f} us")
    d.release_weights()
    wins = [r["gpu_us"] < r["cpu_us"] for r in rows]
    first = next((i for i in range(len(rows)) if all(wins[i:])), None)
    return {"crossover_kn": rows[first]["kn"] if first is not None else None, "rows": rows,
            "host_nproc": os.cpu_count()}


def W_bf16(rng, k: int, n: int) -> np.ndarray:
    """W [k, n] bf16 bits ~ N(0, 0.02) (the x @ W layout)."""
    from demonic_amd import workloads as W
    return W.bf16_rne(np.float32(0.02) * rng.standard_normal((k, n), dtype=np.float32))


def c3(d, W, tokens: int = 10) -> dict:
    """C3: one decode token = 32 layers x 7 row-dot GEMVs of Llama-3-8B
    (13.97 GB of bf16 weights, generated in HBM by the counter generator),
    each layer's activations drawn from the seed.  Scheduled as a decode step
    would be: q/k/v in one grouped launch, o, gate/up in one grouped launch,
    down -- 4 launches per layer -- and replayed from a HIP graph.  Also timed:
    the same token as 7 single launches per layer."""
    lib = d._lib.load()
    t = time.perf_counter()
    table = d.DeviceBuffer.from_numpy(W.normal_table(W.C3_SCALE))
    names = [nm for nm, _, _ in W.LLAMA3_8B_LAYER]
    shape = {nm: (n, k) for nm, n, k in W.LLAMA3_8B_LAYER}
    layers = []
    for layer in range(W.LLAMA3_8B_LAYERS):
        ws = {}
        for idx, nm in enumerate(names):
            n, k = shape[nm]
            ws[nm] = d.DeviceBuffer(2 * n * k)
            d.fill_counter_bf16(ws[nm], n * k, W.counter_seed(0, W.c3_tensor(layer, idx)), table)
        layers.append((ws, d.DeviceBuffer.from_numpy(W.c3_x(layer, 4096)),
                       d.DeviceBuffer.from_numpy(W.c3_x(layer, 14336))))
    ys = {nm: d.DeviceBuffer(4 * shape[nm][0]) for nm in names}
    d.synchronize()
    log(f"C3 weights generated in HBM in {time.perf_counter() - t:.1f}s")
    b_token = sum(b_alg(*shape[nm]) for nm in names) * W.LLAMA3_8B_LAYERS

    def arr(v):
        return (ctypes.c_int64 * len(v))(*v)

    grouped_calls, single_calls = [], []
    for ws, x, x2 in layers:
        def g(nms, xb):
            return (len(nms), arr([xb.addr] * len(nms)), arr([ws[nm].addr for nm in nms]),
                    arr([ys[nm].addr for nm in nms]), arr([shape[nm][0] for nm in nms]), 1, shape[nms[0]][1])
        grouped_calls += [g(["q", "k", "v"], x), g(["o"], x), g(["gate", "up"], x), g(["down"], x2)]
        for nm in names:
            xb = x2 if nm == "down" else x
            single_calls.append((xb.addr, ws[nm].addr, ys[nm].addr, 1, shape[nm][1], shape[nm][0]))

    def run_grouped():
        for c in grouped_calls:
            d._lib.check(lib.dmc_hip_gemv_rd_grouped(*c))

    def run_single():
        for c in single_calls:
            d._lib.check(lib.dmc_hip_gemv_rd(*c))

    out = {"tokens": tokens, "bytes_per_token": b_token}
    for label, fn, launches in (("grouped_4_per_layer", run_grouped, 4), ("single_7_per_layer", run_single, 7)):
        fn()
        d.synchronize()
        g = d.Graph()
        with g:
            fn()
        g.launch()
        d.synchronize()
        ms_graph = batch_us(d, lambda i: g.launch(), tokens, graph=False) / 1e3
        ms_eager = batch_us(d, lambda i: fn(), tokens, graph=False) / 1e3
        g.destroy()
        gbs = b_token / (ms_graph * 1e-3) / 1e9
        out[label] = {"launches_per_token": launches * W.LLAMA3_8B_LAYERS, "ms_per_token_graph": round(ms_graph, 4),
                      "ms_per_token_eager": round(ms_eager, 4), "GB/s": round(gbs, 1),
                      "frac": round(gbs / PEAK_GBS, 4)}
        log(f"C3 {label}: graph {ms_graph:.3f} ms/token ({gbs:.0f} GB/s, {gbs / PEAK_GBS:.1%}), "
            f"eager {ms_eager:.3f} ms/token")
    for nm in names:
        y = ys[nm].download(np.float32, (shape[nm][0],))
        assert np.all(np.isfinite(y)), nm  # parity of the sweep lives in tests/
    for ws, x, x2 in layers:
        for b in list(ws.values()) + [x, x2]:
            b.free()
    for b in list(ys.values()) + [table]:
        b.free()
    return out


if __name__ == "__main__":
    sys.exit(main())
