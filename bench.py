#!/usr/bin/env python3
"""Benchmark: bf16 GEMV achieved HBM GB/s (% of peak) + us/call at 4096x14336, 1 GPU.

Workload (one "step"): the two Llama-3-8B FFN decode GEMVs of config C2 in the
row-dot layout -- up/gate W [14336,4096] @ x[4096] and down W [4096,14336] @
x[14336] -- bf16 weights ~N(0,0.02), f32 activations ~N(0,1), seed 0, weights
resident in HBM.  Cold cache: each weight has COPIES distinct device copies
and consecutive steps rotate through them, so >= 1 GiB of other weights is
streamed between two reads of the same bytes (MI355X's Infinity Cache is
256 MB).  Every launch is bracketed by HIP events on the library stream.

value      whole-job throughput: algorithmic bytes of the K timed steps over
           their wall time (inputs already resident).
roofline   algorithmic bytes per launch / average kernel duration (events),
           against MI355X's 8 TB/s HBM peak.
cpu_baseline  the oracle's restatement of the reference CPU kernel
           dmc_matmul_bf16 (same fmaf chain and threading policy) timed on
           this host on a bounded sample of the same workload.

    python bench.py [--gpus 1] [--steps 50] [--warmup 5] [--extended]
"""
from __future__ import annotations

import argparse
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


def b_alg(n: int, k: int, m: int = 1) -> int:
    """Algorithmic bytes per call: bf16 W + f32 x + f32 y."""
    return 2 * n * k + 4 * k * m + 4 * n * m


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def traffic_from_profiles(kernel_prefix: str):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy-kernel calibration), read from the committed
    summary under profiles/; None when absent."""
    p = ROOT / "profiles" / "traffic.md"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        parts = line.strip().strip("|").split("|")
        if len(parts) >= 3 and parts[0].strip() == kernel_prefix:
            try:
                return int(float(parts[2].strip()))
            except ValueError:
                return None
    return None


def cpu_baseline(seconds: float = 12.0) -> dict:
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
    oracle.matmul_bf16(x, wt)  # warm caches/pages
    calls, t0 = 0, time.perf_counter()
    while True:
        oracle.matmul_bf16(x, wt)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds or calls >= 200:
            break
    per = el / calls
    gbs = b_alg(n, k) / per / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"C2 up/gate x@W W[{k},{n}] bf16, m=1, {calls} calls in {el:.1f}s "
                      f"({per * 1e6:.0f} us/call), oracle restatement of dmc_matmul_bf16 "
                      f"(jit.rs:29488), scalar fmaf, {threads} threads by the reference policy, "
                      f"host nproc={os.cpu_count()}"}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--copies", type=int, default=5, help="distinct device copies per weight")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--extended", action="store_true", help="also time C1, C4, C5 and the CS layout (stderr)")
    a = ap.parse_args(argv)

    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the GEMV shards by output rows with "
              "no reduction; see DESIGN.md); run with --gpus 1", file=sys.stderr)
        return 2

    import demonic_amd as d
    from demonic_amd import workloads as W

    if not d.available():
        print("bench.py: no usable gfx950 device: " + d._lib.load().dmc_hip_last_error().decode(),
              file=sys.stderr)
        return 1
    info = d.device_info()
    log(f"device {info}")

    t = time.perf_counter()
    c2 = W.c2()
    log(f"generated C2 inputs in {time.perf_counter() - t:.1f}s")
    shapes = {}
    bufs = []
    for name, (w, x) in c2.items():
        n, k = w.shape
        first = d.DeviceBuffer.from_numpy(w)
        copies = [first]
        for _ in range(a.copies - 1):
            c = d.DeviceBuffer(w.nbytes)
            c.copy_from(first)
            copies.append(c)
        dx = d.DeviceBuffer.from_numpy(x)
        dy = d.DeviceBuffer(4 * n)
        shapes[name] = (n, k, copies, dx, dy)
        bufs += copies + [dx, dy]
    d.synchronize()
    order = ["up", "down"]

    def launch(name, step):
        n, k, copies, dx, dy = shapes[name]
        d.gemv_rd(dx, copies[step % len(copies)], dy, 1, k, n)

    for i in range(a.warmup):
        for name in order:
            launch(name, i)
    d.synchronize()

    evs = [d.Event() for _ in range(a.steps * len(order) * 2)]
    t0 = time.perf_counter()
    e = 0
    for i in range(a.steps):
        for name in order:
            evs[e].record()
            launch(name, i)
            evs[e + 1].record()
            e += 2
    d.synchronize()
    wall = time.perf_counter() - t0

    per_shape = {name: [] for name in order}
    e = 0
    for i in range(a.steps):
        for name in order:
            per_shape[name].append(evs[e].elapsed_ms(evs[e + 1]) * 1e3)
            e += 2
    bytes_step = sum(b_alg(shapes[nm][0], shapes[nm][1]) for nm in order)
    value = bytes_step * a.steps / wall / 1e9
    kern_us = {nm: float(np.mean(v)) for nm, v in per_shape.items()}
    avg_us = float(np.mean([u for v in per_shape.values() for u in v]))
    achieved = np.mean([b_alg(shapes[nm][0], shapes[nm][1]) for nm in order]) / (avg_us * 1e-6) / 1e9
    # parity spot check of the timed outputs (first rows only; full parity is in tests/)
    for nm in order:
        n, k, copies, dx, dy = shapes[nm]
        y = dy.download(np.float32, (n,))
        assert np.all(np.isfinite(y)), nm

    roofline = {"bound": "hbm", "achieved": round(float(achieved), 1), "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(float(achieved) / PEAK_GBS, 4),
                "traffic": traffic_from_profiles("gemv_rd_kernel<8,4,1>"),
                "kernel": "gemv_rd_kernel<VEC=8,ROWS=4,MT=1>",
                "bytes_per_launch": int(b_alg(14336, 4096))}
    cpu = None if a.no_cpu else cpu_baseline(a.cpu_seconds)
    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(wall / a.steps * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16w-f32acc",
        "data": "synthetic: seeded N(0,0.02) bf16 weights, N(0,1) f32 activations (PCG64 seed 0)",
        "config": {"workload": "C2 Llama-3-8B FFN decode GEMVs, row-dot layout: up/gate W[14336,4096] "
                               "and down W[4096,14336], m=1, weights resident, cold cache "
                               f"({a.copies} rotating copies each)",
                   "us_per_call": {nm: round(u, 3) for nm, u in kern_us.items()},
                   "frac_of_peak_value": round(value / PEAK_GBS, 4)},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if a.extended:
        result["extended"] = extended(d, W)
    for b in bufs:
        b.free()
    print(json.dumps(result), flush=True)
    return 0


def _time_calls(d, fn, reps):
    evs = [d.Event() for _ in range(2 * reps)]
    for i in range(reps):
        evs[2 * i].record()
        fn(i)
        evs[2 * i + 1].record()
    d.synchronize()
    return float(np.mean([evs[2 * i].elapsed_ms(evs[2 * i + 1]) * 1e3 for i in range(reps)]))


def extended(d, W) -> dict:
    """Secondary configurations (stderr + the JSON 'extended' field)."""
    out = {}
    cases = [("C1 rd 4096x4096", W.c1(), "rd", 1)]
    c2 = W.c2()
    cases += [("C2 cs up [4096,14336]", c2["up"], "cs", 1), ("C2 cs down [14336,4096]", c2["down"], "cs", 1)]
    for label, (w, x), layout, m in cases:
        n, k = w.shape
        wl = w if layout == "rd" else np.ascontiguousarray(w.T)
        reps = max(2, int(1.2e9 // wl.nbytes) + 2)
        copies = [d.DeviceBuffer.from_numpy(wl)]
        for _ in range(min(reps, 10) - 1):
            c = d.DeviceBuffer(wl.nbytes)
            c.copy_from(copies[0])
            copies.append(c)
        dx = d.DeviceBuffer.from_numpy(x)
        dy = d.DeviceBuffer(4 * n * m)
        f = (lambda i: d.gemv_rd(dx, copies[i % len(copies)], dy, m, k, n)) if layout == "rd" else \
            (lambda i: d.gemv_cs(dx, copies[i % len(copies)], dy, m, k, n))
        for i in range(3):
            f(i)
        us = _time_calls(d, f, 30)
        gbs = b_alg(n, k, m) / (us * 1e-6) / 1e9
        out[label] = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
        log(f"{label}: {us:.2f} us  {gbs:.0f} GB/s  {gbs / PEAK_GBS:.1%}")
        for c in copies:
            c.free()
        dx.free()
        dy.free()
    # C4 LM head, skinny M (one resident copy: 1.05 GB exceeds the 256 MB cache)
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
        us = _time_calls(d, f, 10)
        gbs = b_alg(n, k, m) / (us * 1e-6) / 1e9
        out[f"C4 rd m={m}"] = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
        log(f"C4 rd m={m}: {us:.1f} us  {gbs:.0f} GB/s  {gbs / PEAK_GBS:.1%}")
        dx.free()
        dy.free()
    dw.free()
    return out


if __name__ == "__main__":
    sys.exit(main())
