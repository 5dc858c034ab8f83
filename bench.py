#!/usr/bin/env python3
"""Benchmark of the gfx950 fp32 path on one MI355X.

Default workload (the config BASELINE's metric is quoted on): C2, the
reductions on fp32 [4096, 4096] ~ U(-1, 1).  One step = the ten reductions
of that config, each a separate kernel launch reading a 64 MiB input:
global sum, global mean, and per-row (axis 1) and per-column (axis 0)
sum / mean / max / argmax.  Inputs rotate over ten device buffers (640 MiB,
more than twice the 256 MiB Infinity Cache), so every launch reads HBM.

``value`` = algorithmic bytes of all launches in the timed steps / wall time
of those steps (HIP events on the launch stream around the K steps, inputs
resident in HBM before timing starts).  Algorithmic bytes count each input
element read once and each output written once.  ``roofline`` is for the
kernel with the largest total time: its algorithmic bytes per launch over
its average launch time, each launch bracketed by its own pair of events.
``cpu_baseline`` times the C restatement of the reference AVX2 path
(oracle/, single thread, as the reference is single-threaded) on the box's
host CPU over a bounded sample of whole steps.

Other workloads (--workload c1|c3|c4|c5) are for profiling; the default
run also reports their headline figures under "workloads".
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0      # MI355X HBM3E, published
PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 MFMA, published
METRIC = "achieved HBM GB/s (% of peak) for fp32 softmax/reductions on 1 MI355X"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", default="c2", choices=["c1", "c2", "c3", "c4", "c5"])
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-extra", action="store_true", help="skip the other workloads")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    return p.parse_args()


class Launch:
    """One kernel launch of a step: a callable plus its algorithmic bytes/flops."""

    def __init__(self, name, kernel, fn, work, unit="B"):
        self.name, self.kernel, self.fn, self.work, self.unit = name, kernel, fn, work, unit


def c2_launches(engine, DeviceArray, nbuf=10):
    from cortexmind_amd.data import c2_reduce

    x = c2_reduce()
    rows, cols = x.shape
    n = x.size
    bufs = [DeviceArray.from_numpy(x) for _ in range(nbuf)]
    z1 = DeviceArray((1,), np.float32)
    zf = DeviceArray((4096,), np.float32)
    zi = DeviceArray((4096,), np.int32)
    xb = 4 * n
    ops = [
        ("sum_global", "k_rows<SumOp,seg>", lambda b: engine.reduce.sum(b, z1, n), xb + 4),
        ("mean_global", "k_rows<SumOp,seg>", lambda b: engine.reduce.mean(b, z1, n), xb + 4),
        ("sum_axis1", "k_rows<SumOp>", lambda b: engine.reduce.sum(b, zf, rows, cols, 1), xb + 4 * rows),
        ("mean_axis1", "k_rows<SumOp>", lambda b: engine.reduce.mean(b, zf, rows, cols, 1), xb + 4 * rows),
        ("max_axis1", "k_rows<MaxOp>", lambda b: engine.reduce.max(b, zf, rows, cols, 1), xb + 4 * rows),
        ("argmax_axis1", "k_rows<ArgMaxOp>", lambda b: engine.reduce.argmax(b, zi, rows, cols, 1), xb + 4 * rows),
        ("sum_axis0", "k_cols<SumOp>", lambda b: engine.reduce.sum(b, zf, 1, rows, cols), xb + 4 * cols),
        ("mean_axis0", "k_cols<SumOp>", lambda b: engine.reduce.mean(b, zf, 1, rows, cols), xb + 4 * cols),
        ("max_axis0", "k_cols<MaxColOp>", lambda b: engine.reduce.max(b, zf, 1, rows, cols), xb + 4 * cols),
        ("argmax_axis0", "k_cols<ArgMaxOp>", lambda b: engine.reduce.argmax(b, zi, 1, rows, cols), xb + 4 * cols),
    ]
    keep = (bufs, z1, zf, zi)
    launches = []
    for i, (name, kern, fn, work) in enumerate(ops):
        launches.append(Launch(name, kern, (lambda fn=fn, i=i: (lambda step: fn(bufs[(step * 10 + i) % nbuf])))(), work))
    desc = {"workload": "C2 reductions fp32 [4096,4096] ~ U(-1,1)", "shape": [rows, cols],
            "ops": [o[0] for o in ops], "rotating_input_buffers": nbuf,
            "buffer_bytes": xb}
    return launches, desc, keep, x


def cpu_c2(x, seconds):
    """Single-thread oracle over whole C2 steps (the same ten reductions)."""
    from oracle import oracle

    rows, cols = x.shape
    step = [lambda: oracle.reduce_flat("sum", x), lambda: oracle.reduce_flat("mean", x)]
    for op in ("sum", "mean", "max", "argmax"):
        step.append(lambda op=op: oracle.reduce_axis(op, x, rows, cols, 1))
    for op in ("sum", "mean", "max", "argmax"):
        step.append(lambda op=op: oracle.reduce_axis(op, x, 1, rows, cols))
    bytes_step = 2 * (4 * x.size + 4) + 4 * (4 * x.size + 4 * rows) + 4 * (4 * x.size + 4 * cols)
    for f in step:  # warm-up
        f()
    t0 = time.perf_counter()
    nsteps = 0
    while True:
        for f in step:
            f()
        nsteps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    return {"value": round(bytes_step * nsteps / dt / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"{nsteps} whole C2 steps (10 reductions of fp32 [4096,4096]) "
                      f"in {dt:.1f} s, oracle/cxm_oracle.c -O3 -mavx2 -mfma, 1 thread"}


def time_launches(launches, steps, warmup, stream_sync, Event):
    """Warm up, then time `steps` steps: one event pair per launch plus an
    event pair around the whole timed region."""
    for s in range(warmup):
        for l in launches:
            l.fn(s)
    stream_sync()
    nl = len(launches)
    ev = [[(Event(), Event()) for _ in range(nl)] for _ in range(steps)]
    t_start, t_stop = Event(), Event()
    stream_sync()
    t_start.record()
    for s in range(steps):
        for i, l in enumerate(launches):
            ev[s][i][0].record()
            l.fn(warmup + s)
            ev[s][i][1].record()
    t_stop.record()
    t_stop.sync()
    stream_sync()
    total_ms = t_start.elapsed_ms(t_stop)
    per = [[ev[s][i][0].elapsed_ms(ev[s][i][1]) for s in range(steps)] for i in range(nl)]
    for row in ev:
        for a, b in row:
            a.close()
            b.close()
    t_start.close()
    t_stop.close()
    return total_ms, per


def summarize(launches, total_ms, per, steps):
    per_op = {}
    by_kernel = {}
    for l, times in zip(launches, per):
        avg = float(np.mean(times))
        rate = l.work / (avg * 1e-3) / (1e9 if l.unit == "B" else 1e12)
        per_op[l.name] = {"avg_ms": round(avg, 5), ("GB/s" if l.unit == "B" else "TFLOP/s"): round(rate, 2)}
        k = by_kernel.setdefault(l.kernel, {"time": 0.0, "work": 0.0, "n": 0, "unit": l.unit})
        k["time"] += float(np.sum(times))
        k["work"] += l.work * len(times)
        k["n"] += len(times)
    dom_name, dom = max(by_kernel.items(), key=lambda kv: kv[1]["time"])
    avg_ms = dom["time"] / dom["n"]
    work_per_launch = dom["work"] / dom["n"]
    if dom["unit"] == "B":
        achieved = work_per_launch / (avg_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4)}
    else:
        achieved = work_per_launch / (avg_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP32_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_TFLOPS, 4)}
    roof.update({"traffic": None, "kernel": dom_name, "avg_launch_ms": round(avg_ms, 5),
                 "algorithmic_per_launch": work_per_launch})
    return per_op, roof


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    from cortexmind_amd import engine
    from cortexmind_amd.device import DeviceArray, Event, device_count, device_info
    from cortexmind_amd._lib import call

    if device_count() < 1:
        print(json.dumps({"error": "no HIP device visible"}))
        sys.exit(1)
    info = device_info()
    sync = lambda: call("cxm_device_sync")  # noqa: E731

    if args.workload != "c2":
        raise SystemExit("only c2 is wired in this build step")
    launches, desc, keep, x = c2_launches(engine, DeviceArray)
    total_ms, per = time_launches(launches, args.steps, args.warmup, sync, Event)
    step_work = sum(l.work for l in launches)
    value = step_work * args.steps / (total_ms * 1e-3) / 1e9
    per_op, roof = summarize(launches, total_ms, per, args.steps)
    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": desc, "frac_of_peak": round(value / PEAK_HBM_GBS, 4),
        "roofline": roof, "per_op": per_op, "device": info,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_c2(x, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
