#!/usr/bin/env python3
"""Benchmark of the gfx950 fp32 path on one MI355X.

Default workload (the config BASELINE's metric is quoted on): C2, the
reductions on fp32 [4096, 4096] ~ U(-1, 1).  One step = the ten reductions
of that config, each one kernel launch reading a 64 MiB input: global sum,
global mean, and per-row (axis 1) and per-column (axis 0) sum / mean / max /
argmax.  Inputs rotate over ten device buffers (640 MiB, more than twice the
256 MiB Infinity Cache), so every launch reads HBM, not the cache.

``value`` = algorithmic bytes of the timed steps / their wall time, from
HIP events on the launch stream around the K steps (inputs resident in HBM
before timing starts).  Algorithmic bytes count each input element read once
and each output written once; re-reads are not credited.  ``roofline`` is
for the kernel with the largest share of step time: algorithmic bytes per
launch over its average launch time, from events around a run of
max(K, 100) back-to-back launches of that op alone (rotating inputs, four
untimed launches queued ahead of the start event).  ``traffic`` is
the HBM bytes per launch measured with rocprofv3 PMC counters (FETCH_SIZE,
WRITE_SIZE, scaled against a plain copy kernel), read from
profiles/pmc_traffic.txt when that file has a line for the kernel.
``measured_peaks`` (bandwidth headlines) gives the copy and read rates this
part reaches at 1 GiB, with the value and the roofline figure as fractions
of the read rate, beside ``frac_of_peak`` against the 8 TB/s specification,
and ``single_launch_floors``: one launch of this library's fastest
streaming kernels at the ops' own sizes (a 64 MiB read; 32 MiB in + 32 MiB
out; 64 MiB in + 32 MiB out), timed like the ops, with each C2 op's (and,
under "workloads", each C4 op's) fraction of its floor.  Every op's
``kernel`` label (``kernel_of``) is the name rocprofv3's trace prints.
``cpu_baseline`` times the C restatement of the reference AVX2 path
(oracle/, one thread, as the reference is single-threaded) on the same host
over a bounded sample of whole steps; each BASELINE workload under
"workloads" (C1, C3, C4, C5) carries its own.

C5's roofline is the whole training step (its FLOP over its time on the
fp32 matrix peak); ``first_10_steps`` times the configured ten steps of a
fresh network from an idle queue (first step and the other nine apart),
before the warm-up steps that precede the steady-state figure.

The default run also reports the other workloads (C1 softmax, C3 affine
fwd/bwd, C4 long-row softmax fwd/bwd, C5 MLP training step, and "more":
the rest of the reduction and elementwise-math surface at the C2/C3
shapes) under "workloads"; --workload NAME makes one of them the headline,
for profiling.
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
PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 matrix, published
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 / fp16 matrix, published (no sparsity)
METRIC = "achieved HBM GB/s (% of peak) for fp32 softmax/reductions on 1 MI355X"
MLP_FLOP_PER_STEP = 39_174_799_360


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", default="c2", choices=["c1", "c2", "c3", "c4", "c5", "more", "g16"])
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-extra", action="store_true", help="skip the other workloads")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline time of the headline workload")
    p.add_argument("--cpu-seconds-other", type=float, default=3.0,
                   help="CPU baseline time of each other BASELINE workload (C1, C3, C4, C5)")
    p.add_argument("--copy-calibration", action="store_true",
                   help="first copy 64 MiB device-to-device three times (the known-size "
                        "kernel that scales FETCH_SIZE / WRITE_SIZE counters)")
    p.add_argument("--timeline", nargs="?", const="c2", choices=["c2", "c4", "c5"],
                   help="instead of the bench line, print per-workgroup timelines from the diagnostics build "
                        "cortexmind_amd/libcxm_hip_timeline.so (make -C cortexmind_amd/csrc timeline): c2 (default) "
                        "the C2 row sum, column sum, global sum and column argmax; c4 the long-row softmax and "
                        "log-softmax, forward and backward; c5 the MLP step's ring products and output-layer head")
    p.add_argument("--summarize", nargs="+", metavar=("KIND", "CSV"),
                   help="summarise rocprofv3 output instead of running: 'trace <kernel_trace.csv>' prints the "
                        "per-kernel table of profiles/*_kernel_trace.md; 'pmc <counter_collection.csv>...' prints "
                        "per-kernel FETCH_SIZE / WRITE_SIZE bytes per launch scaled by the 64 MiB copy "
                        "(profiles/pmc_traffic.txt lines); 'mfma <counter_collection.csv>' prints per-kernel "
                        "MFMA busy from SQ_VALU_MFMA_BUSY_CYCLES, SQ_INSTS_MFMA and GRBM_GUI_ACTIVE; 'tcc <counter_collection.csv>' "
                        "per-kernel L2 hits and misses from TCC_HIT_sum and TCC_MISS_sum; 'counters <counter_collection.csv>' "
                        "every counter's mean per dispatch")
    return p.parse_args()


# ------------------------------------------------------- rocprof summaries

def kernel_name(raw):
    """A kernel's name as bench.py labels it: no return type, namespaces,
    argument list or spaces."""
    import re

    n = re.sub(r"^void ", "", raw)
    n = n.replace("cxm::(anonymous namespace)::", "").replace("(anonymous namespace)::", "").replace("cxm::", "")
    depth, out = 0, []
    for ch in n:  # drop the argument list: the first '(' outside template brackets
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            break
        out.append(ch)
    return "".join(out).replace(" ", "")


def summarize(kind, paths):
    import csv
    from collections import OrderedDict

    if kind == "trace":
        g = OrderedDict()
        for r in csv.DictReader(open(paths[0])):
            grid = r.get("Grid_Size") or (int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"]))
            key = (kernel_name(r["Kernel_Name"]), int(grid))
            g.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
        tot = sum(sum(v) for v in g.values())
        print("| kernel | grid (threads) | calls | avg us | min us | max us | % time |")
        print("|---|---:|---:|---:|---:|---:|---:|")
        for (k, grid), v in sorted(g.items(), key=lambda kv: -sum(kv[1])):
            print(f"| `{k}` | {grid} | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f} | "
                  f"{100 * sum(v) / tot:.1f} |")
        return
    if kind == "mfma":
        # per dispatch: SQ_VALU_MFMA_BUSY_CYCLES, SQ_INSTS_MFMA, GRBM_GUI_ACTIVE (one row per counter)
        disp, meta = {}, {}
        for r in csv.DictReader(open(paths[0])):
            k = int(r["Dispatch_Id"])
            disp.setdefault(k, {})[r["Counter_Name"]] = float(r["Counter_Value"])
            meta[k] = (kernel_name(r["Kernel_Name"]), int(r["Grid_Size"]))
        g = OrderedDict()
        for k, c in disp.items():
            g.setdefault(meta[k], []).append(c)
        print("| kernel | grid (threads) | dispatches | cycles per XCD | MFMA busy cycles / MFMA | MFMA busy |")
        print("|---|---:|---:|---:|---:|---:|")
        tot = lambda cs, n: sum(c.get(n, 0.0) for c in cs)  # noqa: E731
        for (k, grid), cs in sorted(g.items(), key=lambda kv: -tot(kv[1], "SQ_VALU_MFMA_BUSY_CYCLES")):
            mb, mi, ga = tot(cs, "SQ_VALU_MFMA_BUSY_CYCLES"), tot(cs, "SQ_INSTS_MFMA"), tot(cs, "GRBM_GUI_ACTIVE")
            if mi == 0:
                continue
            # GRBM_GUI_ACTIVE sums the 8 XCDs' busy cycles; 1024 SIMDs in all
            print(f"| `{k}` | {grid} | {len(cs)} | {ga / len(cs) / 8:.3g} | {mb / mi:.0f} | {100 * mb / (ga / 8 * 1024):.1f}% |")
        return
    if kind == "counters":
        # every counter of the CSV, mean per dispatch, per kernel and grid
        disp, meta, names = {}, {}, []
        for r in csv.DictReader(open(paths[0])):
            k = int(r["Dispatch_Id"])
            disp.setdefault(k, {})[r["Counter_Name"]] = float(r["Counter_Value"])
            meta[k] = (kernel_name(r["Kernel_Name"]), int(r["Grid_Size"]))
            if r["Counter_Name"] not in names:
                names.append(r["Counter_Name"])
        g = OrderedDict()
        for k, c in disp.items():
            g.setdefault(meta[k], []).append(c)
        print("| kernel | grid (threads) | dispatches | " + " | ".join(names) + " |")
        print("|---|---:|---:|" + "---:|" * len(names))
        for (k, grid), cs in sorted(g.items(), key=lambda kv: kv[0]):
            if k.startswith("__amd_rocclr"):
                continue
            vals = [sum(c.get(n, 0.0) for c in cs) / len(cs) for n in names]
            print(f"| `{k}` | {grid} | {len(cs)} | " + " | ".join(f"{v:.4g}" for v in vals) + " |")
        return
    if kind == "tcc":
        disp, meta = {}, {}
        for r in csv.DictReader(open(paths[0])):
            k = int(r["Dispatch_Id"])
            disp.setdefault(k, {})[r["Counter_Name"]] = float(r["Counter_Value"])
            meta[k] = (kernel_name(r["Kernel_Name"]), int(r["Grid_Size"]))
        g = OrderedDict()
        for k, c in disp.items():
            g.setdefault(meta[k], []).append(c)
        print("| kernel | grid (threads) | dispatches | TCC_HIT | TCC_MISS | misses x 128 B | hit rate |")
        print("|---|---:|---:|---:|---:|---:|---:|")
        for (k, grid), cs in sorted(g.items(), key=lambda kv: kv[0]):
            if k.startswith("__amd_rocclr"):
                continue
            h = sum(c.get("TCC_HIT_sum", 0.0) for c in cs) / len(cs)
            m = sum(c.get("TCC_MISS_sum", 0.0) for c in cs) / len(cs)
            print(f"| `{k}` | {grid} | {len(cs)} | {h:.0f} | {m:.0f} | {m * 128 / 2 ** 20:.2f} MiB | "
                  f"{100 * h / max(1.0, h + m):.1f}% |")
        return
    if kind != "pmc":
        raise SystemExit(f"unknown summary kind {kind}")
    per = {}  # (name, grid) -> {counter: [bytes per dispatch]}
    calib = {}  # counter -> [(dispatch id, bytes)] of the copies
    for path in paths:
        for r in csv.DictReader(open(path)):
            c = r["Counter_Name"]
            if c not in ("FETCH_SIZE", "WRITE_SIZE"):
                continue
            key = (kernel_name(r["Kernel_Name"]), int(r["Grid_Size"]))
            v = float(r["Counter_Value"]) * 1024.0  # KiB
            per.setdefault(key, {}).setdefault(c, []).append(v)
            if key[0].startswith("__amd_rocclr_copyBuffer"):
                calib.setdefault(c, []).append((int(r["Dispatch_Id"]), v))
    scale = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        first = [v for _, v in sorted(calib.get(c, []))[:3]]  # --copy-calibration's copies run first
        scale[c] = (64 * 2 ** 20) / (sum(first) / len(first)) if first else 1.0
    print(f"# scale FETCH_SIZE x{scale['FETCH_SIZE']:.4f}, WRITE_SIZE x{scale['WRITE_SIZE']:.4f} "
          "(a 64 MiB device-to-device copy reads and writes 64 MiB)")
    for (k, grid), d in sorted(per.items(), key=lambda kv: (kv[0][0], -len(next(iter(kv[1].values()))))):
        if k.startswith("__amd_rocclr"):
            continue
        f = sum(d.get("FETCH_SIZE", [0])) / max(1, len(d.get("FETCH_SIZE", []))) * scale["FETCH_SIZE"]
        w = sum(d.get("WRITE_SIZE", [0])) / max(1, len(d.get("WRITE_SIZE", []))) * scale["WRITE_SIZE"]
        print(f"{k}[grid={grid}] {f:.0f} {w:.0f}")


# ------------------------------------------------------- C2 timelines

TL_KINDS, TL_WGS, TL_MARKS = 4, 4096, 4  # reduce.hip's timeline tables


def timeline(reps=40):
    """C2's row sum, column sum, global sum and column argmax launched back to
    back `reps` times (inputs rotating over ten 64 MiB buffers), then the
    diagnostics build's per-workgroup marks of the last round, in us from the
    round's first workgroup start: 0 entry, 1 all waves' loads folded, 2 partial
    published (column ticket taken, or flat tagged slot stored), 3 final
    store issued (the last workgroup of a column tile, the flat reader)."""
    import ctypes

    from cortexmind_amd import _lib

    _lib.LIB_PATH = os.path.join(ROOT, "cortexmind_amd", "libcxm_hip_timeline.so")
    from cortexmind_amd import engine as E
    from cortexmind_amd._lib import call, lib
    from cortexmind_amd.data import c2_reduce
    from cortexmind_amd.device import DeviceArray as D

    x = c2_reduce()
    rows, cols = x.shape
    bufs = [D.from_numpy(x) for _ in range(10)]
    z1, zf, zi = D((1,), np.float32), D((cols,), np.float32), D((cols,), np.int32)
    R = E.reduce
    ops = [("row sum", "k_rows_whole<SumOp,8>", 0, lambda b: R.sum(b, zf, rows, cols, 1)),
           ("column sum", "k_cols_whole<SumOp>", 1, lambda b: R.sum(b, zf, 1, rows, cols)),
           ("global sum", "k_rows<SumOp,8,2>", 2, lambda b: R.sum(b, z1, rows * cols)),
           ("column argmax", "k_cols<ArgMaxOp,true,16,16,true>", 3, lambda b: R.argmax(b, zi, 1, rows, cols))]
    k = 0
    for _ in range(reps):
        for _, _, _, fn in ops:
            fn(bufs[k % len(bufs)])
            k += 1
    call("cxm_device_sync")
    t = np.zeros((TL_KINDS, TL_WGS, TL_MARKS), np.uint64)
    fn = lib().cxm_timeline_read
    fn.argtypes, fn.restype = [ctypes.c_void_p, ctypes.c_size_t], ctypes.c_int
    if fn(t.ctypes.data, t.size) != 0:
        raise RuntimeError("cxm_timeline_read failed")
    timeline_report(t, [(name, kern, kind) for name, kern, kind, _ in ops], {0: rows, 1: 256, 2: 2049, 3: 256})


def timeline_report(t, ops, grids):
    """Prints timeline()'s tables from the raw marks t [kinds, wgs, marks];
    `ops` lists (name, kernel, kind) in launch order, `grids` the workgroups
    per launch of each kind."""
    t = t.astype(np.int64)
    recs = {kind: t[kind, :grids[kind]] for _, _, kind in ops}
    t0 = min(int(r[:, 0][r[:, 0] > 0].min()) for r in recs.values())
    us = lambda v: (np.asarray(v, dtype=np.float64) - t0) / 100.0  # noqa: E731  (100 MHz clock)
    print("| op (kernel) | workgroups | first start | last start | loads folded: median / last | "
          "last partial published | end | combine after the last fold | gap to the next op |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|---:|")
    lines = []
    for name, kern, kind in ops:
        r = recs[kind]
        start, fold, pub, fin = r[:, 0], r[:, 1], r[:, 2], r[:, 3]
        if kind == 2:  # the flat sum: writers 0..2047, the reader last
            wfold, wpub = fold[:-1], pub[:-1]
            end = fin[-1]
            last_pub = wpub.max()
            fold_med, fold_max = np.median(wfold), wfold.max()
        elif kind == 0:
            end = fin.max()
            last_pub = None
            fold_med, fold_max = np.median(fold), fold.max()
        else:  # column tiles: the last workgroup of each writes the result
            ends = np.where(fin > start, fin, pub)
            end = ends.max()
            last_pub = pub.max()
            fold_med, fold_max = np.median(fold), fold.max()
        lines.append([name, kern, r.shape[0], us(start.min()), us(start.max()), us(fold_med), us(fold_max),
                      us(last_pub) if last_pub is not None else None, us(end), start.min(), end, fold_max])
    for i, ln in enumerate(lines):
        gap = (lines[i + 1][9] - ln[10]) / 100.0 if i + 1 < len(lines) else None
        print(f"| {ln[0]} (`{ln[1]}`) | {ln[2]} | {ln[3]:.2f} | {ln[4]:.2f} | {ln[5]:.2f} / {ln[6]:.2f} | "
              + (f"{ln[7]:.2f}" if ln[7] is not None else "—") + f" | {ln[8]:.2f} | {(ln[10] - ln[11]) / 100.0:.2f} | "
              + (f"{gap:.2f}" if gap is not None else "—") + " |")
    print()
    print("| op | loads folded, last workgroup by XCD 0..7 (us from the op's first start) |")
    print("|---|---|")
    for (name, _, kind), ln in zip(ops, lines):
        r = recs[kind][:-1] if kind == 2 else recs[kind]
        xcd = np.arange(r.shape[0]) % 8
        per = [(r[xcd == c, 1].max() - ln[9]) / 100.0 for c in range(8)]
        print(f"| {name} | " + " ".join(f"{v:.2f}" for v in per) + " |")


SM_TL = (4, 1024, 5)  # softmax.hip's long-row tables: kernels, workgroups, marks


def timeline_softmax(reps=40):
    """C4's softmax and log-softmax, forward and backward, [64, 131072], back
    to back `reps` times (inputs rotating over four sets), then the
    diagnostics build's marks of the last round: 0 entry, 1 (forward only)
    its staggered start over, 2 partial published, 3 the row's partials in,
    4 stores issued; in us from the round's first start."""
    import ctypes

    from cortexmind_amd import _lib

    _lib.LIB_PATH = os.path.join(ROOT, "cortexmind_amd", "libcxm_hip_timeline.so")
    from cortexmind_amd import engine as E
    from cortexmind_amd._lib import call, lib
    from cortexmind_amd.data import c4_long_softmax
    from cortexmind_amd.device import DeviceArray as D

    x, dy = c4_long_softmax()
    r, c = x.shape
    nset = 4
    X = [D.from_numpy(x) for _ in range(nset)]
    G = [D.from_numpy(dy) for _ in range(nset)]
    Y = [D((r, c)) for _ in range(nset)]
    dX = [D((r, c)) for _ in range(nset)]
    S = E.softmax
    ops = [("softmax fwd", "k_sm_fwd_x<false>", 0, lambda k: S.forward(X[k], Y[k], r, c)),
           ("log-softmax fwd", "k_sm_fwd_x<true>", 1, lambda k: S.forward(X[k], Y[k], r, c, log=True)),
           ("softmax bwd", "k_sm_bwd_x<false>", 2, lambda k: S.backward(Y[k], G[k], dX[k], r, c)),
           ("log-softmax bwd", "k_sm_bwd_x<true>", 3, lambda k: S.backward(Y[k], G[k], dX[k], r, c, log=True))]
    for i in range(reps):
        for _, _, _, fn in ops:
            fn(i % nset)
    call("cxm_device_sync")
    t = np.zeros(SM_TL, np.uint64)
    fn = lib().cxm_timeline_softmax_read
    fn.argtypes, fn.restype = [ctypes.c_void_p, ctypes.c_size_t], ctypes.c_int
    if fn(t.ctypes.data, t.size) != 0:
        raise RuntimeError("cxm_timeline_softmax_read failed")
    timeline_softmax_report(t, [(n, k, kind) for n, k, kind, _ in ops], r * (c // 8192))


def timeline_softmax_report(t, ops, wgs):
    """Prints timeline_softmax()'s table from the raw marks t [kernels, wgs,
    marks]; `ops` lists (name, kernel, table) in launch order."""
    t = t.astype(np.int64)
    recs = {kind: t[kind, :wgs] for _, _, kind in ops}
    t0 = min(int(r[:, 0].min()) for r in recs.values())
    us = lambda v: (np.asarray(v, dtype=np.float64) - t0) / 100.0  # noqa: E731
    print("| op (kernel) | workgroups | first start | last start | staggered start over: last | first workgroup done | "
          "partial published: median / last | row's partials in: median / last | "
          "exchange wait per workgroup: median / max | end | gap to the next op |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|")
    for i, (name, kern, kind) in enumerate(ops):
        r = recs[kind]
        wait = (r[:, 3] - r[:, 2]) / 100.0
        end = r[:, 4].max()
        gap = (recs[ops[i + 1][2]][:, 0].min() - end) / 100.0 if i + 1 < len(ops) else None
        print(f"| {name} (`{kern}`) | {r.shape[0]} | {us(r[:, 0].min()):.2f} | {us(r[:, 0].max()):.2f} | "
              + (f"{us(r[:, 1].max()):.2f}" if r[:, 1].max() > 0 else "—") + f" | {us(r[:, 4].min()):.2f} | "
              f"{us(np.median(r[:, 2])):.2f} / {us(r[:, 2].max()):.2f} | {us(np.median(r[:, 3])):.2f} / {us(r[:, 3].max()):.2f} | "
              f"{np.median(wait):.2f} / {wait.max():.2f} | {us(end):.2f} | " + (f"{gap:.2f}" if gap is not None else "—") + " |")


GEMM_TL = (4, 1024, 6)  # gemm.hip's ring tables: instances, workgroups, marks
HEAD_TL = (256, 8)  # mlp.hip's head table


def timeline_mlp(steps=40):
    """`steps` C5 MLP steps back to back, then the diagnostics build's marks
    of the last step: per ring product (0 entry, 1 prologue done: the first
    four stages landed, 2 K loop done, 3 epilogue done; 4 and 5 the core
    clock counter at 1 and 2) and per head workgroup (0 entry, 1 W3 and h2
    loaded, 2 W3 in LDS, 3 logits, 4 cross-entropy, 5 dh2 stored, 6 partials
    stored), in us from the step's first workgroup start."""
    import ctypes

    from cortexmind_amd import _lib

    _lib.LIB_PATH = os.path.join(ROOT, "cortexmind_amd", "libcxm_hip_timeline.so")
    from cortexmind_amd import engine as E
    from cortexmind_amd._lib import call, lib
    from cortexmind_amd.data import c5_mlp
    from cortexmind_amd.device import DeviceArray as D

    x, labels, params = c5_mlp()
    B, d0 = x.shape
    d1, d2, d3 = params["w1"].shape[1], params["w2"].shape[1], params["w3"].shape[1]
    dx_, dl_ = D.from_numpy(x), D.from_numpy(labels)
    P = {k: D.from_numpy(v) for k, v in params.items()}
    loss = D((1,))
    net = E.Mlp3(B, d0, d1, d2, d3)
    for _ in range(steps):
        net.step(dx_, dl_, P, 0.01, loss)
    call("cxm_device_sync")
    g = np.zeros(GEMM_TL, np.uint64)
    h = np.zeros(HEAD_TL, np.uint64)
    for name, arr in (("cxm_timeline_gemm_read", g), ("cxm_timeline_head_read", h)):
        fn = getattr(lib(), name)
        fn.argtypes, fn.restype = [ctypes.c_void_p, ctypes.c_size_t], ctypes.c_int
        if fn(arr.ctypes.data, arr.size) != 0:
            raise RuntimeError(f"{name} failed")
    timeline_mlp_report(g, h, {0: 256, 1: 256, 2: 256, 3: 240}, 256)


def timeline_mlp_report(g, h, wgs, head_wgs):
    """Prints timeline_mlp()'s table from the raw marks: g [instances, wgs,
    marks] of the ring products (`wgs` product workgroups per instance), h
    [head workgroups, marks]."""
    g, h = g.astype(np.int64), h.astype(np.int64)
    names = {0: ("layer-1 forward", "k_gemm_ring<true,false,true>"), 1: ("layer-2 forward", "k_gemm_ring<true,false,false>"),
             2: ("layer-2 input gradient", "k_gemm_ring<true,true,false>"),
             3: ("weight gradients, paired", "k_gemm_ring_pair<false,false>")}
    rec = {k: g[k, :n] for k, n in wgs.items()}
    hd = h[:head_wgs]
    t0 = min(int(r[:, 0].min()) for r in rec.values())
    us = lambda v: (np.asarray(v, dtype=np.float64) - t0) / 100.0  # noqa: E731
    rows = []
    for k in (0, 1):
        rows.append((k, rec[k]))
    rows.append(("head", hd))
    rows += [(2, rec[2]), (3, rec[3])]
    print("| kernel | workgroups | first start | last start | prologue (median) | K loop (median / max) | "
          "epilogue (median / max) | end | core clock in the K loop, GHz (median) | gap to the next kernel |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|")
    spans = []
    for k, r in rows:
        if k == "head":
            spans.append((r[:, 0].min(), r[:, 6].max()))
        else:
            spans.append((r[:, 0].min(), r[:, 3].max()))
    for i, (k, r) in enumerate(rows):
        gap = (spans[i + 1][0] - spans[i][1]) / 100.0 if i + 1 < len(rows) else None
        gs = f"{gap:.2f}" if gap is not None else "—"
        if k == "head":
            print(f"| output-layer head (`k_mlp_head`) | {r.shape[0]} | {us(r[:, 0].min()):.2f} | {us(r[:, 0].max()):.2f} | "
                  f"— | — | — | {us(r[:, 6].max()):.2f} | — | {gs} |")
            continue
        pro, loop, epi = (r[:, 1] - r[:, 0]) / 100.0, (r[:, 2] - r[:, 1]) / 100.0, (r[:, 3] - r[:, 2]) / 100.0
        clk = (r[:, 5] - r[:, 4]) / np.maximum(r[:, 2] - r[:, 1], 1) / 10.0  # counter ticks per 10 ns -> GHz
        print(f"| {names[k][0]} (`{names[k][1]}`) | {r.shape[0]} | {us(r[:, 0].min()):.2f} | {us(r[:, 0].max()):.2f} | "
              f"{np.median(pro):.2f} | {np.median(loop):.2f} / {loop.max():.2f} | {np.median(epi):.2f} / {epi.max():.2f} | "
              f"{us(r[:, 3].max()):.2f} | {np.median(clk):.3f} | {gs} |")
    print()
    marks = ["W3 and h2 loaded", "W3 in LDS", "logits", "cross-entropy", "dh2 stored", "partials stored"]
    print("| output-layer head phase | median | last |")
    print("|---|---:|---:|")
    for i, m in enumerate(marks, start=1):
        d = (hd[:, i] - hd[:, 0]) / 100.0
        print(f"| {m} (us after the workgroup's start) | {np.median(d):.2f} | {d.max():.2f} |")


class Op:
    """One op of a step: fn(k) launches it on input rotation slot k.
    `kernel` is the kernel's name as rocprofv3's trace prints it (without
    spaces), or a description for an op of several kernels, whose names
    (one launch each per op) are then `parts`."""

    def __init__(self, name, kernel, fn, work, unit="B", peak=None, parts=None):
        self.name, self.kernel, self.fn, self.work, self.unit = name, kernel, fn, work, unit
        self.peak = peak  # TFLOP/s of the matrix unit this op runs on (FLOP ops); fp32 when None
        self.parts = parts


# ---------------------------------------------------------------- workloads

def wl_c2(E, D):
    from cortexmind_amd.data import c2_reduce

    x = c2_reduce()
    rows, cols = x.shape
    n = x.size
    nbuf = 10
    bufs = [D.from_numpy(x) for _ in range(nbuf)]
    z1, zf, zi = D((1,), np.float32), D((4096,), np.float32), D((4096,), np.int32)
    xb = 4 * n
    R = E.reduce

    def rot(f):
        return lambda k: f(bufs[k % nbuf])

    ops = [
        Op("sum_global", "k_rows<SumOp,8,2>", rot(lambda b: R.sum(b, z1, n)), xb + 4),
        Op("mean_global", "k_rows<SumOp,8,2>", rot(lambda b: R.mean(b, z1, n)), xb + 4),
        Op("sum_axis1", "k_rows_whole<SumOp,8>", rot(lambda b: R.sum(b, zf, rows, cols, 1)), xb + 4 * rows),
        Op("mean_axis1", "k_rows_whole<SumOp,8>", rot(lambda b: R.mean(b, zf, rows, cols, 1)), xb + 4 * rows),
        Op("max_axis1", "k_rows_whole<MaxOp,8>", rot(lambda b: R.max(b, zf, rows, cols, 1)), xb + 4 * rows),
        Op("argmax_axis1", "k_rows_whole<ArgMaxOp,4>", rot(lambda b: R.argmax(b, zi, rows, cols, 1)), xb + 4 * rows),
        Op("sum_axis0", "k_cols_whole<SumOp>", rot(lambda b: R.sum(b, zf, 1, rows, cols)), xb + 4 * cols),
        Op("mean_axis0", "k_cols_whole<SumOp>", rot(lambda b: R.mean(b, zf, 1, rows, cols)), xb + 4 * cols),
        Op("max_axis0", "k_cols_whole<MaxColOp>", rot(lambda b: R.max(b, zf, 1, rows, cols)), xb + 4 * cols),
        Op("argmax_axis0", "k_cols<ArgMaxOp,true,16,16,true>", rot(lambda b: R.argmax(b, zi, 1, rows, cols)), xb + 4 * cols),
    ]
    desc = {"workload": "C2 reductions fp32 [4096,4096] ~ U(-1,1)", "shape": [rows, cols],
            "ops": [o.name for o in ops], "rotating_input_buffers": nbuf, "buffer_bytes": xb}
    return ops, desc, (bufs, z1, zf, zi), x


def wl_c1(E, D):
    from cortexmind_amd.data import c1_softmax

    x = c1_softmax()
    r, c = x.shape
    nbuf = 128  # 2 MiB each: 256 MiB of inputs and 256 MiB of outputs rotate
    xs = [D.from_numpy(x) for _ in range(nbuf)]
    ys = [D((r, c)) for _ in range(nbuf)]
    ops = [Op("softmax_fwd", "k_sm_fwd_wave<4,false,2>",
              lambda k: E.softmax.forward(xs[k % nbuf], ys[k % nbuf], r, c), 2 * 4 * x.size)]
    desc = {"workload": "C1 row softmax fp32 [512,1024] N(0,1)*4", "shape": [r, c],
            "rotating_input_buffers": nbuf,
            "note": "launch-latency bound: one launch moves 4 MiB (0.52 us at 8 TB/s), while an empty kernel "
                    "costs about 1.5 us back to back and one HBM round trip plus two wave reductions about 2 us "
                    "more, so the 80% bandwidth target is out of reach for a single [512,1024] launch; the "
                    "figure is reported, not tuned toward that target"}
    return ops, desc, (xs, ys), x


def wl_c3(E, D):
    from cortexmind_amd.data import c3_affine

    x, s, b, dy = c3_affine()
    m, n = x.shape
    dx_, ds_, db_, dy_ = D.from_numpy(x), D.from_numpy(s), D.from_numpy(b), D.from_numpy(dy)
    y_, dX, dS, dB = D((m, n)), D((m, n)), D((n,)), D((n,))
    A = E.activation
    big = 4 * m * n
    ops = []
    # kernel labels as the trace names them: the activation code is the template argument
    for act, nm in [(E.ACT_RELU, "relu"), (E.ACT_SIGMOID, "sigmoid"), (E.ACT_TANH, "tanh")]:
        ops.append(Op(f"fwd_{nm}", f"k_rowmap4<AffineF<{act}>>",
                      lambda k, act=act: A.affine_fwd(dx_, ds_, db_, y_, m, n, act), 2 * big + 2 * 4 * n))
    for act, nm in [(E.ACT_RELU, "relu"), (E.ACT_SIGMOID, "sigmoid"), (E.ACT_TANH, "tanh")]:
        ops.append(Op(f"bwd_{nm}", f"k_affine_bwd<{act},true,1,4>",
                      lambda k, act=act: A.affine_bwd(dx_, ds_, y_, dy_, dX, dS, dB, m, n, act),
                      4 * big + 3 * 4 * n))
    desc = {"workload": "C3 Y=act(X*scale+bias) fp32 [8192,8192], fwd+bwd, act in relu/sigmoid/tanh",
            "shape": [m, n], "working_set_bytes": 4 * big}
    return ops, desc, (dx_, ds_, db_, dy_, y_, dX, dS, dB), (x, s, b, dy)


def wl_c4(E, D):
    from cortexmind_amd.data import c4_long_softmax

    x, dy = c4_long_softmax()
    r, c = x.shape
    nset = 4
    X = [D.from_numpy(x) for _ in range(nset)]
    G = [D.from_numpy(dy) for _ in range(nset)]
    Y = [D((r, c)) for _ in range(nset)]
    dX = [D((r, c)) for _ in range(nset)]
    big = 4 * x.size
    S = E.softmax
    ops = [
        Op("softmax_fwd", "k_sm_fwd_x<false>", lambda k: S.forward(X[k % nset], Y[k % nset], r, c), 2 * big),
        Op("logsoftmax_fwd", "k_sm_fwd_x<true>", lambda k: S.forward(X[k % nset], Y[k % nset], r, c, log=True),
           2 * big),
        Op("softmax_bwd", "k_sm_bwd_x<false>", lambda k: S.backward(Y[k % nset], G[k % nset], dX[k % nset], r, c),
           3 * big),
        Op("logsoftmax_bwd", "k_sm_bwd_x<true>",
           lambda k: S.backward(Y[k % nset], G[k % nset], dX[k % nset], r, c, log=True), 3 * big),
    ]
    desc = {"workload": "C4 long-row softmax/log-softmax fwd+bwd fp32 [64,131072] N(0,1)*8, 10% -inf",
            "shape": [r, c], "rotating_sets": nset}
    return ops, desc, (X, G, Y, dX), (x, dy)


def wl_c5(E, D):
    from cortexmind_amd.data import c5_mlp

    x, labels, params = c5_mlp()
    B, d0 = x.shape
    d1, d2, d3 = params["w1"].shape[1], params["w2"].shape[1], params["w3"].shape[1]
    dx_, dl_ = D.from_numpy(x), D.from_numpy(labels)
    P = {k: D.from_numpy(v) for k, v in params.items()}
    loss = D((1,))
    net = E.Mlp3(B, d0, d1, d2, d3)
    ops = [Op("mlp_step", "the MLP step (5 kernels; the largest, k_gemm_ring_pair<false,false>, both weight "
              "gradients with their SGD steps)", lambda k: net.step(dx_, dl_, P, 0.01, loss),
              MLP_FLOP_PER_STEP, unit="FLOP",
              parts=["k_gemm_ring<true,false,true>", "k_gemm_ring<true,false,false>", "k_mlp_head",
                     "k_gemm_ring<true,true,false>", "k_gemm_ring_pair<false,false>"])]
    # the step's layer-2 forward GEMM alone (a per-op figure beside the step),
    # on an h1 like the step's (ReLU of N(0, 1): half zeros): the MFMA clock
    # depends on the data (power), so an all-zero operand would time faster
    rng = np.random.default_rng(5)
    h1 = D.from_numpy(np.maximum(rng.standard_normal((B, d1), dtype=np.float32), 0.0))
    w2, h2 = P["w2"], D((B, d2))
    gemm_op = Op("gemm_fwd_4096x1024x1024", "k_gemm_ring<true,false,false>",
                 lambda k: E.gemm(h1, w2, h2, B, d1, d2), 2 * B * d1 * d2, unit="FLOP")
    desc = {"workload": "C5 MLP 784-1024-1024-10 fp32 train step, batch 4096, SGD lr 0.01",
            "flop_per_step": MLP_FLOP_PER_STEP}
    return ops, desc, (dx_, dl_, P, loss, net, h1, h2, gemm_op), (x, labels, params)


def wl_more(E, D):
    """The rest of the operator surface at the C2 / C3 shapes: min, argmin,
    norm1, norm2, var, stdv on fp32 [4096, 4096] (global, axis 1, axis 0),
    and elementwise math on fp32 [8192, 8192] (1 read + 1 write each; pow
    with a tensor exponent reads two)."""
    from cortexmind_amd.data import c2_reduce, c3_affine

    x = c2_reduce()
    rows, cols = x.shape
    n = x.size
    nbuf = 10
    bufs = [D.from_numpy(x) for _ in range(nbuf)]
    z1, zf, zi = D((1,), np.float32), D((4096,), np.float32), D((4096,), np.int32)
    xb = 4 * n
    R = E.reduce

    def rot(f):
        return lambda k: f(bufs[k % nbuf])

    ops = []
    for op in ("min", "argmin", "norm1", "norm2", "var", "stdv"):
        z = zi if op == "argmin" else zf
        fn = getattr(R, op)
        kern = {"min": "MinOp", "argmin": "ArgMinOp", "norm1": "AbsSumOp", "norm2": "SqSumOp",
                "var": "Pow2Op", "stdv": "Pow2Op"}[op]
        wide = kern in ("ArgMinOp", "Pow2Op")  # 64-bit partials: the flat form combines by ticket (MODE 1),
        # whole rows take 256 threads a row, columns the general kernel; the column min starts from slice 0
        ops.append(Op(f"{op}_global", f"k_rows<{kern},8,{1 if wide else 2}>", rot(lambda b, fn=fn: fn(b, z1, n)),
                      xb + 4))
        ops.append(Op(f"{op}_axis1", f"k_rows_whole<{kern},{4 if wide else 8}>",
                      rot(lambda b, fn=fn, z=z: fn(b, z, rows, cols, 1)), xb + 4 * rows))
        ckern = "MinColOp" if kern == "MinOp" else kern
        ops.append(Op(f"{op}_axis0", f"k_cols<{ckern},true,16,16,true>" if wide else f"k_cols_whole<{ckern}>",
                      rot(lambda b, fn=fn, z=z: fn(b, z, 1, rows, cols)), xb + 4 * cols))
    # a flat sum of 2^24 + 3 floats from a base 4 bytes past 16-byte
    # alignment (the unaligned head and the ragged tail are folded in by the
    # first segment; the body still takes 128-bit loads)
    from cortexmind_amd._lib import call as _call

    rag = [D((n + 8,), np.float32) for _ in range(nbuf)]
    for b in rag:
        _call("cxm_memcpy_d2d", b.ptr + 4, bufs[0].ptr, xb, None)
    ops.append(Op("sum_flat_ragged_unaligned", "k_rows<SumOp,8,2>",
                  lambda k: _call("cxm_reduce_sum_flat_f32", rag[k % nbuf].ptr + 4, z1.ptr, n + 3, None), xb + 12 + 4))
    X = c3_affine()[0]
    big = X.size
    xs = [D.from_numpy(X) for _ in range(2)]
    ys = [D((big,), np.float32) for _ in range(2)]
    W = E.wise
    for nm, fname in (("sqrt", "FSqrt"), ("exp", "FExp"), ("sin", "FSin"), ("erf", "FErf")):
        f = getattr(W, nm)
        ops.append(Op(f"wise_{nm}", f"k_map4<{fname}>", lambda k, f=f: f(xs[k % 2], ys[k % 2], big), 8 * big))
    ops.append(Op("wise_pow_scalar", "k_map4<ScalarF<6>>", lambda k: W.pow(xs[k % 2], 2.5, ys[k % 2], big), 8 * big))
    ops.append(Op("wise_pow_tensor", "k_zip4<BinF<6>>", lambda k: W.pow(xs[k % 2], xs[(k + 1) % 2], ys[k % 2], big),
                  12 * big))
    ops.append(Op("wise_lerp", "k_map4<FLerp>", lambda k: W.lerp(xs[k % 2], 3.0, 0.25, ys[k % 2], big), 8 * big))
    desc = {"workload": "reductions min/argmin/norm1/norm2/var/stdv on fp32 [4096,4096] and elementwise "
                        "math on fp32 [8192,8192]", "ops": [o.name for o in ops]}
    return ops, desc, (bufs, rag, z1, zf, zi, xs, ys), x


def wl_g16(E, D):
    """bf16 / fp16 matmul (cxm_matmul_t, row-major NN, the CUDA path's 16-bit
    cublasGemmEx): 8192^3 in both types, 4096^3 and the MLP-like
    4096x1024x1024 in bf16.  Synthetic U(-1, 1) inputs truncated to 16 bits."""
    from cortexmind_amd._lib import DT_BF16, DT_F16

    rng = np.random.default_rng(16)

    def rand16(shape, dt):
        f = rng.random(shape, dtype=np.float32) * 2 - 1
        if dt == DT_BF16:
            return D.from_numpy((f.view(np.uint32) >> 16).astype(np.uint16))
        return D.from_numpy(f.astype(np.float16).view(np.uint16))

    shapes = [("bf16_nn_8192", DT_BF16, 8192, 8192, 8192), ("f16_nn_8192", DT_F16, 8192, 8192, 8192),
              ("bf16_nn_4096", DT_BF16, 4096, 4096, 4096), ("bf16_nn_4096x1024x1024", DT_BF16, 4096, 1024, 1024)]
    ops, keep = [], []
    for name, dt, m, k, n in shapes:
        a, b, c = rand16((m, k), dt), rand16((k, n), dt), D((m, n), np.uint16)
        keep += [a, b, c]
        # the automatic choice for these NN shapes: the 256 ring at >= 128
        # tiles of 256x256, else the 128 ring (B read as stored by both)
        tm = 256 if (m // 256) * (n // 256) >= 128 else 128
        kern = f"k_gemm16_ring<{1 if dt == DT_BF16 else 2},{tm},false>"
        ops.append(Op(name, kern, lambda i, a=a, b=b, c=c, m=m, k=k, n=n, dt=dt: E.matrix_t.matmul_t(a, b, c, m, k, n, dt),
                      2 * m * n * k, unit="FLOP", peak=PEAK_BF16_TFLOPS))
    desc = {"workload": "bf16/fp16 matmul NN (8192^3 bf16 and fp16, 4096^3 and 4096x1024x1024 bf16)",
            "ops": [o.name for o in ops], "shapes": [list(s[2:]) for s in shapes]}
    return ops, desc, tuple(keep), shapes


def torch_gemm16(shapes, steps):
    """torch.matmul (hipBLASLt) on the same shapes, for comparison."""
    import torch

    out = {}
    for name, dt, m, k, n in shapes:
        td = torch.bfloat16 if name.startswith("bf16") else torch.float16
        a = torch.rand(m, k, device="cuda").to(td)
        b = torch.rand(k, n, device="cuda").to(td)
        c = torch.empty(m, n, device="cuda", dtype=td)
        for _ in range(3):
            torch.matmul(a, b, out=c)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            torch.matmul(a, b, out=c)
        e1.record()
        e1.synchronize()
        ms = e0.elapsed_time(e1) / steps
        out[name] = {"avg_ms": round(ms, 5), "TFLOP/s": round(2 * m * n * k / (ms * 1e-3) / 1e12, 2)}
    return out


WORKLOADS = {"c1": wl_c1, "c2": wl_c2, "c3": wl_c3, "c4": wl_c4, "c5": wl_c5, "more": wl_more, "g16": wl_g16}


# ------------------------------------------------------------------ timing

def measured_peaks(E, D, Event, sync, reps=5):
    """Measured bandwidth ceilings to read the HBM figures against, beside
    the 8 TB/s specification, over 1 GiB of fp32: a copy (this library's
    streaming map z = x * 1, the bytes of a copy; the runtime's
    device-to-device hipMemcpy is reported beside it and runs slower) and a
    read (the row sum of [16384, 16384], output 64 KiB), each the mean of
    `reps` launches between events after two untimed ones."""
    from cortexmind_amd._lib import OP_MUL, call

    n = 16384
    a, b, z = D((n * n,)), D((n * n,)), D((n,))
    call("cxm_memset", a.ptr, 0, a.nbytes, None)
    res = {}
    for name, fn, nbytes in [("copy", lambda: call("cxm_scalar_f32", a.ptr, 1.0, b.ptr, n * n, OP_MUL, None),
                              2 * a.nbytes),
                             ("hipmemcpy_d2d", lambda: call("cxm_memcpy_d2d", b.ptr, a.ptr, a.nbytes, None),
                              2 * a.nbytes),
                             ("read", lambda: E.reduce.sum(a, z, n, n, 1), a.nbytes + z.nbytes)]:
        for _ in range(2):
            fn()
        sync()
        t0, t1 = Event(), Event()
        t0.record()
        for _ in range(reps):
            fn()
        t1.record()
        t1.sync()
        ms = t0.elapsed_ms(t1) / reps
        t0.close()
        t1.close()
        res[f"{name}_GBps"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
    del a, b, z
    res["sample"] = ("1 GiB fp32: copy = cxm_scalar_f32 z = x * 1 and hipmemcpy_d2d = cxm_memcpy_d2d (bytes read + "
                     f"written), read = row sum of [16384, 16384]; mean of {reps} launches each")
    return res


def time_steps(ops, steps, warmup, Event, sync):
    """Whole steps: warm-up, then events around `steps` steps."""
    k = 0
    for _ in range(warmup):
        for o in ops:
            o.fn(k)
            k += 1
    sync()
    t0, t1 = Event(), Event()
    t0.record()
    for _ in range(steps):
        for o in ops:
            o.fn(k)
            k += 1
    t1.record()
    t1.sync()
    ms = t0.elapsed_ms(t1)
    t0.close()
    t1.close()
    return ms


def time_op(op, launches, Event, sync, lead=4, warm=30):
    """Average time of one op from events around `launches` back-to-back
    launches of it alone (inputs rotating).  `warm` untimed launches run
    first: the first ~10 launches of an op after other work ran up to 14%
    slower (C4 forward at [64, 131072]: 12.5 against 11.0 us over 100
    launches after two warm-up calls; the same settles after a few).  `lead`
    untimed launches are queued just before the start event, so the timed
    launches begin on a busy queue rather than after the host's first
    enqueue (which added up to 0.8 us per launch to a 12 us kernel over 50
    launches)."""
    for k in range(warm):
        op.fn(k)
    sync()
    t0, t1 = Event(), Event()
    for k in range(lead):
        op.fn(k)
    t0.record()
    for k in range(launches):
        op.fn(k)
    t1.record()
    t1.sync()
    ms = t0.elapsed_ms(t1) / launches
    t0.close()
    t1.close()
    return ms


def rate(work, ms, unit):
    return work / (ms * 1e-3) / (1e9 if unit == "B" else 1e12)


def read_traffic():
    """kernel -> (fetch_bytes, write_bytes) per launch from
    profiles/pmc_traffic.txt (kernel names without spaces; a `[grid=...]`
    suffix is dropped, the first line of a name counts)."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.txt")
    out = {}
    if os.path.exists(path):
        for line in open(path):
            parts = line.split()
            if len(parts) >= 3 and not line.startswith("#"):
                try:
                    out.setdefault(parts[0].split("[grid=")[0], (float(parts[1]), float(parts[2])))
                except ValueError:
                    pass
    return out


def stream_floors(E, D, Event, sync, launches=100):
    """Single-launch floors at the headline's and C4's sizes, from this
    library's fastest streaming kernels, each timed like an op (events
    around `launches` back-to-back launches, inputs rotating over ten
    buffers of 64 MiB): a 64 MiB read (the row sum of [4096, 4096],
    k_rows_whole, 16 KiB output), a 32 MiB in / 32 MiB out copy (z = x * 1,
    k_map4 in its 1 KiB-piece layout) and a 64 MiB in / 32 MiB out zip
    (z = x + y, k_zip4).  Every launch pays the kernel boundary (about
    1.1-1.2 us between one launch's last workgroup and the next one's
    first) on top of its streaming time, as the ops do."""
    from cortexmind_amd._lib import OP_ADD, OP_MUL, call

    n, nbuf = 4096 * 4096, 10
    half = n // 2
    bufs = [D((n,)) for _ in range(nbuf)]
    for b in bufs:
        call("cxm_memset", b.ptr, 0, b.nbytes, None)
    z = D((4096,))
    defs = [
        ("read_64MiB", "k_rows_whole<SumOp,8>", 4 * n + 4 * 4096,
         lambda k: E.reduce.sum(bufs[k % nbuf], z, 4096, 4096, 1)),
        ("copy_32MiB_in_32MiB_out", "k_map4<ScalarF<2>>", 8 * half,
         lambda k: call("cxm_scalar_f32", bufs[k % nbuf].ptr, 1.0, bufs[(k + 5) % nbuf].ptr, half, OP_MUL, None)),
        ("zip_64MiB_in_32MiB_out", "k_zip4<BinF<0>>", 12 * half,
         lambda k: call("cxm_binary_f32", bufs[k % nbuf].ptr, bufs[k % nbuf].ptr + 4 * half,
                        bufs[(k + 5) % nbuf].ptr, half, OP_ADD, None)),
    ]
    res = {}
    for name, kern, nbytes, fn in defs:
        ms = time_op(Op(name, kern, fn, nbytes), launches, Event, sync)
        res[name] = {"avg_ms": round(ms, 5), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1), "kernel": kern,
                     "bytes": nbytes}
    del bufs, z
    return res


def frac_of_floor(per_op, ops_floor, floors):
    """Each op's GB/s over its floor's GB/s."""
    return {name: round(per_op[name]["GB/s"] / floors[f]["GB/s"], 4) for name, f in ops_floor.items()
            if name in per_op}


def cold_steps(ops, steps, Event, sync):
    """`steps` whole steps from an idle queue with no warm-up before them
    (the first call of each kernel loads it, and the first call of an op
    may grow the stream's scratch): {total ms per step, first step ms, ms
    per step of the rest}, from events between the steps."""
    sync()
    ev = [Event() for _ in range(steps + 1)]
    ev[0].record()
    for k in range(steps):
        for o in ops:
            o.fn(k)
        ev[k + 1].record()
    ev[-1].sync()
    total = ev[0].elapsed_ms(ev[-1])
    first = ev[0].elapsed_ms(ev[1])
    for e in ev:
        e.close()
    return {"ms_per_step": round(total / steps, 5), "first_step_ms": round(first, 5),
            "rest_ms_per_step": round((total - first) / (steps - 1), 5)}


def run_workload(name, steps, warmup, E, D, Event, sync):
    ops, desc, keep, host = WORKLOADS[name](E, D)
    cold = cold_steps(ops, 10, Event, sync) if name == "c5" else None
    total_ms = time_steps(ops, steps, warmup, Event, sync)
    step_work = sum(o.work for o in ops)
    unit = ops[0].unit
    per_op = {}
    launches = max(steps, 100)
    for o in ops:
        ms = time_op(o, launches, Event, sync)
        per_op[o.name] = {"avg_ms": round(ms, 5), ("GB/s" if o.unit == "B" else "TFLOP/s"): round(rate(o.work, ms, o.unit), 2)}
    extra_ops = [x for x in keep if isinstance(x, Op)]
    for o in extra_ops:
        ms = time_op(o, launches, Event, sync)
        per_op[o.name] = {"avg_ms": round(ms, 5), "TFLOP/s": round(rate(o.work, ms, o.unit), 2)}
    # dominant kernel: the one with the largest share of step time (C5: the
    # step itself, one op of five kernels)
    by_kernel = {}
    for o in ops:
        by_kernel.setdefault(o.kernel, []).append(o)
    kern, group = max(by_kernel.items(), key=lambda kv: sum(per_op[o.name]["avg_ms"] for o in kv[1]))
    avg_ms = float(np.mean([per_op[o.name]["avg_ms"] for o in group]))
    work = float(np.mean([o.work for o in group]))
    dunit = group[0].unit
    achieved = rate(work, avg_ms, dunit)
    if dunit == "B":
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4)}
    else:
        peak = group[0].peak or PEAK_FP32_TFLOPS
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak,
                "unit": "TFLOP/s", "frac": round(achieved / peak, 4)}
    known = read_traffic()
    if group[0].parts:  # an op of several kernels: the sum of its kernels' lines
        lines = [known.get(k) for k in group[0].parts]
        tr = (sum(t[0] for t in lines), sum(t[1] for t in lines)) if all(lines) else None
    else:
        tr = known.get(kern.replace(" ", ""))
    roof.update({"traffic": (tr[0] + tr[1]) if tr else None, "kernel": kern,
                 "avg_launch_ms": round(avg_ms, 5), "algorithmic_per_launch": work})
    if not tr:
        roof["traffic_note"] = "no line for this kernel in profiles/pmc_traffic.txt"
    value = rate(step_work * steps, total_ms, unit)
    out = {"value": value, "unit": "GB/s" if unit == "B" else "TFLOP/s", "ms_per_step": total_ms / steps,
           "config": desc, "roofline": roof, "per_op": per_op, "host": host,
           "kernel_of": {o.name: o.kernel for o in ops + extra_ops}}
    if cold is not None:
        out["first_10_steps"] = cold
    return out


def host_cpu():
    """lscpu's model name and the host's logical CPU count."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count()


def _pinned(fn):
    """Runs fn() on one core of this process's CPU set (the reference path
    is single-threaded); returns (fn's result, the core)."""
    old_aff = None
    core = None
    if hasattr(os, "sched_getaffinity"):
        old_aff = os.sched_getaffinity(0)
        core = min(old_aff)
        os.sched_setaffinity(0, {core})
    try:
        return fn(), core
    finally:
        if old_aff is not None:
            os.sched_setaffinity(0, old_aff)


def _time_steps_cpu(step, seconds, min_reps):
    """Warm-up, then whole steps until `seconds` have passed and at least
    `min_reps` were timed; returns (median step seconds, reps, total s)."""
    for f in step:
        f()
    times = []
    t0 = time.perf_counter()
    while True:
        ts = time.perf_counter()
        for f in step:
            f()
        times.append(time.perf_counter() - ts)
        if len(times) >= min_reps and time.perf_counter() - t0 >= seconds:
            break
    return float(np.median(times)), len(times), time.perf_counter() - t0


def cpu_baseline(name, host, seconds):
    """The oracle (the C restatement of the reference AVX2 path,
    oracle/cxm_oracle.c, -O3 -mavx2 -mfma) timed on one pinned host core
    over a bounded sample of the workload, in the workload's unit: the
    sample's algorithmic bytes (or FLOP) over its median time."""
    from oracle import oracle as O

    unit, min_reps = "GB/s", 3
    if name == "c2":
        x = host
        rows, cols = x.shape
        step = [lambda: O.reduce_flat("sum", x), lambda: O.reduce_flat("mean", x)]
        for op in ("sum", "mean", "max", "argmax"):
            step.append(lambda op=op: O.reduce_axis(op, x, rows, cols, 1))
        for op in ("sum", "mean", "max", "argmax"):
            step.append(lambda op=op: O.reduce_axis(op, x, 1, rows, cols))
        work = 2 * (4 * x.size + 4) + 4 * (4 * x.size + 4 * rows) + 4 * (4 * x.size + 4 * cols)
        min_reps = 5
        what = "whole C2 steps (10 reductions of fp32 [4096,4096])"
    elif name == "c1":
        x = host
        step = [lambda: O.softmax_fwd(x)]
        work = 2 * 4 * x.size
        min_reps = 20
        what = "whole C1 softmax forwards of fp32 [512,1024]"
    elif name == "c3":
        x, sc, b, dy = host
        rows = 1024  # the first 1024 of 8192 rows: the oracle streams rows, GB/s does not depend on the count
        xs, ds_ = np.ascontiguousarray(x[:rows]), np.ascontiguousarray(dy[:rows])
        n = x.shape[1]
        ys = {a: O.affine_act_fwd(xs, sc, b, a) for a in (O.ACT_RELU, O.ACT_SIGMOID, O.ACT_TANH)}
        step = [lambda a=a: O.affine_act_fwd(xs, sc, b, a) for a in ys]
        step += [lambda a=a: O.affine_act_bwd(xs, sc, ys[a], ds_, a) for a in ys]
        big = 4 * rows * n
        work = 3 * (2 * big + 2 * 4 * n) + 3 * (4 * big + 3 * 4 * n)
        what = (f"C3 steps on rows 0..{rows - 1} of [8192,8192] (affine fwd and bwd for relu, sigmoid, tanh; "
                "sigmoid and tanh by libm expf / tanhf, the reference's SVML being unavailable)")
    elif name == "c4":
        x, dy = host
        y, yl = O.softmax_fwd(x), O.softmax_fwd(x, True)
        step = [lambda: O.softmax_fwd(x), lambda: O.softmax_fwd(x, True), lambda: O.softmax_bwd(y, dy),
                lambda: O.softmax_bwd(yl, dy, True)]
        big = 4 * x.size
        work = 2 * big + 2 * big + 3 * big + 3 * big
        what = "whole C4 steps (softmax and log-softmax fwd + bwd of fp32 [64,131072])"
    elif name == "c5":
        x, labels, params = host
        p = {k: v.copy() for k, v in params.items()}
        step = [lambda: O.mlp_step(x, labels, p, 0.01)]
        work, unit = MLP_FLOP_PER_STEP, "TFLOP/s"
        what = "whole C5 training steps (batch 4096, 784-1024-1024-10, SGD)"
    else:
        return None
    (med, reps, dt), core = _pinned(lambda: _time_steps_cpu(step, seconds, min_reps))
    model, nproc = host_cpu()
    value = work / med / (1e9 if unit == "GB/s" else 1e12)
    return {"value": round(value, 4), "unit": unit, "cores": 1, "kind": "port",
            "sample": f"median of {reps} {what} timed over {dt:.1f} s, oracle/cxm_oracle.c -O3 -mavx2 -mfma, "
                      f"1 thread pinned to core {core}",
            "cpu_model": model, "host_nproc": nproc}


def main():
    args = parse()
    if args.summarize:
        summarize(args.summarize[0], args.summarize[1:])
        return
    if args.timeline == "c2":
        timeline()
        return
    if args.timeline == "c5":
        timeline_mlp()
        return
    if args.timeline == "c4":
        timeline_softmax()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU only (every GPU box here has one); "
                                   "--gpus must be 1", "n_gpus": args.gpus}))
        sys.exit(2)

    torch_ok = False
    if args.workload == "g16":
        # torch (for the hipBLASLt comparison) brings its own HIP runtime; it
        # must initialise before this library's runtime is loaded
        try:
            import torch

            torch.cuda.init()
            torch_ok = torch.cuda.is_available()
        except Exception:  # the comparison is optional
            torch_ok = False
    from cortexmind_amd import engine as E
    from cortexmind_amd._lib import call
    from cortexmind_amd.device import DeviceArray as D
    from cortexmind_amd.device import Event, device_count, device_info

    if device_count() < 1:
        print(json.dumps({"error": "no HIP device visible"}))
        sys.exit(1)
    info = device_info()
    sync = lambda: call("cxm_device_sync")  # noqa: E731

    if args.copy_calibration:
        a, b = D((16 << 20,)), D((16 << 20,))
        for _ in range(3):
            call("cxm_memcpy_d2d", b.ptr, a.ptr, a.nbytes, None)
        sync()
        del a, b

    head = run_workload(args.workload, args.steps, args.warmup, E, D, Event, sync)
    out = {
        "metric": METRIC if args.workload != "c5" else "fp32 MLP training step TFLOP/s on 1 MI355X",
        "value": round(head["value"], 2), "unit": head["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16/f16" if args.workload == "g16" else "f32",
        "data": "synthetic",
        "config": head["config"], "roofline": head["roofline"], "per_op": head["per_op"],
        "kernel_of": head["kernel_of"], "device": info,
    }
    if "first_10_steps" in head:
        out["first_10_steps"] = head["first_10_steps"]
    floors = None
    if head["unit"] == "GB/s":
        out["frac_of_peak"] = round(head["value"] / PEAK_HBM_GBS, 4)
        mp = measured_peaks(E, D, Event, sync)
        mp["value_frac_of_read"] = round(head["value"] / mp["read_GBps"], 4)
        mp["roofline_frac_of_read"] = round(head["roofline"]["achieved"] / mp["read_GBps"], 4)
        floors = stream_floors(E, D, Event, sync)
        mp["single_launch_floors"] = floors
        if args.workload == "c2":
            # every C2 op reads 64 MiB once: its fraction of the 64 MiB read floor
            mp["per_op_frac_of_read_floor"] = frac_of_floor(head["per_op"], {o: "read_64MiB"
                                                                              for o in head["per_op"]}, floors)
        out["measured_peaks"] = mp
    if not args.no_cpu and head["host"] is not None:
        cb = cpu_baseline(args.workload, head["host"], args.cpu_seconds)
        if cb is not None:
            out["cpu_baseline"] = cb
    if args.workload == "g16" and torch_ok:
        out["reference_torch_hipblaslt"] = torch_gemm16(head["host"], args.steps)
    if not args.no_extra:
        wl = {}
        for name in [w for w in ["c1", "c3", "c4", "c5", "more", "g16"] if w != args.workload]:
            # Untimed warm-up of each extra workload: the MLP step runs its
            # first ~100 steps (~35 ms) up to 13% slower on a box that has
            # just run bandwidth work (5 steps: 0.398 ms, 25: 0.370, 100 and
            # after: 0.351), so it gets 100; the others 10.
            r = run_workload(name, max(20, args.steps // 2), 100 if name == "c5" else 10, E, D, Event, sync)
            wl[name] = {"workload": r["config"]["workload"], "value": round(r["value"], 2),
                        "unit": r["unit"], "ms_per_step": round(r["ms_per_step"], 5),
                        "roofline": r["roofline"], "per_op": r["per_op"], "kernel_of": r["kernel_of"]}
            if r["unit"] == "GB/s" and "measured_peaks" in out:
                wl[name]["frac_of_measured_copy"] = round(r["value"] / out["measured_peaks"]["copy_GBps"], 4)
            if name == "c4" and floors:
                # forward: 32 MiB in, 32 MiB out; backward: 64 MiB in, 32 MiB out
                wl[name]["per_op_frac_of_floor"] = frac_of_floor(
                    r["per_op"], {"softmax_fwd": "copy_32MiB_in_32MiB_out", "logsoftmax_fwd": "copy_32MiB_in_32MiB_out",
                                  "softmax_bwd": "zip_64MiB_in_32MiB_out", "logsoftmax_bwd": "zip_64MiB_in_32MiB_out"},
                    floors)
            if "first_10_steps" in r:
                wl[name]["first_10_steps"] = r["first_10_steps"]
            if "note" in r["config"]:
                wl[name]["note"] = r["config"]["note"]
            if not args.no_cpu and name in ("c1", "c3", "c4", "c5"):
                wl[name]["cpu_baseline"] = cpu_baseline(name, r["host"], args.cpu_seconds_other)
            del r
        out["workloads"] = wl
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
