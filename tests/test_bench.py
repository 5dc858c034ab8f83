"""The output contract of bench.py: one JSON line with the headline fields,
`roofline`, `cpu_baseline` and the measured ceilings; one GPU only."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(*args, timeout=300):
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT, capture_output=True,
                       text=True, timeout=timeout)
    lines = [line for line in p.stdout.splitlines() if line.startswith("{")]
    return p.returncode, lines, p.stderr


def test_more_than_one_gpu_is_refused():
    rc, lines, _ = run_bench("--gpus", "2", timeout=120)
    assert rc == 2
    assert len(lines) == 1
    out = json.loads(lines[0])
    assert out["n_gpus"] == 2 and "one GPU" in out["error"]


@pytest.mark.gpu
def test_headline_line(hip):
    rc, lines, err = run_bench("--steps", "3", "--warmup", "1", "--no-extra", "--cpu-seconds", "1")
    assert rc == 0, err[-2000:]
    assert len(lines) == 1
    out = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline", "measured_peaks"):
        assert key in out, key
    assert out["n_gpus"] == 1 and out["steps"] == 3 and out["warmup"] == 1
    assert out["unit"] == "GB/s" and out["higher_is_better"] is True and out["dtype"] == "f32"
    assert out["vs_baseline"] is None and out["data"] == "synthetic"
    assert "C2" in out["config"]["workload"]
    # value = 10 launches of 64 MiB (plus outputs) per step over the step time
    step_bytes = 10 * 4096 * 4096 * 4
    assert out["value"] == pytest.approx(step_bytes / (out["ms_per_step"] * 1e-3) / 1e9, rel=0.01)
    assert 500.0 < out["value"] < 8000.0
    r = out["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in r, key
    assert r["bound"] == "hbm" and r["unit"] == "GB/s" and r["peak"] == 8000.0
    assert r["frac"] == pytest.approx(r["achieved"] / r["peak"], abs=1e-3)
    c = out["cpu_baseline"]
    assert c["kind"] == "port" and c["cores"] == 1 and c["unit"] == "GB/s" and c["value"] > 0 and c["sample"]
    m = out["measured_peaks"]
    assert 1000.0 < m["read_GBps"] < 8000.0 and 1000.0 < m["copy_GBps"] < 8000.0


def test_kernel_name_matches_bench_labels():
    """rocprofv3's demangled names reduce to the labels bench.py uses."""
    sys.path.insert(0, ROOT)
    from bench import kernel_name

    assert kernel_name("void cxm::(anonymous namespace)::k_cols<cxm::ArgMaxOp, true, 16, 16, true>"
                       "(float const*, unsigned long, unsigned long, unsigned int)") == "k_cols<ArgMaxOp,true,16,16,true>"
    assert kernel_name("void cxm::k_map4<cxm::(anonymous namespace)::ScalarF<2> >(cxm::(anonymous namespace)::"
                       "ScalarF<2>, float const*, float*, unsigned long)") == "k_map4<ScalarF<2>>"
    assert kernel_name("cxm::(anonymous namespace)::k_mlp_head(float const*, float const*)") == "k_mlp_head"
    assert kernel_name("__amd_rocclr_copyBuffer") == "__amd_rocclr_copyBuffer"


def _write_csv(path, header, rows):
    import csv

    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_summarize_pmc_scales_by_the_first_copies(tmp_path):
    """Counter values (KiB) scale so that the three calibration copies, the
    first copyBuffer dispatches, read and write 64 MiB; later copies do not
    change the factor."""
    hdr = ["Dispatch_Id", "Grid_Size", "Kernel_Name", "Counter_Name", "Counter_Value"]
    fetch = [[1, 131072, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 32768.0],
             [2, 131072, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 32768.0],
             [3, 131072, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 32768.0],
             [4, 1024, "void cxm::k_map4<cxm::FExp>(cxm::FExp, float const*, float*, unsigned long)", "FETCH_SIZE", 1024.0],
             [5, 131072, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 524288.0]]
    write = [[1, 131072, "__amd_rocclr_copyBuffer", "WRITE_SIZE", 65536.0],
             [2, 131072, "__amd_rocclr_copyBuffer", "WRITE_SIZE", 65536.0],
             [3, 131072, "__amd_rocclr_copyBuffer", "WRITE_SIZE", 65536.0],
             [4, 1024, "void cxm::k_map4<cxm::FExp>(cxm::FExp, float const*, float*, unsigned long)", "WRITE_SIZE", 512.0]]
    _write_csv(tmp_path / "f.csv", hdr, fetch)
    _write_csv(tmp_path / "w.csv", hdr, write)
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--summarize", "pmc", str(tmp_path / "f.csv"),
                        str(tmp_path / "w.csv")], cwd=ROOT, capture_output=True, text=True, timeout=60)
    assert p.returncode == 0, p.stderr
    lines = [ln for ln in p.stdout.splitlines() if not ln.startswith("#")]
    assert lines == ["k_map4<FExp>[grid=1024] 2097152 524288"]  # 1024 KiB x 2, 512 KiB x 1


def test_summarize_trace_table(tmp_path):
    hdr = ["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]
    name = "void cxm::(anonymous namespace)::k_rows_whole<cxm::SumOp, 8>(float const*, unsigned long)"
    _write_csv(tmp_path / "t.csv", hdr, [[name, 1000, 12000, 512, 1, 1], [name, 20000, 33000, 512, 1, 1],
                                         ["k_other", 0, 1000, 64, 2, 1]])
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--summarize", "trace", str(tmp_path / "t.csv")],
                       cwd=ROOT, capture_output=True, text=True, timeout=60)
    assert p.returncode == 0, p.stderr
    rows = [ln for ln in p.stdout.splitlines() if ln.startswith("| `")]
    assert rows[0] == "| `k_rows_whole<SumOp,8>` | 512 | 2 | 12.00 | 11.00 | 13.00 | 96.0 |"
    assert rows[1] == "| `k_other` | 128 | 1 | 1.00 | 1.00 | 1.00 | 4.0 |"


def test_timeline_report_on_synthetic_marks(capsys):
    """timeline_report's arithmetic on hand-made marks (100 MHz ticks): the
    end of a column op is its last tile's final store, stale final marks
    (earlier than the workgroup's start) are ignored, gaps run from one op's
    end to the next op's first start."""
    sys.path.insert(0, ROOT)
    import numpy as np

    from bench import TL_KINDS, TL_MARKS, TL_WGS, timeline_report

    t = np.zeros((TL_KINDS, TL_WGS, TL_MARKS), np.uint64)
    base = 10_000
    # kind 0: 8 row workgroups, start 0..7 ticks, fold +1000, end +1100
    for w in range(8):
        t[0, w] = [base + w, base + w + 1000, 0, base + w + 1100]
    # kind 1: 8 column workgroups starting 200 ticks after the rows' end
    c0 = base + 7 + 1100 + 200
    for w in range(8):
        t[1, w] = [c0 + w, c0 + 1000 + w, c0 + 1100 + w, 5]  # final mark stale (earlier launch)
    t[1, 7, 3] = c0 + 1300  # the last workgroup's final store
    timeline_report(t, [("row sum", "k_r", 0), ("column sum", "k_c", 1)], {0: 8, 1: 8})
    out = capsys.readouterr().out.splitlines()
    row = [ln for ln in out if ln.startswith("| row sum")][0].split("|")
    col = [ln for ln in out if ln.startswith("| column sum")][0].split("|")
    assert row[3].strip() == "0.00" and row[4].strip() == "0.07"
    assert row[7].strip() == "11.07"   # end: 7 + 1100 ticks
    assert row[9].strip() == "2.00"    # gap to the column op: 200 ticks
    assert col[7].strip() == f"{(c0 + 1300 - base) / 100:.2f}"
    assert col[8].strip() == "2.93"    # combine after the last fold: 1300 - 1007 ticks


def test_timeline_mlp_report_on_synthetic_marks(capsys):
    """timeline_mlp_report: prologue / loop / epilogue from the marks, the
    core clock from the s_memtime ticks over the loop's 10 ns ticks, gaps
    from one kernel's last epilogue to the next kernel's first start."""
    sys.path.insert(0, ROOT)
    import numpy as np

    from bench import GEMM_TL, HEAD_TL, timeline_mlp_report

    g = np.zeros(GEMM_TL, np.uint64)
    h = np.zeros(HEAD_TL, np.uint64)
    t = 1000
    for k in range(4):
        for w in range(8):
            g[k, w] = [t, t + 150, t + 5150, t + 5600, 7, 7 + 5000 * 23]  # 50 us loop at 2.3 GHz
        t += 6000 if k != 1 else 8000  # the head runs between the second and third product
    for w in range(4):
        h[w] = [13100, 13400, 13500, 13600, 13700, 13900, 14300, 0]
    timeline_mlp_report(g, h, {0: 8, 1: 8, 2: 8, 3: 8}, 4)
    out = capsys.readouterr().out.splitlines()
    l1 = [ln for ln in out if ln.startswith("| layer-1 forward")][0].split("|")
    assert [c.strip() for c in l1[3:11]] == ["0.00", "0.00", "1.50", "50.00 / 50.00", "4.50 / 4.50", "56.00", "2.300",
                                             "4.00"]
    hd = [ln for ln in out if ln.startswith("| output-layer head (")][0].split("|")
    assert hd[3].strip() == "121.00" and hd[8].strip() == "133.00" and hd[10].strip() == "7.00"


def test_timeline_softmax_report_on_synthetic_marks(capsys):
    sys.path.insert(0, ROOT)
    import numpy as np

    from bench import SM_TL, timeline_softmax_report

    t = np.zeros(SM_TL, np.uint64)
    for k in range(2):
        for w in range(16):
            b = 1000 + 2000 * k
            t[k, w] = [b + w, b + 10 + w, b + 900, b + 950 + (w % 2) * 100, b + 1500]
    timeline_softmax_report(t, [("fwd", "k_f", 0), ("bwd", "k_b", 1)], 16)
    out = capsys.readouterr().out.splitlines()
    f = [ln for ln in out if ln.startswith("| fwd")][0].split("|")
    assert [c.strip() for c in f[3:12]] == ["0.00", "0.15", "0.25", "15.00", "9.00 / 9.00", "10.00 / 10.50",
                                            "1.00 / 1.50", "15.00", "5.00"]
