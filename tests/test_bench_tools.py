"""The measurement tools' arithmetic, on small synthetic rocprofv3 CSVs (no GPU): the per-kernel
summary (bench/rocprof_summary.py), the counter summaries (bench/pmc_summary.py: MFMA issue and busy
cycles, FETCH_SIZE / WRITE_SIZE scaled by the copy-kernel calibration) and the prefill attribution
with its sum-of-parts guard (bench/prefill_breakdown.py)."""
import csv
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench")
sys.path.insert(0, BENCH)

import pmc_summary  # noqa: E402
import rocprof_summary  # noqa: E402

TRACE_COLS = ["Kernel_Name", "Grid_Size_X", "Workgroup_Size_X", "Start_Timestamp", "End_Timestamp"]
PMC_COLS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
MLP = "void g2::k_gemm_dl<48, 32, 3, 2, 6, false, 2, 2, 0>(unsigned short*, unsigned short const*)"


def write_csv(path, cols, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(cols)
        w.writerows(rows)


def test_short_names():
    assert rocprof_summary.short(MLP) == "g2::k_gemm_dl<48, 32, 3, 2, 6, false, 2, 2, 0>"
    assert rocprof_summary.short("k_empty()") == "k_empty"


def test_rocprof_summary_groups_by_kernel_and_grid(tmp_path):
    p = tmp_path / "t.csv"
    rows = [[MLP, 256 * 768, 768, 1000, 1000 + d] for d in (9000, 10000, 11000)]
    rows += [["k_empty()", 64, 64, 0, 1300]]
    write_csv(p, TRACE_COLS, rows)
    out = rocprof_summary.summarize(str(p))
    top = out[0]
    assert top["kernel"].endswith("k_gemm_dl<48, 32, 3, 2, 6, false, 2, 2, 0>")
    assert top["work_groups"] == 256 and top["dispatches"] == 3
    assert top["mean_us"] == 10.0 and top["median_us"] == 10.0 and top["min_us"] == 9.0 and top["max_us"] == 11.0


def bench_line(path):
    shapes = [{"gemm": "mlp_proj", "M": 512, "N": 768, "K": 3072, "kernel": "dl_bn48_bm32_w3x2_s6_k2_u2", "us": 8.0}]
    with open(path, "w") as f:
        f.write("log line\n" + json.dumps({"gemm_shapes": shapes}) + "\n")


def test_pmc_traffic_scaling(tmp_path, capsys, monkeypatch):
    fetch, write, run, js = (tmp_path / n for n in ("f.csv", "w.csv", "run.json", "out.json"))
    bench_line(run)
    # the copy kernel of 1 MiB reads half its bytes in FETCH_SIZE units: scale 2; writes read 1:1
    write_csv(fetch, PMC_COLS, [[1, "k_copy16(int)", "FETCH_SIZE", 512.0, 0, 10],
                                [2, MLP, "FETCH_SIZE", 1000.0, 20, 30], [3, MLP, "FETCH_SIZE", 3000.0, 40, 50]])
    write_csv(write, PMC_COLS, [[1, "k_copy16(int)", "WRITE_SIZE", 1024.0, 0, 10], [2, MLP, "WRITE_SIZE", 768.0, 20, 30]])
    monkeypatch.setattr(sys, "argv", ["pmc_summary.py", "traffic", str(fetch), str(write), str(run), "--copy-bytes",
                                      str(1 << 20), "--json", str(js), "--source", "x.md"])
    pmc_summary.main()
    out = json.load(open(js))
    assert out["fetch_scale"] == 2.0 and out["write_scale"] == 1.0
    row = out["per_shape"]["mlp-proj 512x768x3072"]
    assert row["fetch_kib"] == 2000.0 and row["read_bytes"] == 2000 * 2 * 1024 and row["write_bytes"] == 768 * 1024
    assert row["algo_read_bytes"] == (512 * 3072 + 768 * 3072 + 768) * 2 and row["algo_write_bytes"] == 512 * 768 * 2
    assert "| mlp-proj 512x768x3072 |" in capsys.readouterr().out


def test_pmc_mfma_utilisation(tmp_path, capsys, monkeypatch):
    pmc, run = tmp_path / "p.csv", tmp_path / "run.json"
    bench_line(run)
    flop = 2 * 512 * 768 * 3072
    rows = [[1, MLP, "SQ_INSTS_VALU_MFMA_MOPS_F16", flop / 512, 0, 10000],
            [1, MLP, "SQ_VALU_MFMA_BUSY_CYCLES", flop / 1024, 0, 10000]]
    write_csv(pmc, PMC_COLS, rows)
    monkeypatch.setattr(sys, "argv", ["pmc_summary.py", "mfma", str(pmc), str(run), "--clock-mhz", "2400"])
    pmc_summary.main()
    line = [ln for ln in capsys.readouterr().out.splitlines() if "mlp-proj" in ln][0]
    cells = [c.strip() for c in line.split("|")]
    assert cells[7] == "1.000"                      # busy cycles x 1024 = FLOP: the dense rate
    assert cells[8] == "10.00"                      # kernel us from End - Start (ns)
    util = (flop / 1024) / (1024 * 10.0 * 2400)     # busy / (SIMDs x kernel cycles)
    assert cells[9] == f"{util:.3f}"


def test_prefill_attribution_and_guard(tmp_path):
    """Marker bursts split the trace into forwards; per-kernel medians, the per-forward sum, and the
    guard's three verdicts against the untraced whole."""
    trace = tmp_path / "t.csv"
    rows, t = [], 0

    def add(name, dur):
        nonlocal t
        rows.append([name, 64, 64, t, t + dur])
        t += dur + 100

    for _ in range(4):
        add("k_empty()", 1000)
        add("void g2::k_layernorm<true>(unsigned short*)", 3000)
        add(MLP, 9000)
    add("k_empty()", 1000)
    write_csv(trace, TRACE_COLS, rows)
    for whole_ms, verdict in ((0.0120, "OK"), (0.0200, "SUM < whole"), (0.0080, "SUM > whole")):
        wj = tmp_path / f"w{whole_ms}.json"
        json.dump({"backend": "int8", "T": 512, "iters": 4, "median_ms": whole_ms, "min_ms": whole_ms,
                   "max_ms": whole_ms}, open(wj, "w"))
        out = subprocess.run([sys.executable, os.path.join(BENCH, "prefill_breakdown.py"), "attribute", str(trace),
                              str(wj), "--skip", "1"], capture_output=True, text=True, check=True).stdout
        assert "3 traced forwards (4 marked, 1 skipped), 2 kernels per forward" in out
        assert "| SUM (per forward, median) | | 2 | 12.0 |" in out
        assert verdict in out, (whole_ms, out)
