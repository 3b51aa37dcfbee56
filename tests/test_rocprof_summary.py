"""The rocprofv3 summary writer (host logic, no GPU): per-kernel statistics
from a kernel-trace CSV, and a commands block that names how the summary was
made even when no --command is passed."""
import csv

from spq4k import rocprof_summary


def _trace(d):
    rows = [("gemv_decode_kernel(spq4k::GemvParams)", 1000, 2000, 1), ("gemv_decode_kernel(spq4k::GemvParams)", 3000, 3500, 2),
            ("synth_kernel", 4000, 10000, 3)]
    with open(d / "1_kernel_trace.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Dispatch_Id", "Grid_Size", "Workgroup_Size"])
        for name, t0, t1, i in rows:
            w.writerow([name, t0, t1, i, 256, 64])


def test_stats_table_records_its_own_command(tmp_path):
    _trace(tmp_path)
    out = tmp_path / "s.md"
    assert rocprof_summary.main(["--stats", str(tmp_path), "--out", str(out), "--title", "t t"]) == 0
    text = out.read_text()
    block = text.split("```\n")[1]
    assert "spq4k.rocprof_summary --stats" in block and "'t t'" in block
    # two launches of 1.0 and 0.5 us, then one of 6.0 us: 7.5 us in all
    assert "| `gemv_decode_kernel` | 256 | 64 | 2 | 0.75 | 0.50 | 1.00 | 20.0 |" in text
    assert "| `synth_kernel` | 256 | 64 | 1 | 6.00 | 6.00 | 6.00 | 80.0 |" in text


def test_stats_table_keeps_given_commands(tmp_path):
    _trace(tmp_path)
    out = tmp_path / "s.md"
    rocprof_summary.main(["--stats", str(tmp_path), "--out", str(out), "--title", "t", "--command", "rocprofv3 x",
                          "--command", "summary y"])
    assert out.read_text().split("```\n")[1] == "rocprofv3 x\nsummary y\n"
