"""The stage table's text, without a GPU: the reference's layout
(include/Cuda/Profiler.cuh:119-162) of a 14-wide name column and 10-wide
figure columns between dashed rules, and the rate with one decimal and a K
or M suffix from 1e3 and 1e6 up."""
from carl_amd.profiler import _rate, format_stage_table


def test_rate_suffixes():
    assert _rate(999.94) == "999.9"
    assert _rate(1000.0) == "1.0K"
    assert _rate(654_321.0) == "654.3K"
    assert _rate(1_000_000.0) == "1.0M"
    assert _rate(712_345_678.0) == "712.3M"


def test_table_layout():
    names = ["contact", "car-arena", "ball", "finish", "boost-pads"]
    profile = {
        "stages": dict(zip(names, [10.0, 20.5, 3.25, 1.0, 0.25])),
        "last_workgroup": dict(zip(names + ["start delay"], [12.0, 22.0, 3.5, 1.25, 0.25, 0.5])),
        "span_us": 39.5, "launch_us": 40.0, "ticks": 8,
    }
    lines = format_stage_table(profile, n_sim=65536).splitlines()
    assert lines[0] == "stage             us/tick    last wg"
    assert lines[1] == lines[8] == "-" * 36
    assert lines[2] == "contact            10.000     12.000"
    assert lines[6] == "boost-pads          0.250      0.250"
    assert lines[7] == "start delay                    0.500"
    assert lines[9] == "aggregate          35.000     39.500"
    assert lines[10] == "span               39.500"
    assert lines[11] == "launch             40.000"
    # 65536 simulations per tick in 40 us
    assert lines[12] == "sim ticks/s       1638.4M"
    assert len(lines) == 13


def test_rocprof_summary_windows_follow_the_steps(tmp_path, capsys):
    """bench.py's rocprof summary: set-up dispatches count in no window, and
    each kernel's timed and after windows are the dispatches between the
    packing-kernel dispatches that end env steps warmup-1, warmup+steps-1 and
    warmup+2*steps-1 (durations chosen so that each window has its own mean)."""
    import csv
    import sys
    from pathlib import Path

    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    import bench

    warmup, steps, total = 2, 3, 10
    rows, t = [], 0

    def add(name, us):
        nonlocal t
        rows.append({"Dispatch_Id": len(rows) + 1, "Kernel_Name": name,
                     "Start_Timestamp": t, "End_Timestamp": t + int(us * 1000)})
        t += 10**6

    for _ in range(4):
        add("__amd_rocclr_fillBufferAligned", 50.0)
    for step in range(total):
        window = 1 if warmup <= step < warmup + steps else 2 if warmup + steps <= step < warmup + 2 * steps else 0
        add("(anonymous namespace)::tickWindowKernel(carl::Dev, int)", 100.0 * (window + 1))
        add("(anonymous namespace)::stepEnvKernel(carl::Dev, carl::StepIO)", 10.0 * (window + 1))
        add("at::native::reward", 1.0)
    trace = tmp_path / "trace"
    trace.mkdir()
    with open(trace / "run_kernel_trace.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    bench.summarize_rocprof(str(trace), None, None, None, None, 512, steps, warmup)
    table = {line.split(" | ")[0].strip("| "): line.split(" | ")[1:]
             for line in capsys.readouterr().out.splitlines() if line.startswith("| ") and "---" not in line}
    assert table["tickWindowKernel"] == ["10", "190.0", "200.0", "300.0 |"]
    assert table["stepEnvKernel"] == ["10", "19.0", "20.0", "30.0 |"]
    assert table["__amd_rocclr_fillBufferAligned"] == ["4", "50.0", "nan", "nan |"]
    assert table["at::native::reward"][2:] == ["1.0", "1.0 |"]
