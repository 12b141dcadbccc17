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
