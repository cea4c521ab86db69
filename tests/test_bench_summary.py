"""bench.py's profiler summaries (CPU): the per-sort-mode split of a rocprofv3 dispatch list at the
traced grouped-kernel dispatches, the copy-calibrated HBM traffic, and the committed traffic
summaries the bench line reads its `roofline.traffic` from."""
import csv
import importlib.util
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

UNTRACED = "void gg::gg_grouped_kernel<1, 1, false, false>(gg::GroupedArgs)"
TRACED = "void gg::gg_grouped_kernel<1, 1, true, false>(gg::GroupedArgs)"
FILL = "gg::fill_f32_kernel(float*, long, float)"
COPY = "__amd_rocclr_copyBuffer"


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def write_counters(folder: Path, counter: str, rows):
    """rows: (kernel name, value) in dispatch order; each value is split over two rows of the same
    dispatch, as rocprofv3 does for counters read from several blocks."""
    folder.mkdir(parents=True)
    with open(folder / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Correlation_Id", "Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        # written out of dispatch order: the summary must order by Dispatch_Id
        for i, (name, value) in reversed(list(enumerate(rows, start=1))):
            w.writerow([i, i, name, counter, value / 4])
            w.writerow([i, i, name, counter, 3 * value / 4])


def write_trace(folder: Path, rows):
    folder.mkdir(parents=True)
    with open(folder / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        t = 1000
        for i, (name, us) in enumerate(rows, start=1):
            w.writerow([i, name, t, t + int(us * 1000)])
            t += int(us * 1000) + 500


def dispatch_rows(mode_values, after=(), traced=3):
    """bench.py's dispatch order: each mode's untraced runs, then `traced` traced runs (the
    measured tail idle is a median over several)."""
    rows = [(FILL, 7.0)]
    for vals in mode_values:
        rows += [(UNTRACED, v) for v in vals] + [(TRACED, 1e9)] * traced
    return rows + [(UNTRACED, v) for v in after]


@pytest.mark.parametrize("traced", [1, 3])
def test_segments_split_at_traced_dispatches(bench, tmp_path, traced):
    rows = dispatch_rows([[100.0, 10.0, 20.0], [50.0, 30.0, 40.0]], after=[999.0], traced=traced)
    write_trace(tmp_path / "t", rows)
    segs = bench._segments(bench._dispatches(tmp_path / "t"), r"gg_grouped_kernel<\d+,\s*\d+,\s*false",
                           ["none", "sort_by_k"], last=2)
    assert sorted(s for _, s in segs) == ["after", "none", "sort_by_k"]
    assert segs[(UNTRACED, "none")]["duration_us"] == pytest.approx([10.0, 20.0])
    assert segs[(UNTRACED, "sort_by_k")]["duration_us"] == pytest.approx([30.0, 40.0])
    assert segs[(UNTRACED, "after")]["duration_us"] == pytest.approx([999.0])
    # without mode names everything matching the kernel filter is one segment, traced runs excluded
    whole = bench._segments(bench._dispatches(tmp_path / "t"), r"gg_grouped_kernel<\d+,\s*\d+,\s*false", [], 0)
    assert whole[(UNTRACED, "all")]["duration_us"] == pytest.approx([100, 10, 20, 50, 30, 40, 999])


def test_traffic_summary_scales_by_the_copy_reading(bench, tmp_path, capsys):
    # copy of 1 MiB: FETCH_SIZE reads 512 KiB (scale 0.5), WRITE_SIZE 1024 KiB (scale 1.0)
    write_counters(tmp_path / "cf", "FETCH_SIZE", [(FILL, 1.0)] + [(COPY, 512.0)] * 3)
    write_counters(tmp_path / "cw", "WRITE_SIZE", [(FILL, 1.0)] + [(COPY, 1024.0)] * 3)
    write_counters(tmp_path / "f", "FETCH_SIZE", dispatch_rows([[9e9, 100.0, 300.0], [9e9, 50.0, 50.0]]))
    write_counters(tmp_path / "w", "WRITE_SIZE", dispatch_rows([[9e9, 40.0, 40.0], [9e9, 10.0, 30.0]]))
    dirs = [str(tmp_path / x) for x in ("f", "w", "cf", "cw")]
    assert bench.traffic_summary(dirs, 1, "plumbing16", r"gg_grouped_kernel<\d+,\s*\d+,\s*false",
                                 ["none", "sort_by_k"], 2) == 0
    out = capsys.readouterr().out
    vals = dict(re.findall(r"^(\w+(?: \w+)?): (\S+)$", out, re.M))
    assert float(vals["fetch_scale"]) == pytest.approx(0.5)
    assert float(vals["write_scale"]) == pytest.approx(1.0)
    # none: fetch mean 200 KiB / 0.5, write 40 KiB / 1.0
    assert float(vals["fetch_bytes_per_launch none"]) == pytest.approx(400 * 1024)
    assert float(vals["write_bytes_per_launch none"]) == pytest.approx(40 * 1024)
    assert float(vals["traffic_bytes_per_launch none"]) == pytest.approx(440 * 1024)
    assert float(vals["traffic_bytes_per_launch sort_by_k"]) == pytest.approx((100 + 20) * 1024)


def test_committed_traffic_files_parse(bench):
    """Every committed traffic summary: fetch + write = traffic for each mode it lists, and the bench
    reads each mode's figure back."""
    files = sorted((ROOT / "profiles").glob("gg_grouped_kernel_*_hbm_traffic.txt"))
    assert files, "no committed traffic summary"
    for path in files:
        workload = path.name[len("gg_grouped_kernel_"):-len("_hbm_traffic.txt")]
        text = path.read_text()
        assert text.startswith("# "), f"{path.name}: no header"
        assert "rocprofv3 --pmc FETCH_SIZE" in text and "rocprofv3 --pmc WRITE_SIZE" in text
        lines = dict(re.findall(r"^(\w+ \w+): (\S+)$", text, re.M))
        modes = [k.split()[1] for k in lines if k.startswith("traffic_bytes_per_launch")]
        assert modes, f"{path.name}: no per-mode traffic"
        for m in modes:
            f, w, t = (float(lines[f"{k}_bytes_per_launch {m}"]) for k in ("fetch", "write", "traffic"))
            assert abs(f + w - t) <= 2, f"{path.name} {m}: fetch + write != traffic"
            got = bench.committed_traffic(workload, m)
            assert got is not None and got["bytes"] == pytest.approx(t)


def test_headline_mode_breaks_ties_by_tail_share(bench):
    rows = [{"mode": m, "tail_share": t} for m, t in
            (("none", 0.078), ("sort_by_k", 0.0185), ("sort_by_tiles", 0.0106), ("sort_by_tiles_then_k", 0.0106))]
    # all within 1% of the fastest: the smallest static tail share wins, then the faster of equal shares
    row, ms = bench.headline_mode(rows, [0.2329, 0.2333, 0.2336, 0.2331])
    assert (row["mode"], ms) == ("sort_by_tiles_then_k", 0.2331)
    # a clearly faster mode wins whatever its tail share
    row, ms = bench.headline_mode(rows, [0.2200, 0.2333, 0.2336, 0.2331])
    assert (row["mode"], ms) == ("none", 0.2200)
