"""Writes tests/golden/published_bench_rows.json from the reference's published benchmark CSV
(bench/results_20260331/results.csv): every row (workload, macro-tile, problem count, seed,
persistent grid, sort mode) with its tile total, grid, launch count, static tail share and the
kernel time / TFLOP/s pair.  Data only; run in the build container where the reference is mounted:
    python tests/golden/make_published.py
"""
import csv
import json
from pathlib import Path

SRC = Path("/root/reference/bench/results_20260331/results.csv")
OUT = Path(__file__).resolve().parent / "published_bench_rows.json"

INT_FIELDS = ("run_id", "problems", "warmup", "iters", "seed", "persistent_ctas", "tiles", "grid_ctas", "launches")
FLOAT_FIELDS = ("prep_ms", "kernel_ms", "tflops", "tail_share")


def main():
    rows = []
    with SRC.open() as f:
        for r in csv.DictReader(f):
            row = {"workload": r["workload"], "config": r["config"], "mode": r["mode"]}
            row.update({k: int(r[k]) for k in INT_FIELDS})
            row.update({k: float(r[k]) for k in FLOAT_FIELDS})
            rows.append(row)
    out = {"source": "bench/results_20260331/results.csv", "rows": rows}
    OUT.write_text(json.dumps(out, separators=(",", ":")).replace("},{", "},\n{") + "\n")


if __name__ == "__main__":
    main()
