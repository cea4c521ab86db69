"""Writes tests/golden/published_small_seed42.json from the reference's published benchmark CSV
(bench/results_20260331/results.csv): the small workload (256 problems, seed 42) rows for the three
macro-tiles -- total tiles and the static tail share per sort mode.  Data only; run in the build
container where the reference is mounted:  python tests/golden/make_published.py
"""
import csv
import json
from pathlib import Path

SRC = Path("/root/reference/bench/results_20260331/results.csv")
OUT = Path(__file__).resolve().parent / "published_small_seed42.json"


def main():
    rows = {}
    with SRC.open() as f:
        for r in csv.DictReader(f):
            if r["workload"] != "small" or r["seed"] != "42" or r["problems"] != "256" or r["persistent_ctas"] != "0":
                continue
            if r["mode"] == "baseline_per_problem":
                continue
            cfg = r["config"]
            entry = rows.setdefault(cfg, {"config": cfg, "cta": [int(x) for x in cfg.split("x")],
                                          "tiles": int(r["tiles"]), "grid_ctas": int(r["grid_ctas"]),
                                          "tail_share": {}})
            entry["tail_share"][r["mode"]] = float(r["tail_share"])
    out = {"source": "bench/results_20260331/results.csv (small, seed 42, 256 problems)", "problems": 256,
           "seed": 42, "rows": [rows[c] for c in ("64x64x16", "128x64x32", "64x128x32")]}
    OUT.write_text(json.dumps(out, indent=1) + "\n")


if __name__ == "__main__":
    main()
