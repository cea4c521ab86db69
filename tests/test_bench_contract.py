"""bench.py's command-line contract: one JSON line with the fields the benchmark driver reads, and a
refusal (with a message, before any GPU work) of more than one GPU."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def run_bench(*args, timeout=240):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT, capture_output=True,
                          text=True, timeout=timeout)


def test_more_than_one_gpu_is_refused():
    proc = run_bench("--gpus", "2", timeout=120)
    assert proc.returncode == 2
    assert "one GPU only" in proc.stdout + proc.stderr
    assert proc.stdout.strip() == "" or not proc.stdout.strip().startswith("{")


@pytest.mark.gpu
def test_json_line_fields():
    proc = run_bench("--workload", "plumbing16", "--steps", "3", "--warmup", "1", "--clock-warmup", "0.05",
                     "--no-vendor", "--no-torch-op", "--no-moe-device", "--cpu-seconds", "0.5")
    assert proc.returncode == 0, proc.stderr[-2000:]
    lines = [ln for ln in proc.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, proc.stdout
    line = json.loads(lines[0])
    for key, kind in (("metric", str), ("value", float), ("unit", str), ("n_gpus", int), ("steps", int),
                      ("warmup", int), ("ms_per_step", float), ("higher_is_better", bool), ("scaling", str),
                      ("dtype", str), ("data", str), ("config", dict), ("roofline", dict),
                      ("cpu_baseline", dict)):
        assert isinstance(line[key], kind), key
    assert line["value"] > 0 and line["ms_per_step"] > 0
    assert (line["n_gpus"], line["steps"], line["warmup"]) == (1, 3, 1)
    assert line["higher_is_better"] is True
    assert line["vs_baseline"] is None
    assert line["config"]["workload"] == "plumbing16"
    # value is TFLOP/s of the set over the measured launch time
    assert line["value"] == pytest.approx(line["config"]["gflop"] / line["ms_per_step"], rel=0.02)
    roof = line["roofline"]
    assert roof["bound"] in ("hbm", "mfma") and roof["unit"] in ("GB/s", "TFLOP/s")
    # frac is printed to four decimals
    assert roof["frac"] == pytest.approx(roof["achieved"] / roof["peak"], rel=1e-3, abs=6e-5)
    assert "traffic" in roof
    cpu = line["cpu_baseline"]
    assert cpu["value"] > 0 and cpu["cores"] >= 1 and cpu["kind"] in ("port", "reference")
    assert isinstance(cpu["unit"], str) and isinstance(cpu["sample"], str)
