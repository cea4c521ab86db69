"""The benchmark harness (grouped_gemm_gpu_kernel_amd/bench/benchmark_grouped_gemm.cpp) against the
reference's bench/benchmark_grouped_gemm.cu: command line, header lines, the results table, the
fixed-output cache, and -- on the GPU -- the published tile totals, tail shares and launch counts
(bench/results_20260331/results.csv), which fix the problem sets the harness generates.

CPU tests cover the command line (parsed before any GPU call) and the binary16 conversion the
harness rounds its operands with; GPU tests run the harness as a child process."""
import json
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

ROOT = Path(__file__).resolve().parents[1]
EXE = ROOT / "grouped_gemm_gpu_kernel_amd" / "_build" / "bin" / "benchmark_grouped_gemm"
BENCH_SRC = ROOT / "grouped_gemm_gpu_kernel_amd" / "bench"
PUBLISHED = json.loads((ROOT / "tests" / "golden" / "published_bench_rows.json").read_text())["rows"]
MODES = ["none", "sort_by_k", "sort_by_tiles", "sort_by_tiles_then_k", "baseline_per_problem"]
USAGE_FIRST = "Usage: "


@pytest.fixture(scope="module")
def exe():
    if not EXE.exists():
        from grouped_gemm_gpu_kernel_amd import build

        build.build_bench_driver()
    return EXE


def run(exe, *args, timeout=100):
    print("benchmark_grouped_gemm", *args, flush=True)
    return subprocess.run([str(exe), *map(str, args)], capture_output=True, text=True, timeout=timeout)


# ---------------------------------------------------------------- command line (CPU)

@pytest.mark.parametrize("args, message", [
    (["--help"], None),
    (["-h"], None),
    (["--bogus"], "Unknown option: --bogus"),
    (["--problems"], "Missing value for --problems"),
    (["--config", "256x128x64"], "Unsupported config: 256x128x64"),
    (["--tensor-cores", "maybe"], "Unsupported --tensor-cores mode: maybe"),
    (["--problems", "4", "--fixed-output"], "Missing value for --fixed-output"),
])
def test_command_line_errors_print_usage_and_fail(exe, args, message):
    """bench/benchmark_grouped_gemm.cu:125-233 and :694-698: --help, unknown options, missing values
    and unsupported names print the usage text on stdout and exit with status 1."""
    out = run(exe, *args)
    assert out.returncode == 1
    assert out.stdout.startswith(USAGE_FIRST)
    for flag in ("--problems N", "--warmup N", "--iters N", "--seed N", "--workload NAME", "--config NAME",
                 "--persistent-ctas N", "--tensor-cores MODE", "--fixed-output PATH"):
        assert flag in out.stdout
    if message:
        assert message in out.stderr


def test_host_half_conversion_matches_numpy(tmp_path):
    """The harness rounds its operands to binary16 with host_float_to_half_rn; numpy's float16 cast
    is round-to-nearest-even.  Checked on every binary16 value, the midpoints between neighbours and
    one float ulp either side of them, and a million random float bit patterns."""
    probe = tmp_path / "half_probe.cpp"
    probe.write_text(
        '#include <cstdio>\n#include <cstdint>\n#include <vector>\n#include "host_half.h"\n'
        "int main() {\n  std::vector<uint32_t> in;\n  uint32_t x;\n"
        "  while (std::fread(&x, 4, 1, stdin) == 1) in.push_back(x);\n"
        "  for (uint32_t v : in) { float f; std::memcpy(&f, &v, 4);\n"
        "    uint16_t h = host_float_to_half_rn(f); std::fwrite(&h, 2, 1, stdout); }\n  return 0;\n}\n")
    binary = tmp_path / "half_probe"
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{BENCH_SRC}", str(probe), "-o", str(binary)], check=True)
    halves = np.arange(0x7c00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = ((halves[:-1].astype(np.float64) + halves[1:]) / 2).astype(np.float32)
    bits = np.concatenate([halves.view(np.uint32), mids.view(np.uint32), mids.view(np.uint32) - 1,
                           mids.view(np.uint32) + 1, np.float32([65504, 65519.996, 65520, 1e6]).view(np.uint32)])
    bits = np.concatenate([bits, bits | 0x80000000,
                           np.random.default_rng(3).integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32)])
    finite = np.isfinite(bits.view(np.float32))
    bits = bits[finite]
    got = np.frombuffer(subprocess.run([str(binary)], input=bits.tobytes(), capture_output=True, check=True).stdout,
                        np.uint16)
    with np.errstate(over="ignore"):
        want = bits.view(np.float32).astype(np.float16).view(np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(bits[i]), hex(got[i]), hex(want[i])) for i in bad[:5]]


# ---------------------------------------------------------------- table and header parsing

def parse_table(stdout: str):
    lines = stdout.splitlines()
    head = next(i for i, line in enumerate(lines) if line.startswith("mode"))
    assert lines[head].split() == ["mode", "prep_ms", "kernel_ms", "tflops", "tiles", "grid_ctas", "launches",
                                   "tail_share"]
    rows = {}
    for line in lines[head + 1:]:
        if not line.strip():
            continue
        f = line.split()
        # setw(24) mode then fixed-width numeric columns, three decimals for the float columns
        assert re.fullmatch(r".{24}.{12}.{12}.{12}.{12}.{12}.{14}.{14}", line), line
        assert all(re.fullmatch(r"-?\d+\.\d{3}", v) for v in (f[1], f[2], f[3], f[7])), line
        rows[f[0]] = {"prep_ms": float(f[1]), "kernel_ms": float(f[2]), "tflops": float(f[3]), "tiles": int(f[4]),
                      "grid_ctas": int(f[5]), "launches": int(f[6]), "tail_share": float(f[7])}
    assert list(rows) == MODES
    return rows


def check_header(stdout: str, workload, problems, warmup, iters, cta, persistent=0, tc="on"):
    lines = stdout.splitlines()
    assert lines[0] == f"Workload: {workload}, problems={problems}, warmup={warmup}, iters={iters}"
    assert lines[1] == (f"Kernel config: CTA({cta[0]}, {cta[1]}, {cta[2]}), threads=256, "
                        f"persistent_ctas={persistent}, tensor_cores_requested={tc}")
    assert lines[2] == f"Runtime mode: tensor_cores_enabled={'yes' if tc == 'on' else 'no'}"
    assert re.fullmatch(r"Occupancy: active_blocks_per_sm=\d+, max_blocks_per_sm=\d+, sm_count=256, "
                        r"theoretical=\d+\.\d\d%", lines[3]), lines[3]
    assert re.fullmatch(r"Register pressure: estimated_regs_per_thread=\d+, measured_regs_per_thread=\d+, "
                        r"regs_per_block=\d+, register_limited_blocks_per_sm=\d+", lines[4]), lines[4]
    assert re.fullmatch(r"Shared memory: static=\d+B, dynamic=\d+B", lines[5]), lines[5]


def published(workload, config, problems=256, seed=42, persistent=0):
    rows = {r["mode"]: r for r in PUBLISHED if r["workload"] == workload and r["config"] == config
            and r["problems"] == problems and r["seed"] == seed and r["persistent_ctas"] == persistent}
    assert list(rows) == MODES
    return rows


# ---------------------------------------------------------------- GPU runs

@pytest.mark.gpu
@pytest.mark.parametrize("workload", ["small", "tail"])
@pytest.mark.parametrize("config", ["64x64x16", "128x64x32", "64x128x32"])
def test_published_columns(exe, workload, config):
    """Same flags as the published grid runs (bench/results_20260331/results.csv:2-46): the tiles,
    launches and tail_share columns equal the published ones in every mode, and TFLOP/s x kernel ms
    equals the FLOPs of the oracle's problem set, so the harness multiplies the reference's shapes."""
    cta = [int(x) for x in config.split("x")]
    out = run(exe, "--workload", workload, "--problems", 256, "--seed", 42, "--warmup", 1, "--iters", 3,
              "--config", config)
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-2000:]
    check_header(out.stdout, workload, 256, 1, 3, cta)
    rows = parse_table(out.stdout)
    want = published(workload, config)
    m, n, k = O.bench_shapes(workload, 256, 42)
    gflop = O.total_flops(m, n, k) / 1e9
    for mode in MODES:
        got, ref = rows[mode], want[mode]
        assert (got["tiles"], got["launches"], got["tail_share"]) == (ref["tiles"], ref["launches"],
                                                                      ref["tail_share"]), (mode, got, ref)
        assert got["kernel_ms"] > 0
        t, ms = got["tflops"], got["kernel_ms"]
        assert (t - 5e-4) * (ms - 5e-4) <= gflop <= (t + 5e-4) * (ms + 5e-4), (mode, got, gflop)
    assert rows["baseline_per_problem"]["grid_ctas"] == 0 and rows["baseline_per_problem"]["prep_ms"] == 0
    assert all(rows[m]["grid_ctas"] > 0 for m in MODES[:4])


@pytest.mark.gpu
def test_persistent_grid_and_tensor_cores_off(exe):
    """--persistent-ctas N fixes the grid column at N (results.csv:106-145 sweep) and
    --tensor-cores off runs the FMA path (Runtime mode line reads no)."""
    out = run(exe, "--workload", "tail", "--problems", 512, "--seed", 42, "--warmup", 1, "--iters", 2,
              "--config", "128x64x32", "--persistent-ctas", 24, "--tensor-cores", "off")
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-2000:]
    check_header(out.stdout, "tail", 512, 1, 2, (128, 64, 32), persistent=24, tc="off")
    rows = parse_table(out.stdout)
    want = published("tail", "128x64x32", problems=512, persistent=24)
    for mode in MODES[:4]:
        assert rows[mode]["grid_ctas"] == 24
        assert (rows[mode]["tiles"], rows[mode]["tail_share"]) == (want[mode]["tiles"], want[mode]["tail_share"])


def read_cache(path: Path):
    lines = path.read_text().splitlines()
    assert lines[0] == "magic grouped_gemm_fixed_output_v1"
    assert lines[1].startswith("fingerprint v2;")
    assert lines[2] == "result_count 5"
    assert [line.split()[1] for line in lines[3:]] == MODES
    return dict(kv.split("=", 1) for kv in lines[1].split(" ", 1)[1].split(";")[1:])


@pytest.mark.gpu
def test_fixed_output_cache_round_trip(exe, tmp_path):
    """bench/benchmark_grouped_gemm.cu:237-364 and :724-733: a run with --fixed-output writes the
    v1 cache (creating missing directories); a later run with the same fingerprint prints the cached
    table without running; changing any fingerprint field (here --iters) runs again and rewrites it."""
    cache = tmp_path / "nested" / "dir" / "cache.txt"
    args = ["--workload", "small", "--problems", 64, "--seed", 7, "--warmup", 1, "--iters", 2, "--config",
            "64x128x32", "--fixed-output", cache]
    first = run(exe, *args)
    assert first.returncode == 0, first.stdout[-2000:] + first.stderr[-2000:]
    fp = read_cache(cache)
    assert list(fp) == ["workload", "problems", "warmup", "iters", "seed", "cta_m", "cta_n", "cta_k", "threads",
                        "persistent_ctas", "tensor_cores_requested", "tensor_cores_enabled", "sm_count",
                        "active_blocks_per_sm", "registers_per_thread", "dynamic_shared_bytes"]
    assert fp["workload"] == "small" and fp["problems"] == "64" and fp["iters"] == "2" and fp["seed"] == "7"
    assert (fp["cta_m"], fp["cta_n"], fp["cta_k"], fp["threads"]) == ("64", "128", "32", "256")
    assert fp["tensor_cores_requested"] == "1" and fp["tensor_cores_enabled"] == "1" and fp["sm_count"] == "256"

    # Plant a recognisable kernel time: a cache hit must print it back unchanged.
    lines = cache.read_text().splitlines()
    f = lines[4].split()
    f[3] = "123.456"
    lines[4] = " ".join(f)
    cache.write_text("\n".join(lines) + "\n")
    second = run(exe, *args)
    assert second.returncode == 0
    rows = parse_table(second.stdout)
    assert rows["sort_by_k"]["kernel_ms"] == 123.456
    assert parse_table(first.stdout)["sort_by_k"]["tiles"] == rows["sort_by_k"]["tiles"]

    args[args.index("--iters") + 1] = 3
    third = run(exe, *args)
    assert third.returncode == 0
    assert parse_table(third.stdout)["sort_by_k"]["kernel_ms"] != 123.456
    assert read_cache(cache)["iters"] == "3"

    # A cache whose result count disagrees with its rows is ignored (and rewritten).
    cache.write_text(cache.read_text().replace("result_count 5", "result_count 6"))
    fourth = run(exe, *args)
    assert fourth.returncode == 0 and "result_count 5" in cache.read_text()
    sys.stdout.write(third.stdout)
