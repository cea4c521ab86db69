"""The vendor comparison point: a problem set run by hipBLASLt (grouped GEMM and one GEMM per
problem) next to this library on the same buffers, by the program bench/vendor_hipblaslt.cpp
(built into _build/bin/vendor_hipblaslt).

It runs as a child process because PyTorch-ROCm ships its own libhipblaslt.so.1: in a process
that has imported torch, every later library binds to that copy, whose C++ classes do not match
the ROCm headers the program is compiled against.  The grouped GEMM library never calls it."""
from __future__ import annotations

import json
import subprocess
import tempfile
from pathlib import Path
from typing import Optional

EXE = Path(__file__).resolve().parent / "_build" / "bin" / "vendor_hipblaslt"


def spec_text(spec) -> str:
    """The program's problem-set file for a workloads.WorkloadSpec."""
    lines = [f"seed {int(spec.seed)}"]
    if spec.ab_dist[0] == "uniform":
        lines.append(f"ab uniform {spec.ab_dist[1]!r} {spec.ab_dist[2]!r}")
    else:
        lines.append(f"ab normal {spec.ab_dist[1]!r}")
    if spec.c_dist is None:
        lines.append("c none")
    elif spec.c_dist[0] == "uniform":
        lines.append(f"c uniform {spec.c_dist[1]!r} {spec.c_dist[2]!r}")
    else:
        lines.append("c zero")
    lines.append(f"problems {spec.count}")
    for i in range(spec.count):
        lines.append(f"p {int(spec.m[i])} {int(spec.n[i])} {int(spec.k[i])} {float(spec.alpha[i])!r} "
                     f"{float(spec.beta[i])!r}")
    return "\n".join(lines) + "\n"


def run(spec, steps: int = 20, warmup: int = 5, check: bool = True, config: str = "128x64x32",
        sort_mode: int = 1, timeout: Optional[float] = 300) -> dict:
    """Runs the comparison program on `spec`; returns its JSON result."""
    if not EXE.exists():
        raise RuntimeError(f"{EXE} is not built (grouped_gemm_gpu_kernel_amd.build.build_vendor_baseline)")
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "problems.txt"
        path.write_text(spec_text(spec))
        cmd = [str(EXE), str(path), "--steps", str(steps), "--warmup", str(warmup), "--config", config,
               "--sort-mode", str(int(sort_mode))]
        if not check:
            cmd.append("--no-check")
        out = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    if out.returncode != 0:
        raise RuntimeError(f"vendor_hipblaslt exited with {out.returncode}: {out.stdout[-2000:]}{out.stderr[-2000:]}")
    return json.loads(out.stdout.strip().splitlines()[-1])
