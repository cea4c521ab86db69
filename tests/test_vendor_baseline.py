"""The hipBLASLt comparison program (grouped_gemm_gpu_kernel_amd/bench/vendor_hipblaslt.cpp, run
through grouped_gemm_gpu_kernel_amd/vendor.py): it must multiply the same problems as the
library -- on the GPU its grouped and per-problem vendor results are compared element by element
with the library's D (itself held to the oracle by the parity tests) against twice the parity
bound 1e-3*sqrt(K)*max|A|*max|B|*|alpha| + 1e-6*(|beta|*max|C| + 1) -- otherwise the comparison
would time different work.  The command line and the problem-set file are checked on the CPU."""
import subprocess

import numpy as np
import pytest

from grouped_gemm_gpu_kernel_amd import vendor
from grouped_gemm_gpu_kernel_amd.workloads import custom_spec, make_spec

TEST_SHAPES = [(64, 64, 64), (45, 81, 37), (130, 17, 300), (0, 32, 16), (256, 200, 64), (7, 513, 9),
               (300, 64, 1000), (500, 240, 122)]


def _spec(shapes, **kw):
    m, n, k = (np.array(x) for x in zip(*shapes))
    cnt = len(shapes)
    return custom_spec("vendor-check", m, n, k, alpha=np.linspace(0.5, 2.0, cnt), beta=np.linspace(0.0, 1.0, cnt),
                       **kw)


def _exe():
    if not vendor.EXE.exists():
        from grouped_gemm_gpu_kernel_amd import build

        build.build_vendor_baseline()
    return vendor.EXE


def test_command_line_and_spec_file(tmp_path):
    exe = _exe()
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 2 and "usage" in out.stderr
    bad = tmp_path / "bad.txt"
    bad.write_text("problems 2\np 1 2 3 1.0 0.0\n")  # count disagrees with the lines
    out = subprocess.run([str(exe), str(bad)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 1 and "unreadable spec" in out.stdout
    text = vendor.spec_text(_spec(TEST_SHAPES[:2]))
    lines = text.splitlines()
    assert lines[:4] == ["seed 1", "ab uniform -1.0 1.0", "c uniform -1.0 1.0", "problems 2"]
    assert lines[4].split()[:4] == ["p", "64", "64", "64"] and lines[5].split()[:4] == ["p", "45", "81", "37"]
    assert vendor.spec_text(_spec(TEST_SHAPES[:1], c_dist=None)).splitlines()[2] == "c none"


def _assert_passes(row):
    assert "error" not in row, row
    chk = row["check_vs_library"]
    assert chk["pass"] and not chk["nan"], row
    assert row["kernel_ms"] > 0


@pytest.mark.gpu
@pytest.mark.parametrize("c_dist", [("uniform", -1.0, 1.0), None])
def test_vendor_matches_library_on_edge_shapes(c_dist):
    res = vendor.run(_spec(TEST_SHAPES, c_dist=c_dist), steps=3, warmup=1)
    print(res, flush=True)
    grouped, per_problem, batched = res["vendor"]
    _assert_passes(grouped)
    _assert_passes(per_problem)
    assert "not a uniform set" in batched.get("error", ""), batched
    assert res["library"]["kernel_ms"] > 0


@pytest.mark.gpu
def test_vendor_strided_batched_on_a_uniform_set():
    # Equal problems at evenly spaced addresses also run as one strided-batched hipblasLtMatmul.
    m, n, k = (np.full(4, x) for x in (256, 384, 160))
    spec = custom_spec("vendor-batched", m, n, k, alpha=np.full(4, 1.25), beta=np.full(4, 0.5))
    res = vendor.run(spec, steps=3, warmup=1)
    print(res, flush=True)
    grouped, per_problem, batched = res["vendor"]
    _assert_passes(per_problem)
    _assert_passes(batched)


@pytest.mark.gpu
def test_vendor_on_plumbing_workload_and_unsupported_set():
    # Sets holding very small problems (plumbing16 draws M, N, K from [1, 256]; a lone 1x1x1) leave
    # the vendor's grouped GEMM without an algorithm: that is reported, never a wrong answer.
    res = vendor.run(make_spec("plumbing16"), steps=3, warmup=1)
    print(res, flush=True)
    grouped, per_problem, _ = res["vendor"]
    assert "error" in grouped or grouped["check_vs_library"]["pass"], grouped
    _assert_passes(per_problem)
    res = vendor.run(_spec([(64, 64, 64), (1, 1, 1)]), steps=2, warmup=1)
    print(res, flush=True)
    grouped, per_problem, _ = res["vendor"]
    assert "error" in grouped or grouped["check_vs_library"]["pass"], grouped
    _assert_passes(per_problem)
