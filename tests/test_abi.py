"""The C-ABI library loads and exports every function include/*.h declares (no GPU calls), and the
ctypes binding covers each of them."""
import re
import subprocess
from pathlib import Path

from grouped_gemm_gpu_kernel_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADERS = [ROOT / "include" / "grouped_gemm_amd.h", ROOT / "include" / "grouped_gemm_amd_kernels.h"]
DECL = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*\b((?:gg|ggk)_[a-z0-9_]+)\s*\(", re.M)


def declared_functions():
    names = set()
    for h in HEADERS:
        names |= set(DECL.findall(h.read_text()))
    return names


def test_headers_declare_the_api():
    names = declared_functions()
    for required in ("gg_prepare_problem_set", "gg_executor_build", "gg_executor_run", "gg_query_occupancy",
                     "gg_run_baseline_per_problem", "gg_run_grouped_gemm_once", "ggk_launch_grouped",
                     "ggk_launch_single", "ggk_kernel_resources_get", "ggk_occupancy"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in sorted(declared_functions()):
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert declared_functions() <= exported


def test_binding_covers_every_declared_symbol():
    assert declared_functions() == set(_lib.SIGNATURES)


def test_library_links_hip_and_has_gfx950_code():
    out = subprocess.run(["ldd", str(_lib.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    assert "libamdhip64" in out
    blob = _lib.LIB_PATH.read_bytes()
    assert b"gfx950" in blob


def test_cpp_api_header_mirrors_reference_names():
    text = (ROOT / "include" / "grouped_gemm" / "grouped_gemm.h").read_text()
    for name in ("enum class SortMode", "struct ProblemDesc", "struct KernelConfig", "struct PreparedProblemSet",
                 "struct OccupancyInfo", "class GroupedGemmExecutor", "prepare_problem_set(", "sort_mode_name(",
                 "query_occupancy(", "run_grouped_gemm_once(", "run_baseline_per_problem(",
                 "count_non_empty_problems(", "DeviceProblemDesc"):
        assert name in text, name
