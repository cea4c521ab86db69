"""Build recipe for the gfx950 grouped GEMM library.

Produces, in-tree:
  grouped_gemm_gpu_kernel_amd/lib/libgrouped_gemm_amd.so   the library (C-ABI + C++ API)
  grouped_gemm_gpu_kernel_amd/_build/bin/test_correctness   C++ drop-in test driver
  grouped_gemm_gpu_kernel_amd/_build/bin/benchmark_grouped_gemm   benchmark harness (reference CLI)
  grouped_gemm_gpu_kernel_amd/_build/bin/vendor_hipblaslt   hipBLASLt comparison program (bench only)
  oracle/liboracle.so                                       CPU oracle (test infrastructure)

Steps: hipcc compiles the kernels for gfx950 with the compiler's resource
report, which is parsed into a table the library links in; g++ compiles the
plain C++ host runtime; hipcc links everything into one shared library.
Usage: python -m grouped_gemm_gpu_kernel_amd.build [--no-tests] [--no-oracle]
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC_DIR = PKG / "csrc"
BUILD = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB_NAME = "libgrouped_gemm_amd.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # Packed FP32 instructions stay off (they have given wrong results on these GPUs).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}", f"-I{CSRC_DIR}",
]
CXX_FLAGS = [
    "g++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
    f"-I{ROCM / 'include'}", f"-I{ROOT / 'include'}",
]

_REMARK = re.compile(r"remark:\s+(Function Name|TotalSGPRs|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|"
                     r"Occupancy \[waves/SIMD\]|LDS Size \[bytes/block\]):\s+(\S+)")
# gg_grouped_kernel<variant, path, traced, wide> and gg_single_kernel<variant, path, wide>.
_KERNEL = re.compile(r"gg_(grouped|single)_kernelILi(\d+)ELi(\d+)ELb([01])E(Lb([01])E)?")


def _run(cmd: list[str], capture_stderr: bool = False) -> str:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd[:3])} ...")
    return proc.stderr if capture_stderr else proc.stdout


def parse_resource_report(report: str) -> list[tuple[int, ...]]:
    """Rows (kind, variant, path, vgprs, agprs, sgprs, scratch, waves, lds) for
    the untraced grouped kernels and the single-problem kernels in the 32-bit
    addressing form."""
    rows, cur = [], {}

    def flush():
        m = _KERNEL.search(cur.get("Function Name", ""))
        if not m:
            return
        kind = 0 if m.group(1) == "grouped" else 1
        if kind == 0 and (m.group(4) != "0" or m.group(6) != "0"):
            return  # traced (same code plus instrumentation) or 64-bit addressing form
        if kind == 1 and m.group(4) != "0":
            return  # 64-bit addressing form
        rows.append((kind, int(m.group(2)), int(m.group(3)), int(cur.get("VGPRs", 0)),
                     int(cur.get("AGPRs", 0)), int(cur.get("TotalSGPRs", 0)),
                     int(cur.get("ScratchSize [bytes/lane]", 0)),
                     int(cur.get("Occupancy [waves/SIMD]", 0)), int(cur.get("LDS Size [bytes/block]", 0))))

    for line in report.splitlines():
        m = _REMARK.search(line)
        if not m:
            continue
        if m.group(1) == "Function Name":
            flush()
            cur = {}
        cur[m.group(1)] = m.group(2)
    flush()
    return rows


def build_library(out_path: Path | None = None, defines: tuple[str, ...] = (), csrc: Path | None = None) -> Path:
    """Builds the shared library (default: lib/libgrouped_gemm_amd.so).  `defines`
    adds -D options to the kernel compile and `csrc` replaces the source folder
    (tuning experiments build variants into other paths)."""
    CSRC = Path(csrc) if csrc is not None else CSRC_DIR
    out = Path(out_path) if out_path else LIB_DIR / LIB_NAME
    build_dir = BUILD if out_path is None else out.parent / ("_build_" + out.stem)
    build_dir.mkdir(parents=True, exist_ok=True)
    out.parent.mkdir(parents=True, exist_ok=True)
    kernels_o = build_dir / "gg_kernels.o"
    moe_o = build_dir / "gg_moe.o"
    extra = [f"-D{d}" for d in defines]

    def compile_kernels() -> str:
        return _run([HIPCC, *HIP_FLAGS, *extra, "-Rpass-analysis=kernel-resource-usage", "-c",
                     str(CSRC / "gg_kernels.hip"), "-o", str(kernels_o)], capture_stderr=True)

    def compile_moe() -> None:
        _run([HIPCC, *HIP_FLAGS, "-c", str(CSRC / "gg_moe.hip"), "-o", str(moe_o)])

    def compile_host(name: str) -> Path:
        obj = build_dir / (Path(name).stem + ".o")
        _run([*CXX_FLAGS, *extra, f"-I{CSRC}", "-c", str(CSRC / name), "-o", str(obj)])
        return obj

    with ThreadPoolExecutor(max_workers=4) as pool:
        fut_k = pool.submit(compile_kernels)
        fut_moe = pool.submit(compile_moe)
        host_objs = list(pool.map(compile_host, ["grouped_gemm.cpp", "c_api.cpp"]))
        report = fut_k.result()
        fut_moe.result()

    rows = parse_resource_report(report)
    if len(rows) != 24:
        raise RuntimeError(f"expected 24 kernel resource rows, parsed {len(rows)}")
    table = "".join("    {%d, %d, %d, %d, %d, %d, %d, %d, %d},\n" % r for r in sorted(rows))
    (build_dir / "gg_resources_table.inc").write_text(table)
    res_o = build_dir / "gg_resources.o"
    _run([*CXX_FLAGS, f"-I{build_dir}", "-c", str(CSRC / "gg_resources.cpp"), "-o", str(res_o)])

    tmp = out.parent / (out.name + ".tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), str(kernels_o), str(moe_o),
          *map(str, host_objs), str(res_o)])
    os.replace(tmp, out)
    return out


def build_host_sanitized(out_path: Path) -> Path:
    """The library with its host code (grouped_gemm.cpp, c_api.cpp) built by g++ under
    AddressSanitizer and UndefinedBehaviorSanitizer, linked with the kernel objects of the regular
    build (build_library first).  Host code only: the GPU code is the regular build's.  A process
    that loads it needs the sanitizer runtimes preloaded (libasan, libubsan)."""
    out = Path(out_path)
    out.parent.mkdir(parents=True, exist_ok=True)
    objs = []
    for name in ("grouped_gemm.cpp", "c_api.cpp"):
        obj = out.parent / (Path(name).stem + "_san.o")
        _run([*CXX_FLAGS, "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
              f"-I{CSRC_DIR}", "-c", str(CSRC_DIR / name), "-o", str(obj)])
        objs.append(str(obj))
    kernel_objs = [str(BUILD / n) for n in ("gg_kernels.o", "gg_moe.o", "gg_resources.o")]
    _run(["g++", "-shared", "-fsanitize=address,undefined", "-o", str(out), *kernel_objs, *objs,
          f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}"])
    return out


def build_cpp_tests() -> Path:
    """The C++ drop-in test driver (tests/cpp/test_correctness.cpp), linked
    against the library with an rpath to it."""
    bin_dir = BUILD / "bin"
    bin_dir.mkdir(parents=True, exist_ok=True)
    exe = bin_dir / "test_correctness"
    src = ROOT / "tests" / "cpp" / "test_correctness.cpp"
    oracle_dir = ROOT / "oracle"
    _run([*CXX_FLAGS, f"-I{oracle_dir}", str(src), "-o", str(exe),
          f"-L{LIB_DIR}", "-lgrouped_gemm_amd", f"-L{oracle_dir}", "-loracle",
          f"-L{ROCM / 'lib'}", "-lamdhip64",
          f"-Wl,-rpath,{LIB_DIR}", f"-Wl,-rpath,{oracle_dir}", f"-Wl,-rpath,{ROCM / 'lib'}"])
    return exe


def build_bench_driver() -> Path:
    """The benchmark harness (bench/benchmark_grouped_gemm.cpp): the reference
    benchmark's command line, table and fixed-output cache on this library."""
    bin_dir = BUILD / "bin"
    bin_dir.mkdir(parents=True, exist_ok=True)
    exe = bin_dir / "benchmark_grouped_gemm"
    src = PKG / "bench" / "benchmark_grouped_gemm.cpp"
    _run([*CXX_FLAGS, str(src), "-o", str(exe), f"-L{LIB_DIR}", "-lgrouped_gemm_amd",
          f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{LIB_DIR}", f"-Wl,-rpath,{ROCM / 'lib'}"])
    return exe


def build_vendor_baseline() -> Path:
    """The hipBLASLt comparison program (bench/vendor_hipblaslt.cpp), run by
    bench.py and the tests as a child process; the library does not link it."""
    bin_dir = BUILD / "bin"
    bin_dir.mkdir(parents=True, exist_ok=True)
    exe = bin_dir / "vendor_hipblaslt"
    src = PKG / "bench" / "vendor_hipblaslt.cpp"
    _run([*CXX_FLAGS, str(src), "-o", str(exe), f"-L{LIB_DIR}", "-lgrouped_gemm_amd", f"-L{ROCM / 'lib'}",
          "-lhipblaslt", "-lamdhip64", f"-Wl,-rpath,{LIB_DIR}", f"-Wl,-rpath,{ROCM / 'lib'}"])
    return exe


def build_oracle() -> Path:
    _run(["make", "-s", "-C", str(ROOT / "oracle")])
    return ROOT / "oracle" / "liboracle.so"


def main(argv: list[str]) -> int:
    build_library()
    if "--no-oracle" not in argv:
        build_oracle()
    if "--no-tests" not in argv:
        build_cpp_tests()
    build_bench_driver()
    build_vendor_baseline()
    print(f"built {LIB_DIR / LIB_NAME}")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
