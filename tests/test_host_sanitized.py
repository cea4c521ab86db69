"""The host runtime under AddressSanitizer and UndefinedBehaviorSanitizer (CPU): the library's host
code rebuilt with both (build.build_host_sanitized) runs the host-logic and C-ABI tests in a child
process with the sanitizer runtimes preloaded; any report ends that process with an error."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _runtime(name):
    path = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return path if os.path.isabs(path) and Path(path).exists() else None


def test_host_code_is_sanitizer_clean(tmp_path):
    asan, ubsan = _runtime("libasan.so"), _runtime("libubsan.so")
    if asan is None or ubsan is None:
        pytest.skip("no gcc sanitizer runtimes")
    if not (ROOT / "grouped_gemm_gpu_kernel_amd" / "_build" / "gg_kernels.o").exists():
        pytest.skip("the regular build's kernel objects are missing (build first)")
    sys.path.insert(0, str(ROOT))
    from grouped_gemm_gpu_kernel_amd import build

    lib = build.build_host_sanitized(tmp_path / "libgrouped_gemm_amd_san.so")
    script = (
        "import sys; sys.path.insert(0, %r)\n"
        "from pathlib import Path\n"
        "from grouped_gemm_gpu_kernel_amd import _lib\n"
        "_lib.LIB_PATH = Path(%r)\n"
        "import pytest\n"
        "sys.exit(pytest.main(['-x', '-q', '-m', 'not gpu', '-p', 'no:cacheprovider', %r, %r]))\n"
    ) % (str(ROOT), str(lib), str(ROOT / "tests" / "test_host.py"), str(ROOT / "tests" / "test_abi.py"))
    env = dict(os.environ, LD_PRELOAD=f"{asan}:{ubsan}",
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    proc = subprocess.run([sys.executable, "-c", script], cwd=ROOT, env=env, capture_output=True, text=True,
                          timeout=600)
    assert proc.returncode == 0, (proc.stdout + proc.stderr)[-4000:]
    assert "passed" in proc.stdout
