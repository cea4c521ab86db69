"""Test configuration: the `gpu` marker, import paths, and in-tree builds of the
library and the oracle when they are missing (tests never rebuild what exists)."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    from grouped_gemm_gpu_kernel_amd import _lib

    if not _lib.LIB_PATH.exists():
        from grouped_gemm_gpu_kernel_amd import build

        build.build_library()
    if not (ROOT / "oracle" / "liboracle.so").exists():
        from oracle import oracle

        oracle.build()


_ensure_built()


@pytest.fixture(scope="session")
def torch_cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    torch.cuda.init()
    return torch
