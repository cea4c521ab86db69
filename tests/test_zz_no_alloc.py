"""The allocation-free MoE entry point (gg_moe_run_noalloc) against the allocating one
(gg_moe_create + gg_moe_run + gg_moe_destroy): same layout, counts and sort mode, bit-identical D,
on two calls in a row, the second with fewer experts and fewer rows (the static scratch keeps the
first call's contents).  Both run through the C-ABI.  Rows of D past the counts stay NaN."""
import ctypes

import numpy as np
import pytest

from grouped_gemm_gpu_kernel_amd import _lib
from grouped_gemm_gpu_kernel_amd.api import KernelConfig

pytestmark = pytest.mark.gpu


def _layout(a, b, d, experts, rows):
    k, n = a.shape[1], b.shape[2]
    return _lib.GGKMoeLayout(experts, n, k, a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(1), b.stride(0),
                             None, n, d.data_ptr(), d.stride(0), 1.25, 0.0, rows)


def _counts(experts, rows, seed):
    rng = np.random.default_rng(seed)
    w = 1.0 / np.arange(1, experts + 1) ** 1.2
    rng.shuffle(w)
    w[rng.choice(experts, size=max(1, experts // 5), replace=False)] = 0.0  # some empty experts
    c = np.floor(w / w.sum() * rows).astype(np.int64)
    c[int(np.argmax(w))] += rows - c.sum()
    return c.astype(np.int32)


def test_noalloc_matches_allocating_entry_point(torch_cuda):
    torch = torch_cuda
    L = _lib.lib()
    dev = torch.device("cuda")
    g = torch.Generator(device="cpu").manual_seed(7)
    cases = [(48, 3000, 256, 384, 2, "128x64x32"), (9, 700, 200, 136, 0, "128x64x32")]  # second: smaller
    stream = torch.cuda.current_stream().cuda_stream
    for experts, rows, k, n, mode, config in cases:
        print(f"noalloc: {experts} experts, {rows} rows, k {k}, n {n}, mode {mode}", flush=True)
        cfg = KernelConfig.named(config).to_c()
        a = (torch.rand(rows, k, generator=g) * 2 - 1).half().to(dev)
        b = (torch.rand(experts, k, n, generator=g) * 2 - 1).half().to(dev)
        counts = torch.from_numpy(_counts(experts, rows, experts)).to(dev)
        guard = 16
        d_ref = torch.full((rows + guard, n), float("nan"), device=dev)
        d_new = torch.full((rows + guard, n), float("nan"), device=dev)
        handle = ctypes.c_void_p()
        lay_ref = _layout(a, b, d_ref, experts, rows)
        assert L.gg_moe_create(ctypes.byref(lay_ref), ctypes.byref(cfg), mode, ctypes.byref(handle)) == 0
        assert L.gg_moe_run(handle, counts.data_ptr(), stream) == 0
        torch.cuda.synchronize()
        L.gg_moe_destroy(handle)
        lay_new = _layout(a, b, d_new, experts, rows)
        assert L.gg_moe_run_noalloc(ctypes.byref(lay_new), ctypes.byref(cfg), mode, counts.data_ptr(), stream) == 0
        torch.cuda.synchronize()
        assert not torch.isnan(d_new[:rows]).any(), "rows left unwritten"
        assert torch.isnan(d_new[rows:]).all(), "rows past the counts were written"
        assert torch.equal(d_new.view(torch.int32), d_ref.view(torch.int32)), "D differs from gg_moe_run"
    # limits and bad layouts are clear errors, made before any launch: D keeps its last contents
    torch.cuda.synchronize()
    before = d_new.clone()
    big = _lib.GGKMoeLayout(_lib.GGK_MOE_MAX_EXPERTS + 1, 64, 64, a.data_ptr(), 64, b.data_ptr(), 64, 64 * 64, None,
                            64, d_new.data_ptr(), 64, 1.0, 0.0, 1)
    assert L.gg_moe_run_noalloc(ctypes.byref(big), ctypes.byref(cfg), 0, counts.data_ptr(),
                                stream) == _lib.HIP_ERROR_INVALID_VALUE
    assert L.gg_moe_run_noalloc(ctypes.byref(lay_new), ctypes.byref(cfg), 0, None,
                                stream) == _lib.HIP_ERROR_INVALID_DEVICE_POINTER
    for field, bad in (("lda", 1), ("max_rows", -1), ("ldd", 1)):
        lay_bad = _layout(a, b, d_new, experts, rows)
        setattr(lay_bad, field, bad)
        assert L.gg_moe_run_noalloc(ctypes.byref(lay_bad), ctypes.byref(cfg), 0, counts.data_ptr(),
                                    stream) == _lib.HIP_ERROR_INVALID_VALUE, field
    torch.cuda.synchronize()
    assert torch.equal(d_new.view(torch.int32), before.view(torch.int32)), "a rejected call wrote D"


def test_noalloc_captured_in_a_graph(torch_cuda):
    """After one call outside any capture, the allocation-free call is captured into a graph on
    torch's capture stream and replayed with new counts written in place; every replay equals the
    allocating entry point on the same counts, bit for bit."""
    torch = torch_cuda
    L = _lib.lib()
    dev = torch.device("cuda")
    g = torch.Generator(device="cpu").manual_seed(21)
    experts, rows, k, n, mode = 24, 1500, 192, 256, 3
    cfg = KernelConfig.named("128x64x32").to_c()
    a = (torch.rand(rows, k, generator=g) * 2 - 1).half().to(dev)
    b = (torch.rand(experts, k, n, generator=g) * 2 - 1).half().to(dev)
    counts = torch.from_numpy(_counts(experts, rows, 5)).to(dev)
    d_new = torch.full((rows, n), float("nan"), device=dev)
    d_ref = torch.full((rows, n), float("nan"), device=dev)
    lay_new = _layout(a, b, d_new, experts, rows)
    lay_ref = _layout(a, b, d_ref, experts, rows)
    stream = torch.cuda.current_stream().cuda_stream
    assert L.gg_moe_run_noalloc(ctypes.byref(lay_new), ctypes.byref(cfg), mode, counts.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = torch.cuda.current_stream().cuda_stream
        assert L.gg_moe_run_noalloc(ctypes.byref(lay_new), ctypes.byref(cfg), mode, counts.data_ptr(), cap) == 0
    handle = ctypes.c_void_p()
    assert L.gg_moe_create(ctypes.byref(lay_ref), ctypes.byref(cfg), mode, ctypes.byref(handle)) == 0
    for seed in (31, 32, 33):
        print(f"noalloc graph replay, counts seed {seed}", flush=True)
        counts.copy_(torch.from_numpy(_counts(experts, rows, seed)))
        d_new.fill_(float("nan"))
        d_ref.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert L.gg_moe_run(handle, counts.data_ptr(), stream) == 0
        torch.cuda.synchronize()
        assert not torch.isnan(d_new).any(), seed
        assert torch.equal(d_new.view(torch.int32), d_ref.view(torch.int32)), seed
    L.gg_moe_destroy(handle)
    del graph
