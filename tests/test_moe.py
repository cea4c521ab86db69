"""Device-resident preparation of a mixture-of-experts group (csrc/gg_moe.hip, MoeGroupedGemm).

The prepared set it writes on the GPU must equal, bit for bit, what the host path gives for the same
problems: prepare_problem_set's permutation and tile offsets (src/grouped_gemm.cu:967-1022, itself
pinned to the oracle and the reference's published rows), the descriptors build() uploads, and the
schedule build() plans (longest processing time first, restated in schedule_plan.py).  D must equal the host path's D bit for bit (same kernel, same tiles) and the
oracle's host GEMM within 1e-3*sqrt(K)*max|A|*max|B|*|alpha| + 1e-6*(|beta|*max|C| + 1).  Counts are
untrusted input: negative or oversubscribed counts are clamped and reported, never read or written
out of bounds.  Runs are captured in a graph and replayed with new counts."""
import ctypes
import math
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from grouped_gemm_gpu_kernel_amd import _lib, api, torch_ops
from grouped_gemm_gpu_kernel_amd.api import KernelConfig, ProblemDesc, SortMode
from oracle import oracle as O
from schedule_plan import plan_schedule


def test_moe_symbols_and_layout_struct(tmp_path):
    """The ctypes mirror of ggk_moe_layout has the C compiler's size and field offsets."""
    L = _lib.lib()
    for name in ("ggk_moe_prepare", "ggk_launch_grouped_device", "gg_moe_create", "gg_moe_run", "gg_moe_destroy"):
        assert hasattr(L, name)
    fields = [f for f, _ in _lib.GGKMoeLayout._fields_]
    src = tmp_path / "layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "grouped_gemm_amd_kernels.h"\n'
                   "int main(void) {\n  printf(\"%zu\\n\", sizeof(ggk_moe_layout));\n" +
                   "".join(f'  printf("%zu\\n", offsetof(ggk_moe_layout, {f}));\n' for f in fields) +
                   "  return 0;\n}\n")
    exe = tmp_path / "layout"
    root = Path(__file__).resolve().parents[1]
    subprocess.run(["gcc", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{root / 'include'}", str(src),
                    "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert got[0] == ctypes.sizeof(_lib.GGKMoeLayout)
    assert got[1:] == [getattr(_lib.GGKMoeLayout, f).offset for f in fields]


def test_invalid_layouts_rejected_on_host():
    """ggk_moe_prepare checks the layout before any launch (no GPU needed for these)."""
    lay = _lib.GGKMoeLayout(0, 64, 64, 0x1000, 64, 0x2000, 64, 64 * 64, None, 64, 0x3000, 64, 1.0, 0.0, 100)
    buf = ctypes.c_void_p(0x4000)
    L = _lib.lib()
    assert L.ggk_moe_prepare(1, 1, ctypes.byref(lay), buf, 2, buf, buf, buf, buf, buf, None) == 1  # experts = 0
    lay.experts = _lib.GGK_MOE_MAX_EXPERTS + 1
    assert L.ggk_moe_prepare(1, 1, ctypes.byref(lay), buf, 2, buf, buf, buf, buf, buf, None) == 1
    lay.experts = 4
    lay.lda = 10  # below K
    assert L.ggk_moe_prepare(1, 1, ctypes.byref(lay), buf, 2, buf, buf, buf, buf, buf, None) == 1
    lay.lda = 64
    assert L.ggk_moe_prepare(1, 1, ctypes.byref(lay), buf, 7, buf, buf, buf, buf, buf, None) == 1  # sort mode
    assert L.ggk_moe_prepare(6, 1, ctypes.byref(lay), buf, 2, buf, buf, buf, buf, buf, None) == 1  # variant
    # the same checks on their own, as build() and the allocation-free call make them before any launch
    assert L.ggk_moe_layout_check(1, 1, ctypes.byref(lay)) == 0
    for field, bad in (("lda", 10), ("max_rows", -1), ("ldb", 63), ("ldd", 0), ("stride_b", -1), ("experts", 0)):
        good = getattr(lay, field)
        setattr(lay, field, bad)
        assert L.ggk_moe_layout_check(1, 1, ctypes.byref(lay)) == 1, field
        setattr(lay, field, good)
    lay.b = None
    assert L.ggk_moe_layout_check(1, 1, ctypes.byref(lay)) == _lib.HIP_ERROR_INVALID_DEVICE_POINTER


# ---------------------------------------------------------------- GPU

def _counts(experts, total, seed, zeros=True):
    """Zipf-like token counts summing to `total`, some experts empty."""
    rng = np.random.default_rng(seed)
    w = 1.0 / np.arange(1, experts + 1) ** 1.2
    rng.shuffle(w)
    if zeros and experts > 3:
        w[rng.choice(experts, size=experts // 4, replace=False)] = 0.0
    c = np.floor(w / w.sum() * total).astype(np.int64)
    c[int(np.argmax(w))] += total - c.sum()
    assert c.sum() == total and (c >= 0).all()
    return c.astype(np.int32)


def _setup(experts, rows, n, k, seed, c_present=True, guard=0):
    dev = torch.device("cuda")
    g = torch.Generator(device="cpu").manual_seed(seed)
    a = (torch.rand(rows, k, generator=g) * 2 - 1).half().to(dev)
    b = (torch.rand(experts, k, n, generator=g) * 2 - 1).half().to(dev)
    c = (torch.rand(rows, n, generator=g) * 2 - 1).to(dev) if c_present else None
    d_full = torch.full((rows + guard, n), float("nan"), device=dev)
    return a, b, c, d_full


def _host_problems(a, b, c, d, counts, alpha, beta, max_rows):
    """The same group as a host problem list (rows past max_rows dropped, as on the device)."""
    experts, k, n = b.shape
    out, r0 = [], 0
    for e in range(experts):
        cnt = max(0, int(counts[e]))
        rows = max(0, min(cnt, max_rows - r0))
        out.append(ProblemDesc(m=rows, n=n, k=k, a=a.data_ptr() + 2 * r0 * a.stride(0),
                               b=b.data_ptr() + 2 * e * b.stride(0),
                               c=(c.data_ptr() + 4 * r0 * c.stride(0)) if c is not None else None,
                               d=d.data_ptr() + 4 * r0 * d.stride(0), lda=a.stride(0), ldb=b.stride(1),
                               ldc=c.stride(0) if c is not None else n, ldd=d.stride(0), alpha=alpha, beta=beta))
        r0 += cnt
    return out


def _read_device_set(plan, experts):
    probs_ptr, offs_ptr, perm_ptr, head_ptr, order_ptr = plan.moe.device_buffers()
    L = _lib.lib()
    descs = (_lib.GGDeviceProblemDesc * experts)()
    offs = np.zeros(2 * (experts + 1), np.int32)
    perm = np.zeros(experts, np.int32)
    order = np.zeros(experts, np.int32)
    head = np.zeros(_lib.GGK_MOE_HEADER_INTS, np.int32)
    torch.cuda.synchronize()
    for dst, src, nbytes in ((ctypes.addressof(descs), probs_ptr, ctypes.sizeof(descs)),
                             (offs.ctypes.data, offs_ptr, offs.nbytes), (perm.ctypes.data, perm_ptr, perm.nbytes),
                             (order.ctypes.data, order_ptr, order.nbytes), (head.ctypes.data, head_ptr, head.nbytes)):
        _lib.check(L.ggk_copy_to_host(dst, src, nbytes), "copy")
    return descs, offs, perm, order, head



@pytest.mark.gpu
@pytest.mark.parametrize("config", ["64x64x16", "128x64x32", "64x128x32"])
@pytest.mark.parametrize("experts", [1, 5, 64, 65, 256, 1024])
def test_device_prepare_equals_host_prepare(torch_cuda, config, experts):
    cfg = KernelConfig.named(config)
    rows = 3000
    n, k = 200, 40
    a, b, c, d = _setup(experts, rows, n, k, seed=experts)
    counts = _counts(experts, rows, seed=experts + 1)
    counts_dev = torch.from_numpy(counts).cuda()
    shape = _lib.GGKWorkShape()
    _lib.check(_lib.lib().ggk_work_shape_get({"64x64x16": 0, "128x64x32": 1, "64x128x32": 2}[config], 1,
                                             ctypes.byref(shape)), "work shape")
    for mode in SortMode:
        plan = torch_ops.MoeGroupedGemmPlan(a, b, d, c, 1.5, 0.5, sort_mode=mode, config=cfg)
        plan.run(counts_dev)
        descs, offs, perm, order, head = _read_device_set(plan, experts)
        probs = _host_problems(a, b, c, d, counts, 1.5, 0.5, rows)
        prep = api.prepare_problem_set(probs, cfg, mode)
        assert list(perm) == prep.sorted_to_original, (config, experts, mode)
        assert list(offs[:experts + 1]) == prep.tile_offsets, (config, experts, mode)
        work = []
        for i, p in enumerate(prep.sorted_problems):
            dd = descs[i]
            tm = -(-p.m // cfg.cta_m) if p.m > 0 and p.n > 0 else 0
            tn = -(-p.n // cfg.cta_n) if p.m > 0 and p.n > 0 else 0
            got = (dd.m, dd.n, dd.k, dd.a or 0, dd.b or 0, dd.c or 0, dd.d or 0, dd.lda, dd.ldb, dd.ldc, dd.ldd,
                   dd.alpha, dd.beta, dd.tiles_m, dd.tiles_n)
            want = (p.m, p.n, p.k, p.a, p.b, p.c or 0, p.d, p.lda, p.ldb, p.ldc, p.ldd, p.alpha, p.beta, tm, tn)
            assert got == want, (config, experts, mode, i)
            work.append((-(-tm // shape.tiles_m)) * (-(-tn // shape.tiles_n)))
        want_order, want_offsets, want_bounds = plan_schedule(
            [(p.m, p.n, p.k) for p in prep.sorted_problems], work, cfg.cta_m * shape.tiles_m,
            cfg.cta_n * shape.tiles_n, shape.stage_k, True)
        assert sorted(want_order) == list(range(experts))
        assert list(order) == want_order, (config, experts, mode)
        assert list(offs[experts + 1:]) == want_offsets, (config, experts, mode)
        assert head[0] == prep.total_tiles and head[1] == sum(work)
        assert list(head[2:2 + _lib.GGK_SCHEDULER_CHUNKS + 1]) == want_bounds, (config, experts, mode)
        assert head[_lib.GGK_MOE_STATUS] == 0
        plan.close()


def _check_against_oracle(a, b, c, d, counts, alpha, beta, max_rows, sample=6):
    probs = _host_problems(a, b, c, d, counts, alpha, beta, max_rows)
    rng = np.random.default_rng(0)
    k = b.shape[1]
    a_h = a.cpu().numpy().view(np.uint16)
    b_h = b.cpu().numpy().view(np.uint16)
    c_h = c.cpu().numpy() if c is not None else None
    d_h = d.cpu().numpy()
    r0 = 0
    nonempty = [e for e, p in enumerate(probs) if p.m > 0]
    check = set(rng.choice(nonempty, size=min(sample, len(nonempty)), replace=False).tolist()) if nonempty else set()
    for e, p in enumerate(probs):
        if e in check:
            want = O.gemm(p.m, p.n, k, a_h[r0:r0 + p.m], a.stride(0), b_h[e], b.stride(1),
                          c_h[r0:r0 + p.m] if c_h is not None else None, p.n, alpha, beta)[:p.m * p.n]
            got = d_h[r0:r0 + p.m].reshape(-1)
            tol = 1e-3 * math.sqrt(max(k, 1)) * abs(alpha) + 1e-6 * (abs(beta) + 1.0)
            assert np.abs(got - want).max() <= tol, e
        r0 += max(0, int(counts[e]))


@pytest.mark.gpu
@pytest.mark.parametrize("mode", [SortMode.kNone, SortMode.kByTiles])
def test_moe_results_equal_host_path_and_oracle(torch_cuda, mode):
    experts, rows, n, k = 64, 4096, 384, 256
    a, b, c, d = _setup(experts, rows, n, k, seed=7)
    counts = _counts(experts, rows, seed=8)
    plan = torch_ops.MoeGroupedGemmPlan(a, b, d, c, 1.25, 0.75, sort_mode=mode)
    plan.run(torch.from_numpy(counts).cuda())
    torch.cuda.synchronize()
    assert not torch.isnan(d).any()
    d_dev = d.clone()
    d.fill_(float("nan"))
    probs = _host_problems(a, b, c, d, counts, 1.25, 0.75, rows)
    ex = api.GroupedGemmExecutor()
    cfg = KernelConfig.named("128x64x32")
    _lib.check(ex.build(api.prepare_problem_set(probs, cfg, mode), cfg), "build")
    _lib.check(ex.run(torch.cuda.current_stream()), "run")
    torch.cuda.synchronize()
    assert torch.equal(d, d_dev)  # same kernel, same tiles: bit-identical
    ex.close()
    _check_against_oracle(a, b, c, d, counts, 1.25, 0.75, rows)
    plan.close()


@pytest.mark.gpu
def test_untrusted_counts_are_clamped(torch_cuda):
    """Counts adding up past the rows of A/D, and a negative count: flagged, clamped to the owned
    rows; the guard rows after them stay untouched."""
    experts, rows, n, k, guard = 16, 1000, 96, 64, 64
    a, b, c, d_full = _setup(experts, rows + guard, n, k, seed=3, guard=0)
    d = d_full[:rows]
    counts = _counts(experts, rows, seed=4, zeros=False)
    counts[3] = -5
    counts[5] += 700  # oversubscribed
    plan = torch_ops.MoeGroupedGemmPlan(a[:rows], b, d, c[:rows], 1.0, 1.0)
    plan.run(torch.from_numpy(counts).cuda())
    status = plan.status()
    assert status == _lib.GGK_MOE_NEGATIVE | _lib.GGK_MOE_CLAMPED
    assert torch.isnan(d_full[rows:]).all()  # never written
    _check_against_oracle(a[:rows], b, c[:rows], d, counts, 1.0, 1.0, rows, sample=16)
    # every row a clamped expert owns was written
    owned = min(rows, int(np.maximum(counts, 0).sum()))
    assert not torch.isnan(d[:owned]).any()
    plan.close()


@pytest.mark.gpu
def test_graph_capture_replays_with_new_counts(torch_cuda):
    """prepare + grouped launch captured once, replayed with the counts changed in place between
    replays; every replay equals an eager run with the same counts."""
    experts, rows, n, k = 32, 2048, 256, 128
    a, b, c, d = _setup(experts, rows, n, k, seed=11)
    plan = torch_ops.MoeGroupedGemmPlan(a, b, d, c, 1.0, 0.5)
    counts_dev = torch.from_numpy(_counts(experts, rows, seed=12)).cuda()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        plan.run(counts_dev)  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run(counts_dev)
    for seed in (13, 14, 15):
        counts = _counts(experts, rows, seed=seed)
        counts_dev.copy_(torch.from_numpy(counts))
        d.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        replayed = d.clone()
        d.fill_(float("nan"))
        plan.run(counts_dev)
        torch.cuda.synchronize()
        assert torch.equal(replayed, d), seed
        assert not torch.isnan(d).any()
    plan.close()
