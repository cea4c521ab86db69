"""Full-size GPU parity on every grouped workload of the benchmark (mixed-512, uniform dense
64 x 2048^3, the MoE expert shape K=4096 / N=14336 / sum M = 16384 with empty experts, long-tail
4096), the method of the reference's own test (tests/test_correctness.cu:85-102, 216-247): the
same inputs through every path, then the outputs against the CPU host GEMM.

Bars (size-independent properties at full size, plus checked elements):
  * D is NaN-poisoned before every run; afterwards exactly the padding between the problems' output
    blocks is still NaN (every element of every non-empty problem was written, nothing else was).
  * The four sort modes and the per-problem-launch baseline give bit-identical D (each output tile's
    arithmetic does not depend on the order or the workgroup that computes it); on the MoE shape the
    device-side prepare (MoeGroupedGemm) gives the host-prepared D bit for bit as well.
  * Against the oracle's host GEMM, within
    1e-3 * sqrt(K) * max|A_row| * max|B_col| * |alpha| + 1e-6 * (|beta| * |C| + 1):
      - 8 seeded elements of every non-empty problem, its corners among them;
      - one seeded row in every 32-row band of every non-empty problem, all of its columns (problems
        of at most 2^21 multiply-adds whole): every wave block of every work tile -- 32 x 64 of D at
        the smallest, in whole 32-row groups -- holds checked elements, in every edge class;
      - every element of the largest problem of the set (dense64: problem 0 of 64 equal ones;
        long-tail: 4090 x 3875 x 7430; MoE: the largest expert, 4891 x 14336 x 4096), as the
        reference's check_outputs compares every element (tests/test_correctness.cu:216-247).
"""
import os

import numpy as np
import pytest

from grouped_gemm_gpu_kernel_amd import _lib, api
from grouped_gemm_gpu_kernel_amd.api import GroupedGemmExecutor, KernelConfig, SortMode
from grouped_gemm_gpu_kernel_amd.workloads import DeviceWorkload, make_spec
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SAMPLES_PER_PROBLEM = 8
ROW_BAND = 32  # rows per band of the row-band check: the height of the smallest wave block
WHOLE_MACS = 1 << 21  # problems up to this many multiply-adds are checked whole by the row-band check
ORACLE_THREADS = max(1, min(16, os.cpu_count() or 1))  # the box's CPU share


def say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def torch(torch_cuda):
    return torch_cuda


def _live(spec):
    return (spec.m > 0) & (spec.n > 0)


def _written_elements(spec) -> int:
    live = _live(spec)
    return int(np.sum(spec.m[live].astype(np.int64) * spec.n[live]))


def _check_written(torch, dw, what):
    """Exactly the non-empty problems' m x n blocks were written: the NaN count equals the padding."""
    nan = int(torch.isnan(dw.d).sum().item())
    want = dw.d.numel() - _written_elements(dw.spec)
    assert nan == want, f"{what}: {nan} NaN elements of D, expected {want} (padding only)"


def _ragged(lengths):
    """(starts, within): for a concatenation of runs of the given lengths, each run's first position
    and every position's index within its run."""
    lengths = np.asarray(lengths, np.int64)
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int64)
    within = np.arange(int(lengths.sum()), dtype=np.int64) - np.repeat(starts, lengths)
    return starts, within


def _check_samples(torch, dw, d_pool, seed, what, rows_of=None):
    """SAMPLES_PER_PROBLEM seeded elements of every non-empty problem against the oracle.  Their rows of
    A and columns of B are gathered on the GPU in one index operation each.  rows_of(i, r) maps a
    row of problem i to its element offset in d_pool (default: the workload's own D layout)."""
    spec = dw.spec
    rng = np.random.default_rng(seed)
    probs = np.flatnonzero(_live(spec))
    idx = np.repeat(probs, SAMPLES_PER_PROBLEM)
    m = spec.m[idx].astype(np.int64)
    n = spec.n[idx].astype(np.int64)
    k = spec.k[idx].astype(np.int64)
    rows = (rng.random(idx.size) * m).astype(np.int64)
    cols = (rng.random(idx.size) * n).astype(np.int64)
    # the corners of every problem are among the samples
    rows[::SAMPLES_PER_PROBLEM] = 0
    cols[::SAMPLES_PER_PROBLEM] = 0
    rows[SAMPLES_PER_PROBLEM - 1::SAMPLES_PER_PROBLEM] = m[SAMPLES_PER_PROBLEM - 1::SAMPLES_PER_PROBLEM] - 1
    cols[SAMPLES_PER_PROBLEM - 1::SAMPLES_PER_PROBLEM] = n[SAMPLES_PER_PROBLEM - 1::SAMPLES_PER_PROBLEM] - 1
    starts, within = _ragged(k)
    a_idx = np.repeat(dw.a_off[idx] + rows * k, k) + within                    # lda = k
    b_idx = np.repeat(dw.b_off[idx] + cols, k) + within * np.repeat(n, k)      # ldb = n
    dev = dw.a.device
    a_vals = dw.a[torch.from_numpy(a_idx).to(dev)].cpu().numpy().view(np.uint16)
    b_vals = dw.b[torch.from_numpy(b_idx).to(dev)].cpu().numpy().view(np.uint16)
    c_vals = None
    if dw.has_c:
        c_vals = dw.c[torch.from_numpy(dw.c_off[idx] + rows * n + cols).to(dev)].cpu().numpy()
    if rows_of is None:
        d_idx = dw.d_off[idx] + rows * n + cols
    else:
        d_idx = np.array([rows_of(int(i), int(r)) for i, r in zip(idx, rows)], np.int64) + cols
    got = d_pool[torch.from_numpy(d_idx).to(dev)].cpu().numpy()
    alpha = spec.alpha[idx]
    beta = spec.beta[idx]
    want = O.gemm_samples(k, a_vals, starts, b_vals, starts, c_vals, alpha, beta)
    af = np.abs(O.f16_to_f32(a_vals))
    bf = np.abs(O.f16_to_f32(b_vals))
    amax = np.maximum.reduceat(af, starts) if af.size else np.zeros(idx.size)
    bmax = np.maximum.reduceat(bf, starts) if bf.size else np.zeros(idx.size)
    amax = np.where(k > 0, amax, 0.0)
    bmax = np.where(k > 0, bmax, 0.0)
    cabs = np.abs(c_vals) if c_vals is not None else np.zeros(idx.size)
    tol = 1e-3 * np.sqrt(np.maximum(k, 1)) * amax * bmax * np.abs(alpha) + 1e-6 * (np.abs(beta) * cabs + 1.0)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bad = np.flatnonzero(~(err <= tol))
    assert bad.size == 0, (f"{what}: {bad.size} of {idx.size} samples outside the bound, first: problem "
                           f"{idx[bad[0]]} ({m[bad[0]]}x{n[bad[0]]}x{k[bad[0]]}) element ({rows[bad[0]]}, "
                           f"{cols[bad[0]]}) got {got[bad[0]]} want {want[bad[0]]} tol {tol[bad[0]]}")
    say(f"{what}: {idx.size} samples over {probs.size} problems, max error {float(err.max()):.3g}")


def _check_rows(torch, dw, d_pool, i, rows, what, rows_of=None):
    """Rows `rows` of problem i's D, every column, against the oracle's host GEMM (OpenMP form on the
    host's cores, bit-identical to the literal loop) on the same rows of A and C and all of B.
    Returns the largest error."""
    spec = dw.spec
    m, n, k = int(spec.m[i]), int(spec.n[i]), int(spec.k[i])
    alpha, beta = float(spec.alpha[i]), float(spec.beta[i])
    dev = dw.a.device
    rows = np.asarray(rows, np.int64)
    r = len(rows)
    kk = max(k, 1)
    if k > 0:
        a_idx = torch.from_numpy(int(dw.a_off[i]) + rows[:, None] * k + np.arange(k)[None, :]).to(dev)
        a_rows = dw.a[a_idx]
        b_all = dw.b[int(dw.b_off[i]):int(dw.b_off[i]) + k * n]
        amax = a_rows.view(torch.float16).float().abs().amax(1).cpu().numpy().astype(np.float64)
        bmax = b_all.view(torch.float16).view(k, n).float().abs().amax(0).cpu().numpy().astype(np.float64)
        a_host = a_rows.cpu().numpy().view(np.uint16).reshape(-1)
        b_host = b_all.cpu().numpy().view(np.uint16)
    else:
        amax, bmax = np.zeros(r), np.zeros(n)
        a_host = np.zeros(1, np.uint16)
        b_host = np.zeros(1, np.uint16)
    cols = torch.arange(n, device=dev)
    c_host = None
    if dw.has_c:
        c_idx = torch.from_numpy(int(dw.c_off[i]) + rows * n).to(dev)[:, None] + cols[None, :]
        c_host = dw.c[c_idx].cpu().numpy().reshape(-1)
    if rows_of is None:
        d_start = torch.from_numpy(int(dw.d_off[i]) + rows * n).to(dev)
    else:
        d_start = torch.from_numpy(np.array([rows_of(i, int(x)) for x in rows], np.int64)).to(dev)
    got = d_pool[d_start[:, None] + cols[None, :]].cpu().numpy().astype(np.float64)
    want = O.gemm(r, n, k, a_host, kk, b_host, n, c_host, n, alpha, beta,
                  threads=ORACLE_THREADS)[:r * n].reshape(r, n).astype(np.float64)
    cabs = np.abs(c_host.reshape(r, n)) if c_host is not None else 0.0
    tol = 1e-3 * np.sqrt(kk) * amax[:, None] * bmax[None, :] * abs(alpha) + 1e-6 * (abs(beta) * cabs + 1.0)
    err = np.abs(got - want)
    bad = np.argwhere(~(err <= tol))
    if bad.size:
        y, x = bad[0]
        raise AssertionError(f"{what}: problem {i} ({m}x{n}x{k}): {len(bad)} of {r * n} checked elements outside "
                             f"the bound, first ({rows[y]}, {x}) got {got[y, x]} want {want[y, x]} tol {tol[y, x]}")
    return float(err.max()) if err.size else 0.0


def _check_row_bands(torch, dw, d_pool, seed, what):
    """One seeded row in every ROW_BAND-row band of every non-empty problem, all columns (problems of
    at most WHOLE_MACS multiply-adds whole), against the oracle."""
    spec = dw.spec
    rng = np.random.default_rng(seed)
    live = np.flatnonzero(_live(spec))
    worst, elements = 0.0, 0
    for j, i in enumerate(live):
        m, n, k = int(spec.m[i]), int(spec.n[i]), int(spec.k[i])
        if m * n * max(k, 1) <= WHOLE_MACS:
            rows = np.arange(m, dtype=np.int64)
        else:
            starts = np.arange(0, m, ROW_BAND, dtype=np.int64)
            rows = starts + (rng.random(starts.size) * np.minimum(ROW_BAND, m - starts)).astype(np.int64)
        worst = max(worst, _check_rows(torch, dw, d_pool, int(i), rows, what))
        elements += len(rows) * n
        if (j + 1) % 256 == 0:
            say(f"{what}: row bands of {j + 1} of {live.size} problems checked")
    say(f"{what}: row bands, {elements} elements over {live.size} problems, max error {worst:.3g}")


def _check_whole_problem(torch, dw, d_pool, i, what, rows_of=None):
    """Every element of problem i against the oracle."""
    m, n, k = int(dw.spec.m[i]), int(dw.spec.n[i]), int(dw.spec.k[i])
    say(f"{what}: whole problem {i} ({m}x{n}x{k}) against the oracle on {ORACLE_THREADS} threads")
    worst = _check_rows(torch, dw, d_pool, int(i), np.arange(m, dtype=np.int64), what, rows_of)
    say(f"{what}: whole problem {i}: {m * n} elements, max error {worst:.3g}")


def _largest_problem(spec) -> int:
    return int(np.argmax(spec.m.astype(np.int64) * spec.n * np.maximum(spec.k, 1) * _live(spec)))


def _run_modes_and_baseline(torch, dw, cfg, what, baseline=True):
    """Runs every sort mode (and the per-problem baseline) on freshly poisoned D; all must give the
    same bits.  Returns the bits of D (a GPU tensor) after the first mode."""
    probs = dw.problems()
    ref = None
    modes = list(SortMode) + (["baseline"] if baseline else [])
    for mode in modes:
        dw.poison_d()
        say(f"{what}: mode {mode}")
        if mode == "baseline":
            assert api.run_baseline_per_problem(probs, cfg) == 0
        else:
            ex = GroupedGemmExecutor()
            assert ex.build(api.prepare_problem_set(probs, cfg, mode), cfg) == 0
            assert ex.run() == 0
            torch.cuda.synchronize()
            ex.close()
        torch.cuda.synchronize()
        _check_written(torch, dw, f"{what} {mode}")
        bits = dw.d.view(torch.int32)
        if ref is None:
            ref = bits.clone()
        else:
            assert torch.equal(bits, ref), f"{what}: mode {mode} gives different bits from mode 0"
    return ref


@pytest.mark.parametrize("name", ["mixed512", "dense64", "longtail4096"])
def test_full_size_workload(torch, name):
    say(f"full size {name}")
    spec = make_spec(name)
    dw = DeviceWorkload(spec)
    cfg = KernelConfig.named(spec.config)
    _run_modes_and_baseline(torch, dw, cfg, name)
    _check_samples(torch, dw, dw.d, 21, name)
    _check_row_bands(torch, dw, dw.d, 24, name)
    if name != "mixed512":
        _check_whole_problem(torch, dw, dw.d, _largest_problem(spec), name)
    if name == "mixed512":
        # three whole problems against the oracle
        probs = dw.problems()
        for i in np.argsort(spec.m * spec.n)[:3]:
            p = probs[i]
            want = O.gemm(p.m, p.n, p.k, dw.host_a(i), p.lda, dw.host_b(i), p.ldb, dw.host_c(i), p.ldc, p.alpha,
                          p.beta)
            tol = 1e-3 * np.sqrt(p.k) * abs(p.alpha) + 1e-6 * (abs(p.beta) + 1)
            assert np.abs(dw.host_d(i)[:p.m * p.n] - want[:p.m * p.n]).max() <= tol
    del dw
    torch.cuda.empty_cache()


def test_full_size_moe64_host_and_device_prepare(torch):
    """The MoE expert shape through the host path (4 sort modes + baseline) and through
    MoeGroupedGemm (token counts on the GPU, prepare on the device) in every sort mode: one set of
    bits, and the oracle on samples.  Empty experts stay untouched."""
    from grouped_gemm_gpu_kernel_amd import torch_ops

    spec = make_spec("moe64")
    assert (spec.m == 0).any() and int(spec.m.sum()) == 16384
    dw = DeviceWorkload(spec)
    cfg = KernelConfig.named(spec.config)
    ref = _run_modes_and_baseline(torch, dw, cfg, "moe64 host")
    _check_samples(torch, dw, dw.d, 22, "moe64 host")
    _check_row_bands(torch, dw, dw.d, 25, "moe64 host")
    # the largest expert whole; the device-prepared D of every expert equals this D bit for bit (below)
    _check_whole_problem(torch, dw, dw.d, _largest_problem(spec), "moe64 host")

    e, k, n = spec.count, int(spec.k[0]), int(spec.n[0])
    rows = spec.m.astype(np.int64)
    r0 = np.concatenate([[0], np.cumsum(rows)[:-1]])
    total = int(rows.sum())
    a_pool = dw.a.view(torch.float16)
    a = torch.cat([a_pool[int(o):int(o) + int(m) * k].view(int(m), k) for o, m in zip(dw.a_off, rows)])
    # B of consecutive experts lies k * n elements apart in the pool: view it as [E, K, N]
    assert all(int(o) == i * k * n for i, o in enumerate(dw.b_off))
    b = dw.b.view(torch.float16)[:e * k * n].view(e, k, n)
    d = torch.empty(total, n, dtype=torch.float32, device=a.device)
    counts = torch.from_numpy(rows.astype(np.int32)).cuda()
    for mode in SortMode:
        say(f"moe64 device prepare: mode {mode}")
        d.fill_(float("nan"))
        plan = torch_ops.MoeGroupedGemmPlan(a, b, d, None, 1.0, 0.0, sort_mode=mode, config=cfg)
        plan.run(counts)  # raises on a failed launch
        torch.cuda.synchronize()
        assert plan.status() == 0
        plan.close()
        assert not torch.isnan(d).any(), f"mode {mode}: unwritten rows"
        for i in range(e):
            if rows[i] == 0:
                continue
            got = d[int(r0[i]):int(r0[i] + rows[i])].reshape(-1).view(torch.int32)
            want = ref[int(dw.d_off[i]):int(dw.d_off[i]) + int(rows[i]) * n]
            assert torch.equal(got, want), f"mode {mode}: expert {i} differs from the host path"
    _check_samples(torch, dw, d.reshape(-1), 23, "moe64 device", rows_of=lambda i, r: (int(r0[i]) + r) * n)
    del a, b, d, dw
    torch.cuda.empty_cache()
