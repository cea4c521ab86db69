"""Full-size GPU parity on every grouped workload of the benchmark (mixed-512, uniform dense
64 x 2048^3, the MoE expert shape K=4096 / N=14336 / sum M = 16384 with empty experts, long-tail
4096), the method of the reference's own test (tests/test_correctness.cu:85-102, 216-247): the
same inputs through every path, then the outputs against the CPU host GEMM.

Bars (size-independent properties at full size, plus sampled elements):
  * D is NaN-poisoned before every run; afterwards exactly the padding between the problems' output
    blocks is still NaN (every element of every non-empty problem was written, nothing else was).
  * The four sort modes and the per-problem-launch baseline give bit-identical D (each output tile's
    arithmetic does not depend on the order or the workgroup that computes it); on the MoE shape the
    device-side prepare (MoeGroupedGemm) gives the host-prepared D bit for bit as well.
  * At least 8 seeded elements of every non-empty problem match the oracle's host GEMM within
    1e-3 * sqrt(K) * max|A_row| * max|B_col| * |alpha| + 1e-6 * (|beta| * |C| + 1).
"""
import numpy as np
import pytest

from grouped_gemm_gpu_kernel_amd import _lib, api
from grouped_gemm_gpu_kernel_amd.api import GroupedGemmExecutor, KernelConfig, SortMode
from grouped_gemm_gpu_kernel_amd.workloads import DeviceWorkload, make_spec
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SAMPLES_PER_PROBLEM = 8


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
