"""Grouped FP16 GEMM benchmark on one MI355X.

Headline: grouped TFLOP/s and the fraction of the dense FP16 MFMA peak on the
mixed-512 set (512 problems, m, n log-uniform in [64, 1024], k log-uniform in [64, 2048], seed 42,
macro-tile 128x64x32), for all four sort modes, next to the per-problem-launch baseline, the static
tail share and the measured tail idle.  A step is one executor.run() over the whole set with every
operand already resident in HBM.  `value` is the fastest sort mode's throughput; among modes
within 1% of the fastest (ties within run-to-run noise) the one with the smallest static tail share
is reported, with its tail share.

Prints one JSON line.  --gpus above 1 exits: the bench measures one GPU.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

MFMA_PEAK_TFLOPS = 2516.6   # dense fp16 MFMA, MI355X (AMD public spec)
HBM_PEAK_GBS = 8000.0       # HBM3E, MI355X (AMD public spec)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--clock-warmup", type=float, default=0.3,
                    help="seconds of untimed launches before the first timed mode (at most 0.1 s before every other timed leg)")
    ap.add_argument("--workload", default=None,
                    choices=["plumbing16", "mixed512", "dense64", "moe64", "longtail4096"],
                    help="default mixed512 (summaries: the workload profiled, for useful-work ratios)")
    ap.add_argument("--config", default=None, help="macro-tile, default: the workload's")
    ap.add_argument("--modes", default="0,1,2,3", help="sort modes to time")
    ap.add_argument("--no-baseline", action="store_true", help="skip the per-problem-launch baseline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-torch-op", action="store_true", help="skip the torch binding timings")
    ap.add_argument("--no-vendor", action="store_true", help="skip the hipBLASLt comparison rows")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU baseline sample time")
    ap.add_argument("--cpu-full", action="store_true",
                    help="time the CPU baseline over the whole workload (minutes on mixed-512) instead of samples")
    ap.add_argument("--fma", action="store_true", help="FMA tile path instead of MFMA")
    ap.add_argument("--table", action="store_true", help="also print the reference-style results table")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB a few times (for scaling HBM "
                         "byte counters of a profiler run) and exit")
    ap.add_argument("--no-moe-device", action="store_true", help="skip the device-side MoE prepare timing")
    ap.add_argument("--shards", default="", metavar="N[,N...]",
                    help="also time each rank's share of N-way data-parallel splits (plan_shards), every "
                         "share run on this GPU, as the 'shards' list of the JSON line")
    ap.add_argument("--phases", action="store_true",
                    help="also report per-work-tile phase cycles of each mode (traced launches with phase stamps)")
    ap.add_argument("--profile-summary", nargs="+", metavar="DIR",
                    help="only summarize rocprofv3 CSV output folders (kernel trace and/or counters) and exit")
    ap.add_argument("--traffic-summary", nargs=4, metavar=("FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE"),
                    help="only turn FETCH_SIZE / WRITE_SIZE folders of the grouped kernel and of a "
                         "--calibrate-copy run into HBM bytes per launch of --workload and exit")
    ap.add_argument("--copy-mib", type=int, default=256, help="size of the --calibrate-copy run summarized")
    ap.add_argument("--kernel", default=r"gg_grouped_kernel<\d+,\s*\d+,\s*false",
                    help="kernel-name regex for the summaries (default: the untraced grouped kernel)")
    ap.add_argument("--modes-of-segments", default="",
                    help="summaries: comma-separated sort-mode names of the profiled bench run, in its "
                         "order: dispatches are reported per mode (the bench makes a traced dispatch "
                         "after each mode's timed runs)")
    ap.add_argument("--last", type=int, default=0,
                    help="summaries: count only the last N dispatches of each mode (its --steps)")
    args = ap.parse_args()
    args.workload_given = args.workload is not None
    if args.workload is None:
        args.workload = "mixed512"
    return args


def calibrate_copy(torch, mib: int) -> int:
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes_read": n * 4, "bytes_written": n * 4, "repeats": 5}))
    return 0


def time_runs(torch, fn, steps: int, warmup: int) -> float:
    """Mean ms per call over `steps` calls after `warmup`, HIP events on the current stream (the
    stream fn launches on).  fn returns a hipError_t (non-zero raises) or raises itself."""
    for _ in range(warmup):
        st = fn()
        if isinstance(st, int) and st != 0:
            raise RuntimeError(f"hipError_t {st}")
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        st = fn()
        if isinstance(st, int) and st != 0:
            raise RuntimeError(f"hipError_t {st}")
    stop.record()
    stop.synchronize()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


# Sort modes whose times lie within this fraction of the fastest are taken as tied (the spread of
# repeated runs on one box).
MODE_TIE = 0.01


def headline_mode(rows, times):
    """(row, ms) of the mode the bench line reports: the fastest, or among the modes within MODE_TIE
    of it the one with the smallest static tail share (the reference's tail_share,
    bench/benchmark_grouped_gemm.cu:580-607), so that the reported tail_share is not that of a
    mode which only won by noise."""
    fastest = min(times)
    tied = [(row["tail_share"], ms, i) for i, (row, ms) in enumerate(zip(rows, times)) if ms <= fastest * (1 + MODE_TIE)]
    _, ms, i = min(tied)
    return rows[i], ms


def warm_clock(torch, fn, seconds: float) -> None:
    """Untimed calls of fn for `seconds`: the GPU lowers its clock within milliseconds of idling (a
    build, a traced run, a host copy) and takes tens of milliseconds of load to raise it again, so
    each timed stretch starts after a stretch of its own launches."""
    deadline = time.perf_counter() + seconds
    while time.perf_counter() < deadline:
        for _ in range(20):
            st = fn()
            if isinstance(st, int) and st != 0:
                raise RuntimeError(f"warm-up run: hipError_t {st}")
        torch.cuda.synchronize()


def timed_prepare_and_build(probs, cfg, mode):
    """(executor, ms) for prepare_problem_set + build through the C-ABI, timed on the host."""
    import ctypes

    from grouped_gemm_gpu_kernel_amd import _lib, api

    count = len(probs)
    arr = api._problem_array(probs)
    cfg_c = cfg.to_c()
    out = (_lib.GGProblemDesc * max(1, count))()
    perm = (ctypes.c_int * max(1, count))()
    offs = (ctypes.c_int * (count + 1))()
    ex = api.GroupedGemmExecutor()
    L = _lib.lib()
    t0 = time.perf_counter()
    total = L.gg_prepare_problem_set(arr, count, ctypes.byref(cfg_c), int(mode), out, perm, offs)
    st = L.gg_executor_build(ex._handle, out, count, offs, count + 1, total, ctypes.byref(cfg_c))
    ms = (time.perf_counter() - t0) * 1e3
    if total < 0 or st != 0:
        raise RuntimeError(f"prepare/build failed: total {total}, hipError_t {st}")
    return ex, ms


def measured_tail_idle(torch, ex, runs: int = 3) -> float:
    """Share of workgroup time spent idle after finishing its last tile while others still run:
    sum_w (T_end - end_w) / (W * (T_end - T_start)), from per-workgroup wall clocks; the median
    over `runs` back-to-back traced launches (one launch now and then has a workgroup that starts
    late, which reads as several percent of idle)."""
    import statistics

    grid = ex.grid_ctas()
    clock = torch.zeros(2 * grid, dtype=torch.int64, device="cuda")
    shares = []
    for _ in range(runs):
        st = ex.run_traced(0, clock.data_ptr())
        if st != 0:
            raise RuntimeError(f"traced run hipError_t {st}")
        torch.cuda.synchronize()
        c = clock.cpu().numpy().reshape(grid, 2).astype("float64")
        t0, t1 = c[:, 0].min(), c[:, 1].max()
        shares.append(float(((t1 - c[:, 1]).sum()) / (grid * (t1 - t0))) if t1 > t0 else 0.0)
    return statistics.median(shares)


def tile_phases(torch, ex, runs: int = 3) -> dict:
    """Where a work tile's time goes, from the phase stamps of traced launches (core-clock cycles,
    s_memtime; GGK_PHASE_* in include/grouped_gemm_amd_kernels.h).  Per class of work tile (by its
    rows and columns inside the problem against half the work tile, and the row halves of the
    work table): the mean cycles from its start until one wave's first-stage loads have landed
    (first_stage), until every wave has them (k_loop_start), the k-loop per k-stage (summed cycles
    over summed stages), the hand-over of the next index, the epilogue until its last wave is done,
    next_start: from the last epilogue wave's end to the same workgroup's next tile start
    (negative where its first waves start the next tile while the slowest still stores), and
    middle_step: the per-wave parts of the k-loop step k = stages / 2.  The median launch of
    `runs`."""
    import numpy as np

    from grouped_gemm_gpu_kernel_amd import _lib

    n = ex.launched_work_tiles()
    P = _lib.GGK_PHASE_COUNT
    buf = torch.zeros(P * max(1, n), dtype=torch.int64, device="cuda")
    launches = []
    for _ in range(runs):
        buf.zero_()
        st = ex.run_traced(0, 0, None, buf.data_ptr())
        if st != 0:
            raise RuntimeError(f"traced run hipError_t {st}")
        torch.cuda.synchronize()
        ph = buf.cpu().numpy().reshape(-1, P)[:n]
        ph = ph[ph[:, _lib.GGK_PHASE_START] > 0]
        launches.append((float(ph[:, _lib.GGK_PHASE_EPILOGUE_END].max() - ph[:, _lib.GGK_PHASE_START].min()), ph))
    launches.sort(key=lambda x: x[0])
    ph = launches[len(launches) // 2][1]
    who = ph[:, _lib.GGK_PHASE_WHO]
    wg = who & 0xFFFFF
    half = (who >> 20) & 3
    rows = (who >> 22) & 0xFFF
    cols = (who >> 34) & 0xFFF
    stages = (who >> 46) & 0x1FFFF
    start, first = ph[:, _lib.GGK_PHASE_START], ph[:, _lib.GGK_PHASE_FIRST_STAGE]
    kl, ke = ph[:, _lib.GGK_PHASE_K_LOOP], ph[:, _lib.GGK_PHASE_K_END]
    epi, epi_end = ph[:, _lib.GGK_PHASE_EPILOGUE], ph[:, _lib.GGK_PHASE_EPILOGUE_END]
    # gap: from a tile's last epilogue wave to the same workgroup's next tile start (core clocks of
    # one workgroup's CU, ordered by the wall clock)
    gap = np.full(len(ph), np.nan)
    order = np.lexsort((ph[:, _lib.GGK_PHASE_WALL], wg))
    same = wg[order][1:] == wg[order][:-1]
    gap[order[:-1][same]] = start[order[1:][same]] - epi_end[order[:-1][same]]
    bm = int(rows.max()) if len(rows) else 0
    bn = int(cols.max()) if len(cols) else 0
    classes = {
        "whole": (half == 0) & (rows > bm // 2) & (cols > bn // 2),
        "rows_le_half": (half == 0) & (rows <= bm // 2) & (cols > bn // 2),
        "cols_le_half": (half == 0) & (rows > bm // 2) & (cols <= bn // 2),
        "both_le_half": (half == 0) & (rows <= bm // 2) & (cols <= bn // 2),
        "row_halves": half > 0,
        "all": np.ones(len(ph), bool),
    }
    out = {"work_tiles": int(len(ph)), "work_tile_rows": bm, "work_tile_cols": bn}
    # The middle k-loop step of each tile, per wave: issuing the next stage's loads, issuing the
    # MFMAs and fragment reads, the wait for the loads, the closing barrier (mean over the waves),
    # and the step from the first wave's start to the last wave's barrier.
    step = ph[:, _lib.GGK_PHASE_STEP:].reshape(len(ph), _lib.GGK_PHASE_STEP_WAVES,
                                                _lib.GGK_PHASE_STEP_MARKS).astype(np.float64)
    stamped = (step[:, :, 0] > 0)
    for name, sel in classes.items():
        if not sel.any():
            continue
        g = gap[sel]
        g = g[~np.isnan(g)]
        st = sel & stamped.any(axis=1)
        step_row = None
        if st.any():
            w = stamped[st]
            parts = [np.where(w, step[st, :, i + 1] - step[st, :, i], np.nan) for i in range(4)]
            span = (np.where(w, step[st, :, 4], -np.inf).max(axis=1) - np.where(w, step[st, :, 0], np.inf).min(axis=1))
            step_row = {"issue": round(float(np.nanmean(parts[0]))), "mfma": round(float(np.nanmean(parts[1]))),
                        "wait": round(float(np.nanmean(parts[2]))), "barrier": round(float(np.nanmean(parts[3]))),
                        "barrier_max_wave": round(float(np.nanmean(np.nanmax(parts[3], axis=1)))),
                        "step": round(float(span.mean()))}
        out[name] = {
            "tiles": int(sel.sum()), "stages": round(float(stages[sel].mean()), 2),
            "first_stage": round(float((first - start)[sel].mean())),
            "k_loop_start": round(float((kl - start)[sel].mean())),
            "k_loop_per_stage": round(float((ke - kl)[sel].sum() / max(1, stages[sel].sum()))),
            "hand_over": round(float((epi - ke)[sel].mean())),
            "epilogue": round(float((epi_end - epi)[sel].mean())),
            "next_start": round(float(g.mean())) if g.size else None,
            "middle_step": step_row,
        }
    tile = (epi_end - start).sum()
    out["share"] = {"to_k_loop": round(float((kl - start).sum() / tile), 4),
                    "k_loop": round(float((ke - kl).sum() / tile), 4),
                    "hand_over": round(float((epi - ke).sum() / tile), 4),
                    "epilogue": round(float((epi_end - epi).sum() / tile), 4)}
    return out


def shard_shares(torch, probs, cfg, mode, ranks: int, stream, steps: int, warmup: int, warm_seconds: float,
                 whole_ms: float, flops: float) -> dict:
    """One GPU's share of an N-way data-parallel split, for every rank: plan_shards splits the set
    (whole problems; column ranges of the ones above a rank's share), and each rank's share is built
    and timed on this GPU as the rank would run it on its own.  The N shares of a step would run
    side by side, so the slowest one sets the step: balance = mean / max share time, and
    whole_over_max = the unsplit set's time on one GPU over the slowest share's.  Nothing is
    exchanged between ranks (problems are independent), so no collective is timed."""
    from grouped_gemm_gpu_kernel_amd import api

    pieces = api.plan_shards(probs, cfg, ranks)
    shares, executors = [], []
    for r in range(ranks):
        share = [api.shard_problem(probs[p.problem], p) for p in pieces if p.rank == r]
        ex = api.GroupedGemmExecutor()
        st = ex.build(api.prepare_problem_set(share, cfg, mode), cfg)
        if st != 0:
            raise RuntimeError(f"rank {r} build: hipError_t {st}")
        shares.append(share)
        executors.append(ex)
    # Two passes over the ranks, the faster time of each: the first share timed after the set's
    # own runs otherwise reads slow now and then.
    best_ms = [math.inf] * ranks
    for _ in range(2):
        for r, ex in enumerate(executors):
            warm_clock(torch, lambda: ex.run(stream), warm_seconds)
            best_ms[r] = min(best_ms[r], time_runs(torch, lambda: ex.run(stream), steps, warmup))
    for ex in executors:
        ex.close()
    rank_ms = [round(ms, 4) for ms in best_ms]
    rank_tflops = [round(api.total_flops(share) / (ms * 1e-3) / 1e12, 2) for share, ms in zip(shares, best_ms)]
    slowest = max(rank_ms)
    return {"ranks": ranks, "pieces": len(pieces), "split_problems": len(pieces) - len({p.problem for p in pieces}),
            "rank_ms": rank_ms, "rank_tflops": rank_tflops, "max_ms": slowest,
            "balance": round(sum(rank_ms) / (ranks * slowest), 4), "whole_ms": round(whole_ms, 4),
            "whole_over_max": round(whole_ms / slowest, 3),
            "aggregate_tflops_at_max": round(flops / (slowest * 1e-3) / 1e12, 2)}


def torch_binding(torch, dw, cfg, mode, stream, steps: int, warmup: int, warm_seconds: float) -> dict:
    """The same workload through the torch binding: GroupedGemmPlan.run() (device time, events on
    the launch stream) and one-shot run_grouped_gemm (host wall time per call: prepare, upload,
    launch, wait, release)."""
    from grouped_gemm_gpu_kernel_amd import torch_ops

    a, b, c, d, alpha, beta = dw.tensors()
    plan = torch_ops.GroupedGemmPlan(a, b, c if dw.has_c else None, d, alpha, beta, sort_mode=mode, config=cfg)
    warm_clock(torch, lambda: plan.run(stream), warm_seconds)
    plan_ms = time_runs(torch, lambda: plan.run(stream), steps, warmup)
    plan.close()
    calls = 5
    torch_ops.run_grouped_gemm(a, b, c if dw.has_c else None, alpha, beta, sort_mode=mode, config=cfg, out=d)
    t0 = time.perf_counter()
    for _ in range(calls):
        torch_ops.run_grouped_gemm(a, b, c if dw.has_c else None, alpha, beta, sort_mode=mode, config=cfg, out=d)
    one_shot_ms = (time.perf_counter() - t0) * 1e3 / calls
    out = {"sort_mode": mode.name, "plan_run_ms": round(plan_ms, 4), "one_shot_wall_ms": round(one_shot_ms, 3)}
    print(f"# torch binding {out}", file=sys.stderr, flush=True)
    return out


def moe_device_prepare(torch, dw, spec, cfg, mode, stream, steps: int, warmup: int, warm_seconds: float):
    """A group whose problems share n and k and read no C (moe64) through the device-side prepare:
    the expert rows of A stacked into one [T, k] tensor, B as [E, k, n], the int32 counts on the
    GPU; prepare kernel + grouped launch per run (device time, events on the launch stream), next
    to the grouped launch alone after the host prepare.  None for other workloads."""
    import numpy as np

    from grouped_gemm_gpu_kernel_amd import torch_ops

    n, k = int(spec.n[0]), int(spec.k[0])
    if not ((spec.n == n).all() and (spec.k == k).all()) or dw.has_c:
        return None
    rows = np.asarray(spec.m, dtype=np.int64)
    a_pool = dw.a.view(torch.float16)
    b_pool = dw.b.view(torch.float16)
    a = torch.cat([a_pool[int(o):int(o) + int(m) * k].view(int(m), k) for o, m in zip(dw.a_off, rows)])
    if all(int(o) == i * k * n for i, o in enumerate(dw.b_off)):
        b = b_pool[:spec.count * k * n].view(spec.count, k, n)  # the pool already is [E, K, N]
    else:
        b = torch.stack([b_pool[int(o):int(o) + k * n].view(k, n) for o in dw.b_off])
    d = torch.empty(int(rows.sum()), n, dtype=torch.float32, device=a.device)
    counts = torch.from_numpy(rows.astype(np.int32)).cuda()
    plan = torch_ops.MoeGroupedGemmPlan(a, b, d, None, float(spec.alpha[0]), float(spec.beta[0]), sort_mode=mode,
                                        config=cfg)
    warm_clock(torch, lambda: plan.run(counts, stream), warm_seconds)
    ms = time_runs(torch, lambda: plan.run(counts, stream), steps, warmup)
    status = plan.status()
    plan.close()
    del a, b, d
    out = {"experts": spec.count, "sort_mode": mode.name, "prepare_plus_gemm_ms": round(ms, 4), "status": status}
    print(f"# moe device prepare {out}", file=sys.stderr, flush=True)
    return out


def vendor_baseline(spec, config_name: str, sort_mode: int, steps: int, warmup: int):
    """The same problem set through hipBLASLt, in a child process (see grouped_gemm_gpu_kernel_amd/
    vendor.py): its grouped GEMM (every heuristic candidate timed, the fastest kept) and one vendor
    GEMM per problem, each checked element by element against this library's D on the same
    operands.  Rows read {"error": ...} where the vendor library has no algorithm."""
    from grouped_gemm_gpu_kernel_amd import vendor

    try:
        res = vendor.run(spec, steps=steps, warmup=warmup, config=config_name, sort_mode=sort_mode)
    except Exception as exc:  # reported in the JSON line, not fatal to the bench
        res = {"error": str(exc)}
    print(f"# vendor {res}", file=sys.stderr, flush=True)
    return res


def host_cpu_info() -> dict:
    """The host the CPU baseline ran on: CPU model, logical CPUs, the CPUs this process may use and
    the OpenMP thread setting."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def cpu_gemm_sample(dw, spec, seconds: float, threads, full: bool = False) -> dict:
    """The oracle's host GEMM (tests/test_correctness.cu:85-102) over the workload's problems in index
    order until `seconds` have passed: threads=None runs the literal single-thread i-j-k loop, an int
    the OpenMP i-k-j form on that many threads (bit-identical per element).  Each call computes a
    block of rows of one problem (full=True: every row of every problem, no time limit), so one large
    problem cannot overrun the budget; rows give the same per-element arithmetic as the whole."""
    from oracle import oracle as O

    done_flops, elapsed, problems, rows_done = 0.0, 0.0, 0, 0
    for i in range(spec.count):
        m, n, k = int(spec.m[i]), int(spec.n[i]), int(spec.k[i])
        if m <= 0 or n <= 0:
            continue
        per_row = 2.0 * n * k
        # about 5e7 flops per call single-threaded, `threads` times that in parallel
        rows = m if full else max(1, min(m, int(5e7 * (threads or 1) / max(per_row, 1.0)) + 1))
        a = dw.host_a(i)[:rows * max(1, k)]
        b = dw.host_b(i)
        c = dw.host_c(i)
        c = c[:rows * n] if c is not None else None
        t0 = time.perf_counter()
        O.gemm(rows, n, k, a, max(1, k), b, max(1, n), c, max(1, n), float(spec.alpha[i]), float(spec.beta[i]),
               threads=threads)
        elapsed += time.perf_counter() - t0
        done_flops += per_row * rows
        problems += 1
        rows_done += rows
        if not full and elapsed >= seconds:
            break
    return {"tflops": done_flops / elapsed / 1e12 if elapsed > 0 else None, "gflop": round(done_flops / 1e9, 3),
            "seconds": round(elapsed, 2), "problems": problems, "rows": rows_done}


def cpu_baseline(dw, spec, seconds: float, full: bool = False):
    """CPU baseline on this host's cores: the OpenMP form on every thread OpenMP is given
    (OMP_NUM_THREADS, else every CPU this process may use) is `value`; the literal single-thread loop
    rides along, timed on the 16-problem plumbing set in full and on a sample of this workload.
    full=True times the whole workload in both forms instead of samples."""
    from grouped_gemm_gpu_kernel_amd.workloads import DeviceWorkload, make_spec

    info = host_cpu_info()
    threads = int(info["omp_num_threads"] or info["affinity_cpus"])
    omp = cpu_gemm_sample(dw, spec, seconds / 2, threads, full)
    single = cpu_gemm_sample(dw, spec, seconds / 2, None, full)
    plumbing_spec = make_spec("plumbing16")
    plumbing = cpu_gemm_sample(DeviceWorkload(plumbing_spec), plumbing_spec, 0.0, None, True)

    def what(r):
        return ("all rows of all" if full else f"row blocks of the first {r['problems']} of {spec.count}") + \
            f" problems ({r['gflop']} GFLOP, {r['seconds']} s)"

    out = {
        "value": round(omp["tflops"], 6) if omp["tflops"] else None,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{spec.name}: {what(omp)}; oracle FP32 host GEMM, OpenMP i-k-j form on {threads} threads",
        "host": info,
        "single_thread": {
            "tflops": round(single["tflops"], 6) if single["tflops"] else None,
            "sample": f"{spec.name}: {what(single)}; literal i-j-k loop, 1 thread"},
        "single_thread_plumbing16": {
            "tflops": round(plumbing["tflops"], 6) if plumbing["tflops"] else None,
            "ms": round(plumbing["seconds"] * 1e3, 1), "gflop": plumbing["gflop"]},
    }
    print(f"# cpu baseline {out}", file=sys.stderr, flush=True)
    return out


def _csv_rows(path: Path):
    import csv
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


TRACED_KERNEL = r"gg_grouped_kernel<\d+,\s*\d+,\s*true"


def _dispatches(d: Path):
    """[(dispatch id, kernel name, {"duration_us" or counter: value})] from the rocprofv3 CSV output
    under d (kernel traces and counter collections), in dispatch order; a counter's rows of one
    dispatch are summed."""
    per = {}
    for trace in sorted(d.rglob("*kernel_trace.csv")):
        for r in _csv_rows(trace):
            e = per.setdefault(int(r["Dispatch_Id"]), (r["Kernel_Name"], {}))
            e[1]["duration_us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    for cc in sorted(d.rglob("*counter_collection.csv")):
        for r in _csv_rows(cc):
            e = per.setdefault(int(r["Dispatch_Id"]), (r["Kernel_Name"], {}))
            e[1][r["Counter_Name"]] = e[1].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [(i, per[i][0], per[i][1]) for i in sorted(per)]


def _segments(dispatches, kernel_filter: str, names, last: int):
    """{(kernel, segment name): {metric: [values]}} for the kernels matching kernel_filter.  With
    names, the dispatches are cut into segments at each run of traced grouped-kernel dispatches
    (bench.py makes them after each sort mode's timed runs, so segment i holds mode i's clock
    warm-up, warm-up and timed runs) and only the last `last` dispatches of each segment count (0:
    all of them); dispatches after the last cut form a segment named "after".  Without names: one
    segment "all"."""
    import re
    pat, cut = re.compile(kernel_filter), re.compile(TRACED_KERNEL)
    segs, current, seg, in_cut = {}, {}, 0, False

    def close(name):
        for kname, rows in current.items():
            rows = rows[-last:] if last > 0 else rows
            out = segs.setdefault((kname, name), {})
            for metrics in rows:
                for key, v in metrics.items():
                    out.setdefault(key, []).append(v)

    for _, kname, metrics in dispatches:
        if names and cut.search(kname):
            if not in_cut:
                close(names[seg] if seg < len(names) else f"segment{seg}")
                current, seg, in_cut = {}, seg + 1, True
        elif pat.search(kname):
            current.setdefault(kname, []).append(metrics)
            in_cut = False
    close("after" if names else "all")
    return segs


def _stats(v) -> str:
    return f"dispatches {len(v)}  mean {sum(v) / len(v):.6g}  min {min(v):.6g}  max {max(v):.6g}"


MFMA_CYCLES = 32        # v_mfma_f32_32x32x16_f16: cycles a SIMD is busy per instruction
MFMA_MACS = 32 * 32 * 16
SIMDS_PER_CU = 4
XCDS = 8
CUS = 256


def _derived(metrics, workload) -> list:
    """Ratios of the counters of one sort mode (means per dispatch):
      mfma_busy        SQ_VALU_MFMA_BUSY_CYCLES / (4 SIMDs x SQ_BUSY_CU_CYCLES): share of the SIMD
                       cycles of busy CUs spent in MFMA;
      mfma_executed    SQ_VALU_MFMA_BUSY_CYCLES / 32 cycles per 32x32x16 MFMA, against the
                       workload's useful MFMAs (sum m n k / 16384): padding of partial tiles;
      l2_hit           TCC_HIT / (TCC_HIT + TCC_MISS);
      lds_bank_conflict  SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE (cycles);
      clock_ghz        GRBM_GUI_ACTIVE / 8 XCDs / the dispatch's duration (when traced);
    and, per CU (GRBM_GUI_ACTIVE / 8 cycles of the dispatch, 256 CUs):
      ta_busy          TA_TA_BUSY / (256 x cycles): share of cycles the address unit is busy;
      l1_l2_latency    TCP_TCC_READ_REQ_LATENCY / TCP_TCC_READ_REQ: cycles per 128-byte L1 -> L2
                       read request;
      l1_l2_in_flight  TCP_TCC_READ_REQ_LATENCY / (256 x cycles): mean read requests in flight per
                       CU (Little's law);
      l1_l2_bytes_per_cycle  128 x TCP_TCC_READ_REQ / (256 x cycles)."""
    mean = {k: sum(v) / len(v) for k, v in metrics.items()}
    out = []
    if "SQ_VALU_MFMA_BUSY_CYCLES" in mean and mean.get("SQ_BUSY_CU_CYCLES"):
        out.append(f"mfma_busy: {mean['SQ_VALU_MFMA_BUSY_CYCLES'] / (SIMDS_PER_CU * mean['SQ_BUSY_CU_CYCLES']):.4f}")
    if "SQ_VALU_MFMA_BUSY_CYCLES" in mean and workload:
        from grouped_gemm_gpu_kernel_amd.workloads import make_spec
        useful = make_spec(workload).flops() / 2 / MFMA_MACS
        executed = mean["SQ_VALU_MFMA_BUSY_CYCLES"] / MFMA_CYCLES
        out.append(f"mfma_executed: {executed:.6g} useful: {useful:.6g} ratio: {executed / useful:.4f}")
    if "TCC_HIT_sum" in mean and "TCC_MISS_sum" in mean:
        tot = mean["TCC_HIT_sum"] + mean["TCC_MISS_sum"]
        if tot > 0:
            out.append(f"l2_hit: {mean['TCC_HIT_sum'] / tot:.4f}")
    if "SQ_LDS_BANK_CONFLICT" in mean and mean.get("SQ_LDS_IDX_ACTIVE"):
        out.append(f"lds_bank_conflict: {mean['SQ_LDS_BANK_CONFLICT'] / mean['SQ_LDS_IDX_ACTIVE']:.4f}")
    if "GRBM_GUI_ACTIVE" in mean and mean.get("duration_us"):
        out.append(f"clock_ghz: {mean['GRBM_GUI_ACTIVE'] / XCDS / (mean['duration_us'] * 1e3):.3f}")
    cu_cycles = CUS * mean["GRBM_GUI_ACTIVE"] / XCDS if mean.get("GRBM_GUI_ACTIVE") else None
    if cu_cycles and "TA_TA_BUSY" in mean:
        out.append(f"ta_busy: {mean['TA_TA_BUSY'] / cu_cycles:.4f}")
    if mean.get("TCP_TCC_READ_REQ") and "TCP_TCC_READ_REQ_LATENCY" in mean:
        out.append(f"l1_l2_latency: {mean['TCP_TCC_READ_REQ_LATENCY'] / mean['TCP_TCC_READ_REQ']:.1f}")
        if cu_cycles:
            out.append(f"l1_l2_in_flight: {mean['TCP_TCC_READ_REQ_LATENCY'] / cu_cycles:.1f}")
            out.append(f"l1_l2_bytes_per_cycle: {128 * mean['TCP_TCC_READ_REQ'] / cu_cycles:.2f}")
    return out


def profile_summary(dirs, kernel_filter: str, names=(), last: int = 0, workload=None) -> int:
    """Prints what rocprofv3 --output-format csv folders hold for kernels matching kernel_filter:
    per dispatch, mean/min/max of the duration in us (kernel trace) and of each counter (counter
    collection), per sort mode when the mode names are given (see _segments), and the ratios of
    _derived (useful MFMAs from `workload`)."""
    for d in dirs:
        d = Path(d)
        print(f"== {d}")
        for (kname, seg), metrics in _segments(_dispatches(d), kernel_filter, names, last).items():
            for key, v in sorted(metrics.items()):
                print(f"{kname} [{seg}] {key}: {_stats(v)}")
            for line in _derived(metrics, workload):
                print(f"{kname} [{seg}] {line}")
    if len(dirs) > 1:
        # Counters collected in separate runs of the same command: ratios across them.
        merged = {}
        for d in dirs:
            for key, metrics in _segments(_dispatches(Path(d)), kernel_filter, names, last).items():
                for name, v in metrics.items():
                    merged.setdefault(key, {}).setdefault(name, []).extend(v)
        print("== all folders")
        for (kname, seg), metrics in merged.items():
            for line in _derived(metrics, workload):
                print(f"{kname} [{seg}] {line}")
    return 0


def traffic_summary(dirs, copy_mib: int, workload: str, kernel_filter: str, names, last: int) -> int:
    """HBM bytes per launch from FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each divided by what
    the same counter reads per byte of a plain device-to-device copy of copy_mib MiB (the copy reads
    and writes copy_mib MiB once), per sort mode.  Prints the lines of a
    profiles/gg_grouped_kernel_<workload>_hbm_traffic.txt file."""
    from grouped_gemm_gpu_kernel_amd.workloads import make_spec

    fetch_dir, write_dir, copy_fetch_dir, copy_write_dir = (Path(x) for x in dirs)
    copy_bytes = copy_mib << 20

    def copy_reading(d, counter):
        segs = _segments(_dispatches(d), "copyBuffer", (), 0)
        vals = [v for m in segs.values() for v in m.get(counter, [])]
        if not vals:
            raise SystemExit(f"{d}: no copyBuffer dispatch with {counter}")
        return sum(vals) / len(vals), len(vals)

    cf, ncf = copy_reading(copy_fetch_dir, "FETCH_SIZE")
    cw, ncw = copy_reading(copy_write_dir, "WRITE_SIZE")
    fetch_scale = cf * 1024 / copy_bytes
    write_scale = cw * 1024 / copy_bytes
    fsegs = _segments(_dispatches(fetch_dir), kernel_filter, names, last)
    wsegs = _segments(_dispatches(write_dir), kernel_filter, names, last)
    algo = make_spec(workload).algorithmic_bytes()
    print(f"# copy calibration, {copy_mib} MiB read + {copy_mib} MiB written per dispatch: FETCH_SIZE "
          f"{cf:.0f} KiB ({ncf} dispatches) -> fetch_scale {fetch_scale:.4f}; WRITE_SIZE {cw:.0f} KiB "
          f"({ncw} dispatches) -> write_scale {write_scale:.4f}")
    print("# traffic = FETCH_SIZE * 1024 / fetch_scale + WRITE_SIZE * 1024 / write_scale, bytes per launch")
    print(f"algorithmic_bytes: {algo:.0f}")
    print(f"fetch_scale: {fetch_scale:.4f}")
    print(f"write_scale: {write_scale:.4f}")
    for (kname, seg), fm in fsegs.items():
        wm = wsegs.get((kname, seg), {})
        if "FETCH_SIZE" not in fm or "WRITE_SIZE" not in wm:
            continue
        fv, wv = fm["FETCH_SIZE"], wm["WRITE_SIZE"]
        fb = sum(fv) / len(fv) * 1024 / fetch_scale
        wb = sum(wv) / len(wv) * 1024 / write_scale
        print(f"# {seg}: {kname}")
        print(f"#   FETCH_SIZE KiB {_stats(fv)}")
        print(f"#   WRITE_SIZE KiB {_stats(wv)}")
        print(f"fetch_bytes_per_launch {seg}: {fb:.0f}")
        print(f"write_bytes_per_launch {seg}: {wb:.0f}")
        print(f"traffic_bytes_per_launch {seg}: {fb + wb:.0f}")
        print(f"traffic_over_algorithmic {seg}: {(fb + wb) / algo:.3f}")
    return 0


def committed_traffic(workload: str, mode: str):
    """HBM bytes per launch of the grouped kernel on `workload` in sort mode `mode`, from the committed
    rocprofv3 summary profiles/gg_grouped_kernel_<workload>_hbm_traffic.txt (FETCH_SIZE and WRITE_SIZE
    per dispatch, each scaled by the same counter's reading for a plain copy of known size), or None.
    The file holds one `traffic_bytes_per_launch <mode>: <bytes>` line per sort mode."""
    path = ROOT / "profiles" / f"gg_grouped_kernel_{workload}_hbm_traffic.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch ") and ":" in line:
            key, value = line.split(":", 1)
            if key.split()[1] == mode:
                try:
                    return {"bytes": float(value.strip()), "mode": mode, "source": str(path.relative_to(ROOT))}
                except ValueError:
                    return None
    return None


def main() -> int:
    args = parse_args()
    names = [x for x in args.modes_of_segments.split(",") if x]
    if args.profile_summary:
        return profile_summary(args.profile_summary, args.kernel, names, args.last,
                               args.workload if args.workload_given else None)
    if args.traffic_summary:
        return traffic_summary(args.traffic_summary, args.copy_mib, args.workload, args.kernel, names, args.last)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the grouped GEMM shards "
              "problems across GPUs with no exchange step, see the design notes.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from grouped_gemm_gpu_kernel_amd import api
    from grouped_gemm_gpu_kernel_amd.api import GroupedGemmExecutor, KernelConfig, SortMode
    from grouped_gemm_gpu_kernel_amd.workloads import DeviceWorkload, make_spec

    torch.cuda.set_device(0)
    if args.calibrate_copy:
        return calibrate_copy(torch, args.calibrate_copy)
    spec = make_spec(args.workload)
    config_name = args.config or spec.config
    cfg = KernelConfig.named(config_name, use_tensor_cores=not args.fma)
    dw = DeviceWorkload(spec)
    probs = dw.problems()
    flops = spec.flops()
    algo_bytes = spec.algorithmic_bytes()
    print(f"# workload {spec.name}: {spec.count} problems, {flops / 1e9:.2f} GFLOP, "
          f"{algo_bytes / 1e9:.3f} GB algorithmic, config {config_name}", file=sys.stderr, flush=True)

    modes = [SortMode(int(x)) for x in args.modes.split(",")]
    per_mode = []
    # A stream of our own at default priority: the events that time a run are recorded on the stream
    # the kernel is launched on.
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    # Every mode's executor is built first (host work), then each is timed right after an untimed
    # stretch of its own launches (warm_clock); without it a mode reads 5-10% slower depending only
    # on its place in the order.
    # prep_ms is the reference benchmark's span (bench/benchmark_grouped_gemm.cu:622-632):
    # prepare_problem_set + GroupedGemmExecutor::build, here the two C calls on a problem array
    # converted from Python beforehand.  The first build in a process also queries the device and
    # the kernel's occupancy once (cached afterwards); it is timed apart as first_build_ms.
    first_build_ms = timed_prepare_and_build(probs, cfg, modes[0])[1]
    built = []
    for mode in modes:
        ex, prep_ms = timed_prepare_and_build(probs, cfg, mode)
        prep = api.prepare_problem_set(probs, cfg, mode)
        built.append((mode, prep, ex, prep_ms))

    timed = []
    for i, (mode, prep, ex, prep_ms) in enumerate(built):
        warm_clock(torch, lambda: ex.run(stream), args.clock_warmup if i == 0 else min(args.clock_warmup, 0.1))
        ms = time_runs(torch, lambda: ex.run(stream), args.steps, args.warmup)
        # The traced runs right after a mode's timed runs also mark, in a profiler's dispatch list,
        # where that mode's runs end (--profile-summary / --traffic-summary --modes-of-segments).
        timed.append((ms, measured_tail_idle(torch, ex), tile_phases(torch, ex) if args.phases else None))
    for (mode, prep, ex, prep_ms), (ms, tail_idle, phases) in zip(built, timed):
        row = {
            "mode": api.sort_mode_name(mode), "prep_ms": round(prep_ms, 3), "kernel_ms": round(ms, 4),
            "tflops": round(flops / (ms * 1e-3) / 1e12, 2), "tiles": prep.total_tiles,
            "grid_ctas": ex.grid_ctas(), "launches": 1,
            "tail_share": round(api.tail_work_share(prep, cfg), 4), "tail_idle_measured": round(tail_idle, 4),
        }
        if phases is not None:
            row["tile_phases"] = phases
            print(f"# tile phases {row['mode']}: {json.dumps(phases)}", file=sys.stderr, flush=True)
        per_mode.append(row)
        print(f"# {row}", file=sys.stderr, flush=True)
        ex.close()
    best = headline_mode(per_mode, [ms for ms, _, _ in timed])

    baseline = None
    if not args.no_baseline:
        bsteps = max(1, min(args.steps, 20))
        warm_clock(torch, lambda: api.run_baseline_per_problem(probs, cfg, stream), min(args.clock_warmup, 0.1))
        bms = time_runs(torch, lambda: api.run_baseline_per_problem(probs, cfg, stream), bsteps, 2)
        baseline = {"mode": "baseline_per_problem", "kernel_ms": round(bms, 4),
                    "tflops": round(flops / (bms * 1e-3) / 1e12, 3),
                    "launches": api.count_non_empty_problems(probs, cfg)}
        print(f"# {baseline}", file=sys.stderr, flush=True)

    best_mode = next(m for m in modes if api.sort_mode_name(m) == best[0]["mode"])
    warm_s = min(args.clock_warmup, 0.1)
    moe_device = None if (args.fma or args.no_moe_device) else moe_device_prepare(
        torch, dw, spec, cfg, best_mode, stream, args.steps, args.warmup, warm_s)
    vendor_rows = None if (args.no_vendor or args.fma) else vendor_baseline(spec, config_name, int(best_mode),
                                                                            args.steps, args.warmup)
    torch_op = None if args.no_torch_op else torch_binding(torch, dw, cfg, best_mode, stream, args.steps,
                                                          args.warmup, warm_s)
    cpu = None if args.no_cpu else cpu_baseline(dw, spec, args.cpu_seconds, args.cpu_full)
    shards = None
    if args.shards:
        shards = []
        for ranks in (int(x) for x in args.shards.split(",")):
            shards.append(shard_shares(torch, probs, cfg, best_mode, ranks, stream, args.steps, args.warmup,
                                       warm_s, best[1], flops))
            print(f"# shards {shards[-1]}", file=sys.stderr, flush=True)

    row, ms = best
    tflops = flops / (ms * 1e-3) / 1e12
    achieved_gbs = algo_bytes / (ms * 1e-3) / 1e9
    mfma_frac = tflops / MFMA_PEAK_TFLOPS
    hbm_frac = achieved_gbs / HBM_PEAK_GBS
    ridge = MFMA_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
    bound = "hbm" if flops / algo_bytes < ridge else "mfma"
    traffic = committed_traffic(spec.name, row["mode"]) if not args.fma else None
    if bound == "hbm":
        roofline = {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(hbm_frac, 4), "traffic": round(traffic["bytes"]) if traffic else None}
    else:
        roofline = {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(mfma_frac, 4), "traffic": round(traffic["bytes"]) if traffic else None}
    if traffic:
        roofline["traffic_source"] = f"{traffic['source']} ({traffic['mode']})"
        # FETCH_SIZE / WRITE_SIZE count what L2 moves to and from the data fabric: requests the
        # 256 MB MALL serves count as fetched, and no counter here tells them from DRAM reads.
        roofline["traffic_counts"] = "L2 <-> fabric bytes (MALL hits included)"
        roofline["algorithmic_bytes"] = algo_bytes
    out = {
        "metric": "grouped TFLOP/s + % FP16 MFMA peak on mixed-512, 1 MI355X; tail_share",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded; shapes from numpy RandomState, operands from a counter hash on the GPU)",
        "config": {"workload": spec.name, "problems": spec.count, "cta": config_name,
                   "path": "fma" if args.fma else "mfma", "accumulate": "fp32", "best_sort_mode": row["mode"],
                   "gflop": round(flops / 1e9, 3), "algorithmic_gb": round(algo_bytes / 1e9, 4)},
        "mfma_peak_frac": round(mfma_frac, 4),
        "hbm_roofline_frac": round(hbm_frac, 4),
        "prep_ms": row["prep_ms"],
        "first_build_ms": round(first_build_ms, 3),
        "tail_share": row["tail_share"],
        "tail_idle_measured": row["tail_idle_measured"],
        "per_mode": per_mode,
        "baseline_per_problem": baseline,
        "speedup_vs_per_problem_baseline": round(baseline["kernel_ms"] / ms, 2) if baseline else None,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "torch_op": torch_op,
        "vendor_hipblaslt": vendor_rows,
        "moe_device_prepare": moe_device,
    }
    if shards is not None:
        out["shards"] = shards
    if args.table:
        print(f"{'mode':24}{'prep_ms':>10}{'kernel_ms':>11}{'tflops':>10}{'tiles':>8}{'grid':>7}{'launches':>10}"
              f"{'tail_share':>12}", file=sys.stderr)
        for r in per_mode + ([baseline] if baseline else []):
            print(f"{r['mode']:24}{r.get('prep_ms', 0):>10.3f}{r['kernel_ms']:>11.4f}{r['tflops']:>10.2f}"
                  f"{r.get('tiles', 0):>8}{r.get('grid_ctas', 0):>7}{r['launches']:>10}{r.get('tail_share', 0):>12.4f}",
                  file=sys.stderr)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
