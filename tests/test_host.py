"""Host-side parity of the library, on the CPU: prepare_problem_set (sort permutations, tile offsets,
total tiles), tile counts, sort-mode names and empty-problem counting must equal the oracle bit for
bit, and the executor's launch plan (variant, schedule, grid, work table) its restatement in
schedule_plan.py.  These entry points never touch the GPU."""
import ctypes
import json
from pathlib import Path

import numpy as np
import pytest

from grouped_gemm_gpu_kernel_amd import api
from grouped_gemm_gpu_kernel_amd.api import KernelConfig, ProblemDesc, SortMode
from oracle import oracle as O

CONFIGS = ["64x64x16", "128x64x32", "64x128x32"]


def _problems(m, n, k):
    # Distinct fake pointers: prepare must carry them through unchanged.
    return [ProblemDesc(int(mm), int(nn), int(kk), a=0x1000 + 16 * i, b=0x20000 + 16 * i, c=(0x300000 + 16 * i) if i % 3 else None,
                        d=0x4000000 + 16 * i, lda=max(1, int(kk)), ldb=max(1, int(nn)), ldc=max(1, int(nn)),
                        ldd=max(1, int(nn)), alpha=0.5 + i, beta=0.25 * i)
            for i, (mm, nn, kk) in enumerate(zip(m, n, k))]


@pytest.mark.parametrize("config", CONFIGS)
def test_prepare_matches_oracle(config):
    cfg = KernelConfig.named(config)
    rng = np.random.default_rng(11)
    for trial in range(40):
        cnt = int(rng.integers(0, 600))
        hi = int(rng.choice([4, 70, 700, 5000]))
        m = rng.integers(0, hi, cnt)
        n = rng.integers(0, hi, cnt)
        k = rng.integers(0, hi, cnt)
        probs = _problems(m, n, k)
        for mode in SortMode:
            got = api.prepare_problem_set(probs, cfg, mode)
            perm, offs, total = O.prepare(m, n, k, cfg.cta_m, cfg.cta_n, int(mode))
            assert got.sorted_to_original == list(perm)
            assert got.tile_offsets == list(offs)
            assert got.total_tiles == total
            assert got.sorted_problems == [probs[i] for i in perm]


def test_prepare_reference_shapes_and_bench_workloads():
    """The reference test's shapes (tests/test_correctness.cu:313-322) and the reference bench
    generators (bench/benchmark_grouped_gemm.cu:368-443) at several seeds."""
    cases = [([64, 128, 45, 17, 192, 16, 0, 64], [64, 64, 81, 23, 32, 256, 64, 0], [64, 96, 37, 9, 64, 48, 16, 16])]
    for wl in ("small", "mixed", "tail"):
        for seed in (42, 20260328):
            cases.append(O.bench_shapes(wl, 512, seed))
    for m, n, k in cases:
        probs = _problems(m, n, k)
        for config in CONFIGS:
            cfg = KernelConfig.named(config)
            for mode in SortMode:
                got = api.prepare_problem_set(probs, cfg, mode)
                perm, offs, total = O.prepare(m, n, k, cfg.cta_m, cfg.cta_n, int(mode))
                assert got.sorted_to_original == list(perm) and got.tile_offsets == list(offs)
                assert api.tail_work_share(got, cfg) == pytest.approx(
                    O.tail_work_share(np.asarray(k)[perm], offs, cfg.cta_k), abs=0, rel=1e-15)


def test_published_rows_through_library():
    """bench/results_20260331/results.csv, the 256-problem seed-42 rows of the small and tail
    workloads: the library's prepare gives the published tile totals and tail shares in every mode."""
    rows = json.loads((Path(__file__).resolve().parent / "golden" / "published_bench_rows.json").read_text())["rows"]
    checked = 0
    for row in rows:
        if row["workload"] == "mixed" or row["problems"] != 256 or row["seed"] != 42:
            continue
        if row["mode"] == "baseline_per_problem" or row["persistent_ctas"]:
            continue
        m, n, k = O.bench_shapes(row["workload"], 256, 42)
        cfg = KernelConfig.named(row["config"])
        mode = next(md for md in SortMode if api.sort_mode_name(md) == row["mode"])
        prep = api.prepare_problem_set(_problems(m, n, k), cfg, mode)
        assert prep.total_tiles == row["tiles"], row
        assert round(api.tail_work_share(prep, cfg), 3) == row["tail_share"], row
        checked += 1
    assert checked == 28  # 24 grid rows and a repeat of one tail row in the problem-count sweep


def test_by_tiles_then_k_equals_by_tiles():
    """src/grouped_gemm.cu:1000-1005: both modes use the same comparator."""
    m, n, k = O.bench_shapes("tail", 700, 3)
    probs = _problems(m, n, k)
    for config in CONFIGS:
        cfg = KernelConfig.named(config)
        a = api.prepare_problem_set(probs, cfg, SortMode.kByTiles)
        b = api.prepare_problem_set(probs, cfg, SortMode.kByTilesThenK)
        assert a.sorted_to_original == b.sorted_to_original


def test_tile_count_and_non_empty():
    cfg = KernelConfig.named("128x64x32")
    for mm, nn in [(0, 5), (5, 0), (-3, 4), (1, 1), (128, 64), (129, 65), (4000, 14336)]:
        p = ProblemDesc(mm, nn, 7, 1, 1, None, 1, 7, max(1, nn), max(1, nn), max(1, nn))
        assert api.tile_count_for_problem(p, cfg) == O.tile_count(mm, nn, 128, 64)
    m, n, k = [0, 3, 64, 0, 5], [1, 0, 64, 0, 5], [3, 3, 3, 3, 0]
    assert api.count_non_empty_problems(_problems(m, n, k), cfg) == 2


def test_sort_mode_names():
    assert [api.sort_mode_name(m) for m in range(4)] == ["none", "sort_by_k", "sort_by_tiles",
                                                         "sort_by_tiles_then_k"]
    assert api.sort_mode_name(9) == "unknown"


def test_metric_helpers_match_oracle():
    m, n, k = O.bench_shapes("mixed", 256, 42)
    probs = _problems(m, n, k)
    assert api.total_flops(probs) == O.total_flops(m, n, k)


def _plan_sets():
    """Sets that reach each branch of the launch planning: oversized problems cut across chunks
    (four_big), tail halves (mixed512), zero-tile problems (zeros5000), one tiny problem, the small
    form (plumbing-sized sets), and no work table (a set above 2^22 work tiles)."""
    from grouped_gemm_gpu_kernel_amd.workloads import make_spec
    rng = np.random.default_rng(5)
    sets = {}
    for name in ("mixed512", "dense64", "longtail4096", "plumbing16"):
        spec = make_spec(name)
        sets[name] = (list(spec.m), list(spec.n), list(spec.k))
    cnt = 5000
    mm = rng.integers(0, 300, cnt)
    mm[rng.random(cnt) < 0.3] = 0
    sets["zeros5000"] = (list(mm), list(rng.integers(1, 300, cnt)), list(rng.integers(0, 50, cnt)))
    sets["one"] = ([1], [1], [1])
    sets["four_big"] = ([2048] * 4 + [100] * 5, [2048] * 4 + [300] * 5, [64] * 4 + [20] * 5)
    sets["searched"] = ([1 << 20], [1 << 20], [64])
    return sets


def _restated_plan(sorted_problems, cfg, compute_units, blocks, addr64_rows=None):
    from grouped_gemm_gpu_kernel_amd import _lib
    import schedule_plan as S
    base = {(64, 64): _lib.GGK_VARIANT_64x64x16, (128, 64): _lib.GGK_VARIANT_128x64x32,
            (64, 128): _lib.GGK_VARIANT_64x128x32}[(cfg.cta_m, cfg.cta_n)]
    path = _lib.GGK_PATH_MFMA if cfg.use_tensor_cores else _lib.GGK_PATH_FMA

    def shape(v):
        ws = _lib.GGKWorkShape()
        _lib.check(_lib.lib().ggk_work_shape_get(v, path, ctypes.byref(ws)), "work shape")
        return ws

    cta = dict(m=cfg.cta_m, n=cfg.cta_n, persistent=cfg.persistent_ctas, variant=base,
               small=_lib.lib().ggk_small_variant(base))
    problems = [(p.m, p.n, p.k, p.c is not None and p.beta != 0.0) for p in sorted_problems]
    return S.plan_launch(problems, cta, cfg.use_tensor_cores, compute_units, blocks,
                         lambda v: (shape(v).tiles_m, shape(v).tiles_n, shape(v).stage_k),
                         lambda v: _lib.lib().ggk_work_halves_supported(v, path) == 1,
                         lambda v: addr64_rows is not None and shape(v).rows >= addr64_rows)


def _check_table(plan, sorted_problems, cfg):
    """Properties that hold whatever the schedule: every work tile of every problem is listed once,
    whole or as its two halves (consecutive), in the order of the scheduling positions."""
    if not plan.work_table:
        assert plan.launch_total == plan.total_work and plan.launch_bounds == plan.chunk_bounds
        return
    shift = 28
    seen = {}
    entries = list(zip(plan.work_table[0::2], plan.work_table[1::2]))
    assert len(entries) == plan.launch_total == plan.launch_bounds[-1]
    i = 0
    while i < len(entries):
        prob, code = entries[i]
        local, half = code & ((1 << shift) - 1), code >> shift
        if half == 0:
            seen[(prob, local)] = seen.get((prob, local), 0) + 1
            i += 1
            continue
        assert half == 1 and entries[i + 1] == (prob, local | (2 << shift))
        seen[(prob, local)] = seen.get((prob, local), 0) + 1
        i += 2
    assert set(seen.values()) == {1} and len(seen) == plan.total_work
    positions = [plan.order.index(p) for p, _ in entries]
    assert positions == sorted(positions)
    assert plan.launch_bounds == sorted(plan.launch_bounds) and plan.launch_bounds[0] == 0


@pytest.mark.parametrize("config", CONFIGS + ["128x64x32/fma", "128x64x32/persistent100"])
def test_launch_plan_matches_restatement(config):
    """GroupedGemmExecutor::build's launch plan (variant, schedule, grid, work table with its tail
    halves), computed on the host from plain device values (256 CUs; one workgroup per CU of the
    256 x 256 work-tile kernels, two of the 128 x 128 ones), equals the restatement in
    tests/schedule_plan.py field for field; the table lists every work tile once."""
    name, _, extra = config.partition("/")
    cfg = KernelConfig.named(name, use_tensor_cores=extra != "fma",
                             persistent_ctas=100 if extra == "persistent100" else 0)
    blocks = [1, 1, 1, 2, 2, 2]
    halves_seen = False
    for set_name, (m, n, k) in _plan_sets().items():
        probs = _problems(m, n, k)
        for mode in (SortMode.kNone, SortMode.kByTiles):
            if set_name == "searched" and mode == SortMode.kByTiles:
                continue
            prep = api.prepare_problem_set(probs, cfg, mode)
            got = api.plan_launch(prep.sorted_problems, cfg, 256, blocks)
            want = _restated_plan(prep.sorted_problems, cfg, 256, blocks)
            where = f"{config} {set_name} mode={int(mode)}"
            assert (got.variant, got.addressing, got.total_work, got.grid, got.halves) == (
                want["variant"], want["addressing"], want["total_work"], want["grid"], want["halves"]), where
            assert got.order == want["order"] and got.work_offsets == want["offsets"], where
            assert got.chunk_bounds == want["bounds"], where
            assert got.work_table == want["table"], where
            assert got.launch_total == want["launch_total"] and got.launch_bounds == want["launch_bounds"], where
            _check_table(got, prep.sorted_problems, cfg)
            halves_seen |= got.halves
            if set_name == "searched":
                assert got.total_work > 1 << 22 and not got.work_table, where
    if cfg.use_tensor_cores and not cfg.persistent_ctas:
        assert halves_seen  # mixed512 lists halves


def test_launch_plan_64bit_sets_run_on_small_work_tiles():
    """A set whose row stride needs 64-bit offsets in 256-row work tiles (lda = 5e6: 256 lda > 2^30)
    but not in 128-row ones runs on the 128 x 128 form with 32-bit addressing."""
    from grouped_gemm_gpu_kernel_amd import _lib
    cfg = KernelConfig.named("128x64x32")
    probs = [ProblemDesc(4096, 4096, 64, 1, 1, None, 1, 5_000_000, 4096, 4096, 4096)]
    got = api.plan_launch(probs, cfg, 256, [1, 1, 1, 2, 2, 2])
    want = _restated_plan(probs, cfg, 256, [1, 1, 1, 2, 2, 2], addr64_rows=256)
    assert got.variant == _lib.GGK_VARIANT_128x64x32_SMALL == want["variant"]
    assert got.addressing == _lib.GGK_ADDR_32 == want["addressing"]
    assert got.order == want["order"] and got.work_table == want["table"] and got.grid == want["grid"]


def test_launch_plan_rejects_bad_input():
    from grouped_gemm_gpu_kernel_amd import _lib
    cfg = KernelConfig.named("128x64x32")
    probs = _problems([64], [64], [64])
    for bad_cfg, cus in ((KernelConfig(cta_m=32, cta_n=64, cta_k=16), 256), (cfg, 0)):
        with pytest.raises(_lib.HipError):
            api.plan_launch(probs, bad_cfg, cus, [1] * 6)
    with pytest.raises(_lib.HipError):
        api.plan_launch(_problems([-1], [64], [64]), cfg, 256, [1] * 6)
    arr = api._problem_array(probs)
    plan = _lib.GGLaunchPlan()
    blocks = (ctypes.c_int * 6)(*([1] * 6))
    table = (ctypes.c_int * 1)()
    assert _lib.lib().gg_plan_launch(arr, 1, ctypes.byref(cfg.to_c()), 256, blocks, ctypes.byref(plan), None, None,
                                     table, 1) == _lib.HIP_ERROR_INVALID_VALUE
    assert plan.table_ints == 2 and plan.grid == 256
    assert _lib.lib().gg_plan_launch(arr, 1, ctypes.byref(cfg.to_c()), 256, None, ctypes.byref(plan), None, None,
                                     None, 0) == _lib.HIP_ERROR_INVALID_VALUE


def test_extreme_extents_stay_defined():
    """Tile counts of extents near INT_MAX: ceil(m / cta_m) without overflow (the sanitized run of
    this file checks it), a product past INT_MAX clamped there, prepare's offsets saturating at it,
    and the launch plan refusing a set of more than INT_MAX macro-tiles.  The reference's int
    arithmetic overflows there (src/grouped_gemm.cu:54-65)."""
    from grouped_gemm_gpu_kernel_amd import _lib
    big = 2**31 - 1
    cfg = KernelConfig.named("128x64x32")
    tall = ProblemDesc(big, 1, 1, 1, 1, None, 1, 1, 1, 1, 1)
    assert api.tile_count_for_problem(tall, cfg) == -(-big // 128)
    huge = ProblemDesc(big, big, 1, 1, 1, None, 1, 1, big, big, big)
    assert api.tile_count_for_problem(huge, cfg) == big
    prep = api.prepare_problem_set([tall, huge, tall], cfg, SortMode.kNone)
    assert prep.tile_offsets == [0, -(-big // 128), big, big] and prep.total_tiles == big
    plan = api.plan_launch([tall], cfg, 256, [1, 1, 1, 2, 2, 2])
    assert plan.total_work == -(-(-(-big // 128)) // 2) and plan.work_table == []  # above 2^22: searched
    with pytest.raises(_lib.HipError):
        api.plan_launch([huge], cfg, 256, [1, 1, 1, 2, 2, 2])
    with pytest.raises(_lib.HipError):
        # 2^30 macro-tiles each: the set's 2^31 no longer fits an int
        api.plan_launch([ProblemDesc(2**30, 2**13, 1, 1, 1, None, 1, 1, 2**13, 2**13, 2**13)] * 2, cfg, 256,
                        [1, 1, 1, 2, 2, 2])


@pytest.mark.parametrize("name", ["mixed512", "dense64", "moe64", "longtail4096"])
def test_shard_plan_matches_restatement(name):
    """plan_shards splits a benchmark set across 1, 2, 3 and 8 ranks exactly as restated in
    schedule_plan.py; every problem's columns are covered once, in order, cut only at 256-column
    work-tile boundaries; dense64's 64 equal problems go 8 to each of 8 ranks; moe64's largest expert
    is cut across ranks at 8."""
    import schedule_plan as S
    from grouped_gemm_gpu_kernel_amd.workloads import make_spec
    spec = make_spec(name)
    cfg = KernelConfig.named(spec.config)
    probs = _problems(spec.m, spec.n, spec.k)
    for ranks in (1, 2, 3, 8):
        got = api.plan_shards(probs, cfg, ranks)
        want = S.plan_shards([(p.m, p.n, p.k, p.c is not None and p.beta != 0.0) for p in probs], ranks, 256, 256, 64)
        assert [(p.problem, p.rank, p.col0, p.cols) for p in got] == want, (name, ranks)
        assert len(got) <= len(probs) + ranks
        by_problem = {}
        for p in got:
            assert 0 <= p.rank < ranks and p.col0 % 256 == 0
            by_problem.setdefault(p.problem, []).append(p)
        assert sorted(by_problem) == list(range(len(probs)))
        for i, ps in by_problem.items():
            assert ps[0].col0 == 0 and sum(p.cols for p in ps) == max(probs[i].n, 0)
            assert all(a.col0 + a.cols == b.col0 for a, b in zip(ps, ps[1:]))
        if name == "dense64" and ranks == 8:
            assert sorted(p.rank for p in got) == sorted(list(range(8)) * 8)
        if name == "moe64" and ranks == 8:
            big = int(np.argmax(spec.m))
            assert len({p.rank for p in by_problem[big]}) > 1
    with pytest.raises(Exception):
        api.plan_shards(probs, cfg, 0)


def test_shard_problem_offsets():
    p = ProblemDesc(300, 1000, 70, 0x1000, 0x20000, 0x300000, 0x4000000, 70, 1000, 1000, 1000, 1.5, 0.5)
    q = api.shard_problem(p, api.ShardPiece(0, 1, 512, 488))
    assert (q.m, q.n, q.k, q.a, q.b, q.c, q.d) == (300, 488, 70, 0x1000, 0x20000 + 1024, 0x300000 + 2048, 0x4000000 + 2048)
    assert (q.lda, q.ldb, q.ldc, q.ldd, q.alpha, q.beta) == (70, 1000, 1000, 1000, 1.5, 0.5)
