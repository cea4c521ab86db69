"""Host-side parity of the library, on the CPU: prepare_problem_set (sort permutations, tile offsets,
total tiles), tile counts, sort-mode names and empty-problem counting must equal the oracle bit for
bit.  These entry points never touch the GPU."""
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
