"""GPU parity of the HIP grouped GEMM against the CPU oracle.

Bars:
  * tile -> (problem, tile_m, tile_n) map, sort permutations, tile offsets and grid size: bit-exact.
  * D: max |D - D_oracle| <= 1e-3 * sqrt(K) * max|A| * max|B| * |alpha| + 1e-6 * (|beta| * max|C| + 1)
    per problem (the target bound with |alpha| included, plus a few float32 ulps of the beta*C term).
  * D is NaN-poisoned before every run, so a tile that is skipped cannot pass on stale output.
  * Full-size sets of every benchmark workload: tests/test_full_size.py.
"""
import ctypes
import math
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from grouped_gemm_gpu_kernel_amd import _lib, api
from grouped_gemm_gpu_kernel_amd.api import GroupedGemmExecutor, KernelConfig, ProblemDesc, SortMode
from grouped_gemm_gpu_kernel_amd.workloads import DeviceWorkload, custom_spec, make_spec
from oracle import oracle as O
from schedule_plan import plan_schedule

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
CONFIGS = ["64x64x16", "128x64x32", "64x128x32"]
PATHS = [True, False]  # use_tensor_cores: MFMA path, FMA path
REFERENCE_SHAPES = [(64, 64, 64), (128, 64, 96), (45, 81, 37), (17, 23, 9), (192, 32, 64), (16, 256, 48),
                    (0, 64, 16), (64, 0, 16)]  # tests/test_correctness.cu:313-322


def say(msg):
    print(msg, flush=True)


def tolerance(k, max_a, max_b, max_c, alpha, beta):
    return 1e-3 * math.sqrt(max(k, 1)) * max_a * max_b * abs(alpha) + 1e-6 * (abs(beta) * max_c + 1.0)


class HostSet:
    """Problems whose operands live on the host (numpy) and on the device (torch)."""

    def __init__(self, torch, shapes, inputs, c_present=True):
        self.torch = torch
        self.shapes = shapes
        self.inputs = inputs  # per problem: alpha, beta, a(u16), b(u16), c(f32)
        self.dev = []
        self.problems = []
        for (m, n, k), (alpha, beta, a, b, c) in zip(shapes, inputs):
            da = torch.from_numpy(a.view(np.int16).copy()).cuda()
            db = torch.from_numpy(b.view(np.int16).copy()).cuda()
            dc = torch.from_numpy(c.copy()).cuda() if c_present else None
            dd = torch.full((max(1, m * max(1, n)) if m > 0 and n > 0 else 1,), float("nan"), device="cuda")
            self.dev.append((da, db, dc, dd))
            self.problems.append(ProblemDesc(m, n, k, da.data_ptr(), db.data_ptr(),
                                             dc.data_ptr() if dc is not None else None, dd.data_ptr(),
                                             max(1, k), max(1, n), max(1, n), max(1, n), alpha, beta))

    def poison(self):
        for (_, _, _, dd) in self.dev:
            dd.fill_(float("nan"))
        self.torch.cuda.synchronize()

    def outputs(self):
        self.torch.cuda.synchronize()
        return [dd.cpu().numpy() for (_, _, _, dd) in self.dev]

    def check(self, what):
        outs = self.outputs()
        for i, ((m, n, k), (alpha, beta, a, b, c), d) in enumerate(zip(self.shapes, self.inputs, outs)):
            if m <= 0 or n <= 0:
                assert np.isnan(d).all(), f"{what}: empty problem {i} was written"
                continue
            c_used = c if self.dev[i][2] is not None else None
            want = O.gemm(m, n, k, a, max(1, k), b, max(1, n), c_used, max(1, n), alpha, beta)
            got = d[:m * n]
            assert not np.isnan(got).any(), f"{what}: problem {i} ({m}x{n}x{k}) has unwritten elements"
            af = np.abs(O.f16_to_f32(a)).max() if k > 0 else 0.0
            bf = np.abs(O.f16_to_f32(b)).max() if k > 0 else 0.0
            cf = float(np.abs(c).max()) if c_used is not None else 0.0
            err = float(np.abs(got - want[:m * n]).max())
            assert err <= tolerance(k, af, bf, cf, alpha, beta), f"{what}: problem {i} ({m}x{n}x{k}) err {err}"
        return outs


@pytest.fixture(scope="module")
def torch(torch_cuda):
    return torch_cuda


@pytest.mark.parametrize("config", CONFIGS)
@pytest.mark.parametrize("mfma", PATHS)
def test_reference_test_shapes_all_modes_and_baseline(torch, config, mfma):
    """tests/test_correctness.cu:312-362 with the reference's own inputs (mt19937(20260328))."""
    say(f"reference shapes config={config} mfma={mfma}")
    m, n, k = zip(*REFERENCE_SHAPES)
    hs = HostSet(torch, REFERENCE_SHAPES, O.reference_test_inputs(m, n, k, 20260328))
    cfg = KernelConfig.named(config, use_tensor_cores=mfma)
    for mode in SortMode:
        hs.poison()
        assert api.run_grouped_gemm_once(hs.problems, mode, cfg) == 0
        hs.check(f"{config} mfma={mfma} mode={api.sort_mode_name(mode)}")
    hs.poison()
    assert api.run_baseline_per_problem(hs.problems, cfg) == 0
    hs.check(f"{config} mfma={mfma} baseline")
    # empty problem set (tests/test_correctness.cu:296-307)
    assert api.run_grouped_gemm_once([], SortMode.kByTiles, cfg) == 0
    assert api.run_baseline_per_problem([], cfg) == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("config", CONFIGS)
@pytest.mark.parametrize("mfma", PATHS)
def test_plumbing16_workload(torch, config, mfma):
    """16 problems, m, n, k uniform in [1, 256] (non-multiples of every tile), alpha 1, beta 0.5."""
    say(f"plumbing16 config={config} mfma={mfma}")
    spec = make_spec("plumbing16")
    dw = DeviceWorkload(spec)
    probs = dw.problems()
    cfg = KernelConfig.named(config, use_tensor_cores=mfma)
    ref = None
    for mode in list(SortMode) + ["baseline"]:
        dw.poison_d()
        if mode == "baseline":
            assert api.run_baseline_per_problem(probs, cfg) == 0
        else:
            assert api.run_grouped_gemm_once(probs, mode, cfg) == 0
        torch.cuda.synchronize()
        outs = [dw.host_d(i) for i in range(spec.count)]
        if ref is None:
            for i, p in enumerate(probs):
                a, b, c = dw.host_a(i), dw.host_b(i), dw.host_c(i)
                want = O.gemm(p.m, p.n, p.k, a, p.lda, b, p.ldb, c, p.ldc, p.alpha, p.beta)
                err = float(np.abs(outs[i][:p.m * p.n] - want[:p.m * p.n]).max())
                tol = tolerance(p.k, np.abs(O.f16_to_f32(a)).max(), np.abs(O.f16_to_f32(b)).max(),
                                np.abs(c).max(), p.alpha, p.beta)
                assert err <= tol, (i, p.m, p.n, p.k, err, tol)
            ref = outs
        else:
            for i in range(spec.count):
                assert np.array_equal(outs[i].view(np.uint32), ref[i].view(np.uint32)), (mode, i)


def _dummy_problems(torch, shapes):
    """Problems with real but tiny buffers: the mapping dump never dereferences them."""
    buf = torch.zeros(64, dtype=torch.float32, device="cuda")
    ptr = buf.data_ptr()
    return buf, [ProblemDesc(m, n, k, ptr, ptr, None, ptr, max(1, k), max(1, n), max(1, n), max(1, n))
                 for (m, n, k) in shapes]


def _mapping_sets():
    rng = np.random.default_rng(5)
    sets = {"reference": REFERENCE_SHAPES}
    m, n, k = O.bench_shapes("small", 256, 42)
    sets["small256"] = list(zip(m, n, k))
    spec = make_spec("longtail4096")
    sets["longtail4096"] = list(zip(spec.m, spec.n, spec.k))
    # short enough a launch for the work table to list the last tiles of each chunk as halves
    spec = make_spec("mixed512")
    sets["mixed512"] = list(zip(spec.m, spec.n, spec.k))
    cnt = 5000
    mm = rng.integers(0, 300, cnt)
    mm[rng.random(cnt) < 0.3] = 0  # many zero-tile problems
    sets["zeros5000"] = list(zip(mm, rng.integers(1, 300, cnt), rng.integers(0, 50, cnt)))
    sets["one"] = [(1, 1, 1)]
    # oversized problems cut across chunks: chunk bounds inside problems
    sets["four_big"] = [(2048, 2048, 64)] * 4 + [(100, 300, 20)] * 5
    return sets


def _variant_of(cfg, shape):
    """The kernel variant build() chose: the configuration's own or its small-set form, told apart
    by the work shape."""
    base = {(64, 64): _lib.GGK_VARIANT_64x64x16, (128, 64): _lib.GGK_VARIANT_128x64x32,
            (64, 128): _lib.GGK_VARIANT_64x128x32}[(cfg.cta_m, cfg.cta_n)]
    small = {_lib.GGK_VARIANT_128x64x32: _lib.GGK_VARIANT_128x64x32_SMALL,
             _lib.GGK_VARIANT_64x128x32: _lib.GGK_VARIANT_64x128x32_SMALL,
             _lib.GGK_VARIANT_64x64x16: _lib.GGK_VARIANT_64x64x16_SMALL}.get(base)
    for v in (base, small):
        if v is None:
            continue
        ws = _lib.GGKWorkShape()
        _lib.check(_lib.lib().ggk_work_shape_get(v, _lib.GGK_PATH_MFMA, ctypes.byref(ws)), "work shape")
        if (ws.tiles_m, ws.tiles_n) == (shape.tiles_m, shape.tiles_n):
            return v
    raise AssertionError(f"no variant of {cfg} has work shape {shape.tiles_m}x{shape.tiles_n}")


def _traced_map_by_search(torch, ex, prep, cfg):
    """The traced tile map of the executor's schedule launched through the kernel C-ABI with no work
    table, so that the kernel finds each claimed index's problem with its own search over the
    work-tile offsets (the device-side prepare's form)."""
    shape, order, offsets, bounds = ex.schedule()
    count = len(prep.sorted_problems)
    descs = (_lib.GGDeviceProblemDesc * max(1, count))()
    for i, p in enumerate(prep.sorted_problems):
        live = p.m > 0 and p.n > 0
        descs[i] = _lib.GGDeviceProblemDesc(p.m, p.n, p.k, p.a or None, p.b or None, p.c or None, p.d or None,
                                            p.lda, p.ldb, p.ldc, p.ldd, p.alpha, p.beta,
                                            -(-p.m // cfg.cta_m) if live else 0, -(-p.n // cfg.cta_n) if live else 0)
    d_desc = torch.empty(ctypes.sizeof(descs), dtype=torch.uint8, device="cuda")
    _lib.check(_lib.lib().ggk_copy_to_device(d_desc.data_ptr(), ctypes.addressof(descs), ctypes.sizeof(descs)),
               "descriptors")
    d_tiles = torch.tensor(prep.tile_offsets, dtype=torch.int32, device="cuda")
    d_work = torch.tensor(offsets, dtype=torch.int32, device="cuda")
    d_order = torch.tensor(order if order else [0], dtype=torch.int32, device="cuda")
    d_state = torch.zeros(_lib.GGK_SCHEDULER_STATE_INTS, dtype=torch.int32, device="cuda")
    total = prep.total_tiles
    tmap = torch.full((3 * max(1, total),), -1, dtype=torch.int32, device="cuda")
    c_bounds = (ctypes.c_int * len(bounds))(*bounds)
    st = _lib.lib().ggk_launch_grouped_traced(_variant_of(cfg, shape), _lib.GGK_PATH_MFMA, _lib.GGK_ADDR_32,
                                              d_desc.data_ptr(), d_tiles.data_ptr(), d_work.data_ptr(),
                                              d_order.data_ptr(), None, count, offsets[-1], d_state.data_ptr(),
                                              c_bounds, ex.grid_ctas(), tmap.data_ptr(), None, None, None)
    assert st == 0
    torch.cuda.synchronize()
    return tmap.cpu().numpy()[:3 * total].reshape(total, 3)


@pytest.mark.parametrize("config", CONFIGS)
def test_tile_mapping_bit_exact(torch, config):
    """The scheduler's tile -> (problem, tile_m, tile_n) function equals find_problem_by_tile plus the
    row-major local tile (src/grouped_gemm.cu:219-234, 659-668), for every claimed index: read from
    the executor's work table, and found by the kernel's own search when launched without one."""
    cfg = KernelConfig.named(config)
    for name, shapes in _mapping_sets().items():
        shapes = [(int(a), int(b), int(c)) for a, b, c in shapes]
        buf, probs = _dummy_problems(torch, shapes)
        for mode in (SortMode.kNone, SortMode.kByK, SortMode.kByTiles):
            say(f"mapping {config} {name} mode={int(mode)}")
            prep = api.prepare_problem_set(probs, cfg, mode)
            ex = GroupedGemmExecutor()
            assert ex.build(prep, cfg) == 0
            total = prep.total_tiles
            tmap = torch.full((3 * max(1, total),), -1, dtype=torch.int32, device="cuda")
            assert ex.run_traced(tmap.data_ptr()) == 0
            torch.cuda.synchronize()
            got = tmap.cpu().numpy()[:3 * total].reshape(total, 3)
            sm = np.array([p.m for p in prep.sorted_problems])
            sn = np.array([p.n for p in prep.sorted_problems])
            tiles_n = np.where((sm > 0) & (sn > 0), (sn + cfg.cta_n - 1) // cfg.cta_n, 1)
            want = O.map_tiles(tiles_n, prep.tile_offsets)
            assert np.array_equal(got, want), f"{config} {name} mode {mode} (work table)"
            assert np.array_equal(_traced_map_by_search(torch, ex, prep, cfg), want), \
                f"{config} {name} mode {mode} (search)"
            ex.close()
        del buf


def test_grid_size_and_occupancy(torch):
    for config in CONFIGS:
        for mfma in PATHS:
            cfg = KernelConfig.named(config, use_tensor_cores=mfma)
            st, info = api.query_occupancy(cfg)
            assert st == 0
            say(f"occupancy {config} mfma={mfma}: {info}")
            assert info.sm_count == 256 and info.using_tensor_cores == mfma
            # MFMA kernels compute 256 x 256 of D per workgroup with eight waves of 128 x 64; the FMA
            # kernels use 256 threads.
            want_threads = 512 if mfma else 256
            assert info.threads_per_block == want_threads
            assert info.warps_per_block == want_threads // 64 and info.max_warps_per_sm == 32
            assert info.registers_per_thread > 0 and info.active_blocks_per_sm >= 1
            # The runtime's occupancy calculator and the register/LDS accounting must agree on the
            # binding limit.
            assert info.active_blocks_per_sm == min(info.register_limited_blocks_per_sm,
                                                    info.lds_limited_blocks_per_sm,
                                                    info.wave_limited_blocks_per_sm)
            assert info.theoretical_occupancy == pytest.approx(
                info.active_blocks_per_sm * info.warps_per_block / 32)
            for total in (1, 100, 255, 256, 257, 5000, 100000):
                for persistent in (0, 1, 999):
                    c2 = KernelConfig.named(config, use_tensor_cores=mfma, persistent_ctas=persistent)
                    assert api.grid_ctas_for(c2, total) == O.grid_ctas(total, persistent, info.sm_count,
                                                                       info.active_blocks_per_sm)


@pytest.mark.parametrize("config", CONFIGS)
@pytest.mark.parametrize("count", [30, 700])
def test_host_schedule_is_the_longest_first_plan(torch, config, count):
    """build()'s work-tile schedule (scheduling order, work-tile offsets in that order, chunk
    bounds) equals the longest-first plan restated in schedule_plan.py, with zero-tile problems,
    C on some problems only, and both the small-set and the large work tiles."""
    rng = np.random.default_rng(count)
    buf = torch.zeros(64, dtype=torch.float32, device="cuda")
    ptr = buf.data_ptr()
    problems = []
    for i in range(count):
        m, n, k = (int(x) for x in np.exp(rng.uniform(0, np.log(1500), 3)).astype(int))
        if rng.random() < 0.1:
            m = 0
        with_c = bool(rng.random() < 0.5)
        problems.append(ProblemDesc(m, n, k, ptr, ptr, ptr if with_c else None, ptr, max(1, k), max(1, n),
                                    max(1, n), max(1, n), 1.0, 0.5 if with_c else 0.0))
    cfg = KernelConfig.named(config)
    for mode in SortMode:
        prep = api.prepare_problem_set(problems, cfg, mode)
        ex = GroupedGemmExecutor()
        assert ex.build(prep, cfg) == 0
        shape, order, offsets, bounds = ex.schedule()
        work = []
        for p in prep.sorted_problems:
            tm = -(-p.m // cfg.cta_m) if p.m > 0 and p.n > 0 else 0
            tn = -(-p.n // cfg.cta_n) if p.m > 0 and p.n > 0 else 0
            work.append((-(-tm // shape.tiles_m)) * (-(-tn // shape.tiles_n)))
        want = plan_schedule([(p.m, p.n, p.k) for p in prep.sorted_problems], work, cfg.cta_m * shape.tiles_m,
                             cfg.cta_n * shape.tiles_n, shape.stage_k,
                             [p.c is not None and p.beta != 0.0 for p in prep.sorted_problems])
        say(f"{config} {count} {mode.name}: work shape {shape.tiles_m}x{shape.tiles_n}, {offsets[-1]} work tiles")
        assert (order, offsets, bounds) == want, (config, count, mode)
        # build() is plan_launch with this device's CU count and occupancies.
        plan = api.plan_launch(prep.sorted_problems, cfg, *_device_plan_values(cfg))
        assert (plan.order, plan.work_offsets, plan.chunk_bounds) == (order, offsets, bounds)
        assert (plan.grid, plan.launch_total) == (ex.grid_ctas(), ex.launched_work_tiles())
        assert (plan.work[0], plan.work[1]) == (shape.tiles_m, shape.tiles_n)
        ex.close()


def _device_plan_values(cfg):
    """(compute units, resident workgroups per CU of each variant) of the current device, as
    build() reads them."""
    info = _lib.GGKDeviceInfo()
    _lib.check(_lib.lib().ggk_device_info_get(ctypes.byref(info)), "device info")
    path = _lib.GGK_PATH_MFMA if cfg.use_tensor_cores else _lib.GGK_PATH_FMA
    blocks = []
    for v in range(_lib.GGK_VARIANT_COUNT):
        b = ctypes.c_int(0)
        _lib.check(_lib.lib().ggk_occupancy(v, path, ctypes.byref(b)), "occupancy")
        blocks.append(b.value)
    return info.compute_units, blocks


@pytest.mark.parametrize("name", ["one", "four_equal", "two_big", "one_big_among_many"])
def test_host_schedule_cuts_oversized_problems(torch, name):
    """Problems above one chunk's share of the estimated time are cut across consecutive chunks
    when placing them whole would leave more than a quarter of the work to stealing; the plan
    equals schedule_plan.py's, and the cut ones are exactly the sets where that rule says so (one
    problem alone, four equal ones; a single 1.7-share problem among many small ones stays whole)."""
    rng = np.random.default_rng(11)
    shapes = {
        "one": [(4096, 4096, 1024)],
        "four_equal": [(2048, 2048, 2048)] * 4,
        "two_big": [(3000, 5000, 700), (2500, 4000, 900)] + [(300, 200, 100)] * 20,
        "one_big_among_many": [(7000, 4096, 1024)] + [(int(rng.integers(200, 900)), 4096, 1024) for _ in range(40)],
    }[name]
    buf = torch.zeros(64, dtype=torch.float32, device="cuda")
    ptr = buf.data_ptr()
    problems = [ProblemDesc(m, n, k, ptr, ptr, None, ptr, k, n, n, n) for (m, n, k) in shapes]
    cfg = KernelConfig.named("128x64x32")
    prep = api.prepare_problem_set(problems, cfg, SortMode.kByK)
    ex = GroupedGemmExecutor()
    assert ex.build(prep, cfg) == 0
    shape, order, offsets, bounds = ex.schedule()
    work = [(-(-(-(-p.m // cfg.cta_m)) // shape.tiles_m)) * (-(-(-(-p.n // cfg.cta_n)) // shape.tiles_n))
            for p in prep.sorted_problems]
    want = plan_schedule([(p.m, p.n, p.k) for p in prep.sorted_problems], work, cfg.cta_m * shape.tiles_m,
                         cfg.cta_n * shape.tiles_n, shape.stage_k, False)
    assert (order, offsets, bounds) == want, name
    inside = [b for b in bounds[1:-1] if b not in offsets]  # chunk bounds that fall inside a problem
    say(f"{name}: bounds {bounds}, {len(inside)} inside a problem")
    assert bool(inside) == (name in ("one", "four_equal", "two_big")), (name, bounds, offsets)
    ex.close()


@pytest.mark.parametrize("config", CONFIGS)
@pytest.mark.parametrize("mfma", PATHS)
def test_unread_c_leaves_no_trace(torch, config, mfma):
    """C is read only when it is given and beta != 0 (src/grouped_gemm.cu:475-479, 616-621): a null C
    with an infinite or NaN beta, and a NaN-filled C with beta = 0, give D = alpha * A B (the oracle
    with beta = 0) and no NaN, in every tile class (full, partial rows and columns, a small set)."""
    rng = np.random.default_rng(3)
    cfg = KernelConfig.named(config, use_tensor_cores=mfma)
    shapes = [(300, 270, 100), (64, 64, 16), (129, 40, 33)]
    for (m, n, k) in shapes:
        a = O.f32_to_f16(rng.uniform(-1, 1, m * k).astype(np.float32))
        b = O.f32_to_f16(rng.uniform(-1, 1, k * n).astype(np.float32))
        want = O.gemm(m, n, k, a, k, b, n, None, n, 1.5, 0.0)
        da = torch.from_numpy(a.view(np.int16).copy()).cuda()
        db = torch.from_numpy(b.view(np.int16).copy()).cuda()
        dc = torch.full((m * n,), float("nan"), device="cuda")
        for c_ptr, beta in ((None, float("inf")), (None, float("nan")), (dc.data_ptr(), 0.0)):
            say(f"unread C {config} mfma={mfma} {m}x{n}x{k} c={'set' if c_ptr else 'null'} beta={beta}")
            dd = torch.full((m * n,), float("nan"), device="cuda")
            prob = ProblemDesc(m, n, k, da.data_ptr(), db.data_ptr(), c_ptr, dd.data_ptr(), k, n, n, n, 1.5, beta)
            assert api.run_grouped_gemm_once([prob], SortMode.kByK, cfg) == 0
            torch.cuda.synchronize()
            got = dd.cpu().numpy()
            assert not np.isnan(got).any(), (m, n, k, beta)
            tol = tolerance(k, np.abs(O.f16_to_f32(a)).max(), np.abs(O.f16_to_f32(b)).max(), 0.0, 1.5, 0.0)
            assert float(np.abs(got - want[:m * n]).max()) <= tol, (m, n, k, beta)


def test_error_behaviour(torch):
    """Status codes of src/grouped_gemm.cu:121-123, 1135-1137, 1147-1152, 1169-1174, 1305-1307."""
    good = KernelConfig.named("128x64x32")
    bad = [KernelConfig(cta_m=32, cta_n=32, cta_k=16), KernelConfig.named("128x64x32", threads=128),
           KernelConfig(cta_m=128, cta_n=64, cta_k=16)]
    buf = torch.zeros(16, device="cuda")
    p = ProblemDesc(4, 4, 4, buf.data_ptr(), buf.data_ptr(), None, buf.data_ptr(), 4, 4, 4, 4)
    for cfg in bad:
        assert api.query_occupancy(cfg)[0] == _lib.HIP_ERROR_INVALID_VALUE
        assert api.run_grouped_gemm_once([p], SortMode.kNone, cfg) == _lib.HIP_ERROR_INVALID_VALUE
        assert api.run_baseline_per_problem([p], cfg) == _lib.HIP_ERROR_INVALID_VALUE
    for field in ("a", "b", "d"):
        q = ProblemDesc(**{**p.__dict__, field: 0})
        assert api.run_grouped_gemm_once([q], SortMode.kNone, good) == _lib.HIP_ERROR_INVALID_DEVICE_POINTER
        assert api.run_baseline_per_problem([q], good) == _lib.HIP_ERROR_INVALID_DEVICE_POINTER
    # the baseline rejects null pointers even on an empty problem
    e = ProblemDesc(0, 4, 4, 0, 0, None, 0, 4, 4, 4, 4)
    assert api.run_baseline_per_problem([e], good) == _lib.HIP_ERROR_INVALID_DEVICE_POINTER
    neg = ProblemDesc(**{**p.__dict__, "k": -1})
    assert api.run_grouped_gemm_once([neg], SortMode.kNone, good) == _lib.HIP_ERROR_INVALID_VALUE
    ex = GroupedGemmExecutor()
    prep = api.prepare_problem_set([p], good, SortMode.kNone)
    broken = api.PreparedProblemSet(prep.sorted_problems, prep.sorted_to_original, prep.tile_offsets[:-1],
                                    prep.total_tiles)
    assert ex.build(broken, good) == _lib.HIP_ERROR_INVALID_VALUE
    wrong_total = api.PreparedProblemSet(prep.sorted_problems, prep.sorted_to_original, prep.tile_offsets, 7)
    assert ex.build(wrong_total, good) == _lib.HIP_ERROR_INVALID_VALUE
    inconsistent = api.PreparedProblemSet(prep.sorted_problems, prep.sorted_to_original, [0, 2], 2)
    assert ex.build(inconsistent, good) == _lib.HIP_ERROR_INVALID_VALUE
    ex.close()
    assert _lib.lib().gg_executor_run(None, None) == _lib.HIP_ERROR_INVALID_DEVICE_POINTER
    torch.cuda.synchronize()


@pytest.mark.parametrize("mfma", PATHS)
def test_degenerate_problems(torch, mfma):
    """K = 0 gives D = beta*C; beta = 0 never reads C (NaN C stays out of D); c = nullptr is legal;
    1x1 and single-row/column problems; odd leading dimensions."""
    say(f"degenerate mfma={mfma}")
    shapes = [(5, 7, 0), (1, 1, 1), (1, 300, 77), (300, 1, 77), (33, 65, 1), (129, 63, 200), (64, 64, 64)]
    rng = np.random.default_rng(9)
    inputs = []
    for idx, (m, n, k) in enumerate(shapes):
        a = O.f32_to_f16(rng.uniform(-1, 1, max(1, m * max(1, k))).astype(np.float32))
        b = O.f32_to_f16(rng.uniform(-1, 1, max(1, k * n)).astype(np.float32))
        c = rng.uniform(-1, 1, m * n).astype(np.float32)
        inputs.append((1.5, 0.75 if idx % 2 == 0 else 0.0, a, b, c))
    hs = HostSet(torch, shapes, inputs)
    # beta == 0: poison C with NaN; the kernel must not read it.
    for i, (_, beta, _, _, _) in enumerate(inputs):
        if beta == 0.0:
            hs.dev[i][2].fill_(float("nan"))
            hs.inputs[i] = (inputs[i][0], 0.0, inputs[i][2], inputs[i][3], np.zeros_like(inputs[i][4]))
    for config in CONFIGS:
        cfg = KernelConfig.named(config, use_tensor_cores=mfma)
        hs.poison()
        assert api.run_grouped_gemm_once(hs.problems, SortMode.kByTiles, cfg) == 0
        hs.check(f"degenerate {config}")
        hs.poison()
        assert api.run_baseline_per_problem(hs.problems, cfg) == 0
        hs.check(f"degenerate baseline {config}")
    # c = nullptr
    probs = [ProblemDesc(**{**p.__dict__, "c": None}) for p in hs.problems]
    hs2_inputs = [(al, be, a, b, np.zeros_like(c)) for (al, be, a, b, c) in hs.inputs]
    hs.poison()
    assert api.run_grouped_gemm_once(probs, SortMode.kNone, KernelConfig.named("128x64x32", use_tensor_cores=mfma)) == 0
    hs.inputs = hs2_inputs
    hs.check("c = nullptr")


def test_padded_leading_dimensions(torch):
    """lda > k, ldb/ldc/ldd > n, and matrices starting at 2-byte offsets."""
    rng = np.random.default_rng(13)
    for mfma in PATHS:
        for (m, n, k, pa, pb, pc, pd, off) in [(70, 90, 50, 3, 5, 7, 1, 1), (128, 64, 64, 8, 8, 0, 0, 0),
                                               (33, 130, 129, 1, 2, 3, 4, 1)]:
            lda, ldb, ldc, ldd = k + pa, n + pb, n + pc, n + pd
            a = O.f32_to_f16(rng.uniform(-1, 1, m * lda + off).astype(np.float32))
            b = O.f32_to_f16(rng.uniform(-1, 1, k * ldb + off).astype(np.float32))
            c = rng.uniform(-1, 1, m * ldc).astype(np.float32)
            da = torch.from_numpy(a.view(np.int16)).cuda()
            db = torch.from_numpy(b.view(np.int16)).cuda()
            dc = torch.from_numpy(c).cuda()
            dd = torch.full((m * ldd,), float("nan"), device="cuda")
            p = ProblemDesc(m, n, k, da.data_ptr() + 2 * off, db.data_ptr() + 2 * off, dc.data_ptr(), dd.data_ptr(),
                            lda, ldb, ldc, ldd, 0.5, -1.25)
            for config in CONFIGS:
                dd.fill_(float("nan"))
                assert api.run_grouped_gemm_once([p], SortMode.kNone, KernelConfig.named(config, use_tensor_cores=mfma)) == 0
                torch.cuda.synchronize()
                got = dd.cpu().numpy().reshape(m, ldd)
                want = O.gemm(m, n, k, a[off:], lda, b[off:], ldb, c, ldc, 0.5, -1.25, ldd=ldd).reshape(m, ldd)
                tol = tolerance(k, 1.0, 1.0, 1.0, 0.5, -1.25)
                assert np.abs(got[:, :n] - want[:, :n]).max() <= tol
                assert np.isnan(got[:, n:]).all(), "padding columns of D were written"


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_random_sets_against_oracle(torch, seed):
    """Seeded random problem sets mixing everything at once: sizes 0..320 (K 0..400, odd and even),
    padded leading dimensions, matrices at 2-byte offsets, alpha and beta of either sign or zero, C
    null on some problems.  For every configuration and both paths: the four sort modes and the
    per-problem baseline give bit-identical D, D matches the oracle within the bound, and the
    padding columns of D stay NaN."""
    rng = np.random.default_rng(100 + seed)
    count = 24
    probs_host, keep = [], []
    for i in range(count):
        m, n = (int(x) for x in rng.integers(0, 321, 2))
        k = int(rng.integers(0, 401))
        if rng.random() < 0.1:
            m = 0
        pa, pb, pc, pd = (int(x) for x in rng.integers(0, 9, 4))
        off = int(rng.integers(0, 2))
        lda, ldb, ldc, ldd = max(1, k + pa), max(1, n + pb), max(1, n + pc), max(1, n + pd)
        alpha = float(rng.choice([1.0, -0.75, 1.5]))
        beta = float(rng.choice([0.0, 0.5, -1.25]))
        with_c = bool(rng.random() < 0.8)
        a = O.f32_to_f16(rng.uniform(-1, 1, max(1, m * lda) + off).astype(np.float32))
        b = O.f32_to_f16(rng.uniform(-1, 1, max(1, k * ldb) + off).astype(np.float32))
        c = rng.uniform(-1, 1, max(1, m * ldc)).astype(np.float32)
        da = torch.from_numpy(a.view(np.int16).copy()).cuda()
        db = torch.from_numpy(b.view(np.int16).copy()).cuda()
        dc = torch.from_numpy(c.copy()).cuda()
        dd = torch.full((max(1, m * ldd),), float("nan"), device="cuda")
        keep.append((da, db, dc, dd))
        probs_host.append((m, n, k, a[off:], b[off:], c if with_c else None, lda, ldb, ldc, ldd, alpha, beta))
        probs_host[-1] = probs_host[-1] + (ProblemDesc(m, n, k, da.data_ptr() + 2 * off, db.data_ptr() + 2 * off,
                                                       dc.data_ptr() if with_c else None, dd.data_ptr(),
                                                       lda, ldb, ldc, ldd, alpha, beta),)
    problems = [h[-1] for h in probs_host]
    wants = []
    for (m, n, k, a, b, c, lda, ldb, ldc, ldd, alpha, beta, _) in probs_host:
        if m > 0 and n > 0:
            # The reference reads C only when given with beta != 0.
            c_used = c if (c is not None and beta != 0.0) else None
            wants.append(O.gemm(m, n, k, a, lda, b, ldb, c_used, ldc, alpha, beta if c_used is not None else 0.0,
                                ldd=ldd).reshape(m, ldd))
        else:
            wants.append(None)

    def outputs():
        torch.cuda.synchronize()
        return [kp[3].cpu().numpy() for kp in keep]

    for config in CONFIGS:
        for mfma in PATHS:
            cfg = KernelConfig.named(config, use_tensor_cores=mfma)
            ref = None
            for mode in list(SortMode) + ["baseline"]:
                say(f"random set seed={seed} {config} mfma={mfma} mode={mode}")
                for kp in keep:
                    kp[3].fill_(float("nan"))
                if mode == "baseline":
                    assert api.run_baseline_per_problem(problems, cfg) == 0
                else:
                    assert api.run_grouped_gemm_once(problems, mode, cfg) == 0
                outs = outputs()
                if ref is None:
                    for i, (h, got, want) in enumerate(zip(probs_host, outs, wants)):
                        m, n, k, a, b, c, lda, ldb, ldc, ldd, alpha, beta, _ = h
                        if want is None:
                            assert np.isnan(got).all(), (seed, config, mfma, i, "empty problem written")
                            continue
                        g = got[:m * ldd].reshape(m, ldd)
                        amax = np.abs(O.f16_to_f32(a[:max(1, m * lda)])).max() if k > 0 else 0.0
                        bmax = np.abs(O.f16_to_f32(b[:max(1, k * ldb)])).max() if k > 0 else 0.0
                        cmax = float(np.abs(c).max()) if c is not None and beta != 0.0 else 0.0
                        tol = tolerance(k, amax, bmax, cmax, alpha, beta)
                        assert not np.isnan(g[:, :n]).any(), (seed, config, mfma, i, "unwritten elements")
                        assert float(np.abs(g[:, :n] - want[:, :n]).max()) <= tol, (seed, config, mfma, i, m, n, k)
                        assert np.isnan(g[:, n:]).all(), (seed, config, mfma, i, "padding columns written")
                    ref = outs
                else:
                    for i in range(count):
                        assert np.array_equal(np.nan_to_num(outs[i], nan=7.0).view(np.uint32),
                                              np.nan_to_num(ref[i], nan=7.0).view(np.uint32)), (seed, config, mfma, mode, i)


def test_matrix_end_values(torch):
    """The last value of A and of B (the dword that holds it can reach 2 bytes past the matrix and then
    reads as zero; the loader puts the value back exactly where that happens: odd K for A, odd N for B)
    -- every parity of K and N, matrices starting at even and odd element offsets, tight leading
    dimensions, the last row and column in the first or a later work tile.  Both last values are 8
    and all others at most 1/8 in magnitude, so a lost or overwritten last value is far outside the
    bound."""
    rng = np.random.default_rng(21)
    for mfma in PATHS:
        for config in CONFIGS:
            cfg = KernelConfig.named(config, use_tensor_cores=mfma)
            for (m, n, k) in [(37, 45, 19), (37, 46, 20), (37, 45, 20), (37, 46, 19), (300, 301, 33), (260, 258, 64)]:
                for off in (0, 1):
                    say(f"matrix ends {config} mfma={mfma} {(m, n, k)} off={off}")
                    a = O.f32_to_f16(rng.uniform(-0.125, 0.125, m * k + off).astype(np.float32))
                    b = O.f32_to_f16(rng.uniform(-0.125, 0.125, k * n + off).astype(np.float32))
                    a[off + m * k - 1] = O.f32_to_f16(np.array([8.0], np.float32))[0]
                    b[off + k * n - 1] = O.f32_to_f16(np.array([8.0], np.float32))[0]
                    c = rng.uniform(-1, 1, m * n).astype(np.float32)
                    da = torch.from_numpy(a.view(np.int16)).cuda()
                    db = torch.from_numpy(b.view(np.int16)).cuda()
                    dc = torch.from_numpy(c).cuda()
                    dd = torch.full((m * n,), float("nan"), device="cuda")
                    p = ProblemDesc(m, n, k, da.data_ptr() + 2 * off, db.data_ptr() + 2 * off, dc.data_ptr(),
                                    dd.data_ptr(), k, n, n, n, 1.0, 0.5)
                    assert api.run_grouped_gemm_once([p], SortMode.kNone, cfg) == 0
                    torch.cuda.synchronize()
                    got = dd.cpu().numpy()
                    want = O.gemm(m, n, k, a[off:], k, b[off:], n, c, n, 1.0, 0.5)
                    tol = tolerance(k, 8.0, 8.0, 1.0, 1.0, 0.5)
                    err = np.abs(got - want).max()
                    assert err <= tol, f"{config} mfma={mfma} {(m, n, k)} off={off}: err {err}"
                    # the corner element holds the product of the two last values (64)
                    assert abs(got[-1] - want[-1]) <= tol


def test_wide_leading_dimensions(torch):
    """Leading dimensions too large for 32-bit tile offsets (lda * 256 >= 2^30, ldb * 64 >= 2^30) select
    the 64-bit addressing kernels, in a grouped launch mixed with ordinary problems and per problem."""
    wide_lda, wide_ldb = (1 << 24) + 3, (1 << 25) + 1  # wide for every work-tile shape
    shapes = [(3, 70, 21, wide_lda, 70), (40, 9, 5, 21, wide_ldb), (65, 130, 77, 77, 130)]
    store, probs, dense = [], [], []
    for i, (m, n, k, lda, ldb) in enumerate(shapes):
        a = torch.empty((m - 1) * lda + k + 1, dtype=torch.float16, device="cuda")
        b = torch.empty((k - 1) * ldb + n + 1, dtype=torch.float16, device="cuda")
        a.uniform_(-1, 1)
        b.uniform_(-1, 1)
        c = torch.empty(m * n, dtype=torch.float32, device="cuda").uniform_(-1, 1)
        d = torch.full((m * n,), float("nan"), device="cuda")
        # Matrices start 2 bytes into their buffers: odd element offsets exercise the realignment.
        ah = torch.as_strided(a, (m, k), (lda, 1), 1).cpu().numpy().view(np.uint16)
        bh = torch.as_strided(b, (k, n), (ldb, 1), 1).cpu().numpy().view(np.uint16)
        store += [a, b, c, d]
        dense.append((ah.reshape(-1).copy(), bh.reshape(-1).copy(), c.cpu().numpy()))
        probs.append(ProblemDesc(m, n, k, a.data_ptr() + 2, b.data_ptr() + 2, c.data_ptr(), d.data_ptr(),
                                 lda, ldb, n, n, 1.5, 0.25))
    for mfma in PATHS:
        for config in CONFIGS:
            cfg = KernelConfig.named(config, use_tensor_cores=mfma)
            for run in ("grouped", "baseline"):
                for dd in store[3::4]:
                    dd.fill_(float("nan"))
                if run == "grouped":
                    assert api.run_grouped_gemm_once(probs, SortMode.kByTiles, cfg) == 0
                else:
                    assert api.run_baseline_per_problem(probs, cfg) == 0
                torch.cuda.synchronize()
                for (m, n, k, _, _), (ah, bh, ch), dd in zip(shapes, dense, store[3::4]):
                    got = dd.cpu().numpy()
                    want = O.gemm(m, n, k, ah, k, bh, n, ch, n, 1.5, 0.25)
                    assert np.abs(got - want).max() <= tolerance(k, 1.0, 1.0, 1.0, 1.5, 0.25), \
                        f"{config} mfma={mfma} {run} {(m, n, k)}"


@pytest.mark.parametrize("config", CONFIGS)
def test_wide_set_runs_on_128x128_work_tiles(torch, config):
    """A set large enough for 256 x 256 work tiles, plus one problem whose leading dimension needs
    64-bit addressing, runs on 128 x 128 work tiles of the same macro-tile (the 64-bit 256 x 256 form
    would spill registers): the other problems' D is bit-identical to the same set without the wide
    problem (256 x 256 tiles, 32-bit form), and the wide problem's D is within the oracle bound; the
    per-problem baseline routes the wide problem the same way."""
    cfg = KernelConfig.named(config)
    count, m, n, k = 1100, 128, 128, 16
    g = torch.Generator(device="cpu").manual_seed(21)
    a = (torch.rand(m, k, generator=g) * 2 - 1).half().cuda()
    b = (torch.rand(k, n, generator=g) * 2 - 1).half().cuda()
    c = (torch.rand(m, n, generator=g) * 2 - 1).cuda()
    d = torch.full((count, m, n), float("nan"), device="cuda")
    fill = [ProblemDesc(m, n, k, a.data_ptr(), b.data_ptr(), c.data_ptr(), d[i].data_ptr(), k, n, n, n, 1.25, 0.5)
            for i in range(count)]
    wm, wn, wk, wide_lda = 70, 90, 33, (1 << 24) + 3
    wa = torch.empty((wm - 1) * wide_lda + wk, dtype=torch.float16, device="cuda").uniform_(-1, 1)
    wb = (torch.rand(wk, wn, generator=g) * 2 - 1).half().cuda()
    wd = torch.full((wm, wn), float("nan"), device="cuda")
    wide = ProblemDesc(wm, wn, wk, wa.data_ptr(), wb.data_ptr(), None, wd.data_ptr(), wide_lda, wn, wn, wn, 1.5, 0.0)
    ah = torch.as_strided(wa, (wm, wk), (wide_lda, 1)).cpu().numpy().view(np.uint16).reshape(-1).copy()
    want_wide = O.gemm(wm, wn, wk, ah, wk, wb.cpu().numpy().view(np.uint16).reshape(-1), wn, None, wn, 1.5, 0.0)

    ex = GroupedGemmExecutor()
    assert ex.build(api.prepare_problem_set(fill, cfg, SortMode.kByTiles), cfg) == 0
    assert (ex.schedule()[0].tiles_m, ex.schedule()[0].tiles_n) == (256 // cfg.cta_m, 256 // cfg.cta_n)
    assert ex.run() == 0
    torch.cuda.synchronize()
    d_large = d.clone()
    ex.close()
    d.fill_(float("nan"))
    ex = GroupedGemmExecutor()
    assert ex.build(api.prepare_problem_set(fill + [wide], cfg, SortMode.kByTiles), cfg) == 0
    shape = ex.schedule()[0]
    say(f"wide set: work shape {shape.tiles_m}x{shape.tiles_n}")
    assert (shape.tiles_m, shape.tiles_n) == (128 // cfg.cta_m, 128 // cfg.cta_n)  # 128 x 128 work tiles
    assert ex.run() == 0
    torch.cuda.synchronize()
    assert torch.equal(d, d_large)
    got = wd.cpu().numpy().reshape(-1)
    assert np.abs(got - want_wide).max() <= tolerance(wk, 1.0, 1.0, 0.0, 1.5, 0.0)
    ex.close()
    wd.fill_(float("nan"))
    assert api.run_baseline_per_problem([wide], cfg) == 0
    torch.cuda.synchronize()
    assert np.abs(wd.cpu().numpy().reshape(-1) - want_wide).max() <= tolerance(wk, 1.0, 1.0, 0.0, 1.5, 0.0)


def test_persistent_grid_sizes_and_repeated_runs(torch):
    """Any persistent grid gives bit-identical D; runs of one executor back to back (the scheduler state
    returns to zero by itself) stay identical."""
    spec = make_spec("plumbing16")
    dw = DeviceWorkload(spec)
    probs = dw.problems()
    ref = None
    for persistent in (0, 1, 3, 17, 256, 1000):
        cfg = KernelConfig.named("128x64x32", persistent_ctas=persistent)
        prep = api.prepare_problem_set(probs, cfg, SortMode.kByTiles)
        ex = GroupedGemmExecutor()
        assert ex.build(prep, cfg) == 0
        if persistent:
            assert ex.grid_ctas() == persistent
        for rep in range(3):
            dw.poison_d()
            assert ex.run() == 0
            torch.cuda.synchronize()
            d = dw.d.cpu().numpy()
            if ref is None:
                ref = d
            valid = ~np.isnan(ref)
            assert np.array_equal(np.isnan(d), ~valid)
            assert np.array_equal(d[valid].view(np.uint32), ref[valid].view(np.uint32)), (persistent, rep)
        ex.close()


def test_rebuild_after_captured_run_waits_for_replays(torch):
    """run() captured into a graph, replayed, and the executor rebuilt at once (no host wait): the
    rebuild rewrites the executor's device buffer, which the replay is still reading, only after the
    device is idle, so the replay's D and the rebuilt executor's D both equal eager runs."""
    cfg = KernelConfig.named("128x64x32")
    first = DeviceWorkload(make_spec("mixed512"))
    second = DeviceWorkload(make_spec("plumbing16"))
    prep1 = api.prepare_problem_set(first.problems(), cfg, SortMode.kByTiles)
    prep2 = api.prepare_problem_set(second.problems(), cfg, SortMode.kByK)
    ex = GroupedGemmExecutor()
    assert ex.build(prep1, cfg) == 0
    first.poison_d()
    assert ex.run() == 0
    torch.cuda.synchronize()
    want1 = first.d.cpu().numpy().view(np.uint32).copy()
    ex2 = GroupedGemmExecutor()
    assert ex2.build(prep2, cfg) == 0
    second.poison_d()
    assert ex2.run() == 0
    torch.cuda.synchronize()
    want2 = second.d.cpu().numpy().view(np.uint32).copy()
    ex2.close()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        assert ex.run(torch.cuda.current_stream()) == 0
    side = torch.cuda.Stream()
    for rep in range(3):
        say(f"captured run, replay {rep}, then rebuild without a host wait")
        first.poison_d()
        assert ex.build(prep1, cfg) == 0  # back to the captured set (same buffer, same contents)
        torch.cuda.synchronize()
        with torch.cuda.stream(side):  # a non-blocking stream: the host copies do not order after it
            graph.replay()
        # the replay is in flight: this rebuild must wait for it before rewriting the buffer
        assert ex.build(prep2, cfg) == 0
        second.poison_d()
        assert ex.run() == 0
        torch.cuda.synchronize()
        assert np.array_equal(first.d.cpu().numpy().view(np.uint32), want1), rep
        assert np.array_equal(second.d.cpu().numpy().view(np.uint32), want2), rep
    ex.close()
    del graph


@pytest.mark.parametrize("config", CONFIGS)
def test_small_set_work_tiles_bit_identical(torch, config):
    """A launch with few work tiles runs on the small-set variant (128 x 128 work tiles, two workgroups
    per CU): 400 problems of 128 x 128 give a grid above one workgroup per CU, which only that variant
    allows.  Its D is bit-identical to the per-problem baseline's, which runs the configuration's large
    work tiles (every element goes through the same stages and MFMA steps), and matches the oracle on
    sampled problems."""
    say(f"small-set work tiles {config}")
    count = 400
    rng = np.random.default_rng(31)
    m = np.full(count, 128, np.int64)
    n = np.full(count, 128, np.int64)
    k = rng.integers(33, 400, count)
    spec = custom_spec("small400", m, n, k, alpha=rng.uniform(0.5, 2.0, count), beta=rng.uniform(0, 1, count),
                       c_dist=("uniform", -1.0, 1.0), config=config)
    dw = DeviceWorkload(spec)
    probs = dw.problems()
    cfg = KernelConfig.named(config)
    ex = GroupedGemmExecutor()
    assert ex.build(api.prepare_problem_set(probs, cfg, SortMode.kByK), cfg) == 0
    assert ex.grid_ctas() > 256, "expected the small-set variant (two workgroups per CU)"
    dw.poison_d()
    assert ex.run() == 0
    torch.cuda.synchronize()
    grouped = dw.d.cpu().numpy().copy()
    ex.close()
    dw.poison_d()
    assert api.run_baseline_per_problem(probs, cfg) == 0
    torch.cuda.synchronize()
    baseline = dw.d.cpu().numpy()
    assert not np.isnan(grouped).any()
    assert np.array_equal(grouped.view(np.uint32), baseline.view(np.uint32))
    a = dw.a.cpu().numpy().view(np.uint16)
    b = dw.b.cpu().numpy().view(np.uint16)
    c = dw.c.cpu().numpy()
    for i in (0, 137, count - 1):
        p = probs[i]
        ai = a[dw.a_off[i]:dw.a_off[i] + p.m * p.k]
        bi = b[dw.b_off[i]:dw.b_off[i] + p.k * p.n]
        ci = c[dw.c_off[i]:dw.c_off[i] + p.m * p.n]
        want = O.gemm(p.m, p.n, p.k, ai, p.k, bi, p.n, ci, p.n, p.alpha, p.beta)
        got = grouped[dw.d_off[i]:dw.d_off[i] + p.m * p.n]
        assert np.abs(got - want).max() <= tolerance(p.k, 1.0, 1.0, 1.0, p.alpha, p.beta), i


@pytest.mark.parametrize("config", CONFIGS)
def test_edge_class_work_tiles_bit_identical(torch, config):
    """Work tiles with at most 128 rows and/or 128 columns inside their problem run in the edge
    classes of the 256 x 256 work tile (half-height / half-width stages, more buffers, other wave
    blocks).  A problem that is a row and/or column prefix of a larger one (same A, B and C memory)
    must give exactly the larger problem's bits there: every D element is the same MFMA chain over
    ascending k, whichever class computes it.  Prefixes end inside the first and the second 256-row
    (column) block and on the 128 boundary; K is 64, odd (2-byte aligned rows, a repaired last
    stage) and several stages deep.  A filler problem keeps the launch on the 256 x 256 kernel
    (grid = one workgroup per CU).  The per-problem baseline must give the same bits, and the
    smallest prefix matches the oracle."""
    cfg = KernelConfig.named(config)
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    full = 512
    prefixes = [(100, 512), (512, 100), (100, 100), (356, 512), (512, 356), (356, 356), (128, 128), (129, 129),
                (1, 1), (130, 300)]
    filler_a = torch.rand(4096 * 16, device=dev, generator=g).half()
    filler_b = torch.rand(16 * 4096, device=dev, generator=g).half()
    filler_d = torch.empty(4096 * 4096, device=dev)
    for k in (64, 333, 1000):
        say(f"edge classes, {config}, K = {k}")
        a = (torch.rand(full * k, device=dev, generator=g) * 2 - 1).half()
        b = (torch.rand(k * full, device=dev, generator=g) * 2 - 1).half()
        c = torch.rand(full * full, device=dev, generator=g) * 2 - 1
        ds = [torch.full((full * full,), float("nan"), device=dev) for _ in range(len(prefixes) + 1)]
        shapes = [(full, full)] + prefixes
        probs = [ProblemDesc(m, n, k, a.data_ptr(), b.data_ptr(), c.data_ptr(), d.data_ptr(), k, full, full, full,
                             1.25, 0.5) for (m, n), d in zip(shapes, ds)]
        probs.append(ProblemDesc(4096, 4096, 16, filler_a.data_ptr(), filler_b.data_ptr(), None, filler_d.data_ptr(),
                                 16, 4096, 4096, 4096))
        ex = GroupedGemmExecutor()
        assert ex.build(api.prepare_problem_set(probs, cfg, SortMode.kByK), cfg) == 0
        assert ex.grid_ctas() == 256, "expected the 256 x 256 work-tile kernel"
        assert ex.run() == 0
        torch.cuda.synchronize()
        ex.close()
        ref = ds[0].view(full, full).view(torch.int32)
        for (m, n), d in zip(prefixes, ds[1:]):
            got = d.view(full, full)
            assert not torch.isnan(got[:m, :n]).any(), (m, n, k)
            assert torch.equal(got[:m, :n].view(torch.int32), ref[:m, :n]), f"prefix {m} x {n}, K {k}"
            assert torch.isnan(got[m:, :]).all() and torch.isnan(got[:, n:]).all(), (m, n, k)
        grouped = [d.clone() for d in ds]
        for d in ds:
            d.fill_(float("nan"))
        assert api.run_baseline_per_problem(probs, cfg) == 0
        torch.cuda.synchronize()
        for d0, d1 in zip(grouped, ds):
            assert torch.equal(torch.nan_to_num(d0, nan=7.0).view(torch.int32),
                               torch.nan_to_num(d1, nan=7.0).view(torch.int32))
        m, n = 100, 100
        a_h = a.cpu().numpy().view(np.uint16)
        b_h = b.cpu().numpy().view(np.uint16)
        c_h = c.cpu().numpy()
        want = O.gemm(m, n, k, a_h, k, b_h, full, c_h, full, 1.25, 0.5, ldd=full)
        got = grouped[3].cpu().numpy()
        for r in range(m):
            np.testing.assert_array_less(np.abs(got[r * full:r * full + n] - want[r * full:r * full + n]),
                                         tolerance(k, 1.0, 1.0, 1.0, 1.25, 0.5) + 1e-12)


def test_wall_clock_trace(torch):
    spec = make_spec("plumbing16")
    dw = DeviceWorkload(spec)
    cfg = KernelConfig.named("128x64x32")
    prep = api.prepare_problem_set(dw.problems(), cfg, SortMode.kByTiles)
    ex = GroupedGemmExecutor()
    assert ex.build(prep, cfg) == 0
    clock = torch.zeros(2 * ex.grid_ctas(), dtype=torch.int64, device="cuda")
    assert ex.run_traced(0, clock.data_ptr()) == 0
    torch.cuda.synchronize()
    c = clock.cpu().numpy().reshape(-1, 2)
    assert (c[:, 0] > 0).all() and (c[:, 1] >= c[:, 0]).all()
    assert c[:, 1].max() - c[:, 0].min() < 100_000_000  # under a second at 100 MHz


@pytest.mark.parametrize("name", ["mixed512", "plumbing16"])
def test_tile_phase_stamps(torch, name):
    """A traced launch with a phase buffer computes the same D bits as run() and stamps every
    launched work tile once, its phases in order (start <= first stage <= k-loop <= k-loop end <=
    epilogue <= last epilogue end), by a workgroup of the grid, and each of its waves' five marks of
    the middle k-loop step in order within the k-loop."""
    spec = make_spec(name)
    dw = DeviceWorkload(spec)
    cfg = KernelConfig.named("128x64x32")
    ex = GroupedGemmExecutor()
    assert ex.build(api.prepare_problem_set(dw.problems(), cfg, SortMode.kByTiles), cfg) == 0
    dw.poison_d()
    assert ex.run() == 0
    torch.cuda.synchronize()
    want = dw.d.clone()
    n = ex.launched_work_tiles()
    assert n >= 1
    phases = torch.zeros(_lib.GGK_PHASE_COUNT * n, dtype=torch.int64, device="cuda")
    dw.poison_d()
    assert ex.run_traced(0, 0, None, phases.data_ptr()) == 0
    torch.cuda.synchronize()
    assert torch.equal(dw.d.view(torch.int32), want.view(torch.int32)), "stamped run changed D"
    ph = phases.cpu().numpy().reshape(n, _lib.GGK_PHASE_COUNT)
    assert (ph[:, _lib.GGK_PHASE_START] > 0).all(), "a launched work tile was not stamped"
    order = [_lib.GGK_PHASE_START, _lib.GGK_PHASE_FIRST_STAGE, _lib.GGK_PHASE_K_LOOP, _lib.GGK_PHASE_K_END,
             _lib.GGK_PHASE_EPILOGUE, _lib.GGK_PHASE_EPILOGUE_END]
    for a, b in zip(order, order[1:]):
        assert (ph[:, a] <= ph[:, b]).all(), (a, b)
    wg = ph[:, _lib.GGK_PHASE_WHO] & 0xFFFFF
    assert ((wg >= 0) & (wg < ex.grid_ctas())).all()
    # Every wave stamps the middle k-loop step of every tile with stages, in order, inside the
    # tile's k-loop (one CU's core clock); the waves a tile's kernel does not have stay zero.
    shape, _, _, _ = ex.schedule()
    waves = shape.threads // 64
    stages = (ph[:, _lib.GGK_PHASE_WHO] >> 46) & 0x1FFFF
    step = ph[:, _lib.GGK_PHASE_STEP:].reshape(n, _lib.GGK_PHASE_STEP_WAVES, _lib.GGK_PHASE_STEP_MARKS)
    live = stages > 0
    assert live.any()
    assert (step[live, :waves, :] > 0).all(), "a wave did not stamp its middle step"
    assert (step[:, waves:, :] == 0).all() and (step[~live] == 0).all()
    for i in range(_lib.GGK_PHASE_STEP_MARKS - 1):
        assert (step[live, :waves, i] <= step[live, :waves, i + 1]).all(), i
    assert (step[live, :waves, 0] >= ph[live, _lib.GGK_PHASE_K_LOOP, None]).all()
    assert (step[live, :waves, 4] <= ph[live, _lib.GGK_PHASE_K_END, None]).all()
    say(f"{name}: {n} work tiles stamped, mean k-loop share "
        f"{float(np.mean((ph[:, 4] - ph[:, 3]) / np.maximum(ph[:, 6] - ph[:, 1], 1))):.3f}")
    ex.close()


def test_cpp_dropin_driver(torch):
    """The C++ test driver uses include/grouped_gemm/grouped_gemm.h the way the reference's
    tests/test_correctness.cu uses its header."""
    exe = ROOT / "grouped_gemm_gpu_kernel_amd" / "_build" / "bin" / "test_correctness"
    assert exe.exists(), "C++ driver not built"
    torch.cuda.synchronize()
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=110)
    sys.stdout.write(out.stdout[-4000:])
    assert out.returncode == 0, out.stdout[-2000:] + out.stderr[-2000:]
    assert "All correctness checks passed." in out.stdout


@pytest.mark.parametrize("name,ranks", [("moe64", 8), ("mixed512", 3)])
def test_shards_give_the_unsplit_d(torch, name, ranks):
    """A data-parallel split (plan_shards: whole problems, and column ranges of the ones above a
    rank's share) run rank by rank on this GPU writes the same D bits as the unsplit set: each
    element is computed by the same work tile with the same k order."""
    spec = make_spec(name)
    dw = DeviceWorkload(spec)
    probs = dw.problems()
    cfg = KernelConfig.named(spec.config)
    dw.poison_d()
    assert api.run_grouped_gemm_once(probs, SortMode.kByTiles, cfg) == 0
    torch.cuda.synchronize()
    want = dw.d.clone()
    pieces = api.plan_shards(probs, cfg, ranks)
    assert {p.rank for p in pieces} == set(range(ranks))
    say(f"{name}: {len(pieces)} pieces over {ranks} ranks")
    dw.poison_d()
    for r in range(ranks):
        share = [api.shard_problem(probs[p.problem], p) for p in pieces if p.rank == r]
        assert api.run_grouped_gemm_once(share, SortMode.kByTiles, cfg) == 0
    torch.cuda.synchronize()
    assert torch.equal(dw.d.view(torch.int32), want.view(torch.int32)), "sharded D differs"
    del want
