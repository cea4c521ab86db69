"""Python view of the grouped GEMM API.

Same names, fields and error behaviour as the reference's C++ API
(include/grouped_gemm/grouped_gemm.cuh): functions return hipError_t status
codes as ints (0 = success) where the reference returns cudaError_t, and
problems carry raw device pointers.  Everything runs in the HIP library
through its C-ABI (include/grouped_gemm_amd.h).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field, fields
from enum import IntEnum
from typing import Optional, Sequence

from . import _lib
from ._lib import GGKernelConfig, GGKMoeLayout, GGOccupancyInfo, GGProblemDesc


class SortMode(IntEnum):
    """include/grouped_gemm/grouped_gemm.cuh:11-16"""
    kNone = 0
    kByK = 1
    kByTiles = 2
    kByTilesThenK = 3


@dataclass
class ProblemDesc:
    """include/grouped_gemm/grouped_gemm.cuh:18-35.  a, b: device pointers to
    binary16 row-major A[m x lda], B[k x ldb]; c (0/None allowed), d: float32."""
    m: int
    n: int
    k: int
    a: int
    b: int
    c: Optional[int]
    d: int
    lda: int
    ldb: int
    ldc: int
    ldd: int
    alpha: float = 1.0
    beta: float = 0.0

    def to_c(self) -> GGProblemDesc:
        return GGProblemDesc(self.m, self.n, self.k, self.a or None, self.b or None, self.c or None,
                             self.d or None, self.lda, self.ldb, self.ldc, self.ldd, self.alpha, self.beta)

    @staticmethod
    def from_c(p: GGProblemDesc) -> "ProblemDesc":
        return ProblemDesc(p.m, p.n, p.k, p.a or 0, p.b or 0, p.c or None, p.d or 0, p.lda, p.ldb, p.ldc, p.ldd,
                           p.alpha, p.beta)


@dataclass
class KernelConfig:
    """include/grouped_gemm/grouped_gemm.cuh:37-45"""
    cta_m: int = 64
    cta_n: int = 64
    cta_k: int = 16
    threads: int = 256
    persistent_ctas: int = 0
    use_tensor_cores: bool = True

    def to_c(self) -> GGKernelConfig:
        return GGKernelConfig(self.cta_m, self.cta_n, self.cta_k, self.threads, self.persistent_ctas,
                              1 if self.use_tensor_cores else 0)

    @staticmethod
    def named(name: str, **kw) -> "KernelConfig":
        """'64x64x16', '128x64x32' or '64x128x32' (bench/benchmark_grouped_gemm.cu:112-234)."""
        m, n, k = (int(x) for x in name.split("x"))
        return KernelConfig(cta_m=m, cta_n=n, cta_k=k, **kw)


@dataclass
class PreparedProblemSet:
    """include/grouped_gemm/grouped_gemm.cuh:47-52"""
    sorted_problems: list = field(default_factory=list)
    sorted_to_original: list = field(default_factory=list)
    tile_offsets: list = field(default_factory=lambda: [0])
    total_tiles: int = 0


@dataclass
class OccupancyInfo:
    """include/grouped_gemm/grouped_gemm.cuh:54-83 plus the gfx950 register split."""
    sm_count: int = 0
    max_blocks_per_sm: int = 0
    active_blocks_per_sm: int = 0
    threads_per_block: int = 0
    max_threads_per_sm: int = 0
    warps_per_block: int = 0
    max_warps_per_sm: int = 0
    active_warps_per_sm: int = 0
    max_registers_per_sm: int = 0
    max_registers_per_block: int = 0
    estimated_registers_per_thread: int = 0
    estimated_registers_per_block: int = 0
    registers_per_thread: int = 0
    registers_per_block: int = 0
    register_limited_blocks_per_sm: int = 0
    static_shared_bytes: int = 0
    dynamic_shared_bytes: int = 0
    theoretical_occupancy: float = 0.0
    using_tensor_cores: bool = False
    vgprs_per_thread: int = 0
    agprs_per_thread: int = 0
    sgprs_per_wave: int = 0
    scratch_bytes_per_thread: int = 0
    lds_limited_blocks_per_sm: int = 0
    wave_limited_blocks_per_sm: int = 0


def _problem_array(problems: Sequence[ProblemDesc]):
    arr = (GGProblemDesc * max(1, len(problems)))()
    for i, p in enumerate(problems):
        arr[i] = p.to_c()
    return arr


def _stream_handle(stream) -> Optional[int]:
    """Accepts None, an int hipStream_t, or a torch.cuda.Stream."""
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream or None
    return stream.cuda_stream or None


def sort_mode_name(sort_mode: int) -> str:
    """src/grouped_gemm.cu:952-965"""
    return _lib.lib().gg_sort_mode_name(int(sort_mode)).decode()


def tile_count_for_problem(problem: ProblemDesc, config: KernelConfig) -> int:
    """src/grouped_gemm.cu:54-65"""
    return _lib.lib().gg_tile_count(ctypes.byref(problem.to_c()), ctypes.byref(config.to_c()))


def prepare_problem_set(problems: Sequence[ProblemDesc], config: KernelConfig,
                        sort_mode: int) -> PreparedProblemSet:
    """src/grouped_gemm.cu:967-1022 (host only, no GPU use)."""
    count = len(problems)
    arr = _problem_array(problems)
    out = (GGProblemDesc * max(1, count))()
    perm = (ctypes.c_int * max(1, count))()
    offsets = (ctypes.c_int * (count + 1))()
    total = _lib.lib().gg_prepare_problem_set(arr, count, ctypes.byref(config.to_c()), int(sort_mode), out,
                                              perm, offsets)
    if total < 0:
        raise ValueError("gg_prepare_problem_set rejected its arguments")
    return PreparedProblemSet(
        sorted_problems=[ProblemDesc.from_c(out[i]) for i in range(count)],
        sorted_to_original=[perm[i] for i in range(count)],
        tile_offsets=[offsets[i] for i in range(count + 1)],
        total_tiles=total,
    )


def query_occupancy(config: KernelConfig, info: Optional[OccupancyInfo] = None):
    """src/grouped_gemm.cu:1024-1083.  Returns (status, OccupancyInfo)."""
    raw = GGOccupancyInfo()
    status = _lib.lib().gg_query_occupancy(ctypes.byref(config.to_c()), ctypes.byref(raw))
    info = info if info is not None else OccupancyInfo()
    if status == _lib.HIP_SUCCESS:
        for f in fields(OccupancyInfo):
            value = getattr(raw, f.name)
            setattr(info, f.name, bool(value) if f.name == "using_tensor_cores" else value)
    return status, info


class GroupedGemmExecutor:
    """include/grouped_gemm/grouped_gemm.cuh:94-115 (src/grouped_gemm.cu:1085-1277)."""

    def __init__(self):
        self._handle = _lib.lib().gg_executor_create()
        if not self._handle:
            raise MemoryError("gg_executor_create failed")

    def close(self) -> None:
        if self._handle:
            _lib.lib().gg_executor_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def build(self, prepared: PreparedProblemSet, config: KernelConfig) -> int:
        count = len(prepared.sorted_problems)
        arr = _problem_array(prepared.sorted_problems)
        offs = (ctypes.c_int * max(1, len(prepared.tile_offsets)))(*prepared.tile_offsets)
        return _lib.lib().gg_executor_build(self._handle, arr, count, offs, len(prepared.tile_offsets),
                                            prepared.total_tiles, ctypes.byref(config.to_c()))

    def run(self, stream=None) -> int:
        return _lib.lib().gg_executor_run(self._handle, _stream_handle(stream))

    def run_traced(self, tile_map_ptr: int = 0, wg_clock_ptr: int = 0, stream=None, tile_phases_ptr: int = 0) -> int:
        """Scheduler with instrumentation: tile_map_ptr (device int[3*total_tiles]) receives
        (problem, tile_m, tile_n) per tile instead of computing; wg_clock_ptr (device
        int64[2*grid]) receives each workgroup's start/end wall clock (100 MHz);
        tile_phases_ptr (device int64[GGK_PHASE_COUNT * launched_work_tiles()], zeroed) receives
        each work tile's phase stamps (GGK_PHASE_*)."""
        return _lib.lib().gg_executor_run_traced(self._handle, tile_map_ptr or None, wg_clock_ptr or None,
                                                 tile_phases_ptr or None, _stream_handle(stream))

    def launched_work_tiles(self) -> int:
        """Work-tile indices one launch claims (row halves of the work table counted one each)."""
        return _lib.lib().gg_executor_launched_work_tiles(self._handle)

    def problem_count(self) -> int:
        return _lib.lib().gg_executor_problem_count(self._handle)

    def total_tiles(self) -> int:
        return _lib.lib().gg_executor_total_tiles(self._handle)

    def grid_ctas(self) -> int:
        return _lib.lib().gg_executor_grid_ctas(self._handle)

    def using_tensor_cores(self) -> bool:
        return bool(_lib.lib().gg_executor_using_tensor_cores(self._handle))

    def schedule(self):
        """(work shape, scheduling order, work-tile offsets in that order, chunk bounds) as build()
        planned them (no reference counterpart)."""
        count = self.problem_count()
        shape = _lib.GGKWorkShape()
        order = (ctypes.c_int * max(1, count))()
        offsets = (ctypes.c_int * (count + 1))()
        bounds = (ctypes.c_int * (_lib.GGK_SCHEDULER_CHUNKS + 1))()
        _lib.check(_lib.lib().gg_executor_schedule(self._handle, ctypes.byref(shape), order, offsets, bounds),
                   "gg_executor_schedule")
        return shape, list(order)[:count], list(offsets), list(bounds)


@dataclass
class MoeLayout:
    """A mixture-of-experts group (no reference counterpart, see ggk_moe_prepare): expert e
    multiplies rows [r_e, r_e + count_e) of A (fp16, rows x k, lda) by B + e * stride_b (fp16,
    k x n, ldb) into the same rows of D (fp32, ldd), adding beta * C (fp32, ldc) when c is set."""
    experts: int
    n: int
    k: int
    a: int
    lda: int
    b: int
    ldb: int
    stride_b: int
    c: Optional[int]
    ldc: int
    d: int
    ldd: int
    alpha: float = 1.0
    beta: float = 0.0
    max_rows: int = 0

    def to_c(self) -> GGKMoeLayout:
        return GGKMoeLayout(self.experts, self.n, self.k, self.a or None, self.lda, self.b or None, self.ldb,
                            self.stride_b, self.c or None, self.ldc, self.d or None, self.ldd, self.alpha,
                            self.beta, self.max_rows)


class MoeGroupedGemm:
    """MoeGroupedGemm (include/grouped_gemm/grouped_gemm.h): the problem set is prepared on the
    device from device-side token counts; run() does not synchronise or allocate."""

    def __init__(self, layout: MoeLayout, config: KernelConfig, sort_mode: int = 2):
        self._handle = ctypes.c_void_p()
        self.layout = layout
        st = _lib.lib().gg_moe_create(ctypes.byref(layout.to_c()), ctypes.byref(config.to_c()), int(sort_mode),
                                      ctypes.byref(self._handle))
        _lib.check(st, "gg_moe_create")

    def run(self, counts_ptr: int, stream=None) -> int:
        return _lib.lib().gg_moe_run(self._handle, counts_ptr or None, _stream_handle(stream))

    def grid_ctas(self) -> int:
        return _lib.lib().gg_moe_grid_ctas(self._handle)

    def device_buffers(self) -> tuple:
        """(problems, offsets, sorted_to_original, header, order) device addresses."""
        ptrs = [ctypes.c_void_p() for _ in range(5)]
        _lib.check(_lib.lib().gg_moe_device_buffers(self._handle, *[ctypes.byref(p) for p in ptrs]),
                   "gg_moe_device_buffers")
        return tuple(p.value or 0 for p in ptrs)

    def close(self) -> None:
        if self._handle:
            _lib.lib().gg_moe_destroy(self._handle)
            self._handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def run_grouped_gemm_once(problems: Sequence[ProblemDesc], sort_mode: int, config: KernelConfig,
                          stream=None) -> int:
    """src/grouped_gemm.cu:1279-1291"""
    arr = _problem_array(problems)
    return _lib.lib().gg_run_grouped_gemm_once(arr, len(problems), int(sort_mode), ctypes.byref(config.to_c()),
                                               _stream_handle(stream))


def run_baseline_per_problem(problems: Sequence[ProblemDesc], config: KernelConfig, stream=None) -> int:
    """src/grouped_gemm.cu:1293-1317"""
    arr = _problem_array(problems)
    return _lib.lib().gg_run_baseline_per_problem(arr, len(problems), ctypes.byref(config.to_c()),
                                                  _stream_handle(stream))


def count_non_empty_problems(problems: Sequence[ProblemDesc], config: KernelConfig) -> int:
    """src/grouped_gemm.cu:1319-1329"""
    arr = _problem_array(problems)
    return _lib.lib().gg_count_non_empty_problems(arr, len(problems), ctypes.byref(config.to_c()))


def grid_ctas_for(config: KernelConfig, total_tiles: int) -> int:
    """Persistent grid size build() chooses on this device (src/grouped_gemm.cu:1228-1236)."""
    value = _lib.lib().gg_grid_ctas_for(ctypes.byref(config.to_c()), total_tiles)
    if value < 0:
        raise _lib.HipError(-value, "gg_grid_ctas_for")
    return value


@dataclass
class LaunchPlan:
    """gg_launch_plan plus its arrays: what GroupedGemmExecutor.build() plans for a sorted set."""
    variant: int
    path: int
    addressing: int
    work: tuple  # (tiles_m, tiles_n, threads, rows, stage_k) of the work tile
    total_work: int
    launch_total: int
    grid: int
    halves: bool
    order: list
    work_offsets: list
    chunk_bounds: list
    work_table: list  # (problem, work tile | half << GGK_WORK_HALF_SHIFT) pairs, flattened
    launch_bounds: list


def plan_launch(sorted_problems: Sequence[ProblemDesc], config: KernelConfig, compute_units: int,
                blocks_per_cu: Sequence[int]) -> LaunchPlan:
    """The launch plan build() makes (no reference counterpart), from plain device values:
    compute_units CUs and blocks_per_cu[v] resident workgroups per CU of variant v.  Host only."""
    count = len(sorted_problems)
    arr = _problem_array(sorted_problems)
    blocks = (ctypes.c_int * _lib.GGK_VARIANT_COUNT)(*blocks_per_cu)
    plan = _lib.GGLaunchPlan()
    order = (ctypes.c_int * max(1, count))()
    offsets = (ctypes.c_int * (count + 1))()
    cfg = config.to_c()
    _lib.check(_lib.lib().gg_plan_launch(arr, count, ctypes.byref(cfg), compute_units, blocks, ctypes.byref(plan),
                                         order, offsets, None, 0), "gg_plan_launch")
    table = (ctypes.c_int * max(1, plan.table_ints))()
    _lib.check(_lib.lib().gg_plan_launch(arr, count, ctypes.byref(cfg), compute_units, blocks, ctypes.byref(plan),
                                         None, None, table, plan.table_ints), "gg_plan_launch")
    w = plan.work
    return LaunchPlan(plan.variant, plan.path, plan.addressing, (w.tiles_m, w.tiles_n, w.threads, w.rows, w.stage_k),
                      plan.total_work, plan.launch_total, plan.grid, bool(plan.halves), list(order)[:count],
                      list(offsets), list(plan.chunk_bounds), list(table)[:plan.table_ints],
                      list(plan.launch_bounds))


@dataclass
class ShardPiece:
    """One piece of a data-parallel split (no reference counterpart): columns [col0, col0 + cols) of
    problem `problem`, computed by rank `rank`."""
    problem: int
    rank: int
    col0: int
    cols: int


def plan_shards(problems: Sequence[ProblemDesc], config: KernelConfig, ranks: int) -> list:
    """A split of the problems across `ranks` GPUs (grouped_gemm::plan_shards): a list of ShardPiece
    in problem and column order.  Host only."""
    count = len(problems)
    arr = _problem_array(problems)
    cap = count + ranks
    out = (_lib.GGShardPiece * max(1, cap))()
    got = _lib.lib().gg_plan_shards(arr, count, ctypes.byref(config.to_c()), ranks, out, cap)
    if got < 0:
        raise _lib.HipError(-got, "gg_plan_shards")
    return [ShardPiece(p.problem, p.rank, p.col0, p.cols) for p in out[:got]]


def shard_problem(problem: ProblemDesc, piece: ShardPiece) -> ProblemDesc:
    """The problem a piece computes: the same A, B, C and D from column col0 on, n = cols
    (grouped_gemm::shard_problem)."""
    from dataclasses import replace
    return replace(problem, n=piece.cols, b=(problem.b + 2 * piece.col0) if problem.b else problem.b,
                   c=(problem.c + 4 * piece.col0) if problem.c else problem.c,
                   d=(problem.d + 4 * piece.col0) if problem.d else problem.d)


def total_flops(problems: Sequence[ProblemDesc]) -> float:
    """sum of 2*m*n*k (bench/benchmark_grouped_gemm.cu:570-576)."""
    return float(sum(2.0 * p.m * p.n * p.k for p in problems))


def tail_work_share(prepared: PreparedProblemSet, config: KernelConfig) -> float:
    """Static tail share (bench/benchmark_grouped_gemm.cu:580-607): work = tiles * ceil(k / cta_k)
    per problem in sorted order; the share of the last max(1, count // 10) problems."""
    n = len(prepared.sorted_problems)
    if n == 0:
        return 0.0
    tail = max(1, n // 10)
    total = tail_w = 0.0
    for i, p in enumerate(prepared.sorted_problems):
        w = float(prepared.tile_offsets[i + 1] - prepared.tile_offsets[i]) * ((p.k + config.cta_k - 1) // config.cta_k)
        total += w
        if i >= n - tail:
            tail_w += w
    return tail_w / total if total > 0 else 0.0
