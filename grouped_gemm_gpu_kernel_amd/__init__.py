"""MI355X (gfx950) grouped FP16 GEMM: D_p = alpha_p * A_p @ B_p + beta_p * C_p for many problems
in one persistent launch, behind the C++/C-ABI host interface of the reference grouped GEMM.

The HIP library lives in lib/libgrouped_gemm_amd.so (built by grouped_gemm_gpu_kernel_amd.build);
this package is its Python binding.
"""
from .api import (  # noqa: F401
    GroupedGemmExecutor,
    KernelConfig,
    OccupancyInfo,
    PreparedProblemSet,
    ProblemDesc,
    SortMode,
    count_non_empty_problems,
    grid_ctas_for,
    prepare_problem_set,
    query_occupancy,
    run_baseline_per_problem,
    run_grouped_gemm_once,
    sort_mode_name,
    tail_work_share,
    tile_count_for_problem,
    total_flops,
)

__all__ = [
    "GroupedGemmExecutor", "KernelConfig", "OccupancyInfo", "PreparedProblemSet", "ProblemDesc", "SortMode",
    "count_non_empty_problems", "grid_ctas_for", "prepare_problem_set", "query_occupancy",
    "run_baseline_per_problem", "run_grouped_gemm_once", "sort_mode_name", "tail_work_share",
    "tile_count_for_problem", "total_flops",
]
