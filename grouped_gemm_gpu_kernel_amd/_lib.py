"""ctypes binding of libgrouped_gemm_amd.so (include/grouped_gemm_amd.h and
include/grouped_gemm_amd_kernels.h).

The library is built in-tree by grouped_gemm_gpu_kernel_amd.build; importing
this module without it raises, so no code path can silently run without the
HIP library.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libgrouped_gemm_amd.so"

# hipError_t values used by the API (hip_runtime_api.h).
HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1
HIP_ERROR_OUT_OF_MEMORY = 2
HIP_ERROR_INVALID_DEVICE_POINTER = 17

GGK_VARIANT_64x64x16 = 0
GGK_VARIANT_128x64x32 = 1
GGK_VARIANT_64x128x32 = 2
GGK_VARIANT_128x64x32_SMALL = 3  # 128x64x32 on 128 x 128 work tiles (launches with few work tiles)
GGK_VARIANT_64x128x32_SMALL = 4  # 64x128x32 on 128 x 128 work tiles
GGK_VARIANT_64x64x16_SMALL = 5  # 64x64x16 on 128 x 128 work tiles
GGK_VARIANT_COUNT = 6
GGK_PATH_FMA = 0
GGK_PATH_MFMA = 1
GGK_KERNEL_GROUPED = 0
GGK_KERNEL_SINGLE = 1
GGK_ADDR_32 = 0
GGK_ADDR_64 = 1
GGK_SCHEDULER_CHUNKS = 8
GGK_SCHEDULER_COUNTER_STRIDE = 32
GGK_SCHEDULER_STATE_INTS = GGK_SCHEDULER_COUNTER_STRIDE * (GGK_SCHEDULER_CHUNKS + 1)
GGK_WORK_HALF_SHIFT = 28  # work-table entry: local work tile | (1: first, 2: second half of rows) << shift
GGK_PHASE_WALL, GGK_PHASE_START, GGK_PHASE_FIRST_STAGE, GGK_PHASE_K_LOOP = 0, 1, 2, 3
GGK_PHASE_K_END, GGK_PHASE_EPILOGUE, GGK_PHASE_EPILOGUE_END, GGK_PHASE_WHO = 4, 5, 6, 7
GGK_PHASE_STEP, GGK_PHASE_STEP_MARKS, GGK_PHASE_STEP_WAVES = 8, 5, 8
GGK_PHASE_COUNT = 48
GGK_MOE_MAX_EXPERTS = 1024
GGK_MOE_HEADER_INTS = 16
GGK_MOE_STATUS = 12
GGK_MOE_NEGATIVE = 1
GGK_MOE_CLAMPED = 2
GG_MOE_NOALLOC_SCRATCH_BYTES = 99840

c_int_p = ctypes.POINTER(ctypes.c_int)
c_ll_p = ctypes.POINTER(ctypes.c_longlong)


class GGProblemDesc(ctypes.Structure):
    """gg_problem_desc: ProblemDesc (include/grouped_gemm/grouped_gemm.cuh:18-35)."""
    _fields_ = [
        ("m", ctypes.c_int), ("n", ctypes.c_int), ("k", ctypes.c_int),
        ("a", ctypes.c_void_p), ("b", ctypes.c_void_p), ("c", ctypes.c_void_p), ("d", ctypes.c_void_p),
        ("lda", ctypes.c_int), ("ldb", ctypes.c_int), ("ldc", ctypes.c_int), ("ldd", ctypes.c_int),
        ("alpha", ctypes.c_float), ("beta", ctypes.c_float),
    ]


class GGDeviceProblemDesc(ctypes.Structure):
    """gg_device_problem_desc: DeviceProblemDesc (src/grouped_gemm.cu:25-45)."""
    _fields_ = GGProblemDesc._fields_ + [("tiles_m", ctypes.c_int), ("tiles_n", ctypes.c_int)]


class GGKernelConfig(ctypes.Structure):
    """gg_kernel_config: KernelConfig (include/grouped_gemm/grouped_gemm.cuh:37-45)."""
    _fields_ = [
        ("cta_m", ctypes.c_int), ("cta_n", ctypes.c_int), ("cta_k", ctypes.c_int),
        ("threads", ctypes.c_int), ("persistent_ctas", ctypes.c_int), ("use_tensor_cores", ctypes.c_int),
    ]


class GGOccupancyInfo(ctypes.Structure):
    """gg_occupancy_info: OccupancyInfo (include/grouped_gemm/grouped_gemm.cuh:54-83) plus the
    gfx950 register split."""
    _fields_ = [(name, ctypes.c_int) for name in (
        "sm_count", "max_blocks_per_sm", "active_blocks_per_sm", "threads_per_block",
        "max_threads_per_sm", "warps_per_block", "max_warps_per_sm", "active_warps_per_sm",
        "max_registers_per_sm", "max_registers_per_block", "estimated_registers_per_thread",
        "estimated_registers_per_block", "registers_per_thread", "registers_per_block",
        "register_limited_blocks_per_sm", "static_shared_bytes", "dynamic_shared_bytes")] + [
        ("theoretical_occupancy", ctypes.c_float),
    ] + [(name, ctypes.c_int) for name in (
        "using_tensor_cores", "vgprs_per_thread", "agprs_per_thread", "sgprs_per_wave",
        "scratch_bytes_per_thread", "lds_limited_blocks_per_sm", "wave_limited_blocks_per_sm")]


class GGKDeviceInfo(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int) for name in (
        "device", "compute_units", "max_threads_per_cu", "max_wgs_per_cu", "wave_size", "regs_per_cu",
        "regs_per_block", "lds_per_cu", "lds_per_block", "l2_bytes", "clock_khz", "major", "minor")] + [
        ("arch_name", ctypes.c_char * 64)]


class GGKKernelResources(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int) for name in (
        "vgprs", "agprs", "sgprs", "scratch_bytes_per_lane", "compiler_waves_per_simd", "lds_bytes",
        "num_regs", "lds_static", "lds_dynamic", "local_bytes", "max_threads")]


class GGKWorkShape(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int) for name in ("tiles_m", "tiles_n", "threads", "rows", "stage_k")]


class GGLaunchPlan(ctypes.Structure):
    """gg_launch_plan (grouped_gemm_amd.h)"""
    _fields_ = [
        ("variant", ctypes.c_int), ("path", ctypes.c_int), ("addressing", ctypes.c_int), ("work", GGKWorkShape),
        ("total_work", ctypes.c_int), ("launch_total", ctypes.c_int), ("table_ints", ctypes.c_int),
        ("grid", ctypes.c_int), ("halves", ctypes.c_int),
        ("chunk_bounds", ctypes.c_int * (GGK_SCHEDULER_CHUNKS + 1)),
        ("launch_bounds", ctypes.c_int * (GGK_SCHEDULER_CHUNKS + 1)),
    ]


class GGShardPiece(ctypes.Structure):
    """gg_shard_piece (grouped_gemm_amd.h)"""
    _fields_ = [("problem", ctypes.c_int), ("rank", ctypes.c_int), ("col0", ctypes.c_int), ("cols", ctypes.c_int)]


class GGKMoeLayout(ctypes.Structure):
    """ggk_moe_layout (grouped_gemm_amd_kernels.h)"""
    _fields_ = [
        ("experts", ctypes.c_int), ("n", ctypes.c_int), ("k", ctypes.c_int),
        ("a", ctypes.c_void_p), ("lda", ctypes.c_int),
        ("b", ctypes.c_void_p), ("ldb", ctypes.c_int), ("stride_b", ctypes.c_longlong),
        ("c", ctypes.c_void_p), ("ldc", ctypes.c_int),
        ("d", ctypes.c_void_p), ("ldd", ctypes.c_int),
        ("alpha", ctypes.c_float), ("beta", ctypes.c_float), ("max_rows", ctypes.c_int),
    ]


_P = ctypes.POINTER
_vp = ctypes.c_void_p
_i = ctypes.c_int

# name: (restype, argtypes) -- every function declared in include/grouped_gemm_amd.h and
# include/grouped_gemm_amd_kernels.h.
SIGNATURES = {
    # grouped_gemm_amd.h
    "gg_version": (ctypes.c_char_p, []),
    "gg_sort_mode_name": (ctypes.c_char_p, [_i]),
    "gg_tile_count": (_i, [_P(GGProblemDesc), _P(GGKernelConfig)]),
    "gg_prepare_problem_set": (_i, [_P(GGProblemDesc), _i, _P(GGKernelConfig), _i, _P(GGProblemDesc),
                                    c_int_p, c_int_p]),
    "gg_query_occupancy": (_i, [_P(GGKernelConfig), _P(GGOccupancyInfo)]),
    "gg_executor_create": (_vp, []),
    "gg_executor_destroy": (None, [_vp]),
    "gg_executor_build": (_i, [_vp, _P(GGProblemDesc), _i, c_int_p, _i, _i, _P(GGKernelConfig)]),
    "gg_executor_run": (_i, [_vp, _vp]),
    "gg_executor_run_traced": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "gg_executor_launched_work_tiles": (_i, [_vp]),
    "gg_executor_problem_count": (_i, [_vp]),
    "gg_executor_total_tiles": (_i, [_vp]),
    "gg_executor_grid_ctas": (_i, [_vp]),
    "gg_executor_using_tensor_cores": (_i, [_vp]),
    "gg_executor_schedule": (_i, [_vp, _P(GGKWorkShape), _vp, _vp, _vp]),
    "gg_run_grouped_gemm_once": (_i, [_P(GGProblemDesc), _i, _i, _P(GGKernelConfig), _vp]),
    "gg_run_baseline_per_problem": (_i, [_P(GGProblemDesc), _i, _P(GGKernelConfig), _vp]),
    "gg_count_non_empty_problems": (_i, [_P(GGProblemDesc), _i, _P(GGKernelConfig)]),
    "gg_grid_ctas_for": (_i, [_P(GGKernelConfig), _i]),
    "gg_plan_shards": (_i, [_P(GGProblemDesc), _i, _P(GGKernelConfig), _i, _P(GGShardPiece), _i]),
    "gg_plan_launch": (_i, [_P(GGProblemDesc), _i, _P(GGKernelConfig), _i, c_int_p, _P(GGLaunchPlan), c_int_p,
                            c_int_p, c_int_p, _i]),
    "gg_moe_create": (_i, [_P(GGKMoeLayout), _P(GGKernelConfig), _i, _P(_vp)]),
    "gg_moe_run": (_i, [_vp, _vp, _vp]),
    "gg_moe_grid_ctas": (_i, [_vp]),
    "gg_moe_device_buffers": (_i, [_vp, _P(_vp), _P(_vp), _P(_vp), _P(_vp), _P(_vp)]),
    "gg_moe_destroy": (None, [_vp]),
    "gg_moe_run_noalloc": (_i, [_P(GGKMoeLayout), _P(GGKernelConfig), _i, _vp, _vp]),
    # grouped_gemm_amd_kernels.h
    "ggk_alloc": (_i, [_P(_vp), ctypes.c_size_t]),
    "ggk_free": (_i, [_vp]),
    "ggk_copy_to_device": (_i, [_vp, _vp, ctypes.c_size_t]),
    "ggk_copy_to_host": (_i, [_vp, _vp, ctypes.c_size_t]),
    "ggk_zero": (_i, [_vp, ctypes.c_size_t]),
    "ggk_stream_synchronize": (_i, [_vp]),
    "ggk_device_synchronize": (_i, []),
    "ggk_event_create": (_i, [_P(_vp)]),
    "ggk_event_destroy": (_i, [_vp]),
    "ggk_event_record_launch": (_i, [_vp, _vp, c_int_p]),
    "ggk_event_synchronize": (_i, [_vp]),
    "ggk_current_device": (_i, [c_int_p]),
    "ggk_device_info_get": (_i, [_P(GGKDeviceInfo)]),
    "ggk_work_shape_get": (_i, [_i, _i, _P(GGKWorkShape)]),
    "ggk_needs_addr64": (_i, [_i, _i, _P(GGDeviceProblemDesc)]),
    "ggk_work_halves_supported": (_i, [_i, _i]),
    "ggk_small_variant": (_i, [_i]),
    "ggk_launch_grouped": (_i, [_i, _i, _i, _vp, _vp, _vp, _vp, _i, _i, _vp, c_int_p, _i, _vp]),
    "ggk_launch_grouped_traced": (_i, [_i, _i, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, c_int_p, _i, _vp, _vp,
                                       _vp, _vp]),
    "ggk_launch_single": (_i, [_i, _i, _P(GGDeviceProblemDesc), _vp]),
    "ggk_moe_prepare": (_i, [_i, _i, _P(GGKMoeLayout), _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ggk_moe_layout_check": (_i, [_i, _i, _P(GGKMoeLayout)]),
    "ggk_launch_grouped_device": (_i, [_i, _i, _i, _vp, _vp, _vp, _i, _vp, _vp, _i, _vp]),
    "ggk_kernel_resources_get": (_i, [_i, _i, _i, _P(GGKKernelResources)]),
    "ggk_occupancy": (_i, [_i, _i, c_int_p]),
    "ggk_fill_uniform_f16": (_i, [_vp, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float,
                                  ctypes.c_float, _vp]),
    "ggk_fill_uniform_f32": (_i, [_vp, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float,
                                  ctypes.c_float, _vp]),
    "ggk_fill_normal_f16": (_i, [_vp, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float,
                                 _vp]),
    "ggk_fill_f32": (_i, [_vp, ctypes.c_int64, ctypes.c_float, _vp]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m grouped_gemm_gpu_kernel_amd.build` "
                "(or __graft_entry__.build()); there is no fallback implementation")
        handle = ctypes.CDLL(os.fspath(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


class HipError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what} failed with hipError_t {status}")
        self.status = status


def check(status: int, what: str) -> None:
    if status != HIP_SUCCESS:
        raise HipError(status, what)
