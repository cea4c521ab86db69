/*
 * grouped_gemm_amd.h -- C-ABI of the MI355X grouped FP16 GEMM.
 *
 * The FFI boundary of the library: every entry point of the reference's C++
 * API (include/grouped_gemm/grouped_gemm.cuh) as an extern "C" function over
 * plain structs, pointers and sizes, returning hipError_t codes as int.  A
 * binding (ctypes, cgo, JNI, N-API) needs only this header.  The C++ API in
 * include/grouped_gemm/grouped_gemm.h is the same library seen from C++.
 *
 * Problem arrays are passed as gg_problem_desc, which has the layout of the
 * C++ ProblemDesc (static_asserts in the implementation keep them in step).
 */
#ifndef GROUPED_GEMM_AMD_H_
#define GROUPED_GEMM_AMD_H_

#include <stdint.h>

#include "grouped_gemm_amd_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ProblemDesc (include/grouped_gemm/grouped_gemm.cuh:18-35).  a, b: binary16
 * device pointers; c may be NULL. */
typedef struct gg_problem_desc {
  int m;
  int n;
  int k;
  const void* a;
  const void* b;
  const float* c;
  float* d;
  int lda;
  int ldb;
  int ldc;
  int ldd;
  float alpha;
  float beta;
} gg_problem_desc;

/* KernelConfig (include/grouped_gemm/grouped_gemm.cuh:37-45); use_tensor_cores
 * is 0 or 1. */
typedef struct gg_kernel_config {
  int cta_m;
  int cta_n;
  int cta_k;
  int threads;
  int persistent_ctas;
  int use_tensor_cores;
} gg_kernel_config;

/* OccupancyInfo (include/grouped_gemm/grouped_gemm.cuh:54-83) plus the gfx950
 * register split. */
typedef struct gg_occupancy_info {
  int sm_count;
  int max_blocks_per_sm;
  int active_blocks_per_sm;
  int threads_per_block;
  int max_threads_per_sm;
  int warps_per_block;
  int max_warps_per_sm;
  int active_warps_per_sm;
  int max_registers_per_sm;
  int max_registers_per_block;
  int estimated_registers_per_thread;
  int estimated_registers_per_block;
  int registers_per_thread;
  int registers_per_block;
  int register_limited_blocks_per_sm;
  int static_shared_bytes;
  int dynamic_shared_bytes;
  float theoretical_occupancy;
  int using_tensor_cores;
  int vgprs_per_thread;
  int agprs_per_thread;
  int sgprs_per_wave;
  int scratch_bytes_per_thread;
  int lds_limited_blocks_per_sm;
  int wave_limited_blocks_per_sm;
} gg_occupancy_info;

/* SortMode values (include/grouped_gemm/grouped_gemm.cuh:11-16). */
enum { GG_SORT_NONE = 0, GG_SORT_BY_K = 1, GG_SORT_BY_TILES = 2, GG_SORT_BY_TILES_THEN_K = 3 };

typedef struct gg_executor gg_executor;

/* Library version string. */
const char* gg_version(void);

/* sort_mode_name (src/grouped_gemm.cu:952-965): "none", "sort_by_k",
 * "sort_by_tiles", "sort_by_tiles_then_k", or "unknown". */
const char* gg_sort_mode_name(int sort_mode);

/* Tile count of one problem (tile_count_for_problem, src/grouped_gemm.cu:54-65). */
int gg_tile_count(const gg_problem_desc* problem, const gg_kernel_config* config);

/* prepare_problem_set (src/grouped_gemm.cu:967-1022).  Host only, no GPU use.
 * Writes count sorted problems, the count-entry permutation sorted_to_original
 * and the count+1 tile_offsets; any output may be NULL.  Returns total_tiles. */
int gg_prepare_problem_set(const gg_problem_desc* problems, int count, const gg_kernel_config* config,
                           int sort_mode, gg_problem_desc* sorted_problems, int* sorted_to_original,
                           int* tile_offsets);

/* query_occupancy (src/grouped_gemm.cu:1024-1083). */
int gg_query_occupancy(const gg_kernel_config* config, gg_occupancy_info* info);

/* GroupedGemmExecutor (include/grouped_gemm/grouped_gemm.cuh:94-115). */
gg_executor* gg_executor_create(void);
void gg_executor_destroy(gg_executor* executor);
/* build (src/grouped_gemm.cu:1132-1239) from a prepared set: count sorted
 * problems, offsets_len (must be count + 1) tile offsets, total_tiles. */
int gg_executor_build(gg_executor* executor, const gg_problem_desc* sorted_problems, int count,
                      const int* tile_offsets, int offsets_len, int total_tiles,
                      const gg_kernel_config* config);
/* run (src/grouped_gemm.cu:1241-1265); stream is a hipStream_t (NULL: default). */
int gg_executor_run(const gg_executor* executor, hipStream_t stream);
/* Instrumented run, see ggk_launch_grouped_traced (d_tile_phases may be NULL). */
int gg_executor_run_traced(const gg_executor* executor, int* d_tile_map, long long* d_wg_clock,
                           long long* d_tile_phases, hipStream_t stream);
/* GroupedGemmExecutor::launched_work_tiles (no reference counterpart). */
int gg_executor_launched_work_tiles(const gg_executor* executor);
int gg_executor_problem_count(const gg_executor* executor);
int gg_executor_total_tiles(const gg_executor* executor);
int gg_executor_grid_ctas(const gg_executor* executor);
int gg_executor_using_tensor_cores(const gg_executor* executor);
/* GroupedGemmExecutor::schedule (no reference counterpart): work-tile shape,
 * order[problem_count], work_offsets[problem_count + 1],
 * chunk_bounds[GGK_SCHEDULER_CHUNKS + 1]; any output may be NULL. */
int gg_executor_schedule(const gg_executor* executor, ggk_work_shape* shape, int* order, int* work_offsets,
                         int* chunk_bounds);

/* run_grouped_gemm_once (src/grouped_gemm.cu:1279-1291). */
int gg_run_grouped_gemm_once(const gg_problem_desc* problems, int count, int sort_mode,
                             const gg_kernel_config* config, hipStream_t stream);

/* run_baseline_per_problem (src/grouped_gemm.cu:1293-1317). */
int gg_run_baseline_per_problem(const gg_problem_desc* problems, int count,
                                const gg_kernel_config* config, hipStream_t stream);

/* count_non_empty_problems (src/grouped_gemm.cu:1319-1329). */
int gg_count_non_empty_problems(const gg_problem_desc* problems, int count,
                                const gg_kernel_config* config);

/* Persistent grid size that build() would choose for total_tiles on this
 * device (src/grouped_gemm.cu:1228-1236); negative hipError_t on failure. */
int gg_grid_ctas_for(const gg_kernel_config* config, int total_tiles);

/* The launch plan that gg_executor_build makes for count sorted problems
 * (grouped_gemm::plan_launch; no reference counterpart), from plain values
 * and with no device call: compute_units CUs and blocks_per_cu[v] resident
 * workgroups per CU of variant v's grouped kernel on the configuration's path
 * (GGK_VARIANT_COUNT entries).  The problems' pointers are not read.  Writes
 * *plan, order[count], work_offsets[count + 1] and the work table,
 * plan->table_ints ints (none for a set above 2^22 work tiles, which the
 * kernel searches instead), into table[table_capacity]; any array may be
 * NULL.  hipErrorInvalidValue for a table that does not fit, with *plan
 * filled. */
typedef struct gg_launch_plan {
  int variant;
  int path;
  int addressing;
  ggk_work_shape work;
  int total_work;   /* work tiles */
  int launch_total; /* work-tile indices one launch claims */
  int table_ints;   /* ints of the work table (0: none) */
  int grid;
  int halves;       /* 1 when the table lists tail halves */
  int chunk_bounds[GGK_SCHEDULER_CHUNKS + 1];
  int launch_bounds[GGK_SCHEDULER_CHUNKS + 1];
} gg_launch_plan;
int gg_plan_launch(const gg_problem_desc* sorted_problems, int count, const gg_kernel_config* config,
                   int compute_units, const int* blocks_per_cu, gg_launch_plan* plan, int* order,
                   int* work_offsets, int* table, int table_capacity);

/* grouped_gemm::plan_shards (no reference counterpart): a data-parallel split
 * of count problems across `ranks` GPUs, see grouped_gemm.h.  Writes the
 * pieces, in problem order, to pieces[capacity] and returns their number (at
 * most count + ranks), or a negative hipError_t; fewer than that many slots:
 * -hipErrorInvalidValue. */
typedef struct gg_shard_piece {
  int problem;
  int rank;
  int col0;
  int cols;
} gg_shard_piece;
int gg_plan_shards(const gg_problem_desc* problems, int count, const gg_kernel_config* config, int ranks,
                   gg_shard_piece* pieces, int capacity);

/* MoeGroupedGemm (no reference counterpart): a mixture-of-experts group whose
 * problem set is prepared on the device from device-side token counts, see
 * ggk_moe_prepare for the layout.  gg_moe_create checks the layout and
 * allocates once; gg_moe_run launches prepare + grouped kernel on the stream
 * with no host synchronisation or allocation (capturable in a HIP graph).
 * gg_moe_device_buffers returns the device-side prepared set, the scheduling
 * order last (any output may be NULL). */
typedef struct gg_moe gg_moe;
int gg_moe_create(const ggk_moe_layout* layout, const gg_kernel_config* config, int sort_mode, gg_moe** out);
int gg_moe_run(const gg_moe* moe, const int* d_counts, hipStream_t stream);
int gg_moe_grid_ctas(const gg_moe* moe);
int gg_moe_device_buffers(const gg_moe* moe, const gg_device_problem_desc** problems, const int** offsets,
                          const int** sorted_to_original, const int** header, const int** order);
void gg_moe_destroy(gg_moe* moe);

/* Allocation-free MoE group.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory -- code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc.  The same result as
 * gg_moe_create(layout, config, sort_mode), gg_moe_run(d_counts, stream) and
 * gg_moe_destroy, with the prepared set and the scheduler state in a static
 * device array of GG_MOE_NOALLOC_SCRATCH_BYTES per GPU (held until the
 * process ends) instead of an allocation: nothing is allocated or freed and
 * the host does not wait.  At most GGK_MOE_MAX_EXPERTS experts (more is
 * hipErrorInvalidValue).  Every call on a GPU uses that GPU's one array, which
 * keeps the last call's contents: each call clears the scheduler state
 * itself, and calls that overlap on one GPU (on different streams, or from
 * different threads without stream order between them) race and give wrong
 * results; calls in one stream's order do not overlap. */
#define GG_MOE_NOALLOC_SCRATCH_BYTES 99840
int gg_moe_run_noalloc(const ggk_moe_layout* layout, const gg_kernel_config* config, int sort_mode,
                       const int* d_counts, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GROUPED_GEMM_AMD_H_ */
