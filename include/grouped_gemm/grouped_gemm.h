// grouped_gemm.h -- C++ host API of the MI355X grouped FP16 GEMM.
//
// Drop-in for include/grouped_gemm/grouped_gemm.cuh of the reference: the same
// namespace, names, fields, defaults and semantics, with HIP types in place of
// CUDA ones (hipError_t, hipStream_t, __half from <hip/hip_fp16.h>).
//
// Each batch computes, for every problem p, D_p = alpha_p * A_p * B_p + beta_p * C_p
// with A_p [m x k] and B_p [k x n] row-major binary16, C_p / D_p [m x n]
// row-major float32, and float32 accumulation.  C is read only when c != nullptr
// and beta != 0.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <array>
#include <cstdint>
#include <functional>
#include <vector>

#include "grouped_gemm_amd_kernels.h"

namespace grouped_gemm {

// include/grouped_gemm/grouped_gemm.cuh:11-16
enum class SortMode {
  kNone = 0,
  kByK = 1,
  kByTiles = 2,
  kByTilesThenK = 3,
};

// include/grouped_gemm/grouped_gemm.cuh:18-35
struct ProblemDesc {
  int m;
  int n;
  int k;

  const __half* a;
  const __half* b;
  const float* c;
  float* d;

  int lda;
  int ldb;
  int ldc;
  int ldd;

  float alpha = 1.0f;
  float beta = 0.0f;
};

// include/grouped_gemm/grouped_gemm.cuh:37-45.  Accepted shapes, as in the
// reference: threads == 256 and (cta_m, cta_n, cta_k) one of (64, 64, 16),
// (128, 64, 32), (64, 128, 32).  use_tensor_cores selects the MFMA tile path;
// false selects the FMA tile path.
struct KernelConfig {
  int cta_m = 64;
  int cta_n = 64;
  int cta_k = 16;
  int threads = 256;

  int persistent_ctas = 0;
  bool use_tensor_cores = true;
};

// include/grouped_gemm/grouped_gemm.cuh:47-52
struct PreparedProblemSet {
  std::vector<ProblemDesc> sorted_problems;
  std::vector<int> sorted_to_original;
  std::vector<int> tile_offsets;
  int total_tiles = 0;
};

// include/grouped_gemm/grouped_gemm.cuh:54-83.  "sm" reads "compute unit" and
// "warp" reads "wavefront" (64 lanes) on this GPU.  The fields after
// using_tensor_cores are additions that report the gfx950 register split.
struct OccupancyInfo {
  int sm_count = 0;
  int max_blocks_per_sm = 0;
  int active_blocks_per_sm = 0;

  int threads_per_block = 0;
  int max_threads_per_sm = 0;
  int warps_per_block = 0;
  int max_warps_per_sm = 0;
  int active_warps_per_sm = 0;

  int max_registers_per_sm = 0;
  int max_registers_per_block = 0;

  // Formula estimate from the tile shape and the MFMA accumulator layout.
  int estimated_registers_per_thread = 0;
  int estimated_registers_per_block = 0;

  // Measured on the compiled kernel: VGPRs + AGPRs per lane.
  int registers_per_thread = 0;
  int registers_per_block = 0;
  int register_limited_blocks_per_sm = 0;

  int static_shared_bytes = 0;
  int dynamic_shared_bytes = 0;

  float theoretical_occupancy = 0.0f;
  bool using_tensor_cores = false;

  // gfx950 additions.
  int vgprs_per_thread = 0;
  int agprs_per_thread = 0;
  int sgprs_per_wave = 0;
  int scratch_bytes_per_thread = 0;
  int lds_limited_blocks_per_sm = 0;
  int wave_limited_blocks_per_sm = 0;
};

// DeviceProblemDesc (src/grouped_gemm.cu:25-45): ProblemDesc plus tiles_m and
// tiles_n, as the kernels read it.
using DeviceProblemDesc = gg_device_problem_desc;

// include/grouped_gemm/grouped_gemm.cuh:85-88
PreparedProblemSet prepare_problem_set(
    const std::vector<ProblemDesc>& problems,
    const KernelConfig& config,
    SortMode sort_mode);

// include/grouped_gemm/grouped_gemm.cuh:90
const char* sort_mode_name(SortMode sort_mode);

// include/grouped_gemm/grouped_gemm.cuh:92
hipError_t query_occupancy(const KernelConfig& config, OccupancyInfo* info);

// include/grouped_gemm/grouped_gemm.cuh:94-115.  build() uploads the sorted
// descriptors and tile offsets once; run() launches one persistent grid on the
// given stream.  Not thread-safe: runs of one executor must not overlap (they
// share one scheduler state).  Device buffers are rewritten or released on
// rebuild, move-assignment and destruction only after the executor's last
// launch has completed (an event recorded on that launch's stream); once a
// run was captured into a graph, after a device synchronisation instead, since
// the graph's replays may run on any stream (no capture may then be in
// progress on the device).
class GroupedGemmExecutor {
 public:
  GroupedGemmExecutor();
  ~GroupedGemmExecutor();

  GroupedGemmExecutor(const GroupedGemmExecutor&) = delete;
  GroupedGemmExecutor& operator=(const GroupedGemmExecutor&) = delete;

  GroupedGemmExecutor(GroupedGemmExecutor&& other) noexcept;
  GroupedGemmExecutor& operator=(GroupedGemmExecutor&& other) noexcept;

  hipError_t build(const PreparedProblemSet& prepared, const KernelConfig& config);
  hipError_t run(hipStream_t stream = nullptr) const;

  int problem_count() const;
  int total_tiles() const;
  int grid_ctas() const;

  // Additions for measurement and parity checks.  run_traced() runs the same
  // scheduler with instrumentation (see ggk_launch_grouped_traced);
  // d_tile_phases holds GGK_PHASE_COUNT int64s per launched work tile
  // (launched_work_tiles()).
  hipError_t run_traced(int* d_tile_map, long long* d_wg_clock, hipStream_t stream = nullptr,
                        long long* d_tile_phases = nullptr) const;
  // Work-tile indices one launch claims: the work tiles, with the row halves
  // the work table lists counted one each.
  int launched_work_tiles() const;
  bool using_tensor_cores() const;
  // The schedule build() planned: the work-tile shape of the kernel it chose,
  // the scheduling order (sorted position at each scheduling position), the
  // work-tile offsets in that order and the per-XCD chunk bounds.  Reads the
  // device copy back (synchronous); any output may be null.
  hipError_t schedule(ggk_work_shape* shape, std::vector<int>* order, std::vector<int>* work_offsets,
                      std::vector<int>* chunk_bounds) const;

 private:
  struct Impl;
  Impl* impl_;
};

// include/grouped_gemm/grouped_gemm.cuh:117-121.  Synchronises the stream
// before returning so that the executor's device buffers can be released.
hipError_t run_grouped_gemm_once(
    const std::vector<ProblemDesc>& problems,
    SortMode sort_mode,
    const KernelConfig& config,
    hipStream_t stream = nullptr);

// include/grouped_gemm/grouped_gemm.cuh:123-126
hipError_t run_baseline_per_problem(
    const std::vector<ProblemDesc>& problems,
    const KernelConfig& config,
    hipStream_t stream = nullptr);

// include/grouped_gemm/grouped_gemm.cuh:128-130
int count_non_empty_problems(
    const std::vector<ProblemDesc>& problems,
    const KernelConfig& config);

// src/grouped_gemm.cu:912-930
DeviceProblemDesc to_device_problem(const ProblemDesc& problem, const KernelConfig& config);

// src/grouped_gemm.cu:54-65.  Clamped at INT_MAX (the reference's int product
// overflows); prepare_problem_set's offsets saturate there too, and build()
// rejects such a set (its offsets no longer step by the tile counts).
int tile_count_for_problem(const ProblemDesc& problem, const KernelConfig& config);

// Persistent grid size build() chooses (src/grouped_gemm.cu:1228-1236):
// config.persistent_ctas if positive, else
// max(1, min(sm_count * max(1, active_blocks_per_sm), max(total_tiles, sm_count)));
// 0 when total_tiles is 0.
int grid_ctas_for(int total_tiles, const KernelConfig& config, const OccupancyInfo& occupancy);

// Addition with no counterpart in the reference: the launch plan that
// GroupedGemmExecutor::build() makes for a set of sorted problems, computed
// from plain values with no device call.
//  * variant: the configuration's own, or its 128 x 128 work-tile form when
//    the set has at most 4 such work tiles per CU (compute_units CUs) or
//    needs 64-bit addressing in the 256 x 256 form; addressing as it needs.
//  * schedule: order, work_offsets and chunk_bounds as
//    GroupedGemmExecutor::schedule() reports them.
//  * grid: grid_ctas_for(total_work) with blocks_per_cu(variant, path)
//    resident workgroups per CU.
//  * work_table: (problem, work tile) pairs in claim order, a work tile among
//    the last of its chunk listed as its two row halves (GGK_WORK_HALF_SHIFT)
//    when the kernel reads halves and the planned schedule leaves a ragged
//    end; empty above 2^22 work tiles (the kernel then searches).
//    launch_total and launch_bounds count its entries (without a table, the
//    work tiles and chunk_bounds).
struct LaunchPlan {
  int variant = -1;
  int path = -1;
  int addressing = GGK_ADDR_32;
  ggk_work_shape work{};
  std::vector<int> order;
  std::vector<int> work_offsets;
  std::array<int, GGK_SCHEDULER_CHUNKS + 1> chunk_bounds{};
  std::vector<int> work_table;
  std::array<int, GGK_SCHEDULER_CHUNKS + 1> launch_bounds{};
  int total_work = 0;
  int launch_total = 0;
  int grid = 0;
  bool halves = false;
};

// Resident workgroups per CU of the grouped kernel of (variant, path).
using BlocksPerCu = std::function<hipError_t(int variant, int path, int* blocks)>;

// hipErrorInvalidValue for a configuration without a kernel, compute_units
// below 1, a negative extent, tile counts that are not the ceilings of
// m / cta_m and n / cta_n (zero for an empty problem), or a set of more than
// INT_MAX macro-tiles.
hipError_t plan_launch(const std::vector<DeviceProblemDesc>& problems, const KernelConfig& config,
                       int compute_units, const BlocksPerCu& blocks_per_cu, LaunchPlan* plan);

// Addition with no counterpart in the reference: a data-parallel split of a
// problem list across `ranks` GPUs.  Problems are independent, so no data
// moves between ranks.  Each piece is a whole problem or, for a problem whose
// estimated time exceeds one rank's share (the total over `ranks`), one of
// several ranges of its columns cut at work-tile column boundaries, so D comes
// out bit for bit as in the unsplit set.  The estimate is the executor's
// schedule model on the configuration's own work tile.  Pieces go longest
// first, each to the rank with the least estimated time so far (ties: the
// lowest rank).  `pieces` lists them in problem order and column order.
// Empty problems stay whole (on rank 0).  At most problems.size() + ranks
// pieces result.  hipErrorInvalidValue for a configuration without a kernel,
// ranks below 1 or a negative extent.
struct ShardPiece {
  int problem;  // index into the problem list
  int rank;     // 0 .. ranks - 1
  int col0;     // first column of D (and of B and C) the piece covers
  int cols;     // columns covered
};
hipError_t plan_shards(const std::vector<ProblemDesc>& problems, const KernelConfig& config, int ranks,
                       std::vector<ShardPiece>* pieces);
// The problem a piece computes: columns [col0, col0 + cols) of `problem`.
ProblemDesc shard_problem(const ProblemDesc& problem, const ShardPiece& piece);

// ---------------------------------------------------------------------------
// Additions with no counterpart in the reference: the grouped GEMM of a
// mixture-of-experts layer, prepared on the device from device-side token
// counts (see ggk_moe_prepare).  Expert e multiplies rows [r_e, r_e + count_e)
// of A (rows x k) by B + e * stride_b (k x n) into the same rows of D, adding
// beta * C when c is set; r_e is the prefix sum of the counts.
struct MoeLayout {
  int experts = 0;
  int n = 0;
  int k = 0;
  const __half* a = nullptr;
  int lda = 0;
  const __half* b = nullptr;
  int ldb = 0;
  int64_t stride_b = 0;  // elements between consecutive experts' B
  const float* c = nullptr;
  int ldc = 0;
  float* d = nullptr;
  int ldd = 0;
  float alpha = 1.0f;
  float beta = 0.0f;
  int max_rows = 0;  // rows of A, C and D the caller owns; rows past it are dropped
};

// build() checks the layout and allocates the device-side set once; run()
// launches the prepare kernel and the grouped kernel on the stream, with no
// host synchronisation and no allocation, so it can be captured in a HIP
// graph and replayed with new counts.  Runs must not overlap (one scheduler
// state per object).
class MoeGroupedGemm {
 public:
  MoeGroupedGemm();
  ~MoeGroupedGemm();
  MoeGroupedGemm(const MoeGroupedGemm&) = delete;
  MoeGroupedGemm& operator=(const MoeGroupedGemm&) = delete;
  MoeGroupedGemm(MoeGroupedGemm&& other) noexcept;
  MoeGroupedGemm& operator=(MoeGroupedGemm&& other) noexcept;

  hipError_t build(const MoeLayout& layout, const KernelConfig& config, SortMode sort_mode);
  // d_counts: device int[experts], rows per expert.
  hipError_t run(const int* d_counts, hipStream_t stream = nullptr) const;

  int grid_ctas() const;
  // The prepared set as the last run wrote it (device memory, stream order):
  // experts descriptors, 2 * (experts + 1) offsets (reference tiles, then work
  // tiles in scheduling order), the permutation, the scheduling order
  // (experts sorted positions) and GGK_MOE_HEADER_INTS header ints.
  const DeviceProblemDesc* device_problems() const;
  const int* device_offsets() const;
  const int* device_sorted_to_original() const;
  const int* device_order() const;
  const int* device_header() const;

 private:
  struct Impl;
  Impl* impl_;
};

// Allocation-free form of MoeGroupedGemm (build + run + destroy in one call),
// for callers that cannot allocate device memory; no counterpart in the
// reference.  See gg_moe_run_noalloc (grouped_gemm_amd.h) for the limits and
// the rule that calls on one GPU must not overlap.
hipError_t run_moe_grouped_gemm_noalloc(const MoeLayout& layout, const KernelConfig& config, SortMode sort_mode,
                                        const int* d_counts, hipStream_t stream = nullptr);

}  // namespace grouped_gemm
