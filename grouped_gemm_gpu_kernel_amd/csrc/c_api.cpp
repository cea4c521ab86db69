// c_api.cpp -- extern "C" facade (include/grouped_gemm_amd.h) over the C++ API.
//
// Each entry point converts plain structs to the C++ types, calls the
// namespace grouped_gemm function of the same name and returns its hipError_t
// as int.  No exception crosses this boundary.
#include "grouped_gemm_amd.h"

#include <algorithm>
#include <cstddef>
#include <new>
#include <vector>

#include "grouped_gemm/grouped_gemm.h"

namespace gg = grouped_gemm;

// gg_problem_desc and grouped_gemm::ProblemDesc must stay layout-identical.
static_assert(sizeof(gg_problem_desc) == sizeof(gg::ProblemDesc), "ProblemDesc layout");
static_assert(offsetof(gg_problem_desc, a) == offsetof(gg::ProblemDesc, a), "ProblemDesc.a");
static_assert(offsetof(gg_problem_desc, d) == offsetof(gg::ProblemDesc, d), "ProblemDesc.d");
static_assert(offsetof(gg_problem_desc, ldd) == offsetof(gg::ProblemDesc, ldd), "ProblemDesc.ldd");
static_assert(offsetof(gg_problem_desc, beta) == offsetof(gg::ProblemDesc, beta), "ProblemDesc.beta");

struct gg_executor {
  gg::GroupedGemmExecutor executor;
};

struct gg_moe {
  gg::MoeGroupedGemm moe;
};

namespace {

gg::ProblemDesc to_cpp(const gg_problem_desc& p) {
  gg::ProblemDesc out{};
  out.m = p.m;
  out.n = p.n;
  out.k = p.k;
  out.a = static_cast<const __half*>(p.a);
  out.b = static_cast<const __half*>(p.b);
  out.c = p.c;
  out.d = p.d;
  out.lda = p.lda;
  out.ldb = p.ldb;
  out.ldc = p.ldc;
  out.ldd = p.ldd;
  out.alpha = p.alpha;
  out.beta = p.beta;
  return out;
}

gg_problem_desc to_c(const gg::ProblemDesc& p) {
  gg_problem_desc out{};
  out.m = p.m;
  out.n = p.n;
  out.k = p.k;
  out.a = p.a;
  out.b = p.b;
  out.c = p.c;
  out.d = p.d;
  out.lda = p.lda;
  out.ldb = p.ldb;
  out.ldc = p.ldc;
  out.ldd = p.ldd;
  out.alpha = p.alpha;
  out.beta = p.beta;
  return out;
}

gg::KernelConfig to_cpp(const gg_kernel_config& c) {
  gg::KernelConfig out;
  out.cta_m = c.cta_m;
  out.cta_n = c.cta_n;
  out.cta_k = c.cta_k;
  out.threads = c.threads;
  out.persistent_ctas = c.persistent_ctas;
  out.use_tensor_cores = c.use_tensor_cores != 0;
  return out;
}

std::vector<gg::ProblemDesc> to_cpp(const gg_problem_desc* problems, int count) {
  std::vector<gg::ProblemDesc> out;
  if (count > 0 && problems != nullptr) {
    out.reserve(count);
    for (int i = 0; i < count; ++i) out.push_back(to_cpp(problems[i]));
  }
  return out;
}

gg::MoeLayout to_cpp(const ggk_moe_layout& layout) {
  gg::MoeLayout L;
  L.experts = layout.experts;
  L.n = layout.n;
  L.k = layout.k;
  L.a = static_cast<const __half*>(layout.a);
  L.lda = layout.lda;
  L.b = static_cast<const __half*>(layout.b);
  L.ldb = layout.ldb;
  L.stride_b = layout.stride_b;
  L.c = layout.c;
  L.ldc = layout.ldc;
  L.d = layout.d;
  L.ldd = layout.ldd;
  L.alpha = layout.alpha;
  L.beta = layout.beta;
  L.max_rows = layout.max_rows;
  return L;
}

bool bad_list(const gg_problem_desc* problems, int count) {
  return count < 0 || (count > 0 && problems == nullptr);
}

}  // namespace

extern "C" {

const char* gg_version(void) { return "grouped_gemm_amd 0.1 gfx950"; }

const char* gg_sort_mode_name(int sort_mode) {
  return gg::sort_mode_name(static_cast<gg::SortMode>(sort_mode));
}

int gg_tile_count(const gg_problem_desc* problem, const gg_kernel_config* config) {
  if (problem == nullptr || config == nullptr) return 0;
  return gg::tile_count_for_problem(to_cpp(*problem), to_cpp(*config));
}

int gg_prepare_problem_set(const gg_problem_desc* problems, int count, const gg_kernel_config* config,
                           int sort_mode, gg_problem_desc* sorted_problems, int* sorted_to_original,
                           int* tile_offsets) {
  if (config == nullptr || bad_list(problems, count)) return -1;
  try {
    const gg::PreparedProblemSet prepared =
        gg::prepare_problem_set(to_cpp(problems, count), to_cpp(*config), static_cast<gg::SortMode>(sort_mode));
    for (int i = 0; i < count; ++i) {
      if (sorted_problems != nullptr) sorted_problems[i] = to_c(prepared.sorted_problems[i]);
      if (sorted_to_original != nullptr) sorted_to_original[i] = prepared.sorted_to_original[i];
    }
    if (tile_offsets != nullptr) {
      for (int i = 0; i <= count; ++i) tile_offsets[i] = prepared.tile_offsets[i];
    }
    return prepared.total_tiles;
  } catch (...) {
    return -1;
  }
}

int gg_query_occupancy(const gg_kernel_config* config, gg_occupancy_info* info) {
  if (config == nullptr || info == nullptr) return hipErrorInvalidValue;
  gg::OccupancyInfo o;
  const hipError_t status = gg::query_occupancy(to_cpp(*config), &o);
  if (status != hipSuccess) return status;
  info->sm_count = o.sm_count;
  info->max_blocks_per_sm = o.max_blocks_per_sm;
  info->active_blocks_per_sm = o.active_blocks_per_sm;
  info->threads_per_block = o.threads_per_block;
  info->max_threads_per_sm = o.max_threads_per_sm;
  info->warps_per_block = o.warps_per_block;
  info->max_warps_per_sm = o.max_warps_per_sm;
  info->active_warps_per_sm = o.active_warps_per_sm;
  info->max_registers_per_sm = o.max_registers_per_sm;
  info->max_registers_per_block = o.max_registers_per_block;
  info->estimated_registers_per_thread = o.estimated_registers_per_thread;
  info->estimated_registers_per_block = o.estimated_registers_per_block;
  info->registers_per_thread = o.registers_per_thread;
  info->registers_per_block = o.registers_per_block;
  info->register_limited_blocks_per_sm = o.register_limited_blocks_per_sm;
  info->static_shared_bytes = o.static_shared_bytes;
  info->dynamic_shared_bytes = o.dynamic_shared_bytes;
  info->theoretical_occupancy = o.theoretical_occupancy;
  info->using_tensor_cores = o.using_tensor_cores ? 1 : 0;
  info->vgprs_per_thread = o.vgprs_per_thread;
  info->agprs_per_thread = o.agprs_per_thread;
  info->sgprs_per_wave = o.sgprs_per_wave;
  info->scratch_bytes_per_thread = o.scratch_bytes_per_thread;
  info->lds_limited_blocks_per_sm = o.lds_limited_blocks_per_sm;
  info->wave_limited_blocks_per_sm = o.wave_limited_blocks_per_sm;
  return hipSuccess;
}

gg_executor* gg_executor_create(void) { return new (std::nothrow) gg_executor(); }

void gg_executor_destroy(gg_executor* executor) { delete executor; }

int gg_executor_build(gg_executor* executor, const gg_problem_desc* sorted_problems, int count,
                      const int* tile_offsets, int offsets_len, int total_tiles,
                      const gg_kernel_config* config) {
  if (executor == nullptr) return hipErrorInvalidDevicePointer;
  try {
    // Unusable arguments reach build() as an empty set or a rejected
    // configuration, so that the executor records the failure (run() then
    // refuses to launch) exactly as for any other rejected build.
    gg::KernelConfig cpp_config;
    cpp_config.threads = 0;
    if (config != nullptr) cpp_config = to_cpp(*config);
    gg::PreparedProblemSet prepared;
    if (!bad_list(sorted_problems, count) && offsets_len > 0 && tile_offsets != nullptr) {
      prepared.sorted_problems = to_cpp(sorted_problems, count);
      prepared.sorted_to_original.resize(count);
      for (int i = 0; i < count; ++i) prepared.sorted_to_original[i] = i;
      prepared.tile_offsets.assign(tile_offsets, tile_offsets + offsets_len);
      prepared.total_tiles = total_tiles;
    }
    const hipError_t status = executor->executor.build(prepared, cpp_config);
    if (status == hipSuccess && config == nullptr) return hipErrorInvalidValue;
    return status;
  } catch (...) {
    return hipErrorOutOfMemory;
  }
}

int gg_executor_run(const gg_executor* executor, hipStream_t stream) {
  if (executor == nullptr) return hipErrorInvalidDevicePointer;
  return executor->executor.run(stream);
}

int gg_executor_run_traced(const gg_executor* executor, int* d_tile_map, long long* d_wg_clock,
                           long long* d_tile_phases, hipStream_t stream) {
  if (executor == nullptr) return hipErrorInvalidDevicePointer;
  return executor->executor.run_traced(d_tile_map, d_wg_clock, stream, d_tile_phases);
}

int gg_executor_launched_work_tiles(const gg_executor* executor) {
  return executor != nullptr ? executor->executor.launched_work_tiles() : 0;
}

int gg_executor_problem_count(const gg_executor* executor) {
  return executor != nullptr ? executor->executor.problem_count() : 0;
}

int gg_executor_total_tiles(const gg_executor* executor) {
  return executor != nullptr ? executor->executor.total_tiles() : 0;
}

int gg_executor_grid_ctas(const gg_executor* executor) {
  return executor != nullptr ? executor->executor.grid_ctas() : 0;
}

int gg_executor_using_tensor_cores(const gg_executor* executor) {
  return executor != nullptr && executor->executor.using_tensor_cores() ? 1 : 0;
}

int gg_executor_schedule(const gg_executor* executor, ggk_work_shape* shape, int* order, int* work_offsets,
                         int* chunk_bounds) {
  if (executor == nullptr) return hipErrorInvalidDevicePointer;
  std::vector<int> o, w, b;
  const hipError_t status = executor->executor.schedule(shape, &o, &w, &b);
  if (status != hipSuccess) return status;
  if (order != nullptr) std::copy(o.begin(), o.end(), order);
  if (work_offsets != nullptr) std::copy(w.begin(), w.end(), work_offsets);
  if (chunk_bounds != nullptr) std::copy(b.begin(), b.end(), chunk_bounds);
  return hipSuccess;
}

int gg_run_grouped_gemm_once(const gg_problem_desc* problems, int count, int sort_mode,
                             const gg_kernel_config* config, hipStream_t stream) {
  if (config == nullptr || bad_list(problems, count)) return hipErrorInvalidValue;
  try {
    return gg::run_grouped_gemm_once(to_cpp(problems, count), static_cast<gg::SortMode>(sort_mode),
                                     to_cpp(*config), stream);
  } catch (...) {
    return hipErrorOutOfMemory;
  }
}

int gg_run_baseline_per_problem(const gg_problem_desc* problems, int count, const gg_kernel_config* config,
                                hipStream_t stream) {
  if (config == nullptr || bad_list(problems, count)) return hipErrorInvalidValue;
  try {
    return gg::run_baseline_per_problem(to_cpp(problems, count), to_cpp(*config), stream);
  } catch (...) {
    return hipErrorOutOfMemory;
  }
}

int gg_count_non_empty_problems(const gg_problem_desc* problems, int count, const gg_kernel_config* config) {
  if (config == nullptr || bad_list(problems, count)) return 0;
  return gg::count_non_empty_problems(to_cpp(problems, count), to_cpp(*config));
}

int gg_grid_ctas_for(const gg_kernel_config* config, int total_tiles) {
  if (config == nullptr) return -static_cast<int>(hipErrorInvalidValue);
  const gg::KernelConfig cfg = to_cpp(*config);
  gg::OccupancyInfo o;
  const hipError_t status = gg::query_occupancy(cfg, &o);
  if (status != hipSuccess) return -static_cast<int>(status);
  return gg::grid_ctas_for(total_tiles, cfg, o);
}

int gg_plan_launch(const gg_problem_desc* sorted_problems, int count, const gg_kernel_config* config,
                   int compute_units, const int* blocks_per_cu, gg_launch_plan* plan, int* order,
                   int* work_offsets, int* table, int table_capacity) {
  if (config == nullptr || plan == nullptr || blocks_per_cu == nullptr || bad_list(sorted_problems, count)) {
    return hipErrorInvalidValue;
  }
  *plan = gg_launch_plan{};
  try {
    const gg::KernelConfig cfg = to_cpp(*config);
    std::vector<gg::DeviceProblemDesc> problems;
    problems.reserve(count);
    for (int i = 0; i < count; ++i) problems.push_back(gg::to_device_problem(to_cpp(sorted_problems[i]), cfg));
    gg::LaunchPlan p;
    const hipError_t status = gg::plan_launch(
        problems, cfg, compute_units,
        [blocks_per_cu](int variant, int, int* blocks) {
          if (variant < 0 || variant >= GGK_VARIANT_COUNT) return hipErrorInvalidValue;
          *blocks = blocks_per_cu[variant];
          return hipSuccess;
        },
        &p);
    if (status != hipSuccess) return status;
    plan->variant = p.variant;
    plan->path = p.path;
    plan->addressing = p.addressing;
    plan->work = p.work;
    plan->total_work = p.total_work;
    plan->launch_total = p.launch_total;
    plan->table_ints = static_cast<int>(p.work_table.size());
    plan->grid = p.grid;
    plan->halves = p.halves ? 1 : 0;
    std::copy(p.chunk_bounds.begin(), p.chunk_bounds.end(), plan->chunk_bounds);
    std::copy(p.launch_bounds.begin(), p.launch_bounds.end(), plan->launch_bounds);
    if (order != nullptr) std::copy(p.order.begin(), p.order.end(), order);
    if (work_offsets != nullptr) std::copy(p.work_offsets.begin(), p.work_offsets.end(), work_offsets);
    if (table != nullptr) {
      if (table_capacity < plan->table_ints) return hipErrorInvalidValue;
      std::copy(p.work_table.begin(), p.work_table.end(), table);
    }
    return hipSuccess;
  } catch (...) {
    return hipErrorOutOfMemory;
  }
}

int gg_plan_shards(const gg_problem_desc* problems, int count, const gg_kernel_config* config, int ranks,
                   gg_shard_piece* pieces, int capacity) {
  if (config == nullptr || bad_list(problems, count) || (capacity > 0 && pieces == nullptr)) {
    return -static_cast<int>(hipErrorInvalidValue);
  }
  try {
    std::vector<gg::ShardPiece> out;
    const hipError_t status = gg::plan_shards(to_cpp(problems, count), to_cpp(*config), ranks, &out);
    if (status != hipSuccess) return -static_cast<int>(status);
    if (static_cast<int>(out.size()) > capacity) return -static_cast<int>(hipErrorInvalidValue);
    for (size_t i = 0; i < out.size(); ++i) {
      pieces[i] = gg_shard_piece{out[i].problem, out[i].rank, out[i].col0, out[i].cols};
    }
    return static_cast<int>(out.size());
  } catch (...) {
    return -static_cast<int>(hipErrorOutOfMemory);
  }
}

int gg_moe_create(const ggk_moe_layout* layout, const gg_kernel_config* config, int sort_mode, gg_moe** out) {
  if (out == nullptr) return hipErrorInvalidValue;
  *out = nullptr;
  if (layout == nullptr || config == nullptr) return hipErrorInvalidValue;
  gg_moe* m = new (std::nothrow) gg_moe;
  if (m == nullptr) return hipErrorOutOfMemory;
  const gg::MoeLayout L = to_cpp(*layout);
  const hipError_t status = m->moe.build(L, to_cpp(*config), static_cast<gg::SortMode>(sort_mode));
  if (status != hipSuccess) {
    delete m;
    return status;
  }
  *out = m;
  return hipSuccess;
}

int gg_moe_run(const gg_moe* moe, const int* d_counts, hipStream_t stream) {
  if (moe == nullptr) return hipErrorInvalidDevicePointer;
  return moe->moe.run(d_counts, stream);
}

int gg_moe_grid_ctas(const gg_moe* moe) { return moe != nullptr ? moe->moe.grid_ctas() : 0; }

int gg_moe_device_buffers(const gg_moe* moe, const gg_device_problem_desc** problems, const int** offsets,
                          const int** sorted_to_original, const int** header, const int** order) {
  if (moe == nullptr) return hipErrorInvalidDevicePointer;
  if (problems != nullptr) *problems = moe->moe.device_problems();
  if (offsets != nullptr) *offsets = moe->moe.device_offsets();
  if (sorted_to_original != nullptr) *sorted_to_original = moe->moe.device_sorted_to_original();
  if (header != nullptr) *header = moe->moe.device_header();
  if (order != nullptr) *order = moe->moe.device_order();
  return hipSuccess;
}

void gg_moe_destroy(gg_moe* moe) { delete moe; }

int gg_moe_run_noalloc(const ggk_moe_layout* layout, const gg_kernel_config* config, int sort_mode,
                       const int* d_counts, hipStream_t stream) {
  if (layout == nullptr || config == nullptr) return hipErrorInvalidValue;
  const gg::MoeLayout L = to_cpp(*layout);
  return gg::run_moe_grouped_gemm_noalloc(L, to_cpp(*config), static_cast<gg::SortMode>(sort_mode), d_counts, stream);
}

}  // extern "C"
