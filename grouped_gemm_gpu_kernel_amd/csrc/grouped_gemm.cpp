// grouped_gemm.cpp -- host runtime of the grouped FP16 GEMM (C++ API of
// include/grouped_gemm/grouped_gemm.h).
//
// Plain C++17: every GPU interaction goes through the thin kernel C-ABI
// (grouped_gemm_amd_kernels.h).  Reference counterparts: src/grouped_gemm.cu
// host section (:912-1331) and the variant/occupancy model (:47-217).
#include "grouped_gemm/grouped_gemm.h"

#include <algorithm>
#include <array>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <numeric>
#include <tuple>
#include <utility>

// The static scratch array of the allocation-free MoE entry point
// (gg_moe.hip, not exported): its address on the current device and its size.
extern "C" hipError_t gg_moe_scratch(void** ptr, size_t* bytes);

// 128 x 128 work tiles per CU at or below which a 128x64x32 / 64x128x32 set
// runs on the small-set variant.
#ifndef GG_SMALL_SET_TILES_PER_CU
#define GG_SMALL_SET_TILES_PER_CU 4
#endif

namespace grouped_gemm {
namespace {

constexpr int kThreadsPerBlock = 256;
constexpr int kWaveSize = 64;
// gfx950: 512 registers per lane per SIMD shared by VGPRs and AGPRs, allocated
// in blocks of 8; at most 8 waves per SIMD.
constexpr int kRegsPerLanePerSimd = 512;
constexpr int kRegAllocGranule = 8;
constexpr int kMaxWavesPerSimd = 8;
constexpr int kSimdsPerCu = 4;

// ceil(x / y) for x >= 0, y > 0, without forming x + y - 1 (which overflows near INT_MAX).
int ceil_div(int x, int y) { return x / y + (x % y != 0 ? 1 : 0); }

// a + b for non-negative ints, saturating at INT_MAX.
int add_saturating(int a, int b) { return a > INT_MAX - b ? INT_MAX : a + b; }

// The three accepted shapes (resolve_variant, src/grouped_gemm.cu:67-81).
int resolve_variant(const KernelConfig& config) {
  if (config.threads != kThreadsPerBlock) return -1;
  if (config.cta_m == 64 && config.cta_n == 64 && config.cta_k == 16) return GGK_VARIANT_64x64x16;
  if (config.cta_m == 128 && config.cta_n == 64 && config.cta_k == 32) return GGK_VARIANT_128x64x32;
  if (config.cta_m == 64 && config.cta_n == 128 && config.cta_k == 32) return GGK_VARIANT_64x128x32;
  return -1;
}

struct RuntimeMode {
  int variant = -1;
  int path = GGK_PATH_FMA;
  ggk_device_info device{};
  ggk_work_shape work{};
};

// Per-process cache of what does not change while a process runs: each
// device's properties and, per (device, variant, path), the kernel's
// occupancy report.  The reference queries the device properties on every
// build and occupancy query (src/grouped_gemm.cu:1141, 1222, 1032); here the
// first call on a device pays for them.
constexpr int kCachedDevices = 64;
struct DeviceCache {
  bool ready = false;
  ggk_device_info info{};
  bool occupancy_ready[GGK_VARIANT_COUNT][GGK_PATH_COUNT] = {};
  OccupancyInfo occupancy[GGK_VARIANT_COUNT][GGK_PATH_COUNT];
};
std::mutex g_cache_mutex;
DeviceCache g_device_cache[kCachedDevices];

// The current device's cache entry (nullptr past kCachedDevices devices),
// with its properties filled in.  Call with g_cache_mutex held.
hipError_t device_cache(DeviceCache** out, ggk_device_info* info) {
  *out = nullptr;
  int device = 0;
  hipError_t status = ggk_current_device(&device);
  if (status != hipSuccess) return status;
  if (device < 0 || device >= kCachedDevices) return ggk_device_info_get(info);
  DeviceCache& c = g_device_cache[device];
  if (!c.ready) {
    status = ggk_device_info_get(&c.info);
    if (status != hipSuccess) return status;
    c.ready = true;
  }
  *info = c.info;
  *out = &c;
  return hipSuccess;
}

// resolve_runtime_mode (src/grouped_gemm.cu:111-143): unsupported shapes are
// InvalidValue; the MFMA path is used when requested.  The library is built
// for gfx950 only, where every accepted shape has an MFMA kernel.
hipError_t resolve_runtime_mode(const KernelConfig& config, RuntimeMode* mode) {
  const int variant = resolve_variant(config);
  if (variant < 0) return hipErrorInvalidValue;
  DeviceCache* cache = nullptr;
  hipError_t status;
  {
    std::lock_guard<std::mutex> lock(g_cache_mutex);
    status = device_cache(&cache, &mode->device);
  }
  if (status != hipSuccess) return status;
  mode->variant = variant;
  mode->path = config.use_tensor_cores ? GGK_PATH_MFMA : GGK_PATH_FMA;
  return ggk_work_shape_get(mode->variant, mode->path, &mode->work);
}

// Formula estimate of registers per lane (the role of
// estimated_*_registers_per_thread, src/grouped_gemm.cu:175-217), for this
// build's kernels.  Work tile BM x BN (a block of tiles_m x tiles_n
// macro-tiles), stage depth 64, T threads; a staged global piece holds 5
// registers plus 2 of offsets.  MFMA: BM*BN/T float accumulators, two A and
// two B operand fragments of 4 registers, staging, ~24 for addresses and loop
// state.  FMA: RM*RN accumulators, RM 16-byte A slices, RN B values, staging, ~24.
int estimated_registers_per_thread(const KernelConfig& config, const ggk_work_shape& work, bool mfma) {
  const int bm = config.cta_m * work.tiles_m;
  const int bn = config.cta_n * work.tiles_n;
  const int bk = 64;
  const int threads = work.threads > 0 ? work.threads : kThreadsPerBlock;
  const int pieces = (bm * bk / 8 + bk * bn / 8) / threads;
  const int staging = pieces * 7;
  if (mfma) {
    const int acc = bm * bn / threads;
    return acc + 16 + staging + 24;
  }
  const int rm = bm / 16;
  const int rn = bn / 16;
  return rm * rn + rm * 4 + rn + staging + 24;
}

int round_up(int x, int granule) { return (x + granule - 1) / granule * granule; }

hipError_t fill_occupancy(const KernelConfig& config, const RuntimeMode& mode, OccupancyInfo* info) {
  const ggk_device_info& dev = mode.device;
  const bool mfma = mode.path == GGK_PATH_MFMA;
  const int wave = dev.wave_size > 0 ? dev.wave_size : kWaveSize;
  const int threads = mode.work.threads > 0 ? mode.work.threads : kThreadsPerBlock;
  *info = OccupancyInfo{};
  info->sm_count = dev.compute_units;
  info->max_blocks_per_sm = dev.max_wgs_per_cu;
  info->threads_per_block = threads;
  info->max_threads_per_sm = dev.max_threads_per_cu;
  info->warps_per_block = threads / wave;
  info->max_warps_per_sm = dev.max_threads_per_cu / wave;
  info->max_registers_per_sm = dev.regs_per_cu;
  info->max_registers_per_block = dev.regs_per_block;
  info->estimated_registers_per_thread = estimated_registers_per_thread(config, mode.work, mfma);
  info->estimated_registers_per_block = info->estimated_registers_per_thread * threads;
  info->using_tensor_cores = mfma;

  ggk_kernel_resources res{};
  hipError_t status = ggk_kernel_resources_get(GGK_KERNEL_GROUPED, mode.variant, mode.path, &res);
  if (status != hipSuccess) return status;
  status = ggk_occupancy(mode.variant, mode.path, &info->active_blocks_per_sm);
  if (status != hipSuccess) return status;

  info->vgprs_per_thread = res.vgprs;
  info->agprs_per_thread = res.agprs;
  info->sgprs_per_wave = res.sgprs;
  info->scratch_bytes_per_thread = res.scratch_bytes_per_lane;
  // VGPRs and AGPRs come from one register file; when the compiler report is
  // unavailable, fall back to what hipFuncGetAttributes reports.
  const int regs = (res.vgprs + res.agprs) > 0 ? res.vgprs + res.agprs : res.num_regs;
  info->registers_per_thread = regs;
  info->registers_per_block = regs * threads;
  info->static_shared_bytes = res.lds_static > 0 ? res.lds_static : res.lds_bytes;
  info->dynamic_shared_bytes = res.lds_dynamic;

  // A workgroup's waves are spread evenly over the 4 SIMDs of a CU, so
  // resident workgroups per CU are limited by waves per SIMD (registers), by
  // LDS and by the wave slots.
  const int waves_per_simd =
      regs > 0 ? std::min(kMaxWavesPerSimd, kRegsPerLanePerSimd / round_up(regs, kRegAllocGranule))
               : kMaxWavesPerSimd;
  const int block_waves_per_simd = std::max(1, ceil_div(info->warps_per_block, kSimdsPerCu));
  info->register_limited_blocks_per_sm = waves_per_simd / block_waves_per_simd;
  const int lds_per_block = info->static_shared_bytes + info->dynamic_shared_bytes;
  info->lds_limited_blocks_per_sm =
      lds_per_block > 0 ? dev.lds_per_cu / lds_per_block : info->max_blocks_per_sm;
  info->wave_limited_blocks_per_sm =
      info->warps_per_block > 0 ? info->max_warps_per_sm / info->warps_per_block : 0;

  info->active_warps_per_sm = info->active_blocks_per_sm * info->warps_per_block;
  if (info->max_warps_per_sm > 0) {
    info->theoretical_occupancy =
        static_cast<float>(info->active_warps_per_sm) / static_cast<float>(info->max_warps_per_sm);
  }
  return hipSuccess;
}

// fill_occupancy through the per-process cache: the report depends only on
// the device and the kernel (the variant fixes the macro-tile).
hipError_t cached_occupancy(const KernelConfig& config, const RuntimeMode& mode, OccupancyInfo* info) {
  std::lock_guard<std::mutex> lock(g_cache_mutex);
  DeviceCache* cache = nullptr;
  ggk_device_info dev{};
  hipError_t status = device_cache(&cache, &dev);
  if (status != hipSuccess) return status;
  if (cache == nullptr) return fill_occupancy(config, mode, info);
  if (!cache->occupancy_ready[mode.variant][mode.path]) {
    status = fill_occupancy(config, mode, &cache->occupancy[mode.variant][mode.path]);
    if (status != hipSuccess) return status;
    cache->occupancy_ready[mode.variant][mode.path] = true;
  }
  *info = cache->occupancy[mode.variant][mode.path];
  return hipSuccess;
}

// The order in which the grouped kernel meets the problems' work tiles, and
// its split into GGK_SCHEDULER_CHUNKS contiguous chunks, one per XCD.
struct Schedule {
  std::vector<int> order;         // problem (sorted index) at each position
  std::vector<int> work_offsets;  // prefix sums of the work-tile counts in that order
  std::vector<double> tile_time;  // estimated time of one work tile of the problem at each position
  std::array<int, GGK_SCHEDULER_CHUNKS + 1> bounds{};
};

// Estimated time of all work tiles of problem p, in hundredths of a cycle of
// one CU.  Per work tile: a fixed part (finding the tile, the first stage's
// latency, the claim), a k-loop whose stages cost mostly their latency plus a
// little per row and column they move, and an epilogue that moves rows x cols
// floats (twice when C is read):
//   150 + stages * (31 + 0.029 (rows + cols)) + 0.0023 rows cols  (x 100)
// The constants are a least-squares fit to per-tile clock stamps of the
// grouped kernel on mixed shapes (median error 7%); only the ratios between
// problems matter.  Summed over the tm x tn work tiles, the rows add up to
// m tn, the columns to n tm and the areas to m n, so the total is a sum of
// integer products, evaluated in double one operation at a time: the
// device-side prepare (gg_moe.hip) evaluates the same expression in the same
// order and gets the same value, hence the same schedule.
double problem_work_time(int m, int n, int k, int tm, int tn, int bk, bool reads_c) {
  if (m <= 0 || n <= 0 || tm <= 0 || tn <= 0) return 0.0;
  const double w = static_cast<double>(tm) * tn;
  const double stages = k > 0 ? (k - 1) / bk + 1 : 0;
  const double edge = static_cast<double>(m) * tn + static_cast<double>(n) * tm;
  const double stage = 310000.0 * w + 290.0 * edge;
  const double area = static_cast<double>(m) * n;
  return 1500000.0 * w + stages * stage + (reads_c ? 46.0 : 23.0) * area;
}

// A problem's estimated time as the integer the schedule ranks and adds up:
// clamped to 2^52 (below 2^53 the double is an exact integer already), so
// that up to 2^11 of them sum exactly in 64 bits; the chunk loads saturate
// beyond that.
int64_t problem_time_units(double t) { return t < 4503599627370496.0 ? static_cast<int64_t>(t) : (int64_t{1} << 52); }

// Longest processing time first at two levels, after spreading oversized
// problems.  A problem whose estimated time exceeds one chunk's share (the
// total over the chunks, rounded up) would overload whichever chunk took it
// whole: the other XCDs would then take its tiles one claim at a time,
// interleaved, and each XCD's L2 would hold scattered panels of it.  Such
// problems run first instead, back to back, largest first, and the chunk
// boundaries cut that run into consecutive pieces of one share each (at the
// work tile nearest to where the run's estimated time reaches c shares), so
// that each XCD multiplies a contiguous block of their tiles.  The other
// problems go whole to the chunk with the least estimated work so far (the
// chunk that holds the end of the run starts with its remainder), largest
// first (a problem's tiles share A and B panels, which that XCD's L2 then
// serves); within a chunk the tiles with the longest estimated time come
// first, after the run's remainder (which stays contiguous with its earlier
// pieces), so the last tiles any workgroup starts are short ones.  Without
// oversized problems this is the two-level LPT alone.  Every order yields the
// same D: each work tile is computed the same way wherever it runs.
Schedule plan_schedule(const std::vector<DeviceProblemDesc>& problems, const std::vector<int>& work, int bm, int bn,
                       int bk) {
  constexpr int kChunks = GGK_SCHEDULER_CHUNKS;
  const int count = static_cast<int>(problems.size());
  std::vector<double> tile_time(count);
  std::vector<int64_t> total(count);
  int64_t sum = 0;  // saturating
  for (int i = 0; i < count; ++i) {
    const DeviceProblemDesc& p = problems[i];
    const bool reads_c = p.c != nullptr && p.beta != 0.0f;
    const int tm = p.m > 0 ? (p.m - 1) / bm + 1 : 0;  // work tiles along M and N
    const int tn = p.n > 0 ? (p.n - 1) / bn + 1 : 0;
    const double t = work[i] > 0 ? problem_work_time(p.m, p.n, p.k, tm, tn, bk, reads_c) : 0.0;
    total[i] = problem_time_units(t);
    tile_time[i] = work[i] > 0 ? t / work[i] : 0.0;
    sum = sum > INT64_MAX - total[i] ? INT64_MAX : sum + total[i];
  }
  const int64_t share = sum / kChunks + (sum % kChunks != 0 ? 1 : 0);
  std::vector<int> by_total(count);
  for (int i = 0; i < count; ++i) by_total[i] = i;
  std::stable_sort(by_total.begin(), by_total.end(), [&](int x, int y) { return total[x] > total[y]; });
  int oversized = 0;  // they lead by_total
  while (oversized < count && total[by_total[oversized]] > share) ++oversized;
  if (oversized > 0) {
    // Placed whole, the oversized problems leave other chunks short of a
    // share, and those XCDs take the difference from the overloaded chunks by
    // stealing.  Stealing a little is cheap (and balances at run time what
    // the estimate misjudged); the run is cut only when whole placement would
    // leave more than a quarter of the work to it.
    std::array<int64_t, kChunks> whole{};
    for (const int i : by_total) {
      int c = 0;
      for (int d = 1; d < kChunks; ++d) {
        if (whole[d] < whole[c]) c = d;
      }
      whole[c] = whole[c] > INT64_MAX - total[i] ? INT64_MAX : whole[c] + total[i];
    }
    double stolen = 0.0;
    for (const int64_t l : whole) stolen += l < share ? static_cast<double>(share - l) : 0.0;
    if (stolen * 4.0 <= static_cast<double>(sum)) oversized = 0;
  }

  Schedule s;
  s.order.reserve(count);
  s.tile_time.reserve(count);
  s.work_offsets.assign(1, 0);
  s.work_offsets.reserve(count + 1);
  s.bounds[0] = 0;
  auto place = [&](int i) {
    s.order.push_back(i);
    s.work_offsets.push_back(s.work_offsets.back() + work[i]);
    s.tile_time.push_back(tile_time[i]);
  };
  std::array<int64_t, kChunks> load{};
  int first = 0;  // the first chunk open to the LPT pass
  if (oversized > 0) {
    // share < 2^52 here (a total above it is clamped to 2^52), so c * share
    // and the run's time stay far from overflow.
    int64_t run_time = 0;  // estimated time of the run before problem i
    int c = 1;             // the next chunk boundary to place
    for (int r = 0; r < oversized; ++r) {
      const int i = by_total[r];
      for (; c < kChunks && c * share < run_time + total[i]; ++c) {
        const double x = static_cast<double>(c * share - run_time) / static_cast<double>(total[i]) * work[i];
        const int j = static_cast<int>(std::floor(x + 0.5));
        s.bounds[c] = s.work_offsets.back() + std::min(std::max(j, 0), work[i]);
      }
      place(i);
      run_time += total[i];
    }
    first = c - 1;
    load[first] = run_time - first * share;
  }
  std::array<std::vector<int>, kChunks> members;
  for (int r = oversized; r < count; ++r) {
    const int i = by_total[r];
    int c = first;
    for (int d = first + 1; d < kChunks; ++d) {
      if (load[d] < load[c]) c = d;
    }
    load[c] = load[c] > INT64_MAX - total[i] ? INT64_MAX : load[c] + total[i];
    members[c].push_back(i);
  }
  for (int c = first; c < kChunks; ++c) {
    std::vector<int>& m = members[c];
    std::stable_sort(m.begin(), m.end(), [&](int x, int y) {
      return tile_time[x] != tile_time[y] ? tile_time[x] > tile_time[y] : x < y;
    });
    for (const int i : m) place(i);
    s.bounds[c + 1] = s.work_offsets.back();
  }
  return s;
}

// One device allocation per executor: descriptors, then ints, then the
// scheduler state, each part starting on a 256-byte boundary (the state's
// counters then sit on 128-byte lines of their own).  Launches read it until
// they end, so it is rewritten or freed only after the last launch's event
// (recorded on that launch's stream) has completed.  A launch captured into a
// graph records no event, and the graph may be replayed on any stream at any
// later time: once a launch was captured, every wait is for the whole device
// instead, until the allocation is released (the device must then not be
// capturing).
struct DeviceBuffer {
  void* base = nullptr;
  size_t capacity = 0;  // bytes
  int device = -1;
  hipEvent_t last_launch = nullptr;
  bool launched = false;  // an event was recorded since the last wait
  bool captured = false;  // a launch was captured since the allocation was made

  static size_t round256(size_t x) { return (x + 255) / 256 * 256; }

  hipError_t wait_launches() {
    if (captured) {
      // Replays of the captured launch may be running on any stream; a
      // device-wide wait also covers the recorded event.
      launched = false;
      return ggk_device_synchronize();
    }
    if (!launched) return hipSuccess;
    launched = false;
    return ggk_event_synchronize(last_launch);
  }

  // Records the event after a launch on `stream`, or notes that the launch
  // was captured.
  hipError_t note_launch(hipStream_t stream) {
    if (last_launch == nullptr) return hipSuccess;
    int recorded = 0;
    const hipError_t status = ggk_event_record_launch(last_launch, stream, &recorded);
    if (recorded == GGK_LAUNCH_RECORDED) launched = true;
    if (recorded == GGK_LAUNCH_CAPTURED) captured = true;
    return status;
  }

  // At least `bytes` on the current device, reusing the allocation when it is
  // large enough; waits for earlier launches either way.
  hipError_t reserve(size_t bytes) {
    hipError_t status = wait_launches();
    if (status != hipSuccess) return status;
    int current = 0;
    status = ggk_current_device(&current);
    if (status != hipSuccess) return status;
    if (last_launch == nullptr || current != device) {
      release();
      status = ggk_event_create(&last_launch);
      if (status != hipSuccess) return status;
      device = current;
    }
    if (base != nullptr && capacity >= bytes) return hipSuccess;
    (void)ggk_free(base);
    base = nullptr;
    capacity = 0;
    status = ggk_alloc(&base, bytes);
    if (status != hipSuccess) {
      base = nullptr;
      return status;
    }
    capacity = bytes;
    return hipSuccess;
  }

  // Teardown: a failure here has nobody to report to.
  void release() {
    (void)wait_launches();
    (void)ggk_free(base);
    (void)ggk_event_destroy(last_launch);
    base = nullptr;
    capacity = 0;
    device = -1;
    last_launch = nullptr;
    launched = false;
    captured = false;
  }
};

}  // namespace

// Grid size (src/grouped_gemm.cu:1228-1236): the requested persistent size,
// else every resident workgroup slot but no more than max(total_tiles, CUs).
int grid_ctas_for(int total_tiles, const KernelConfig& config, const OccupancyInfo& occupancy) {
  if (total_tiles <= 0) return 0;
  int grid;
  if (config.persistent_ctas > 0) {
    grid = config.persistent_ctas;
  } else {
    const int resident = occupancy.sm_count * std::max(1, occupancy.active_blocks_per_sm);
    grid = std::min(resident, std::max(total_tiles, occupancy.sm_count));
  }
  return std::max(1, grid);
}

// Clamped at INT_MAX: a problem (or set) of more tiles than an int holds gets tile offsets that do
// not match its tile count, which build() rejects.
int tile_count_for_problem(const ProblemDesc& problem, const KernelConfig& config) {
  if (problem.m <= 0 || problem.n <= 0 || config.cta_m <= 0 || config.cta_n <= 0) return 0;
  const int64_t tiles = static_cast<int64_t>(ceil_div(problem.m, config.cta_m)) * ceil_div(problem.n, config.cta_n);
  return tiles > INT_MAX ? INT_MAX : static_cast<int>(tiles);
}

DeviceProblemDesc to_device_problem(const ProblemDesc& p, const KernelConfig& config) {
  DeviceProblemDesc out{};
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
  const bool empty = p.m <= 0 || p.n <= 0 || config.cta_m <= 0 || config.cta_n <= 0;
  out.tiles_m = empty ? 0 : ceil_div(p.m, config.cta_m);
  out.tiles_n = empty ? 0 : ceil_div(p.n, config.cta_n);
  return out;
}

const char* sort_mode_name(SortMode sort_mode) {
  switch (sort_mode) {
    case SortMode::kNone:
      return "none";
    case SortMode::kByK:
      return "sort_by_k";
    case SortMode::kByTiles:
      return "sort_by_tiles";
    case SortMode::kByTilesThenK:
      return "sort_by_tiles_then_k";
  }
  return "unknown";
}

// prepare_problem_set (src/grouped_gemm.cu:967-1022).  The permutation must
// equal the reference's std::stable_sort bit for bit, so the orderings are the
// reference's: by K = larger k first, ties by larger int64 m*n; by tiles = more
// tiles first, ties by the by-K order.  kByTilesThenK orders exactly like
// kByTiles, as in the reference (:1000-1005).  Ties keep input order.
PreparedProblemSet prepare_problem_set(const std::vector<ProblemDesc>& problems,
                                       const KernelConfig& config, SortMode sort_mode) {
  const int count = static_cast<int>(problems.size());
  struct Key {
    int tiles;
    int k;
    int64_t area;
  };
  std::vector<Key> keys(count);
  for (int i = 0; i < count; ++i) {
    keys[i] = Key{tile_count_for_problem(problems[i], config), problems[i].k,
                  static_cast<int64_t>(problems[i].m) * problems[i].n};
  }

  PreparedProblemSet prepared;
  prepared.sorted_to_original.resize(count);
  std::iota(prepared.sorted_to_original.begin(), prepared.sorted_to_original.end(), 0);
  const bool tiles_first = sort_mode == SortMode::kByTiles || sort_mode == SortMode::kByTilesThenK;
  if (sort_mode == SortMode::kByK || tiles_first) {
    // Descending lexicographic order on (tiles if tiles_first, k, area).
    std::stable_sort(prepared.sorted_to_original.begin(), prepared.sorted_to_original.end(),
                     [&keys, tiles_first](int lhs, int rhs) {
                       const Key& l = keys[lhs];
                       const Key& r = keys[rhs];
                       if (tiles_first && l.tiles != r.tiles) return l.tiles > r.tiles;
                       return std::tie(l.k, l.area) > std::tie(r.k, r.area);
                     });
  }

  prepared.sorted_problems.reserve(count);
  prepared.tile_offsets.assign(1, 0);
  prepared.tile_offsets.reserve(count + 1);
  for (int idx : prepared.sorted_to_original) {
    prepared.sorted_problems.push_back(problems[idx]);
    prepared.tile_offsets.push_back(add_saturating(prepared.tile_offsets.back(), keys[idx].tiles));
  }
  prepared.total_tiles = prepared.tile_offsets.back();
  return prepared;
}

hipError_t query_occupancy(const KernelConfig& config, OccupancyInfo* info) {
  if (info == nullptr) return hipErrorInvalidValue;
  RuntimeMode mode;
  const hipError_t status = resolve_runtime_mode(config, &mode);
  if (status != hipSuccess) return status;
  return cached_occupancy(config, mode, info);
}

struct GroupedGemmExecutor::Impl {
  DeviceBuffer buffer;
  DeviceProblemDesc* d_problems = nullptr;
  // [problem_count + 1] reference tile offsets, then [problem_count + 1]
  // work-tile offsets in scheduling order, then [problem_count] the
  // scheduling order, then (if work_table) [2 * launch_total] the work table.
  int* d_ints = nullptr;
  int* d_state = nullptr;

  int problem_count = 0;
  int total_tiles = 0;
  int total_work = 0;
  int grid_ctas = 0;
  bool failed = false;  // the last build() returned an error

  KernelConfig config{};
  int variant = -1;
  int path = GGK_PATH_FMA;
  int addressing = GGK_ADDR_32;
  std::array<int, GGK_SCHEDULER_CHUNKS + 1> chunk_bounds{};
  bool work_table = false;
  // What a launch claims: work-table entries (a work tile split into its two
  // halves counts twice) and the chunk bounds over them; without a table,
  // total_work and chunk_bounds.
  int launch_total = 0;
  std::array<int, GGK_SCHEDULER_CHUNKS + 1> launch_bounds{};

  const int* d_work_table() const {
    return work_table ? d_ints + 3 * static_cast<size_t>(problem_count) + 2 : nullptr;
  }

  // Forgets the last build (the buffer is kept for the next one).
  void reset() {
    d_problems = nullptr;
    d_ints = nullptr;
    d_state = nullptr;
    problem_count = total_tiles = total_work = grid_ctas = 0;
    variant = -1;
    path = GGK_PATH_FMA;
    addressing = GGK_ADDR_32;
    chunk_bounds = {};
    work_table = false;
    launch_total = 0;
    launch_bounds = {};
  }
};

namespace {

// Work tables up to this many work tiles (8 bytes each) are uploaded; larger
// sets are searched.
constexpr int kWorkTableMax = 1 << 22;

// Work tiles among the last of each chunk that the work table lists as two
// halves (rows), for kernels that read such entries, in sets of at most
// kTailHalvesMaxPerSlot work tiles per workgroup slot.  The workgroups of a
// chunk run dry one by one, each after its last tile; the tiles still running
// then decide when the launch ends, so halving the last ones (the shortest
// of the chunk already) cuts the time the others wait.  A half costs more
// than half a tile (it stages all of the tile's B), so sets whose launch is
// long against one tile keep whole tiles: there the tail is a small share.
#ifndef GG_TAIL_HALVES
#define GG_TAIL_HALVES 64
#endif
constexpr int kTailHalves = GG_TAIL_HALVES;
constexpr int kTailHalvesMaxPerSlot = 12;

// Idle share of the planned schedule below which no tile is halved.
constexpr double kTailHalvesMinIdle = 0.02;

// The share of workgroup time the planned schedule leaves idle at its end, by
// the tile-time estimate: each chunk's work tiles, in claim order, go to
// whichever of the chunk's workgroups is free first (as its counter hands them
// out), and the idle share is the time workgroups spend finished while the
// last one still runs, over grid x the longest chunk.  Halving tail tiles only
// shortens an end that is ragged: a set of equal tiles that keep every
// workgroup busy to the same end (one 8192^3 problem: 128 tiles per chunk, 4
// per workgroup) would only pay the halves' extra B loads (8% measured).
double planned_idle_share(const Schedule& s, int grid) {
  constexpr int kChunks = GGK_SCHEDULER_CHUNKS;
  double busy = 0.0, longest = 0.0;
  int slots_total = 0;
  size_t pos = 0;  // the position holding work-tile index t
  std::vector<double> ends;
  for (int c = 0; c < kChunks; ++c) {
    const int slots = c < grid ? (grid - 1 - c) / kChunks + 1 : 0;  // workgroups whose home is chunk c
    ends.assign(static_cast<size_t>(slots), 0.0);                     // a min-heap of finishing times
    for (int t = s.bounds[c]; t < s.bounds[c + 1] && slots > 0; ++t) {
      while (s.work_offsets[pos + 1] <= t) ++pos;
      std::pop_heap(ends.begin(), ends.end(), std::greater<double>());
      ends.back() += s.tile_time[pos];
      std::push_heap(ends.begin(), ends.end(), std::greater<double>());
      busy += s.tile_time[pos];
    }
    for (const double e : ends) longest = std::max(longest, e);
    slots_total += slots;
  }
  return longest > 0.0 && slots_total > 0 ? 1.0 - busy / (slots_total * longest) : 0.0;
}

// Row of work tiles of work tile `local` in a problem with wtm x wtn of them,
// in the grouped kernel's order (groups of 4 rows, column by column within a
// group; gg_kernels.hip, work_tile_position).
int work_tile_row(int local, int wtm, int wtn) {
  constexpr int kGroupRows = 4;
  const int group = local / (kGroupRows * wtn);
  const int first = group * kGroupRows;
  const int rows = std::min(kGroupRows, wtm - first);
  const int within = local - group * kGroupRows * wtn;
  return first + within % rows;
}

}  // namespace

hipError_t plan_launch(const std::vector<DeviceProblemDesc>& problems, const KernelConfig& config,
                       int compute_units, const BlocksPerCu& blocks_per_cu, LaunchPlan* plan) {
  if (plan == nullptr) return hipErrorInvalidValue;
  *plan = LaunchPlan{};
  const int base_variant = resolve_variant(config);
  if (base_variant < 0 || compute_units < 1 || !blocks_per_cu) return hipErrorInvalidValue;
  const int count = static_cast<int>(problems.size());
  int64_t tiles = 0;  // the set's macro-tiles: the work-tile counts below stay under it
  for (const DeviceProblemDesc& p : problems) {
    if (p.m < 0 || p.n < 0 || p.k < 0) return hipErrorInvalidValue;
    const bool live = p.m > 0 && p.n > 0;
    if (p.tiles_m != (live ? ceil_div(p.m, config.cta_m) : 0) || p.tiles_n != (live ? ceil_div(p.n, config.cta_n) : 0)) {
      return hipErrorInvalidValue;
    }
    tiles += static_cast<int64_t>(p.tiles_m) * p.tiles_n;
    if (tiles > INT_MAX) return hipErrorInvalidValue;
  }
  int variant = base_variant;
  const int path = config.use_tensor_cores ? GGK_PATH_MFMA : GGK_PATH_FMA;
  ggk_work_shape shape{};
  hipError_t status = ggk_work_shape_get(variant, path, &shape);
  if (status != hipSuccess) return status;

  // A launch with few work tiles is bound by the latency of each tile's
  // stages rather than by bandwidth: when the 128 x 128 work tiles of the
  // small-set variants number at most two per workgroup slot (two
  // workgroups per CU), the set runs on those instead of the 256 x 256 ones.
  // The reference tile map is the same either way.
  const int small_variant = ggk_small_variant(variant);
  if (path == GGK_PATH_MFMA && small_variant >= 0) {
    ggk_work_shape small{};
    status = ggk_work_shape_get(small_variant, path, &small);
    if (status != hipSuccess) return status;
    int64_t work = 0;
    for (const DeviceProblemDesc& p : problems) {
      work += static_cast<int64_t>(ceil_div(p.tiles_m, small.tiles_m)) * ceil_div(p.tiles_n, small.tiles_n);
    }
    if (work <= GG_SMALL_SET_TILES_PER_CU * static_cast<int64_t>(compute_units)) {
      variant = small_variant;
      shape = small;
    }
  }
  auto addressing_for = [&](int v) {
    for (const DeviceProblemDesc& p : problems) {
      if (ggk_needs_addr64(v, path, &p) == 1) return GGK_ADDR_64;
    }
    return GGK_ADDR_32;
  };
  int addressing = addressing_for(variant);
  // The 64-bit form of the 256 x 256 work tile spills registers: a set that
  // needs it runs on 128 x 128 work tiles of the same macro-tile (same D).
  if (addressing == GGK_ADDR_64 && path == GGK_PATH_MFMA && ggk_small_variant(variant) >= 0) {
    variant = ggk_small_variant(variant);
    status = ggk_work_shape_get(variant, path, &shape);
    if (status != hipSuccess) return status;
    addressing = addressing_for(variant);
  }

  std::vector<int> work(count);
  for (int i = 0; i < count; ++i) {
    // Never above the problem's tile count, so the sums fit an int.
    work[i] = ceil_div(problems[i].tiles_m, shape.tiles_m) * ceil_div(problems[i].tiles_n, shape.tiles_n);
  }
  const int bm = config.cta_m * shape.tiles_m;
  Schedule schedule = plan_schedule(problems, work, bm, config.cta_n * shape.tiles_n, shape.stage_k);
  const int total_work = schedule.work_offsets.back();
  const bool work_table = total_work > 0 && total_work <= kWorkTableMax;

  int blocks = 0;
  status = blocks_per_cu(variant, path, &blocks);
  if (status != hipSuccess) return status;
  OccupancyInfo occupancy{};
  occupancy.sm_count = compute_units;
  occupancy.active_blocks_per_sm = blocks;
  // The persistent grid is sized by the units it claims: work tiles.
  const int grid = grid_ctas_for(total_work, config, occupancy);

  // The work table in claim order: (problem, work tile within it) of every
  // work-tile index, so that the kernel reads it with one load instead of
  // searching.  Within the last kTailHalves entries of each chunk, a work tile
  // with more than half its rows inside the problem is listed as its two
  // halves, consecutively.
  std::vector<int> table;
  std::array<int, GGK_SCHEDULER_CHUNKS + 1> launch_bounds = schedule.bounds;
  bool halves = false;
  if (work_table) {
    halves = kTailHalves > 0 && ggk_work_halves_supported(variant, path) == 1 &&
             total_work <= kTailHalvesMaxPerSlot * grid && planned_idle_share(schedule, grid) >= kTailHalvesMinIdle;
    table.reserve(2 * static_cast<size_t>(total_work) + 4 * GGK_SCHEDULER_CHUNKS * std::max(kTailHalves, 0));
    int index = 0;  // work-tile index of the entry being listed
    int chunk = 0;
    launch_bounds[0] = 0;
    for (const int prob : schedule.order) {
      const DeviceProblemDesc& dp = problems[prob];
      const int wtm = ceil_div(dp.tiles_m, shape.tiles_m);
      const int wtn = ceil_div(dp.tiles_n, shape.tiles_n);
      for (int w = 0; w < work[prob]; ++w, ++index) {
        while (chunk < GGK_SCHEDULER_CHUNKS && index >= schedule.bounds[chunk + 1]) {
          launch_bounds[++chunk] = static_cast<int>(table.size() / 2);
        }
        const bool tail = halves && index >= schedule.bounds[chunk + 1] - kTailHalves;
        if (tail && dp.m - work_tile_row(w, wtm, wtn) * bm > bm / 2) {
          table.insert(table.end(), {prob, w | (1 << GGK_WORK_HALF_SHIFT), prob, w | (2 << GGK_WORK_HALF_SHIFT)});
        } else {
          table.insert(table.end(), {prob, w});
        }
      }
    }
    while (chunk < GGK_SCHEDULER_CHUNKS) launch_bounds[++chunk] = static_cast<int>(table.size() / 2);
  }

  plan->variant = variant;
  plan->path = path;
  plan->addressing = addressing;
  plan->work = shape;
  plan->order = std::move(schedule.order);
  plan->work_offsets = std::move(schedule.work_offsets);
  plan->chunk_bounds = schedule.bounds;
  plan->launch_total = work_table ? static_cast<int>(table.size() / 2) : total_work;
  plan->work_table = std::move(table);
  plan->launch_bounds = launch_bounds;
  plan->total_work = total_work;
  plan->grid = grid;
  plan->halves = halves;
  return hipSuccess;
}

GroupedGemmExecutor::GroupedGemmExecutor() : impl_(new Impl()) {}

GroupedGemmExecutor::~GroupedGemmExecutor() {
  if (impl_ != nullptr) {
    impl_->buffer.release();
    delete impl_;
    impl_ = nullptr;
  }
}

GroupedGemmExecutor::GroupedGemmExecutor(GroupedGemmExecutor&& other) noexcept : impl_(other.impl_) {
  other.impl_ = nullptr;
}

GroupedGemmExecutor& GroupedGemmExecutor::operator=(GroupedGemmExecutor&& other) noexcept {
  if (this != &other) {
    if (impl_ != nullptr) {
      impl_->buffer.release();
      delete impl_;
    }
    impl_ = other.impl_;
    other.impl_ = nullptr;
  }
  return *this;
}

// build (src/grouped_gemm.cu:1132-1239).  Beyond the reference's checks it
// verifies that tile_offsets is the prefix sum of the sorted problems' tile
// counts, so that a launch can never address a tile outside its problem.  The
// descriptors, offsets, schedule and zeroed scheduler state go to the device
// in one copy, into the executor's allocation when it is large enough (after
// the last run's launch has ended).  After a failed build, run() returns
// hipErrorInvalidValue until a build succeeds.
hipError_t GroupedGemmExecutor::build(const PreparedProblemSet& prepared, const KernelConfig& config) {
  if (impl_ == nullptr) return hipErrorInvalidDevicePointer;
  impl_->reset();
  impl_->failed = true;

  RuntimeMode mode;
  hipError_t status = resolve_runtime_mode(config, &mode);
  if (status != hipSuccess) return status;

  const int problem_count = static_cast<int>(prepared.sorted_problems.size());
  if (static_cast<int>(prepared.tile_offsets.size()) != problem_count + 1) return hipErrorInvalidValue;
  if (prepared.tile_offsets.back() != prepared.total_tiles) return hipErrorInvalidValue;
  if (prepared.tile_offsets[0] != 0) return hipErrorInvalidValue;

  std::vector<DeviceProblemDesc> device_problems;
  device_problems.reserve(problem_count);
  for (int i = 0; i < problem_count; ++i) {
    const ProblemDesc& p = prepared.sorted_problems[i];
    if (p.m < 0 || p.n < 0 || p.k < 0) return hipErrorInvalidValue;
    if (p.a == nullptr || p.b == nullptr || p.d == nullptr) return hipErrorInvalidDevicePointer;
    const DeviceProblemDesc dp = to_device_problem(p, config);
    const int64_t tiles = static_cast<int64_t>(dp.tiles_m) * dp.tiles_n;
    if (static_cast<int64_t>(prepared.tile_offsets[i + 1]) - prepared.tile_offsets[i] != tiles) {
      return hipErrorInvalidValue;
    }
    device_problems.push_back(dp);
  }
  // The variant, schedule, grid and work table, with the occupancy of the
  // variant the plan chooses.
  LaunchPlan plan;
  status = plan_launch(device_problems, config, mode.device.compute_units,
                       [&](int variant, int path, int* blocks) {
                         RuntimeMode chosen = mode;
                         chosen.variant = variant;
                         chosen.path = path;
                         hipError_t s = ggk_work_shape_get(variant, path, &chosen.work);
                         if (s != hipSuccess) return s;
                         OccupancyInfo occupancy{};
                         s = cached_occupancy(config, chosen, &occupancy);
                         *blocks = occupancy.active_blocks_per_sm;
                         return s;
                       },
                       &plan);
  if (status != hipSuccess) return status;
  const std::vector<int>& table = plan.work_table;

  // Device ints: the reference tile offsets (sorted order), the work-tile
  // offsets (scheduling order), the scheduling order, then the work table.
  const size_t int_count = 3 * static_cast<size_t>(problem_count) + 2 + table.size();
  const size_t desc_bytes = DeviceBuffer::round256(problem_count * sizeof(DeviceProblemDesc));
  const size_t int_bytes = DeviceBuffer::round256(int_count * sizeof(int));
  const size_t state_bytes = DeviceBuffer::round256(GGK_SCHEDULER_STATE_INTS * sizeof(int));
  const size_t total_bytes = desc_bytes + int_bytes + state_bytes;
  std::vector<unsigned char> host(total_bytes, 0);
  if (problem_count > 0) std::memcpy(host.data(), device_problems.data(), problem_count * sizeof(DeviceProblemDesc));
  int* ints = reinterpret_cast<int*>(host.data() + desc_bytes);
  ints = std::copy(prepared.tile_offsets.begin(), prepared.tile_offsets.end(), ints);
  ints = std::copy(plan.work_offsets.begin(), plan.work_offsets.end(), ints);
  ints = std::copy(plan.order.begin(), plan.order.end(), ints);
  ints = std::copy(table.begin(), table.end(), ints);

  status = impl_->buffer.reserve(total_bytes);
  if (status != hipSuccess) return status;
  status = ggk_copy_to_device(impl_->buffer.base, host.data(), total_bytes);
  if (status != hipSuccess) return status;

  unsigned char* base = static_cast<unsigned char*>(impl_->buffer.base);
  impl_->d_problems = reinterpret_cast<DeviceProblemDesc*>(base);
  impl_->d_ints = reinterpret_cast<int*>(base + desc_bytes);
  impl_->d_state = reinterpret_cast<int*>(base + desc_bytes + int_bytes);
  impl_->problem_count = problem_count;
  impl_->total_tiles = prepared.total_tiles;
  impl_->total_work = plan.total_work;
  impl_->config = config;
  impl_->variant = plan.variant;
  impl_->path = plan.path;
  impl_->addressing = plan.addressing;
  impl_->chunk_bounds = plan.chunk_bounds;
  impl_->work_table = !table.empty();
  impl_->launch_total = plan.launch_total;
  impl_->launch_bounds = plan.launch_bounds;
  impl_->grid_ctas = plan.grid;
  impl_->failed = false;
  return hipSuccess;
}

// run (src/grouped_gemm.cu:1241-1265).  No counter reset is launched: the
// grouped kernel returns its scheduler state to zero when its last workgroup
// retires, so consecutive runs in stream order start from zero.
hipError_t GroupedGemmExecutor::run(hipStream_t stream) const {
  if (impl_ == nullptr) return hipErrorInvalidDevicePointer;
  if (impl_->failed) return hipErrorInvalidValue;
  if (impl_->total_tiles == 0 || impl_->problem_count == 0) return hipSuccess;
  const hipError_t status =
      ggk_launch_grouped(impl_->variant, impl_->path, impl_->addressing, impl_->d_problems,
                         impl_->d_ints + impl_->problem_count + 1, impl_->d_ints + 2 * (impl_->problem_count + 1),
                         impl_->d_work_table(), impl_->problem_count, impl_->launch_total, impl_->d_state,
                         impl_->launch_bounds.data(), impl_->grid_ctas, stream);
  if (status != hipSuccess) return status;
  return impl_->buffer.note_launch(stream);
}

hipError_t GroupedGemmExecutor::run_traced(int* d_tile_map, long long* d_wg_clock, hipStream_t stream,
                                           long long* d_tile_phases) const {
  if (impl_ == nullptr) return hipErrorInvalidDevicePointer;
  if (impl_->failed) return hipErrorInvalidValue;
  if (impl_->total_tiles == 0 || impl_->problem_count == 0) return hipSuccess;
  const hipError_t status = ggk_launch_grouped_traced(
      impl_->variant, impl_->path, impl_->addressing, impl_->d_problems, impl_->d_ints,
      impl_->d_ints + impl_->problem_count + 1, impl_->d_ints + 2 * (impl_->problem_count + 1), impl_->d_work_table(),
      impl_->problem_count, impl_->launch_total, impl_->d_state, impl_->launch_bounds.data(), impl_->grid_ctas, d_tile_map,
      d_wg_clock, d_tile_phases, stream);
  if (status != hipSuccess) return status;
  return impl_->buffer.note_launch(stream);
}

int GroupedGemmExecutor::problem_count() const { return impl_ != nullptr ? impl_->problem_count : 0; }

int GroupedGemmExecutor::launched_work_tiles() const {
  return impl_ != nullptr && !impl_->failed ? impl_->launch_total : 0;
}

int GroupedGemmExecutor::total_tiles() const { return impl_ != nullptr ? impl_->total_tiles : 0; }

int GroupedGemmExecutor::grid_ctas() const { return impl_ != nullptr ? impl_->grid_ctas : 0; }

bool GroupedGemmExecutor::using_tensor_cores() const {
  return impl_ != nullptr && impl_->path == GGK_PATH_MFMA;
}

hipError_t GroupedGemmExecutor::schedule(ggk_work_shape* shape, std::vector<int>* order,
                                         std::vector<int>* work_offsets, std::vector<int>* chunk_bounds) const {
  if (impl_ == nullptr || impl_->variant < 0) return hipErrorInvalidDevicePointer;
  const int count = impl_->problem_count;
  if (shape != nullptr) {
    const hipError_t status = ggk_work_shape_get(impl_->variant, impl_->path, shape);
    if (status != hipSuccess) return status;
  }
  // Device ints: [count + 1] reference tile offsets, [count + 1] work-tile
  // offsets, [count] scheduling order.
  std::vector<int> ints(count > 0 ? 3 * static_cast<size_t>(count) + 2 : 0);
  if (count > 0) {
    const hipError_t status = ggk_copy_to_host(ints.data(), impl_->d_ints, ints.size() * sizeof(int));
    if (status != hipSuccess) return status;
  }
  if (work_offsets != nullptr) {
    work_offsets->assign(1, 0);
    if (count > 0) work_offsets->assign(ints.begin() + count + 1, ints.begin() + 2 * count + 2);
  }
  if (order != nullptr) {
    order->clear();
    if (count > 0) order->assign(ints.begin() + 2 * count + 2, ints.end());
  }
  if (chunk_bounds != nullptr) chunk_bounds->assign(impl_->chunk_bounds.begin(), impl_->chunk_bounds.end());
  return hipSuccess;
}

// run_grouped_gemm_once (src/grouped_gemm.cu:1279-1291).
hipError_t run_grouped_gemm_once(const std::vector<ProblemDesc>& problems, SortMode sort_mode,
                                 const KernelConfig& config, hipStream_t stream) {
  const PreparedProblemSet prepared = prepare_problem_set(problems, config, sort_mode);
  GroupedGemmExecutor executor;
  hipError_t status = executor.build(prepared, config);
  if (status != hipSuccess) return status;
  status = executor.run(stream);
  if (status != hipSuccess) return status;
  return ggk_stream_synchronize(stream);
}

// run_baseline_per_problem (src/grouped_gemm.cu:1293-1317): one launch per
// problem with tiles; a null a, b or d on any problem is InvalidDevicePointer.
hipError_t run_baseline_per_problem(const std::vector<ProblemDesc>& problems, const KernelConfig& config,
                                    hipStream_t stream) {
  RuntimeMode mode;
  hipError_t status = resolve_runtime_mode(config, &mode);
  if (status != hipSuccess) return status;
  for (const ProblemDesc& p : problems) {
    if (p.a == nullptr || p.b == nullptr || p.d == nullptr) return hipErrorInvalidDevicePointer;
    const DeviceProblemDesc dp = to_device_problem(p, config);
    status = ggk_launch_single(mode.variant, mode.path, &dp, stream);
    if (status != hipSuccess) return status;
  }
  return hipSuccess;
}

// count_non_empty_problems (src/grouped_gemm.cu:1319-1329).
int count_non_empty_problems(const std::vector<ProblemDesc>& problems, const KernelConfig& config) {
  int count = 0;
  for (const ProblemDesc& p : problems) {
    if (tile_count_for_problem(p, config) > 0) ++count;
  }
  return count;
}

// The problems are independent, so a split across GPUs needs no exchange: each piece (a whole
// problem or a range of its columns) goes to one rank.  Pieces are cut at work-tile column
// boundaries, so every element of D is computed by the same work tile, with the same k order, as
// in the unsplit set.
hipError_t plan_shards(const std::vector<ProblemDesc>& problems, const KernelConfig& config, int ranks,
                       std::vector<ShardPiece>* pieces) {
  if (pieces == nullptr) return hipErrorInvalidValue;
  pieces->clear();
  const int variant = resolve_variant(config);
  if (variant < 0 || ranks < 1) return hipErrorInvalidValue;
  const int path = config.use_tensor_cores ? GGK_PATH_MFMA : GGK_PATH_FMA;
  ggk_work_shape shape{};
  const hipError_t status = ggk_work_shape_get(variant, path, &shape);
  if (status != hipSuccess) return status;
  const int bm = config.cta_m * shape.tiles_m;
  const int bn = config.cta_n * shape.tiles_n;
  // Estimated time of columns [col0, col0 + cols) of problem p (the schedule's tile-time model).
  auto estimate = [&](const ProblemDesc& p, int cols) {
    if (p.m <= 0 || cols <= 0) return 0.0;
    const bool reads_c = p.c != nullptr && p.beta != 0.0f;
    return problem_work_time(p.m, cols, p.k, ceil_div(p.m, bm), ceil_div(cols, bn), shape.stage_k, reads_c);
  };
  double total = 0.0;
  for (const ProblemDesc& p : problems) {
    if (p.m < 0 || p.n < 0 || p.k < 0) return hipErrorInvalidValue;
    total += estimate(p, p.n);
  }
  const double share = total / ranks;
  std::vector<ShardPiece> out;
  std::vector<double> time;
  for (int i = 0; i < static_cast<int>(problems.size()); ++i) {
    const ProblemDesc& p = problems[i];
    const double t = estimate(p, p.n);
    const int wtn = p.n > 0 ? ceil_div(p.n, bn) : 0;
    // A problem above one rank's share is cut into that many column ranges (at most one per
    // work-tile column), as even as whole work-tile columns allow.
    int parts = 1;
    if (share > 0.0 && t > share && wtn > 1) {
      parts = static_cast<int>(std::min<double>(wtn, std::ceil(t / share)));
    }
    int first = 0;
    for (int part = 0; part < parts; ++part) {
      const int span = wtn / parts + (part < wtn % parts ? 1 : 0);
      const int col0 = first * bn;
      const int cols = parts == 1 ? p.n : std::min(p.n - col0, span * bn);
      out.push_back(ShardPiece{i, 0, col0, cols});
      time.push_back(parts == 1 ? t : estimate(p, cols));
      first += span;
    }
  }
  // Longest piece first (stable), each to the rank with the least estimated time so far (ties:
  // the lowest rank).
  std::vector<int> by_time(out.size());
  std::iota(by_time.begin(), by_time.end(), 0);
  std::stable_sort(by_time.begin(), by_time.end(), [&](int x, int y) { return time[x] > time[y]; });
  std::vector<double> load(ranks, 0.0);
  for (const int j : by_time) {
    if (time[j] <= 0.0) continue;  // an empty problem: rank 0
    const int r = static_cast<int>(std::min_element(load.begin(), load.end()) - load.begin());
    out[j].rank = r;
    load[r] += time[j];
  }
  *pieces = std::move(out);
  return hipSuccess;
}

ProblemDesc shard_problem(const ProblemDesc& problem, const ShardPiece& piece) {
  ProblemDesc out = problem;
  out.n = piece.cols;
  out.b = problem.b != nullptr ? problem.b + piece.col0 : nullptr;
  out.c = problem.c != nullptr ? problem.c + piece.col0 : nullptr;
  out.d = problem.d != nullptr ? problem.d + piece.col0 : nullptr;
  return out;
}

// ---------------------------------------------------------------------------
// MoeGroupedGemm: device-side prepare + grouped launch (no reference counterpart).

struct MoeGroupedGemm::Impl {
  ggk_moe_layout layout{};
  int variant = -1;
  int path = GGK_PATH_FMA;
  int addressing = GGK_ADDR_32;
  int sort_mode = 0;
  int grid_ctas = 0;
  DeviceBuffer buffer;
  DeviceProblemDesc* d_problems = nullptr;
  int* d_ints = nullptr;  // offsets [2 * (E + 1)] | permutation [E] | order [E] | header
  int* d_state = nullptr;

  int* offsets() const { return d_ints; }
  int* perm() const { return d_ints + 2 * (layout.experts + 1); }
  int* order() const { return perm() + layout.experts; }
  int* header() const { return order() + layout.experts; }

  // Forgets the last build: run() refuses to launch until a build succeeds.
  void reset() {
    layout = ggk_moe_layout{};
    variant = -1;
    grid_ctas = 0;
    d_problems = nullptr;
    d_ints = nullptr;
    d_state = nullptr;
  }
};

MoeGroupedGemm::MoeGroupedGemm() : impl_(new Impl()) {}

MoeGroupedGemm::~MoeGroupedGemm() {
  if (impl_ != nullptr) {
    impl_->buffer.release();
    delete impl_;
    impl_ = nullptr;
  }
}

MoeGroupedGemm::MoeGroupedGemm(MoeGroupedGemm&& other) noexcept : impl_(other.impl_) { other.impl_ = nullptr; }

MoeGroupedGemm& MoeGroupedGemm::operator=(MoeGroupedGemm&& other) noexcept {
  if (this != &other) {
    if (impl_ != nullptr) {
      impl_->buffer.release();
      delete impl_;
    }
    impl_ = other.impl_;
    other.impl_ = nullptr;
  }
  return *this;
}

namespace {

// How a MoE group launches: its layout as the kernels read it, the kernel
// (variant, path), the addressing form and the grid.
struct MoePlan {
  ggk_moe_layout layout{};
  RuntimeMode mode;
  int addressing = GGK_ADDR_32;
  int grid = 0;
};

hipError_t plan_moe(const MoeLayout& layout, const KernelConfig& config, SortMode sort_mode, MoePlan* plan) {
  hipError_t status = resolve_runtime_mode(config, &plan->mode);
  if (status != hipSuccess) return status;
  RuntimeMode& mode = plan->mode;
  const int e = layout.experts;
  const int sm = static_cast<int>(sort_mode);
  if (e < 1 || e > GGK_MOE_MAX_EXPERTS || sm < 0 || sm > 3) return hipErrorInvalidValue;
  if (layout.a == nullptr || layout.b == nullptr || layout.d == nullptr) return hipErrorInvalidDevicePointer;

  ggk_moe_layout& L = plan->layout;
  L = ggk_moe_layout{};
  L.experts = e;
  L.n = layout.n;
  L.k = layout.k;
  L.a = layout.a;
  L.lda = layout.lda;
  L.b = layout.b;
  L.ldb = layout.ldb;
  L.stride_b = layout.stride_b;
  L.c = layout.c;
  L.ldc = layout.ldc;
  L.d = layout.d;
  L.ldd = layout.ldd;
  L.alpha = layout.alpha;
  L.beta = layout.beta;
  L.max_rows = layout.max_rows;

  // The addressing form from the strides alone (they bound every in-problem
  // offset, whatever the counts turn out to be).
  DeviceProblemDesc probe{};
  probe.m = std::max(1, L.max_rows);
  probe.n = std::max(1, L.n);
  probe.k = L.k;
  probe.a = L.a;
  probe.b = L.b;
  probe.c = L.c;
  probe.d = L.d;
  probe.lda = L.lda;
  probe.ldb = L.ldb;
  probe.ldc = L.ldc;
  probe.ldd = L.ldd;
  probe.alpha = L.alpha;
  probe.beta = L.beta;
  probe.tiles_m = 1;
  probe.tiles_n = 1;
  int wide = ggk_needs_addr64(mode.variant, mode.path, &probe);
  if (wide < 0) return hipErrorInvalidValue;
  // As in GroupedGemmExecutor::build: no 64-bit 256 x 256 work tiles.
  if (wide == 1 && mode.path == GGK_PATH_MFMA && ggk_small_variant(mode.variant) >= 0) {
    mode.variant = ggk_small_variant(mode.variant);
    status = ggk_work_shape_get(mode.variant, mode.path, &mode.work);
    if (status != hipSuccess) return status;
    wide = ggk_needs_addr64(mode.variant, mode.path, &probe);
  }
  plan->addressing = wide == 1 ? GGK_ADDR_64 : GGK_ADDR_32;
  // The prepare kernel's own layout checks, made here so that a layout it
  // would reject fails build() and the allocation-free call before anything
  // is launched.
  status = ggk_moe_layout_check(mode.variant, mode.path, &L);
  if (status != hipSuccess) return status;

  OccupancyInfo occupancy{};
  status = cached_occupancy(config, mode, &occupancy);
  if (status != hipSuccess) return status;
  // The total is known only on the device: one workgroup per resident slot
  // (or the requested persistent size); idle ones retire at once.
  plan->grid = config.persistent_ctas > 0
                   ? config.persistent_ctas
                   : std::max(1, occupancy.sm_count * std::max(1, occupancy.active_blocks_per_sm));
  return hipSuccess;
}

// Byte layout of a MoE group's device-side set of E experts: descriptors,
// ints (offsets [2 (E + 1)] | permutation [E] | order [E] | header), then the
// scheduler state, each part on a 256-byte boundary.
struct MoeBytes {
  size_t desc, ints, state;
  size_t total() const { return desc + ints + state; }
};
MoeBytes moe_bytes(int experts) {
  const size_t ints = 2 * static_cast<size_t>(experts + 1) + 2 * static_cast<size_t>(experts) + GGK_MOE_HEADER_INTS;
  return MoeBytes{DeviceBuffer::round256(experts * sizeof(DeviceProblemDesc)), DeviceBuffer::round256(ints * sizeof(int)),
                  DeviceBuffer::round256(GGK_SCHEDULER_STATE_INTS * sizeof(int))};
}

}  // namespace

// Checks the layout and sizes the device-side set: E descriptors, 2 (E + 1) +
// 2 E + GGK_MOE_HEADER_INTS ints and the scheduler state, in one allocation
// (kept from the previous build when large enough).  On any failure the
// object is reset and run() returns hipErrorInvalidDevicePointer.
hipError_t MoeGroupedGemm::build(const MoeLayout& layout, const KernelConfig& config, SortMode sort_mode) {
  if (impl_ == nullptr) return hipErrorInvalidDevicePointer;
  impl_->reset();
  MoePlan plan;
  hipError_t status = plan_moe(layout, config, sort_mode, &plan);
  if (status != hipSuccess) return status;
  const MoeBytes bytes = moe_bytes(plan.layout.experts);
  status = impl_->buffer.reserve(bytes.total());
  if (status != hipSuccess) return status;
  status = ggk_zero(impl_->buffer.base, bytes.total());
  if (status != hipSuccess) return status;

  unsigned char* base = static_cast<unsigned char*>(impl_->buffer.base);
  impl_->d_problems = reinterpret_cast<DeviceProblemDesc*>(base);
  impl_->d_ints = reinterpret_cast<int*>(base + bytes.desc);
  impl_->d_state = reinterpret_cast<int*>(base + bytes.desc + bytes.ints);
  impl_->layout = plan.layout;
  impl_->variant = plan.mode.variant;
  impl_->path = plan.mode.path;
  impl_->addressing = plan.addressing;
  impl_->sort_mode = static_cast<int>(sort_mode);
  impl_->grid_ctas = plan.grid;
  return hipSuccess;
}

hipError_t MoeGroupedGemm::run(const int* d_counts, hipStream_t stream) const {
  if (impl_ == nullptr || impl_->d_problems == nullptr || impl_->variant < 0) return hipErrorInvalidDevicePointer;
  if (d_counts == nullptr) return hipErrorInvalidDevicePointer;
  hipError_t status = ggk_moe_prepare(impl_->variant, impl_->path, &impl_->layout, d_counts, impl_->sort_mode,
                                      impl_->d_problems, impl_->offsets(), impl_->perm(), impl_->order(),
                                      impl_->header(), stream);
  if (status != hipSuccess) return status;
  status = ggk_launch_grouped_device(impl_->variant, impl_->path, impl_->addressing, impl_->d_problems,
                                     impl_->offsets() + impl_->layout.experts + 1, impl_->order(),
                                     impl_->layout.experts, impl_->header(), impl_->d_state, impl_->grid_ctas,
                                     stream);
  if (status != hipSuccess) return status;
  return impl_->buffer.note_launch(stream);
}

int MoeGroupedGemm::grid_ctas() const { return impl_ != nullptr ? impl_->grid_ctas : 0; }
const DeviceProblemDesc* MoeGroupedGemm::device_problems() const {
  return impl_ != nullptr ? impl_->d_problems : nullptr;
}
const int* MoeGroupedGemm::device_offsets() const {
  return impl_ != nullptr && impl_->d_ints ? impl_->offsets() : nullptr;
}
const int* MoeGroupedGemm::device_sorted_to_original() const {
  return impl_ != nullptr && impl_->d_ints ? impl_->perm() : nullptr;
}
const int* MoeGroupedGemm::device_order() const { return impl_ != nullptr && impl_->d_ints ? impl_->order() : nullptr; }
const int* MoeGroupedGemm::device_header() const { return impl_ != nullptr && impl_->d_ints ? impl_->header() : nullptr; }

// The allocation-free MoE group: the set MoeGroupedGemm keeps in its own
// allocation lives in the library's static scratch array of the current
// device (gg_moe.hip).  The scheduler state is cleared by a fill kernel
// before the prepare kernel (no memset node, so the sequence can be captured
// in a graph); the prepare kernel rewrites the rest.
hipError_t run_moe_grouped_gemm_noalloc(const MoeLayout& layout, const KernelConfig& config, SortMode sort_mode,
                                        const int* d_counts, hipStream_t stream) {
  MoePlan plan;
  hipError_t status = plan_moe(layout, config, sort_mode, &plan);
  if (status != hipSuccess) return status;
  if (d_counts == nullptr) return hipErrorInvalidDevicePointer;
  void* scratch = nullptr;
  size_t capacity = 0;
  status = gg_moe_scratch(&scratch, &capacity);
  if (status != hipSuccess) return status;
  const MoeBytes bytes = moe_bytes(plan.layout.experts);
  if (bytes.total() > capacity) return hipErrorInvalidValue;
  unsigned char* base = static_cast<unsigned char*>(scratch);
  auto* problems = reinterpret_cast<DeviceProblemDesc*>(base);
  int* ints = reinterpret_cast<int*>(base + bytes.desc);
  int* state = reinterpret_cast<int*>(base + bytes.desc + bytes.ints);
  const int e = plan.layout.experts;
  int* perm = ints + 2 * (e + 1);
  int* order = perm + e;
  int* header = order + e;
  // 0.0f is the all-zero bit pattern.
  status = ggk_fill_f32(reinterpret_cast<float*>(state), GGK_SCHEDULER_STATE_INTS, 0.0f, stream);
  if (status != hipSuccess) return status;
  status = ggk_moe_prepare(plan.mode.variant, plan.mode.path, &plan.layout, d_counts, static_cast<int>(sort_mode),
                           problems, ints, perm, order, header, stream);
  if (status != hipSuccess) return status;
  return ggk_launch_grouped_device(plan.mode.variant, plan.mode.path, plan.addressing, problems, ints + e + 1, order, e,
                                   header, state, plan.grid, stream);
}

}  // namespace grouped_gemm
