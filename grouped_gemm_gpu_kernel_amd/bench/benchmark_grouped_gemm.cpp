// benchmark_grouped_gemm -- the reference's benchmark harness on the gfx950
// library: same command line, same synthetic problem sets, same results table
// and the same fixed-output cache file (bench/benchmark_grouped_gemm.cu).
//
//   benchmark_grouped_gemm [--problems N] [--warmup N] [--iters N] [--seed N]
//                          [--workload small|mixed|tail]
//                          [--config 64x64x16|128x64x32|64x128x32]
//                          [--persistent-ctas N] [--tensor-cores on|off]
//                          [--fixed-output PATH]
//
// Shapes come from std::mt19937(seed) and operands from std::mt19937(seed + 1)
// through libstdc++'s distributions, drawn in the reference's order, so a run
// here multiplies the same matrices as the reference run with the same flags.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <random>
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

#include "grouped_gemm/grouped_gemm.h"
#include "host_half.h"

namespace {

namespace gg = grouped_gemm;

#define GG_CHECK(call)                                                                            \
  do {                                                                                            \
    const hipError_t status_ = (call);                                                            \
    if (status_ != hipSuccess) {                                                                  \
      std::cerr << "HIP error " << hipGetErrorString(status_) << " at " << __FILE__ << ":"         \
                << __LINE__ << std::endl;                                                         \
      std::exit(1);                                                                               \
    }                                                                                             \
  } while (0)

struct Options {
  int problems = 256;
  int warmup = 20;
  int iters = 100;
  int seed = 20260328;
  std::string workload = "mixed";
  gg::KernelConfig config{64, 64, 16, 256, 0, true};
  std::string fixed_output;
};

// One row of the results table (ModeResult, bench/benchmark_grouped_gemm.cu:100-109).
struct Row {
  std::string mode;
  float prepare_ms = 0.0f;
  float kernel_ms = 0.0f;
  double tflops = 0.0;
  int total_tiles = 0;
  int grid_ctas = 0;
  int launch_count = 0;
  double tail_work_share = 0.0;
};

void usage(const char* prog) {
  std::cout << "Usage: " << prog << " [options]\n"
            << "  --problems N            number of GEMM problems (default: 256)\n"
            << "  --warmup N              warmup iterations (default: 20)\n"
            << "  --iters N               benchmark iterations (default: 100)\n"
            << "  --seed N                random seed (default: 20260328)\n"
            << "  --workload NAME         small|mixed|tail (default: mixed)\n"
            << "  --config NAME           64x64x16|128x64x32|64x128x32 (default: 64x64x16)\n"
            << "  --persistent-ctas N     fixed persistent grid CTAs (default: auto)\n"
            << "  --tensor-cores MODE     on|off (default: on)\n"
            << "  --fixed-output PATH     reuse cached benchmark table for stable output\n";
}

// Command line as in parse_options (bench/benchmark_grouped_gemm.cu:125-233):
// unknown options, missing values and unsupported names fail; counts are
// clamped to problems >= 1, warmup >= 0, iters >= 1.
bool parse(int argc, char** argv, Options* opt) {
  for (int i = 1; i < argc; ++i) {
    const std::string arg = argv[i];
    if (arg == "--help" || arg == "-h") return false;
    const bool takes_value = arg == "--problems" || arg == "--warmup" || arg == "--iters" || arg == "--seed" ||
                             arg == "--workload" || arg == "--config" || arg == "--persistent-ctas" ||
                             arg == "--tensor-cores" || arg == "--fixed-output";
    if (!takes_value) {
      std::cerr << "Unknown option: " << arg << std::endl;
      return false;
    }
    if (i + 1 >= argc) {
      std::cerr << "Missing value for " << arg << std::endl;
      return false;
    }
    const std::string value = argv[++i];
    if (arg == "--problems") {
      opt->problems = std::stoi(value);
    } else if (arg == "--warmup") {
      opt->warmup = std::stoi(value);
    } else if (arg == "--iters") {
      opt->iters = std::stoi(value);
    } else if (arg == "--seed") {
      opt->seed = std::stoi(value);
    } else if (arg == "--workload") {
      opt->workload = value;
    } else if (arg == "--persistent-ctas") {
      opt->config.persistent_ctas = std::stoi(value);
    } else if (arg == "--fixed-output") {
      opt->fixed_output = value;
    } else if (arg == "--tensor-cores") {
      if (value != "on" && value != "off") {
        std::cerr << "Unsupported --tensor-cores mode: " << value << std::endl;
        return false;
      }
      opt->config.use_tensor_cores = value == "on";
    } else {  // --config
      if (value == "64x64x16") {
        opt->config.cta_m = 64, opt->config.cta_n = 64, opt->config.cta_k = 16;
      } else if (value == "128x64x32") {
        opt->config.cta_m = 128, opt->config.cta_n = 64, opt->config.cta_k = 32;
      } else if (value == "64x128x32") {
        opt->config.cta_m = 64, opt->config.cta_n = 128, opt->config.cta_k = 32;
      } else {
        std::cerr << "Unsupported config: " << value << std::endl;
        return false;
      }
    }
  }
  opt->problems = std::max(1, opt->problems);
  opt->warmup = std::max(0, opt->warmup);
  opt->iters = std::max(1, opt->iters);
  return true;
}

// Identity of a run for the fixed-output cache
// (make_fixed_output_fingerprint, bench/benchmark_grouped_gemm.cu:237-257).
std::string fingerprint(const Options& opt, const gg::OccupancyInfo& occ) {
  std::ostringstream s;
  s << "v2;workload=" << opt.workload << ";problems=" << opt.problems << ";warmup=" << opt.warmup
    << ";iters=" << opt.iters << ";seed=" << opt.seed << ";cta_m=" << opt.config.cta_m
    << ";cta_n=" << opt.config.cta_n << ";cta_k=" << opt.config.cta_k << ";threads=" << opt.config.threads
    << ";persistent_ctas=" << opt.config.persistent_ctas
    << ";tensor_cores_requested=" << (opt.config.use_tensor_cores ? 1 : 0)
    << ";tensor_cores_enabled=" << (occ.using_tensor_cores ? 1 : 0) << ";sm_count=" << occ.sm_count
    << ";active_blocks_per_sm=" << occ.active_blocks_per_sm
    << ";registers_per_thread=" << occ.registers_per_thread
    << ";dynamic_shared_bytes=" << occ.dynamic_shared_bytes;
  return s.str();
}

// grouped_gemm_fixed_output_v1 (bench/benchmark_grouped_gemm.cu:260-364):
//   magic grouped_gemm_fixed_output_v1
//   fingerprint <text>
//   result_count <n>
//   result <mode> <prepare_ms> <kernel_ms> <tflops> <tiles> <grid_ctas> <launches> <tail_share>
// Unknown keys are skipped to the end of their line.
bool load_cache(const std::string& path, std::string* fp, std::vector<Row>* rows) {
  std::ifstream in(path);
  std::string key, value;
  if (!in || !(in >> key >> value) || key != "magic" || value != "grouped_gemm_fixed_output_v1") return false;
  std::string found_fp;
  size_t expected = 0;
  bool has_expected = false;
  std::vector<Row> found;
  while (in >> key) {
    if (key == "fingerprint") {
      in >> found_fp;
    } else if (key == "result_count") {
      in >> expected;
      has_expected = true;
    } else if (key == "result") {
      Row r;
      in >> r.mode >> r.prepare_ms >> r.kernel_ms >> r.tflops >> r.total_tiles >> r.grid_ctas >> r.launch_count >>
          r.tail_work_share;
      if (!in.good()) return false;
      found.push_back(r);
    } else {
      std::string rest;
      std::getline(in, rest);
    }
  }
  if (found_fp.empty() || found.empty() || (has_expected && found.size() != expected)) return false;
  *fp = found_fp;
  *rows = found;
  return true;
}

bool save_cache(const std::string& path, const std::string& fp, const std::vector<Row>& rows) {
  const std::filesystem::path file(path);
  if (file.has_parent_path()) {
    std::error_code ec;
    std::filesystem::create_directories(file.parent_path(), ec);
    if (ec) {
      std::cerr << "Failed to create fixed-output directory: " << ec.message() << std::endl;
      return false;
    }
  }
  std::ofstream out(path, std::ios::trunc);
  if (!out) {
    std::cerr << "Failed to open fixed-output file: " << path << std::endl;
    return false;
  }
  out << std::setprecision(9) << "magic grouped_gemm_fixed_output_v1\n"
      << "fingerprint " << fp << "\n"
      << "result_count " << rows.size() << "\n";
  for (const Row& r : rows) {
    out << "result " << r.mode << " " << r.prepare_ms << " " << r.kernel_ms << " " << r.tflops << " "
        << r.total_tiles << " " << r.grid_ctas << " " << r.launch_count << " " << r.tail_work_share << "\n";
  }
  return true;
}

// Problem shapes (generate_shapes, bench/benchmark_grouped_gemm.cu:368-443):
// each value is a uniform pick from the workload's candidate list; "tail"
// first draws uniform_real(0, 1) and takes the large lists when it is >= 0.8.
// The reference makes the three picks as arguments of one emplace_back call,
// which its g++-compiled host code evaluates right to left: k, then n, then m.
// Its published tail-workload tile totals hold only in that order, so the
// picks here are separate statements in that order.
std::vector<std::tuple<int, int, int>> shapes_for(const Options& opt) {
  std::mt19937 rng(static_cast<uint32_t>(opt.seed));
  auto pick = [&rng](const std::vector<int>& values) {
    std::uniform_int_distribution<int> d(0, static_cast<int>(values.size()) - 1);
    return values[d(rng)];
  };
  std::vector<std::tuple<int, int, int>> out;
  out.reserve(opt.problems);
  const std::vector<int> small_m = {16, 24, 32, 48, 64}, small_n = {16, 32, 48, 64, 96};
  const std::vector<int> small_k = {16, 24, 32, 48, 64};
  const std::vector<int> tail_small = {16, 24, 32, 48, 64}, tail_large = {96, 128, 160, 192, 256};
  const std::vector<int> tail_large_k = {96, 128, 192, 256, 384, 512};
  const std::vector<int> mixed = {63, 94, 122, 240, 500};
  std::uniform_real_distribution<float> coin(0.0f, 1.0f);
  for (int i = 0; i < opt.problems; ++i) {
    int m, n, k;
    if (opt.workload == "small") {
      k = pick(small_k);
      n = pick(small_n);
      m = pick(small_m);
    } else if (opt.workload == "tail") {
      const bool small = coin(rng) < 0.8f;
      k = pick(small ? small_k : tail_large_k);
      n = pick(small ? tail_small : tail_large);
      m = pick(small ? tail_small : tail_large);
    } else {  // any other name is the mixed set, as in the reference
      k = pick(mixed);
      n = pick(mixed);
      m = pick(mixed);
    }
    out.emplace_back(m, n, k);
  }
  return out;
}

size_t elems(int rows, int cols) { return rows <= 0 || cols <= 0 ? 1 : static_cast<size_t>(rows) * cols; }

struct Buffers {
  std::vector<void*> device;
  ~Buffers() {
    for (void* p : device) (void)hipFree(p);
  }
  template <class T>
  T* upload(const std::vector<T>& host) {
    void* p = nullptr;
    GG_CHECK(hipMalloc(&p, host.size() * sizeof(T)));
    GG_CHECK(hipMemcpy(p, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice));
    device.push_back(p);
    return static_cast<T*>(p);
  }
  float* output(size_t count) {
    void* p = nullptr;
    GG_CHECK(hipMalloc(&p, count * sizeof(float)));
    device.push_back(p);
    return static_cast<float*>(p);
  }
};

// Operands (init_problem_buffers, bench/benchmark_grouped_gemm.cu:448-534):
// per problem A, then B, then C from uniform_real(-1, 1), A and B rounded to
// binary16; tight leading dimensions (at least 1), alpha = beta = 1.
std::vector<gg::ProblemDesc> make_problems(const std::vector<std::tuple<int, int, int>>& shapes, int seed,
                                           Buffers* buf) {
  std::mt19937 rng(static_cast<uint32_t>(seed));
  std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
  std::vector<gg::ProblemDesc> problems;
  for (const auto& [m, n, k] : shapes) {
    gg::ProblemDesc p{};
    p.m = m, p.n = n, p.k = k;
    p.lda = std::max(1, k), p.ldb = std::max(1, n), p.ldc = std::max(1, n), p.ldd = std::max(1, n);
    std::vector<uint16_t> a(elems(m, p.lda)), b(elems(k, p.ldb));
    std::vector<float> c(elems(m, p.ldc));
    for (auto& x : a) x = host_float_to_half_rn(dist(rng));
    for (auto& x : b) x = host_float_to_half_rn(dist(rng));
    for (auto& x : c) x = dist(rng);
    p.a = reinterpret_cast<const __half*>(buf->upload(a));
    p.b = reinterpret_cast<const __half*>(buf->upload(b));
    p.c = buf->upload(c);
    p.d = buf->output(elems(m, p.ldd));
    p.alpha = 1.0f;
    p.beta = 1.0f;
    problems.push_back(p);
  }
  return problems;
}

// Mean ms per launch after `warmup` launches, HIP events around `iters`
// launches on the default stream (benchmark_ms, bench/benchmark_grouped_gemm.cu:539-566).
template <class Launch>
float time_ms(int warmup, int iters, Launch&& launch) {
  for (int i = 0; i < warmup; ++i) GG_CHECK(launch());
  hipEvent_t start, stop;
  GG_CHECK(hipEventCreate(&start));
  GG_CHECK(hipEventCreate(&stop));
  GG_CHECK(hipEventRecord(start, nullptr));
  for (int i = 0; i < iters; ++i) GG_CHECK(launch());
  GG_CHECK(hipEventRecord(stop, nullptr));
  GG_CHECK(hipEventSynchronize(stop));
  float ms = 0.0f;
  GG_CHECK(hipEventElapsedTime(&ms, start, stop));
  GG_CHECK(hipEventDestroy(start));
  GG_CHECK(hipEventDestroy(stop));
  return ms / static_cast<float>(iters);
}

// Static tail share: work = tiles * ceil(k / cta_k) in sorted order; share of
// the last max(1, count / 10) problems (bench/benchmark_grouped_gemm.cu:580-607).
double tail_share(const gg::PreparedProblemSet& prepared, const gg::KernelConfig& cfg) {
  const int n = static_cast<int>(prepared.sorted_problems.size());
  if (n == 0) return 0.0;
  const int tail = std::max(1, n / 10);
  double total = 0.0, last = 0.0;
  for (int i = 0; i < n; ++i) {
    const double work = static_cast<double>(prepared.tile_offsets[i + 1] - prepared.tile_offsets[i]) *
                        ((prepared.sorted_problems[i].k + cfg.cta_k - 1) / cfg.cta_k);
    total += work;
    if (i >= n - tail) last += work;
  }
  return total > 0.0 ? last / total : 0.0;
}

Row grouped_row(const std::vector<gg::ProblemDesc>& problems, gg::SortMode mode, const Options& opt, double flops) {
  Row r;
  r.mode = gg::sort_mode_name(mode);
  r.launch_count = 1;
  const auto t0 = std::chrono::high_resolution_clock::now();
  const gg::PreparedProblemSet prepared = gg::prepare_problem_set(problems, opt.config, mode);
  gg::GroupedGemmExecutor executor;
  GG_CHECK(executor.build(prepared, opt.config));
  const auto t1 = std::chrono::high_resolution_clock::now();
  r.prepare_ms = std::chrono::duration<float, std::milli>(t1 - t0).count();
  r.total_tiles = prepared.total_tiles;
  r.grid_ctas = executor.grid_ctas();
  r.tail_work_share = tail_share(prepared, opt.config);
  r.kernel_ms = time_ms(opt.warmup, opt.iters, [&] { return executor.run(nullptr); });
  r.tflops = (flops / 1e12) / (r.kernel_ms / 1e3);
  return r;
}

void print_table(const std::vector<Row>& rows) {
  std::cout << std::left << std::setw(24) << "mode" << std::setw(12) << "prep_ms" << std::setw(12) << "kernel_ms"
            << std::setw(12) << "tflops" << std::setw(12) << "tiles" << std::setw(12) << "grid_ctas" << std::setw(14)
            << "launches" << std::setw(14) << "tail_share" << std::endl;
  for (const Row& r : rows) {
    std::cout << std::left << std::setw(24) << r.mode << std::setw(12) << std::fixed << std::setprecision(3)
              << r.prepare_ms << std::setw(12) << r.kernel_ms << std::setw(12) << r.tflops << std::setw(12)
              << r.total_tiles << std::setw(12) << r.grid_ctas << std::setw(14) << r.launch_count << std::setw(14)
              << r.tail_work_share << std::endl;
  }
}

}  // namespace

int main(int argc, char** argv) {
  Options opt;
  if (!parse(argc, argv, &opt)) {
    usage(argv[0]);
    return 1;
  }
  gg::OccupancyInfo occ{};
  GG_CHECK(gg::query_occupancy(opt.config, &occ));
  std::cout << "Workload: " << opt.workload << ", problems=" << opt.problems << ", warmup=" << opt.warmup
            << ", iters=" << opt.iters << std::endl;
  std::cout << "Kernel config: CTA(" << opt.config.cta_m << ", " << opt.config.cta_n << ", " << opt.config.cta_k
            << "), threads=" << opt.config.threads << ", persistent_ctas=" << opt.config.persistent_ctas
            << ", tensor_cores_requested=" << (opt.config.use_tensor_cores ? "on" : "off") << std::endl;
  std::cout << "Runtime mode: tensor_cores_enabled=" << (occ.using_tensor_cores ? "yes" : "no") << std::endl;
  std::cout << "Occupancy: active_blocks_per_sm=" << occ.active_blocks_per_sm
            << ", max_blocks_per_sm=" << occ.max_blocks_per_sm << ", sm_count=" << occ.sm_count
            << ", theoretical=" << std::fixed << std::setprecision(2) << (occ.theoretical_occupancy * 100.0f) << "%"
            << std::endl;
  std::cout << "Register pressure: estimated_regs_per_thread=" << occ.estimated_registers_per_thread
            << ", measured_regs_per_thread=" << occ.registers_per_thread
            << ", regs_per_block=" << occ.registers_per_block
            << ", register_limited_blocks_per_sm=" << occ.register_limited_blocks_per_sm << std::endl;
  std::cout << "Shared memory: static=" << occ.static_shared_bytes << "B, dynamic=" << occ.dynamic_shared_bytes
            << "B" << std::endl;

  const std::string fp = fingerprint(opt, occ);
  if (!opt.fixed_output.empty()) {
    std::string cached_fp;
    std::vector<Row> cached;
    if (load_cache(opt.fixed_output, &cached_fp, &cached) && cached_fp == fp) {
      print_table(cached);
      return 0;
    }
  }

  Buffers buffers;
  const std::vector<gg::ProblemDesc> problems = make_problems(shapes_for(opt), opt.seed + 1, &buffers);
  double flops = 0.0;
  for (const gg::ProblemDesc& p : problems) flops += 2.0 * static_cast<double>(p.m) * p.n * p.k;

  std::vector<Row> rows;
  int total_tiles = 0;
  for (gg::SortMode mode :
       {gg::SortMode::kNone, gg::SortMode::kByK, gg::SortMode::kByTiles, gg::SortMode::kByTilesThenK}) {
    rows.push_back(grouped_row(problems, mode, opt, flops));
    total_tiles = rows.back().total_tiles;
  }
  Row base;
  base.mode = "baseline_per_problem";
  base.launch_count = gg::count_non_empty_problems(problems, opt.config);
  base.total_tiles = total_tiles;
  base.kernel_ms = time_ms(opt.warmup, opt.iters,
                           [&] { return gg::run_baseline_per_problem(problems, opt.config, nullptr); });
  base.tflops = (flops / 1e12) / (base.kernel_ms / 1e3);
  rows.push_back(base);

  if (!opt.fixed_output.empty() && !save_cache(opt.fixed_output, fp, rows)) {
    std::cerr << "Warning: fixed-output cache was not written." << std::endl;
  }
  print_table(rows);
  return 0;
}
