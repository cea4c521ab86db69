// C++ drop-in check of include/grouped_gemm/grouped_gemm.h.
//
// Uses the C++ API the way a caller of the reference's header does
// (tests/test_correctness.cu): device buffers from hipMalloc, problems as
// grouped_gemm::ProblemDesc, every sort mode through run_grouped_gemm_once,
// then run_baseline_per_problem and the empty set.  Inputs are drawn exactly as
// the reference test draws them (std::mt19937(20260328), uniform_real(-1, 1):
// alpha, beta, A, B, C per problem); the expected D comes from the CPU oracle.
// D is poisoned with NaN before every run.  Exit status 0 means every check
// passed.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "gg_oracle.h"
#include "grouped_gemm/grouped_gemm.h"

namespace {

bool ok_status(hipError_t st, const char* what) {
  if (st != hipSuccess) {
    std::printf("FAIL %s: %s\n", what, hipGetErrorString(st));
    return false;
  }
  return true;
}

struct Operands {
  int m, n, k;
  float alpha, beta;
  std::vector<uint16_t> a, b;
  std::vector<float> c, want;
  void* da = nullptr;
  void* db = nullptr;
  float* dc = nullptr;
  float* dd = nullptr;
  size_t d_elems = 1;
};

size_t at_least_one(int rows, int cols) {
  return (rows > 0 && cols > 0) ? static_cast<size_t>(rows) * cols : 1;
}

uint16_t half_bits(float x) {
  const __half h = __float2half_rn(x);
  uint16_t bits;
  std::memcpy(&bits, &h, sizeof(bits));
  return bits;
}

bool make_operands(const std::vector<std::vector<int>>& shapes, std::vector<Operands>* out,
                   std::vector<grouped_gemm::ProblemDesc>* problems) {
  std::mt19937 rng(20260328);
  std::uniform_real_distribution<float> uni(-1.0f, 1.0f);
  out->resize(shapes.size());
  problems->clear();
  for (size_t i = 0; i < shapes.size(); ++i) {
    Operands& o = (*out)[i];
    o.m = shapes[i][0];
    o.n = shapes[i][1];
    o.k = shapes[i][2];
    const int lda = o.k > 1 ? o.k : 1, ldn = o.n > 1 ? o.n : 1;
    o.alpha = uni(rng);
    o.beta = uni(rng);
    o.a.resize(at_least_one(o.m, lda));
    o.b.resize(at_least_one(o.k, ldn));
    o.c.resize(at_least_one(o.m, ldn));
    for (auto& x : o.a) x = half_bits(uni(rng));
    for (auto& x : o.b) x = half_bits(uni(rng));
    for (auto& x : o.c) x = uni(rng);
    o.d_elems = at_least_one(o.m, ldn);
    o.want.assign(o.d_elems, 0.0f);
    go_gemm(o.m, o.n, o.k, o.a.data(), lda, o.b.data(), ldn, o.c.data(), ldn, o.alpha, o.beta, o.want.data(), ldn);
    if (!ok_status(hipMalloc(&o.da, o.a.size() * 2), "hipMalloc a") ||
        !ok_status(hipMalloc(&o.db, o.b.size() * 2), "hipMalloc b") ||
        !ok_status(hipMalloc(reinterpret_cast<void**>(&o.dc), o.c.size() * 4), "hipMalloc c") ||
        !ok_status(hipMalloc(reinterpret_cast<void**>(&o.dd), o.d_elems * 4), "hipMalloc d")) {
      return false;
    }
    hipMemcpy(o.da, o.a.data(), o.a.size() * 2, hipMemcpyHostToDevice);
    hipMemcpy(o.db, o.b.data(), o.b.size() * 2, hipMemcpyHostToDevice);
    hipMemcpy(o.dc, o.c.data(), o.c.size() * 4, hipMemcpyHostToDevice);
    grouped_gemm::ProblemDesc p{};
    p.m = o.m;
    p.n = o.n;
    p.k = o.k;
    p.a = static_cast<const __half*>(o.da);
    p.b = static_cast<const __half*>(o.db);
    p.c = o.dc;
    p.d = o.dd;
    p.lda = lda;
    p.ldb = ldn;
    p.ldc = ldn;
    p.ldd = ldn;
    p.alpha = o.alpha;
    p.beta = o.beta;
    problems->push_back(p);
  }
  return true;
}

void poison(std::vector<Operands>* ops) {
  std::vector<float> nan_fill;
  for (Operands& o : *ops) {
    nan_fill.assign(o.d_elems, std::nanf(""));
    hipMemcpy(o.dd, nan_fill.data(), o.d_elems * 4, hipMemcpyHostToDevice);
  }
}

bool verify(const std::vector<Operands>& ops, const char* what) {
  double worst = 0.0;
  for (size_t i = 0; i < ops.size(); ++i) {
    const Operands& o = ops[i];
    std::vector<float> got(o.d_elems);
    hipMemcpy(got.data(), o.dd, o.d_elems * 4, hipMemcpyDeviceToHost);
    if (o.m <= 0 || o.n <= 0) {
      if (!std::isnan(got[0])) {
        std::printf("FAIL %s: empty problem %zu was written\n", what, i);
        return false;
      }
      continue;
    }
    const double tol = 1e-3 * std::sqrt(static_cast<double>(o.k > 1 ? o.k : 1)) * std::fabs(o.alpha) +
                       1e-6 * (std::fabs(o.beta) + 1.0);
    for (size_t e = 0; e < static_cast<size_t>(o.m) * o.n; ++e) {
      const double err = std::fabs(static_cast<double>(got[e]) - o.want[e]);
      if (!(err <= tol)) {
        std::printf("FAIL %s: problem %zu element %zu got %g want %g\n", what, i, e, got[e], o.want[e]);
        return false;
      }
      if (err > worst) worst = err;
    }
  }
  std::printf("[PASS] %s max_abs_error=%.3g\n", what, worst);
  return true;
}

bool run_config(const grouped_gemm::KernelConfig& config) {
  const std::vector<std::vector<int>> shapes = {{64, 64, 64}, {128, 64, 96}, {45, 81, 37}, {17, 23, 9},
                                                {192, 32, 64}, {16, 256, 48}, {0, 64, 16}, {64, 0, 16}};
  std::vector<Operands> ops;
  std::vector<grouped_gemm::ProblemDesc> problems;
  if (!make_operands(shapes, &ops, &problems)) return false;

  grouped_gemm::OccupancyInfo occ{};
  if (!ok_status(grouped_gemm::query_occupancy(config, &occ), "query_occupancy")) return false;
  std::printf("config CTA(%d, %d, %d) mfma=%d: active_blocks_per_sm=%d sm_count=%d vgprs=%d agprs=%d "
              "lds=%d theoretical=%.2f%%\n",
              config.cta_m, config.cta_n, config.cta_k, occ.using_tensor_cores ? 1 : 0, occ.active_blocks_per_sm,
              occ.sm_count, occ.vgprs_per_thread, occ.agprs_per_thread, occ.static_shared_bytes,
              occ.theoretical_occupancy * 100.0f);

  const grouped_gemm::SortMode modes[] = {grouped_gemm::SortMode::kNone, grouped_gemm::SortMode::kByK,
                                          grouped_gemm::SortMode::kByTiles,
                                          grouped_gemm::SortMode::kByTilesThenK};
  char label[128];
  for (grouped_gemm::SortMode mode : modes) {
    poison(&ops);
    if (!ok_status(grouped_gemm::run_grouped_gemm_once(problems, mode, config, nullptr), "grouped")) return false;
    if (!ok_status(hipDeviceSynchronize(), "sync")) return false;
    std::snprintf(label, sizeof(label), "grouped mode=%s", grouped_gemm::sort_mode_name(mode));
    if (!verify(ops, label)) return false;
  }

  // Executor reuse: build once, run twice.
  const grouped_gemm::PreparedProblemSet prepared =
      grouped_gemm::prepare_problem_set(problems, config, grouped_gemm::SortMode::kByTiles);
  grouped_gemm::GroupedGemmExecutor executor;
  if (!ok_status(executor.build(prepared, config), "build")) return false;
  for (int rep = 0; rep < 2; ++rep) {
    poison(&ops);
    if (!ok_status(executor.run(nullptr), "run") || !ok_status(hipDeviceSynchronize(), "sync")) return false;
    if (!verify(ops, "executor rerun")) return false;
  }
  grouped_gemm::GroupedGemmExecutor moved(std::move(executor));
  if (executor.run(nullptr) != hipErrorInvalidDevicePointer) {
    std::printf("FAIL moved-from executor did not report InvalidDevicePointer\n");
    return false;
  }
  if (moved.total_tiles() != prepared.total_tiles) return false;

  poison(&ops);
  if (!ok_status(grouped_gemm::run_baseline_per_problem(problems, config, nullptr), "baseline")) return false;
  if (!ok_status(hipDeviceSynchronize(), "sync")) return false;
  if (!verify(ops, "baseline per-problem")) return false;

  const std::vector<grouped_gemm::ProblemDesc> empty;
  if (!ok_status(grouped_gemm::run_grouped_gemm_once(empty, grouped_gemm::SortMode::kByTiles, config, nullptr),
                 "empty grouped") ||
      !ok_status(grouped_gemm::run_baseline_per_problem(empty, config, nullptr), "empty baseline")) {
    return false;
  }
  std::printf("[PASS] empty problem set\n");
  for (Operands& o : ops) {
    hipFree(o.da);
    hipFree(o.db);
    hipFree(o.dc);
    hipFree(o.dd);
  }
  return true;
}

}  // namespace

int main() {
  bool ok = true;
  const int shapes[3][3] = {{64, 64, 16}, {128, 64, 32}, {64, 128, 32}};
  for (const auto& s : shapes) {
    for (int mfma = 1; mfma >= 0 && ok; --mfma) {
      grouped_gemm::KernelConfig config;
      config.cta_m = s[0];
      config.cta_n = s[1];
      config.cta_k = s[2];
      config.threads = 256;
      config.persistent_ctas = 0;
      config.use_tensor_cores = mfma == 1;
      ok = run_config(config);
    }
  }
  if (!ok) {
    std::printf("Correctness test failed.\n");
    return 1;
  }
  std::printf("All correctness checks passed.\n");
  return 0;
}
