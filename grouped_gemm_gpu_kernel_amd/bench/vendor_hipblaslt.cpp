// vendor_hipblaslt -- the vendor comparison point for the grouped GEMM: a
// problem list (row-major fp16 A/B, fp32 C/D, fp32 accumulate, per-problem
// alpha/beta) run by hipBLASLt as one hipblaslt_ext::GroupedGemm, as one
// hipblasLtMatmul per problem and, for sets of equal problems at evenly spaced
// addresses, as one strided-batched hipblasLtMatmul, next to this library's
// grouped launch on the same buffers.  This is the taskbook's library baseline option
// (taskbook_grouped_gemm.md:147-159); it is measured beside the library and is
// not part of it.
//
// A program of its own, not a library loaded into Python: PyTorch-ROCm ships
// its own libhipblaslt.so.1, and a process that has imported torch binds every
// later library to that copy, whose C++ classes do not match the headers this
// file is compiled against.
//
//   vendor_hipblaslt SPEC [--steps N] [--warmup N] [--max-algos N] [--no-check]
//                         [--config 128x64x32] [--sort-mode 0..3]
//
// SPEC is a text file:
//   seed S
//   ab uniform LO HI   |  ab normal SIGMA
//   c uniform LO HI    |  c zero  |  c none
//   problems N
//   p M N K ALPHA BETA          (N lines)
// Operands are drawn by the library's counter-hash fill kernels
// (ggk_fill_*), so they depend only on the seed and the pool layout.  Prints
// one JSON object.  With checking on, every vendor D is compared with the
// library's D element by element against twice the parity bound
// 1e-3*sqrt(K)*max|A|*max|B|*|alpha| + 1e-6*(|beta|*max|C| + 1).
//
// hipBLASLt is column-major: a row-major D[m x n] = A[m x k] B[k x n] is the
// column-major D^T[n x m] = B^T[n x k] A^T[k x m], so each problem is handed
// over as (m', n', k') = (n, m, k) with the B pointer as the first operand.
// Problems with m == 0 or n == 0 write nothing and are left out.
#include <hip/hip_runtime_api.h>
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <fstream>
#include <functional>
#include <sstream>
#include <string>
#include <vector>

#include "grouped_gemm/grouped_gemm.h"
#include "grouped_gemm_amd_kernels.h"

namespace {

namespace gg = grouped_gemm;

struct Spec {
  uint64_t seed = 42;
  std::string ab = "uniform", c = "uniform";
  float ab_lo = -1.0f, ab_hi = 1.0f, ab_sigma = 0.0f, c_lo = -1.0f, c_hi = 1.0f;
  std::vector<int> m, n, k;
  std::vector<float> alpha, beta;
};

bool read_spec(const char* path, Spec* s) {
  std::ifstream in(path);
  std::string key;
  int count = -1;
  while (in >> key) {
    if (key == "seed") {
      in >> s->seed;
    } else if (key == "ab") {
      in >> s->ab;
      if (s->ab == "uniform") in >> s->ab_lo >> s->ab_hi;
      else if (s->ab == "normal") in >> s->ab_sigma;
      else return false;
    } else if (key == "c") {
      in >> s->c;
      if (s->c == "uniform") in >> s->c_lo >> s->c_hi;
      else if (s->c != "zero" && s->c != "none") return false;
    } else if (key == "problems") {
      in >> count;
    } else if (key == "p") {
      int m, n, k;
      float a, b;
      in >> m >> n >> k >> a >> b;
      s->m.push_back(m), s->n.push_back(n), s->k.push_back(k), s->alpha.push_back(a), s->beta.push_back(b);
    } else {
      return false;
    }
    if (!in) return false;
  }
  return count == static_cast<int>(s->m.size());
}

#define HIP_OK(call)                                                                 \
  do {                                                                               \
    hipError_t e_ = (call);                                                          \
    if (e_ != hipSuccess) {                                                          \
      std::printf("{\"error\": \"%s: %s\"}\n", #call, hipGetErrorString(e_));         \
      std::exit(1);                                                                  \
    }                                                                                \
  } while (0)

int64_t elems(int rows, int cols) { return rows > 0 && cols > 0 ? static_cast<int64_t>(rows) * cols : 1; }
int64_t round_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// Operand pools: one allocation per operand kind, problems at 256-byte aligned offsets.
struct Pools {
  std::vector<int64_t> a_off, b_off, c_off, d_off;
  uint16_t *a = nullptr, *b = nullptr;
  float *c = nullptr, *d_ours = nullptr, *d_vendor = nullptr;
  int64_t a_n = 0, b_n = 0, c_n = 0, d_n = 0;
};

void make_pools(const Spec& s, Pools* p) {
  const size_t cnt = s.m.size();
  for (size_t i = 0; i < cnt; ++i) {
    p->a_off.push_back(p->a_n), p->a_n += round_up(elems(s.m[i], s.k[i]), 128);
    p->b_off.push_back(p->b_n), p->b_n += round_up(elems(s.k[i], s.n[i]), 128);
    p->c_off.push_back(p->c_n), p->c_n += round_up(elems(s.m[i], s.n[i]), 64);
    p->d_off.push_back(p->d_n), p->d_n += round_up(elems(s.m[i], s.n[i]), 64);
  }
  HIP_OK(hipMalloc(&p->a, std::max<int64_t>(p->a_n, 1) * 2));
  HIP_OK(hipMalloc(&p->b, std::max<int64_t>(p->b_n, 1) * 2));
  HIP_OK(hipMalloc(&p->c, std::max<int64_t>(p->c_n, 1) * 4));
  HIP_OK(hipMalloc(&p->d_ours, std::max<int64_t>(p->d_n, 1) * 4));
  HIP_OK(hipMalloc(&p->d_vendor, std::max<int64_t>(p->d_n, 1) * 4));
  if (s.ab == "uniform") {
    HIP_OK(ggk_fill_uniform_f16(p->a, p->a_n, s.seed, 1, s.ab_lo, s.ab_hi, nullptr));
    HIP_OK(ggk_fill_uniform_f16(p->b, p->b_n, s.seed, 2, s.ab_lo, s.ab_hi, nullptr));
  } else {
    HIP_OK(ggk_fill_normal_f16(p->a, p->a_n, s.seed, 1, s.ab_sigma, nullptr));
    HIP_OK(ggk_fill_normal_f16(p->b, p->b_n, s.seed, 2, s.ab_sigma, nullptr));
  }
  if (s.c == "uniform") HIP_OK(ggk_fill_uniform_f32(p->c, p->c_n, s.seed, 3, s.c_lo, s.c_hi, nullptr));
  else HIP_OK(ggk_fill_f32(p->c, std::max<int64_t>(p->c_n, 1), 0.0f, nullptr));
  HIP_OK(ggk_fill_f32(p->d_ours, std::max<int64_t>(p->d_n, 1), NAN, nullptr));
  HIP_OK(ggk_fill_f32(p->d_vendor, std::max<int64_t>(p->d_n, 1), NAN, nullptr));
  HIP_OK(hipDeviceSynchronize());
}

std::vector<gg::ProblemDesc> problems_for(const Spec& s, const Pools& p, float* d_pool) {
  std::vector<gg::ProblemDesc> out;
  for (size_t i = 0; i < s.m.size(); ++i) {
    gg::ProblemDesc q{};
    q.m = s.m[i], q.n = s.n[i], q.k = s.k[i];
    q.a = reinterpret_cast<const __half*>(p.a + p.a_off[i]);
    q.b = reinterpret_cast<const __half*>(p.b + p.b_off[i]);
    q.c = s.c == "none" ? nullptr : p.c + p.c_off[i];
    q.d = d_pool + p.d_off[i];
    q.lda = std::max(1, q.k), q.ldb = std::max(1, q.n), q.ldc = std::max(1, q.n), q.ldd = std::max(1, q.n);
    q.alpha = s.alpha[i], q.beta = s.beta[i];
    out.push_back(q);
  }
  return out;
}

float time_ms(int steps, int warmup, const std::function<int()>& fn) {
  for (int i = 0; i < warmup; ++i)
    if (fn() != 0) return -1.0f;
  HIP_OK(hipDeviceSynchronize());
  hipEvent_t start, stop;
  HIP_OK(hipEventCreate(&start));
  HIP_OK(hipEventCreate(&stop));
  HIP_OK(hipEventRecord(start, nullptr));
  for (int i = 0; i < steps; ++i)
    if (fn() != 0) return -1.0f;
  HIP_OK(hipEventRecord(stop, nullptr));
  HIP_OK(hipEventSynchronize(stop));
  float ms = 0.0f;
  HIP_OK(hipEventElapsedTime(&ms, start, stop));
  HIP_OK(hipEventDestroy(start));
  HIP_OK(hipEventDestroy(stop));
  return ms / steps;
}

float half_to_float(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h >> 15) << 31, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
  uint32_t bits;
  if (exp == 0x1f) bits = sign | 0x7f800000u | (man << 13);
  else if (exp == 0) {
    const float v = std::ldexp(static_cast<float>(man), -24);
    return sign ? -v : v;
  } else bits = sign | ((exp + 112u) << 23) | (man << 13);
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// Largest |D_vendor - D_ours| / bound over all problems (<= 1 passes), and whether any D is NaN.
struct Check {
  double worst_ratio = 0.0;
  double max_abs_diff = 0.0;
  int worst_problem = -1;
  bool nan = false;
};

Check compare(const Spec& s, const Pools& p, const std::vector<int>& skipped_mask) {
  std::vector<uint16_t> a(p.a_n), b(p.b_n);
  std::vector<float> c(s.c == "uniform" ? p.c_n : 0), d0(p.d_n), d1(p.d_n);
  HIP_OK(hipMemcpy(a.data(), p.a, a.size() * 2, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(b.data(), p.b, b.size() * 2, hipMemcpyDeviceToHost));
  if (!c.empty()) HIP_OK(hipMemcpy(c.data(), p.c, c.size() * 4, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(d0.data(), p.d_ours, d0.size() * 4, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(d1.data(), p.d_vendor, d1.size() * 4, hipMemcpyDeviceToHost));
  Check out;
  for (size_t i = 0; i < s.m.size(); ++i) {
    if (skipped_mask[i] || s.m[i] == 0 || s.n[i] == 0) continue;
    double max_a = 0, max_b = 0, max_c = 0;
    for (int64_t e = 0; e < elems(s.m[i], s.k[i]); ++e) max_a = std::max(max_a, (double)std::fabs(half_to_float(a[p.a_off[i] + e])));
    for (int64_t e = 0; e < elems(s.k[i], s.n[i]); ++e) max_b = std::max(max_b, (double)std::fabs(half_to_float(b[p.b_off[i] + e])));
    if (!c.empty())
      for (int64_t e = 0; e < elems(s.m[i], s.n[i]); ++e) max_c = std::max(max_c, (double)std::fabs(c[p.c_off[i] + e]));
    const double bound = 2.0 * (1e-3 * std::sqrt(std::max(s.k[i], 1)) * max_a * max_b * std::fabs(s.alpha[i]) +
                                1e-6 * (std::fabs(s.beta[i]) * max_c + 1.0));
    for (int64_t e = 0; e < static_cast<int64_t>(s.m[i]) * s.n[i]; ++e) {
      const float x = d0[p.d_off[i] + e], y = d1[p.d_off[i] + e];
      if (std::isnan(x) || std::isnan(y)) {
        out.nan = true;
        out.worst_problem = static_cast<int>(i);
        continue;
      }
      const double diff = std::fabs(static_cast<double>(x) - y);
      out.max_abs_diff = std::max(out.max_abs_diff, diff);
      if (diff / bound > out.worst_ratio) out.worst_ratio = diff / bound, out.worst_problem = static_cast<int>(i);
    }
  }
  return out;
}

std::string json_escape(const std::string& s) {
  std::string o;
  for (char ch : s) {
    if (ch == '"' || ch == '\\') o += '\\';
    if (static_cast<unsigned char>(ch) >= 0x20) o += ch;
  }
  return o;
}

// One problem in hipBLASLt's terms.
struct Matmul {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr, ld = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  const void *a = nullptr, *b = nullptr, *c = nullptr;
  void* d = nullptr;
  float alpha = 1.0f, beta = 0.0f;
};

struct Vendor {
  hipblasLtHandle_t handle = nullptr;
  std::vector<Matmul> mm;
  void* workspace = nullptr;
  size_t workspace_bytes = 128u << 20;
  std::string error;
  ~Vendor() {
    for (Matmul& x : mm) {
      if (x.la) hipblasLtMatrixLayoutDestroy(x.la);
      if (x.lb) hipblasLtMatrixLayoutDestroy(x.lb);
      if (x.lc) hipblasLtMatrixLayoutDestroy(x.lc);
      if (x.ld) hipblasLtMatrixLayoutDestroy(x.ld);
      if (x.desc) hipblasLtMatmulDescDestroy(x.desc);
    }
    if (workspace) (void)hipFree(workspace);
    if (handle) hipblasLtDestroy(handle);
  }
};

bool vendor_setup(const std::vector<gg::ProblemDesc>& problems, Vendor* v, std::vector<int>* skipped) {
  if (hipblasLtCreate(&v->handle) != HIPBLAS_STATUS_SUCCESS) return v->error = "hipblasLtCreate failed", false;
  HIP_OK(hipMalloc(&v->workspace, v->workspace_bytes));
  for (size_t i = 0; i < problems.size(); ++i) {
    const gg::ProblemDesc& p = problems[i];
    if (p.m == 0 || p.n == 0) {
      (*skipped)[i] = 1;
      continue;
    }
    if (p.k <= 0) return v->error = "k <= 0 is not accepted by hipBLASLt", false;
    const bool reads_c = p.c != nullptr && p.beta != 0.0f;
    Matmul x;
    x.a = p.b, x.b = p.a, x.c = reads_c ? static_cast<const void*>(p.c) : p.d, x.d = p.d;
    x.alpha = p.alpha, x.beta = reads_c ? p.beta : 0.0f;
    hipblasLtMatmulDescCreate(&x.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    const hipblasOperation_t op = HIPBLAS_OP_N;
    hipblasLtMatmulDescSetAttribute(x.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op, sizeof(op));
    hipblasLtMatmulDescSetAttribute(x.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op, sizeof(op));
    hipblasLtMatrixLayoutCreate(&x.la, HIP_R_16F, p.n, p.k, p.ldb);
    hipblasLtMatrixLayoutCreate(&x.lb, HIP_R_16F, p.k, p.m, p.lda);
    hipblasLtMatrixLayoutCreate(&x.lc, HIP_R_32F, p.n, p.m, reads_c ? p.ldc : p.ldd);
    hipblasLtMatrixLayoutCreate(&x.ld, HIP_R_32F, p.n, p.m, p.ldd);
    v->mm.push_back(x);
  }
  return true;
}

// Per-problem form: each problem on its heuristic's first algorithm.
bool per_problem_setup(Vendor* v) {
  hipblasLtMatmulPreference_t pref = nullptr;
  hipblasLtMatmulPreferenceCreate(&pref);
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &v->workspace_bytes,
                                        sizeof(v->workspace_bytes));
  bool ok = true;
  for (Matmul& x : v->mm) {
    hipblasLtMatmulHeuristicResult_t r{};
    int returned = 0;
    if (hipblasLtMatmulAlgoGetHeuristic(v->handle, x.desc, x.la, x.lb, x.lc, x.ld, pref, 1, &r, &returned) !=
            HIPBLAS_STATUS_SUCCESS ||
        returned == 0) {
      v->error = "no hipblasLtMatmul algorithm for a problem";
      ok = false;
      break;
    }
    x.algo = r.algo;
  }
  hipblasLtMatmulPreferenceDestroy(pref);
  return ok;
}

int per_problem_run(Vendor* v) {
  for (Matmul& x : v->mm) {
    if (hipblasLtMatmul(v->handle, x.desc, &x.alpha, x.a, x.la, x.b, x.lb, &x.beta, x.c, x.lc, x.d, x.ld, &x.algo,
                        v->workspace, v->workspace_bytes, nullptr) != HIPBLAS_STATUS_SUCCESS) {
      return 1;
    }
  }
  return 0;
}

// Strided-batched form, for sets whose problems all have the same shape,
// leading dimensions and scalars and sit at evenly spaced addresses (uniform
// sets such as 64 x 2048^3): one hipblasLtMatmul over the whole batch, the
// best of up to max_algos heuristic candidates.  Returns false (and a reason)
// when the set is not uniform.
struct Batched {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr, ld = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  std::string solution;
  ~Batched() {
    if (la) hipblasLtMatrixLayoutDestroy(la);
    if (lb) hipblasLtMatrixLayoutDestroy(lb);
    if (lc) hipblasLtMatrixLayoutDestroy(lc);
    if (ld) hipblasLtMatrixLayoutDestroy(ld);
    if (desc) hipblasLtMatmulDescDestroy(desc);
  }
};

bool uniform_set(const std::vector<gg::ProblemDesc>& ps, std::string* why) {
  if (ps.size() < 2) return *why = "fewer than two problems", false;
  const gg::ProblemDesc& p0 = ps[0];
  if (p0.m <= 0 || p0.n <= 0 || p0.k <= 0) return *why = "empty problem", false;
  auto gap = [](const void* x, const void* y) {
    return reinterpret_cast<const char*>(y) - reinterpret_cast<const char*>(x);
  };
  const bool with_c = p0.c != nullptr && p0.beta != 0.0f;
  for (size_t i = 1; i < ps.size(); ++i) {
    const gg::ProblemDesc& p = ps[i];
    const gg::ProblemDesc& q = ps[i - 1];
    if (p.m != p0.m || p.n != p0.n || p.k != p0.k || p.lda != p0.lda || p.ldb != p0.ldb || p.ldc != p0.ldc ||
        p.ldd != p0.ldd || p.alpha != p0.alpha || p.beta != p0.beta || (p.c != nullptr) != (p0.c != nullptr)) {
      return *why = "problems differ", false;
    }
    if (gap(q.a, p.a) != gap(p0.a, ps[1].a) || gap(q.b, p.b) != gap(p0.b, ps[1].b) ||
        gap(q.d, p.d) != gap(p0.d, ps[1].d) || (with_c && gap(q.c, p.c) != gap(p0.c, ps[1].c))) {
      return *why = "uneven spacing", false;
    }
  }
  return true;
}

struct Result {
  std::string error, solution;
  float ms = -1.0f;
  int candidates = 0;
  Check check;
  bool checked = false;
};

std::string result_json(const char* mode, const Result& r, double flops) {
  std::ostringstream o;
  o << "{\"mode\": \"" << mode << "\"";
  if (!r.error.empty()) {
    o << ", \"error\": \"" << json_escape(r.error) << "\"}";
    return o.str();
  }
  o << ", \"kernel_ms\": " << r.ms << ", \"tflops\": " << (flops / (r.ms * 1e-3) / 1e12);
  if (!r.solution.empty()) o << ", \"solution\": \"" << json_escape(r.solution) << "\"";
  if (r.candidates) o << ", \"candidates_timed\": " << r.candidates;
  if (r.checked) {
    o << ", \"check_vs_library\": {\"max_abs_diff\": " << r.check.max_abs_diff
      << ", \"worst_fraction_of_bound\": " << r.check.worst_ratio << ", \"nan\": " << (r.check.nan ? "true" : "false")
      << ", \"pass\": " << ((!r.check.nan && r.check.worst_ratio <= 1.0) ? "true" : "false") << "}";
  }
  o << "}";
  return o.str();
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: %s SPEC [--steps N] [--warmup N] [--max-algos N] [--no-check] "
                         "[--config 128x64x32] [--sort-mode M]\n", argv[0]);
    return 2;
  }
  int steps = 20, warmup = 5, max_algos = 16, sort_mode = 1;
  bool check = true;
  gg::KernelConfig cfg{128, 64, 32, 256, 0, true};
  for (int i = 2; i < argc; ++i) {
    const std::string a = argv[i];
    auto next = [&]() -> std::string { return i + 1 < argc ? argv[++i] : std::string(); };
    if (a == "--steps") steps = std::max(1, std::atoi(next().c_str()));
    else if (a == "--warmup") warmup = std::max(0, std::atoi(next().c_str()));
    else if (a == "--max-algos") max_algos = std::max(1, std::atoi(next().c_str()));
    else if (a == "--no-check") check = false;
    else if (a == "--sort-mode") sort_mode = std::atoi(next().c_str());
    else if (a == "--config") {
      const std::string v = next();
      if (std::sscanf(v.c_str(), "%dx%dx%d", &cfg.cta_m, &cfg.cta_n, &cfg.cta_k) != 3) return 2;
    } else {
      std::fprintf(stderr, "unknown option %s\n", a.c_str());
      return 2;
    }
  }
  Spec spec;
  if (!read_spec(argv[1], &spec)) {
    std::printf("{\"error\": \"unreadable spec %s\"}\n", json_escape(argv[1]).c_str());
    return 1;
  }
  double flops = 0.0;
  for (size_t i = 0; i < spec.m.size(); ++i) flops += 2.0 * spec.m[i] * static_cast<double>(spec.n[i]) * spec.k[i];
  Pools pools;
  make_pools(spec, &pools);

  // This library: the reference answer for the check and a same-process timing.
  const std::vector<gg::ProblemDesc> ours = problems_for(spec, pools, pools.d_ours);
  const gg::PreparedProblemSet prepared = gg::prepare_problem_set(ours, cfg, static_cast<gg::SortMode>(sort_mode));
  gg::GroupedGemmExecutor executor;
  HIP_OK(executor.build(prepared, cfg));
  HIP_OK(executor.run(nullptr));
  HIP_OK(hipDeviceSynchronize());
  const float ours_ms = time_ms(steps, warmup, [&] { return static_cast<int>(executor.run(nullptr)); });

  const std::vector<gg::ProblemDesc> theirs = problems_for(spec, pools, pools.d_vendor);
  std::vector<int> skipped(spec.m.size(), 0);
  Result grouped, singles;
  Vendor v;
  bool ready = false;
  try {
    ready = vendor_setup(theirs, &v, &skipped);
  } catch (const std::exception& e) {
    v.error = std::string("hipBLASLt raised: ") + e.what();
  }
  if (!ready) grouped.error = singles.error = v.error;

  if (ready) {  // grouped form
    try {
      const hipDataType ab = HIP_R_16F, cd = HIP_R_32F;
      hipblaslt_ext::GroupedGemm group(v.handle, HIPBLAS_OP_N, HIPBLAS_OP_N, ab, ab, cd, cd, HIPBLAS_COMPUTE_32F);
      const size_t cnt = v.mm.size();
      std::vector<int64_t> m(cnt), n(cnt), k(cnt), batch(cnt, 1), lda(cnt), ldb(cnt), ldc(cnt), ldd(cnt), sa(cnt),
          sb(cnt), sc(cnt), sd(cnt);
      std::vector<hipblaslt_ext::GemmEpilogue> epilogue(cnt);
      std::vector<hipblaslt_ext::GemmInputs> inputs(cnt);
      size_t j = 0;
      for (size_t i = 0; i < theirs.size(); ++i) {
        if (skipped[i]) continue;
        const gg::ProblemDesc& p = theirs[i];
        const Matmul& x = v.mm[j];
        m[j] = p.n, n[j] = p.m, k[j] = p.k;
        const bool reads_c = x.c != x.d;
        lda[j] = p.ldb, ldb[j] = p.lda, ldc[j] = reads_c ? p.ldc : p.ldd, ldd[j] = p.ldd;
        sa[j] = lda[j] * p.k, sb[j] = ldb[j] * p.m, sc[j] = ldc[j] * p.m, sd[j] = ldd[j] * p.m;
        inputs[j].setA(x.a), inputs[j].setB(x.b), inputs[j].setC(x.c), inputs[j].setD(x.d);
        inputs[j].setAlpha(&x.alpha), inputs[j].setBeta(&x.beta);
        ++j;
      }
      hipblaslt_ext::GemmProblemType type(HIPBLAS_OP_N, HIPBLAS_OP_N, ab, ab, cd, cd, HIPBLAS_COMPUTE_32F);
      hipblasStatus_t st = group.setProblem(m, n, k, batch, lda, ldb, ldc, ldd, sa, sb, sc, sd, epilogue, inputs, type);
      hipblaslt_ext::GemmPreference pref;
      pref.setMaxWorkspaceBytes(v.workspace_bytes);
      std::vector<hipblasLtMatmulHeuristicResult_t> heuristics;
      if (st != HIPBLAS_STATUS_SUCCESS) {
        grouped.error = "GroupedGemm::setProblem returned " + std::to_string(st);
      } else if ((st = group.algoGetHeuristic(max_algos, pref, heuristics)) != HIPBLAS_STATUS_SUCCESS ||
                 heuristics.empty()) {
        grouped.error = "hipBLASLt grouped GEMM has no algorithm for this problem set (status " +
                        std::to_string(st) + ")";
      } else {
        int best = -1;
        std::string why;
        for (size_t i = 0; i < heuristics.size(); ++i) {
          size_t ws = 0;
          st = group.isAlgoSupported(heuristics[i].algo, ws);
          if (st != HIPBLAS_STATUS_SUCCESS || ws > v.workspace_bytes) {
            why += " [" + std::to_string(i) + ": isAlgoSupported " + std::to_string(st) + ", workspace " +
                   std::to_string(ws) + "]";
            continue;
          }
          st = group.initialize(heuristics[i].algo, v.workspace, /*useUserArgs=*/false);
          if (st != HIPBLAS_STATUS_SUCCESS) {
            why += " [" + std::to_string(i) + ": initialize " + std::to_string(st) + "]";
            continue;
          }
          const float ms = time_ms(std::max(1, std::min(steps, 10)), 2, [&] { return group.run(nullptr) == HIPBLAS_STATUS_SUCCESS ? 0 : 1; });
          ++grouped.candidates;
          if (ms > 0 && (best < 0 || ms < grouped.ms)) best = static_cast<int>(i), grouped.ms = ms;
          if (ms <= 0) why += " [" + std::to_string(i) + ": run failed]";
        }
        if (best < 0) {
          grouped.error = "no hipBLASLt grouped algorithm could be run:" + why;
        } else {
          group.initialize(heuristics[best].algo, v.workspace, /*useUserArgs=*/false);
          grouped.solution = group.getSolutionName();
          HIP_OK(ggk_fill_f32(pools.d_vendor, std::max<int64_t>(pools.d_n, 1), NAN, nullptr));
          if (group.run(nullptr) != HIPBLAS_STATUS_SUCCESS) grouped.error = "GroupedGemm::run failed";
          HIP_OK(hipDeviceSynchronize());
          if (grouped.error.empty() && check) grouped.check = compare(spec, pools, skipped), grouped.checked = true;
          if (grouped.error.empty())
            grouped.ms = time_ms(steps, warmup, [&] { return group.run(nullptr) == HIPBLAS_STATUS_SUCCESS ? 0 : 1; });
        }
      }
    } catch (const std::exception& e) {
      grouped.error = std::string("hipBLASLt raised: ") + e.what();
    }
  }

  if (ready) {  // per-problem form
    try {
      if (!per_problem_setup(&v)) {
        singles.error = v.error;
      } else {
        singles.solution = "hipblasLtMatmul per problem (heuristic first choice)";
        if (!v.mm.empty())
          singles.solution += "; first problem: " + hipblaslt_ext::getSolutionNameFromAlgo(v.handle, v.mm[0].algo);
        HIP_OK(ggk_fill_f32(pools.d_vendor, std::max<int64_t>(pools.d_n, 1), NAN, nullptr));
        if (per_problem_run(&v) != 0) singles.error = "hipblasLtMatmul failed";
        HIP_OK(hipDeviceSynchronize());
        if (singles.error.empty() && check) singles.check = compare(spec, pools, skipped), singles.checked = true;
        if (singles.error.empty())
          singles.ms = time_ms(std::max(1, std::min(steps, 20)), 2, [&] { return per_problem_run(&v); });
      }
    } catch (const std::exception& e) {
      singles.error = std::string("hipBLASLt raised: ") + e.what();
    }
  }

  Result batched;  // strided-batched form (uniform sets only)
  if (ready) {
    std::string why;
    if (!uniform_set(theirs, &why)) {
      batched.error = "not a uniform set: " + why;
    } else {
      try {
        const gg::ProblemDesc& p = theirs[0];
        const bool reads_c = p.c != nullptr && p.beta != 0.0f;
        const int64_t count = static_cast<int64_t>(theirs.size());
        auto stride = [](const void* x, const void* y, int64_t elem) {
          return (reinterpret_cast<const char*>(y) - reinterpret_cast<const char*>(x)) / elem;
        };
        const int64_t sa = stride(theirs[0].b, theirs[1].b, 2), sb = stride(theirs[0].a, theirs[1].a, 2);
        const int64_t sd = stride(theirs[0].d, theirs[1].d, 4);
        const int64_t sc = reads_c ? stride(theirs[0].c, theirs[1].c, 4) : sd;
        Batched bt;
        hipblasLtMatmulDescCreate(&bt.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
        const hipblasOperation_t op = HIPBLAS_OP_N;
        hipblasLtMatmulDescSetAttribute(bt.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op, sizeof(op));
        hipblasLtMatmulDescSetAttribute(bt.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op, sizeof(op));
        hipblasLtMatrixLayoutCreate(&bt.la, HIP_R_16F, p.n, p.k, p.ldb);
        hipblasLtMatrixLayoutCreate(&bt.lb, HIP_R_16F, p.k, p.m, p.lda);
        hipblasLtMatrixLayoutCreate(&bt.lc, HIP_R_32F, p.n, p.m, reads_c ? p.ldc : p.ldd);
        hipblasLtMatrixLayoutCreate(&bt.ld, HIP_R_32F, p.n, p.m, p.ldd);
        const int32_t batch = static_cast<int32_t>(count);
        for (auto [layout, st] : {std::pair{bt.la, sa}, std::pair{bt.lb, sb}, std::pair{bt.lc, sc}, std::pair{bt.ld, sd}}) {
          hipblasLtMatrixLayoutSetAttribute(layout, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &batch, sizeof(batch));
          hipblasLtMatrixLayoutSetAttribute(layout, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &st, sizeof(st));
        }
        hipblasLtMatmulPreference_t pref = nullptr;
        hipblasLtMatmulPreferenceCreate(&pref);
        hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &v.workspace_bytes,
                                              sizeof(v.workspace_bytes));
        std::vector<hipblasLtMatmulHeuristicResult_t> cand(std::max(1, max_algos));
        int returned = 0;
        const float alpha = p.alpha, beta = reads_c ? p.beta : 0.0f;
        const void* c_ptr = reads_c ? static_cast<const void*>(p.c) : p.d;
        if (hipblasLtMatmulAlgoGetHeuristic(v.handle, bt.desc, bt.la, bt.lb, bt.lc, bt.ld, pref,
                                            static_cast<int>(cand.size()), cand.data(), &returned) !=
                HIPBLAS_STATUS_SUCCESS ||
            returned == 0) {
          batched.error = "no strided-batched algorithm";
        } else {
          auto run_with = [&](const hipblasLtMatmulAlgo_t& algo) {
            return hipblasLtMatmul(v.handle, bt.desc, &alpha, p.b, bt.la, p.a, bt.lb, &beta, c_ptr, bt.lc, p.d, bt.ld,
                                   &algo, v.workspace, v.workspace_bytes, nullptr) == HIPBLAS_STATUS_SUCCESS
                       ? 0
                       : 1;
          };
          int best = -1;
          for (int i = 0; i < returned; ++i) {
            const float ms = time_ms(std::max(1, std::min(steps, 10)), 2, [&] { return run_with(cand[i].algo); });
            ++batched.candidates;
            if (ms > 0 && (best < 0 || ms < batched.ms)) best = i, batched.ms = ms;
          }
          if (best < 0) {
            batched.error = "no strided-batched algorithm could be run";
          } else {
            bt.algo = cand[best].algo;
            batched.solution = hipblaslt_ext::getSolutionNameFromAlgo(v.handle, bt.algo);
            HIP_OK(ggk_fill_f32(pools.d_vendor, std::max<int64_t>(pools.d_n, 1), NAN, nullptr));
            if (run_with(bt.algo) != 0) batched.error = "strided-batched hipblasLtMatmul failed";
            HIP_OK(hipDeviceSynchronize());
            if (batched.error.empty() && check) batched.check = compare(spec, pools, skipped), batched.checked = true;
            if (batched.error.empty()) batched.ms = time_ms(steps, warmup, [&] { return run_with(bt.algo); });
          }
        }
        hipblasLtMatmulPreferenceDestroy(pref);
      } catch (const std::exception& e) {
        batched.error = std::string("hipBLASLt raised: ") + e.what();
      }
    }
  }

  std::printf("{\"problems\": %zu, \"gflop\": %.3f, \"library\": {\"mode\": \"%s\", \"kernel_ms\": %g, \"tflops\": %g}, "
              "\"vendor\": [%s, %s, %s]}\n",
              spec.m.size(), flops / 1e9, gg::sort_mode_name(static_cast<gg::SortMode>(sort_mode)), ours_ms,
              flops / (ours_ms * 1e-3) / 1e12, result_json("hipblaslt_grouped", grouped, flops).c_str(),
              result_json("hipblaslt_per_problem", singles, flops).c_str(),
              result_json("hipblaslt_strided_batched", batched, flops).c_str());
  HIP_OK(hipFree(pools.a));
  HIP_OK(hipFree(pools.b));
  HIP_OK(hipFree(pools.c));
  HIP_OK(hipFree(pools.d_ours));
  HIP_OK(hipFree(pools.d_vendor));
  return 0;
}
