/*
 * gg_oracle.c -- CPU oracle for the grouped FP16 GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY: a plain-C restatement of the reference's
 * grouped-GEMM semantics: the expected answer for tests/ and
 * __graft_entry__.smoke(), and the timed CPU baseline in bench.py.  The
 * product library never links or calls it.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).  The FP32 GEMM
 * depends on -ffp-contract=off: every product and every sum is rounded on its
 * own, as in the reference's host loop.
 */
#include "gg_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* binary16 <-> binary32                                                     */
/* ------------------------------------------------------------------------ */

static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof(u));
  return u;
}

static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof(f));
  return f;
}

float go_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31;
  const uint32_t exp = (h >> 10) & 0x1f;
  const uint32_t man = h & 0x3ff;
  if (exp == 0x1f) {                      /* inf / nan: keep payload */
    return bits_f32(sign | 0x7f800000u | (man << 13));
  }
  if (exp == 0) {
    if (man == 0) return bits_f32(sign);  /* signed zero */
    /* subnormal: value = man * 2^-24, exact in float */
    float v = (float)man * (1.0f / 16777216.0f);
    return (h >> 15) ? -v : v;
  }
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t go_f32_to_f16_rne(float f) {
  const uint32_t u = f32_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
  const uint32_t abs = u & 0x7fffffffu;
  if (abs >= 0x7f800000u) {               /* inf or nan */
    if (abs == 0x7f800000u) return sign | 0x7c00;
    return sign | 0x7e00 | (uint16_t)((abs >> 13) & 0x3ff);  /* quiet nan */
  }
  const int e = (int)(abs >> 23) - 127;   /* unbiased exponent */
  if (e > 15) return sign | 0x7c00;       /* overflow before rounding */
  uint32_t mant;                          /* significand with the hidden bit */
  int shift;                              /* bits dropped to reach half precision */
  uint32_t base_exp;
  if (e >= -14) {                         /* normal half range */
    mant = (abs & 0x7fffff) | 0x800000;
    shift = 13;
    base_exp = (uint32_t)(e + 15);
  } else {                                /* subnormal half or underflow */
    if (e < -25) return sign;             /* below half of the smallest subnormal */
    mant = (abs & 0x7fffff) | (abs >= 0x00800000u ? 0x800000u : 0u);
    shift = 13 + (-14 - e);
    base_exp = 0;
  }
  uint32_t q = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1u;
  uint32_t out;
  if (base_exp == 0) {
    out = q;                              /* may carry into the smallest normal: correct encoding */
  } else {
    out = (base_exp << 10) + (q - 0x400u); /* q includes the hidden bit (0x400) */
    /* a carry out of the significand bumps the exponent; 0x7c00 means overflow to inf */
  }
  if (out >= 0x7c00) return sign | 0x7c00;
  return sign | (uint16_t)out;
}

void go_f32_to_f16_array(const float* src, uint16_t* dst, int64_t count) {
  for (int64_t i = 0; i < count; ++i) dst[i] = go_f32_to_f16_rne(src[i]);
}

void go_f16_to_f32_array(const uint16_t* src, float* dst, int64_t count) {
  for (int64_t i = 0; i < count; ++i) dst[i] = go_f16_to_f32(src[i]);
}

/* ------------------------------------------------------------------------ */
/* mt19937 (Matsumoto & Nishimura 1998, parameters as in [rand.predef])      */
/* ------------------------------------------------------------------------ */

enum { MT_N = 624, MT_M = 397 };

void go_mt_seed(go_mt19937* mt, uint32_t seed) {
  mt->state[0] = seed;
  for (int i = 1; i < MT_N; ++i) {
    const uint32_t prev = mt->state[i - 1];
    mt->state[i] = 1812433253u * (prev ^ (prev >> 30)) + (uint32_t)i;
  }
  mt->index = MT_N;
}

static void mt_twist(go_mt19937* mt) {
  for (int i = 0; i < MT_N; ++i) {
    const uint32_t y = (mt->state[i] & 0x80000000u) | (mt->state[(i + 1) % MT_N] & 0x7fffffffu);
    uint32_t v = mt->state[(i + MT_M) % MT_N] ^ (y >> 1);
    if (y & 1u) v ^= 0x9908b0dfu;
    mt->state[i] = v;
  }
  mt->index = 0;
}

uint32_t go_mt_next(go_mt19937* mt) {
  if (mt->index >= MT_N) mt_twist(mt);
  uint32_t y = mt->state[mt->index++];
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

/* libstdc++ 11 uniform_int_distribution: for a 32-bit engine and a range that
 * fits, Lemire's multiply-shift with rejection of the biased low words. */
int go_uniform_int(go_mt19937* mt, int lo, int hi) {
  const uint32_t urange = (uint32_t)hi - (uint32_t)lo;
  if (urange == 0xffffffffu) {
    return (int)((uint32_t)lo + go_mt_next(mt));
  }
  const uint32_t span = urange + 1u;
  uint64_t product = (uint64_t)go_mt_next(mt) * (uint64_t)span;
  uint32_t low = (uint32_t)product;
  if (low < span) {
    const uint32_t threshold = (uint32_t)(0u - span) % span;
    while (low < threshold) {
      product = (uint64_t)go_mt_next(mt) * (uint64_t)span;
      low = (uint32_t)product;
    }
  }
  return (int)((uint32_t)lo + (uint32_t)(product >> 32));
}

/* libstdc++ 11 uniform_real_distribution<float>: generate_canonical<float,24>
 * takes one 32-bit draw, converts it to float, divides by 2^32 and clamps a
 * result of 1 to the largest float below 1; then x * (hi - lo) + lo. */
float go_uniform_real_f32(go_mt19937* mt, float lo, float hi) {
  float r = (float)go_mt_next(mt) / 4294967296.0f;
  if (r >= 1.0f) r = nextafterf(1.0f, 0.0f);
  return r * (hi - lo) + lo;
}

static int pick(go_mt19937* mt, const int* values, int count) {
  return values[go_uniform_int(mt, 0, count - 1)];
}

/* bench/benchmark_grouped_gemm.cu:368-443.  The reference writes each shape as
 * out.emplace_back(pick(m_values), pick(n_values), pick(k_values)); C++ leaves
 * the order of those three calls open and the g++ host compiler makes them
 * right to left, so the engine is drawn for k, then n, then m.  The published
 * tail-workload tile totals (bench/results_20260331/results.csv:31-45,
 * 630/447/444 at 256 problems, seed 42) hold only in that order; m, n, k order
 * gives 668/467/468. */
void go_bench_shapes_lists(int count, uint32_t seed, const int* mv, int mc, const int* nv, int nc, const int* kv,
                           int kc, int* m, int* n, int* k) {
  go_mt19937 mt;
  go_mt_seed(&mt, seed);
  for (int i = 0; i < count; ++i) {
    k[i] = pick(&mt, kv, kc);
    n[i] = pick(&mt, nv, nc);
    m[i] = pick(&mt, mv, mc);
  }
}

int go_bench_shapes(const char* workload, int count, uint32_t seed, int* m, int* n, int* k) {
  if (strcmp(workload, "small") == 0) {
    static const int mv[] = {16, 24, 32, 48, 64};
    static const int nv[] = {16, 32, 48, 64, 96};
    static const int kv[] = {16, 24, 32, 48, 64};
    go_bench_shapes_lists(count, seed, mv, 5, nv, 5, kv, 5, m, n, k);
    return 0;
  }
  if (strcmp(workload, "mixed") == 0) {
    static const int v[] = {63, 94, 122, 240, 500};
    go_bench_shapes_lists(count, seed, v, 5, v, 5, v, 5, m, n, k);
    return 0;
  }
  go_mt19937 mt;
  go_mt_seed(&mt, seed);
  if (strcmp(workload, "tail") == 0) {
    static const int small_mn[] = {16, 24, 32, 48, 64};
    static const int large_mn[] = {96, 128, 160, 192, 256};
    static const int small_k[] = {16, 24, 32, 48, 64};
    static const int large_k[] = {96, 128, 192, 256, 384, 512};
    for (int i = 0; i < count; ++i) {
      if (go_uniform_real_f32(&mt, 0.0f, 1.0f) < 0.8f) {
        k[i] = pick(&mt, small_k, 5);
        n[i] = pick(&mt, small_mn, 5);
        m[i] = pick(&mt, small_mn, 5);
      } else {
        k[i] = pick(&mt, large_k, 6);
        n[i] = pick(&mt, large_mn, 5);
        m[i] = pick(&mt, large_mn, 5);
      }
    }
    return 0;
  }
  return -1;
}

static int64_t safe_elems(int rows, int cols) {
  if (rows <= 0 || cols <= 0) return 1;
  return (int64_t)rows * cols;
}

static int max1(int x) { return x > 1 ? x : 1; }

void go_reference_test_inputs(int count, const int* m, const int* n, const int* k, uint32_t seed,
                              float* alpha, float* beta,
                              int64_t* a_len, int64_t* b_len, int64_t* c_len,
                              uint16_t* a, uint16_t* b, float* c) {
  go_mt19937 mt;
  go_mt_seed(&mt, seed);
  int64_t ao = 0, bo = 0, co = 0;
  for (int p = 0; p < count; ++p) {
    const int lda = max1(k[p]), ldb = max1(n[p]), ldc = max1(n[p]);
    const int64_t na = safe_elems(m[p], lda), nb = safe_elems(k[p], ldb), nc = safe_elems(m[p], ldc);
    a_len[p] = na;
    b_len[p] = nb;
    c_len[p] = nc;
    if (a == NULL) continue;
    alpha[p] = go_uniform_real_f32(&mt, -1.0f, 1.0f);
    beta[p] = go_uniform_real_f32(&mt, -1.0f, 1.0f);
    for (int64_t i = 0; i < na; ++i) a[ao + i] = go_f32_to_f16_rne(go_uniform_real_f32(&mt, -1.0f, 1.0f));
    for (int64_t i = 0; i < nb; ++i) b[bo + i] = go_f32_to_f16_rne(go_uniform_real_f32(&mt, -1.0f, 1.0f));
    for (int64_t i = 0; i < nc; ++i) c[co + i] = go_uniform_real_f32(&mt, -1.0f, 1.0f);
    ao += na;
    bo += nb;
    co += nc;
  }
}

/* ------------------------------------------------------------------------ */
/* Host prepare path                                                         */
/* ------------------------------------------------------------------------ */

static int ceil_div_int(int x, int y) { return (x + y - 1) / y; }

int go_tile_count(int m, int n, int cta_m, int cta_n) {
  if (m <= 0 || n <= 0) return 0;
  return ceil_div_int(m, cta_m) * ceil_div_int(n, cta_n);
}

typedef struct sort_ctx {
  const int* m;
  const int* n;
  const int* k;
  const int* tiles;
  int mode;
} sort_ctx;

/* "lhs strictly before rhs" for the reference comparators:
 * by K: larger k first, then larger (int64) m*n (src/grouped_gemm.cu:977-984);
 * by tiles: more tiles first, then the by-K order (:986-993). */
static int goes_before(const sort_ctx* s, int lhs, int rhs) {
  if (s->mode == 2 || s->mode == 3) {
    if (s->tiles[lhs] != s->tiles[rhs]) return s->tiles[lhs] > s->tiles[rhs];
  }
  if (s->k[lhs] != s->k[rhs]) return s->k[lhs] > s->k[rhs];
  const int64_t la = (int64_t)s->m[lhs] * s->n[lhs];
  const int64_t ra = (int64_t)s->m[rhs] * s->n[rhs];
  return la > ra;
}

/* Stable bottom-up merge sort: on ties the left run wins. */
static void stable_sort_idx(const sort_ctx* s, int* idx, int count) {
  if (count < 2) return;
  int* tmp = (int*)malloc(sizeof(int) * (size_t)count);
  int* src = idx;
  int* dst = tmp;
  for (int width = 1; width < count; width *= 2) {
    for (int lo = 0; lo < count; lo += 2 * width) {
      int mid = lo + width < count ? lo + width : count;
      int hi = lo + 2 * width < count ? lo + 2 * width : count;
      int i = lo, j = mid, o = lo;
      while (i < mid && j < hi) {
        if (goes_before(s, src[j], src[i])) dst[o++] = src[j++];
        else dst[o++] = src[i++];
      }
      while (i < mid) dst[o++] = src[i++];
      while (j < hi) dst[o++] = src[j++];
    }
    int* t = src;
    src = dst;
    dst = t;
  }
  if (src != idx) memcpy(idx, src, sizeof(int) * (size_t)count);
  free(tmp);
}

int go_prepare(int count, const int* m, const int* n, const int* k, int cta_m, int cta_n, int mode,
               int* sorted_to_original, int* tile_offsets) {
  int* tiles = (int*)malloc(sizeof(int) * (size_t)(count > 0 ? count : 1));
  for (int i = 0; i < count; ++i) {
    tiles[i] = go_tile_count(m[i], n[i], cta_m, cta_n);
    sorted_to_original[i] = i;
  }
  if (mode == 1 || mode == 2 || mode == 3) {
    sort_ctx s = {m, n, k, tiles, mode};
    stable_sort_idx(&s, sorted_to_original, count);
  }
  tile_offsets[0] = 0;
  for (int i = 0; i < count; ++i) tile_offsets[i + 1] = tile_offsets[i] + tiles[sorted_to_original[i]];
  free(tiles);
  return tile_offsets[count];
}

int go_find_problem(const int* tile_offsets, int count, int tile) {
  int p = 0;
  while (p < count && tile_offsets[p + 1] <= tile) ++p;
  return p;
}

void go_map_tiles(int count, const int* sorted_tiles_n, const int* tile_offsets, int* out) {
  const int total = tile_offsets[count];
  int p = 0;
  for (int t = 0; t < total; ++t) {
    while (tile_offsets[p + 1] <= t) ++p;  /* offsets are non-decreasing and t < total */
    const int local = t - tile_offsets[p];
    out[3 * t + 0] = p;
    out[3 * t + 1] = local / sorted_tiles_n[p];
    out[3 * t + 2] = local % sorted_tiles_n[p];
  }
}

int go_grid_ctas(int total_tiles, int persistent_ctas, int sm_count, int active_blocks_per_sm) {
  if (total_tiles <= 0) return 0;
  int grid;
  if (persistent_ctas > 0) {
    grid = persistent_ctas;
  } else {
    const int resident = sm_count * (active_blocks_per_sm > 1 ? active_blocks_per_sm : 1);
    const int want = total_tiles > sm_count ? total_tiles : sm_count;
    grid = resident < want ? resident : want;
  }
  return grid > 1 ? grid : 1;
}

/* ------------------------------------------------------------------------ */
/* CPU reference GEMM                                                        */
/* ------------------------------------------------------------------------ */

float go_gemm_element(int i, int j, int k, const uint16_t* a, int lda, const uint16_t* b, int ldb,
                      const float* c, int ldc, float alpha, float beta) {
  float acc = 0.0f;
  for (int kk = 0; kk < k; ++kk) {
    const float av = go_f16_to_f32(a[(int64_t)i * lda + kk]);
    const float bv = go_f16_to_f32(b[(int64_t)kk * ldb + j]);
    const float prod = av * bv;
    acc = acc + prod;
  }
  const float cv = c != NULL ? c[(int64_t)i * ldc + j] : 0.0f;
  const float lhs = alpha * acc;
  const float rhs = beta * cv;
  return lhs + rhs;
}

void go_gemm_samples(int count, const int* k, const uint16_t* a, const int64_t* a_start, const uint16_t* b,
                     const int64_t* b_start, const float* c, const float* alpha, const float* beta, float* out) {
  for (int s = 0; s < count; ++s) {
    out[s] = go_gemm_element(0, 0, k[s], a + a_start[s], 1, b + b_start[s], 1, c != NULL ? c + s : NULL, 1,
                             alpha[s], beta[s]);
  }
}

void go_gemm(int m, int n, int k, const uint16_t* a, int lda, const uint16_t* b, int ldb,
             const float* c, int ldc, float alpha, float beta, float* d, int ldd) {
  if (m <= 0 || n <= 0) return;
  for (int i = 0; i < m; ++i) {
    for (int j = 0; j < n; ++j) {
      d[(int64_t)i * ldd + j] = go_gemm_element(i, j, k, a, lda, b, ldb, c, ldc, alpha, beta);
    }
  }
}

void go_gemm_omp(int m, int n, int k, const uint16_t* a, int lda, const uint16_t* b, int ldb,
                 const float* c, int ldc, float alpha, float beta, float* d, int ldd, int threads) {
  if (m <= 0 || n <= 0) return;
#ifdef _OPENMP
  const int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
  {
    float* acc = (float*)malloc(sizeof(float) * (size_t)n);
    float* brow = (float*)malloc(sizeof(float) * (size_t)n);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int i = 0; i < m; ++i) {
      for (int j = 0; j < n; ++j) acc[j] = 0.0f;
      for (int kk = 0; kk < k; ++kk) {
        const float av = go_f16_to_f32(a[(int64_t)i * lda + kk]);
        const uint16_t* br = b + (int64_t)kk * ldb;
        for (int j = 0; j < n; ++j) brow[j] = go_f16_to_f32(br[j]);
        for (int j = 0; j < n; ++j) {
          const float prod = av * brow[j];
          acc[j] = acc[j] + prod;
        }
      }
      for (int j = 0; j < n; ++j) {
        const float cv = c != NULL ? c[(int64_t)i * ldc + j] : 0.0f;
        const float lhs = alpha * acc[j];
        const float rhs = beta * cv;
        d[(int64_t)i * ldd + j] = lhs + rhs;
      }
    }
    free(acc);
    free(brow);
  }
}

/* ------------------------------------------------------------------------ */
/* Metric helpers                                                            */
/* ------------------------------------------------------------------------ */

double go_total_flops(int count, const int* m, const int* n, const int* k) {
  double flops = 0.0;
  for (int i = 0; i < count; ++i) flops += 2.0 * (double)m[i] * n[i] * k[i];
  return flops;
}

double go_tail_work_share(int count, const int* sorted_k, const int* tile_offsets, int cta_k) {
  if (count == 0) return 0.0;
  const int tail = count / 10 > 1 ? count / 10 : 1;
  double total = 0.0, tail_work = 0.0;
  for (int i = 0; i < count; ++i) {
    const int tiles = tile_offsets[i + 1] - tile_offsets[i];
    const int ksteps = ceil_div_int(sorted_k[i], cta_k);
    const double w = (double)tiles * ksteps;
    total += w;
    if (i >= count - tail) tail_work += w;
  }
  return total > 0.0 ? tail_work / total : 0.0;
}

int go_omp_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
