/*
 * gg_oracle.h -- CPU oracle for the grouped FP16 GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library restates, in plain C, what the
 * reference implementation (Intersect-Suo/Grouped_GEMM_gpu_kernel) computes on
 * the grouped-GEMM path, so that the HIP library can be checked against it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it, and only as the expected answer or the timed CPU baseline.  The product library
 * (grouped_gemm_gpu_kernel_amd) never links, loads or calls it.
 *
 * Every function names the reference file:line it follows.  How each one is
 * pinned (known answers, closed forms, brute force, libstdc++ itself) is listed
 * beside it; none is "parity unpinned".
 */
#ifndef GG_ORACLE_H_
#define GG_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- IEEE-754 binary16 <-> binary32 (closed form). ----------------------
 * Reference inputs are produced with __float2half_rn (round to nearest even)
 * and read back with __half2float (tests/test_correctness.cu:94-95,143-147).
 * Pinned against numpy's float16 conversion over all 65536 half patterns and a
 * sweep of float32 values including every rounding tie. */
float go_f16_to_f32(uint16_t h);
uint16_t go_f32_to_f16_rne(float f);
void go_f32_to_f16_array(const float* src, uint16_t* dst, int64_t count);
void go_f16_to_f32_array(const uint16_t* src, float* dst, int64_t count);

/* ---- std::mt19937 and the libstdc++ (GCC 11) distributions. --------------
 * Used by the reference's test (tests/test_correctness.cu:114-150) and bench
 * (bench/benchmark_grouped_gemm.cu:368-443, 451-495) input generators.
 * Pinned by the C++ standard's known answer (10000th output of a default
 * seeded engine is 4123659995) and against libstdc++ itself. */
typedef struct go_mt19937 {
  uint32_t state[624];
  int index;
} go_mt19937;

void go_mt_seed(go_mt19937* mt, uint32_t seed);
uint32_t go_mt_next(go_mt19937* mt);
/* std::uniform_int_distribution<int>(lo, hi)(mt) as libstdc++ 11 computes it. */
int go_uniform_int(go_mt19937* mt, int lo, int hi);
/* std::uniform_real_distribution<float>(lo, hi)(mt) as libstdc++ 11 computes it. */
float go_uniform_real_f32(go_mt19937* mt, float lo, float hi);

/* Shapes of the reference benchmark's workloads "small", "tail", "mixed"
 * (bench/benchmark_grouped_gemm.cu:368-443), picks drawn k, n, m as the
 * reference binary draws them.  Returns 0, or -1 for an unknown workload name. */
int go_bench_shapes(const char* workload, int count, uint32_t seed, int* m, int* n, int* k);

/* The "small"/"mixed" recipe over caller-given candidate lists: per problem a
 * uniform pick for k, then n, then m.  Lets the published rows made with the
 * reference's earlier mixed lists (bench/benchmark_grouped_gemm.cu:409-411,
 * now commented out) be regenerated. */
void go_bench_shapes_lists(int count, uint32_t seed, const int* mv, int mc, const int* nv, int nc, const int* kv,
                           int kc, int* m, int* n, int* k);

/* The reference test's inputs (tests/test_correctness.cu:106-150): for each
 * shape draws alpha, beta, then A (m x max(1,k)), B (k x max(1,n)),
 * C (m x max(1,n)) from one mt19937(seed) stream with uniform_real(-1,1); A and
 * B are rounded to half.  A zero-sized matrix still consumes one draw
 * (safe_matrix_elems, tests/test_correctness.cu:75-80).  Output buffers are
 * laid out back to back per problem; the *_len arrays give the element counts.
 * Pass NULL data pointers to only query the lengths. */
void go_reference_test_inputs(int count, const int* m, const int* n, const int* k, uint32_t seed,
                              float* alpha, float* beta,
                              int64_t* a_len, int64_t* b_len, int64_t* c_len,
                              uint16_t* a, uint16_t* b, float* c);

/* ---- Host prepare path. -------------------------------------------------- */

/* tile_count_for_problem (src/grouped_gemm.cu:54-65). */
int go_tile_count(int m, int n, int cta_m, int cta_n);

/* prepare_problem_set (src/grouped_gemm.cu:967-1022): the stable sort
 * permutation for mode 0 none, 1 by K, 2 by tiles, 3 by tiles then K (which the
 * reference sorts with the same comparator as mode 2, :1000-1005), and the
 * exclusive prefix sum of tile counts in sorted order.  sorted_to_original has
 * count entries, tile_offsets count+1.  Returns total_tiles.
 * The sort is a hand-written stable merge sort; pinned against libstdc++'s
 * std::stable_sort and Python's sorted() with the same keys. */
int go_prepare(int count, const int* m, const int* n, const int* k, int cta_m, int cta_n, int mode,
               int* sorted_to_original, int* tile_offsets);

/* find_problem_by_tile (src/grouped_gemm.cu:219-234) restated as a linear
 * count: the number of problems p with tile_offsets[p+1] <= tile.  Pinned by
 * brute force against bisect.bisect_right. */
int go_find_problem(const int* tile_offsets, int count, int tile);

/* The whole tile -> (problem, tile_m, tile_n) map of grouped_gemm_kernel
 * (src/grouped_gemm.cu:659-668) for sorted per-problem tiles_n.
 * out has 3*total_tiles ints. */
void go_map_tiles(int count, const int* sorted_tiles_n, const int* tile_offsets, int* out);

/* Persistent grid size (src/grouped_gemm.cu:1228-1236). */
int go_grid_ctas(int total_tiles, int persistent_ctas, int sm_count, int active_blocks_per_sm);

/* ---- CPU reference GEMM (tests/test_correctness.cu:85-102). --------------
 * D[i][j] = alpha * acc + beta * C[i][j], acc = sum over kk ascending of
 * float(A[i][kk]) * float(B[kk][j]) in float32, each product and sum rounded
 * separately (this file is built with -ffp-contract=off).  C is read for every
 * element, as in the reference; a NULL C reads as 0.  Nothing is written when
 * m <= 0 or n <= 0.  Pinned by closed forms (K=0, identity, exactly
 * representable integer inputs against int64 arithmetic) and by float64
 * products within the rounding bound. */
void go_gemm(int m, int n, int k, const uint16_t* a, int lda, const uint16_t* b, int ldb,
             const float* c, int ldc, float alpha, float beta, float* d, int ldd);
/* Same per-element arithmetic in i-k-j order, rows spread over `threads`
 * OpenMP threads (0 = OpenMP default).  Bit-identical to go_gemm. */
void go_gemm_omp(int m, int n, int k, const uint16_t* a, int lda, const uint16_t* b, int ldb,
                 const float* c, int ldc, float alpha, float beta, float* d, int ldd, int threads);
/* One element (i, j) of go_gemm. */
float go_gemm_element(int i, int j, int k, const uint16_t* a, int lda, const uint16_t* b, int ldb,
                      const float* c, int ldc, float alpha, float beta);
/* count independent elements of go_gemm, each given as its own row of A and
 * column of B: element s takes k[s] values from a + a_start[s] and
 * b + b_start[s] (both contiguous), c[s] (c may be NULL: 0), alpha[s] and
 * beta[s], with go_gemm_element's arithmetic in the same order; results to
 * out[s].  Pinned against go_gemm bit for bit (tests/test_oracle.py). */
void go_gemm_samples(int count, const int* k, const uint16_t* a, const int64_t* a_start, const uint16_t* b,
                     const int64_t* b_start, const float* c, const float* alpha, const float* beta, float* out);

/* ---- Metric helpers (bench/benchmark_grouped_gemm.cu:570-607). ----------- */
double go_total_flops(int count, const int* m, const int* n, const int* k);
/* Static tail share: work = tiles * ceil(k / cta_k) per problem in sorted
 * order; share of the last max(1, count/10) problems. */
double go_tail_work_share(int count, const int* sorted_k, const int* tile_offsets, int cta_k);

int go_omp_max_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* GG_ORACLE_H_ */
