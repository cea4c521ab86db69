// gg_moe.hip -- device-resident preparation of a mixture-of-experts group.
//
// The host prepare path (prepare_problem_set + GroupedGemmExecutor::build,
// src/grouped_gemm.cu:967-1022 and :1178-1239 in the reference) needs the
// problem shapes on the host.  In MoE use the shapes are the per-expert token
// counts, which a router produces on the GPU.  This kernel turns them into
// the same prepared set -- descriptors in the sort mode's order, reference
// tile offsets, work-tile offsets, the permutation, the per-XCD chunk bounds
// -- in one workgroup, so the grouped launch can follow in stream order with
// no host round trip.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "grouped_gemm_amd_kernels.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kWave = 64;
constexpr int kWaves = kThreads / kWave;
constexpr int kChunks = GGK_SCHEDULER_CHUNKS;
constexpr int kMaxExperts = GGK_MOE_MAX_EXPERTS;
static_assert(kMaxExperts <= kThreads, "one thread per expert");
static_assert(kWaves <= kWave, "wave totals are scanned by one wave");
static_assert(2 + kChunks < GGK_MOE_STATUS && GGK_MOE_STATUS < GGK_MOE_HEADER_INTS, "header layout");

struct MoeArgs {
  ggk_moe_layout layout;
  const int* counts;
  int sort_mode;
  int cta_m, cta_n;      // reference macro-tile
  int work_tm, work_tn;  // reference tiles per work tile
  gg_device_problem_desc* problems;
  int* offsets;
  int* perm;
  int* header;
};

// Exclusive prefix sum of one value per thread over the workgroup, in thread
// order; *total receives the sum.  Every thread must call it.
template <class T>
__device__ T block_exclusive_scan(T v, T* s_waves, T* total) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  T x = v;
  for (int d = 1; d < kWave; d *= 2) {
    const T y = __shfl_up(x, d, kWave);
    if (lane >= d) x += y;
  }
  T before_lane = __shfl_up(x, 1, kWave);
  if (lane == 0) before_lane = T(0);
  if (lane == kWave - 1) s_waves[wave] = x;
  __syncthreads();
  if (wave == 0) {
    T w = lane < kWaves ? s_waves[lane] : T(0);
    for (int d = 1; d < kWaves; d *= 2) {
      const T y = __shfl_up(w, d, kWave);
      if (lane >= d) w += y;
    }
    if (lane < kWaves) s_waves[lane] = w;
  }
  __syncthreads();
  const T before_wave = wave > 0 ? s_waves[wave - 1] : T(0);
  *total = s_waves[kWaves - 1];
  __syncthreads();  // s_waves may be reused once every thread has read it
  return before_wave + before_lane;
}

__global__ __launch_bounds__(kThreads) void moe_prepare_kernel(MoeArgs args) {
  __shared__ long long s_waves_ll[kWaves];
  __shared__ int s_waves_i[kWaves];
  __shared__ double s_waves_d[kWaves];
  __shared__ int s_rows[kMaxExperts];
  __shared__ long long s_row0[kMaxExperts];
  __shared__ int s_tiles[kMaxExperts];
  __shared__ int s_perm[kMaxExperts];
  __shared__ int s_work_off[kMaxExperts + 1];
  __shared__ double s_cum[kMaxExperts];   // cost of the work tiles before sorted position i
  __shared__ double s_cost[kMaxExperts];  // cost of one work tile of sorted position i
  __shared__ int s_bounds[kChunks + 1];
  __shared__ int s_status;

  const ggk_moe_layout& L = args.layout;
  const int experts = L.experts;
  const int tid = threadIdx.x;
  if (tid == 0) s_status = 0;
  __syncthreads();

  // Rows of each expert: counts clamped to >= 0, origins by prefix sum, and
  // nothing at or past max_rows.
  int count = 0;
  if (tid < experts) {
    count = args.counts[tid];
    if (count < 0) {
      count = 0;
      atomicOr(&s_status, GGK_MOE_NEGATIVE);
    }
  }
  long long all_rows;
  const long long row0 = block_exclusive_scan<long long>(count, s_waves_ll, &all_rows);
  const int tiles_n = L.n > 0 ? (L.n + args.cta_n - 1) / args.cta_n : 0;
  if (tid < experts) {
    const long long room = (long long)L.max_rows - row0;
    const int rows = room <= 0 ? 0 : ((long long)count < room ? count : (int)room);
    if (rows < count) atomicOr(&s_status, GGK_MOE_CLAMPED);
    s_rows[tid] = rows;
    s_row0[tid] = row0;
    s_perm[tid] = tid;  // every slot holds a valid expert even before the ranks land
    const int tiles_m = rows > 0 && tiles_n > 0 ? (rows + args.cta_m - 1) / args.cta_m : 0;
    s_tiles[tid] = tiles_m * tiles_n;
  }
  __syncthreads();

  // Stable rank under the reference comparators (src/grouped_gemm.cu:977-993):
  // by K, larger k first, then larger m * n; by tiles, more tiles first, then
  // the by-K order.  Every expert has the same k here, so ties fall to m * n,
  // then to the expert index.
  if (tid < experts) {
    int rank = tid;
    if (args.sort_mode != 0) {
      const bool tiles_first = args.sort_mode == 2 || args.sort_mode == 3;
      const int my_tiles = s_tiles[tid];
      const long long my_area = (long long)s_rows[tid] * L.n;
      rank = 0;
      for (int j = 0; j < experts; ++j) {
        const int t = s_tiles[j];
        const long long area = (long long)s_rows[j] * L.n;
        const bool by_tiles = tiles_first && t != my_tiles;
        const bool before = by_tiles ? t > my_tiles : area > my_area;
        const bool tie = !by_tiles && area == my_area;
        rank += (before || (tie && j < tid)) ? 1 : 0;
      }
    }
    s_perm[rank] = tid;
  }
  __syncthreads();

  // Sorted order: offsets, descriptors, permutation.
  const int pos = tid;
  int ex = 0, rows = 0, tiles = 0, work = 0, tiles_m = 0;
  if (pos < experts) {
    ex = s_perm[pos];
    rows = s_rows[ex];
    tiles = s_tiles[ex];
    tiles_m = tiles > 0 ? tiles / tiles_n : 0;
    work = tiles > 0 ? ((tiles_m + args.work_tm - 1) / args.work_tm) * ((tiles_n + args.work_tn - 1) / args.work_tn)
                     : 0;
  }
  int total_tiles, total_work;
  const int tile_off = block_exclusive_scan<int>(tiles, s_waves_i, &total_tiles);
  const int work_off = block_exclusive_scan<int>(work, s_waves_i, &total_work);
  const bool reads_c = L.c != nullptr && L.beta != 0.0f;
  if (pos < experts) {
    args.offsets[pos] = tile_off;
    args.offsets[experts + 1 + pos] = work_off;
    s_work_off[pos] = work_off;
    args.perm[pos] = ex;
    const long long r0 = s_row0[ex];
    gg_device_problem_desc p;
    p.m = rows;
    p.n = L.n;
    p.k = L.k;
    p.a = static_cast<const uint16_t*>(L.a) + r0 * L.lda;
    p.b = static_cast<const uint16_t*>(L.b) + (long long)ex * L.stride_b;
    p.c = L.c != nullptr ? L.c + r0 * L.ldc : nullptr;
    p.d = L.d + r0 * L.ldd;
    p.lda = L.lda;
    p.ldb = L.ldb;
    p.ldc = L.ldc;
    p.ldd = L.ldd;
    p.alpha = L.alpha;
    p.beta = L.beta;
    p.tiles_m = tiles_m;
    p.tiles_n = tiles > 0 ? tiles_n : 0;
    args.problems[pos] = p;
  }
  if (pos == 0) {
    args.offsets[experts] = total_tiles;
    args.offsets[2 * experts + 1] = total_work;
    s_work_off[experts] = total_work;
  }

  // Chunk bounds by memory cost, as the host plan does: a work tile moves up to
  // (BM + BN) * k binary16 values in and BM * BN floats out (twice with C).
  double cost = 0.0;
  if (pos < experts) {
    const double r = (double)min(args.cta_m * args.work_tm, rows);
    const double c = (double)min(args.cta_n * args.work_tn, max(L.n, 0));
    cost = 2.0 * (r + c) * (double)max(L.k, 0) + 4.0 * r * c * (reads_c ? 2.0 : 1.0);
    s_cost[pos] = cost;
  }
  double sum;
  const double cum = block_exclusive_scan<double>(cost * (double)work, s_waves_d, &sum);
  if (pos < experts) s_cum[pos] = cum;
  __syncthreads();
  if (tid >= 1 && tid < kChunks) {
    // The first sorted position whose work tiles reach the target cost.
    const double target = sum * tid / kChunks;
    int lo = 0, hi = experts;  // answer in [lo, hi]; hi = experts means none
    while (lo < hi) {
      const int mid = (lo + hi) / 2;
      const double end = s_cum[mid] + s_cost[mid] * (double)(s_work_off[mid + 1] - s_work_off[mid]);
      if (end >= target) hi = mid;
      else lo = mid + 1;
    }
    int t = total_work;
    if (lo < experts) {
      const double into = s_cost[lo] > 0.0 ? (target - s_cum[lo]) / s_cost[lo] : 0.0;
      const double room = (double)(s_work_off[lo + 1] - s_work_off[lo]);
      t = s_work_off[lo] + (int)(into < room ? into : room);
    }
    s_bounds[tid] = t < total_work ? t : total_work;
  }
  __syncthreads();
  if (tid == 0) {
    int prev = 0;
    args.header[0] = total_tiles;
    args.header[1] = total_work;
    args.header[2] = 0;
    for (int c = 1; c < kChunks; ++c) {
      prev = s_bounds[c] > prev ? s_bounds[c] : prev;
      args.header[2 + c] = prev;
    }
    args.header[2 + kChunks] = total_work;
    for (int h = 3 + kChunks; h < GGK_MOE_HEADER_INTS; ++h) args.header[h] = 0;
    args.header[GGK_MOE_STATUS] = s_status;
  }
}

// Reference macro-tile of each variant (GGK_VARIANT_*).
constexpr int kCta[GGK_VARIANT_COUNT][2] = {{64, 64}, {128, 64}, {64, 128}, {128, 64}, {64, 128}};

}  // namespace

extern "C" hipError_t ggk_moe_prepare(int variant, int path, const ggk_moe_layout* layout, const int* d_counts,
                                      int sort_mode, gg_device_problem_desc* d_problems, int* d_offsets,
                                      int* d_sorted_to_original, int* d_header, hipStream_t stream) {
  if (layout == nullptr || variant < 0 || variant >= GGK_VARIANT_COUNT || sort_mode < 0 || sort_mode > 3) {
    return hipErrorInvalidValue;
  }
  ggk_work_shape work{};
  hipError_t st = ggk_work_shape_get(variant, path, &work);
  if (st != hipSuccess) return st;
  const ggk_moe_layout& L = *layout;
  const int n1 = L.n > 1 ? L.n : 1;
  const int k1 = L.k > 1 ? L.k : 1;
  if (L.experts < 1 || L.experts > GGK_MOE_MAX_EXPERTS || L.n < 0 || L.k < 0 || L.max_rows < 0 ||
      L.lda < k1 || L.ldb < n1 || L.ldd < n1 || L.stride_b < 0 || (L.c != nullptr && L.ldc < n1)) {
    return hipErrorInvalidValue;
  }
  // Every tile count and offset must fit an int, however the rows are split:
  // at most (max_rows / cta_m + experts) row tiles in all.
  const int cta_m = kCta[variant][0], cta_n = kCta[variant][1];
  const long long row_tiles = (long long)L.max_rows / cta_m + L.experts;
  const long long col_tiles = ((long long)L.n + cta_n - 1) / cta_n;
  if (row_tiles * col_tiles > 0x7fffffffLL) return hipErrorInvalidValue;
  if (L.a == nullptr || L.b == nullptr || L.d == nullptr || d_counts == nullptr || d_problems == nullptr ||
      d_offsets == nullptr || d_sorted_to_original == nullptr || d_header == nullptr) {
    return hipErrorInvalidDevicePointer;
  }
  MoeArgs args{L, d_counts, sort_mode, cta_m, cta_n, work.tiles_m, work.tiles_n, d_problems, d_offsets,
               d_sorted_to_original, d_header};
  void* params[] = {&args};
  return hipLaunchKernel(reinterpret_cast<const void*>(moe_prepare_kernel), dim3(1), dim3(kThreads), params, 0,
                         stream);
}
