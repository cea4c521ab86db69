// gg_moe.hip -- device-resident preparation of a mixture-of-experts group.
//
// The host prepare path (prepare_problem_set + GroupedGemmExecutor::build,
// src/grouped_gemm.cu:967-1022 and :1178-1239 in the reference) needs the
// problem shapes on the host.  In MoE use the shapes are the per-expert token
// counts, which a router produces on the GPU.  This kernel turns them into
// the same prepared set -- descriptors in the sort mode's order, reference
// tile offsets, the permutation, and the schedule the host build would plan:
// the scheduling order, work-tile offsets in that order, the per-XCD chunk
// bounds -- in one workgroup, so the grouped launch can follow in stream
// order with no host round trip.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "grouped_gemm_amd.h"
#include "grouped_gemm_amd_kernels.h"

namespace {

// The prepare runs in one workgroup with one thread per expert: 1024 threads, or one wave for
// groups of at most 64 experts (no cross-wave scans; its barriers cost next to nothing).
constexpr int kThreads = 1024;
constexpr int kWave = 64;
constexpr int kChunks = GGK_SCHEDULER_CHUNKS;
constexpr int kMaxExperts = GGK_MOE_MAX_EXPERTS;
static_assert(kMaxExperts <= kThreads, "one thread per expert");
static_assert(kMaxExperts % 4 == 0, "per-expert arrays are read four entries at a time");
typedef int int4v __attribute__((ext_vector_type(4)));
typedef double double2v __attribute__((ext_vector_type(2)));
static_assert(kThreads / kWave <= kWave, "wave totals are scanned by one wave");
static_assert(2 + kChunks < GGK_MOE_STATUS && GGK_MOE_STATUS < GGK_MOE_HEADER_INTS, "header layout");

struct MoeArgs {
  ggk_moe_layout layout;
  const int* counts;
  int sort_mode;
  int cta_m, cta_n;      // reference macro-tile
  int work_tm, work_tn;  // reference tiles per work tile
  int stage_k;           // depth of one LDS stage
  gg_device_problem_desc* problems;
  int* offsets;
  int* perm;
  int* order;
  int* header;
};

// Estimated time of all work tiles of one problem (tm x tn work tiles), in
// hundredths of a cycle of one CU: per work tile 150 + stages * (31 + 0.029
// (rows + cols)) + 0.0023 rows cols (twice that last term when C is read),
// summed as integer products.  This is the host build's model
// (problem_work_time in grouped_gemm.cpp), evaluated in the same order with
// no fused multiply-add, so both give the same value and the same schedule.
__device__ double problem_work_time(int m, int n, int k, int tm, int tn, int bk, bool reads_c) {
#pragma clang fp contract(off)
  if (m <= 0 || n <= 0 || tm <= 0 || tn <= 0) return 0.0;
  const double w = static_cast<double>(tm) * tn;
  const double stages = k > 0 ? (k - 1) / bk + 1 : 0;
  const double edge = static_cast<double>(m) * tn + static_cast<double>(n) * tm;
  const double stage = 310000.0 * w + 290.0 * edge;
  const double area = static_cast<double>(m) * n;
  return 1500000.0 * w + stages * stage + (reads_c ? 46.0 : 23.0) * area;
}

// A problem's estimated time as the integer the schedule ranks and adds up:
// clamped to 2^52, so that up to GGK_MOE_MAX_EXPERTS of them sum exactly in
// 64 bits (below 2^53 the double is an exact integer already).
__device__ long long problem_time_units(double t) { return t < 4503599627370496.0 ? (long long)t : (1LL << 52); }

// Lane i takes lane i + SH's (value, index) pair when it is the lesser one
// (row shift within 16 lanes; the lanes it leaves undefined are not used).
template <int SH>
__device__ __forceinline__ void least_from(unsigned long long& v, int& idx) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, 0x100 + SH, 0xf, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), 0x100 + SH, 0xf, 0xf, false);
  const int pidx = __builtin_amdgcn_update_dpp(0, idx, 0x100 + SH, 0xf, 0xf, false);
  const unsigned long long pv = ((unsigned long long)hi << 32) | lo;
  const bool take = pv < v || (pv == v && pidx < idx);
  v = take ? pv : v;
  idx = take ? pidx : idx;
}

// Exclusive prefix sum of one value per thread over the workgroup of THREADS
// threads, in thread order; *total receives the sum.  Every thread must call it.
template <int THREADS, class T>
__device__ T block_exclusive_scan(T v, T* s_waves, T* total) {
  constexpr int kWaves = THREADS / kWave;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  T x = v;
  for (int d = 1; d < kWave; d *= 2) {
    const T y = __shfl_up(x, d, kWave);
    if (lane >= d) x += y;
  }
  T before_lane = __shfl_up(x, 1, kWave);
  if (lane == 0) before_lane = T(0);
  if constexpr (kWaves == 1) {
    *total = __shfl(x, kWave - 1, kWave);
    // Callers rely on the scan as a barrier for their shared-memory traffic around it.
    __syncthreads();
    return before_lane;
  }
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

template <int THREADS>
__global__ __launch_bounds__(THREADS) void moe_prepare_kernel(MoeArgs args) {
  constexpr int kWaves = THREADS / kWave;
  __shared__ long long s_waves_ll[kWaves];
  __shared__ int s_waves_i[kWaves];
  __shared__ __attribute__((aligned(16))) int s_rows[kMaxExperts];
  __shared__ long long s_row0[kMaxExperts];
  __shared__ __attribute__((aligned(16))) int s_tiles[kMaxExperts];
  __shared__ int s_perm[kMaxExperts];
  __shared__ long long s_total[kMaxExperts];    // estimated time of sorted position i (clamped units)
  __shared__ __attribute__((aligned(16))) double s_key[kMaxExperts];  // estimated time per work tile
  __shared__ long long s_by_total[kMaxExperts]; // estimated times, longest first
  __shared__ __attribute__((aligned(16))) int s_chunk[kMaxExperts];  // chunk of sorted position i
  __shared__ int s_order[kMaxExperts];       // sorted position at each scheduling position
  __shared__ int s_work[kMaxExperts];        // work tiles of sorted position i
  __shared__ int s_chunk_work[kChunks];
  __shared__ long long s_load[kChunks];  // chunk loads of the whole placement
  __shared__ int s_cut[kChunks + 1];  // chunk bounds inside the run of oversized positions
  __shared__ int s_run[3];            // oversized positions cut across chunks (0: none), first LPT chunk, run's work tiles
  __shared__ int s_status;

  const ggk_moe_layout& L = args.layout;
  const int experts = L.experts;
  const int tid = threadIdx.x;
  if (tid == 0) s_status = 0;
  if (tid < kChunks) s_chunk_work[tid] = 0;
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
  const long long row0 = block_exclusive_scan<THREADS, long long>(count, s_waves_ll, &all_rows);
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
      // Four experts per step (16-byte LDS reads; entries past E are never counted).
#pragma unroll 2
      for (int j0 = 0; j0 < experts; j0 += 4) {
        const int4v t4 = *reinterpret_cast<const int4v*>(&s_tiles[j0]);
        const int4v r4 = *reinterpret_cast<const int4v*>(&s_rows[j0]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = j0 + e;
          const int t = t4[e];
          const long long area = (long long)r4[e] * L.n;
          const bool by_tiles = tiles_first && t != my_tiles;
          const bool before = by_tiles ? t > my_tiles : area > my_area;
          const bool tie = !by_tiles && area == my_area;
          rank += (j < experts && (before || (tie && j < tid))) ? 1 : 0;
        }
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
  int total_tiles;
  const int tile_off = block_exclusive_scan<THREADS, int>(tiles, s_waves_i, &total_tiles);
  const bool reads_c = L.c != nullptr && L.beta != 0.0f;
  if (pos < experts) {
    args.offsets[pos] = tile_off;
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
  if (pos == 0) args.offsets[experts] = total_tiles;

  // The schedule, as the host build plans it (plan_schedule in
  // grouped_gemm.cpp): longest processing time first at two levels, after
  // spreading oversized positions.  One share is the total estimated time over
  // the chunks, rounded up.  Sorted positions above one share are cut across
  // chunks when placing every position whole (longest first, ties: lower
  // position first, each onto the first least-loaded chunk) would leave more
  // than a quarter of the total to stealing: they run first, back to back,
  // longest first, and chunk boundary c falls at the work tile nearest to where
  // the run's time reaches c shares.  The other positions go whole to the first
  // least-loaded chunk from the one holding the run's end on (which starts
  // with the remainder), longest first; within a chunk they run longest work
  // tile first (ties: lower position first), after the run.
  long long total = 0;  // estimated time, clamped (problem_time_units)
  double key = 0.0;     // estimated time per work tile
  if (pos < experts) {
    if (work > 0) {
      const int bm = args.cta_m * args.work_tm, bn = args.cta_n * args.work_tn;
      const double t =
          problem_work_time(rows, L.n, L.k, (rows - 1) / bm + 1, (L.n - 1) / bn + 1, args.stage_k, reads_c);
      total = problem_time_units(t);
      key = t / work;
    }
    s_total[pos] = total;
    s_key[pos] = key;
    s_work[pos] = work;
  }
  // At most GGK_MOE_MAX_EXPERTS (2^10) totals of at most 2^52: the sum is exact.
  long long sum_all;
  (void)block_exclusive_scan<THREADS, long long>(total, s_waves_ll, &sum_all);
  const long long share = sum_all / kChunks + (sum_all % kChunks != 0 ? 1 : 0);
  if (pos < experts) {
    int rank = 0;
#pragma unroll 8
    for (int j = 0; j < experts; ++j) {
      const long long t = s_total[j];
      rank += (t > total || (t == total && j < pos)) ? 1 : 0;
    }
    s_by_total[rank] = total;
    s_order[rank] = pos;
  }
  __syncthreads();
  // Greedy assignment by wave 0, one position at a time onto the first
  // least-loaded chunk.  Lane c < kChunks holds chunk c's load (an exact
  // integer), the other lanes a load no chunk reaches; the least (load, lane)
  // pair reaches lane 0 in three row shifts, so ties go to the lower chunk as
  // in a scan.  The estimated times come from LDS 64 at a time, one per lane;
  // each step takes its own from its lane and leaves its choice in that lane.
  // Returns each lane's final load.
  const int lane = tid & (kWave - 1);
  auto greedy = [&](int from, unsigned long long load) {
    for (int r0 = from; r0 < experts; r0 += kWave) {
      const int r = r0 + lane;
      const unsigned long long mine = r < experts ? (unsigned long long)s_by_total[r] : 0ull;
      const int mine_lo = (int)(uint32_t)mine;
      const int mine_hi = (int)(uint32_t)(mine >> 32);
      const int steps = min(kWave, experts - r0);
      int chosen = 0;  // lane j: the chunk of by-total rank r0 + j
      for (int j = 0; j < steps; ++j) {
        const unsigned long long t = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane(mine_hi, j) << 32) |
                                     (uint32_t)__builtin_amdgcn_readlane(mine_lo, j);
        unsigned long long v = load;
        int idx = lane;
        least_from<4>(v, idx);
        least_from<2>(v, idx);
        least_from<1>(v, idx);
        const int best = __builtin_amdgcn_readfirstlane(idx);
        load = lane == best ? load + t : load;
        chosen = lane == j ? best : chosen;
      }
      if (r < experts) s_chunk[s_order[r]] = chosen;
    }
    return load;
  };
  // Every position placed whole.
  if (tid < kWave) {
    const unsigned long long load = greedy(0, lane < kChunks ? 0ull : ~0ull);
    if (lane < kChunks) s_load[lane] = (long long)load;
  }
  __syncthreads();
  if (tid == 0) {
#pragma clang fp contract(off)
    int oversized = 0;  // they lead the by-total order
    while (oversized < experts && oversized < kChunks && s_by_total[oversized] > share) ++oversized;
    if (oversized > 0) {
      double stolen = 0.0;  // the chunks' shortfall below one share, in chunk order
      for (int c = 0; c < kChunks; ++c) stolen += s_load[c] < share ? (double)(share - s_load[c]) : 0.0;
      if (stolen * 4.0 <= (double)sum_all) oversized = 0;
    }
    int first = 0, run_work = 0;
    long long run_time = 0;
    if (oversized > 0) {
      int c = 1;
      for (int r = 0; r < oversized; ++r) {
        const int i = s_order[r];
        const long long t = s_by_total[r];
        const int w = s_work[i];
        for (; c < kChunks && c * share < run_time + t; ++c) {
          const double x = (double)(c * share - run_time) / (double)t * w;
          const int j = (int)floor(x + 0.5);
          s_cut[c] = run_work + (j < 0 ? 0 : (j > w ? w : j));
        }
        s_chunk[i] = r - kChunks;  // ahead of every chunk, in run order
        run_time += t;
        run_work += w;
      }
      first = c - 1;
      s_cut[0] = 0;
    }
    s_run[0] = oversized;
    s_run[1] = first;
    s_run[2] = run_work;
    s_load[0] = run_time - first * share;  // the first open chunk's starting load
  }
  __syncthreads();
  // The other positions, onto chunks from the one holding the run's end.
  if (tid < kWave && s_run[0] > 0) {
    const int first = s_run[1];
    const unsigned long long start = (unsigned long long)s_load[0];
    (void)greedy(s_run[0], lane < first || lane >= kChunks ? ~0ull : (lane == first ? start : 0ull));
  }
  __syncthreads();
  int chunk = 0;
  if (pos < experts) {
    chunk = s_chunk[pos];
    int before = 0;  // positions scheduled ahead of this one
#pragma unroll 2
    for (int j0 = 0; j0 < experts; j0 += 4) {
      const int4v c4 = *reinterpret_cast<const int4v*>(&s_chunk[j0]);
      const double2v k01 = *reinterpret_cast<const double2v*>(&s_key[j0]);
      const double2v k23 = *reinterpret_cast<const double2v*>(&s_key[j0 + 2]);
      const double kj[4] = {k01[0], k01[1], k23[0], k23[1]};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int j = j0 + e;
        const int cj = c4[e];
        before += (j < experts && (cj < chunk || (cj == chunk && (kj[e] > key || (kj[e] == key && j < pos))))) ? 1
                                                                                                             : 0;
      }
    }
    if (chunk >= 0) atomicAdd(&s_chunk_work[chunk], work);
    s_order[before] = pos;  // its by-total contents were last read by the greedy pass
  }
  __syncthreads();
  int sched_work = 0;
  if (pos < experts) sched_work = s_work[s_order[pos]];
  int total_work;
  const int work_off = block_exclusive_scan<THREADS, int>(sched_work, s_waves_i, &total_work);
  if (pos < experts) {
    args.order[pos] = s_order[pos];
    args.offsets[experts + 1 + pos] = work_off;
  }
  if (tid == 0) {
    args.offsets[2 * experts + 1] = total_work;
    args.header[0] = total_tiles;
    args.header[1] = total_work;
    // Chunks up to the one holding the run's end start where the run was cut.
    const int split = s_run[0] > 0;
    const int first = s_run[1];
    int bound = split ? s_run[2] : 0;
    for (int c = 0; c < kChunks; ++c) {
      if (split && c <= first) {
        args.header[2 + c] = s_cut[c];
      } else {
        args.header[2 + c] = bound;
      }
      if (c >= first) bound += s_chunk_work[c];
    }
    args.header[2 + kChunks] = bound;
    for (int h = 3 + kChunks; h < GGK_MOE_HEADER_INTS; ++h) args.header[h] = 0;
    args.header[GGK_MOE_STATUS] = s_status;
  }
}

// Reference macro-tile of each variant (GGK_VARIANT_*).
constexpr int kCta[GGK_VARIANT_COUNT][2] = {{64, 64}, {128, 64}, {64, 128}, {128, 64}, {64, 128}, {64, 64}};

}  // namespace

// ---------------------------------------------------------------------------
// Scratch of the allocation-free MoE entry point (gg_moe_run_noalloc): the
// prepared set of up to GGK_MOE_MAX_EXPERTS experts -- descriptors, offsets,
// permutation, scheduling order, header -- and the scheduler state, laid out
// as gg_moe_scratch_layout describes.  Every GPU holds one copy for the life
// of the process, shared by all calls on that GPU.
namespace {
constexpr size_t round256(size_t x) { return (x + 255) / 256 * 256; }
constexpr size_t kScratchBytes =
    round256(GGK_MOE_MAX_EXPERTS * sizeof(gg_device_problem_desc)) +
    round256((2 * (GGK_MOE_MAX_EXPERTS + 1) + 2 * GGK_MOE_MAX_EXPERTS + GGK_MOE_HEADER_INTS) * sizeof(int)) +
    round256(GGK_SCHEDULER_STATE_INTS * sizeof(int));
static_assert(kScratchBytes <= GG_MOE_NOALLOC_SCRATCH_BYTES, "the stated maximum holds the largest set");
}  // namespace

static __device__ __align__(256) unsigned char scratch[GG_MOE_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kScratchDevices] = {};
}  // namespace

// The current device's address of `scratch` (host code never uses the
// array's name itself: on the host it is a stand-in, not a device address).
// Found with hipGetSymbolAddress on the first call on each device, with that
// device current, then kept.  Not exported: the library's own entry point is
// its only caller.
extern "C" __attribute__((visibility("hidden"))) hipError_t gg_moe_scratch(void** ptr, size_t* bytes) {
  if (ptr == nullptr || bytes == nullptr) return hipErrorInvalidValue;
  int device = 0;
  hipError_t st = hipGetDevice(&device);
  if (st != hipSuccess) return st;
  if (device < 0 || device >= kScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    void* p = nullptr;
    st = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (st != hipSuccess) return st;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[device] = p;
  }
  *ptr = g_scratch_ptr[device];
  *bytes = GG_MOE_NOALLOC_SCRATCH_BYTES;
  return hipSuccess;
}

extern "C" hipError_t ggk_moe_layout_check(int variant, int path, const ggk_moe_layout* layout) {
  if (layout == nullptr || variant < 0 || variant >= GGK_VARIANT_COUNT) return hipErrorInvalidValue;
  ggk_work_shape work{};
  const hipError_t st = ggk_work_shape_get(variant, path, &work);
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
  if (L.a == nullptr || L.b == nullptr || L.d == nullptr) return hipErrorInvalidDevicePointer;
  return hipSuccess;
}

extern "C" hipError_t ggk_moe_prepare(int variant, int path, const ggk_moe_layout* layout, const int* d_counts,
                                      int sort_mode, gg_device_problem_desc* d_problems, int* d_offsets,
                                      int* d_sorted_to_original, int* d_order, int* d_header, hipStream_t stream) {
  if (sort_mode < 0 || sort_mode > 3) return hipErrorInvalidValue;
  hipError_t st = ggk_moe_layout_check(variant, path, layout);
  if (st != hipSuccess) return st;
  ggk_work_shape work{};
  st = ggk_work_shape_get(variant, path, &work);
  if (st != hipSuccess) return st;
  const ggk_moe_layout& L = *layout;
  const int cta_m = kCta[variant][0], cta_n = kCta[variant][1];
  if (d_counts == nullptr || d_problems == nullptr || d_offsets == nullptr || d_sorted_to_original == nullptr ||
      d_order == nullptr || d_header == nullptr) {
    return hipErrorInvalidDevicePointer;
  }
  MoeArgs args{L,         d_counts,  sort_mode,  cta_m, cta_n, work.tiles_m, work.tiles_n, work.stage_k, d_problems,
               d_offsets, d_sorted_to_original, d_order, d_header};
  void* params[] = {&args};
  if (L.experts <= kWave) {
    return hipLaunchKernel(reinterpret_cast<const void*>(moe_prepare_kernel<kWave>), dim3(1), dim3(kWave), params, 0,
                           stream);
  }
  return hipLaunchKernel(reinterpret_cast<const void*>(moe_prepare_kernel<kThreads>), dim3(1), dim3(kThreads), params,
                         0, stream);
}
