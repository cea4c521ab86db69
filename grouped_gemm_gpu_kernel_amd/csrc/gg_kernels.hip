// gg_kernels.hip -- gfx950 kernels of the grouped FP16 GEMM and the thin C-ABI
// (grouped_gemm_amd_kernels.h) the C++ host runtime calls.
//
// Kernels:
//   gg_grouped_kernel  persistent scheduler (grouped_gemm_kernel,
//                      src/grouped_gemm.cu:640-675): one launch, workgroups
//                      claim work-tile indices from device-wide counters until
//                      all are taken; each index is mapped to (problem, work
//                      tile) by a search over the work-tile offsets.  A work
//                      tile is a TM x TN block of the reference's macro-tiles
//                      (KernelShape), so every reference tile index t maps to
//                      the same (problem, tile_m, tile_n) as in the reference.
//   gg_single_kernel   one problem, one workgroup per work tile
//                      (single_problem_gemm_kernel, src/grouped_gemm.cu:677-688).
//   fill kernels       synthetic inputs and output poisoning for tests/benches.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <string.h>

#include "gg_common.h"
#include "gg_tiles.h"
#include "grouped_gemm_amd_kernels.h"

// Compiler resource table of the compiled kernels (generated from the compiler's
// resource-usage report; see gg_resources.cpp).
extern "C" int gg_compiler_resources(int kind, int variant, int path, int* vgprs, int* agprs,
                                     int* sgprs, int* scratch, int* waves_per_simd, int* lds);

namespace gg {

typedef const GG_CONST int* const_int_ptr;
typedef const GG_CONST uint32_t* const_u32_ptr;

// Reads descriptor `index` with a wave-uniform index from memory no thread
// writes during the launch, so the compiler can use scalar loads.
__device__ __forceinline__ gg_device_problem_desc load_problem(const gg_device_problem_desc* problems,
                                                               int index) {
  static_assert(sizeof(gg_device_problem_desc) % 4 == 0, "descriptor is whole dwords");
  constexpr int kWords = sizeof(gg_device_problem_desc) / 4;
  const_u32_ptr src = (const_u32_ptr)(problems + index);
  struct Words { uint32_t w[kWords]; } words;
#pragma unroll
  for (int i = 0; i < kWords; ++i) words.w[i] = src[i];
  return __builtin_bit_cast(gg_device_problem_desc, words);
}

constexpr int kChunks = GGK_SCHEDULER_CHUNKS;  // one per XCD
constexpr int kStride = GGK_SCHEDULER_COUNTER_STRIDE;
static_assert((kChunks & (kChunks - 1)) == 0 && kChunks <= kWave, "chunks are a power of two, one lane each");

struct GroupedArgs {
  const gg_device_problem_desc* __restrict__ problems;
  const int* __restrict__ tile_offsets;  // reference tiles: [count + 1]
  const int* __restrict__ work_offsets;  // work tiles, in scheduling order: [count + 1]
  // Problem at each scheduling position (NULL: position = problem index).
  const int* __restrict__ order;
  // (problem, work tile within it) of each work-tile index: [2 * total]
  // (NULL: found from work_offsets and order).
  const int* __restrict__ work_table;
  int count;
  int total;           // work tiles
  int* state;          // chunk c's claim counter at [c * kStride], retired workgroups at [kChunks * kStride]
  int* tile_map;       // traced launches only
  long long* wg_clock; // traced launches only
  long long* tile_phases;  // traced launches only: GGK_PHASE_COUNT per work-tile index
  int bounds[kChunks + 1];  // chunk c owns work-tile indices [bounds[c], bounds[c + 1])
  // When set, the total and the bounds are read from this device header
  // (written by a device-side prepare in stream order) instead of the two
  // fields above: [1] work tiles, [2, 2 + kChunks] bounds.
  const int* header;
};

// Scheduling.  Workgroups are dispatched to the XCDs round-robin, so
// workgroup w runs on XCD w % kChunks and starts on that chunk (its home):
// the tiles of one problem, which share A and B panels, are then multiplied
// on one XCD and its L2 serves the re-reads.  Workgroup w's first tile is
// fixed, index bounds[home] + w / kChunks, so a launch starts without any
// counter traffic; the rest of chunk c, [bounds[c] + fixed_slots(c),
// bounds[c + 1]), is handed out one index per atomicAdd on the chunk's
// counter.  A counter request takes microseconds (device-scope atomics are
// resolved past the XCDs' L2s), so it is made while the current tile is being
// computed and read after it.  When a chunk runs dry the workgroup moves on
// to the next one (stealing); `visit` counts the chunks it has left behind,
// in the order home, home + 1, ... (mod kChunks).  All claim logic runs in
// wave 0, uniformly; lane 0 makes the requests.

// Workgroups whose first tile is fixed in chunk c.
__device__ __forceinline__ int fixed_slots(int c, int grid) {
  return c < grid ? (grid - 1 - c) / kChunks + 1 : 0;
}

// First index of chunk c handed out by its counter.
__device__ __forceinline__ int counted_from(const int* bounds, int c, int grid) {
  return bounds[c] + fixed_slots(c, grid);
}

// The first visit at or after `visit` whose chunk has indices for its counter
// to hand out (kChunks if none).
__device__ __forceinline__ int first_counted(const int* bounds, int grid, int home, int visit) {
  for (; visit < kChunks; ++visit) {
    const int c = (home + visit) & (kChunks - 1);
    if (counted_from(bounds, c, grid) < bounds[c + 1]) break;
  }
  return visit;
}

// Claims an index now (wave 0): one lane per remaining chunk reads that
// chunk's counter, the first chunk with indices left is asked, and the search
// goes on past it if the request comes back empty.  Counters only grow
// during a launch, so a chunk read as dry stays dry.  Returns total, with
// visit = kChunks, when every chunk is exhausted.
__device__ __forceinline__ int claim_now(int* state, const int* bounds, int grid, int home, int& visit, int total) {
  const int lane = threadIdx.x & (kWave - 1);
  while (visit < kChunks) {
    bool open = false;
    const int v = visit + lane;
    if (v < kChunks) {
      const int c = (home + v) & (kChunks - 1);
      const int from = counted_from(bounds, c, grid);
      const int end = bounds[c + 1];
      if (from < end) {
        open = from + __hip_atomic_load(state + c * kStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < end;
      }
    }
    const uint64_t found = __ballot(open);
    if (found == 0) break;
    visit += __builtin_ctzll(found);
    const int c = (home + visit) & (kChunks - 1);
    int got = 0;
    if (lane == 0) got = atomicAdd(state + c * kStride, 1);
    const int t = counted_from(bounds, c, grid) + __builtin_amdgcn_readfirstlane(got);
    if (t < bounds[c + 1]) return t;
    ++visit;
  }
  visit = kChunks;
  return total;
}

// The schedule of one launch in LDS: s[0, kChunks] the chunk bounds, s[kChunks + 1]
// the work-tile total, from the arguments or from the device header.
__device__ __forceinline__ void load_schedule(const GroupedArgs& args, int* s) {
  const int tid = threadIdx.x;
  if (args.header != nullptr) {
    if (tid <= kChunks) s[tid] = args.header[2 + tid];
    if (tid == kChunks + 1) s[tid] = args.header[1];
  } else {
#pragma unroll
    for (int c = 0; c <= kChunks; ++c) {
      if (tid == c) s[c] = args.bounds[c];
    }
    if (tid == kChunks + 1) s[tid] = args.total;
  }
}

// Index of the problem that owns index t: the number of problems p with
// offsets[p + 1] <= t, i.e. upper_bound over offsets[1..count] -- the same
// function as find_problem_by_tile (src/grouped_gemm.cu:219-234), here over
// the work-tile offsets.  Problems with zero tiles never own an index.
//
// Evaluated by the whole wave at once: each step tests 64 evenly spaced
// candidates in parallel and keeps the span between the last true and the
// first false one, so count <= 4096 takes one coarse and one exact step (two
// dependent loads) instead of log2(count) serial probes.  The result is
// wave-uniform.
__device__ __forceinline__ int find_problem(const int* __restrict__ offsets, int count, int t) {
  const int lane = threadIdx.x & (kWave - 1);
  int lo = 0;
  int hi = count;  // the answer lies in [lo, hi]; candidates p in [lo, hi)
  while (hi - lo > kWave) {
    const int step = (hi - lo + kWave - 1) / kWave;
    const int p = lo + (lane + 1) * step - 1;
    const bool below = (p < hi) && (offsets[p + 1] <= t);
    const int passed = __popcll(__ballot(below));
    const int next_lo = lo + passed * step;
    const int probe_false = lo + (passed + 1) * step - 1;
    hi = probe_false < hi ? probe_false : hi;
    lo = next_lo;
  }
  const int p = lo + lane;
  const bool below = (p < hi) && (offsets[p + 1] <= t);
  return __builtin_amdgcn_readfirstlane(lo + __popcll(__ballot(below)));
}

// Work tiles of a problem along M and N.
template <int TM, int TN>
__device__ __forceinline__ int work_tiles_n(const gg_device_problem_desc& p) {
  return (p.tiles_n + TN - 1) / TN;
}

// Position (wm, wn) of work tile `local` of a problem with wtm x wtn work
// tiles, in the order the grouped kernel meets them: groups of kGroupRows rows
// (fewer in the last group), column by column within a group, row by row
// within a column.  Any run of consecutive tiles then covers a block a few
// rows tall, so the workgroups of one XCD, which claim consecutive indices,
// share A row panels and B column panels in that XCD's L2 (32 tiles touch 12
// panels instead of 33 for a long row).  A bijection of [0, wtm * wtn): it
// decides only the order, and every tile is computed the same way.
#ifndef GG_GROUP_ROWS
#define GG_GROUP_ROWS 4
#endif
constexpr int kGroupRows = GG_GROUP_ROWS;
__device__ __forceinline__ void work_tile_position(int local, int wtm, int wtn, int& wm, int& wn) {
  const int group_size = kGroupRows * wtn;
  const int group = local / group_size;
  const int first = group * kGroupRows;
  const int rows = wtm - first < kGroupRows ? wtm - first : kGroupRows;
  const int within = local - group * group_size;
  wn = within / rows;
  wm = first + (within - wn * rows);
}

// The start stamps of a traced work tile: wall clock, core clock, and what it
// is (workgroup, row half, rows and columns inside the problem, k-stages).
template <class G>
__device__ __forceinline__ void mark_tile_start(const PhaseStamps& stamps, int half, const gg_device_problem_desc& p,
                                                int m0, int n0) {
  if (stamps.slot != nullptr && __builtin_amdgcn_readfirstlane(threadIdx.x / kWave) == 0) {
    const long long rows = p.m - m0 < G::BM ? p.m - m0 : G::BM;
    const long long cols = p.n - n0 < G::BN ? p.n - n0 : G::BN;
    const long long stages = (p.k + G::BK - 1) / G::BK;
    stamps.slot[GGK_PHASE_WALL] = wall_clock64();
    stamps.slot[GGK_PHASE_WHO] =
        (long long)blockIdx.x | ((long long)half << 20) | (rows << 22) | (cols << 34) | (stages << 46);
  }
  stamps.mark(GGK_PHASE_START);
}

// At least KernelShape::WAVES_PER_EU waves per SIMD: 2 allows 256 VGPRs +
// AGPRs per lane (a 512-thread workgroup, or two 256-thread ones), 1 allows 512.
#define GG_KERNEL_ATTRS(V, PATH)                          \
  __launch_bounds__((KernelShape<V, PATH>::G::THREADS)) \
      __attribute__((amdgpu_waves_per_eu(KernelShape<V, PATH>::WAVES_PER_EU)))

template <int V, int PATH, bool TRACED, bool WIDE>
__global__ GG_KERNEL_ATTRS(V, PATH) void gg_grouped_kernel(GroupedArgs args) {
  using S = KernelShape<V, PATH>;
  using G = typename S::G;
  __shared__ __attribute__((aligned(16))) uint16_t lds[KernelLds<S>::HALVES];
  __shared__ int s_claim[2];
  __shared__ int s_schedule[kChunks + 2];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const bool wave0 = __builtin_amdgcn_readfirstlane(tid / kWave) == 0;
  long long clock_start = 0;
  long long clock_end = 0;
  if (TRACED) {
    clock_start = wall_clock64();
    clock_end = clock_start;
  }

  const int grid = gridDim.x;
  const int home = blockIdx.x % kChunks;
  load_schedule(args, s_schedule);
  __syncthreads();
  const int total = __builtin_amdgcn_readfirstlane(s_schedule[kChunks + 1]);
  // Whether any chunk has indices beyond the fixed first tiles: when none has,
  // no counter is touched and none needs resetting.
  const bool counted = first_counted(s_schedule, grid, 0, 0) < kChunks;

  int visit = 0;  // wave 0
  int t = __builtin_amdgcn_readfirstlane(s_schedule[home] + (int)blockIdx.x / kChunks);
  int parity = 0;
  if (t >= __builtin_amdgcn_readfirstlane(s_schedule[home + 1])) {
    // No fixed tile for this workgroup (its chunk is smaller than its share
    // of the grid): claim one now.
    if (wave0) {
      const int c = counted ? claim_now(args.state, s_schedule, grid, home, visit, total) : total;
      if (lane == 0) s_claim[0] = c;
    }
    __syncthreads();
    t = __builtin_amdgcn_readfirstlane(s_claim[0]);
    parity = 1;
  }

  while (t < total) {
    // The request for the next index, made once while this tile is computed.
    bool asked = false;
    int chunk = -1;  // wave 0: the chunk asked, -1 if none
    int got = 0;     // wave 0, lane 0: what the request returned
    auto request = [&]() -> bool {
      asked = true;
      if (!wave0 || !counted) return false;
      visit = first_counted(s_schedule, grid, home, visit);
      if (visit >= kChunks) return false;
      chunk = (home + visit) & (kChunks - 1);
      if (lane == 0) got = atomicAdd(args.state + chunk * kStride, 1);
      return true;
    };

    // The next index, resolved once this tile's request is back (wave 0:
    // its chunk's counter value, or a claim of its own once the chunk is
    // dry), then handed to every wave through LDS and one barrier.  A tile
    // that is computed does this as soon as its k-loop ends, before its
    // epilogue: the waves then need no barrier after the epilogue, and those
    // done first start the next tile's stage loads while the others still
    // store (the epilogue reads no LDS, and the barrier after the k-loop has
    // seen every LDS read of this tile).  Slot `parity` was last read before
    // the previous tile's handover barrier.
    int next_t = total;
    bool handed = false;
    auto hand_over = [&]() {
      if (wave0) {
        int next = total;
        if (chunk >= 0) {
          next = counted_from(s_schedule, chunk, grid) + __builtin_amdgcn_readfirstlane(got);
          if (next >= s_schedule[chunk + 1]) {
            ++visit;
            next = claim_now(args.state, s_schedule, grid, home, visit, total);
          }
        }
        if (lane == 0) s_claim[parity] = next;
      }
      __syncthreads();
      next_t = __builtin_amdgcn_readfirstlane(s_claim[parity]);
      handed = true;
    };
    // Phase stamps of this work tile (traced launches with a phase buffer only).
    static_assert(G::THREADS <= kWave * GGK_PHASE_STEP_WAVES, "one step-stamp row per wave");
    PhaseStamps stamps{TRACED && args.tile_phases != nullptr ? args.tile_phases + (long long)GGK_PHASE_COUNT * t
                                                             : nullptr};
    auto after_k_loop = [&]() {
      stamps.mark(GGK_PHASE_K_END);
      if (!asked) request();
      hand_over();
      stamps.mark(GGK_PHASE_EPILOGUE);
    };

    static_assert(!S::CLASSES || S::TM % 2 == 0, "a half of the rows is whole rows of macro-tiles");
    int prob, local;
    int half = 0;  // 0: the whole work tile; 1, 2: its first or second half of rows
    if (args.work_table != nullptr) {
      // One scalar load instead of the search's chain of dependent ones.
      prob = ((const_int_ptr)args.work_table)[2 * t];
      const int word = ((const_int_ptr)args.work_table)[2 * t + 1];
      local = word & GGK_WORK_LOCAL_MASK;
      half = S::CLASSES ? (word >> GGK_WORK_HALF_SHIFT) & 3 : 0;
    } else {
      const int pos = find_problem(args.work_offsets, args.count, t);
      prob = args.order != nullptr ? ((const_int_ptr)args.order)[pos] : pos;
      local = t - ((const_int_ptr)args.work_offsets)[pos];
    }
    // Uniform index into read-only memory: scalar loads of the 80-byte descriptor.
    const gg_device_problem_desc p = load_problem(args.problems, prob);
    const int wtn = work_tiles_n<S::TM, S::TN>(p);
    const int wtm = (p.tiles_m + S::TM - 1) / S::TM;
    if (wtn > 0 && wtm > 0 && local < wtm * wtn) {
      int wm, wn;
      work_tile_position(local, wtm, wtn, wm, wn);
      if (TRACED && args.tile_map != nullptr) {
        // Record every reference tile this work tile covers under its
        // reference index.
        const int base = ((const_int_ptr)args.tile_offsets)[prob];
        if (tid < S::TM * S::TN) {
          const int tm = wm * S::TM + tid / S::TN;
          const int tn = wn * S::TN + tid % S::TN;
          constexpr int kHalfRows = S::TM >= 2 ? S::TM / 2 : 1;  // macro-tile rows per half
          const bool in_half = half == 0 || (tid / S::TN) / kHalfRows == half - 1;
          if (in_half && tm < p.tiles_m && tn < p.tiles_n) {
            const int ref = base + tm * p.tiles_n + tn;
            args.tile_map[3 * ref + 0] = prob;
            args.tile_map[3 * ref + 1] = tm;
            args.tile_map[3 * ref + 2] = tn;
          }
        }
      } else if (half == 0) {
        if constexpr (TRACED) {
          mark_tile_start<G>(stamps, 0, p, wm * G::BM, wn * G::BN);
          run_work_tile<S, PATH, WIDE>(p, wm * G::BM, wn * G::BN, lds, request, after_k_loop, stamps);
        } else {
          run_work_tile<S, PATH, WIDE>(p, wm * G::BM, wn * G::BN, lds, request, after_k_loop);
        }
      } else {
        // One half of the rows (whole rows of macro-tiles), computed as a
        // problem that ends with that half: its tile has at most BM / 2 rows
        // and runs in a half-height edge class, and each of its D elements is
        // computed as in the whole tile.
        gg_device_problem_desc q = p;
        const int m0 = wm * G::BM + (half - 1) * (G::BM / 2);
        const int end = m0 + G::BM / 2;
        q.m = end < p.m ? end : p.m;
        if constexpr (TRACED) {
          mark_tile_start<G>(stamps, half, q, m0, wn * G::BN);
          run_work_tile<S, PATH, WIDE>(q, m0, wn * G::BN, lds, request, after_k_loop, stamps);
        } else {
          run_work_tile<S, PATH, WIDE>(q, m0, wn * G::BN, lds, request, after_k_loop);
        }
      }
    }
    if (!asked) request();
    if (!handed) hand_over();  // nothing computed (or the traced map): hand over now
    if (TRACED) clock_end = wall_clock64();
    t = next_t;
    parity ^= 1;
  }

  if (tid == 0) {
    if (TRACED && args.wg_clock != nullptr) {
      args.wg_clock[2 * blockIdx.x + 0] = clock_start;
      args.wg_clock[2 * blockIdx.x + 1] = clock_end;
    }
    // A workgroup leaves only after finding every chunk exhausted, with no
    // request in flight, so when the last one leaves nobody will touch the
    // counters again: it returns them to zero for the next launch in stream
    // order.
    if (counted) {
      const int retired = atomicAdd(args.state + kChunks * kStride, 1);
      if (retired == grid - 1) {
        for (int c = 0; c <= kChunks; ++c) atomicExch(args.state + c * kStride, 0);
      }
    }
  }
}

template <int V, int PATH, bool WIDE>
__global__ GG_KERNEL_ATTRS(V, PATH) void gg_single_kernel(gg_device_problem_desc p) {
  using S = KernelShape<V, PATH>;
  using G = typename S::G;
  __shared__ __attribute__((aligned(16))) uint16_t lds[KernelLds<S>::HALVES];
  const int t = blockIdx.x;
  const int wtn = work_tiles_n<S::TM, S::TN>(p);
  const int wtm = (p.tiles_m + S::TM - 1) / S::TM;
  if (wtn <= 0 || t >= wtm * wtn) return;
  const int wm = t / wtn;
  const int wn = t - wm * wtn;
  run_work_tile<S, PATH, WIDE>(p, wm * G::BM, wn * G::BN, lds, [] { return false; }, [] {});
}

// ---------------------------------------------------------------------------
// Synthetic data: a counter-based hash (splitmix64 finaliser) so that element i
// depends only on (seed, stream, i) and any element can be recomputed alone.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t x) {
  x ^= x >> 30;
  x *= 0xbf58476d1ce4e5b9ull;
  x ^= x >> 27;
  x *= 0x94d049bb133111ebull;
  x ^= x >> 31;
  return x;
}

__device__ __forceinline__ float unit_draw(uint64_t key, uint64_t i) {
  const uint64_t h = mix64(key + i * 0x9e3779b97f4a7c15ull);
  return (float)(h >> 40) * 5.9604644775390625e-08f;  // [0, 1) in steps of 2^-24
}

__global__ void fill_uniform_f16_kernel(uint16_t* dst, int64_t count, uint64_t key, float lo, float span) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * blockDim.x) {
    const _Float16 h = (_Float16)(lo + span * unit_draw(key, (uint64_t)i));
    dst[i] = __builtin_bit_cast(uint16_t, h);
  }
}

__global__ void fill_uniform_f32_kernel(float* dst, int64_t count, uint64_t key, float lo, float span) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * blockDim.x) {
    dst[i] = lo + span * unit_draw(key, (uint64_t)i);
  }
}

__global__ void fill_normal_f16_kernel(uint16_t* dst, int64_t count, uint64_t key, float sigma) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float u1 = 1.0f - unit_draw(key, 2 * (uint64_t)i);  // (0, 1]
    const float u2 = unit_draw(key, 2 * (uint64_t)i + 1);
    const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
    const _Float16 h = (_Float16)(sigma * z);
    dst[i] = __builtin_bit_cast(uint16_t, h);
  }
}

__global__ void fill_f32_kernel(float* dst, int64_t count, float value) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * blockDim.x) {
    dst[i] = value;
  }
}

// ---------------------------------------------------------------------------
// Kernel tables: [variant][path] (and [traced] for the grouped kernel).
// ---------------------------------------------------------------------------
using GroupedFn = void (*)(GroupedArgs);
using SingleFn = void (*)(gg_device_problem_desc);

// Index [0] of each kernel array is the 32-bit-offset form, [1] the WIDE form.
template <int V, int P>
struct KernelEntry {
  static constexpr int threads = KernelShape<V, P>::G::THREADS;
  static constexpr int tm = KernelShape<V, P>::TM;
  static constexpr int tn = KernelShape<V, P>::TN;
  static constexpr int bm = KernelShape<V, P>::G::BM;
  static constexpr int bn = KernelShape<V, P>::G::BN;
  static constexpr int bk = KernelShape<V, P>::G::BK;
};

#define GG_ENTRY(V, P)                                                                               \
  {{gg_grouped_kernel<V, P, false, false>, gg_grouped_kernel<V, P, false, true>},                   \
   {gg_grouped_kernel<V, P, true, false>, gg_grouped_kernel<V, P, true, true>},                     \
   {gg_single_kernel<V, P, false>, gg_single_kernel<V, P, true>}, KernelEntry<V, P>::threads,        \
   KernelEntry<V, P>::tm, KernelEntry<V, P>::tn, KernelEntry<V, P>::bm, KernelEntry<V, P>::bn,      \
   KernelEntry<V, P>::bk, KernelShape<V, P>::CLASSES}
#define GG_ROW(V) {GG_ENTRY(V, 0), GG_ENTRY(V, 1)}

struct KernelSet {
  GroupedFn grouped[2];
  GroupedFn traced[2];
  SingleFn single[2];
  int threads;
  int tm;
  int tn;
  int bm;  // work-tile rows
  int bn;  // work-tile columns
  int bk;  // stage depth
  bool halves;  // reads half-work-tile table entries
};

static const KernelSet kKernels[GGK_VARIANT_COUNT][GGK_PATH_COUNT] = {
    GG_ROW(GGK_VARIANT_64x64x16), GG_ROW(GGK_VARIANT_128x64x32), GG_ROW(GGK_VARIANT_64x128x32),
    GG_ROW(GGK_VARIANT_128x64x32_SMALL), GG_ROW(GGK_VARIANT_64x128x32_SMALL), GG_ROW(GGK_VARIANT_64x64x16_SMALL)};
#undef GG_ROW
#undef GG_ENTRY

static bool valid_kernel(int variant, int path) {
  return variant >= 0 && variant < GGK_VARIANT_COUNT && path >= 0 && path < GGK_PATH_COUNT;
}

static hipError_t fill_launch_shape(int64_t count, dim3* grid) {
  if (count < 0) return hipErrorInvalidValue;
  int64_t blocks = (count + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  *grid = dim3((unsigned)blocks);
  return hipSuccess;
}

static uint64_t fill_key(uint64_t seed, uint64_t stream_id) {
  return mix64(seed ^ mix64(stream_id + 0x632be59bd9b4e019ull));
}

}  // namespace gg

using namespace gg;

extern "C" {

hipError_t ggk_alloc(void** ptr, size_t bytes) {
  if (ptr == nullptr) return hipErrorInvalidValue;
  return hipMalloc(ptr, bytes);
}

hipError_t ggk_free(void* ptr) { return ptr == nullptr ? hipSuccess : hipFree(ptr); }

hipError_t ggk_copy_to_device(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return hipSuccess;
  return hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice);
}

hipError_t ggk_copy_to_host(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return hipSuccess;
  return hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
}

hipError_t ggk_zero(void* ptr, size_t bytes) {
  if (bytes == 0) return hipSuccess;
  return hipMemset(ptr, 0, bytes);
}

hipError_t ggk_stream_synchronize(hipStream_t stream) { return hipStreamSynchronize(stream); }

hipError_t ggk_device_synchronize(void) { return hipDeviceSynchronize(); }

hipError_t ggk_event_create(hipEvent_t* event) {
  if (event == nullptr) return hipErrorInvalidValue;
  return hipEventCreateWithFlags(event, hipEventDisableTiming);
}

hipError_t ggk_event_destroy(hipEvent_t event) { return event == nullptr ? hipSuccess : hipEventDestroy(event); }

hipError_t ggk_event_record_launch(hipEvent_t event, hipStream_t stream, int* recorded) {
  if (recorded != nullptr) *recorded = 0;
  if (event == nullptr) return hipErrorInvalidValue;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  hipError_t st = hipStreamIsCapturing(stream, &capture);
  if (st != hipSuccess) return st;
  if (capture != hipStreamCaptureStatusNone) {
    if (recorded != nullptr) *recorded = GGK_LAUNCH_CAPTURED;
    return hipSuccess;
  }
  st = hipEventRecord(event, stream);
  if (st == hipSuccess && recorded != nullptr) *recorded = GGK_LAUNCH_RECORDED;
  return st;
}

hipError_t ggk_event_synchronize(hipEvent_t event) { return event == nullptr ? hipSuccess : hipEventSynchronize(event); }

hipError_t ggk_current_device(int* device) {
  if (device == nullptr) return hipErrorInvalidValue;
  return hipGetDevice(device);
}

hipError_t ggk_device_info_get(ggk_device_info* out) {
  if (out == nullptr) return hipErrorInvalidValue;
  int device = 0;
  hipError_t st = hipGetDevice(&device);
  if (st != hipSuccess) return st;
  hipDeviceProp_t prop;
  st = hipGetDeviceProperties(&prop, device);
  if (st != hipSuccess) return st;
  memset(out, 0, sizeof(*out));
  out->device = device;
  out->compute_units = prop.multiProcessorCount;
  out->max_threads_per_cu = prop.maxThreadsPerMultiProcessor;
  out->max_wgs_per_cu = prop.maxBlocksPerMultiProcessor;
  out->wave_size = prop.warpSize;
  out->regs_per_cu = prop.regsPerMultiprocessor;
  out->regs_per_block = prop.regsPerBlock;
  out->lds_per_cu = (int)prop.maxSharedMemoryPerMultiProcessor;
  out->lds_per_block = (int)prop.sharedMemPerBlock;
  out->l2_bytes = prop.l2CacheSize;
  out->clock_khz = prop.clockRate;
  out->major = prop.major;
  out->minor = prop.minor;
  strncpy(out->arch_name, prop.gcnArchName, sizeof(out->arch_name) - 1);
  return hipSuccess;
}

static void fill_bounds(GroupedArgs& args, const int* chunk_bounds) {
  for (int c = 0; c <= kChunks; ++c) {
    args.bounds[c] = chunk_bounds != nullptr ? chunk_bounds[c]
                                             : (int)((int64_t)args.total * c / kChunks);
  }
}

static bool bounds_valid(const int* chunk_bounds, int total) {
  if (chunk_bounds == nullptr) return true;
  if (chunk_bounds[0] != 0 || chunk_bounds[kChunks] != total) return false;
  for (int c = 0; c < kChunks; ++c) {
    if (chunk_bounds[c + 1] < chunk_bounds[c]) return false;
  }
  return true;
}

static hipError_t launch_grouped(int variant, int path, int addressing, bool traced,
                                 const gg_device_problem_desc* d_problems, const int* d_tile_offsets,
                                 const int* d_work_offsets, const int* d_order, const int* d_work_table,
                                 int problem_count, int total_work, int* d_state, const int* chunk_bounds, int grid,
                                 int* d_tile_map, long long* d_wg_clock, long long* d_tile_phases,
                                 hipStream_t stream) {
  if (!valid_kernel(variant, path) || grid <= 0 || problem_count < 0 || total_work < 0 ||
      (addressing != GGK_ADDR_32 && addressing != GGK_ADDR_64)) {
    return hipErrorInvalidValue;
  }
  if (total_work == 0 || problem_count == 0) return hipSuccess;
  if (d_problems == nullptr || d_work_offsets == nullptr || d_state == nullptr) {
    return hipErrorInvalidDevicePointer;
  }
  if (traced && d_tile_map != nullptr && d_tile_offsets == nullptr) return hipErrorInvalidDevicePointer;
  if (!bounds_valid(chunk_bounds, total_work)) return hipErrorInvalidValue;
  GroupedArgs args{d_problems,  d_tile_offsets, d_work_offsets, d_order, d_work_table, problem_count, total_work,
                   d_state,     traced ? d_tile_map : nullptr, traced ? d_wg_clock : nullptr,
                   traced ? d_tile_phases : nullptr, {}, nullptr};
  fill_bounds(args, chunk_bounds);
  void* params[] = {&args};
  const KernelSet& k = kKernels[variant][path];
  return hipLaunchKernel(reinterpret_cast<const void*>(traced ? k.traced[addressing] : k.grouped[addressing]),
                         dim3(grid), dim3(k.threads), params, 0, stream);
}

// 32-bit offsets from a work tile's origin reach every A and B value the
// tile reads when 0 <= lda, 0 <= ldb, BM * lda + K + 8 BK < 2^30 and
// BK * ldb < 2^30 (binary16 elements; the bound leaves room past K), and
// every C and D value of the tile when 0 <= ldc, ldd and BM * ld + BN < 2^29
// (float elements; ldc only matters when C is read).  Every byte offset then
// stays below 2^31, which the loader's out-of-range marker relies on.
static bool fits_addr32(const KernelSet& k, const gg_device_problem_desc& p) {
  constexpr int64_t kLimit = int64_t(1) << 30;
  constexpr int64_t kOutLimit = int64_t(1) << 29;
  const bool reads_c = p.c != nullptr && p.beta != 0.0f;
  return p.lda >= 0 && p.ldb >= 0 && p.k >= 0 && (int64_t)k.bm * p.lda + p.k + 8 * k.bk < kLimit &&
         (int64_t)k.bk * p.ldb < kLimit && p.ldd >= 0 && (int64_t)k.bm * p.ldd + k.bn < kOutLimit &&
         (!reads_c || (p.ldc >= 0 && (int64_t)k.bm * p.ldc + k.bn < kOutLimit));
}

hipError_t ggk_work_shape_get(int variant, int path, ggk_work_shape* out) {
  if (!valid_kernel(variant, path) || out == nullptr) return hipErrorInvalidValue;
  const KernelSet& k = kKernels[variant][path];
  out->tiles_m = k.tm;
  out->tiles_n = k.tn;
  out->threads = k.threads;
  out->rows = k.bm;
  out->stage_k = k.bk;
  return hipSuccess;
}

int ggk_small_variant(int variant) {
  switch (variant) {
    case GGK_VARIANT_64x64x16: return GGK_VARIANT_64x64x16_SMALL;
    case GGK_VARIANT_128x64x32: return GGK_VARIANT_128x64x32_SMALL;
    case GGK_VARIANT_64x128x32: return GGK_VARIANT_64x128x32_SMALL;
    default: return -1;
  }
}

int ggk_work_halves_supported(int variant, int path) {
  if (!valid_kernel(variant, path)) return -1;
  return kKernels[variant][path].halves ? 1 : 0;
}

int ggk_needs_addr64(int variant, int path, const gg_device_problem_desc* problem) {
  if (!valid_kernel(variant, path) || problem == nullptr) return -1;
  if (problem->tiles_m <= 0 || problem->tiles_n <= 0) return 0;
  return fits_addr32(kKernels[variant][path], *problem) ? 0 : 1;
}

hipError_t ggk_launch_grouped(int variant, int path, int addressing, const gg_device_problem_desc* d_problems,
                              const int* d_work_offsets, const int* d_order, const int* d_work_table,
                              int problem_count, int total_work, int* d_state, const int* chunk_bounds, int grid,
                              hipStream_t stream) {
  return launch_grouped(variant, path, addressing, false, d_problems, nullptr, d_work_offsets, d_order, d_work_table,
                        problem_count, total_work, d_state, chunk_bounds, grid, nullptr, nullptr, nullptr, stream);
}

hipError_t ggk_launch_grouped_device(int variant, int path, int addressing, const gg_device_problem_desc* d_problems,
                                     const int* d_work_offsets, const int* d_order, int problem_count,
                                     const int* d_header, int* d_state, int grid, hipStream_t stream) {
  if (!valid_kernel(variant, path) || grid <= 0 || problem_count < 0 ||
      (addressing != GGK_ADDR_32 && addressing != GGK_ADDR_64)) {
    return hipErrorInvalidValue;
  }
  if (problem_count == 0) return hipSuccess;
  if (d_problems == nullptr || d_work_offsets == nullptr || d_state == nullptr || d_header == nullptr) {
    return hipErrorInvalidDevicePointer;
  }
  GroupedArgs args{d_problems, nullptr, d_work_offsets, d_order, nullptr, problem_count, 0, d_state, nullptr, nullptr,
                   nullptr, {}, d_header};
  void* params[] = {&args};
  const KernelSet& k = kKernels[variant][path];
  return hipLaunchKernel(reinterpret_cast<const void*>(k.grouped[addressing]), dim3(grid), dim3(k.threads), params,
                         0, stream);
}

hipError_t ggk_launch_grouped_traced(int variant, int path, int addressing,
                                     const gg_device_problem_desc* d_problems, const int* d_tile_offsets,
                                     const int* d_work_offsets, const int* d_order, const int* d_work_table,
                                     int problem_count, int total_work, int* d_state, const int* chunk_bounds,
                                     int grid, int* d_tile_map, long long* d_wg_clock, long long* d_tile_phases,
                                     hipStream_t stream) {
  return launch_grouped(variant, path, addressing, true, d_problems, d_tile_offsets, d_work_offsets, d_order,
                        d_work_table, problem_count, total_work, d_state, chunk_bounds, grid, d_tile_map, d_wg_clock,
                        d_tile_phases, stream);
}

hipError_t ggk_launch_single(int variant, int path, const gg_device_problem_desc* problem,
                             hipStream_t stream) {
  if (!valid_kernel(variant, path) || problem == nullptr) return hipErrorInvalidValue;
  // The 64-bit form of the 256 x 256 work tile spills registers: such a
  // problem runs on 128 x 128 work tiles of the same macro-tile (same D).
  if (path == GGK_PATH_MFMA && ggk_small_variant(variant) >= 0 && !fits_addr32(kKernels[variant][path], *problem)) {
    variant = ggk_small_variant(variant);
  }
  const KernelSet& k = kKernels[variant][path];
  if (problem->tiles_m <= 0 || problem->tiles_n <= 0) return hipSuccess;
  const int64_t work = (int64_t)((problem->tiles_m + k.tm - 1) / k.tm) * ((problem->tiles_n + k.tn - 1) / k.tn);
  if (work > 0x7fffffff) return hipErrorInvalidValue;
  gg_device_problem_desc p = *problem;
  void* params[] = {&p};
  const int addressing = fits_addr32(k, p) ? GGK_ADDR_32 : GGK_ADDR_64;
  return hipLaunchKernel(reinterpret_cast<const void*>(k.single[addressing]), dim3((unsigned)work),
                         dim3(k.threads), params, 0, stream);
}

hipError_t ggk_kernel_resources_get(int kernel_kind, int variant, int path, ggk_kernel_resources* out) {
  if (!valid_kernel(variant, path) || out == nullptr) return hipErrorInvalidValue;
  if (kernel_kind != GGK_KERNEL_GROUPED && kernel_kind != GGK_KERNEL_SINGLE) return hipErrorInvalidValue;
  memset(out, 0, sizeof(*out));
  gg_compiler_resources(kernel_kind, variant, path, &out->vgprs, &out->agprs, &out->sgprs,
                        &out->scratch_bytes_per_lane, &out->compiler_waves_per_simd, &out->lds_bytes);
  const void* fn = kernel_kind == GGK_KERNEL_GROUPED
                       ? reinterpret_cast<const void*>(kKernels[variant][path].grouped[GGK_ADDR_32])
                       : reinterpret_cast<const void*>(kKernels[variant][path].single[GGK_ADDR_32]);
  hipFuncAttributes attr;
  hipError_t st = hipFuncGetAttributes(&attr, fn);
  if (st != hipSuccess) return st;
  out->num_regs = attr.numRegs;
  out->lds_static = (int)attr.sharedSizeBytes;
  out->lds_dynamic = 0;
  out->local_bytes = (int)attr.localSizeBytes;
  out->max_threads = attr.maxThreadsPerBlock;
  return hipSuccess;
}

hipError_t ggk_occupancy(int variant, int path, int* active_wgs_per_cu) {
  if (!valid_kernel(variant, path) || active_wgs_per_cu == nullptr) return hipErrorInvalidValue;
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(
      active_wgs_per_cu, reinterpret_cast<const void*>(kKernels[variant][path].grouped[GGK_ADDR_32]),
      kKernels[variant][path].threads, 0);
}

hipError_t ggk_fill_uniform_f16(void* d_dst, int64_t count, uint64_t seed, uint64_t stream_id, float lo,
                                float hi, hipStream_t stream) {
  dim3 grid;
  hipError_t st = fill_launch_shape(count, &grid);
  if (st != hipSuccess || count == 0) return st;
  if (d_dst == nullptr) return hipErrorInvalidDevicePointer;
  hipLaunchKernelGGL(fill_uniform_f16_kernel, grid, dim3(256), 0, stream, static_cast<uint16_t*>(d_dst),
                     count, fill_key(seed, stream_id), lo, hi - lo);
  return hipGetLastError();
}

hipError_t ggk_fill_uniform_f32(float* d_dst, int64_t count, uint64_t seed, uint64_t stream_id, float lo,
                                float hi, hipStream_t stream) {
  dim3 grid;
  hipError_t st = fill_launch_shape(count, &grid);
  if (st != hipSuccess || count == 0) return st;
  if (d_dst == nullptr) return hipErrorInvalidDevicePointer;
  hipLaunchKernelGGL(fill_uniform_f32_kernel, grid, dim3(256), 0, stream, d_dst, count,
                     fill_key(seed, stream_id), lo, hi - lo);
  return hipGetLastError();
}

hipError_t ggk_fill_normal_f16(void* d_dst, int64_t count, uint64_t seed, uint64_t stream_id, float sigma,
                               hipStream_t stream) {
  dim3 grid;
  hipError_t st = fill_launch_shape(count, &grid);
  if (st != hipSuccess || count == 0) return st;
  if (d_dst == nullptr) return hipErrorInvalidDevicePointer;
  hipLaunchKernelGGL(fill_normal_f16_kernel, grid, dim3(256), 0, stream, static_cast<uint16_t*>(d_dst),
                     count, fill_key(seed, stream_id), sigma);
  return hipGetLastError();
}

hipError_t ggk_fill_f32(float* d_dst, int64_t count, float value, hipStream_t stream) {
  dim3 grid;
  hipError_t st = fill_launch_shape(count, &grid);
  if (st != hipSuccess || count == 0) return st;
  if (d_dst == nullptr) return hipErrorInvalidDevicePointer;
  hipLaunchKernelGGL(fill_f32_kernel, grid, dim3(256), 0, stream, d_dst, count, value);
  return hipGetLastError();
}

}  // extern "C"
