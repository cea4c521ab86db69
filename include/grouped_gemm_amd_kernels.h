/*
 * grouped_gemm_amd_kernels.h -- the thin C-ABI between the C++ host runtime and
 * the gfx950 kernels of the grouped FP16 GEMM.
 *
 * Everything that touches the GPU goes through these functions: device memory,
 * kernel launches, kernel resource accounting and occupancy.  The host runtime
 * above (include/grouped_gemm/grouped_gemm.h) is plain C++ that includes HIP's
 * headers only for the types hipError_t, hipStream_t and __half.
 *
 * Plain C: POD structs, pointers and sizes, hipError_t status codes, no
 * exceptions.  Reference counterparts are cited per entry point.
 */
#ifndef GROUPED_GEMM_AMD_KERNELS_H_
#define GROUPED_GEMM_AMD_KERNELS_H_

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One problem as the device reads it.  Same fields, order and meaning as
 * DeviceProblemDesc (src/grouped_gemm.cu:25-45): the caller's ProblemDesc plus
 * tiles_m / tiles_n, which are 0 when m <= 0 or n <= 0.  a and b point to
 * IEEE binary16 data, row-major A[m x lda] and B[k x ldb]; c (may be NULL) and
 * d are row-major float32 with leading dimensions ldc and ldd. */
typedef struct gg_device_problem_desc {
  int m;
  int n;
  int k;
  const void* a;
  const void* b;
  const float* c;
  float* d;
  int lda;
  int ldb;
  int ldc;
  int ldd;
  float alpha;
  float beta;
  int tiles_m;
  int tiles_n;
} gg_device_problem_desc;

/* Macro-tile shapes (src/grouped_gemm.cu:47-52).  On the MFMA path all three
 * compute 256 x 256 work tiles (4 x 4, 2 x 4 or 4 x 2 macro-tiles).  The _SMALL
 * variants have no counterpart in the reference: the same macro-tiles on
 * 128 x 128 work tiles (two workgroups per CU), which the executor picks for
 * launches with few work tiles and for sets that need 64-bit addressing (see
 * GroupedGemmExecutor::build). */
enum {
  GGK_VARIANT_64x64x16 = 0,
  GGK_VARIANT_128x64x32 = 1,
  GGK_VARIANT_64x128x32 = 2,
  GGK_VARIANT_128x64x32_SMALL = 3,
  GGK_VARIANT_64x128x32_SMALL = 4,
  GGK_VARIANT_64x64x16_SMALL = 5,
  GGK_VARIANT_COUNT = 6
};

/* Tile compute path: FMA (the reference's SIMT path) or MFMA (the reference's
 * tensor-core path). */
enum { GGK_PATH_FMA = 0, GGK_PATH_MFMA = 1, GGK_PATH_COUNT = 2 };

/* Kernel kinds for resource queries. */
enum { GGK_KERNEL_GROUPED = 0, GGK_KERNEL_SINGLE = 1 };

/* The persistent grid claims tiles from GGK_SCHEDULER_CHUNKS contiguous
 * chunks of the tile index range, one per XCD (an MI355X has 8); workgroup w
 * starts on chunk w % GGK_SCHEDULER_CHUNKS -- its first tile there is fixed by
 * w, later ones are claimed from the chunk's counter -- and moves to the next
 * chunk when its own is exhausted. */
#define GGK_SCHEDULER_CHUNKS 8

/* Ints between two scheduler counters: each sits on a 128-byte line of its
 * own, so the workgroups claiming from different chunks do not queue on one
 * line. */
#define GGK_SCHEDULER_COUNTER_STRIDE 32

/* A work-table entry's second int: the work tile's index within its problem
 * in the low bits (GGK_WORK_LOCAL_MASK), and in bits GGK_WORK_HALF_SHIFT and
 * up 0 for the whole work tile or 1 / 2 for its first / second half of rows
 * (128 rows: one or two rows of macro-tiles; only for kernels whose 256-row
 * work tile has half-height edge classes: ggk_work_halves_supported). */
#define GGK_WORK_HALF_SHIFT 28
#define GGK_WORK_LOCAL_MASK ((1 << GGK_WORK_HALF_SHIFT) - 1)

/* Ints of scheduler state one grouped launch needs: a claim counter per chunk
 * and a retire counter, GGK_SCHEDULER_COUNTER_STRIDE apart.  Must be zero
 * before the first launch; every launch leaves it zero again. */
#define GGK_SCHEDULER_STATE_INTS (GGK_SCHEDULER_COUNTER_STRIDE * (GGK_SCHEDULER_CHUNKS + 1))

typedef struct ggk_device_info {
  int device;
  int compute_units;
  int max_threads_per_cu;
  int max_wgs_per_cu;
  int wave_size;
  int regs_per_cu;
  int regs_per_block;
  int lds_per_cu;
  int lds_per_block;
  int l2_bytes;
  int clock_khz;
  int major;
  int minor;
  char arch_name[64];
} ggk_device_info;

/* Resources of one compiled kernel.  vgprs/agprs/sgprs/scratch come from the
 * compiler's resource report of the library as compiled; num_regs, lds_static, local_bytes
 * and max_threads from hipFuncGetAttributes. */
typedef struct ggk_kernel_resources {
  int vgprs;
  int agprs;
  int sgprs;
  int scratch_bytes_per_lane;
  int compiler_waves_per_simd;
  int lds_bytes;
  int num_regs;
  int lds_static;
  int lds_dynamic;
  int local_bytes;
  int max_threads;
} ggk_kernel_resources;

/* Device memory and copies (the cudaMalloc / cudaMemcpy / cudaFree calls of
 * GroupedGemmExecutor::build and release_device_buffers,
 * src/grouped_gemm.cu:932-948, 1178-1219). */
hipError_t ggk_alloc(void** ptr, size_t bytes);
hipError_t ggk_free(void* ptr);
hipError_t ggk_copy_to_device(void* dst, const void* src, size_t bytes);
hipError_t ggk_copy_to_host(void* dst, const void* src, size_t bytes);
hipError_t ggk_zero(void* ptr, size_t bytes);
hipError_t ggk_stream_synchronize(hipStream_t stream);
hipError_t ggk_device_synchronize(void);

/* Completion tracking of an executor's launches (no reference counterpart: the
 * reference frees its buffers with cudaFree, which waits for the whole device).
 * An executor records its event after each launch on the launch's stream and
 * waits for it before it rewrites or frees the buffers those launches read.  A
 * launch captured into a graph has no event (its replays run later, on streams
 * the executor never sees): the executor then waits for the whole device
 * instead.  Events are created with timing disabled. */
hipError_t ggk_event_create(hipEvent_t* event);
hipError_t ggk_event_destroy(hipEvent_t event);
/* Records `event` on `stream` unless the stream is capturing.  *recorded (may
 * be NULL) tells which: GGK_LAUNCH_RECORDED (1) when the event was recorded,
 * GGK_LAUNCH_CAPTURED (2) when the stream is capturing, 0 on failure. */
#define GGK_LAUNCH_RECORDED 1
#define GGK_LAUNCH_CAPTURED 2
hipError_t ggk_event_record_launch(hipEvent_t event, hipStream_t stream, int* recorded);
hipError_t ggk_event_synchronize(hipEvent_t event);

/* Index of the current device (hipGetDevice). */
hipError_t ggk_current_device(int* device);

/* Device properties of the current device (cudaGetDeviceProperties in
 * resolve_runtime_mode and query_occupancy, src/grouped_gemm.cu:111-143,
 * 1024-1083). */
hipError_t ggk_device_info_get(ggk_device_info* out);

/* Work tile of a kernel: one claim of the grouped kernel, or one workgroup of
 * the single-problem kernel, computes a tiles_m x tiles_n block of the
 * variant's macro-tiles (src/grouped_gemm.cu:54-65) with `threads` threads;
 * rows = tiles_m * cta_m, and stage_k is the depth of one LDS stage.
 * The work-tile count of a problem is ceil(tiles_m_p / tiles_m) *
 * ceil(tiles_n_p / tiles_n); the reference tile (tm, tn) belongs to work
 * tile (wm, wn) = (tm / tiles_m, tn / tiles_n).  The grouped kernel numbers a
 * problem's work tiles in groups of 4 work-tile rows, column by column within
 * a group (index = first row of the group * wn_count + column * rows in the
 * group + row within the group), so that the work tiles in flight at once
 * share A and B panels; the single-problem kernel numbers them row-major.
 * No reference counterpart: the reference computes one macro-tile per CTA
 * and numbers tiles row-major. */
typedef struct ggk_work_shape {
  int tiles_m;
  int tiles_n;
  int threads;
  int rows;
  int stage_k;
} ggk_work_shape;
hipError_t ggk_work_shape_get(int variant, int path, ggk_work_shape* out);

/* 1 when the grouped kernel of (variant, path) reads work-table entries for
 * half work tiles (GGK_WORK_HALF_SHIFT), 0 when it does not, -1 for a bad
 * argument.  No reference counterpart. */
int ggk_work_halves_supported(int variant, int path);

/* The variant with the same macro-tile on 128 x 128 work tiles (the _SMALL
 * form, which the executor uses for launches with few work tiles and for sets
 * that need 64-bit addressing; same D), or -1 when variant has none.  No
 * reference counterpart. */
int ggk_small_variant(int variant);

/* Addressing form of a grouped launch.  GGK_ADDR_32: A and B are addressed
 * and C/D with 32-bit offsets from per-tile origins, which needs, for every
 * problem of the launch, 0 <= lda, 0 <= ldb, rows * lda + k + 8 * stage_k <
 * 2^30, stage_k * ldb < 2^30 (ggk_work_shape), 0 <= ldd, rows * ldd + cols <
 * 2^29 (cols = tiles_n x the configuration's macro-tile width) and, when C is
 * read (c != NULL and beta != 0), the same for ldc.  GGK_ADDR_64: 64-bit
 * addresses, any layout, slower.
 * ggk_needs_addr64 returns 1 when `problem` (host memory) needs GGK_ADDR_64,
 * 0 when not (also for a problem without tiles), -1 for a bad argument.  The
 * single-problem launch chooses by itself.  No reference counterpart. */
enum { GGK_ADDR_32 = 0, GGK_ADDR_64 = 1 };
int ggk_needs_addr64(int variant, int path, const gg_device_problem_desc* problem);

/* Persistent grouped launch (launch_grouped_by_variant + grouped_gemm_kernel,
 * src/grouped_gemm.cu:640-675, 728-751, 800-869).  d_problems[problem_count]
 * in sorted order.  Work tiles are numbered in a scheduling order of the
 * problems: d_order[problem_count] (device memory, or NULL for the sorted
 * order itself) gives the problem at each position, and
 * d_work_offsets[problem_count + 1] is the prefix sum of the work-tile counts
 * in that order (the role of the reference's d_tile_offsets, which it equals
 * when the work tile is one macro-tile and d_order is NULL); d_state holds
 * GGK_SCHEDULER_STATE_INTS zeroed ints.  chunk_bounds (host memory,
 * GGK_SCHEDULER_CHUNKS + 1 non-decreasing ints from 0 to total_work, or NULL
 * for equal counts) splits the work-tile indices into the per-XCD chunks.
 * d_work_table[2 * total_work] (device memory, or NULL) holds for each
 * work-tile index the problem (in sorted order) and the work tile's index
 * within that problem (numbered as described at ggk_work_shape, encoded as
 * at GGK_WORK_HALF_SHIFT), which the kernel then reads instead of
 * searching d_work_offsets for them; a table may list both halves of a work
 * tile instead of the whole, and then counts them as two work-tile indices.  grid workgroups claim work tiles until
 * total_work are done. */
hipError_t ggk_launch_grouped(int variant, int path, int addressing, const gg_device_problem_desc* d_problems,
                              const int* d_work_offsets, const int* d_order, const int* d_work_table,
                              int problem_count, int total_work, int* d_state, const int* chunk_bounds, int grid,
                              hipStream_t stream);

/* The same scheduler with instrumentation.  d_tile_map (may be NULL; needs
 * d_tile_offsets, the reference tile offsets of the problems in sorted
 * order): for each reference tile t of a claimed work tile, ints [3t, 3t+3)
 * receive (problem, tile_m, tile_n), problem in sorted order, and no
 * GEMM is computed.  d_wg_clock (may be NULL): for workgroup w, the 100 MHz
 * wall clock at its start and at the end of its last tile go to [2w, 2w+2);
 * the GEMM is computed as usual.  d_tile_phases (may be NULL; zeroed by the
 * caller): for work-tile index t (of total_work), GGK_PHASE_COUNT int64s at
 * [GGK_PHASE_COUNT t, ...) receive its phase stamps (GGK_PHASE_*); the GEMM
 * is computed as usual.  No reference counterpart: measurement only. */
enum {
  GGK_PHASE_WALL = 0,         /* 100 MHz wall clock at the work tile's start */
  GGK_PHASE_START = 1,        /* core clock (s_memtime) at its start */
  GGK_PHASE_FIRST_STAGE = 2,  /* the first stage's loads of one wave have landed */
  GGK_PHASE_K_LOOP = 3,       /* every wave has its first stage: the k-loop starts */
  GGK_PHASE_K_END = 4,        /* the k-loop has ended (before the hand-over of the next index) */
  GGK_PHASE_EPILOGUE = 5,     /* the hand-over is done: the epilogue starts */
  GGK_PHASE_EPILOGUE_END = 6, /* the last wave has issued its epilogue (latest over the waves) */
  GGK_PHASE_WHO = 7,          /* workgroup | half << 20 (0 whole, 1 / 2 a row half) | rows << 22 |
                                 cols << 34 | stages << 46: the tile's rows and columns inside its
                                 problem (at most the work tile's), its k-stages */
  /* Entry GGK_PHASE_STEP + GGK_PHASE_STEP_MARKS w + i: wave w's core clock in the k-loop step
   * k = stages / 2 (LDS-DMA k-loops only; zero elsewhere): i = 0 the step starts, 1 its loads of
   * the next stage are issued, 2 its MFMAs and fragment reads are issued, 3 its loads have landed
   * (the step's vmcnt wait is over), 4 the step's closing barrier is passed. */
  GGK_PHASE_STEP = 8,
  GGK_PHASE_STEP_MARKS = 5,
  GGK_PHASE_STEP_WAVES = 8,   /* waves per workgroup at most */
  GGK_PHASE_COUNT = 48        /* GGK_PHASE_STEP + GGK_PHASE_STEP_MARKS GGK_PHASE_STEP_WAVES */
};
hipError_t ggk_launch_grouped_traced(int variant, int path, int addressing,
                                     const gg_device_problem_desc* d_problems, const int* d_tile_offsets,
                                     const int* d_work_offsets, const int* d_order, const int* d_work_table,
                                     int problem_count, int total_work, int* d_state, const int* chunk_bounds,
                                     int grid, int* d_tile_map, long long* d_wg_clock, long long* d_tile_phases,
                                     hipStream_t stream);

/* Device-resident preparation of a mixture-of-experts group (no reference
 * counterpart: it is the step before the grouped launch in MoE use, done here
 * without a host round trip).  The E experts share N and K: expert e
 * multiplies rows [r_e, r_e + count_e) of A (binary16, rows x K, lda) by
 * B + e * stride_b (binary16, K x N, ldb) into the same rows of D (float,
 * rows x N, ldd), adding beta * C (float, ldc; NULL for none); r_e is the
 * exclusive prefix sum of the counts in expert order.  One workgroup reads
 * d_counts[E] (device memory) and writes, in stream order and with no host
 * synchronisation: d_problems[E], the descriptors in the order
 * prepare_problem_set gives for sort_mode (src/grouped_gemm.cu:967-1022);
 * d_offsets[2 * (E + 1)], the reference tile offsets then the work-tile
 * offsets in scheduling order; d_sorted_to_original[E]; d_order[E], the
 * sorted position at each scheduling position; and
 * d_header[GGK_MOE_HEADER_INTS]: [0] total tiles, [1] total work tiles,
 * [2, 2 + GGK_SCHEDULER_CHUNKS] the chunk bounds, [GGK_MOE_STATUS] status
 * bits.  The schedule (order, work-tile offsets, chunk bounds) is the one
 * GroupedGemmExecutor::build plans for the same descriptors: longest
 * processing time first, whole problems per chunk.  Counts are not trusted: a
 * negative count is taken as 0 (GGK_MOE_NEGATIVE) and rows at or past
 * max_rows are dropped (GGK_MOE_CLAMPED), so no launch touches rows outside
 * [0, max_rows) of A, C and D.  1 <= E <= GGK_MOE_MAX_EXPERTS. */
#define GGK_MOE_MAX_EXPERTS 1024
#define GGK_MOE_HEADER_INTS 16
#define GGK_MOE_STATUS 12
enum { GGK_MOE_NEGATIVE = 1, GGK_MOE_CLAMPED = 2 };

typedef struct ggk_moe_layout {
  int experts;
  int n;
  int k;
  const void* a;
  int lda;
  const void* b;
  int ldb;
  long long stride_b; /* elements between consecutive experts' B */
  const float* c;
  int ldc;
  float* d;
  int ldd;
  float alpha;
  float beta;
  int max_rows; /* rows of A, C and D the caller owns */
} ggk_moe_layout;

hipError_t ggk_moe_prepare(int variant, int path, const ggk_moe_layout* layout, const int* d_counts, int sort_mode,
                           gg_device_problem_desc* d_problems, int* d_offsets, int* d_sorted_to_original,
                           int* d_order, int* d_header, hipStream_t stream);

/* The host-side checks ggk_moe_prepare makes of a layout before it launches
 * anything (no reference counterpart: the reference has no device-side
 * prepare): hipErrorInvalidValue for an expert count outside
 * [1, GGK_MOE_MAX_EXPERTS], negative n, k or max_rows, lda < k, ldb or ldd
 * < n, a negative stride_b, ldc < n with C given, or a tile count that could
 * overflow an int; hipErrorInvalidDevicePointer for a null A, B or D.
 * MoeGroupedGemm::build and the allocation-free entry point call it before
 * any launch, so a rejected layout writes nothing. */
hipError_t ggk_moe_layout_check(int variant, int path, const ggk_moe_layout* layout);

/* The grouped launch of a device-prepared set: the same kernel as
 * ggk_launch_grouped, which reads the work-tile total and the chunk bounds
 * from d_header (as ggk_moe_prepare writes it) when it starts.  grid is fixed
 * by the caller (e.g. every resident workgroup); workgroups that find no work
 * retire at once.  d_order as for ggk_launch_grouped (NULL: scheduling order
 * = descriptor order). */
hipError_t ggk_launch_grouped_device(int variant, int path, int addressing, const gg_device_problem_desc* d_problems,
                                     const int* d_work_offsets, const int* d_order, int problem_count,
                                     const int* d_header, int* d_state, int grid, hipStream_t stream);

/* One problem, one workgroup per work tile, row-major work-tile order
 * (single_problem_gemm_kernel + launch_single_problem_variant,
 * src/grouped_gemm.cu:677-688, 753-769).  *problem is read on the host and
 * passed by value; a problem with zero tiles launches nothing.  The
 * addressing form is chosen here; an MFMA problem that needs 64-bit
 * addressing runs on the 128 x 128 work tiles of its variant's _SMALL form
 * (same macro-tile, same D). */
hipError_t ggk_launch_single(int variant, int path, const gg_device_problem_desc* problem,
                             hipStream_t stream);

/* Resources of a compiled kernel (cudaFuncGetAttributes in
 * query_occupancy_variant, src/grouped_gemm.cu:785-797). */
hipError_t ggk_kernel_resources_get(int kernel_kind, int variant, int path, ggk_kernel_resources* out);

/* Resident workgroups per CU for the grouped kernel
 * (cudaOccupancyMaxActiveBlocksPerMultiprocessor, src/grouped_gemm.cu:778-784). */
hipError_t ggk_occupancy(int variant, int path, int* active_wgs_per_cu);

/* Fills count elements at d_dst with a counter-based hash draw from
 * uniform[lo, hi) (fp16: rounded to nearest even; fp32: as drawn).  Element i
 * depends only on (seed, stream_id, i).  Synthetic-input generator for tests
 * and benchmarks. */
hipError_t ggk_fill_uniform_f16(void* d_dst, int64_t count, uint64_t seed, uint64_t stream_id,
                                float lo, float hi, hipStream_t stream);
hipError_t ggk_fill_uniform_f32(float* d_dst, int64_t count, uint64_t seed, uint64_t stream_id,
                                float lo, float hi, hipStream_t stream);
/* Same draw mapped to a normal(0, sigma) value by Box-Muller on two hashes. */
hipError_t ggk_fill_normal_f16(void* d_dst, int64_t count, uint64_t seed, uint64_t stream_id,
                               float sigma, hipStream_t stream);
/* Writes value to count floats (NaN poisoning of outputs in tests). */
hipError_t ggk_fill_f32(float* d_dst, int64_t count, float value, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GROUPED_GEMM_AMD_KERNELS_H_ */
