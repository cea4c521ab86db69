// gg_tiles.h -- macro-tile compute for the gfx950 grouped GEMM.
//
// Both tile paths share one pipeline: each K stage is read from global memory
// into registers while the previous stage, held in LDS, is being multiplied;
// the registers are then written to the other LDS buffer and one barrier ends
// the stage.  The reference's equivalents are compute_gemm_tile_tensor_core and
// compute_gemm_tile_simt (src/grouped_gemm.cu:373-626); the k-loop structure,
// register blocking and LDS layout here are gfx950's own.
#pragma once

#include "gg_common.h"

namespace gg {

// Runs the staged k-loop of one tile: compute(stage_pointer) is called once
// per stage with that stage's LDS buffer, and on_start() once, by every
// thread, after the first loads are on their way (the persistent scheduler
// requests its next tile there, so that the request's latency overlaps this
// tile's).  on_start returns whether the calling wave issued one global
// memory request of its own.
//
// Stage s is fetched into register set s % DEPTH.  While stage k is
// multiplied out of LDS buffer k % 2, the loads of stage k + DEPTH - 1 are
// issued and stage k + 1 (issued DEPTH - 1 stages earlier) is written to the
// other LDS buffer; one barrier closes the step.  Loads and LDS writes are
// issued for every step, also for stages past K (which read as zero without
// touching memory and land in a buffer nobody reads): a load under a branch
// would make the compiler wait for every load in flight before the next LDS
// write, and only DEPTH - 1 = 1 stage could ever be in flight.  The main loop
// runs whole groups of DEPTH steps with no branch; the last steps of a tile
// are guarded.  The body is unrolled DEPTH times so that every register set
// is addressed statically.
template <class G, bool WIDE, class Compute, class OnStart, class Stamps>
__device__ __forceinline__ void run_k_loop(const gg_device_problem_desc& p, int m0, int n0, uint16_t* lds,
                                           Compute&& compute, OnStart&& on_start, const Stamps& stamps) {
  constexpr int D = G::DEPTH;
  const int nk = (p.k + G::BK - 1) / G::BK;
  if (nk <= 0) {
    on_start();
    return;
  }
  const StageLoader<G, WIDE> loader(p, m0, n0);
  RawStage<G, WIDE> ring[D];
#pragma unroll
  for (int s = 0; s < D - 1; ++s) loader.issue(s, ring[s]);
  on_start();  // the compiler's waits count the request like any other load
  loader.store(ring[0], 0, lds, 0);
  stamps.mark(GGK_PHASE_FIRST_STAGE);
  __syncthreads();
  stamps.mark(GGK_PHASE_K_LOOP);
  auto step = [&](int k, int u) {
    loader.issue(k + D - 1, ring[(u + D - 1) % D]);
    compute(lds + (k & 1) * G::STAGE);
    loader.store(ring[(u + 1) % D], k + 1, lds, (k + 1) & 1);
    __syncthreads();
  };
  int k0 = 0;
  for (; k0 + D <= nk; k0 += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) step(k0 + u, u);
  }
#pragma unroll
  for (int u = 0; u < D - 1; ++u) {
    if (k0 + u < nk) step(k0 + u, u);
  }
}

// The k-loop with stage loads straight into LDS (32-bit offsets): BUFFERS
// LDS buffers, BUFFERS - 1 stages in flight.  While stage k is multiplied out
// of buffer k % BUFFERS, the loads of stage k + BUFFERS - 1 go to the buffer
// every wave finished multiplying in the previous step; each wave then waits
// until its own loads of stage k + 1 have landed (the stage holding K - 1 is
// repaired then), and a barrier without a memory fence closes the step -- a
// fenced barrier would also wait for the stages still in flight.  Loads are
// issued for stages past K too (they read as zero or land unread).
//
// on_start runs in the first step, after the loads of stage L are issued: a
// request it makes is then the youngest in flight, and the first step's wait
// lets it stay in flight (loads complete in order, so one more outstanding
// operation is exactly that request).  The second step's wait retires it, so
// it has two stage computations to come back.
template <class G, class Compute, class OnStart, class Stamps>
__device__ __forceinline__ void run_k_loop_dma(const gg_device_problem_desc& p, int m0, int n0, uint16_t* lds,
                                               Compute&& compute, OnStart&& on_start, const Stamps& stamps) {
  constexpr int NBUF = G::BUFFERS;
  constexpr int L = NBUF - 1;
  constexpr int PENDING = (L - 1) * DmaLoader<G>::LOADS;  // loads of later stages allowed in flight
  const int nk = (p.k + G::BK - 1) / G::BK;
  if (nk <= 0) {
    on_start();
    return;
  }
  const DmaLoader<G> loader(p, m0, n0);
#pragma unroll
  for (int s = 0; s < L; ++s) loader.issue(s, lds + s * G::STAGE);
  wait_vmcnt<PENDING>();
  stamps.mark(GGK_PHASE_FIRST_STAGE);
  if (loader.last_stage == 0) loader.fix_last_stage(0, lds);
  stage_barrier();
  stamps.mark(GGK_PHASE_K_LOOP);
  // One step per iteration, not unrolled: no register set has to be indexed
  // statically, and one copy of the step keeps the code a launch has to fetch
  // into a cold instruction cache small.  u is the buffer of stage k.
  int u = 0;
#pragma unroll 1
  for (int k = 0; k < nk; ++k) {
    const int ul = u == 0 ? L : u - 1;  // (u + L) % NBUF
    const int un = u == NBUF - 1 ? 0 : u + 1;
    const bool stamped = k == nk / 2;  // the step whose timing a traced launch records
    if (stamped) stamps.step_mark(0);
    loader.issue(k + L, lds + ul * G::STAGE);
    const bool extra = k == 0 && __builtin_amdgcn_readfirstlane(on_start() ? 1 : 0) != 0;
    if (stamped) stamps.step_mark(1);
    compute(lds + u * G::STAGE);
    if (stamped) stamps.step_mark(2);
    if (extra) {
      wait_vmcnt<PENDING + 1>();
    } else {
      wait_vmcnt<PENDING>();
    }
    if (stamped) stamps.step_mark(3);
    if (k + 1 == loader.last_stage) loader.fix_last_stage(k + 1, lds + un * G::STAGE);
    stage_barrier();
    if (stamped) stamps.step_mark(4);
    u = un;
  }
}

// ---------------------------------------------------------------------------
// MFMA tile: v_mfma_f32_32x32x16_f16, (BM/WM) x (BN/WN) waves, each owning a
// WM x WN block of D held as (WM/32) x (WN/32) 32x32 accumulators.
//
// Operand layouts of v_mfma_f32_32x32x16_f16 (lane l of 64):
//   A: row l%32, k = 8*(l/32) + e, e = 0..7 (one 16-byte read of an A row)
//   B: col l%32, k = 8*(l/32) + e
//   D: acc[4*g + r] = D[8*g + 4*(l/32) + r][l%32], g, r = 0..3
// B sits in LDS row-major ([k][n]); ds_read_b64_tr_b16 turns four k-rows of
// 16 columns into the k-contiguous operand.  Within each group of 16 lanes it
// returns, to lane i, element i%4 of the 8-byte chunk addressed by lane
// 4*e + i/4 of the group, for e = 0..3.  Lane j of the group therefore
// addresses row kb + j/4, columns nb + 4*(j%4), and lane i receives
// B[kb + e][nb + i].
// ---------------------------------------------------------------------------
// Epilogue chunks of C requested ahead of the one being written (for blocks
// written in three or more chunks): C comes from HBM, and with two chunks in
// flight its latency is paid about half as often.
#ifndef GG_EPI_AHEAD
#define GG_EPI_AHEAD 2
#endif
template <class G, int WM_>
struct MfmaTile {
  static constexpr int WM = WM_;
  static constexpr int WAVES_M = G::BM / WM;
  static constexpr int WAVES_N = G::THREADS / kWave / WAVES_M;
  static constexpr int WN = G::BN / WAVES_N;
  static constexpr int FM = WM / 32;
  static constexpr int FN = WN / 32;
  static_assert(WAVES_M * WAVES_N * kWave == G::THREADS, "one wave per block of D");
  static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must hold whole 32x32 blocks");
  // 32-row groups of D per epilogue chunk: the whole block for blocks of up
  // to 2 x 2 accumulators (16 C vectors, 64 registers), one row of
  // accumulators per chunk for larger blocks, which hold more registers.
  static constexpr int EPI_ROWS = FM * FN <= 4 ? FM : 1;
  static_assert(FM % EPI_ROWS == 0, "whole chunks");

  // Multiplies one LDS stage into acc.  All MFMAs of a stage are issued
  // unconditionally; skipping is decided once per tile for the whole wave.
  __device__ __forceinline__ static void compute_stage(const uint16_t* stage, int lane, int wm, int wn,
                                                       floatx16_t (&acc)[FM][FN]) {
    const uint16_t* as = stage;
    const uint16_t* bs = stage + G::A_STAGE;
    lane = opaque_tid() & (kWave - 1);
    const int g = lane >> 4;
    const int j = lane & 15;
    // Operand fragments of k-step s (16 deep) of the stage.
    auto load_frags = [&](int s, half8_t (&af)[FM], half8_t (&bf)[FN]) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const uint16_t* src = as + G::a_piece(wm * WM + fm * 32 + (lane & 31), 2 * s + (lane >> 5));
        af[fm] = *reinterpret_cast<const half8_t*>(src);
      }
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int nb = wn * WN + fn * 32 + 16 * (g & 1);
        const int kb = s * 16 + 8 * (g >> 1);
        // Rows kb + j/4 and kb + 4 + j/4 share one swizzle (it depends on k mod 4).
        const uint16_t* src = bs + G::b_chunk(kb + (j >> 2), nb + 4 * (j & 3));
        const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((GG_LDS short4_t*)(src));
        const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((GG_LDS short4_t*)(src + 4 * G::SB));
        bf[fn] = __builtin_bit_cast(half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    };
    auto multiply = [&](const half8_t (&af)[FM], const half8_t (&bf)[FN]) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[fm], bf[fn], acc[fm][fn], 0, 0, 0);
        }
      }
    };
    constexpr int STEPS = G::BK / 16;
    if constexpr (FM * FN <= 4) {
      // Small wave blocks: the compiler may schedule the whole stage freely.
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        half8_t af[FM];
        half8_t bf[FN];
        load_frags(s, af, bf);
        multiply(af, bf);
      }
    } else {
      // Large wave blocks: fragments of step s + 1 are read while step s is
      // multiplied, and no further -- reading the whole stage ahead would
      // need more registers than the accumulators leave.
      half8_t af[2][FM];
      half8_t bf[2][FN];
      load_frags(0, af[0], bf[0]);
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        if (s + 1 < STEPS) load_frags(s + 1, af[(s + 1) & 1], bf[(s + 1) & 1]);
        multiply(af[s & 1], bf[s & 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // Computes the work tile at (m0, n0); on_start as in the k-loops, and
  // after_k_loop() once by every thread when the k-loop is over (no LDS read
  // of this tile follows it: the epilogue works from registers).
  template <bool WIDE, class OnStart, class AfterKLoop, class Stamps>
  __device__ __forceinline__ static void run(const gg_device_problem_desc& p, int m0, int n0, uint16_t* lds,
                                             OnStart&& on_start, AfterKLoop&& after_k_loop, const Stamps& stamps) {
    const int tid = opaque_tid();
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int wm = wave / WAVES_N;
    const int wn = wave % WAVES_N;
    // A wave whose block starts past the problem's edge has nothing to
    // multiply or store; it still stages its share of A and B for the others.
    const bool live = m0 + wm * WM < p.m && n0 + wn * WN < p.n;

    floatx16_t acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[fm][fn][e] = 0.0f;

    auto compute = [&](const uint16_t* stage) {
      if (live) compute_stage(stage, lane, wm, wn, acc);
    };
    if constexpr (WIDE) {
      run_k_loop<G, WIDE>(p, m0, n0, lds, compute, on_start, stamps);
    } else {
      run_k_loop_dma<G>(p, m0, n0, lds, compute, on_start, stamps);
    }
    after_k_loop();

    if (live) store_tile<WIDE>(p, m0 + wm * WM, n0 + wn * WN, lane, acc);
    stamps.wave_done();
  }

  // 4 x 4 transpose across the 4 lanes of a quad: lane q holds x[k] = M[q][k]
  // and receives M[k][q], in two exchange steps (partner q^1, then q^2).
  __device__ __forceinline__ static void quad_transpose(float (&x)[4], int q) {
    const bool odd = (q & 1) != 0;
    const float s0 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(odd ? x[0] : x[1]), 0xB1, 0xf, 0xf, true));
    const float s1 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(odd ? x[2] : x[3]), 0xB1, 0xf, 0xf, true));
    float y[4];
    y[0] = odd ? s0 : x[0];
    y[1] = odd ? x[1] : s0;
    y[2] = odd ? s1 : x[2];
    y[3] = odd ? x[3] : s1;
    const bool hi = (q & 2) != 0;
    const float t0 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(hi ? y[0] : y[2]), 0x4E, 0xf, 0xf, true));
    const float t1 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(hi ? y[1] : y[3]), 0x4E, 0xf, 0xf, true));
    x[0] = hi ? t0 : y[0];
    x[1] = hi ? t1 : y[1];
    x[2] = hi ? y[2] : t0;
    x[3] = hi ? y[3] : t1;
  }

  // D = alpha * acc + beta * C for the wave's block at (r0, c0).
  //
  // Accumulator element 4g + r of 32x32 block (fm, fn) is D[8g + 4h + r][c] of
  // the block for lane (h, c) = (lane / 32, lane % 32).  A 4 x 4 transpose in
  // each quad of lanes (c = 4j .. 4j+3) gives lane (h, 4j + q) row 8g + 4h + q,
  // columns 4j .. 4j+3, so C is read and D written as 16-byte vectors: a
  // dword access costs the address unit as much as a 16-byte one.
  //
  // With 32-bit addressing C is read through a buffer resource from (r0, c0)
  // to the end of C: rows past M read as zero, so the loads need no branch.
  // The block is written in chunks of EPI_ROWS 32-row groups, and all C
  // vectors of the next chunk (two, for blocks of three or more chunks) are
  // requested before the current one is written, so their latencies overlap.  Stores go through the same kind of resource; columns that cross
  // N go element by element.
  // D = alpha * acc + beta * C for a wave block two 32-column blocks wide (FN == 2), written so
  // that one 16-byte access instruction covers 4 rows x 64 columns (256 contiguous bytes of each
  // row) instead of 8 rows x 32 columns.  After the quad transpose, lane (h, c) holds row
  // 8g + 4h + (c & 3) of both column blocks; one v_permlane32_swap per value then gives every
  // lane rows 8g + (c & 3) and 8g + 4 + (c & 3), lanes 0..31 of column block 0 and lanes 32..63
  // of block 1.  Rows of tightly packed matrices (ldc = ldd = N) seldom start on a 128-byte line,
  // and 256 contiguous bytes of such a row span 3 lines where two separate 128-byte pieces span
  // 4: C reads and D writes make a quarter fewer L1 -> L2 requests.  Loading C, multiplying and
  // storing follow store_tile (chunks of EPI_ROWS accumulator rows, the next chunks' C requested
  // ahead).
  __device__ __forceinline__ static void store_pairs(const gg_device_problem_desc& p, int r0, int c0, int lane,
                                                     const floatx16_t (&acc)[FM][FN], bool use_c) {
    static_assert(FN == 2, "two 32-column blocks");
    const int q = lane & 3;
    const int col = 32 * (lane >> 5) + ((lane & 31) & ~3);  // first of the lane's 4 columns in the block
    const int ncol = p.n - (c0 + col);                        // how many of them lie inside the matrix
    const __amdgpu_buffer_rsrc_t drs =
        buffer_rsrc(p.d + ((int64_t)r0 * p.ldd + c0), 4 * ((int64_t)(p.m - 1 - r0) * p.ldd + (p.n - c0)));
    constexpr int CHUNKS = FM / EPI_ROWS;
    constexpr int AHEAD = CHUNKS >= 3 ? GG_EPI_AHEAD : 1;
    // C vectors of a chunk: [accumulator row][row group g][rows 8g + q, 8g + 4 + q].
    floatx4_t cv[AHEAD + 1][EPI_ROWS][4][2];
    auto load_c = [&](int chunk, floatx4_t (&dst)[EPI_ROWS][4][2]) {
      if (use_c) {
        const __amdgpu_buffer_rsrc_t crs =
            buffer_rsrc(p.c + ((int64_t)r0 * p.ldc + c0), 4 * ((int64_t)(p.m - 1 - r0) * p.ldc + (p.n - c0)));
#pragma unroll
        for (int i = 0; i < EPI_ROWS; ++i)
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
              const int row = (chunk * EPI_ROWS + i) * 32 + 8 * g + 4 * hf + q;
              // Vectors wholly past N would read the next row's head: an offset past the resource.
              const uint32_t off =
                  ncol > 0 ? 4u * ((uint32_t)row * (uint32_t)p.ldc + col) : DmaLoader<G>::kOutOfRange;
              dst[i][g][hf] =
                  __builtin_bit_cast(floatx4_t, __builtin_amdgcn_raw_buffer_load_b128(crs, (int)off, 0, 0));
            }
      } else {
#pragma unroll
        for (int i = 0; i < EPI_ROWS; ++i)
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) dst[i][g][hf] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
    };
#pragma unroll
    for (int c = 0; c < AHEAD; ++c) {
      if (c < CHUNKS) load_c(c, cv[c]);
    }
#pragma unroll
    for (int chunk = 0; chunk < CHUNKS; ++chunk) {
      if (chunk + AHEAD < CHUNKS) load_c(chunk + AHEAD, cv[(chunk + AHEAD) % (AHEAD + 1)]);
#pragma unroll
      for (int i = 0; i < EPI_ROWS; ++i) {
        const int fm = chunk * EPI_ROWS + i;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float v0[4] = {acc[fm][0][4 * g + 0], acc[fm][0][4 * g + 1], acc[fm][0][4 * g + 2], acc[fm][0][4 * g + 3]};
          float v1[4] = {acc[fm][1][4 * g + 0], acc[fm][1][4 * g + 1], acc[fm][1][4 * g + 2], acc[fm][1][4 * g + 3]};
          quad_transpose(v0, q);
          quad_transpose(v1, q);
          float vh[2][4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v0[e]), __float_as_uint(v1[e]), false,
                                                            false);
            vh[0][e] = __uint_as_float(r[0]);
            vh[1][e] = __uint_as_float(r[1]);
          }
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int row = fm * 32 + 8 * g + 4 * hf + q;
            floatx4_t out;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              out[e] = epilogue_value(vh[hf][e], cv[chunk % (AHEAD + 1)][i][g][hf][e], p.alpha, use_c ? p.beta : 0.0f);
            }
            if (r0 + row >= p.m || ncol <= 0) continue;
            const uint32_t off = 4u * ((uint32_t)row * (uint32_t)p.ldd + col);
            if (ncol >= 4) {
              __builtin_amdgcn_raw_buffer_store_b128(
                  __builtin_bit_cast(__attribute__((ext_vector_type(4))) int, out), drs, (int)off, 0, 0);
            } else {
#pragma unroll
              for (int e = 0; e < 3; ++e) {
                if (e < ncol) __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(out[e]), drs, (int)(off + 4 * e), 0, 0);
              }
            }
          }
        }
      }
      // Keep each chunk's loads and stores in place (see store_tile).
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  template <bool WIDE>
  __device__ __forceinline__ static void store_tile(const gg_device_problem_desc& p, int r0, int c0, int lane,
                                                    const floatx16_t (&acc)[FM][FN]) {
    const bool use_c = p.c != nullptr && p.beta != 0.0f;
    const int q = lane & 3;
    const int lrow = 4 * (lane >> 5) + q;  // row within an 8-row group
    const int lcol = (lane & 31) & ~3;     // first column of the lane's vector
    if constexpr (!WIDE && FN == 2) {
      store_pairs(p, r0, c0, lane, acc, use_c);
    } else if constexpr (!WIDE) {
      const __amdgpu_buffer_rsrc_t drs =
          buffer_rsrc(p.d + ((int64_t)r0 * p.ldd + c0), 4 * ((int64_t)(p.m - 1 - r0) * p.ldd + (p.n - c0)));
      // C vectors of EPI_ROWS 32-row groups per chunk; the C of the next
      // AHEAD chunks is requested before the current chunk is stored.
      constexpr int CHUNKS = FM / EPI_ROWS;
      constexpr int AHEAD = CHUNKS >= 3 ? GG_EPI_AHEAD : 1;  // chunks of C requested ahead
      floatx4_t cv[AHEAD + 1][EPI_ROWS][FN][4];
      auto load_c = [&](int chunk, floatx4_t (&dst)[EPI_ROWS][FN][4]) {
        if (use_c) {
          const __amdgpu_buffer_rsrc_t crs =
              buffer_rsrc(p.c + ((int64_t)r0 * p.ldc + c0), 4 * ((int64_t)(p.m - 1 - r0) * p.ldc + (p.n - c0)));
#pragma unroll
          for (int i = 0; i < EPI_ROWS; ++i)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                const int fm = chunk * EPI_ROWS + i;
                // Vectors wholly past N would read the next row's head (inside
                // the resource) for nothing: they take an offset past it.
                const bool in_n = c0 + fn * 32 + lcol < p.n;
                const uint32_t off =
                    in_n ? 4u * ((uint32_t)(fm * 32 + 8 * g + lrow) * (uint32_t)p.ldc + fn * 32 + lcol)
                         : DmaLoader<G>::kOutOfRange;
                dst[i][fn][g] = __builtin_bit_cast(floatx4_t, __builtin_amdgcn_raw_buffer_load_b128(crs, (int)off, 0, 0));
              }
        } else {
#pragma unroll
          for (int i = 0; i < EPI_ROWS; ++i)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
#pragma unroll
              for (int g = 0; g < 4; ++g) dst[i][fn][g] = floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
        }
      };
#pragma unroll
      for (int c = 0; c < AHEAD; ++c) {
        if (c < CHUNKS) load_c(c, cv[c]);
      }
#pragma unroll
      for (int chunk = 0; chunk < CHUNKS; ++chunk) {
        if (chunk + AHEAD < CHUNKS) load_c(chunk + AHEAD, cv[(chunk + AHEAD) % (AHEAD + 1)]);
#pragma unroll
        for (int i = 0; i < EPI_ROWS; ++i) {
          const int fm = chunk * EPI_ROWS + i;
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) {
            const int ncol = p.n - (c0 + fn * 32 + lcol);  // columns of the vector inside the matrix
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              float v[4] = {acc[fm][fn][4 * g + 0], acc[fm][fn][4 * g + 1], acc[fm][fn][4 * g + 2],
                            acc[fm][fn][4 * g + 3]};
              quad_transpose(v, q);
              const int rrow = fm * 32 + 8 * g + lrow;
              floatx4_t out;
#pragma unroll
              for (int e = 0; e < 4; ++e) out[e] = epilogue_value(v[e], cv[chunk % (AHEAD + 1)][i][fn][g][e], p.alpha, use_c ? p.beta : 0.0f);
              if (r0 + rrow >= p.m || ncol <= 0) continue;
              const uint32_t off = 4u * ((uint32_t)rrow * (uint32_t)p.ldd + fn * 32 + lcol);
              if (ncol >= 4) {
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(__attribute__((ext_vector_type(4))) int, out), drs, (int)off, 0, 0);
              } else {
#pragma unroll
                for (int e = 0; e < 3; ++e) {
                  if (e < ncol) __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(out[e]), drs, (int)(off + 4 * e), 0, 0);
                }
              }
            }
          }
        }
        // Keep each chunk's loads and stores in place: hoisting every C load
        // to the top would hold the whole block's C in registers.
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          const int col = c0 + fn * 32 + lcol;
          const int ncol = p.n - col;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            float v[4] = {acc[fm][fn][4 * g + 0], acc[fm][fn][4 * g + 1], acc[fm][fn][4 * g + 2],
                          acc[fm][fn][4 * g + 3]};
            quad_transpose(v, q);
            const int row = r0 + fm * 32 + 8 * g + lrow;
            if (row >= p.m || ncol <= 0) continue;
            g_cf32_t* crow = (g_cf32_t*)p.c + ((int64_t)row * p.ldc + col);
            g_f32_t* drow = (g_f32_t*)p.d + ((int64_t)row * p.ldd + col);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (e < ncol) drow[e] = epilogue_value(v[e], use_c ? crow[e] : 0.0f, p.alpha, use_c ? p.beta : 0.0f);
            }
          }
        }
      }
    }
  }
};

// ---------------------------------------------------------------------------
// FMA tile: 256 threads as a 16 x 16 grid, thread (tm, tn) owns rows
// tm*RM .. tm*RM+RM-1 and columns tn*RN .. tn*RN+RN-1 of the macro-tile, with
// RM = BM/16, RN = BN/16 float32 accumulators.  Per 8-deep k slice a thread
// reads one 16-byte piece of each of its A rows and one RN-wide piece of each
// B row from LDS, then issues RM*RN*8 fused multiply-adds in ascending k.
// Used when MFMA is not requested (use_tensor_cores = false).
// ---------------------------------------------------------------------------
template <class G>
struct FmaTile {
  static constexpr int RM = G::BM / 16;
  static constexpr int RN = G::BN / 16;
  static_assert(RN == 4 || RN == 8, "column block must be one or two LDS chunks");
  static_assert(G::THREADS == 256, "16 x 16 thread grid");

  __device__ __forceinline__ static void compute_stage(const uint16_t* stage, int krem, int tm, int tn,
                                                       float (&acc)[RM][RN]) {
    const uint16_t* as = stage;
    const uint16_t* bs = stage + G::A_STAGE;
#pragma unroll
    for (int k8 = 0; k8 < G::BK / 8; ++k8) {
      if (k8 * 8 >= krem) break;
      half8_t av[RM];
#pragma unroll
      for (int i = 0; i < RM; ++i) {
        av[i] = *reinterpret_cast<const half8_t*>(as + G::a_piece(tm * RM + i, k8));
      }
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const uint16_t* brow = bs + G::b_chunk(k8 * 8 + kk, tn * RN);
        float bv[RN];
        if constexpr (RN == 4) {
          const half4_t h = *reinterpret_cast<const half4_t*>(brow);
#pragma unroll
          for (int j = 0; j < RN; ++j) bv[j] = (float)h[j];
        } else {
          const half8_t h = *reinterpret_cast<const half8_t*>(brow);
#pragma unroll
          for (int j = 0; j < RN; ++j) bv[j] = (float)h[j];
        }
#pragma unroll
        for (int i = 0; i < RM; ++i) {
          const float a = (float)av[i][kk];
#pragma unroll
          for (int j = 0; j < RN; ++j) acc[i][j] = __builtin_fmaf(a, bv[j], acc[i][j]);
        }
      }
    }
  }

  // Computes the work tile at (m0, n0); on_start and after_k_loop as in
  // MfmaTile::run.
  template <bool WIDE, class OnStart, class AfterKLoop, class Stamps>
  __device__ __forceinline__ static void run(const gg_device_problem_desc& p, int m0, int n0, uint16_t* lds,
                                             OnStart&& on_start, AfterKLoop&& after_k_loop, const Stamps& stamps) {
    const int tid = threadIdx.x;
    const int tm = tid >> 4;
    const int tn = tid & 15;
    // Wave w holds tm = 4w .. 4w+3, i.e. rows [4w*RM, 4w*RM + 4*RM) of the tile.
    const bool active = m0 + (tid / kWave) * 4 * RM < p.m;

    float acc[RM][RN];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
      for (int j = 0; j < RN; ++j) acc[i][j] = 0.0f;

    int kt = 0;
    run_k_loop<G, WIDE>(p, m0, n0, lds, [&](const uint16_t* stage) {
      if (active) compute_stage(stage, p.k - kt * G::BK, tm, tn, acc);
      ++kt;
    }, on_start, stamps);
    after_k_loop();

    if (!active) {
      stamps.wave_done();
      return;
    }
    const bool use_c = p.c != nullptr && p.beta != 0.0f;
    g_cf32_t* cptr = (g_cf32_t*)p.c;
    g_f32_t* dptr = (g_f32_t*)p.d;
#pragma unroll
    for (int i = 0; i < RM; ++i) {
      const int row = m0 + tm * RM + i;
      if (row >= p.m) continue;
      float cv[RN];
#pragma unroll
      for (int j = 0; j < RN; ++j) {
        const int col = n0 + tn * RN + j;
        cv[j] = (use_c && col < p.n) ? cptr[(int64_t)row * p.ldc + col] : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < RN; ++j) {
        const int col = n0 + tn * RN + j;
        if (col < p.n) dptr[(int64_t)row * p.ldd + col] = epilogue_value(acc[i][j], cv[j], p.alpha, use_c ? p.beta : 0.0f);
      }
    }
    stamps.wave_done();
  }
};

// The tile code of kernel shape S (gg_common.h).
template <class S, int PATH> struct TileFor;
template <class S> struct TileFor<S, GGK_PATH_MFMA> { using type = MfmaTile<typename S::G, S::WAVE_M>; };
template <class S> struct TileFor<S, GGK_PATH_FMA> { using type = FmaTile<typename S::G>; };

// LDS (binary16 values) a kernel of shape S needs: the largest stage ring of
// the forms its work tiles take.
template <class S, bool CLASSES = S::CLASSES>
struct KernelLds {
  static constexpr int HALVES = S::G::LDS_HALVES;
};
template <class S>
struct KernelLds<S, true> {
  static constexpr int a = S::G::LDS_HALVES, r = S::GR::LDS_HALVES, c = S::GC::LDS_HALVES, rc = S::GRC::LDS_HALVES;
  static constexpr int ab = a > r ? a : r;
  static constexpr int cd = c > rc ? c : rc;
  static constexpr int HALVES = ab > cd ? ab : cd;
  static_assert(2 * HALVES <= 150 * 1024, "the stage rings and the scheduler's words fit the 160 KB of LDS");
};

// Computes the work tile at (m0, n0): in the edge class its extent inside the
// problem selects (KernelShape::CLASSES), else in the kernel's own form.  The
// class is uniform across the workgroup (scalar descriptor and origin).
template <class S, int PATH, bool WIDE, class OnStart, class AfterKLoop, class Stamps = NoStamps>
__device__ __forceinline__ void run_work_tile(const gg_device_problem_desc& p, int m0, int n0, uint16_t* lds,
                                              OnStart&& on_start, AfterKLoop&& after_k_loop,
                                              const Stamps& stamps = Stamps{}) {
  if constexpr (PATH == GGK_PATH_MFMA && !WIDE && S::CLASSES) {
    const bool rows = p.m - m0 <= S::G::BM / 2;
    const bool cols = p.n - n0 <= S::G::BN / 2;
    // The full form first: its code then follows the dispatch as it would
    // without the edge classes.
    if (__builtin_expect(!rows && !cols, 1)) {
      TileFor<S, PATH>::type::template run<false>(p, m0, n0, lds, on_start, after_k_loop, stamps);
    } else if (!cols) {
      MfmaTile<typename S::GR, S::WAVE_M_R>::template run<false>(p, m0, n0, lds, on_start, after_k_loop, stamps);
    } else if (!rows) {
      MfmaTile<typename S::GC, S::WAVE_M_C>::template run<false>(p, m0, n0, lds, on_start, after_k_loop, stamps);
    } else {
      MfmaTile<typename S::GRC, S::WAVE_M_RC>::template run<false>(p, m0, n0, lds, on_start, after_k_loop, stamps);
    }
  } else {
    TileFor<S, PATH>::type::template run<WIDE>(p, m0, n0, lds, on_start, after_k_loop, stamps);
  }
}

}  // namespace gg
