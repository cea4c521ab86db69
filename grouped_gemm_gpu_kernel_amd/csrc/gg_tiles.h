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
// per stage with that stage's LDS buffer.
//
// Stage s is fetched into register set s % DEPTH.  While stage k is
// multiplied out of LDS buffer k % 2, the loads of stage k + DEPTH - 1 are
// issued and stage k + 1 (issued DEPTH - 1 stages earlier) is written to the
// other LDS buffer; one barrier closes the step.  The loop body is unrolled
// DEPTH times so that every register set is addressed statically.
template <class G, class Compute>
__device__ __forceinline__ void run_k_loop(const gg_device_problem_desc& p, int m0, int n0, uint16_t* lds,
                                           Compute&& compute) {
  constexpr int D = G::DEPTH;
  const int nk = (p.k + G::BK - 1) / G::BK;
  if (nk <= 0) return;
  const StageLoader<G> loader(p, m0, n0);
  RawStage<G> ring[D];
#pragma unroll
  for (int s = 0; s < D - 1; ++s) {
    if (s < nk) loader.issue(s, ring[s]);
  }
  loader.store(ring[0], 0, lds, 0);
  __syncthreads();
  for (int k0 = 0; k0 < nk; k0 += D) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int k = k0 + u;
      if (k < nk) {
        if (k + D - 1 < nk) loader.issue(k + D - 1, ring[(u + D - 1) % D]);
        compute(lds + (k & 1) * G::STAGE);
        if (k + 1 < nk) loader.store(ring[(u + 1) % D], k + 1, lds, (k + 1) & 1);
        __syncthreads();
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA tile: v_mfma_f32_32x32x16_f16, 4 waves in a 2 x 2 grid, each wave owns a
// (BM/2) x (BN/2) block of D held as (BM/64) x (BN/64) 32x32 accumulators.
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
template <class G>
struct MfmaTile {
  static constexpr int WM = G::BM / 2;
  static constexpr int WN = G::BN / 2;
  static constexpr int FM = WM / 32;
  static constexpr int FN = WN / 32;
  static_assert(FM >= 1 && FN >= 1, "wave tile must hold whole 32x32 blocks");

  // Multiplies one LDS stage into acc.  Every wave runs every MFMA of the
  // stage, also over zero padding: a branch around the MFMAs would make the
  // accumulators flow through control-flow joins, which costs a copy of all of
  // them out of and back into the accumulation registers per stage.
  __device__ __forceinline__ static void compute_stage(const uint16_t* stage, int lane, int wm, int wn,
                                                       floatx16_t (&acc)[FM][FN]) {
    const uint16_t* as = stage;
    const uint16_t* bs = stage + G::A_STAGE;
    const int g = lane >> 4;
    const int j = lane & 15;
#pragma unroll
    for (int s = 0; s < G::BK / 16; ++s) {
      half8_t af[FM];
      half8_t bf[FN];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const uint16_t* src = as + (wm * WM + fm * 32 + (lane & 31)) * G::SA + s * 16 + (lane >> 5) * 8;
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
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[fm], bf[fn], acc[fm][fn], 0, 0, 0);
        }
      }
    }
  }

  __device__ __forceinline__ static void run(const gg_device_problem_desc& p, int tile_m, int tile_n,
                                             uint16_t* lds) {
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int wm = wave >> 1;
    const int wn = wave & 1;
    const int m0 = tile_m * G::BM;
    const int n0 = tile_n * G::BN;

    floatx16_t acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[fm][fn][e] = 0.0f;

    run_k_loop<G>(p, m0, n0, lds, [&](const uint16_t* stage) { compute_stage(stage, lane, wm, wn, acc); });

    // A wave whose block starts past the problem's edge multiplied zeros and
    // stores nothing.
    if (m0 + wm * WM >= p.m || n0 + wn * WN >= p.n) return;
    const bool use_c = p.c != nullptr && p.beta != 0.0f;
    g_cf32_t* cptr = (g_cf32_t*)p.c;
    g_f32_t* dptr = (g_f32_t*)p.d;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int col = n0 + wn * WN + fn * 32 + (lane & 31);
        const int row0 = m0 + wm * WM + fm * 32 + 4 * (lane >> 5);
        const bool col_ok = col < p.n;
        float cv[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = row0 + 8 * (e >> 2) + (e & 3);
          cv[e] = (use_c && col_ok && row < p.m) ? cptr[(int64_t)row * p.ldc + col] : 0.0f;
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = row0 + 8 * (e >> 2) + (e & 3);
          if (col_ok && row < p.m) {
            dptr[(int64_t)row * p.ldd + col] = epilogue_value(acc[fm][fn][e], cv[e], p.alpha, p.beta);
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
        av[i] = *reinterpret_cast<const half8_t*>(as + (tm * RM + i) * G::SA + k8 * 8);
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

  __device__ __forceinline__ static void run(const gg_device_problem_desc& p, int tile_m, int tile_n,
                                             uint16_t* lds) {
    const int tid = threadIdx.x;
    const int tm = tid >> 4;
    const int tn = tid & 15;
    const int m0 = tile_m * G::BM;
    const int n0 = tile_n * G::BN;
    // Wave w holds tm = 4w .. 4w+3, i.e. rows [4w*RM, 4w*RM + 4*RM) of the tile.
    const bool active = m0 + (tid / kWave) * 4 * RM < p.m;

    float acc[RM][RN];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
      for (int j = 0; j < RN; ++j) acc[i][j] = 0.0f;

    int kt = 0;
    run_k_loop<G>(p, m0, n0, lds, [&](const uint16_t* stage) {
      if (active) compute_stage(stage, p.k - kt * G::BK, tm, tn, acc);
      ++kt;
    });

    if (!active) return;
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
        if (col < p.n) dptr[(int64_t)row * p.ldd + col] = epilogue_value(acc[i][j], cv[j], p.alpha, p.beta);
      }
    }
  }
};

template <int PATH, class G> struct TileFor;
template <class G> struct TileFor<GGK_PATH_MFMA, G> { using type = MfmaTile<G>; };
template <class G> struct TileFor<GGK_PATH_FMA, G> { using type = FmaTile<G>; };

}  // namespace gg
