// gg_common.h -- shared device definitions for the gfx950 grouped GEMM kernels:
// vector types, macro-tile geometry, and the global -> LDS staging of A and B.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "grouped_gemm_amd_kernels.h"

namespace gg {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#define GG_LDS __attribute__((address_space(3)))
#define GG_CONST __attribute__((address_space(4)))

constexpr int kThreads = 256;  // 4 wave64 per workgroup
constexpr int kWave = 64;

// Macro-tile geometry of one variant.  BM x BN is the tile of D a workgroup
// owns (it fixes the tile -> problem mapping, src/grouped_gemm.cu:54-65,666-668);
// BK is the depth of one LDS stage, an internal choice.
//
// LDS layout per stage (binary16):
//   A: BM rows x SA, row-major as in global memory (k contiguous); SA = BK + 8
//      keeps the 16-byte MFMA operand reads of 16 consecutive rows on distinct
//      banks.
//   B: BK rows x SB, row-major as in global memory (n contiguous); SB = BN + 32
//      puts the four k-rows one transposing read touches on disjoint banks.
template <int BM_, int BN_, int BK_>
struct Geometry {
  static constexpr int BM = BM_;
  static constexpr int BN = BN_;
  static constexpr int BK = BK_;
  static constexpr int SA = BK + 8;
  static constexpr int SB = BN + 32;
  static constexpr int A_STAGE = BM * SA;  // halves
  static constexpr int B_STAGE = BK * SB;  // halves
  static constexpr int STAGE = A_STAGE + B_STAGE;
  static constexpr int LDS_HALVES = 2 * STAGE;  // double buffered
  // 16-byte vectors per stage and per thread.
  static constexpr int A_VECS = BM * BK / 8;
  static constexpr int B_VECS = BK * BN / 8;
  static constexpr int A_PER_THREAD = A_VECS / kThreads;
  static constexpr int B_PER_THREAD = B_VECS / kThreads;
  static_assert(A_VECS % kThreads == 0 && B_VECS % kThreads == 0, "staging must split evenly");
  static_assert(BK % 16 == 0, "stage depth must be a multiple of the MFMA k");
};

// Variant -> geometry (ids follow GGK_VARIANT_*).
template <int V> struct VariantGeometry;
template <> struct VariantGeometry<GGK_VARIANT_64x64x16> { using type = Geometry<64, 64, 32>; };
template <> struct VariantGeometry<GGK_VARIANT_128x64x32> { using type = Geometry<128, 64, 32>; };
template <> struct VariantGeometry<GGK_VARIANT_64x128x32> { using type = Geometry<64, 128, 32>; };

// Global-memory views.  Descriptor pointers arrive as generic pointers; the
// kernels only ever point them at device memory, so they are read and written
// through the global address space (no flat instructions).
typedef __attribute__((address_space(1))) const uint32_t g_u32_t;
typedef __attribute__((address_space(1))) const float g_cf32_t;
typedef __attribute__((address_space(1))) float g_f32_t;

// One 16-byte piece of a row: 8 consecutive binary16 values of row `row`,
// columns [col, col + 8), of a row-major matrix with leading dimension ld;
// values outside rows x cols read as 0.
//
// Rows of a tightly packed matrix with odd ld start on 2-byte boundaries, so a
// 16-byte load is not always possible.  The piece is fetched as the five
// dwords from the 4-byte aligned address q at or below it; a dword that holds
// none of the wanted bytes is instead fetched from q itself (always a wanted
// dword), so every access stays inside the matrix, and is zeroed later.  A
// piece with no valid value fetches the matrix's first dword.  Splitting the
// fetch (issue_piece) from the realignment (finish_piece) lets the loads stay
// in flight while the previous stage is being multiplied.
struct RawPiece {
  uint32_t w[5];
  uint32_t lead;    // bytes between q and the first wanted value: 0 or 2
  uint32_t nvalid;  // valid values in the piece, 0..8
};

__device__ __forceinline__ void issue_piece(const uint16_t* base, int ld, int rows, int cols, int row,
                                            int col, RawPiece& out) {
  int nvalid = cols - col;
  nvalid = nvalid < 0 ? 0 : (nvalid > 8 ? 8 : nvalid);
  if (row >= rows) nvalid = 0;
  const uint16_t* p = nvalid > 0 ? base + (int64_t)row * ld + col : base;
  const uintptr_t addr = reinterpret_cast<uintptr_t>(p);
  const uintptr_t q = addr & ~uintptr_t(3);
  const uint32_t lead = (uint32_t)(addr - q);
  const uint32_t span = lead + 2u * (uint32_t)nvalid;  // wanted bytes counted from q
  if (nvalid == 8) {
    // Full piece: dwords 0-3 all hold wanted bytes; dword 4 only when lead == 2.
    const u32x4_t v = *(__attribute__((address_space(1))) const u32x4_t*)q;
    out.w[0] = v.x;
    out.w[1] = v.y;
    out.w[2] = v.z;
    out.w[3] = v.w;
    out.w[4] = *(g_u32_t*)(lead != 0 ? q + 16u : q);
  } else {
    // Right edge or outside the matrix.
#pragma unroll
    for (int i = 0; i < 5; ++i) {
      const uintptr_t a = (4u * i < span) ? q + 4u * i : q;
      out.w[i] = *(g_u32_t*)a;
    }
  }
  out.lead = lead;
  out.nvalid = (uint32_t)nvalid;
}

__device__ __forceinline__ u32x4_t finish_piece(const RawPiece& r) {
  const uint32_t span = r.lead + 2u * r.nvalid;
  uint32_t w[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) w[i] = (4u * i < span) ? r.w[i] : 0u;
  u32x4_t out;
  out.x = __builtin_amdgcn_alignbyte(w[1], w[0], r.lead);
  out.y = __builtin_amdgcn_alignbyte(w[2], w[1], r.lead);
  out.z = __builtin_amdgcn_alignbyte(w[3], w[2], r.lead);
  out.w = __builtin_amdgcn_alignbyte(w[4], w[3], r.lead);
  // Clear values past nvalid (the right edge of the matrix).
  const uint32_t n = r.nvalid;
  out.x &= (n >= 2) ? 0xffffffffu : (n == 1 ? 0xffffu : 0u);
  out.y &= (n >= 4) ? 0xffffffffu : (n == 3 ? 0xffffu : 0u);
  out.z &= (n >= 6) ? 0xffffffffu : (n == 5 ? 0xffffu : 0u);
  out.w &= (n >= 8) ? 0xffffffffu : (n == 7 ? 0xffffu : 0u);
  return out;
}

// Register staging of one LDS stage: the A and B pieces this thread moves.
template <class G>
struct StageRegs {
  RawPiece a[G::A_PER_THREAD];
  RawPiece b[G::B_PER_THREAD];
};

// Issues the loads of stage kt of tile (m0, n0).  A piece v covers row
// v / (BK/8), columns 8 * (v % (BK/8)); B piece v covers k-row v / (BN/8),
// columns 8 * (v % (BN/8)).  Consecutive threads read consecutive pieces of
// one row.
template <class G>
__device__ __forceinline__ void load_stage(const gg_device_problem_desc& p, int m0, int n0, int kt,
                                           StageRegs<G>& r) {
  const int tid = threadIdx.x;
  const int k0 = kt * G::BK;
  const uint16_t* a = static_cast<const uint16_t*>(p.a);
  const uint16_t* b = static_cast<const uint16_t*>(p.b);
#pragma unroll
  for (int i = 0; i < G::A_PER_THREAD; ++i) {
    const int v = tid + i * kThreads;
    const int row = v / (G::BK / 8);
    const int c8 = v % (G::BK / 8);
    issue_piece(a, p.lda, p.m, p.k, m0 + row, k0 + c8 * 8, r.a[i]);
  }
#pragma unroll
  for (int i = 0; i < G::B_PER_THREAD; ++i) {
    const int v = tid + i * kThreads;
    const int krow = v / (G::BN / 8);
    const int c8 = v % (G::BN / 8);
    issue_piece(b, p.ldb, p.k, p.n, k0 + krow, n0 + c8 * 8, r.b[i]);
  }
}

// Realigns the staged pieces and writes them into LDS stage `s` (16-byte stores).
template <class G>
__device__ __forceinline__ void store_stage(uint16_t* lds, int s, const StageRegs<G>& r) {
  const int tid = threadIdx.x;
  uint16_t* as = lds + s * G::STAGE;
  uint16_t* bs = as + G::A_STAGE;
#pragma unroll
  for (int i = 0; i < G::A_PER_THREAD; ++i) {
    const int v = tid + i * kThreads;
    const int row = v / (G::BK / 8);
    const int c8 = v % (G::BK / 8);
    *reinterpret_cast<u32x4_t*>(as + row * G::SA + c8 * 8) = finish_piece(r.a[i]);
  }
#pragma unroll
  for (int i = 0; i < G::B_PER_THREAD; ++i) {
    const int v = tid + i * kThreads;
    const int krow = v / (G::BN / 8);
    const int c8 = v % (G::BN / 8);
    *reinterpret_cast<u32x4_t*>(bs + krow * G::SB + c8 * 8) = finish_piece(r.b[i]);
  }
}

// D = alpha * acc + beta * C for one element; C is read only when c != nullptr
// and beta != 0 (src/grouped_gemm.cu:475-479, 616-621).
__device__ __forceinline__ float epilogue_value(float acc, float c, float alpha, float beta) {
  return alpha * acc + beta * c;
}

}  // namespace gg
