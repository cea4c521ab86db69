// gg_common.h -- shared device definitions for the gfx950 grouped GEMM kernels:
// vector types, macro-tile geometry and LDS layout, and the global -> LDS
// staging of A and B.
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
// LDS layout of one stage (binary16), double buffered:
//   A: BM rows of SA = BK + 8 values, row-major as in global memory.  The 8
//      values of padding put the 16-byte operand reads of 16 consecutive rows
//      on distinct banks.
//   B: BK rows of BN values, row-major as in global memory, with the 8-byte
//      chunks of row k stored at chunk index (c ^ b_swizzle(k)).  The
//      transposing operand read touches 4 consecutive rows x 16 columns per
//      16 lanes; the swizzle spreads those rows over disjoint banks without
//      padding.  It flips only chunk-index bits >= 3, so 16-byte pieces
//      (2 chunks) stay contiguous and every 32-column block stays intact.
//
// DEPTH stages are in flight in registers at once: the loads of stage k + DEPTH - 1
// are issued while stage k is multiplied (a ring of DEPTH register sets).
template <int BM_, int BN_, int BK_, int DEPTH_>
struct Geometry {
  static constexpr int BM = BM_;
  static constexpr int BN = BN_;
  static constexpr int BK = BK_;
  static constexpr int DEPTH = DEPTH_;
  static_assert(DEPTH >= 2, "at least one stage must be in flight while another is multiplied");
  static constexpr int SA = BK + 8;
  static constexpr int SB = BN;
  static constexpr int A_STAGE = BM * SA;  // halves
  static constexpr int B_STAGE = BK * SB;  // halves
  static constexpr int STAGE = A_STAGE + B_STAGE;
  static constexpr int LDS_HALVES = 2 * STAGE;
  // 16-byte pieces per stage and per thread.
  static constexpr int A_VECS = BM * BK / 8;
  static constexpr int B_VECS = BK * BN / 8;
  static constexpr int A_PER_THREAD = A_VECS / kThreads;
  static constexpr int B_PER_THREAD = B_VECS / kThreads;
  static_assert(A_VECS % kThreads == 0 && B_VECS % kThreads == 0, "staging must split evenly");
  static_assert(BK % 16 == 0, "stage depth must be a multiple of the MFMA k");
  static_assert(BN == 64 || BN == 128, "B swizzle is defined for 64- and 128-column tiles");

  // 64 banks x 4 bytes hold 256 bytes: two 64-column rows or one 128-column
  // row.  XOR-ing the chunk index with 8 moves a chunk by 64 bytes, so rows
  // k..k+3 (k a multiple of 4) land on 4 different 64-byte bank windows.
  __device__ static __forceinline__ int b_swizzle(int k) {
    if constexpr (BN == 64) {
      return 8 * ((k >> 1) & 1);
    } else {
      return 8 * (k & 3);
    }
  }
  // Element offset, within a B stage, of the 4-value chunk that holds (k, n)
  // for n a multiple of 4.
  __device__ static __forceinline__ int b_chunk(int k, int n) { return k * SB + 4 * ((n >> 2) ^ b_swizzle(k)); }
};

// Variant -> geometry (ids follow GGK_VARIANT_*).
template <int V> struct VariantGeometry;
#ifndef GG_STAGE_K
#define GG_STAGE_K 64
#endif
#ifndef GG_STAGE_DEPTH
#define GG_STAGE_DEPTH 2
#endif
template <> struct VariantGeometry<GGK_VARIANT_64x64x16> {
  using type = Geometry<64, 64, GG_STAGE_K, GG_STAGE_DEPTH>;
};
template <> struct VariantGeometry<GGK_VARIANT_128x64x32> {
  using type = Geometry<128, 64, GG_STAGE_K, GG_STAGE_DEPTH>;
};
template <> struct VariantGeometry<GGK_VARIANT_64x128x32> {
  using type = Geometry<64, 128, GG_STAGE_K, GG_STAGE_DEPTH>;
};

// Global-memory views.  Descriptor pointers arrive as generic pointers; the
// kernels only ever point them at device memory, so they are read and written
// through the global address space (no flat instructions).
typedef __attribute__((address_space(1))) const uint32_t g_u32_t;
typedef __attribute__((address_space(1))) const u32x4_t g_u32x4_t;
typedef __attribute__((address_space(1))) const float g_cf32_t;
typedef __attribute__((address_space(1))) float g_f32_t;

// One 16-byte piece of a row: 8 consecutive binary16 values.  Rows of a
// tightly packed matrix with odd ld start on 2-byte boundaries, so a 16-byte
// load is not always possible: the piece is fetched as the dwords from the
// 4-byte aligned address q at or below it (16 bytes from q, plus one more
// dword when the piece starts 2 bytes past q) and shifted into place when it
// is written to LDS.  Only the fetched dwords are held while the loads are in
// flight; where the piece starts (lead) and how many of its values lie inside
// the matrix (nvalid) are recomputed when it is written.
struct RawPiece {
  uint32_t w[5];
};

// Placement of a piece that may cross the matrix edge.  A piece with no valid
// value stands on the matrix's first element.
struct EdgePlace {
  const uint16_t* p;
  uint32_t lead;    // bytes between q and the first value: 0 or 2
  uint32_t nvalid;  // values of the piece inside the matrix, 0..8
};

__device__ __forceinline__ EdgePlace edge_place(const uint16_t* base, int ld, int rows, int cols, int row,
                                                int col) {
  int nvalid = cols - col;
  nvalid = nvalid < 0 ? 0 : (nvalid > 8 ? 8 : nvalid);
  if (row >= rows) nvalid = 0;
  const uint16_t* p = nvalid > 0 ? base + (int64_t)row * ld + col : base;
  return EdgePlace{p, (uint32_t)(reinterpret_cast<uintptr_t>(p) & 2), (uint32_t)nvalid};
}

// General fetch: a dword with no wanted byte is fetched from q itself (always
// a wanted dword, or the matrix's first one) and zeroed when the piece is
// finished.  Every access stays inside the matrix.
__device__ __forceinline__ void issue_piece_edge(const EdgePlace& e, RawPiece& out) {
  const uintptr_t q = reinterpret_cast<uintptr_t>(e.p) & ~uintptr_t(3);
  const uint32_t span = e.lead + 2u * e.nvalid;  // wanted bytes counted from q
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const uintptr_t a = (4u * i < span) ? q + 4u * i : q;
    out.w[i] = *(g_u32_t*)a;
  }
}

// Fast fetch of a piece known to lie inside its row: 16 bytes from q and,
// when the piece starts 2 bytes past q, the dword after them (otherwise the
// first dword again, which the shift ignores).
__device__ __forceinline__ void issue_piece_inside(const uint16_t* p, RawPiece& out) {
  const uintptr_t addr = reinterpret_cast<uintptr_t>(p);
  const uintptr_t q = addr & ~uintptr_t(3);
  const u32x4_t v = *(g_u32x4_t*)q;
  out.w[0] = v.x;
  out.w[1] = v.y;
  out.w[2] = v.z;
  out.w[3] = v.w;
  out.w[4] = *(g_u32_t*)(q + 8u * (uint32_t)(addr & 2));
}

// Shifts a fetched piece into place.  `edge` selects the general form, which
// also clears dwords that were fetched as stand-ins and values past nvalid;
// otherwise nvalid is 8 or 0 (a row past the matrix edge).
__device__ __forceinline__ u32x4_t finish_piece(const RawPiece& r, uint32_t lead, uint32_t nvalid, bool edge) {
  uint32_t w[5];
  if (edge) {
    const uint32_t span = lead + 2u * nvalid;
#pragma unroll
    for (int i = 0; i < 5; ++i) w[i] = (4u * i < span) ? r.w[i] : 0u;
  } else {
#pragma unroll
    for (int i = 0; i < 5; ++i) w[i] = r.w[i];
  }
  u32x4_t out;
  out.x = __builtin_amdgcn_alignbyte(w[1], w[0], lead);
  out.y = __builtin_amdgcn_alignbyte(w[2], w[1], lead);
  out.z = __builtin_amdgcn_alignbyte(w[3], w[2], lead);
  out.w = __builtin_amdgcn_alignbyte(w[4], w[3], lead);
  const uint32_t n = nvalid;
  if (edge) {
    out.x &= (n >= 2) ? 0xffffffffu : (n == 1 ? 0xffffu : 0u);
    out.y &= (n >= 4) ? 0xffffffffu : (n == 3 ? 0xffffu : 0u);
    out.z &= (n >= 6) ? 0xffffffffu : (n == 5 ? 0xffffu : 0u);
    out.w &= (n >= 8) ? 0xffffffffu : (n == 7 ? 0xffffu : 0u);
  } else {
    const uint32_t keep = n != 0 ? 0xffffffffu : 0u;
    out.x &= keep;
    out.y &= keep;
    out.z &= keep;
    out.w &= keep;
  }
  return out;
}

// The loads of one stage in flight: this thread's A and B pieces.
template <class G>
struct RawStage {
  RawPiece a[G::A_PER_THREAD];
  RawPiece b[G::B_PER_THREAD];
};

// Moves the A and B stages of one tile from global memory into LDS.
//
// A piece v (v = tid + 256 i) covers tile row v / (BK/8), columns
// 8 * (v % (BK/8)) of the stage; B piece v covers k-row v / (BN/8), columns
// 8 * (v % (BN/8)).  Consecutive threads read consecutive pieces of one row.
//
// Inside stages (all k of the stage below K) use an offset form set up once per
// tile: the stage's origin is a wave-uniform byte address (advanced with
// scalar arithmetic) and each piece has a fixed 32-bit byte offset from it, so
// a piece costs two loads and four byte shifts.  Rows of A past M read row m0
// instead, and nothing is masked: those values only reach rows of D past M,
// which are never stored.  B uses the offset form only on tiles whose columns
// all lie inside N.  Every other stage uses the general, masked fetch.
template <class G>
struct StageLoader {
  static constexpr int NA = G::A_PER_THREAD;
  static constexpr int NB = G::B_PER_THREAD;

  const gg_device_problem_desc& p;
  int m0, n0;
  bool a_offsets;          // A offsets of this tile fit in 32 bits
  bool b_offsets;          // B offsets fit in 32 bits and the tile lies inside N
  uintptr_t a_base0;       // 4-byte aligned origin of stage 0; stage kt adds 2*BK*kt bytes
  uintptr_t b_base0;       // stage kt adds 2*BK*ldb*kt bytes
  uint32_t a_off[NA];      // 4-byte aligned offset of piece i from the stage origin
  uint32_t a_off4[NA];     // offset of the piece's fifth dword (a_off[i] itself when not needed)
  uint32_t b_off[NB];
  uint32_t b_off4[NB];
  uint32_t a_lead, b_lead; // 0 or 2; one value per thread (its pieces are 32 rows apart)

  __device__ __forceinline__ StageLoader(const gg_device_problem_desc& prob, int m0_, int n0_)
      : p(prob), m0(m0_), n0(n0_) {
    const int tid = threadIdx.x;
    const uintptr_t A = reinterpret_cast<uintptr_t>(p.a);
    const uintptr_t B = reinterpret_cast<uintptr_t>(p.b);
    a_offsets = (int64_t)G::BM * p.lda < (int64_t(1) << 30);
    b_offsets = n0 + G::BN <= p.n && (int64_t)G::BK * p.ldb < (int64_t(1) << 30);
    a_base0 = (A & ~uintptr_t(3)) + (uintptr_t)((int64_t)m0 * p.lda * 2);
    b_base0 = (B & ~uintptr_t(3)) + (uintptr_t)((int64_t)n0 * 2);
    a_lead = 0;
    b_lead = 0;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int v = tid + i * kThreads;
      const int r = v / (G::BK / 8);
      const uint32_t col_bytes = (uint32_t)(16 * (v % (G::BK / 8))) + (uint32_t)(A & 3);
      const uint32_t rel_real = (uint32_t)r * (uint32_t)p.lda * 2u + col_bytes;
      const uint32_t rel = m0 + r < p.m ? rel_real : col_bytes;  // row m0 stands in
      if (i == 0) a_lead = rel_real & 2u;
      a_off[i] = rel & ~3u;
      a_off4[i] = a_off[i] + 8u * (rel & 2u);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int v = tid + i * kThreads;
      const uint32_t rel = (uint32_t)(v / (G::BN / 8)) * (uint32_t)p.ldb * 2u +
                           (uint32_t)(16 * (v % (G::BN / 8))) + (uint32_t)(B & 3);
      if (i == 0) b_lead = rel & 2u;
      b_off[i] = rel & ~3u;
      b_off4[i] = b_off[i] + 8u * (rel & 2u);
    }
  }

  __device__ __forceinline__ bool a_fast(int kt) const { return a_offsets && (kt + 1) * G::BK <= p.k; }
  __device__ __forceinline__ bool b_fast(int kt) const { return b_offsets && (kt + 1) * G::BK <= p.k; }

  // Placement of A piece i and B piece i of stage kt in the general form.
  __device__ __forceinline__ EdgePlace a_edge(int i, int kt) const {
    const int v = threadIdx.x + i * kThreads;
    return edge_place(static_cast<const uint16_t*>(p.a), p.lda, p.m, p.k, m0 + v / (G::BK / 8),
                      kt * G::BK + 8 * (v % (G::BK / 8)));
  }
  __device__ __forceinline__ EdgePlace b_edge(int i, int kt) const {
    const int v = threadIdx.x + i * kThreads;
    return edge_place(static_cast<const uint16_t*>(p.b), p.ldb, p.k, p.n, kt * G::BK + v / (G::BN / 8),
                      n0 + 8 * (v % (G::BN / 8)));
  }

  static __device__ __forceinline__ void fetch(uintptr_t base, uint32_t off, uint32_t off4, RawPiece& out) {
    const u32x4_t v = *(g_u32x4_t*)(base + off);
    out.w[0] = v.x;
    out.w[1] = v.y;
    out.w[2] = v.z;
    out.w[3] = v.w;
    out.w[4] = *(g_u32_t*)(base + off4);
  }

  // Issues the loads of stage kt into r.
  __device__ __forceinline__ void issue(int kt, RawStage<G>& r) const {
    if (a_fast(kt)) {
      const uintptr_t base = a_base0 + (uintptr_t)(2 * G::BK) * (uintptr_t)kt;
#pragma unroll
      for (int i = 0; i < NA; ++i) fetch(base, a_off[i], a_off4[i], r.a[i]);
    } else {
#pragma unroll
      for (int i = 0; i < NA; ++i) issue_piece_edge(a_edge(i, kt), r.a[i]);
    }
    if (b_fast(kt)) {
      const uintptr_t base = b_base0 + (uintptr_t)((int64_t)2 * G::BK * p.ldb) * (uintptr_t)kt;
#pragma unroll
      for (int i = 0; i < NB; ++i) fetch(base, b_off[i], b_off4[i], r.b[i]);
    } else {
#pragma unroll
      for (int i = 0; i < NB; ++i) issue_piece_edge(b_edge(i, kt), r.b[i]);
    }
  }

  static __device__ __forceinline__ u32x4_t shift(const RawPiece& r, uint32_t lead) {
    u32x4_t out;
    out.x = __builtin_amdgcn_alignbyte(r.w[1], r.w[0], lead);
    out.y = __builtin_amdgcn_alignbyte(r.w[2], r.w[1], lead);
    out.z = __builtin_amdgcn_alignbyte(r.w[3], r.w[2], lead);
    out.w = __builtin_amdgcn_alignbyte(r.w[4], r.w[3], lead);
    return out;
  }

  // Writes stage kt, fetched into r, into LDS buffer s (16-byte stores).
  __device__ __forceinline__ void store(const RawStage<G>& r, int kt, uint16_t* lds, int s) const {
    const int tid = threadIdx.x;
    uint16_t* as = lds + s * G::STAGE;
    uint16_t* bs = as + G::A_STAGE;
    if (a_fast(kt)) {
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int v = tid + i * kThreads;
        *reinterpret_cast<u32x4_t*>(as + (v / (G::BK / 8)) * G::SA + 8 * (v % (G::BK / 8))) = shift(r.a[i], a_lead);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int v = tid + i * kThreads;
        const EdgePlace e = a_edge(i, kt);
        *reinterpret_cast<u32x4_t*>(as + (v / (G::BK / 8)) * G::SA + 8 * (v % (G::BK / 8))) =
            finish_piece(r.a[i], e.lead, e.nvalid, true);
      }
    }
    if (b_fast(kt)) {
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int v = tid + i * kThreads;
        *reinterpret_cast<u32x4_t*>(bs + G::b_chunk(v / (G::BN / 8), 8 * (v % (G::BN / 8)))) = shift(r.b[i], b_lead);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int v = tid + i * kThreads;
        const EdgePlace e = b_edge(i, kt);
        *reinterpret_cast<u32x4_t*>(bs + G::b_chunk(v / (G::BN / 8), 8 * (v % (G::BN / 8)))) =
            finish_piece(r.b[i], e.lead, e.nvalid, true);
      }
    }
  }
};

// D = alpha * acc + beta * C for one element; C is read only when c != nullptr
// and beta != 0 (src/grouped_gemm.cu:475-479, 616-621).
__device__ __forceinline__ float epilogue_value(float acc, float c, float alpha, float beta) {
  return alpha * acc + beta * c;
}

}  // namespace gg
