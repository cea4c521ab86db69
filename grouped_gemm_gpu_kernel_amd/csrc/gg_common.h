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

constexpr int kWave = 64;

// Geometry of one kernel's work tile.  BM x BN is the block of D a workgroup
// computes per claim; BK is the depth of one LDS stage; THREADS is the
// workgroup size.  The reference's macro-tile (cta_m x cta_n,
// src/grouped_gemm.cu:47-65) fixes the tile -> problem mapping; a work tile
// covers a whole number of those tiles.
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
template <int BM_, int BN_, int BK_, int DEPTH_, int THREADS_>
struct Geometry {
  static constexpr int BM = BM_;
  static constexpr int BN = BN_;
  static constexpr int BK = BK_;
  static constexpr int DEPTH = DEPTH_;
  static constexpr int THREADS = THREADS_;
  static_assert(DEPTH >= 2, "at least one stage must be in flight while another is multiplied");
  static_assert(THREADS % kWave == 0, "whole waves");
  static constexpr int SA = BK + 8;
  static constexpr int SB = BN;
  static constexpr int A_STAGE = BM * SA;  // halves
  static constexpr int B_STAGE = BK * SB;  // halves
  static constexpr int STAGE = A_STAGE + B_STAGE;
  static constexpr int LDS_HALVES = 2 * STAGE;
  // 16-byte pieces per stage and per thread.
  static constexpr int A_VECS = BM * BK / 8;
  static constexpr int B_VECS = BK * BN / 8;
  static constexpr int A_PER_THREAD = A_VECS / THREADS;
  static constexpr int B_PER_THREAD = B_VECS / THREADS;
  static_assert(A_VECS % THREADS == 0 && B_VECS % THREADS == 0, "staging must split evenly");
  static_assert(BK % 16 == 0, "stage depth must be a multiple of the MFMA k");
  static_assert(BN == 64 || BN == 128 || BN == 256, "B swizzle is defined for 64-, 128- and 256-column tiles");
  static_assert(2 * LDS_HALVES <= 160 * 1024, "two stages must fit the 160 KB of LDS");

  // 64 banks x 4 bytes hold 256 bytes: two 64-column rows or half of a
  // 256-column row.  XOR-ing the chunk index with 8 moves a chunk by 64 bytes,
  // so rows k..k+3 (k a multiple of 4) land on 4 different 64-byte bank windows.
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

#ifndef GG_STAGE_K
#define GG_STAGE_K 64
#endif
#ifndef GG_STAGE_DEPTH
#define GG_STAGE_DEPTH 2
#endif

// Reference macro-tile of each variant (ids follow GGK_VARIANT_*).
template <int V> struct VariantTile;
template <> struct VariantTile<GGK_VARIANT_64x64x16> { static constexpr int M = 64, N = 64; };
template <> struct VariantTile<GGK_VARIANT_128x64x32> { static constexpr int M = 128, N = 64; };
template <> struct VariantTile<GGK_VARIANT_64x128x32> { static constexpr int M = 64, N = 128; };

// Kernel shape of (variant, path).  The MFMA path computes a 2 x 2 block of
// reference tiles per claim with one wave per 64 x 64 block of D: each A and B
// value fetched from L2 feeds twice the multiply-adds it would feed in a
// single reference tile, which halves the L2 -> CU traffic that bounds these
// kernels.  The FMA path computes one reference tile with 256 threads.
template <int V, int PATH> struct KernelShape;
template <int V> struct KernelShape<V, GGK_PATH_MFMA> {
  static constexpr int TM = 2;  // reference tiles per work tile, along M
  static constexpr int TN = 2;  // and along N
  static constexpr int BM = TM * VariantTile<V>::M;
  static constexpr int BN = TN * VariantTile<V>::N;
  using G = Geometry<BM, BN, GG_STAGE_K, GG_STAGE_DEPTH, (BM / 64) * (BN / 64) * kWave>;
};
template <int V> struct KernelShape<V, GGK_PATH_FMA> {
  static constexpr int TM = 1;
  static constexpr int TN = 1;
  using G = Geometry<VariantTile<V>::M, VariantTile<V>::N, GG_STAGE_K, GG_STAGE_DEPTH, 256>;
};

// threadIdx.x behind an empty asm: the compiler must assume it changes at
// every call, so values derived from it are recomputed where they are used
// instead of being held in registers for the whole persistent kernel.
__device__ __forceinline__ int opaque_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

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

// Placement of a piece that may cross the matrix edge.
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

// Zeroes a piece that is not fetched.  Every issue defines all registers of
// its stage, so no register set stays live from one stage to the next.
__device__ __forceinline__ void skip_piece(RawPiece& out) {
#pragma unroll
  for (int i = 0; i < 5; ++i) out.w[i] = 0u;
}

// General fetch: only dwords that hold a wanted value are read, so every
// access stays inside the matrix; a piece with no valid value reads nothing.
__device__ __forceinline__ void issue_piece_edge(const EdgePlace& e, RawPiece& out) {
  if (e.nvalid == 0) {
    skip_piece(out);
    return;
  }
  const uintptr_t q = reinterpret_cast<uintptr_t>(e.p) & ~uintptr_t(3);
  const uint32_t span = e.lead + 2u * e.nvalid;  // wanted bytes counted from q
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const uintptr_t a = (4u * i < span) ? q + 4u * i : q;
    out.w[i] = *(g_u32_t*)a;
  }
}

// Shifts a piece fetched by issue_piece_edge into place, clearing dwords that
// were fetched as stand-ins and values past nvalid.
__device__ __forceinline__ u32x4_t finish_piece(const RawPiece& r, uint32_t lead, uint32_t nvalid) {
  const uint32_t span = lead + 2u * nvalid;
  uint32_t w[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) w[i] = (4u * i < span) ? r.w[i] : 0u;
  u32x4_t out;
  out.x = __builtin_amdgcn_alignbyte(w[1], w[0], lead);
  out.y = __builtin_amdgcn_alignbyte(w[2], w[1], lead);
  out.z = __builtin_amdgcn_alignbyte(w[3], w[2], lead);
  out.w = __builtin_amdgcn_alignbyte(w[4], w[3], lead);
  const uint32_t n = nvalid;
  out.x &= (n >= 2) ? 0xffffffffu : (n == 1 ? 0xffffu : 0u);
  out.y &= (n >= 4) ? 0xffffffffu : (n == 3 ? 0xffffu : 0u);
  out.z &= (n >= 6) ? 0xffffffffu : (n == 5 ? 0xffffu : 0u);
  out.w &= (n >= 8) ? 0xffffffffu : (n == 7 ? 0xffffu : 0u);
  return out;
}

// The loads of one stage in flight: this thread's A and B pieces.
template <class G>
struct RawStage {
  RawPiece a[G::A_PER_THREAD];
  RawPiece b[G::B_PER_THREAD];
};

// Moves the A and B stages of one work tile from global memory into LDS.
//
// A piece v (v = tid + THREADS * i) covers tile row v / (BK/8), columns
// 8 * (v % (BK/8)) of the stage; B piece v covers k-row v / (BN/8), columns
// 8 * (v % (BN/8)).  Consecutive threads read consecutive pieces of one row.
//
// Which values must be exact: D[i][j] depends only on row i of A and column j
// of B, so rows of A past M and columns of B past N only reach elements of D
// that are never stored.  Pieces that start past M or N are therefore not
// loaded at all (their LDS slots receive zeros), and a B piece that straddles
// N may bring in whatever follows column N - 1 in memory.  Values at k >= K
// meet each other in the products, so a stage that reaches past K zero-fills
// both operands.
//
// Addressing (WIDE = false): the stage's origin is a wave-uniform byte address
// (advanced with scalar arithmetic) and each piece has a fixed 32-bit byte
// offset from it, set up once per tile; the host selects this form when
// BM * lda and BK * ldb are below 2^30 and both are non-negative.  Inside
// stages fetch a piece as 16 bytes plus, when it starts 2 bytes past a dword,
// one more dword.  Inside means: for A, all k of the stage below K; for B, the
// same, and when the tile's columns run past N also no row K - 1 in the stage
// and ldb >= 8 -- a straddling piece then reads at most 18 bytes past its
// row's last value, which lie in the next row, never past the matrix.  Other
// stages fetch only the dwords that hold wanted values (same offsets).
// WIDE = true computes 64-bit addresses per piece and uses that careful
// fetch everywhere.
template <class G, bool WIDE>
struct StageLoader {
  static constexpr int T = G::THREADS;
  static constexpr int NA = G::A_PER_THREAD;
  static constexpr int NB = G::B_PER_THREAD;
  static constexpr int APR = G::BK / 8;  // A pieces per row
  static constexpr int BPR = G::BN / 8;  // B pieces per k-row
  // A thread's pieces lie an even number of rows apart, so they share the
  // 2-byte misalignment (lead) of their first piece.
  static_assert((T / APR) % 2 == 0 && (T / BPR) % 2 == 0, "pieces of a thread must be an even number of rows apart");
  static_assert(NA <= 32 && NB <= 32, "one live bit per piece");

  const gg_device_problem_desc& p;
  int tid;
  int m0, n0;
  bool b_inside;           // the tile's columns all lie below N
  bool b_straddle_ok;      // b_inside, or ldb >= 8 (see above)
  uintptr_t a_base0;       // 4-byte aligned origin of stage 0; stage kt adds 2*BK*kt bytes
  uintptr_t b_base0;       // stage kt adds 2*BK*ldb*kt bytes
  // Piece i lies i * (THREADS / APR) rows (A) or i * (THREADS / BPR) k-rows (B)
  // below piece 0: its offset is off + i * step, with step wave-uniform.
  uint32_t a_off, b_off;   // 4-byte aligned offset of piece 0 from the stage origin
  uint32_t a_step, b_step; // byte distance between consecutive pieces of a thread
  uint32_t a_live, b_live; // bit i: piece i starts below M (A) or below N (B)
  uint32_t a_lead, b_lead; // 0 or 2: a thread's pieces share it

  __device__ __forceinline__ StageLoader(const gg_device_problem_desc& prob, int m0_, int n0_)
      : p(prob), tid(opaque_tid()), m0(m0_), n0(n0_) {
    b_inside = n0 + G::BN <= p.n;
    b_straddle_ok = b_inside || p.ldb >= 8;
    a_live = 0;
    b_live = 0;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      if (m0 + (tid + i * T) / APR < p.m) a_live |= 1u << i;
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      if (n0 + 8 * ((tid + i * T) % BPR) < p.n) b_live |= 1u << i;
    }
    if constexpr (!WIDE) {
      const uintptr_t A = reinterpret_cast<uintptr_t>(p.a);
      const uintptr_t B = reinterpret_cast<uintptr_t>(p.b);
      a_base0 = (A & ~uintptr_t(3)) + (uintptr_t)((int64_t)m0 * p.lda * 2);
      b_base0 = (B & ~uintptr_t(3)) + (uintptr_t)((int64_t)n0 * 2);
      const uint32_t a_rel = (uint32_t)(tid / APR) * (uint32_t)p.lda * 2u + (uint32_t)(16 * (tid % APR)) + (uint32_t)(A & 3);
      const uint32_t b_rel = (uint32_t)(tid / BPR) * (uint32_t)p.ldb * 2u + (uint32_t)(16 * (tid % BPR)) + (uint32_t)(B & 3);
      a_off = a_rel & ~3u;
      b_off = b_rel & ~3u;
      a_lead = a_rel & 2u;
      b_lead = b_rel & 2u;
      a_step = (uint32_t)(T / APR) * (uint32_t)p.lda * 2u;
      b_step = (uint32_t)(T / BPR) * (uint32_t)p.ldb * 2u;
    }
  }

  __device__ __forceinline__ bool a_fast(int kt) const { return !WIDE && (kt + 1) * G::BK <= p.k; }
  __device__ __forceinline__ bool b_fast(int kt) const {
    return !WIDE && ((kt + 1) * G::BK < p.k ? b_straddle_ok : (b_inside && (kt + 1) * G::BK == p.k));
  }

  // Values of A piece i / B piece i of stage kt inside the matrix (0..8).
  __device__ __forceinline__ uint32_t a_nvalid(int i, int kt) const {
    const int v = tid + i * T;
    const int n = p.k - (kt * G::BK + 8 * (v % APR));
    return (a_live & (1u << i)) ? (uint32_t)(n < 0 ? 0 : (n > 8 ? 8 : n)) : 0u;
  }
  __device__ __forceinline__ uint32_t b_nvalid(int i, int kt) const {
    const int v = tid + i * T;
    const int n = p.n - (n0 + 8 * (v % BPR));
    return ((b_live & (1u << i)) && kt * G::BK + v / BPR < p.k) ? (uint32_t)(n < 0 ? 0 : (n > 8 ? 8 : n)) : 0u;
  }

  // Placement of A piece i and B piece i of stage kt with 64-bit addresses (WIDE).
  __device__ __forceinline__ EdgePlace a_edge(int i, int kt) const {
    const int v = tid + i * T;
    return edge_place(static_cast<const uint16_t*>(p.a), p.lda, p.m, p.k, m0 + v / APR, kt * G::BK + 8 * (v % APR));
  }
  __device__ __forceinline__ EdgePlace b_edge(int i, int kt) const {
    const int v = tid + i * T;
    return edge_place(static_cast<const uint16_t*>(p.b), p.ldb, p.k, p.n, kt * G::BK + v / BPR, n0 + 8 * (v % BPR));
  }

  // 16 bytes from off and, when the piece starts 2 bytes past off (lead 2),
  // the dword after them, else the first dword again (the shift ignores it).
  // Unconditional: a branch here costs more than the extra load.
  static __device__ __forceinline__ void fetch(uintptr_t base, uint32_t off, uint32_t lead, RawPiece& out) {
    const u32x4_t v = *(g_u32x4_t*)(base + off);
    out.w[0] = v.x;
    out.w[1] = v.y;
    out.w[2] = v.z;
    out.w[3] = v.w;
    out.w[4] = *(g_u32_t*)(base + off + 8u * lead);
  }

  // Fetches only the dwords of a piece that hold one of its nvalid values; a
  // dword past them is fetched from off itself (a wanted dword).
  static __device__ __forceinline__ void fetch_careful(uintptr_t base, uint32_t off, uint32_t lead, uint32_t nvalid,
                                                       RawPiece& out) {
    if (nvalid == 0) {
      skip_piece(out);
      return;
    }
    const uint32_t span = lead + 2u * nvalid;
#pragma unroll
    for (int j = 0; j < 5; ++j) out.w[j] = *(g_u32_t*)(base + ((4u * j < span) ? off + 4u * j : off));
  }

  __device__ __forceinline__ uintptr_t a_stage_base(int kt) const {
    return a_base0 + (uintptr_t)(2 * G::BK) * (uintptr_t)kt;
  }
  __device__ __forceinline__ uintptr_t b_stage_base(int kt) const {
    return b_base0 + (uintptr_t)((int64_t)2 * G::BK * p.ldb) * (uintptr_t)kt;
  }

  // Issues the loads of stage kt into r.
  __device__ __forceinline__ void issue(int kt, RawStage<G>& r) const {
    if constexpr (WIDE) {
#pragma unroll
      for (int i = 0; i < NA; ++i) issue_piece_edge(a_edge(i, kt), r.a[i]);
#pragma unroll
      for (int i = 0; i < NB; ++i) issue_piece_edge(b_edge(i, kt), r.b[i]);
    } else {
      const uintptr_t abase = a_stage_base(kt);
      if (a_fast(kt)) {
#pragma unroll
        for (int i = 0; i < NA; ++i) {
          if (a_live & (1u << i)) {
            fetch(abase, a_off + i * a_step, a_lead, r.a[i]);
          } else {
            skip_piece(r.a[i]);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < NA; ++i) fetch_careful(abase, a_off + i * a_step, a_lead, a_nvalid(i, kt), r.a[i]);
      }
      const uintptr_t bbase = b_stage_base(kt);
      if (b_fast(kt)) {
#pragma unroll
        for (int i = 0; i < NB; ++i) {
          if (b_live & (1u << i)) {
            fetch(bbase, b_off + i * b_step, b_lead, r.b[i]);
          } else {
            skip_piece(r.b[i]);
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < NB; ++i) fetch_careful(bbase, b_off + i * b_step, b_lead, b_nvalid(i, kt), r.b[i]);
      }
    }
  }

  // Shifts a piece fetched by `fetch` into place.
  static __device__ __forceinline__ u32x4_t shift_fast(const RawPiece& r, uint32_t lead) {
    u32x4_t out;
    out.x = __builtin_amdgcn_alignbyte(r.w[1], r.w[0], lead);
    out.y = __builtin_amdgcn_alignbyte(r.w[2], r.w[1], lead);
    out.z = __builtin_amdgcn_alignbyte(r.w[3], r.w[2], lead);
    out.w = __builtin_amdgcn_alignbyte(r.w[4], r.w[3], lead);
    return out;
  }

  // Writes stage kt, fetched into r, into LDS buffer s (16-byte stores).
  __device__ __forceinline__ void store(const RawStage<G>& r, int kt, uint16_t* lds, int s) const {
    const int tid = opaque_tid();
    uint16_t* as = lds + s * G::STAGE;
    uint16_t* bs = as + G::A_STAGE;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int v = tid + i * T;
      u32x4_t val;
      if constexpr (WIDE) {
        const EdgePlace e = a_edge(i, kt);
        val = finish_piece(r.a[i], e.lead, e.nvalid);
      } else {
        val = a_fast(kt) ? shift_fast(r.a[i], a_lead) : finish_piece(r.a[i], a_lead, a_nvalid(i, kt));
      }
      *reinterpret_cast<u32x4_t*>(as + (v / APR) * G::SA + 8 * (v % APR)) = val;
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int v = tid + i * T;
      u32x4_t val;
      if constexpr (WIDE) {
        const EdgePlace e = b_edge(i, kt);
        val = finish_piece(r.b[i], e.lead, e.nvalid);
      } else {
        val = b_fast(kt) ? shift_fast(r.b[i], b_lead) : finish_piece(r.b[i], b_lead, b_nvalid(i, kt));
      }
      *reinterpret_cast<u32x4_t*>(bs + G::b_chunk(v / BPR, 8 * (v % BPR))) = val;
    }
  }
};

// D = alpha * acc + beta * C for one element; C is read only when c != nullptr
// and beta != 0 (src/grouped_gemm.cu:475-479, 616-621).
__device__ __forceinline__ float epilogue_value(float acc, float c, float alpha, float beta) {
  return alpha * acc + beta * c;
}

}  // namespace gg
