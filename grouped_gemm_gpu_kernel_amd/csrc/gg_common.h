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
// LDS layout of one stage (binary16), BUFFERS stages:
//   A: BM rows of BK values, each row's 16-byte pieces stored at piece index
//      (c ^ a_swizzle(row)).  64 banks x 4 bytes hold 256 bytes, i.e. 256 / (2 BK)
//      rows; the swizzle gives the rows that share a bank window distinct
//      piece positions, so the 16-byte operand reads of 16 consecutive rows hit
//      distinct banks.  Rows are not padded: a 64-lane load straight into LDS
//      writes 1 KB contiguously.
//   B: BK rows of BN values, row-major as in global memory, with the 8-byte
//      chunks of row k stored at chunk index (c ^ b_swizzle(k)).  The
//      transposing operand read touches 4 consecutive rows x 16 columns per
//      16 lanes; the swizzle spreads those rows over disjoint banks without
//      padding.  It flips only chunk-index bits >= 3, so 16-byte pieces
//      (2 chunks) stay contiguous and every 32-column block stays intact.
//
// Register staging: DEPTH stages are in flight in registers at once, the
// loads of stage k + DEPTH - 1 issued while stage k is multiplied (a ring of
// DEPTH register sets), written to two LDS buffers.  Loads straight into LDS
// use BUFFERS LDS buffers, BUFFERS - 1 stages in flight.
template <int BM_, int BN_, int BK_, int DEPTH_, int THREADS_, int BUFFERS_ = 2, bool A_SWIZZLED_ = false>
struct Geometry {
  static constexpr int BM = BM_;
  static constexpr int BN = BN_;
  static constexpr int BK = BK_;
  static constexpr int DEPTH = DEPTH_;
  static constexpr int THREADS = THREADS_;
  static constexpr int BUFFERS = BUFFERS_;
  // Swizzled, unpadded A rows (needed by loads straight into LDS), or rows
  // padded by 8 values (the FMA tile, whose operand reads then need no
  // per-piece index arithmetic).
  static constexpr bool A_SWIZZLED = A_SWIZZLED_;
  static_assert(DEPTH >= 2, "at least one stage must be in flight while another is multiplied");
  static_assert(BUFFERS >= 2, "at least double buffered");
  static_assert(THREADS % kWave == 0, "whole waves");
  static constexpr int SA = A_SWIZZLED ? BK : BK + 8;
  static constexpr int SB = BN;
  static constexpr int APR = BK / 8;  // 16-byte pieces per A row
  static_assert(APR == 4 || APR == 8, "A swizzle is defined for 32- and 64-deep stages");
  static constexpr int A_STAGE = BM * SA;  // halves
  static constexpr int B_STAGE = BK * SB;  // halves
  static constexpr int STAGE = A_STAGE + B_STAGE;
  static constexpr int LDS_HALVES = BUFFERS * STAGE;
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

  // A: rows that share a 256-byte bank window (row / RPW equal) get distinct
  // piece positions; RPW = 256 / (2 BK) rows per window.
  static constexpr int A_RPW = 128 / BK;
  __device__ static __forceinline__ int a_swizzle(int row) { return A_SWIZZLED ? (row / A_RPW) & (APR - 1) : 0; }
  // Element offset, within an A stage, of the 16-byte piece c (values 8c ..
  // 8c + 7 of the stage's k range) of a row.
  __device__ static __forceinline__ int a_piece(int row, int c) { return row * SA + 8 * (c ^ a_swizzle(row)); }
};

#ifndef GG_STAGE_K
#define GG_STAGE_K 64
#endif
#ifndef GG_STAGE_DEPTH
#define GG_STAGE_DEPTH 3
#endif

// Reference macro-tile of each variant (ids follow GGK_VARIANT_*).
template <int V> struct VariantTile;
template <> struct VariantTile<GGK_VARIANT_64x64x16> { static constexpr int M = 64, N = 64; };
template <> struct VariantTile<GGK_VARIANT_128x64x32> { static constexpr int M = 128, N = 64; };
template <> struct VariantTile<GGK_VARIANT_64x128x32> { static constexpr int M = 64, N = 128; };
template <> struct VariantTile<GGK_VARIANT_128x64x32_SMALL> { static constexpr int M = 128, N = 64; };
template <> struct VariantTile<GGK_VARIANT_64x128x32_SMALL> { static constexpr int M = 64, N = 128; };
template <> struct VariantTile<GGK_VARIANT_64x64x16_SMALL> { static constexpr int M = 64, N = 64; };

// Kernel shape of (variant, path).  The MFMA path computes a block of TM x TN
// reference tiles per claim: each A and B value fetched from L2 then feeds TN
// (A) or TM (B) times the multiply-adds it would feed in a single reference
// tile, which cuts the L2 -> CU traffic that bounds these kernels, and each
// wave owns a WAVE_M x WAVE_N block of D, so that every operand fragment it
// reads from LDS feeds several MFMAs.  Every configuration computes 256 x 256
// of D per claim, eight waves of 128 x 64: 2 x 4 tiles of 128x64x32 (the
// configuration the reference benchmarks by default), 4 x 4 of 64x64x16, 4 x 2
// of 64x128x32.  For launches with few work tiles each also comes on 128 x 128
// work tiles, four waves of 64 x 64 (the _SMALL variants).  The FMA path
// computes one reference tile with 256 threads.
template <int V, int PATH> struct KernelShape;
#ifndef GG_WORK_TM
#define GG_WORK_TM 2
#endif
#ifndef GG_WORK_TN
#define GG_WORK_TN 4
#endif
#ifndef GG_WAVE_N
#define GG_WAVE_N 64
#endif
#ifndef GG_WAVE_M
#define GG_WAVE_M 128
#endif
#ifndef GG_TUNED_WAVES_PER_EU
#define GG_TUNED_WAVES_PER_EU 2
#endif
#ifndef GG_DMA_BUFFERS
#define GG_DMA_BUFFERS 0  // 0: see KernelShape::BUFFERS
#endif
#ifndef GG_TILE_CLASSES
#define GG_TILE_CLASSES 1  // 0: every work tile in the full 256 x 256 form
#endif

template <int V> struct KernelShape<V, GGK_PATH_MFMA> {
  // The three reference macro-tiles share one work tile, 256 x 256 of D; the
  // GG_WORK_* macros retune the 128x64x32 variant's, the other GG_* shape
  // macros all three.
  static constexpr bool kLarge = V == GGK_VARIANT_128x64x32 || V == GGK_VARIANT_64x64x16 || V == GGK_VARIANT_64x128x32;
  static constexpr int TM = V == GGK_VARIANT_128x64x32 ? GG_WORK_TM
                            : kLarge                    ? 256 / VariantTile<V>::M
                                                        : 128 / VariantTile<V>::M;  // tiles along M
  static constexpr int TN = V == GGK_VARIANT_128x64x32 ? GG_WORK_TN
                            : kLarge                    ? 256 / VariantTile<V>::N
                                                        : 128 / VariantTile<V>::N;  // and along N
  static constexpr int BM = TM * VariantTile<V>::M;
  static constexpr int BN = TN * VariantTile<V>::N;
  static constexpr int WAVE_N = kLarge && GG_WAVE_N < BN ? GG_WAVE_N : (BN < 64 ? BN : 64);  // columns of D per wave
  static constexpr int WAVE_M = kLarge && GG_WAVE_M < BM ? GG_WAVE_M : 64;                    // rows of D per wave
  static constexpr int THREADS = (BM / WAVE_M) * (BN / WAVE_N) * kWave;
  // Waves each SIMD must be able to hold (bounds the registers per lane).
  static constexpr int WAVES_PER_EU = kLarge ? GG_TUNED_WAVES_PER_EU : 2;
  // Stages load straight into LDS.  A 512-thread workgroup has a CU to
  // itself and takes three buffers (two stages in flight) when they fit in
  // LDS, else two; a 256-thread one takes two, so that two of its workgroups
  // share a CU.
  static constexpr int STAGE_BYTES = 2 * GG_STAGE_K * (BM + BN);
  static constexpr int BUFFERS =
      GG_DMA_BUFFERS > 0 ? GG_DMA_BUFFERS : (THREADS >= 512 && 3 * STAGE_BYTES <= 150 * 1024 ? 3 : 2);
  // Register staging serves only the 64-bit addressing form here; a ring of
  // two stages keeps it within the registers beside the accumulators (the
  // 256 x 256 work tile's still spills: launches route that form to the
  // 128 x 128 work tile of the same macro-tile).
  using G = Geometry<BM, BN, GG_STAGE_K, 2, THREADS, BUFFERS, true>;
  // Edge classes of the 256 x 256 work tile (32-bit addressing form): a work
  // tile with at most BM / 2 rows or BN / 2 columns inside the problem stages
  // only that half of A or B, so a stage is 48 KB (32 KB when both) and three
  // (four) LDS buffers fit -- two (three) stages in flight instead of one,
  // which is what a tile that streams its operands from HBM is bound by.  The
  // same 512 threads compute it in 64 x 64 (32 x 64) wave blocks; every D
  // element is still one lane's 32x32x16 MFMA chain over ascending k with the
  // same epilogue, so D does not depend on the class.
  static constexpr bool CLASSES = GG_TILE_CLASSES != 0 && kLarge && BM == 256 && BN == 256 && THREADS == 512;
  using GR = Geometry<BM / 2, BN, GG_STAGE_K, 2, THREADS, 3, true>;       // rows <= BM / 2
  using GC = Geometry<BM, BN / 2, GG_STAGE_K, 2, THREADS, 3, true>;       // columns <= BN / 2
  using GRC = Geometry<BM / 2, BN / 2, GG_STAGE_K, 2, THREADS, 4, true>;  // both
  static constexpr int WAVE_M_R = 64, WAVE_M_C = 64, WAVE_M_RC = 32;
};
template <int V> struct KernelShape<V, GGK_PATH_FMA> {
  static constexpr int TM = 1;
  static constexpr int TN = 1;
  static constexpr int WAVES_PER_EU = 2;
  using G = Geometry<VariantTile<V>::M, VariantTile<V>::N, GG_STAGE_K, GG_STAGE_DEPTH, 256>;
  static constexpr bool CLASSES = false;
};

// Per-work-tile phase stamps of a traced launch: 8 int64 per work-tile index
// (GGK_PHASE_* in grouped_gemm_amd_kernels.h).  Core-clock stamps are
// s_memtime; one wave's record stands for the workgroup except the epilogue
// end, the latest over the waves.  NoStamps, the untraced kernels' type,
// compiles to nothing.
struct NoStamps {
  __device__ __forceinline__ void mark(int) const {}
  __device__ __forceinline__ void step_mark(int) const {}
  __device__ __forceinline__ void wave_done() const {}
};
struct PhaseStamps {
  long long* slot;  // this work tile's 8 entries, or null
  __device__ __forceinline__ void mark(int i) const {
    if (slot != nullptr && __builtin_amdgcn_readfirstlane(threadIdx.x / kWave) == 0) {
      slot[i] = static_cast<long long>(__builtin_amdgcn_s_memtime());
    }
  }
  // Every wave (lane 0): mark i of the k-loop step that is stamped (GGK_PHASE_STEP).
  __device__ __forceinline__ void step_mark(int i) const {
    if (slot != nullptr && (threadIdx.x & (kWave - 1)) == 0) {
      const int wave = threadIdx.x / kWave;
      slot[GGK_PHASE_STEP + GGK_PHASE_STEP_MARKS * wave + i] = static_cast<long long>(__builtin_amdgcn_s_memtime());
    }
  }
  // Every wave, when its epilogue has been issued.
  __device__ __forceinline__ void wave_done() const {
    if (slot != nullptr && (threadIdx.x & (kWave - 1)) == 0) {
      atomicMax(reinterpret_cast<unsigned long long*>(slot + GGK_PHASE_EPILOGUE_END),
                static_cast<unsigned long long>(__builtin_amdgcn_s_memtime()));
    }
  }
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
template <class G, bool WIDE>
struct RawStage;
template <class G>
struct RawStage<G, false> {
  u32x4_t a[G::A_PER_THREAD];
  u32x4_t b[G::B_PER_THREAD];
};
template <class G>
struct RawStage<G, true> {
  RawPiece a[G::A_PER_THREAD];
  RawPiece b[G::B_PER_THREAD];
};

// Buffer resource over [base, base + bytes) for raw (unstrided) loads; bytes
// is clamped to 2^32 - 1.  Loads of dwords outside the range return 0 without
// touching memory, dword by dword (a 16-byte load that straddles the end
// returns its in-range dwords), and a 16-byte load from a 2-byte aligned
// offset returns the bytes at that offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int64_t bytes) {
  const int64_t n = bytes < 0 ? 0 : (bytes > 0xffffffffll ? 0xffffffffll : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)(uint32_t)n, 0x00020000);
}

__device__ __forceinline__ u32x4_t buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}

// Replaces binary16 value idx of a 16-byte piece with h (low 16 bits); an idx
// outside 0..7 leaves the piece unchanged.
__device__ __forceinline__ u32x4_t put_value(u32x4_t v, int idx, uint32_t h) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    w[j] = idx == 2 * j ? (w[j] & 0xffff0000u) | h : w[j];
    w[j] = idx == 2 * j + 1 ? (w[j] & 0xffffu) | (h << 16) : w[j];
  }
  return u32x4_t{w[0], w[1], w[2], w[3]};
}

// The binary16 value at p, read through the aligned dword that holds it
// (wave-uniform address: a scalar load).
__device__ __forceinline__ uint32_t load_value_uniform(const uint16_t* p) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t w = *(const __attribute__((address_space(4))) uint32_t*)(a & ~uintptr_t(3));
  return (a & 2) ? (w >> 16) : (w & 0xffffu);
}

// Keeps the first n (0..8) binary16 values of a 16-byte piece, zeroes the rest.
__device__ __forceinline__ u32x4_t keep_values(u32x4_t v, int n) {
  v.x &= n >= 2 ? 0xffffffffu : (n == 1 ? 0xffffu : 0u);
  v.y &= n >= 4 ? 0xffffffffu : (n == 3 ? 0xffffu : 0u);
  v.z &= n >= 6 ? 0xffffffffu : (n == 5 ? 0xffffu : 0u);
  v.w &= n >= 8 ? 0xffffffffu : (n == 7 ? 0xffffu : 0u);
  return v;
}

// Moves the A and B stages of one work tile from global memory into LDS.
//
// A piece v (v = tid + THREADS * i) covers tile row v / (BK/8), columns
// 8 * (v % (BK/8)) of the stage; B piece v covers k-row v / (BN/8), columns
// 8 * (v % (BN/8)).  Consecutive threads read consecutive pieces of one row.
//
// Which values must be exact: D[i][j] depends only on row i of A and column j
// of B, so rows of A past M and columns of B past N only reach elements of D
// that are never stored and may hold anything.  Values at k >= K meet each
// other in the products, so both operands are zeroed there.
//
// WIDE = false: every piece is one 16-byte buffer load at its exact byte
// offset (2-byte aligned rows need no realignment), through a buffer resource
// that spans from the tile's origin to the end of the matrix: rows of A past
// M and rows of B past K lie beyond it (for ld >= the row length) and read as
// zero without touching memory, and nothing past the matrix is ever read.  A
// values at k >= K (the next row's head) and B rows at k >= K are zeroed when
// the stage is written.  Every stage issues the same loads, with no branch,
// so the compiler can count the loads in flight exactly.  The host selects
// this form when the per-tile byte offsets fit in 31 bits
// (rows * lda < 2^30, stage_k * ldb < 2^30, non-negative ld).  The range check
// works on the access's dwords: when a piece starts 2 bytes past a dword, the
// dword that holds the matrix's last value reaches 2 bytes past the matrix
// and reads as 0, so the last value of A and of B is read separately (through
// its aligned dword) and put back when the last stage is written.
//
// WIDE = true: 64-bit addresses per piece; each piece is fetched as the
// dwords from the 4-byte aligned address at or below it that hold wanted
// values (a dword past them is fetched from the first one again) and shifted
// into place when written; values outside the matrix are zero-filled.
template <class G, bool WIDE>
struct StageLoader;

template <class G>
struct StageLoader<G, false> {
  static constexpr int T = G::THREADS;
  static constexpr int NA = G::A_PER_THREAD;
  static constexpr int NB = G::B_PER_THREAD;
  static constexpr int APR = G::BK / 8;  // A pieces per row
  static constexpr int BPR = G::BN / 8;  // B pieces per k-row
  // LDS distance between a thread's consecutive pieces.  The B swizzle
  // repeats every 4 k-rows, so it is the same for all of a thread's pieces.
  static constexpr int A_LDS_STEP = (T / APR) * G::SA;
  static constexpr int B_LDS_STEP = (T / BPR) * G::SB;
  static_assert((T / BPR) % 4 == 0, "a thread's B pieces must share their swizzle");
  static_assert(!G::A_SWIZZLED || (T / APR) % (G::A_RPW * APR) == 0, "a thread's A pieces must share their swizzle");

  const gg_device_problem_desc& p;
  __amdgpu_buffer_rsrc_t a_rsrc;  // A from (m0, 0) to the matrix end
  const uint16_t* b_tile;         // B at (0, n0)
  int64_t b_bytes;                // bytes from b_tile to the end of B
  uint32_t a_off, b_off;          // byte offset of this thread's piece 0 from its origin
  uint32_t a_step, b_step;        // byte distance between a thread's pieces (wave-uniform)
  int a_lds, b_lds;               // LDS offset (values) of piece 0 within a stage's A / B part
  int m0, n0;
  int last_stage;                 // index of the stage that holds k = K - 1
  uint32_t a_last, b_last;        // A[m-1][k-1] and B[k-1][n-1]

  __device__ __forceinline__ StageLoader(const gg_device_problem_desc& prob, int m0_, int n0_)
      : p(prob), m0(m0_), n0(n0_) {
    const int tid = opaque_tid();
    const uint16_t* A = static_cast<const uint16_t*>(p.a);
    const uint16_t* B = static_cast<const uint16_t*>(p.b);
    const uint16_t* a_tile = A + (int64_t)m0 * p.lda;
    // Last element of A is (m - 1, k - 1); of B, (k - 1, n - 1).
    a_rsrc = buffer_rsrc(a_tile, 2 * ((int64_t)(p.m - 1 - m0) * p.lda + p.k));
    b_tile = B + n0;
    b_bytes = 2 * ((int64_t)(p.k - 1) * p.ldb + p.n - n0);
    a_off = 2u * ((uint32_t)(tid / APR) * (uint32_t)p.lda + (uint32_t)(8 * (tid % APR)));
    b_off = 2u * ((uint32_t)(tid / BPR) * (uint32_t)p.ldb + (uint32_t)(8 * (tid % BPR)));
    a_step = 2u * (uint32_t)(T / APR) * (uint32_t)p.lda;
    b_step = 2u * (uint32_t)(T / BPR) * (uint32_t)p.ldb;
    a_lds = G::a_piece(tid / APR, tid % APR);  // the thread's pieces share the swizzle (rows 64 apart)
    b_lds = G::b_chunk(tid / BPR, 8 * (tid % BPR));
    last_stage = (p.k - 1) / G::BK;
    a_last = p.k > 0 ? load_value_uniform(A + (int64_t)(p.m - 1) * p.lda + (p.k - 1)) : 0u;
    b_last = p.k > 0 ? load_value_uniform(B + (int64_t)(p.k - 1) * p.ldb + (p.n - 1)) : 0u;
  }

  // Issues the loads of stage kt into r.  The per-piece and per-stage parts of
  // the offsets are wave-uniform (scalar offset operand).
  __device__ __forceinline__ void issue(int kt, RawStage<G, false>& r) const {
#pragma unroll
    for (int i = 0; i < NA; ++i) r.a[i] = buffer_load16(a_rsrc, a_off, 2u * G::BK * (uint32_t)kt + i * a_step);
    const int64_t skip = 2 * (int64_t)G::BK * kt * p.ldb;
    const __amdgpu_buffer_rsrc_t b_rsrc = buffer_rsrc(b_tile + skip / 2, b_bytes - skip);
#pragma unroll
    for (int i = 0; i < NB; ++i) r.b[i] = buffer_load16(b_rsrc, b_off, i * b_step);
  }

  // Writes stage kt, fetched into r, into LDS buffer s (16-byte stores).  Only
  // the stage that holds k = K - 1 needs masking: A values at k >= K (the next
  // row's head), B rows at k >= K, and the matrices' last values.
  __device__ __forceinline__ void store(const RawStage<G, false>& r, int kt, uint16_t* lds, int s) const {
    uint16_t* as = lds + s * G::STAGE + a_lds;
    uint16_t* bs = lds + s * G::STAGE + G::A_STAGE + b_lds;
    if (kt != last_stage) {
#pragma unroll
      for (int i = 0; i < NA; ++i) *reinterpret_cast<u32x4_t*>(as + i * A_LDS_STEP) = r.a[i];
#pragma unroll
      for (int i = 0; i < NB; ++i) *reinterpret_cast<u32x4_t*>(bs + i * B_LDS_STEP) = r.b[i];
      return;
    }
    const int t = opaque_tid();
    const int a_col = kt * G::BK + 8 * (t % APR);  // a thread's pieces share their columns
    const int a_row = m0 + t / APR;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      u32x4_t val = keep_values(r.a[i], p.k - a_col);
      val = put_value(val, a_row + i * (T / APR) == p.m - 1 ? p.k - 1 - a_col : -1, a_last);
      *reinterpret_cast<u32x4_t*>(as + i * A_LDS_STEP) = val;
    }
    const int b_col = n0 + 8 * (t % BPR);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int krow = kt * G::BK + t / BPR + i * (T / BPR);
      const u32x4_t zero = {0u, 0u, 0u, 0u};
      u32x4_t val = krow < p.k ? r.b[i] : zero;
      val = put_value(val, krow == p.k - 1 ? p.n - 1 - b_col : -1, b_last);
      *reinterpret_cast<u32x4_t*>(bs + i * B_LDS_STEP) = val;
    }
  }
};

template <class G>
struct StageLoader<G, true> {
  static constexpr int T = G::THREADS;
  static constexpr int NA = G::A_PER_THREAD;
  static constexpr int NB = G::B_PER_THREAD;
  static constexpr int APR = G::BK / 8;
  static constexpr int BPR = G::BN / 8;

  const gg_device_problem_desc& p;
  int tid;
  int m0, n0;

  __device__ __forceinline__ StageLoader(const gg_device_problem_desc& prob, int m0_, int n0_)
      : p(prob), tid(opaque_tid()), m0(m0_), n0(n0_) {}

  __device__ __forceinline__ EdgePlace a_edge(int i, int kt) const {
    const int v = tid + i * T;
    return edge_place(static_cast<const uint16_t*>(p.a), p.lda, p.m, p.k, m0 + v / APR, kt * G::BK + 8 * (v % APR));
  }
  __device__ __forceinline__ EdgePlace b_edge(int i, int kt) const {
    const int v = tid + i * T;
    return edge_place(static_cast<const uint16_t*>(p.b), p.ldb, p.k, p.n, kt * G::BK + v / BPR, n0 + 8 * (v % BPR));
  }

  __device__ __forceinline__ void issue(int kt, RawStage<G, true>& r) const {
#pragma unroll
    for (int i = 0; i < NA; ++i) issue_piece_edge(a_edge(i, kt), r.a[i]);
#pragma unroll
    for (int i = 0; i < NB; ++i) issue_piece_edge(b_edge(i, kt), r.b[i]);
  }

  __device__ __forceinline__ void store(const RawStage<G, true>& r, int kt, uint16_t* lds, int s) const {
    const int t = opaque_tid();
    uint16_t* as = lds + s * G::STAGE;
    uint16_t* bs = as + G::A_STAGE;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int v = t + i * T;
      const EdgePlace e = a_edge(i, kt);
      *reinterpret_cast<u32x4_t*>(as + G::a_piece(v / APR, v % APR)) = finish_piece(r.a[i], e.lead, e.nvalid);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int v = t + i * T;
      const EdgePlace e = b_edge(i, kt);
      *reinterpret_cast<u32x4_t*>(bs + G::b_chunk(v / BPR, 8 * (v % BPR))) = finish_piece(r.b[i], e.lead, e.nvalid);
    }
  }
};

// One 16-byte load per lane straight into LDS: lane l's piece, read through
// the raw buffer resource {base, num_records} at byte offset voff + soff
// (range-checked per dword like any buffer load), lands at LDS byte address
// lds + 16 l.  Written as inline assembly on purpose: the compiler's
// wait-count pass, which cannot tell one LDS stage buffer from another, would
// otherwise put a wait for every load in flight before each LDS read, which
// serialises the stage pipeline.  Callers wait for these loads themselves
// (wait_vmcnt); the compiler's own waits stay correct because loads complete
// in order.  The LDS address is an operand bound to M0 ("{m0}"): the compiler
// itself writes M0 before the statement and knows that it is read there, and
// the statement changes no register.
//
// The compiler's hazard pass does not know that the statement is a
// vector-memory instruction, so the statement provides the wait states the
// hardware needs itself: a VALU write of an SGPR (v_readfirstlane of the
// offset or of a resource word, which the compiler may place right before the
// statement) needs 5 before a vector-memory instruction reads that SGPR, and
// a SALU write of M0 needs 1 before an LDS load reads it.  s_nop 4 gives 5.
__device__ __forceinline__ void load_to_lds16(const void* base, uint32_t num_records, uint32_t lds, uint32_t voff,
                                              uint32_t soff) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const u32x4_t rsrc = {static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b))),
                        static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32))) & 0xffffu,
                        static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(num_records)), 0x00020000u};
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  const uint32_t so = __builtin_amdgcn_readfirstlane(soff);
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "{m0}"(m0), "v"(voff), "s"(rsrc), "s"(so)
               : "memory");
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((GG_LDS const void*)p));
}

// Stage loads straight into LDS (buffer_load_dwordx4 ... lds), 32-bit offsets.
//
// A load instruction writes its 64 lanes' 16-byte pieces to 1 KB of LDS in
// lane order, so the LDS layout is fixed by the instruction and the swizzle
// is applied on the global side: lane l of wave w's instruction i fills LDS
// slot s = (i * WAVES + w) * 64 + l of the stage's A (or B) part, i.e. row
// s / PIECES_PER_ROW at piece position s % PIECES_PER_ROW, and therefore
// fetches the global piece that position holds (position ^ swizzle(row)).
// A thread's pieces are rows 8 * WAVES (A) or 4 * WAVES (B, 128 columns)
// apart, which keeps one swizzle per thread, so piece i's global offset is
// piece 0's plus a wave-uniform step (scalar offset operand).
//
// Range checks do what the register path's masking did, except inside the
// stage that holds k = K - 1: A values at k >= K there are the next row's
// head, and a final value whose dword straddles the end of a matrix reads as
// zero.  fix_last_stage repairs the thread's own pieces of that stage in LDS
// once its loads have landed.
template <class G>
struct DmaLoader {
  static_assert(G::A_SWIZZLED, "a load into LDS writes unpadded rows");
  static constexpr int T = G::THREADS;
  static constexpr int WAVES = T / kWave;
  static constexpr int NA = G::A_PER_THREAD;
  static constexpr int NB = G::B_PER_THREAD;
  static constexpr int APR = G::APR;     // A pieces per row
  static constexpr int BPR = G::BN / 8;  // B pieces per k-row
  static_assert((kWave * WAVES / APR) % (G::A_RPW * APR) == 0, "a thread's A pieces must share their swizzle");
  static_assert((kWave * WAVES / BPR) % 4 == 0, "a thread's B pieces must share their swizzle");
  static constexpr int A_ROWS_STEP = kWave * WAVES / APR;  // rows between a thread's A pieces
  static constexpr int B_ROWS_STEP = kWave * WAVES / BPR;  // k-rows between a thread's B pieces
  static constexpr int LOADS = NA + NB;                    // load instructions per stage and wave

  int m, n, k, ldb;
  const uint16_t* a_tile;  // A at (m0, 0)
  int64_t a_bytes;         // bytes from a_tile to the end of A
  const uint16_t* b_tile;  // B at (0, n0)
  int64_t b_bytes;         // bytes from b_tile to the end of B
  uint32_t a_off, b_off;   // byte offset of this thread's piece 0 from its origin
  uint32_t a_step, b_step; // byte distance between a thread's pieces (wave-uniform)
  int wave;                // wave index (uniform)
  int a_row, a_col8;       // piece 0: tile row and global piece index within the stage
  int b_row, b_col8;       // piece 0: k-row within the stage and global piece index
  int m0, n0;
  int last_stage;
  bool a_fix, b_fix;  // whether the matrices' last values must be put back (see the constructor)
  uint32_t a_last, b_last;

  __device__ __forceinline__ DmaLoader(const gg_device_problem_desc& p, int m0_, int n0_)
      : m(p.m), n(p.n), k(p.k), ldb(p.ldb), m0(m0_), n0(n0_) {
    const int tid = opaque_tid();
    const int lane = tid & (kWave - 1);
    wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const uint16_t* A = static_cast<const uint16_t*>(p.a);
    const uint16_t* B = static_cast<const uint16_t*>(p.b);
    a_tile = A + (int64_t)m0 * p.lda;
    a_bytes = 2 * ((int64_t)(p.m - 1 - m0) * p.lda + p.k);
    b_tile = B + n0;
    b_bytes = 2 * ((int64_t)(p.k - 1) * p.ldb + p.n - n0);
    const int sa = wave * kWave + lane;  // A slot of piece 0
    a_row = sa / APR;
    a_col8 = (sa % APR) ^ G::a_swizzle(a_row);
    const int sb = wave * kWave + lane;  // B slot of piece 0
    b_row = sb / BPR;
    b_col8 = (sb % BPR) ^ (G::b_swizzle(b_row) >> 1);  // b_swizzle counts 4-value chunks
    a_off = 2u * ((uint32_t)a_row * (uint32_t)p.lda + (uint32_t)(8 * a_col8));
    b_off = 2u * ((uint32_t)b_row * (uint32_t)p.ldb + (uint32_t)(8 * b_col8));
    // A thread's B pieces all start at column n0 + 8 b_col8; past N they only
    // feed columns of D that are never stored, so they are not fetched.
    if (n0 + 8 * b_col8 >= p.n) b_off = kOutOfRange;
    a_step = 2u * (uint32_t)A_ROWS_STEP * (uint32_t)p.lda;
    b_step = 2u * (uint32_t)B_ROWS_STEP * (uint32_t)p.ldb;
    last_stage = (p.k - 1) / G::BK;
    // A matrix's last value reads as zero only where the dword that holds it
    // would reach 2 bytes past the matrix, i.e. where it sits at an even
    // element of its 16-byte piece.  Pieces start at k = 8c for A and at
    // column n0 + 8c (n0 even) for B, so that happens for A exactly when K is
    // odd and for B when N is odd, and only in the tile holding A's last row
    // or B's last column: only then is the value read (a scalar load from
    // memory, which a barrier's wait would otherwise sit out for every tile).
    a_fix = (p.k & 1) != 0 && m0 + G::BM >= p.m;
    b_fix = (p.n & 1) != 0 && n0 + G::BN >= p.n;
    a_last = a_fix ? load_value_uniform(A + (int64_t)(p.m - 1) * p.lda + (p.k - 1)) : 0u;
    b_last = b_fix ? load_value_uniform(B + (int64_t)(p.k - 1) * p.ldb + (p.n - 1)) : 0u;
  }

  // Byte offset no load reaches: the 32-bit addressing form keeps every
  // offset a tile reads below 2^31, so record counts are capped there and an
  // offset of 2^31 (plus any soffset) reads zeros without touching memory.
  static constexpr uint32_t kOutOfRange = 0x80000000u;
  __device__ static __forceinline__ uint32_t records(int64_t bytes) {
    return (uint32_t)(bytes < 0 ? 0 : (bytes > (int64_t)kOutOfRange ? (int64_t)kOutOfRange : bytes));
  }

  // Issues the loads of stage kt into LDS buffer `stage` (a stage's first element).
  __device__ __forceinline__ void issue(int kt, uint16_t* stage) const {
    const uint32_t base = lds_address(stage) + 2u * (uint32_t)(wave * kWave * 8);
    const uint32_t a_n = records(a_bytes);
    // A pieces that start at k >= K are zero in the product; they are not
    // fetched (the piece that straddles K is, and is repaired afterwards).
    const uint32_t a_voff = kt * G::BK + 8 * a_col8 < k ? a_off : kOutOfRange;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      load_to_lds16(a_tile, a_n, base + 2u * (uint32_t)(i * WAVES * kWave * 8), a_voff,
                    2u * G::BK * (uint32_t)kt + i * a_step);
    }
    const int64_t skip = 2 * (int64_t)G::BK * kt * ldb;
    const uint32_t b_n = records(b_bytes - skip);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      load_to_lds16(b_tile + skip / 2, b_n, base + 2u * (uint32_t)(G::A_STAGE + i * WAVES * kWave * 8), b_off,
                    i * b_step);
    }
  }

  // Repairs this thread's pieces of stage kt (the one that holds k = K - 1)
  // in LDS buffer `stage`, after their loads have landed: A values at k >= K
  // and B rows at k >= K become zero, and the matrices' last values are put
  // back where a straddling dword read them as zero.
  __device__ __forceinline__ void fix_last_stage(int kt, uint16_t* stage) const {
    // The inputs pass through empty asm statements: everything computed from
    // them stays inside the caller's branch (computed early, the masks below
    // would cost vector instructions and registers in every k-step, though
    // only one stage per tile needs them).
    int k = this->k, m = this->m, n = this->n, a_row = this->a_row, b_row = this->b_row;
    int a_col8 = this->a_col8, b_col8 = this->b_col8, m0 = this->m0, n0 = this->n0;
    asm volatile("" : "+s"(k), "+s"(m), "+s"(n), "+s"(m0), "+s"(n0), "+s"(kt));
    asm volatile("" : "+v"(a_row), "+v"(b_row), "+v"(a_col8), "+v"(b_col8));
    const int lane = opaque_tid() & (kWave - 1);
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      u32x4_t* slot = reinterpret_cast<u32x4_t*>(stage + (i * WAVES + wave) * (kWave * 8) + 8 * lane);
      const int col = kt * G::BK + 8 * a_col8;
      const int row = m0 + a_row + i * A_ROWS_STEP;
      u32x4_t val = keep_values(*slot, k - col);
      val = put_value(val, a_fix && row == m - 1 ? k - 1 - col : -1, a_last);
      *slot = val;
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      u32x4_t* slot = reinterpret_cast<u32x4_t*>(stage + G::A_STAGE + (i * WAVES + wave) * (kWave * 8) + 8 * lane);
      const int krow = kt * G::BK + b_row + i * B_ROWS_STEP;
      const int col = n0 + 8 * b_col8;
      const u32x4_t zero = {0u, 0u, 0u, 0u};
      u32x4_t val = krow < k ? *slot : zero;
      val = put_value(val, b_fix && krow == k - 1 ? n - 1 - col : -1, b_last);
      *slot = val;
    }
  }
};

// Waits until at most `n` vector-memory operations of this wave are in flight
// (other counters unconstrained).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier that waits for this wave's LDS accesses (lgkmcnt 0) but
// not for its global loads: the caller waits for the loads it needs first.
// The empty asm keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void stage_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4) | (0x0 << 8));  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// D = alpha * acc + beta * C for one element; C is read only when c != nullptr
// and beta != 0 (src/grouped_gemm.cu:475-479, 616-621).  One fixed rounding
// sequence -- beta * C rounded, then one fused multiply-add -- so that every
// work-tile shape, addressing form and path gives the same bits (left to the
// compiler, the contraction differs between code shapes).  Where C is not
// read the callers pass beta = 0 and c = 0, so D is alpha * acc whatever beta
// holds (an infinite or NaN beta with a null C gives no NaN).
__device__ __forceinline__ float epilogue_value(float acc, float c, float alpha, float beta) {
  return __builtin_fmaf(alpha, acc, beta * c);
}

}  // namespace gg
